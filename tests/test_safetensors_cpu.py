"""The checkpoint container of src/io/safetensor.rs (C++: soklyn_amd/host/safetensors.cpp)
against the `safetensors` library and a Python restatement of the reference's header
layout (serde_json 1.0.150 without preserve_order: to_string_pretty of a sorted map),
both directions, on the CPU."""
from __future__ import annotations

import json
import os
import struct
import subprocess

import numpy as np
import pytest

safetensors_numpy = pytest.importorskip("safetensors.numpy")
from safetensors import safe_open  # noqa: E402

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "soklyn_amd", "host", "soklyn_tool")


def tool(*args) -> str:
    p = subprocess.run([TOOL, *map(str, args)], capture_output=True, text=True, timeout=60)
    assert p.returncode == 0, p.stdout + p.stderr
    return p.stdout


def serde_pretty_header(tensors: dict, metadata: dict) -> bytes:
    """What serde_json::to_string_pretty writes for the reference's header map, padded
    with spaces to a multiple of 8 (safetensor.rs:151-191)."""
    top = {}
    if metadata:
        top["__metadata__"] = dict(metadata)
    for name, (dtype, shape, o0, o1) in tensors.items():
        top[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [o0, o1]}
    s = json.dumps(top, indent=2, sort_keys=True, ensure_ascii=False).encode()
    return s + b" " * (-len(s) % 8)


def test_written_file_matches_library_and_reference_header(tmp_path):
    path = str(tmp_path / "demo.safetensors")
    tool("st-demo", path)
    blob = open(path, "rb").read()
    n = struct.unpack("<Q", blob[:8])[0]
    header = blob[8:8 + n]
    name = 'demo "quoted" \\ / é \t tab\n line\x01'
    want = serde_pretty_header({"layer1.w": ("F32", (2, 3), 0, 24), "alpha": ("F16", (5,), 24, 34),
                                "scalar": ("F32", (), 34, 38), "empty": ("F32", (0, 3), 38, 38)},
                               {"name": name, "epoch": "7"})
    assert header == want
    t = safetensors_numpy.load_file(path)
    assert np.array_equal(t["layer1.w"], (0.5 * np.arange(6, dtype=np.float32) - 1.25).reshape(2, 3))
    assert t["alpha"].dtype == np.float16
    assert np.array_equal(t["alpha"].view(np.uint16),
                          np.array([1.5, -2.0, 0.1, 65504.0, -0.0], np.float16).view(np.uint16))
    assert t["scalar"].shape == () and t["scalar"] == np.float32(3.25)
    assert t["empty"].shape == (0, 3)
    with safe_open(path, "np") as f:
        assert f.metadata() == {"name": name, "epoch": "7"}


def test_reads_library_written_file(tmp_path):
    path = str(tmp_path / "lib.safetensors")
    g = np.random.default_rng(3)
    w = g.standard_normal((4, 3)).astype(np.float32)
    h = g.standard_normal(7).astype(np.float16)
    safetensors_numpy.save_file({"layer1.w": w, "layer2.norm_b": h}, path, metadata={"k": "v", "x": "1"})
    lines = tool("st-dump", path).strip().splitlines()
    assert lines[0] == 'meta "k" "v"' and lines[1] == 'meta "x" "1"'
    rows = {l.split()[1]: l.split()[2:] for l in lines[2:]}
    assert rows["layer1.w"][:2] == ["F32", "[4,3]"] and bytes.fromhex(rows["layer1.w"][2]) == w.tobytes()
    assert rows["layer2.norm_b"][:2] == ["F16", "[7]"] and bytes.fromhex(rows["layer2.norm_b"][2]) == h.tobytes()


def test_rejects_unsupported_dtype_and_malformed_header(tmp_path):
    bad = str(tmp_path / "i32.safetensors")
    safetensors_numpy.save_file({"a": np.arange(4, dtype=np.int32)}, bad)
    p = subprocess.run([TOOL, "st-dump", bad], capture_output=True, text=True, timeout=60)
    assert p.returncode == 3 and "Unrecognized tensor key" in p.stderr
    junk = str(tmp_path / "junk.safetensors")
    with open(junk, "wb") as fh:
        fh.write(struct.pack("<Q", 7) + b'{"a": 1')          # unterminated object
    p = subprocess.run([TOOL, "st-dump", junk], capture_output=True, text=True, timeout=60)
    assert p.returncode == 3 and "JSON error" in p.stderr
    short = str(tmp_path / "short.safetensors")
    with open(short, "wb") as fh:
        fh.write(struct.pack("<Q", 64) + b"{}")               # header shorter than announced
    p = subprocess.run([TOOL, "st-dump", short], capture_output=True, text=True, timeout=60)
    assert p.returncode == 3 and "I/O error" in p.stderr
