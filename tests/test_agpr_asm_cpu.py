"""The one-wave-per-SIMD GEMM kernels issue their MFMAs from inline asm with the
accumulators bound to AGPRs (gemm_dma.h, DmaMma<16>::run_agpr).  The compiler's
hazard checks do not look into asm, so the kernel supplies the wait states itself.
This test disassembles the gfx950 code object of the built libsoklyn_hip.so and
checks, for every such kernel, the invariants those wait states rely on:

  * between the first and the last MFMA of the kernel, nothing but an MFMA writes an
    AGPR (no v_accvgpr_write / v_accvgpr_mov / other VALU with an AGPR destination);
  * the accumulators' zeroing (v_accvgpr_write) is at least 2 wait states before the
    first MFMA (a VALU write of an MFMA source needs 2);
  * the first instruction after the last MFMA that touches an AGPR (the epilogue's
    v_accvgpr_read, or a ds_write storing AGPRs to LDS directly) is at least 19 wait
    states later (an XDL write followed by a VALU or memory read needs up to 19 for
    the longest pass count).

Wait states are counted as issued instructions, s_nop N counting N + 1.

A second test reads the kernel metadata of every code object (one per source file)
and requires every kernel of the library to use no scratch memory (private segment size 0): a GEMM whose
accumulators or fragment arrays land in scratch (an epilogue loop the compiler does
not fully unroll indexes them dynamically) still computes the right result, but an
order of magnitude slower.  No GPU is needed: only the compiler's output is read.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "soklyn_amd", "libsoklyn_hip.so")
LLVM = "/opt/rocm/llvm/bin"
ONE_WAVE = re.compile(r"_ZN3skl15gemm_dma_kernel\S*Li4ELb0ELi16ELi256E\S*")


def _tool(name):
    p = os.path.join(LLVM, name)
    return p if os.path.exists(p) else shutil.which(name)


def _code_objects(d):
    """The gfx950 code objects of libsoklyn_hip.so (one offload bundle per source file in
    its .hip_fatbin section), extracted into directory d."""
    tools = [_tool(t) for t in ("llvm-objcopy", "clang-offload-bundler")]
    if not os.path.exists(LIB) or not all(tools):
        pytest.skip("libsoklyn_hip.so or the ROCm LLVM tools are not available")
    objcopy, bundler = tools
    fat = os.path.join(d, "fatbin.bin")
    subprocess.run([objcopy, "--dump-section", f".hip_fatbin={fat}", LIB], check=True)
    with open(fat, "rb") as f:
        data = f.read()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts, i = [], data.find(magic)
    while i >= 0:
        starts.append(i)
        i = data.find(magic, i + 1)
    cos = []
    for k, a in enumerate(starts):
        part, co = os.path.join(d, f"bundle{k}.bin"), os.path.join(d, f"co{k}.o")
        with open(part, "wb") as f:
            f.write(data[a:starts[k + 1] if k + 1 < len(starts) else len(data)])
        subprocess.run([bundler, "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={part}",
                        f"--output={co}", "--unbundle"], check=True)
        cos.append(co)
    assert cos, "no offload bundle in libsoklyn_hip.so"
    return cos


def _disassembly():
    objdump = _tool("llvm-objdump")
    if not objdump:
        pytest.skip("llvm-objdump is not available")
    kernels = {}
    with tempfile.TemporaryDirectory() as d:
        for co in _code_objects(d):
            syms = sorted({m.group(0) for m in ONE_WAVE.finditer(
                subprocess.run([objdump, "-t", co], check=True, capture_output=True, text=True).stdout)
                if not m.group(0).endswith(".kd")})
            if not syms:
                continue
            out = subprocess.run([objdump, "-d", "--mcpu=gfx950", "--disassemble-symbols=" + ",".join(syms), co],
                                 check=True, capture_output=True, text=True).stdout
            cur = None
            for line in out.splitlines():
                m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
                if m:
                    cur = m.group(1)
                    kernels[cur] = []
                elif cur and line.startswith("\t"):
                    ins = line.strip().split("//")[0].strip()
                    if ins:
                        kernels[cur].append(ins)
    return kernels


def _wait_states(instrs):
    n = 0
    for ins in instrs:
        m = re.match(r"s_nop (\d+|0x[0-9a-f]+)", ins)
        n += int(m.group(1), 0) + 1 if m else 1
    return n


def _writes_agpr(ins):
    # destination operand (the first one) is an AGPR or AGPR tuple
    parts = ins.split(None, 1)
    return len(parts) == 2 and re.match(r"a(\d+|\[\d+:\d+\])\b", parts[1]) is not None


def test_one_wave_kernels_keep_the_asm_mfma_hazard_invariants():
    kernels = _disassembly()
    assert kernels, "no one-wave-per-SIMD GEMM kernel found in libsoklyn_hip.so"
    for name, ins in kernels.items():
        mfma = [i for i, s in enumerate(ins) if s.startswith("v_mfma")]
        assert len(mfma) >= 128, f"{name}: {len(mfma)} MFMAs"
        first, last = mfma[0], mfma[-1]
        bad = [s for s in ins[first:last + 1] if _writes_agpr(s) and not s.startswith("v_mfma")]
        assert not bad, f"{name}: AGPR written between MFMAs by {bad[:3]}"
        zero = [i for i, s in enumerate(ins[:first]) if s.startswith("v_accvgpr_write")]
        if zero:
            assert _wait_states(ins[zero[-1] + 1:first]) >= 2, f"{name}: accumulator zeroing too close to MFMA"
        reads = [i for i, s in enumerate(ins) if i > last and re.search(r"\ba(\d+|\[\d+:\d+\])", s)]
        assert reads, f"{name}: no epilogue read of the accumulators"
        assert _wait_states(ins[last + 1:reads[0]]) >= 19, f"{name}: epilogue reads AGPRs too soon after MFMA"


def test_no_kernel_uses_scratch():
    readelf = _tool("llvm-readelf")
    if not readelf:
        pytest.skip("llvm-readelf is not available")
    sizes = {}
    with tempfile.TemporaryDirectory() as d:
        for co in _code_objects(d):
            notes = subprocess.run([readelf, "--notes", co], check=True, capture_output=True, text=True).stdout
            name = None
            for line in notes.splitlines():
                m = re.match(r"\s*\.name:\s+(\S+)", line)
                if m:
                    name = m.group(1)
                m = re.match(r"\s*\.private_segment_fixed_size:\s+(\d+)", line)
                if m and name:
                    sizes[name] = int(m.group(1))
                    name = None
    assert len(sizes) >= 20, f"kernel metadata not found ({len(sizes)} kernels)"
    assert any("gemm_dma_kernel" in k for k in sizes)
    assert any("error_flat_kernel" in k for k in sizes) and any("norm_rows" in k for k in sizes)
    bad = {k: v for k, v in sizes.items() if v}
    assert not bad, f"kernels using scratch memory: {bad}"
