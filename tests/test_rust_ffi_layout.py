"""The Rust binding of the C ABI (rust/src/io/device/hip_ffi.rs) against include/soklyn_hip.h.

There is no Rust toolchain in this image, so the binding cannot be compiled here;
this test makes it checkable instead.  It parses the Rust `#[repr(C)]` structs and
`extern "C"` block and the header's structs and prototypes, and requires:

  * every function the header declares is declared in Rust with the same name,
    parameter count, parameter types and return type (C types mapped to their
    Rust FFI equivalents: uint32_t -> u32, size_t -> usize, const float * ->
    *const f32, skl_ctx ** -> *mut *mut SklCtx, ...), and no other;
  * every struct has the same fields in the same order with mapped types, and
    each field's offset and the struct's size, computed by the repr(C) layout
    rules (each field at the next multiple of its alignment, the size rounded to
    the largest alignment), equal what the C compiler reports (offsetof /
    sizeof from a program compiled here with gcc against the header);
  * the Python ctypes binding (soklyn_amd/abi.py) has the same offsets.

A field added to skl_dense_desc, or a parameter changed in a prototype, without
the same change in the Rust file fails here.
"""
from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "soklyn_hip.h")
RUST = os.path.join(ROOT, "rust", "src", "io", "device", "hip_ffi.rs")

STRUCTS = {"skl_dense_desc": "SklDenseDesc", "skl_optimiser": "SklOptimiser", "skl_train_ctx": "SklTrainCtx"}
C_TO_RUST = {
    "uint32_t": "u32", "int32_t": "i32", "float": "f32", "size_t": "usize",
    "void*": "*mut c_void", "constvoid*": "*const c_void", "void**": "*mut *mut c_void",
    "float*": "*mut f32", "constfloat*": "*const f32", "constchar*": "*const c_char",
    "skl_ctx*": "*mut SklCtx", "skl_ctx**": "*mut *mut SklCtx",
    "constskl_dense_desc*": "*const SklDenseDesc", "constskl_train_ctx*": "*const SklTrainCtx",
    "skl_optimiser": "SklOptimiser",
}
RUST_SCALARS = {"u32": (4, 4), "i32": (4, 4), "f32": (4, 4), "usize": (8, 8)}


def strip_c_comments(txt: str) -> str:
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", txt, flags=re.S))


def norm_c_type(t: str) -> str:
    return re.sub(r"\s+", "", t)


def norm_rust_type(t: str) -> str:
    return re.sub(r"\s+", " ", t.strip())


# ---- header -----------------------------------------------------------------------------------------
def header_structs() -> dict[str, list[tuple[str, str]]]:
    txt = strip_c_comments(open(HEADER).read())
    out = {}
    for body, name in re.findall(r"typedef\s+struct\s+\w+\s*\{(.*?)\}\s*(\w+)\s*;", txt, flags=re.S):
        fields = []
        for decl in filter(None, (d.strip() for d in body.split(";"))):
            m = re.match(r"((?:const\s+)?[A-Za-z_]\w*)\s+(.*)$", decl, flags=re.S)
            base, declarators = m.group(1), m.group(2)
            for d in declarators.split(","):
                d = d.strip()
                stars = d.count("*")
                fields.append((d.replace("*", "").strip(), norm_c_type(base + "*" * stars)))
        out[name] = fields
    return out


def header_functions() -> dict[str, tuple[str, list[str]]]:
    txt = strip_c_comments(open(HEADER).read())
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w\s\*]*?)\s*\b(skl_\w+)\s*\(([^;]*?)\)\s*;", txt, flags=re.S):
        ps = []
        for p in filter(None, (q.strip() for q in params.split(","))):
            if p == "void":
                continue
            m = re.match(r"(.*?)(\w+)$", p, flags=re.S)
            ps.append(norm_c_type(m.group(1)))
        out[name] = (norm_c_type(ret.split("\n")[-1]), ps)
    return out


# ---- rust ---------------------------------------------------------------------------------------------
def rust_source() -> str:
    return re.sub(r"//[^\n]*", "", open(RUST).read())


def rust_structs() -> dict[str, list[tuple[str, str]]]:
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct (\w+)\s*\{(.*?)\}",
                                 rust_source(), flags=re.S):
        out[name] = [(f, norm_rust_type(t)) for f, t in re.findall(r"pub\s+(\w+)\s*:\s*([^,]+),", body)]
    return out


def rust_functions() -> dict[str, tuple[str, list[str]]]:
    src = rust_source()
    block = re.search(r'extern\s+"C"\s*\{(.*)\n\}', src, flags=re.S).group(1)
    out = {}
    for name, params, ret in re.findall(r"pub\s+fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        ps = [norm_rust_type(p.split(":", 1)[1]) for p in filter(None, (q.strip() for q in params.split(",")))]
        out[name] = (norm_rust_type(ret) if ret else "()", ps)
    return out


def rust_layout(structs, name):
    """repr(C): each field at the next multiple of its alignment; size rounded to the largest."""
    off, align, offsets = 0, 1, []
    for fname, t in structs[name]:
        if t in RUST_SCALARS:
            size, al = RUST_SCALARS[t]
        elif t.startswith("*"):
            size, al = 8, 8
        else:
            size, al, _ = rust_layout(structs, t)
        off = (off + al - 1) // al * al
        offsets.append((fname, off, size))
        off += size
        align = max(align, al)
    return (off + align - 1) // align * align, align, offsets


def c_layout(structs) -> dict[str, dict]:
    """sizeof / offsetof / field sizes of the header's structs, from gcc."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        pytest.skip("no C compiler")
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for s, fields in structs.items():
        lines.append(f'printf("S {s} %zu\\n", sizeof({s}));')
        for f, _ in fields:
            lines.append(f'printf("F {s} {f} %zu %zu\\n", offsetof({s}, {f}), sizeof((({s} *)0)->{f}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(src, "w").write("\n".join(lines))
        subprocess.run([cc, "-std=c99", "-Wall", "-Werror", src, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    res: dict[str, dict] = {}
    for line in out.splitlines():
        parts = line.split()
        if parts[0] == "S":
            res.setdefault(parts[1], {"fields": []})["size"] = int(parts[2])
        else:
            res.setdefault(parts[1], {"fields": []})["fields"].append((parts[2], int(parts[3]), int(parts[4])))
    return res


# ---- tests --------------------------------------------------------------------------------------------
def test_rust_declares_every_header_function_with_its_types():
    hf, rf = header_functions(), rust_functions()
    # the prototype parser saw every skl_* name the header declares
    declared = set(re.findall(r"\b(skl_[a-z0-9_]+)\s*\(", strip_c_comments(open(HEADER).read())))
    assert set(hf) == declared and len(hf) >= 24
    assert sorted(hf) == sorted(rf), f"header only: {sorted(set(hf) - set(rf))}; rust only: {sorted(set(rf) - set(hf))}"
    for name, (ret, params) in hf.items():
        rret, rparams = rf[name]
        want_ret = "()" if ret == "void" else C_TO_RUST[ret]
        assert rret == want_ret, f"{name}: returns {rret}, header {ret}"
        assert len(rparams) == len(params), f"{name}: {len(rparams)} parameters, header {len(params)}"
        for i, (c, r) in enumerate(zip(params, rparams)):
            assert C_TO_RUST[c] == r, f"{name} parameter {i}: rust {r}, header {c}"


def test_rust_structs_match_header_fields_and_types():
    hs, rs = header_structs(), rust_structs()
    for c_name, r_name in STRUCTS.items():
        assert c_name in hs and r_name in rs, (c_name, r_name)
        cf, rf = hs[c_name], rs[r_name]
        assert [f for f, _ in cf] == [f for f, _ in rf], f"{r_name}: field names / order differ from {c_name}"
        for (f, ct), (_, rt) in zip(cf, rf):
            assert C_TO_RUST[ct] == rt, f"{r_name}.{f}: rust {rt}, header {ct}"


def test_rust_repr_c_layout_equals_the_c_compilers():
    hs, rs = header_structs(), rust_structs()
    cl = c_layout({c: hs[c] for c in STRUCTS})
    for c_name, r_name in STRUCTS.items():
        size, _, offsets = rust_layout(rs, r_name)
        assert size == cl[c_name]["size"], f"{r_name}: size {size}, C sizeof {cl[c_name]['size']}"
        assert offsets == cl[c_name]["fields"], f"{r_name}: offsets differ from C"
    assert cl["skl_dense_desc"]["size"] == 12 * 4 + 28 * 8


def test_python_binding_has_the_c_offsets():
    from soklyn_amd import abi
    hs = header_structs()
    cl = c_layout({c: hs[c] for c in STRUCTS})
    for c_name, py in (("skl_dense_desc", abi.SklDenseDesc), ("skl_optimiser", abi.SklOptimiser),
                       ("skl_train_ctx", abi.SklTrainCtx)):
        assert ctypes.sizeof(py) == cl[c_name]["size"], c_name
        for f, off, size in cl[c_name]["fields"]:
            assert getattr(py, f).offset == off and getattr(py, f).size == size, f"{c_name}.{f}"


def test_checker_catches_a_field_added_to_the_header(tmp_path, monkeypatch):
    """The same checks on a copy of the header with one field inserted into
    skl_dense_desc and one parameter type changed: the Rust file no longer matches."""
    txt = open(HEADER).read()
    added = txt.replace("    uint32_t reserved0;\n", "    uint32_t reserved0;\n    uint32_t added;\n")
    retyped = txt.replace("int32_t skl_dense_input_grad(skl_ctx *ctx, const skl_dense_desc *blk, uint32_t batch, float *dx)",
                          "int32_t skl_dense_input_grad(skl_ctx *ctx, const skl_dense_desc *blk, size_t batch, float *dx)")
    assert added != txt and retyped != txt
    for variant, check, msg in ((added, test_rust_structs_match_header_fields_and_types, "field names"),
                                (retyped, test_rust_declares_every_header_function_with_its_types, "parameter 2")):
        p = tmp_path / "soklyn_hip.h"
        p.write_text(variant)
        monkeypatch.setitem(globals(), "HEADER", str(p))
        with pytest.raises(AssertionError, match=msg):
            check()
