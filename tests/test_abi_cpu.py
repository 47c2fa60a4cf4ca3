"""CPU checks of the C-ABI library: it loads without a GPU and exports every
entry point include/soklyn_hip.h declares (no compute calls here)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from soklyn_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols() -> list[str]:
    txt = open(os.path.join(ROOT, "include", "soklyn_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(skl_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "skl_dense_forward" in names and "skl_dense_backward" in names
    assert len(names) >= 20


def test_library_loads_and_exports_every_declared_symbol():
    if not os.path.exists(abi.LIB_PATH):
        pytest.skip("libsoklyn_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(abi.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    assert sorted(abi.EXPORTED) == declared_symbols()


def test_scramble_seed_is_host_only_and_matches_oracle():
    """skl_scramble_seed runs on the host: compare with the oracle restatement."""
    if not os.path.exists(abi.LIB_PATH):
        pytest.skip("libsoklyn_hip.so not built")
    from oracle import oracle as O
    lib = abi.load()
    for step, lid in [(0, 0), (1, 5), (7, 123456), (2**32 - 1, 2**31 + 3), (1000, 27)]:
        assert lib.skl_scramble_seed(step, lid) == O.scramble_seed(step, lid)


def test_descriptor_layout_matches_header():
    """Field order / sizes of skl_dense_desc as the header lays them out (12 scalars, 28 pointers)."""
    assert ctypes.sizeof(abi.SklDenseDesc) == 12 * 4 + 28 * 8
    assert abi.SklDenseDesc.w.offset == 48
    assert abi.SklDenseDesc.d_prenorm_h.offset == 48 + 27 * 8
    assert ctypes.sizeof(abi.SklTrainCtx) == 2 * 20 + 12
