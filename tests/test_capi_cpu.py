"""CPU-side checks of the drop-in boundary: the built library loads and exports every
entry point include/jasmine_hip.h declares (no device calls are made here)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "jasmine_hip.h")
LIB = os.path.join(ROOT, "jasmine_amd", "libjasmine_hip.so")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(jas_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared()
    for must in ("jas_ew_eval", "jas_softmax", "jas_layernorm", "jas_rmsnorm", "jas_gemm", "jas_attn_prefill",
                 "jas_attn_decode", "jas_rope_jasmine", "jas_rope_llama", "jas_lm_decode"):
        assert must in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (jas_[a-z0-9_]+)", out))
    assert set(declared()) <= exported


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_binding_covers_header():
    import jasmine_amd.capi as capi
    assert set(declared()) == set(capi.EXPORTED)


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_has_no_oracle_dependency():
    # the product library never links the CPU oracle or the reference build
    out = subprocess.run(["ldd", LIB], capture_output=True, text=True).stdout
    assert "oracle" not in out and "jasref" not in out
    syms = subprocess.run(["nm", "-D", LIB], capture_output=True, text=True).stdout
    assert "orc_" not in syms and "ref_" not in syms


def test_lowering_stack_bound():
    # Sethi-Ullman ordering keeps a balanced 8-leaf tree within the 4-slot device stack
    from jasmine_amd import expr as E

    class FakeLeaf:
        vrows, vcols = 4, 4

    def lf():
        return E.Node("leaf", E.F32, 4, 4, leaf=FakeLeaf())

    t = ((lf() * lf()) + (lf() * lf())) - ((lf() / lf()) + (lf() - lf()))
    prog, leaves = E.lower(t)
    depth = mx = 0
    for op, dt, arg, imm in prog:
        if op in (0, 1):
            depth += 1
        elif op <= 7:
            depth -= 1
        mx = max(mx, depth)
    assert mx <= 4 and depth == 1 and len(leaves) == 8
    # promotion: float matrix * double scalar -> double node; float * int -> float
    assert (lf() * 0.5).dtype == E.F64 and (lf() * 2).dtype == E.F32
