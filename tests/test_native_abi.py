"""The C-ABI library loads and exports every declared symbol; argument
validation (which returns before any HIP call) behaves as documented.  No
compute call is made here, so these run without a GPU."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qdl_flash_born.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qdl_flash_(?:purified_)?born_\w+)\s*\(", text)))


def _header_macros():
    vals = {}
    for name, val in re.findall(r"#define\s+(QDL_BORN_\w+)\s+\(?(-?\d+)\)?", open(HEADER).read()):
        vals[name] = int(val)
    return vals


@pytest.fixture(scope="module")
def lib():
    from quantumdlblocks_amd import _native

    return _native.load()


def test_library_exports_every_declared_symbol(lib):
    from quantumdlblocks_amd import _native

    declared = _declared_functions()
    assert declared, "header parse found no functions"
    assert sorted(_native.EXPORTED_SYMBOLS) == declared
    for name in declared:
        assert getattr(lib, name) is not None


def test_constants_match_header():
    from quantumdlblocks_amd import _native

    m = _header_macros()
    assert m["QDL_BORN_DTYPE_F32"] == _native.DTYPE_F32
    assert m["QDL_BORN_DTYPE_F16"] == _native.DTYPE_F16
    assert m["QDL_BORN_DTYPE_BF16"] == _native.DTYPE_BF16
    assert m["QDL_BORN_OK"] == 0
    assert all(v < 0 for k, v in m.items() if k.startswith("QDL_BORN_E_"))


def test_version_and_errors(lib):
    assert lib.qdl_flash_born_version().decode().startswith("qdl_flash_born")
    m = _header_macros()
    for name, code in m.items():
        if name.startswith("QDL_BORN_E_"):
            assert lib.qdl_flash_born_strerror(code).decode() not in ("", "unknown error")
    assert lib.qdl_flash_born_strerror(-12345).decode() == "unknown error"


def test_supported(lib):
    from quantumdlblocks_amd import _native

    for dt in (_native.DTYPE_F32, _native.DTYPE_F16, _native.DTYPE_BF16):
        for d in (8, 16, 64, 128, 256):
            assert lib.qdl_flash_born_supported(dt, d) == 1
        for d in (0, 4, 12, 264, 1024):
            assert lib.qdl_flash_born_supported(dt, d) == 0
    assert lib.qdl_flash_born_supported(7, 64) == 0


def _fwd(lib, **over):
    a = dict(dtype=2, B=1, H=2, T=16, D=64, q=16, k=16, v=16, out=16, z=16, scale=16, n_scale=1,
             doc=None, causal=1, window=0, eps=1e-12, stream=None)
    a.update(over)
    return lib.qdl_flash_born_fwd(a["dtype"], a["B"], a["H"], a["T"], a["D"], a["q"], a["k"], a["v"],
                                  a["out"], a["z"], a["scale"], a["n_scale"], a["doc"], a["causal"],
                                  a["window"], a["eps"], a["stream"])


def test_forward_argument_validation(lib):
    """Every rejection below happens before any launch (pointers are dummies)."""
    m = _header_macros()
    assert _fwd(lib, dtype=5) == m["QDL_BORN_E_DTYPE"]
    assert _fwd(lib, B=-1) == m["QDL_BORN_E_SHAPE"]
    assert _fwd(lib, D=12) == m["QDL_BORN_E_HEADDIM"]
    assert _fwd(lib, D=264) == m["QDL_BORN_E_HEADDIM"]
    assert _fwd(lib, n_scale=3) == m["QDL_BORN_E_SCALE"]
    assert _fwd(lib, window=-2) == m["QDL_BORN_E_WINDOW"]
    assert _fwd(lib, eps=-1.0) == m["QDL_BORN_E_SHAPE"]
    assert _fwd(lib, q=None) == m["QDL_BORN_E_NULL"]
    assert _fwd(lib, q=18) == m["QDL_BORN_E_ALIGN"]
    assert _fwd(lib, T=1 << 29) == m["QDL_BORN_E_SHAPE"]
    # empty problems succeed without launching anything
    assert _fwd(lib, T=0, q=None, k=None, v=None, out=None, z=None) == 0
    assert _fwd(lib, B=0) == 0


def test_backward_argument_validation(lib):
    m = _header_macros()
    ws = lib.qdl_flash_born_bwd_workspace_size(2, 2, 3, 100, 64, 1)
    assert ws >= 2 * 2 * 3 * 100 * 4

    def bwd(**over):
        a = dict(dtype=2, B=2, H=3, T=100, D=64, ptr=16, n_scale=1, ws=16, ws_bytes=ws)
        a.update(over)
        p = a["ptr"]
        return lib.qdl_flash_born_bwd(a["dtype"], a["B"], a["H"], a["T"], a["D"], p, p, p, p, p, p, p,
                                      a["n_scale"], None, 1, 0, 1e-12, p, p, p, p, a["ws"], a["ws_bytes"], None)

    assert bwd(dtype=9) == m["QDL_BORN_E_DTYPE"]
    assert bwd(D=100) == m["QDL_BORN_E_HEADDIM"]
    assert bwd(n_scale=2) == m["QDL_BORN_E_SCALE"]
    assert bwd(ws=None) == m["QDL_BORN_E_WORKSPACE"]
    assert bwd(ws_bytes=ws - 4) == m["QDL_BORN_E_WORKSPACE"]
    assert bwd(ptr=20) == m["QDL_BORN_E_ALIGN"]


def test_qk_prologue_argument_validation(lib):
    """Rejections of the fused Q/K prologue entry points (before any launch)."""
    m = _header_macros()
    st = (ctypes.c_int64 * 3)(16 * 64 * 2, 16 * 64, 64)

    def fwd(**over):
        a = dict(dtype=2, B=1, H=2, T=16, D=64, q=16, qs=st, k=16, ks=st, cos=16, sin=16,
                 nf=32, ld=32, eps=1e-12, qo=16, ko=16, qr=16, kr=16)
        a.update(over)
        return lib.qdl_flash_born_qk_prologue_fwd(
            a["dtype"], a["B"], a["H"], a["T"], a["D"], a["q"], a["qs"], a["k"], a["ks"],
            a["cos"], a["sin"], a["nf"], a["ld"], a["eps"], a["qo"], a["ko"], a["qr"], a["kr"], None)

    def bwd(**over):
        a = dict(dtype=2, B=1, H=2, T=16, D=64, gq=16, gk=16, qo=16, ko=16, qr=16, kr=16,
                 cos=16, sin=16, nf=32, ld=32, dq=16, dqs=st, dk=16, dks=st)
        a.update(over)
        return lib.qdl_flash_born_qk_prologue_bwd(
            a["dtype"], a["B"], a["H"], a["T"], a["D"], a["gq"], a["gk"], a["qo"], a["ko"],
            a["qr"], a["kr"], a["cos"], a["sin"], a["nf"], a["ld"], a["dq"], a["dqs"], a["dk"],
            a["dks"], None)

    for call in (fwd, bwd):
        assert call(dtype=4) == m["QDL_BORN_E_DTYPE"]
        assert call(T=-1) == m["QDL_BORN_E_SHAPE"]
        assert call(D=63) == m["QDL_BORN_E_ROPEDIM"]
        assert call(D=258) == m["QDL_BORN_E_ROPEDIM"]
        assert call(D=0) == m["QDL_BORN_E_ROPEDIM"]
        assert call(nf=33) == m["QDL_BORN_E_TABLE"]
        assert call(ld=16) == m["QDL_BORN_E_TABLE"]
        assert call(sin=None) == m["QDL_BORN_E_NULL"]
        assert call(B=0) == 0  # empty: nothing to launch
    assert fwd(eps=-1.0) == m["QDL_BORN_E_SHAPE"]
    assert fwd(qo=None) == m["QDL_BORN_E_NULL"]
    # (q_rinv / k_rinv may be NULL: 1/norm not written; exercised on the GPU.)
    assert fwd(ko=None) == m["QDL_BORN_E_NULL"]
    assert fwd(qs=None) == m["QDL_BORN_E_NULL"]
    assert fwd(q=None, k=None) == 0  # neither tensor given
    assert bwd(qo=None) == m["QDL_BORN_E_NULL"]
    assert bwd(dks=None) == m["QDL_BORN_E_NULL"]
    assert bwd(gq=None, gk=None) == 0
