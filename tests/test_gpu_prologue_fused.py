"""The Q/K prologue folded into the attention forward
(``qdl_flash_born_fwd_qk_prologue`` / ``flash_born_attention_qk_prologue``:
K through the prologue kernel, Q normalised by the attention kernel as it
loads each query block).

Bars:
  * bit for bit: the fused path (bf16, D = 64, dense or causal; with
    document ids also a causal window, on the document kernel) gives the
    same O, Z, normalised Q and K and 1/norm as the standalone prologue kernel
    on Q and K followed by the attention kernel, on
    contiguous and projection-layout inputs, full, partial and no rotary
    tables, both scale signs, per-head scales, ragged T, sorted and unsorted
    document ids and the C3 shape;
  * against the oracles: the normalised rows equal the prologue oracle's
    rounding model given the kernel's 1/norm, 1/norm within 4 ulps, and O
    within 2e-2 (normwise) of ``born_oracle.forward`` applied to the
    oracle's normalised rows, Z within its rounding bound;
  * gradients: the autograd entry gives bit-identical gradients to the
    composition ``flash_born_attention(fused_qk_rope_l2_normalize(...))``
    (the backward is the attention backward then the prologue backward);
  * other shapes (fp16, D = 32, windows without documents, documents with a
    window but no causality) take the two-launch path through the same entry
    and equal the composition.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc
from oracle import qk_prologue_oracle as po
from util import f64, rel_err, z_row_bound

pytestmark = pytest.mark.gpu


def _tables(T, n, base=1024.0):
    freqs = 1.0 / base ** (torch.arange(n, dtype=torch.float32) / max(n, 1))
    ang = torch.outer(torch.arange(T, dtype=torch.float32), freqs)
    return torch.cos(ang).view(1, 1, T, n), torch.sin(ang).view(1, 1, T, n)


def _inputs(B, H, T, D, dtype, strided, seed, dev, std=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    if strided:  # (B, T, H, D) projection output viewed as (B, H, T, D)
        q = (torch.randn(B, T, H, D, generator=g) * std).to(dtype).to(dev).transpose(1, 2)
        k = (torch.randn(B, T, H, D, generator=g) * std).to(dtype).to(dev).transpose(1, 2)
    else:
        q = (torch.randn(B, H, T, D, generator=g) * std).to(dtype).to(dev)
        k = (torch.randn(B, H, T, D, generator=g) * std).to(dtype).to(dev)
    v = torch.randn(B, H, T, D, generator=g).to(dtype).to(dev)
    do = torch.randn(B, H, T, D, generator=g).to(dtype).to(dev)
    return q, k, v, do


def _abi(fused, q, k, v, scale, cos, sin, causal=True, eps=1e-12, doc=None, window=0, rinv=True):
    """Through the C ABI: the fused entry (fused=True) or the prologue entry
    followed by the forward entry.  Returns out, z, q', k', q_rinv, k_rinv
    (rinv=False: 1/norm pointers NULL, as when no backward follows; the
    returned 1/norm buffers then hold NaN, their fill)."""
    from quantumdlblocks_amd import _native
    from quantumdlblocks_amd.kernels.flash_born import _DTYPE_CODE
    from quantumdlblocks_amd.kernels.qk_prologue import _prep_tables, _strides

    lib = _native.load()
    B, H, T, D = q.shape
    dev = q.device
    code = _DTYPE_CODE[q.dtype]
    cos2, sin2 = _prep_tables(cos, sin, D // 2, T, dev)
    tabs = (cos2.data_ptr() if cos2 is not None else None, sin2.data_ptr() if sin2 is not None else None,
            cos2.shape[1] if cos2 is not None else 0, cos2.stride(0) if cos2 is not None else 0)
    sc = torch.as_tensor(np.asarray(scale, np.float32).reshape(-1), device=dev)
    doc_t = None if doc is None else torch.as_tensor(doc, dtype=torch.int32, device=dev)
    out = torch.empty((B, H, T, D), dtype=q.dtype, device=dev)
    z = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    qo, ko = torch.empty_like(out), torch.empty_like(out)
    qr, kr = torch.full_like(z, float("nan")), torch.full_like(z, float("nan"))
    qrp, krp = (qr.data_ptr(), kr.data_ptr()) if rinv else (None, None)
    qs, ks = _strides(q), _strides(k)
    stream = torch.cuda.current_stream(dev).cuda_stream
    docp = None if doc_t is None else doc_t.data_ptr()
    if fused:
        rc = lib.qdl_flash_born_fwd_qk_prologue(code, B, H, T, D, q.data_ptr(), qs.data_ptr(), k.data_ptr(),
                                                ks.data_ptr(), v.data_ptr(), *tabs, 1e-12, sc.data_ptr(),
                                                sc.numel(), docp, int(causal), window, eps, out.data_ptr(),
                                                z.data_ptr(), qo.data_ptr(), ko.data_ptr(), qrp, krp, stream)
        _native.check(rc, "qdl_flash_born_fwd_qk_prologue")
    else:
        rc = lib.qdl_flash_born_qk_prologue_fwd(code, B, H, T, D, q.data_ptr(), qs.data_ptr(), k.data_ptr(),
                                                ks.data_ptr(), *tabs, 1e-12, qo.data_ptr(), ko.data_ptr(),
                                                qrp, krp, stream)
        _native.check(rc, "qdl_flash_born_qk_prologue_fwd")
        rc = lib.qdl_flash_born_fwd(code, B, H, T, D, qo.data_ptr(), ko.data_ptr(), v.data_ptr(), out.data_ptr(),
                                    z.data_ptr(), sc.data_ptr(), sc.numel(), docp, int(causal), window, eps, stream)
        _native.check(rc, "qdl_flash_born_fwd")
    torch.cuda.synchronize(dev)
    return out, z, qo, ko, qr, kr


def _same(a, b):
    iv = torch.int32 if a.dtype == torch.float32 else torch.int16
    return torch.equal(a.view(iv), b.view(iv))


CASES = [
    # (B, H, T, nfreq or None, strided, causal, scale)
    (2, 3, 300, 32, True, True, 8.0),
    (2, 3, 300, 32, False, True, 8.0),
    (1, 2, 1024, 20, True, True, -3.0),
    (1, 4, 777, None, True, False, 8.0),
    (2, 2, 65, 32, True, True, np.array([1.5, 9.0])),
    (1, 1, 1, 32, False, True, 8.0),
    (1, 2, 2500, 32, True, True, 8.0),
    (3, 2, 513, 7, False, False, 2.0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}-n{c[3]}-{'strided' if c[4] else 'dense'}-{'causal' if c[5] else 'full'}")
def test_fused_equals_prologue_then_attention_bitwise(cuda_device, case):
    B, H, T, nf, strided, causal, scale = case
    q, k, v, _ = _inputs(B, H, T, 64, torch.bfloat16, strided, seed=T + 3, dev=cuda_device, std=0.7)
    cos = sin = None
    if nf is not None:
        cos, sin = (x.to(cuda_device) for x in _tables(T, nf))
    print(f"fused case B{B} H{H} T{T} n={nf} strided={strided} causal={causal}", flush=True)
    a = _abi(True, q, k, v, scale, cos, sin, causal)
    b = _abi(False, q, k, v, scale, cos, sin, causal)
    for name, x, y in zip(("out", "z", "q'", "k'", "q_rinv", "k_rinv"), a, b):
        assert _same(x, y), name


DOC_CASES = [
    # (B, H, T, nfreq or None, strided, causal, window, mean document length or "unsorted", scale)
    (2, 3, 700, 32, True, True, 0, 90.0, 8.0),
    (1, 2, 1500, 20, True, False, 0, 200.0, -3.0),
    (2, 2, 513, 32, False, True, 100, 60.0, np.array([1.5, 9.0])),
    (1, 4, 777, None, True, True, 0, 50.0, 8.0),
    (1, 1, 1, 32, False, True, 0, 4.0, 8.0),
    (1, 2, 2500, 7, True, True, 256, 300.0, 8.0),
    (2, 2, 640, 32, True, True, 0, "unsorted", 8.0),
    (1, 2, 900, 32, True, True, 64, "unsorted", 2.0),
]


def _doc_ids(B, T, how, seed):
    if how == "unsorted":  # ids repeat in no order: documents are sets of positions
        return np.random.default_rng(seed).integers(0, 5, size=(B, T)).astype(np.int32)
    return orc.geometric_doc_ids(B, T, how, seed=seed)


@pytest.mark.parametrize("case", DOC_CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}-n{c[3]}-{'strided' if c[4] else 'dense'}-{'causal' if c[5] else 'full'}-W{c[6]}-{c[7]}")
def test_fused_documents_equal_prologue_then_attention_bitwise(cuda_device, case):
    """Document ids (and with them a causal window) on the document kernel
    with the Q prologue in its Q load: bit for bit against the two launches."""
    B, H, T, nf, strided, causal, window, how, scale = case
    q, k, v, _ = _inputs(B, H, T, 64, torch.bfloat16, strided, seed=T + 5, dev=cuda_device, std=0.7)
    cos = sin = None
    if nf is not None:
        cos, sin = (x.to(cuda_device) for x in _tables(T, nf))
    doc = _doc_ids(B, T, how, seed=T)
    print(f"fused documents B{B} H{H} T{T} n={nf} strided={strided} causal={causal} W={window} docs={how}",
          flush=True)
    a = _abi(True, q, k, v, scale, cos, sin, causal, doc=doc, window=window)
    b = _abi(False, q, k, v, scale, cos, sin, causal, doc=doc, window=window)
    for name, x, y in zip(("out", "z", "q'", "k'", "q_rinv", "k_rinv"), a, b):
        assert _same(x, y), name
    for fused in (True, False):  # no backward follows: O, Z and k' as with the 1/norm outputs
        part = _abi(fused, q, k, v, scale, cos, sin, causal, doc=doc, window=window, rinv=False)
        for name, i in (("out", 0), ("z", 1), ("k'", 3)):
            assert _same(part[i], a[i]), (fused, name)
        assert torch.isnan(part[4]).all() and torch.isnan(part[5]).all(), fused


def test_fused_documents_c4_shape_against_oracles(cuda_device):
    """C4's shape (B4 H16 T8192, documents of mean 512) in the projection
    layout: bit for bit against the two launches; sampled heads against the
    composition of the prologue and attention oracles."""
    B, H, T, D = 4, 16, 8192, 64
    q, k, v, _ = _inputs(B, H, T, D, torch.bfloat16, True, seed=13, dev=cuda_device)
    cos, sin = _tables(T, D // 2, base=10000.0)
    cos_np, sin_np = cos[0, 0].numpy(), sin[0, 0].numpy()
    cos, sin = cos.to(cuda_device), sin.to(cuda_device)
    doc = orc.geometric_doc_ids(B, T, 512.0, seed=3)
    a = _abi(True, q, k, v, 8.0, cos, sin, doc=doc)
    b = _abi(False, q, k, v, 8.0, cos, sin, doc=doc)
    for name, x, y in zip(("out", "z", "q'", "k'", "q_rinv", "k_rinv"), a, b):
        assert _same(x, y), name
    out, z, qo, ko, qr, kr = a
    for bb, hh in ((0, 0), (3, 15)):
        rows = slice(0, 1536)  # causal: the first 1536 rows see keys among themselves only
        qn = po.prologue_forward(q[bb, hh, rows].float().cpu().numpy(), cos_np[rows], sin_np[rows], 1e-12, "bf16")[0]
        kn = po.prologue_forward(k[bb, hh, rows].float().cpu().numpy(), cos_np[rows], sin_np[rows], 1e-12, "bf16")[0]
        vn = v[bb, hh, rows].float().cpu().numpy()
        d = doc[bb:bb + 1, rows]
        ref, zref = orc.forward(qn[None, None], kn[None, None], vn[None, None], 8.0, doc_ids=d)
        err = rel_err(f64(out[bb, hh, rows]), ref[0, 0])
        print(f"C4 fused head ({bb},{hh}): O rel {err:.3e}", flush=True)
        assert err <= 2e-2
        bound = z_row_bound(qn[None, None], kn[None, None], 8.0, zref, 1e-12, torch.bfloat16,
                            orc.visible_mask(1536, True, 0, d))
        assert np.all(np.abs(f64(z[bb, hh, rows]) - zref[0, 0]) <= bound[0, 0])


@pytest.mark.parametrize("causal", [True, False])
def test_fused_without_backward_outputs(cuda_device, causal):
    """1/norm pointers NULL (no backward follows): O and Z bit for bit as
    with them, k' still written (the attention reads it), 1/norm buffers
    untouched; the same through the two launches."""
    q, k, v, _ = _inputs(2, 3, 700, 64, torch.bfloat16, True, seed=41, dev=cuda_device, std=0.7)
    cos, sin = (x.to(cuda_device) for x in _tables(700, 32))
    full = _abi(True, q, k, v, 8.0, cos, sin, causal)
    for fused in (True, False):
        part = _abi(fused, q, k, v, 8.0, cos, sin, causal, rinv=False)
        for name, i in (("out", 0), ("z", 1), ("k'", 3)):
            assert _same(part[i], full[i]), (fused, name)
        assert torch.isnan(part[4]).all() and torch.isnan(part[5]).all(), fused
    from quantumdlblocks_amd import flash_born_attention_qk_prologue

    with torch.no_grad():
        o_ng = flash_born_attention_qk_prologue(q, k, v, 8.0, cos, sin, is_causal=causal)
    assert _same(o_ng, full[0])


def test_fused_c3_shape_bitwise_and_oracle(cuda_device):
    """C3's shape in the projection layout: bit for bit against the two
    launches; sampled heads against the composition of the oracles."""
    B, H, T, D = 16, 16, 1024, 64
    q, k, v, _ = _inputs(B, H, T, D, torch.bfloat16, True, seed=11, dev=cuda_device)
    cos, sin = _tables(T, D // 2, base=10000.0)
    cos_np, sin_np = cos[0, 0].numpy(), sin[0, 0].numpy()
    cos, sin = cos.to(cuda_device), sin.to(cuda_device)
    a = _abi(True, q, k, v, 8.0, cos, sin)
    b = _abi(False, q, k, v, 8.0, cos, sin)
    for name, x, y in zip(("out", "z", "q'", "k'", "q_rinv", "k_rinv"), a, b):
        assert _same(x, y), name
    out, z, qo, ko, qr, kr = a
    for bb, hh in ((0, 0), (15, 15), (7, 3), (9, 12)):
        for x, xo, xr in ((q, qo, qr), (k, ko, kr)):
            xn = x[bb, hh].float().cpu().numpy()
            want, want_r = po.prologue_forward(xn, cos_np, sin_np, 1e-12, "bf16")
            got_r = xr[bb, hh].cpu().numpy()
            np.testing.assert_allclose(got_r, want_r, rtol=4 * 2.0 ** -23, atol=0)
            y = po.rope(xn, cos_np, sin_np, "bf16")
            np.testing.assert_array_equal(xo[bb, hh].float().cpu().numpy(),
                                          po.round_to((y * got_r[:, None]).astype(np.float32), "bf16"))
        # attention of the oracle's normalised rows
        qn = po.prologue_forward(q[bb, hh].float().cpu().numpy(), cos_np, sin_np, 1e-12, "bf16")[0]
        kn = po.prologue_forward(k[bb, hh].float().cpu().numpy(), cos_np, sin_np, 1e-12, "bf16")[0]
        vn = v[bb, hh].float().cpu().numpy()
        ref, zref = orc.forward(qn[None, None], kn[None, None], vn[None, None], 8.0)
        err = rel_err(f64(out[bb, hh]), ref[0, 0])
        print(f"C3 fused head ({bb},{hh}): O rel {err:.3e}", flush=True)
        assert err <= 2e-2
        bound = z_row_bound(qn[None, None], kn[None, None], 8.0, zref, 1e-12, torch.bfloat16,
                            orc.visible_mask(T, True, 0))
        assert np.all(np.abs(f64(z[bb, hh]) - zref[0, 0]) <= bound[0, 0])


@pytest.mark.parametrize("strided, docs, window", [(True, False, 0), (False, False, 0), (True, True, 0),
                                                   (True, True, 80)])
def test_fused_autograd_equals_composition(cuda_device, strided, docs, window):
    from quantumdlblocks_amd import flash_born_attention, flash_born_attention_qk_prologue, fused_qk_rope_l2_normalize

    B, H, T, D = 2, 4, 333, 64
    q, k, v, do = _inputs(B, H, T, D, torch.bfloat16, strided, seed=5, dev=cuda_device)
    cos, sin = (x.to(cuda_device) for x in _tables(T, 32))
    sc = torch.tensor([2.0, -3.0, 8.0, 0.5], device=cuda_device)
    doc_t = torch.as_tensor(orc.geometric_doc_ids(B, T, 60.0, seed=2), device=cuda_device) if docs else None
    kw = dict(window_size=window, doc_ids=doc_t)

    def run(fused):
        qa, ka, va = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        s = sc.detach().clone().requires_grad_(True)
        if fused:
            out = flash_born_attention_qk_prologue(qa, ka, va, s, cos, sin, **kw)
        else:
            qn, kn = fused_qk_rope_l2_normalize(qa, ka, cos, sin)
            out = flash_born_attention(qn, kn, va, s, **kw)
        out.backward(do)
        torch.cuda.synchronize()
        return out, qa.grad, ka.grad, va.grad, s.grad

    a, b = run(True), run(False)
    for name, x, y in zip(("out", "dq", "dk", "dv", "dscale"), a, b):
        assert x.shape == y.shape and x.dtype == y.dtype, name
        assert _same(x, y), name
    assert a[1].stride() == q.stride()


@pytest.mark.parametrize("dtype, D, doc, window, causal", [
    (torch.float16, 64, False, 0, True), (torch.bfloat16, 32, False, 0, True), (torch.bfloat16, 64, True, 0, True),
    (torch.bfloat16, 64, False, 50, True), (torch.bfloat16, 64, True, 50, False), (torch.float32, 128, False, 0, True)])
def test_other_shapes_take_the_two_launch_path(cuda_device, dtype, D, doc, window, causal):
    """The entry against the composition through the public functions (the
    bf16 D = 64 document case is the fused one)."""
    from quantumdlblocks_amd import flash_born_attention, flash_born_attention_qk_prologue, fused_qk_rope_l2_normalize

    B, H, T = 2, 2, 200
    q, k, v, do = _inputs(B, H, T, D, dtype, True, seed=D, dev=cuda_device)
    cos, sin = (x.to(cuda_device) for x in _tables(T, D // 2))
    doc_t = torch.as_tensor(orc.geometric_doc_ids(B, T, 40.0, seed=1), device=cuda_device) if doc else None
    kw = dict(window_size=window, doc_ids=doc_t, is_causal=causal)
    a = flash_born_attention_qk_prologue(q, k, v, 4.0, cos, sin, **kw)
    qn, kn = fused_qk_rope_l2_normalize(q, k, cos, sin)
    b = flash_born_attention(qn, kn, v, 4.0, **kw)
    torch.cuda.synchronize()
    assert _same(a, b)
