"""GPU parity of purified-Born attention (flash_born.py:693-1341) against the
float64 oracle on the same (dtype-rounded) inputs: output, dq, dk, dv,
dscale and dtau, through the public ``flash_purified_born_attention``.

Tolerances (normwise relative error): 2e-2 for bf16 / fp16, 1e-5 for fp32
outputs (1e-4 for fp32 gradients, whose backward rounds nothing but sums in
fp32 over long rows).  Gradients that cancel to ~0 are judged against the
scale of their terms (oracle.purified_backward_magnitudes).  dscale and dtau
are compared with the oracle's value relative to the sum of their terms'
magnitudes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc
from util import TOL, f64, max_abs, rel_err, seeded_inputs

pytestmark = pytest.mark.gpu

GTOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}
FLOOR = {torch.float32: 1e-6, torch.bfloat16: 1e-4, torch.float16: 1e-4}


def _run(q, k, v, do, scale, tau, **kw):
    from quantumdlblocks_amd import flash_purified_born_attention

    q, k, v = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    sc = scale.detach().clone().requires_grad_(True)
    ta = tau.detach().clone().requires_grad_(True)
    out = flash_purified_born_attention(q, k, v, sc, ta, **kw)
    out.backward(do)
    torch.cuda.synchronize()
    return out, q.grad, k.grad, v.grad, sc.grad, ta.grad


CASES = [
    # (B, H, T, D, dtype, kwargs, scale, tau, std)
    (2, 3, 130, 64, torch.bfloat16, dict(is_causal=True), 8.0, 0.0625, 0.3),
    (1, 2, 200, 64, torch.float16, dict(is_causal=True), 8.0, 0.0625, 0.3),
    (2, 2, 97, 64, torch.float32, dict(is_causal=True), 8.0, 0.0625, 0.3),
    (1, 4, 150, 128, torch.bfloat16, dict(is_causal=False), [4.0, 6.0, 8.0, 2.0], [0.0, 0.1, -0.1, 0.05], 0.2),
    (2, 2, 120, 24, torch.bfloat16, dict(is_causal=True, window_size=17), 8.0, [0.1, -0.05], 0.5),
    (1, 2, 64, 256, torch.float32, dict(is_causal=True), 3.0, 0.0, 0.1),
    (2, 2, 160, 64, torch.bfloat16, dict(is_causal=True, eps_base=0.2, eps=1e-6), [8.0, 5.0], 0.0625, 0.3),
    (1, 1, 1, 64, torch.bfloat16, dict(is_causal=True), 8.0, 0.0625, 0.3),
    (1, 2, 33, 32, torch.float32, dict(is_causal=False, window_size=5), 2.0, -0.3, 0.4),
]


def _check_pur(case, dev, doc=None):
    B, H, T, D, dtype, kw, scale, tau, std = case
    q, k, v, do = (x.to(dev) for x in seeded_inputs((B, H, T, D), seed=T + D, std=std, n=4, dtype=dtype))
    sc = torch.tensor(np.asarray(scale, dtype=np.float32), device=dev)
    ta = torch.tensor(np.asarray(tau, dtype=np.float32), device=dev)
    print(f"purified B{B} H{H} T{T} D{D} {dtype} {kw} doc={doc is not None}", flush=True)
    doc_t = None if doc is None else torch.as_tensor(doc, dtype=torch.int32, device=dev)
    out, dq, dk, dv, dsc, dta = _run(q, k, v, do, sc, ta, doc_ids=doc_t, **kw)
    assert out.dtype == dtype and dq.dtype == dtype
    assert dsc.shape == sc.shape and dta.shape == ta.shape
    okw = dict(eps_base=kw.get("eps_base", 0.05), is_causal=kw.get("is_causal", True), eps=kw.get("eps", 1e-8),
               window_size=kw.get("window_size", 0), doc_ids=doc)
    O_ref, _ = orc.purified_forward(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau), **okw)
    e = rel_err(f64(out), O_ref)
    assert e <= TOL[dtype], f"output rel err {e:.3e} (max abs {max_abs(f64(out), O_ref):.3e})"
    ref = orc.purified_backward(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau), f64(do), **okw)
    mag = orc.purified_backward_magnitudes(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau),
                                           f64(do), **okw)
    for name, got, want, m in zip(("dq", "dk", "dv"), (dq, dk, dv), ref[:3], mag[:3]):
        er = rel_err(f64(got), want)
        ef = max_abs(f64(got), want) / m.max() if m.max() > 0 else max_abs(f64(got), want)
        assert er <= GTOL[dtype] or ef <= FLOOR[dtype], f"{name}: rel {er:.3e}, vs term scale {ef:.3e}"
    # dscale / dtau: against the oracle, within the tolerance of their value or
    # the floor of the magnitude of the terms they sum (they can cancel).
    for name, got, want, m in (("dscale", dsc, ref[3], mag[3]), ("dtau", dta, ref[4], mag[4])):
        got = np.atleast_1d(f64(got))
        err = np.abs(got - want)
        ok = (err <= GTOL[dtype] * np.abs(want)) | (err <= FLOOR[dtype] * m)
        assert ok.all(), f"{name}: {got} vs {want} (term scale {m})"


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}D{c[3]}-{str(c[4])[6:]}")
def test_purified_forward_backward(cuda_device, case):
    _check_pur(case, cuda_device)


F16_MODES = [dict(is_causal=True), dict(is_causal=False), dict(is_causal=True, window_size=100),
             dict(is_causal=False, window_size=100)]


@pytest.mark.parametrize("D", [64, 32, 128, 96])
@pytest.mark.parametrize("kw", F16_MODES, ids=lambda kw: f"causal{int(kw['is_causal'])}-W{kw.get('window_size', 0)}")
def test_purified_f16_backward_fast(cuda_device, D, kw):
    """fp16 purified gradients on the 16-bit-MFMA backward kernels (the
    reference rounds p/Z and dR to fp16 before its dots, flash_born.py:926,
    939, 1058, as these kernels do), after the 16-bit-MFMA forward.  D = 64
    and 128, and 32 / 96 with zero columns; dense,
    causal and windows with and without causality; tau < 0, per-head gamma
    and tau, T not a multiple of the tile."""
    _check_pur((2, 2, 700, D, torch.float16, kw, [8.0, 5.0], [-0.05, 0.1], 0.25), cuda_device)


@pytest.mark.parametrize("D", [64, 32, 128, 96])
@pytest.mark.parametrize("mode", ["causal", "dense", "window", "window_nc", "docs", "docs_window", "v_subnormal"])
def test_purified_f16_forward_fast(cuda_device, D, mode):
    """fp16 purified forward on the 16-bit-MFMA kernels: the overlap on the
    fp16 MFMA (exact products, fp32 sums, as the reference's fp16 dot), the
    fp32 weights split into two bf16 terms and V split exactly into two bf16
    terms, so P.V keeps ~16 bits of each product (the reference's is an fp32
    dot): O and Z held to the float64 oracle to 1e-4.  Documents on the D =
    64 document kernel and the D = 128 kernel's document mode (at D = 32 and
    96 on the fp32-MFMA kernels, held to the same bar); V scaled into fp16's
    subnormal range for the split's low end."""
    B, H, T = 2, 2, 700
    print(f"purified f16 forward D{D} {mode}", flush=True)
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=D + 41, std=0.25, n=3,
                                                       dtype=torch.float16))
    if mode == "v_subnormal":
        v = (v.float() * 2.0 ** -18).to(torch.float16)
    causal = mode not in ("dense", "window_nc")
    window = {"window": 100, "window_nc": 100, "docs_window": 150}.get(mode, 0)
    doc = orc.geometric_doc_ids(B, T, 90.0, seed=D) if mode.startswith("docs") else None
    doc_t = None if doc is None else torch.tensor(doc, dtype=torch.int32, device=cuda_device)
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    o32, z32 = _pur_fwd_abi(q, k, v, scale, tau, 0.05, causal, 1e-8, doc=doc_t, window=window)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, causal,
                                        1e-8, window, doc)
    assert rel_err(f64(o32), O_ref) <= 1e-4, rel_err(f64(o32), O_ref)
    assert np.max(np.abs(f64(z32) - Z_ref) / Z_ref) <= 1e-4


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [1, 37, 129])
@pytest.mark.parametrize("kw", [dict(is_causal=False), dict(is_causal=False, window_size=3)],
                         ids=lambda kw: f"W{kw.get('window_size', 0)}")
def test_purified_ragged_16bit(cuda_device, D, dtype, T, kw):
    """16-bit purified attention on short and ragged lengths (one partial
    tile; the keys past T weigh zero though their overlap is zero), dense and
    with a non-causal window, on the D = 64, D = 128 and generic kernels."""
    _check_pur((1, 2, T, D, dtype, kw, [8.0, 5.0], [-0.05, 0.1], 0.25), cuda_device)


WIDE_MODES = ["causal", "dense", "window", "window_nc", "docs"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [136, 160, 192, 224, 256])
@pytest.mark.parametrize("mode", WIDE_MODES)
def test_purified_wide_head_dims(cuda_device, dtype, D, mode):
    """16-bit purified attention above head dim 128: without documents the
    wide-row DMA-ring kernels' purified mode (born_fwd_d256.h,
    born_bwd_d256.h; D < 256 with zero columns), with documents the generic
    16-bit-MFMA kernels' purified mode (masks as runtime flags; the 192-256
    dK/dV split in two column halves, of which the first writes the dgamma /
    dtau partials): forward (fp32 output, split weights) and Z against the
    oracle to 1e-4, gradients, dgamma and dtau to the 16-bit bars; tau < 0,
    per-head gamma and tau, T not a multiple of the tiles."""
    B, H, T = 1, 2, 300
    print(f"purified wide D{D} {dtype} {mode}", flush=True)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=D + 7, std=0.15, n=4, dtype=dtype))
    causal = mode not in ("dense", "window_nc")
    window = 70 if mode in ("window", "window_nc") else 0
    doc = orc.geometric_doc_ids(B, T, 60.0, seed=D) if mode == "docs" else None
    doc_t = None if doc is None else torch.tensor(doc, dtype=torch.int32, device=cuda_device)
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    o32, z32 = _pur_fwd_abi(q, k, v, scale, tau, 0.05, causal, 1e-8, doc=doc_t, window=window)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, causal,
                                        1e-8, window, doc)
    assert rel_err(f64(o32), O_ref) <= 1e-4, rel_err(f64(o32), O_ref)
    assert np.max(np.abs(f64(z32) - Z_ref) / Z_ref) <= 1e-4
    _check_pur((B, H, T, D, dtype, dict(is_causal=causal, window_size=window), scale, tau, 0.15), cuda_device, doc)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [200, 256])
@pytest.mark.parametrize("kw", [dict(is_causal=True), dict(is_causal=False), dict(is_causal=True, window_size=200),
                                dict(is_causal=False, window_size=129)],
                         ids=lambda kw: f"causal{int(kw['is_causal'])}-W{kw.get('window_size', 0)}")
def test_purified_wide_dma_kernels_long(cuda_device, dtype, D, kw):
    """The wide-row kernels' purified mode over several 128-row blocks and
    64-key tiles (T = 700: a partial last tile and block), causal, dense and
    windows with and without causality; per-head gamma and tau (one tau < 0),
    forward against the oracle to 1e-4, gradients, dgamma and dtau."""
    B, H, T = 1, 2, 700
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=D + 11, std=0.15, dtype=dtype))
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    causal, window = kw["is_causal"], kw.get("window_size", 0)
    o32, z32 = _pur_fwd_abi(q, k, v, scale, tau, 0.05, causal, 1e-8, window=window)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, causal,
                                        1e-8, window, None)
    assert rel_err(f64(o32), O_ref) <= 1e-4, rel_err(f64(o32), O_ref)
    assert np.max(np.abs(f64(z32) - Z_ref) / Z_ref) <= 1e-4
    _check_pur((B, H, T, D, dtype, kw, scale, tau, 0.15), cuda_device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [96, 200, 256])
@pytest.mark.parametrize("kw", [dict(is_causal=True), dict(is_causal=False), dict(is_causal=True, window_size=120)],
                         ids=lambda kw: f"causal{int(kw['is_causal'])}-W{kw.get('window_size', 0)}")
def test_purified_wide_documents(cuda_device, dtype, D, kw):
    """Purified attention with documents off D = 64 and 128: the wide-row
    kernels' purified document mode (200, 256) and the D = 128 kernels' with
    zero columns (96); weights masked through a per-lane bit mask, T = 700
    with documents of mean length 90, tau < 0 on one head: forward against
    the oracle to 1e-4, gradients, dgamma and dtau."""
    B, H, T = 1, 2, 700
    doc = orc.geometric_doc_ids(B, T, 90.0, seed=D)
    doc_t = torch.tensor(doc, dtype=torch.int32, device=cuda_device)
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=D + 13, std=0.15, dtype=dtype))
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    causal, window = kw["is_causal"], kw.get("window_size", 0)
    o32, z32 = _pur_fwd_abi(q, k, v, scale, tau, 0.05, causal, 1e-8, doc=doc_t, window=window)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, causal,
                                        1e-8, window, doc)
    assert rel_err(f64(o32), O_ref) <= 1e-4, rel_err(f64(o32), O_ref)
    assert np.max(np.abs(f64(z32) - Z_ref) / Z_ref) <= 1e-4
    _check_pur((B, H, T, D, dtype, kw, scale, tau, 0.15), cuda_device, doc)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kw", [dict(is_causal=True), dict(is_causal=False), dict(is_causal=True, window_size=150)],
                         ids=lambda kw: f"causal{int(kw['is_causal'])}-W{kw.get('window_size', 0)}")
def test_purified_f16_documents_backward_fast(cuda_device, D, kw):
    """fp16 purified gradients with document ids on the document variants of
    the 16-bit-MFMA backward kernels."""
    doc = orc.geometric_doc_ids(2, 700, 90.0, seed=D)
    _check_pur((2, 2, 700, D, torch.float16, kw, [8.0, 5.0], [-0.05, 0.1], 0.25), cuda_device, doc)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 96, 128, 200, 256])
@pytest.mark.parametrize("is_causal", [True, False])
def test_purified_unsorted_document_ids(cuda_device, dtype, D, is_causal):
    """Arbitrary (unsorted, repeating) document ids, tau < 0 (masked pairs
    would weigh relu(-gamma tau) > 0): the span of tiles each block visits,
    from document-id ranges, must keep every tile with a visible pair."""
    rng = np.random.default_rng(D + 2)
    doc = rng.integers(0, 4, size=(2, 500)).astype(np.int32)
    doc[1, 250:] = rng.integers(10, 12, size=250)
    _check_pur((2, 2, 500, D, dtype, dict(is_causal=is_causal), 8.0, -0.05, 0.3), cuda_device, doc)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("is_causal", [True, False])
def test_purified_document_tile_edges(cuda_device, dtype, D, is_causal):
    """Sorted documents with edges on and next to the 32- and 64-row tile
    edges, one-token documents, negative ids, one batch row in descending
    order, and tau < 0."""
    lens = [64, 1, 63, 129, 32, 1, 1, 31, 97, 65, 12, 33, 256, 3]
    ids = np.concatenate([np.full(n, i - 3, np.int32) for i, n in enumerate(lens)])
    doc = np.stack([ids, -ids[::-1]])
    _check_pur((2, 2, ids.size, D, dtype, dict(is_causal=is_causal), [8.0, 4.0], [-0.05, 0.1], 0.3), cuda_device,
               doc)


def test_purified_documents_many_tiles(cuda_device):
    """Sorted documents over more candidate tiles than a block has threads
    (fp32, D = 256), so the span's screening loop strides."""
    doc = orc.geometric_doc_ids(1, 4500, 400.0, seed=4)
    _check_pur((1, 1, 4500, 256, torch.float32, dict(is_causal=True), 3.0, 0.0, 0.1), cuda_device, doc)


def test_purified_documents(cuda_device):
    B, H, T, D = 2, 2, 300, 64
    dtype = torch.bfloat16
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=7, std=0.3, n=4, dtype=dtype))
    docs = orc.geometric_doc_ids(B, T, 40.0, seed=3)
    doc_t = torch.tensor(docs, dtype=torch.int32, device=cuda_device)
    sc = torch.tensor(8.0, device=cuda_device)
    ta = torch.tensor(0.0625, device=cuda_device)
    out, dq, dk, dv, dsc, dta = _run(q, k, v, do, sc, ta, is_causal=True, doc_ids=doc_t)
    O_ref, _ = orc.purified_forward(f64(q), f64(k), f64(v), 8.0, 0.0625, 0.05, True, 1e-8, 0, docs)
    assert rel_err(f64(out), O_ref) <= 2e-2
    ref = orc.purified_backward(f64(q), f64(k), f64(v), 8.0, 0.0625, f64(do), 0.05, True, 1e-8, 0, docs)
    for got, want in zip((dq, dk, dv), ref[:3]):
        assert rel_err(f64(got), want) <= 2e-2
    assert abs(float(dsc) - ref[3][0]) <= 2e-2 * abs(ref[3][0]) + 1e-12
    assert abs(float(dta) - ref[4][0]) <= 2e-2 * abs(ref[4][0]) + 1e-12


def test_purified_deterministic_and_default_args(cuda_device):
    from quantumdlblocks_amd import flash_purified_born_attention

    q, k, v = (x.to(cuda_device) for x in seeded_inputs((2, 4, 257, 64), seed=11, std=0.3, n=3, dtype=torch.bfloat16))
    a = flash_purified_born_attention(q, k, v)  # gamma 8, tau 0.0625, eps_base 0.05, eps 1e-8, causal
    b = flash_purified_born_attention(q, k, v, gamma_h=8.0, tau_h=0.0625, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    O_ref, _ = orc.purified_forward(f64(q), f64(k), f64(v), 8.0, 0.0625, 0.05, True, 1e-8)
    assert rel_err(f64(a), O_ref) <= 2e-2


# ---------------------------------------------------------------------------
# The bf16 D = 64 forward (dense or causal, no window / documents) runs the
# bf16-MFMA kernel with each weight split into two bf16 terms.  Its error is
# that of fp32 accumulation (the split keeps ~16 bits of every weight), so it
# is held to 1e-4 against the float64 oracle on the same bf16 inputs (not just
# the 2e-2 bf16 bar), and to the fp32-MFMA kernel, which the same inputs reach
# through an all-zero document id tensor (one document: the same visibility).
# ---------------------------------------------------------------------------
FAST_CASES = [
    # (B, H, T, causal, scale, tau, eps_base, eps, std)
    (2, 3, 130, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (1, 2, 200, False, 8.0, -0.1, 0.05, 1e-8, 0.3),   # dense, T % 64 != 0, tau < 0: keys past T masked
    (2, 2, 64, False, [4.0, 9.0], [0.0, 0.2], 0.2, 1e-6, 0.3),
    (1, 1, 1, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (1, 2, 600, True, [8.0, 5.0], [-0.05, 0.1], 0.05, 1e-8, 0.2),
    (1, 1, 1000, False, 8.0, -0.2, 0.05, 1e-8, 0.2),
]


def _pur_fwd_abi(q, k, v, scale, tau, eps_base, causal, eps, doc=None, window=0):
    from quantumdlblocks_amd import _native
    from quantumdlblocks_amd.kernels.flash_born import _DTYPE_CODE

    lib = _native.load()
    B, H, T, D = q.shape
    out = torch.empty((B, H, T, D), dtype=torch.float32, device=q.device)
    z = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    sc = torch.tensor(np.atleast_1d(np.asarray(scale, dtype=np.float32)), device=q.device)
    ta = torch.tensor(np.atleast_1d(np.asarray(tau, dtype=np.float32)), device=q.device)
    rc = lib.qdl_flash_purified_born_fwd(
        _DTYPE_CODE[q.dtype], B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), z.data_ptr(),
        sc.data_ptr(), sc.numel(), ta.data_ptr(), ta.numel(), float(eps_base),
        doc.data_ptr() if doc is not None else None, int(causal), int(window), float(eps),
        torch.cuda.current_stream(q.device).cuda_stream)
    _native.check(rc, "qdl_flash_purified_born_fwd")
    torch.cuda.synchronize()
    return out, z


@pytest.mark.parametrize("case", FAST_CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}-{'causal' if c[3] else 'dense'}")
def test_purified_fast_forward(cuda_device, case):
    B, H, T, causal, scale, tau, eps_base, eps, std = case
    print(f"purified fast fwd case B{B} H{H} T{T} causal={causal}", flush=True)
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 64), seed=T + 5, std=std, n=3,
                                                          dtype=torch.bfloat16))
    out, z = _pur_fwd_abi(q, k, v, scale, tau, eps_base, causal, eps)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau),
                                        eps_base, causal, eps)
    assert rel_err(f64(out), O_ref) <= 1e-4, rel_err(f64(out), O_ref)
    assert np.max(np.abs(f64(z) - Z_ref) / Z_ref) <= 1e-4
    zero_doc = torch.zeros((B, T), dtype=torch.int32, device=cuda_device)
    out_g, z_g = _pur_fwd_abi(q, k, v, scale, tau, eps_base, causal, eps, doc=zero_doc)
    assert rel_err(f64(out), f64(out_g)) <= 1e-4
    assert np.max(np.abs(f64(z) - f64(z_g)) / f64(z_g)) <= 1e-4


# bf16, D = 128, dense or causal: the D = 128 forward kernel's purified mode
# (eight waves on 256 query rows); ragged T around its 256-row blocks and 64-key
# tiles, and shapes with enough heads for two query blocks per workgroup.
D128_CASES = [
    # (B, H, T, causal, scale, tau, eps_base, eps, std)
    (1, 1, 1, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (2, 3, 130, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (1, 2, 200, False, 8.0, -0.1, 0.05, 1e-8, 0.3),
    (2, 2, 256, False, [4.0, 9.0], [0.0, 0.2], 0.2, 1e-6, 0.3),
    (1, 2, 300, True, [8.0, 5.0], [-0.05, 0.1], 0.05, 1e-8, 0.2),
    (1, 1, 777, False, 8.0, -0.2, 0.05, 1e-8, 0.2),
    (1, 2, 1100, True, 8.0, 0.0625, 0.05, 1e-8, 0.15),
    (4, 32, 700, True, 8.0, -0.05, 0.05, 1e-8, 0.15),
    (4, 32, 1100, False, 6.0, 0.0625, 0.05, 1e-8, 0.15),
    (2, 64, 1024, False, 6.0, -0.05, 0.05, 1e-8, 0.15),  # dense, paired
]


@pytest.mark.parametrize("case", D128_CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}-{'causal' if c[3] else 'dense'}")
def test_purified_d128_forward(cuda_device, case):
    B, H, T, causal, scale, tau, eps_base, eps, std = case
    print(f"purified d128 fwd case B{B} H{H} T{T} causal={causal}", flush=True)
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 128), seed=T + 11, std=std, n=3,
                                                          dtype=torch.bfloat16))
    out, z = _pur_fwd_abi(q, k, v, scale, tau, eps_base, causal, eps)
    heads = [(0, 0), (B - 1, H - 1), (B // 2, H // 3)] if B * H > 8 else [(b, h) for b in range(B) for h in range(H)]
    sc, ta = np.atleast_1d(scale), np.atleast_1d(tau)
    for b, h in heads:
        sl = (slice(b, b + 1), slice(h, h + 1))
        O_ref, Z_ref = orc.purified_forward(f64(q[sl]), f64(k[sl]), f64(v[sl]), sc[h % sc.size], ta[h % ta.size],
                                            eps_base, causal, eps)
        assert rel_err(f64(out[sl]), O_ref) <= 1e-4, (b, h, rel_err(f64(out[sl]), O_ref))
        assert np.max(np.abs(f64(z[sl]) - Z_ref) / Z_ref) <= 1e-4, (b, h)
    # The same call through the fp32-MFMA kernels (an all-zero document id
    # tensor: the same visibility).
    zero_doc = torch.zeros((B, T), dtype=torch.int32, device=cuda_device)
    out_g, z_g = _pur_fwd_abi(q, k, v, scale, tau, eps_base, causal, eps, doc=zero_doc)
    assert rel_err(f64(out), f64(out_g)) <= 1e-4
    assert np.max(np.abs(f64(z) - f64(z_g)) / f64(z_g)) <= 1e-4


@pytest.mark.parametrize("D", [8, 24, 32, 56, 72, 96, 120])
@pytest.mark.parametrize("causal", [True, False])
def test_purified_padded_head_dims(cuda_device, D, causal):
    """bf16 head dims below 64 run the D = 64 purified kernels, 64 < D < 128
    the D = 128 ones, with the columns past D zero: forward against the
    oracle to 1e-4, gradients, dgamma and dtau against the oracle and the
    fp32-MFMA kernels (through a window longer than T), tau < 0 with T not a
    multiple of 64."""
    B, H, T = 1, 2, 333
    print(f"purified padded D{D} causal={causal}", flush=True)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=D + 17, std=0.25, n=4,
                                                              dtype=torch.bfloat16))
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    out, z = _pur_fwd_abi(q, k, v, scale, tau, 0.05, causal, 1e-8)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, causal,
                                        1e-8)
    assert rel_err(f64(out), O_ref) <= 1e-4, rel_err(f64(out), O_ref)
    assert np.max(np.abs(f64(z) - Z_ref) / Z_ref) <= 1e-4
    sc = torch.tensor(np.asarray(scale, dtype=np.float32), device=cuda_device)
    ta = torch.tensor(np.asarray(tau, dtype=np.float32), device=cuda_device)
    kw = dict(eps_base=0.05, is_causal=causal, eps=1e-8)
    fast = _run(q, k, v, do, sc, ta, **kw)
    generic = _run(q, k, v, do, sc, ta, window_size=T + 1, **kw)
    ref = orc.purified_backward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do), **kw)
    mag = orc.purified_backward_magnitudes(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do),
                                           **kw)
    for i, name in enumerate(("dq", "dk", "dv")):
        got, gen, want, m = f64(fast[1 + i]), f64(generic[1 + i]), ref[i], mag[i]
        ef = max_abs(got, want) / m.max()
        assert rel_err(got, want) <= 2e-2 or ef <= 1e-4, (name, rel_err(got, want), ef)
        assert rel_err(got, gen) <= 5e-3 or max_abs(got, gen) / m.max() <= 1e-4, (name, rel_err(got, gen))
    for name, got, gen, want, m in (("dscale", fast[4], generic[4], ref[3], mag[3]),
                                    ("dtau", fast[5], generic[5], ref[4], mag[4])):
        got, gen = np.atleast_1d(f64(got)), np.atleast_1d(f64(gen))
        ok = (np.abs(got - want) <= 2e-2 * np.abs(want)) | (np.abs(got - want) <= 1e-4 * m)
        assert ok.all(), (name, got, want, m)
        ok = (np.abs(got - gen) <= 5e-3 * np.abs(gen)) | (np.abs(got - gen) <= 1e-4 * m)
        assert ok.all(), (name, got, gen)


@pytest.mark.parametrize("causal", [True, False])
def test_purified_d128_documents(cuda_device, causal):
    """bf16, D = 128 with document ids: the D = 128 kernels' purified
    document mode; tau < 0 (masked pairs weigh zero only if zeroed), T not a
    multiple of the tile or block, per-head gamma and tau; forward (fp32
    output) against the oracle and the fp32-MFMA kernels to 1e-4, gradients,
    dgamma and dtau against both to the bf16 bars."""
    B, H, T, D = 2, 2, 1100, 128
    print(f"purified d128 documents causal={causal}", flush=True)
    docs = orc.geometric_doc_ids(B, T, 90.0, seed=5)
    doc_t = torch.tensor(docs, dtype=torch.int32, device=cuda_device)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=23, std=0.2, n=4,
                                                              dtype=torch.bfloat16))
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    o32, z32 = _pur_fwd_abi(q, k, v, scale, tau, 0.05, causal, 1e-8, doc=doc_t)
    o32g, z32g = _pur_fwd_abi(q, k, v, scale, tau, 0.05, causal, 1e-8, doc=doc_t, window=T + 1)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, causal,
                                        1e-8, 0, docs)
    assert rel_err(f64(o32), O_ref) <= 1e-4, rel_err(f64(o32), O_ref)
    assert rel_err(f64(o32), f64(o32g)) <= 1e-4
    assert np.max(np.abs(f64(z32) - Z_ref) / Z_ref) <= 1e-4
    sc = torch.tensor(np.asarray(scale, dtype=np.float32), device=cuda_device)
    ta = torch.tensor(np.asarray(tau, dtype=np.float32), device=cuda_device)
    kw = dict(eps_base=0.05, is_causal=causal, eps=1e-8)
    fast = _run(q, k, v, do, sc, ta, doc_ids=doc_t, **kw)
    generic = _run(q, k, v, do, sc, ta, doc_ids=doc_t, window_size=T + 1, **kw)
    okw = dict(kw, window_size=0, doc_ids=docs)
    ref = orc.purified_backward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do), **okw)
    mag = orc.purified_backward_magnitudes(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do),
                                           **okw)
    for i, name in enumerate(("dq", "dk", "dv")):
        got, gen, want, m = f64(fast[1 + i]), f64(generic[1 + i]), ref[i], mag[i]
        assert rel_err(got, want) <= 2e-2 or max_abs(got, want) / m.max() <= 1e-4, (name, rel_err(got, want))
        assert rel_err(got, gen) <= 5e-3 or max_abs(got, gen) / m.max() <= 1e-4, (name, rel_err(got, gen))
    for name, got, gen, want, m in (("dscale", fast[4], generic[4], ref[3], mag[3]),
                                    ("dtau", fast[5], generic[5], ref[4], mag[4])):
        got, gen = np.atleast_1d(f64(got)), np.atleast_1d(f64(gen))
        ok = (np.abs(got - want) <= 2e-2 * np.abs(want)) | (np.abs(got - want) <= 1e-4 * m)
        assert ok.all(), (name, got, want, m)
        ok = (np.abs(got - gen) <= 5e-3 * np.abs(gen)) | (np.abs(got - gen) <= 1e-4 * m)
        assert ok.all(), (name, got, gen)


@pytest.mark.parametrize("D", [64, 32, 128, 96])
@pytest.mark.parametrize("window", [1, 33, 100, 300, 2000])
@pytest.mark.parametrize("docs", [False, True])
def test_purified_window_fast(cuda_device, D, window, docs):
    """bf16 purified attention with a causal sliding window (the wavelet
    models' purified layers pass one, with document ids): the D = 64 and
    D = 128 kernels' window mode (D = 32 and 96 with zero columns), and their
    document modes with a window; tau < 0, per-head gamma and tau.  Forward
    (fp32 output) against the oracle to 1e-4; gradients, dgamma and dtau to
    the bf16 bars.  With documents at D = 32 and 96 the calls take the
    fp32-MFMA purified kernels (the document modes of the bf16-MFMA kernels
    are built for D = 64 and 128), held to the same bars."""
    B, H, T = 2, 2, 700
    print(f"purified window D{D} W{window} docs={docs}", flush=True)
    doc = orc.geometric_doc_ids(B, T, 120.0, seed=window) if docs else None
    doc_t = None if doc is None else torch.tensor(doc, dtype=torch.int32, device=cuda_device)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=window + D, std=0.25, n=4,
                                                              dtype=torch.bfloat16))
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    o32, z32 = _pur_fwd_abi(q, k, v, scale, tau, 0.05, True, 1e-8, doc=doc_t, window=window)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, True,
                                        1e-8, window, doc)
    assert rel_err(f64(o32), O_ref) <= 1e-4, rel_err(f64(o32), O_ref)
    assert np.max(np.abs(f64(z32) - Z_ref) / Z_ref) <= 1e-4
    sc = torch.tensor(np.asarray(scale, dtype=np.float32), device=cuda_device)
    ta = torch.tensor(np.asarray(tau, dtype=np.float32), device=cuda_device)
    fast = _run(q, k, v, do, sc, ta, eps_base=0.05, is_causal=True, eps=1e-8, window_size=window, doc_ids=doc_t)
    okw = dict(eps_base=0.05, is_causal=True, eps=1e-8, window_size=window, doc_ids=doc)
    ref = orc.purified_backward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do), **okw)
    mag = orc.purified_backward_magnitudes(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do),
                                           **okw)
    for i, name in enumerate(("dq", "dk", "dv")):
        got, want, m = f64(fast[1 + i]), ref[i], mag[i]
        assert rel_err(got, want) <= 2e-2 or max_abs(got, want) / m.max() <= 1e-4, (name, rel_err(got, want))
    for name, got, want, m in (("dscale", fast[4], ref[3], mag[3]), ("dtau", fast[5], ref[4], mag[4])):
        got = np.atleast_1d(f64(got))
        ok = (np.abs(got - want) <= 2e-2 * np.abs(want)) | (np.abs(got - want) <= 1e-4 * m)
        assert ok.all(), (name, got, want, m)


@pytest.mark.parametrize("D", [64, 32, 128, 96])
@pytest.mark.parametrize("window", [1, 33, 100, 300, 2000])
def test_purified_window_noncausal_fast(cuda_device, D, window):
    """bf16 purified attention with a sliding window and no causality: the
    D = 64 and D = 128 kernels' kWindowNC mode (D = 32 and 96 with zero
    columns); tau < 0 (a
    masked pair with a zero overlap still weighs relu(-gamma tau)^4, so the
    window's edge and the keys past T are zeroed per weight), per-head gamma
    and tau, T not a multiple of the tile.  Forward (fp32 output) against the
    oracle to 1e-4; gradients, dgamma and dtau to the bf16 bars."""
    B, H, T = 2, 2, 700
    print(f"purified non-causal window D{D} W{window}", flush=True)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=window + D + 3, std=0.25, n=4,
                                                              dtype=torch.bfloat16))
    scale, tau = [8.0, 5.0], [-0.05, 0.1]
    o32, z32 = _pur_fwd_abi(q, k, v, scale, tau, 0.05, False, 1e-8, window=window)
    O_ref, Z_ref = orc.purified_forward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), 0.05, False,
                                        1e-8, window)
    assert rel_err(f64(o32), O_ref) <= 1e-4, rel_err(f64(o32), O_ref)
    assert np.max(np.abs(f64(z32) - Z_ref) / Z_ref) <= 1e-4
    sc = torch.tensor(np.asarray(scale, dtype=np.float32), device=cuda_device)
    ta = torch.tensor(np.asarray(tau, dtype=np.float32), device=cuda_device)
    fast = _run(q, k, v, do, sc, ta, eps_base=0.05, is_causal=False, eps=1e-8, window_size=window)
    okw = dict(eps_base=0.05, is_causal=False, eps=1e-8, window_size=window)
    ref = orc.purified_backward(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do), **okw)
    mag = orc.purified_backward_magnitudes(f64(q), f64(k), f64(v), np.asarray(scale), np.asarray(tau), f64(do),
                                           **okw)
    for i, name in enumerate(("dq", "dk", "dv")):
        got, want, m = f64(fast[1 + i]), ref[i], mag[i]
        assert rel_err(got, want) <= 2e-2 or max_abs(got, want) / m.max() <= 1e-4, (name, rel_err(got, want))
    for name, got, want, m in (("dscale", fast[4], ref[3], mag[3]), ("dtau", fast[5], ref[4], mag[4])):
        got = np.atleast_1d(f64(got))
        ok = (np.abs(got - want) <= 2e-2 * np.abs(want)) | (np.abs(got - want) <= 1e-4 * m)
        assert ok.all(), (name, got, want, m)


def test_purified_d128_window_paired_launch(cuda_device):
    """Head dim 128 with a causal window on a grid of 256 block pairs
    (B4 H16 T2048, window 384: the launch pairs blocks nmb-1-mb and mb);
    sampled heads against the oracle, fp32 output to 1e-4."""
    B, H, T, D, W = 4, 16, 2048, 128, 384
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=11, std=0.125, n=3,
                                                          dtype=torch.bfloat16))
    out, z = _pur_fwd_abi(q, k, v, 8.0, 0.0625, 0.05, True, 1e-8, window=W)
    for b, h in ((0, 0), (1, 7), (3, 15), (2, 10)):
        O_ref, Z_ref = orc.purified_forward(f64(q[b:b + 1, h:h + 1]), f64(k[b:b + 1, h:h + 1]),
                                            f64(v[b:b + 1, h:h + 1]), 8.0, 0.0625, 0.05, True, 1e-8, W)
        assert rel_err(f64(out[b:b + 1, h:h + 1]), O_ref) <= 1e-4, (b, h)
        assert np.max(np.abs(f64(z[b:b + 1, h:h + 1]) - Z_ref) / Z_ref) <= 1e-4, (b, h)


@pytest.mark.parametrize("T,W", [(1800, 50), (1850, 1)])
def test_purified_d128_window_paired_short_first_block(cuda_device, T, W):
    """Paired window launch whose first item (the last query block) has two
    key tiles (T 1800, W 50) or one (T 1850, W 1): the second item (block 0)
    starts before the usual waits cover its Q block, which the kernel drains
    first.  Every head's block 0 comes from such a pair, so whole heads are
    held to the oracle (fp32 output to 1e-4, Z to 1e-4 per row)."""
    B, H, D = 4, 16, 128
    print(f"purified d128 window paired T{T} W{W}", flush=True)
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=T + W, std=0.125, n=3,
                                                          dtype=torch.bfloat16))
    out, z = _pur_fwd_abi(q, k, v, 8.0, 0.0625, 0.05, True, 1e-8, window=W)
    for b, h in ((0, 0), (1, 9), (3, 15)):
        O_ref, Z_ref = orc.purified_forward(f64(q[b:b + 1, h:h + 1]), f64(k[b:b + 1, h:h + 1]),
                                            f64(v[b:b + 1, h:h + 1]), 8.0, 0.0625, 0.05, True, 1e-8, W)
        assert rel_err(f64(out[b:b + 1, h:h + 1]), O_ref) <= 1e-4, (b, h)
        assert rel_err(f64(out[b:b + 1, h:h + 1, :256]), O_ref[:, :, :256]) <= 1e-4, (b, h, "block 0")
        assert np.max(np.abs(f64(z[b:b + 1, h:h + 1]) - Z_ref) / Z_ref) <= 1e-4, (b, h)


def test_purified_fast_forward_paired_launch(cuda_device):
    """The C3 shape (B16 H16 T1024): workgroups take two query blocks each;
    checked on sampled heads against the oracle."""
    B, H, T = 16, 16, 1024
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 64), seed=3, std=0.125, n=3,
                                                          dtype=torch.bfloat16))
    out, z = _pur_fwd_abi(q, k, v, 8.0, 0.0625, 0.05, True, 1e-8)
    for b, h in ((0, 0), (7, 5), (15, 15), (3, 12)):
        O_ref, Z_ref = orc.purified_forward(f64(q[b:b + 1, h:h + 1]), f64(k[b:b + 1, h:h + 1]),
                                            f64(v[b:b + 1, h:h + 1]), 8.0, 0.0625, 0.05, True, 1e-8)
        assert rel_err(f64(out[b:b + 1, h:h + 1]), O_ref) <= 1e-4
        assert np.max(np.abs(f64(z[b:b + 1, h:h + 1]) - Z_ref) / Z_ref) <= 1e-4


# The bf16 D = 64 backward (dense or causal) runs the bf16-MFMA dQ and dK/dV
# kernels (the reference rounds p/Z and dR to the input dtype before its dots,
# so these contract bf16 operands as it does).  Held to the bf16 bar against
# the oracle and to 5e-3 (normwise) against the fp32-MFMA kernels, reached
# through a window longer than T (every pair stays visible: the same
# visibility); dgamma and dtau likewise.  An all-zero document id tensor (one
# document: the same visibility) runs the same kernels' document variants,
# held to the same bars.
FAST_BWD_CASES = [
    # (B, H, T, causal, scale, tau, eps_base, eps, std)
    (2, 3, 130, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (1, 2, 200, False, 8.0, -0.1, 0.05, 1e-8, 0.3),
    (2, 2, 64, False, [4.0, 9.0], [0.0, 0.2], 0.2, 1e-6, 0.3),
    (1, 1, 1, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (1, 2, 600, True, [8.0, 5.0], [-0.05, 0.1], 0.05, 1e-8, 0.2),
    (1, 1, 1000, False, 8.0, -0.2, 0.05, 1e-8, 0.2),
]


@pytest.mark.parametrize("case", FAST_BWD_CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}-{'causal' if c[3] else 'dense'}")
def test_purified_fast_backward(cuda_device, case):
    B, H, T, causal, scale, tau, eps_base, eps, std = case
    print(f"purified fast bwd case B{B} H{H} T{T} causal={causal}", flush=True)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 64), seed=T + 9, std=std, n=4,
                                                              dtype=torch.bfloat16))
    sc = torch.tensor(np.asarray(scale, dtype=np.float32), device=cuda_device)
    ta = torch.tensor(np.asarray(tau, dtype=np.float32), device=cuda_device)
    kw = dict(eps_base=eps_base, is_causal=causal, eps=eps)
    fast = _run(q, k, v, do, sc, ta, **kw)
    generic = _run(q, k, v, do, sc, ta, window_size=T + 1, **kw)
    zero_doc = torch.zeros((B, T), dtype=torch.int32, device=cuda_device)
    fast_doc = _run(q, k, v, do, sc, ta, doc_ids=zero_doc, **kw)
    okw = dict(eps_base=eps_base, is_causal=causal, eps=eps)
    ref = orc.purified_backward(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau), f64(do), **okw)
    mag = orc.purified_backward_magnitudes(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau),
                                           f64(do), **okw)
    for label, res in (("fast", fast), ("fast, documents", fast_doc)):
        for i, name in enumerate(("dq", "dk", "dv")):
            got, gen, want, m = f64(res[1 + i]), f64(generic[1 + i]), ref[i], mag[i]
            er = rel_err(got, want)
            ef = max_abs(got, want) / m.max() if m.max() > 0 else max_abs(got, want)
            assert er <= 2e-2 or ef <= 1e-4, f"{label} {name}: rel {er:.3e} vs oracle (term scale {ef:.3e})"
            eg = rel_err(got, gen)
            efg = max_abs(got, gen) / m.max() if m.max() > 0 else max_abs(got, gen)
            assert eg <= 5e-3 or efg <= 1e-4, f"{label} {name}: rel {eg:.3e} vs the fp32-MFMA kernel"
        for name, got, gen, want, m in (("dscale", res[4], generic[4], ref[3], mag[3]),
                                        ("dtau", res[5], generic[5], ref[4], mag[4])):
            got = np.atleast_1d(f64(got))
            gen = np.atleast_1d(f64(gen))
            ok = (np.abs(got - want) <= 2e-2 * np.abs(want)) | (np.abs(got - want) <= 1e-4 * m)
            assert ok.all(), f"{label} {name}: {got} vs oracle {want} (term scale {m})"
            ok = (np.abs(got - gen) <= 5e-3 * np.abs(gen)) | (np.abs(got - gen) <= 1e-4 * m)
            assert ok.all(), f"{label} {name}: {got} vs fp32-MFMA kernel {gen}"


# bf16, D = 128, dense or causal: the D = 128 dQ and dK/dV kernels' purified
# mode, held to the same bars as the D = 64 kernels above (against the oracle,
# and against the fp32-MFMA kernels reached through a window longer than T).
D128_BWD_CASES = [
    # (B, H, T, causal, scale, tau, eps_base, eps, std)
    (1, 1, 1, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (2, 3, 130, True, 8.0, 0.0625, 0.05, 1e-8, 0.3),
    (1, 2, 200, False, 8.0, -0.1, 0.05, 1e-8, 0.3),
    (2, 2, 256, False, [4.0, 9.0], [0.0, 0.2], 0.2, 1e-6, 0.3),
    (1, 2, 300, True, [8.0, 5.0], [-0.05, 0.1], 0.05, 1e-8, 0.2),
    (1, 1, 777, False, 8.0, -0.2, 0.05, 1e-8, 0.2),
    (1, 2, 1100, True, 6.0, 0.0625, 0.05, 1e-8, 0.15),
]


@pytest.mark.parametrize("case", D128_BWD_CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}-{'causal' if c[3] else 'dense'}")
def test_purified_d128_backward(cuda_device, case):
    B, H, T, causal, scale, tau, eps_base, eps, std = case
    print(f"purified d128 bwd case B{B} H{H} T{T} causal={causal}", flush=True)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 128), seed=T + 13, std=std, n=4,
                                                              dtype=torch.bfloat16))
    sc = torch.tensor(np.asarray(scale, dtype=np.float32), device=cuda_device)
    ta = torch.tensor(np.asarray(tau, dtype=np.float32), device=cuda_device)
    kw = dict(eps_base=eps_base, is_causal=causal, eps=eps)
    fast = _run(q, k, v, do, sc, ta, **kw)
    generic = _run(q, k, v, do, sc, ta, window_size=T + 1, **kw)
    ref = orc.purified_backward(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau), f64(do), **kw)
    mag = orc.purified_backward_magnitudes(f64(q), f64(k), f64(v), np.atleast_1d(scale), np.atleast_1d(tau),
                                           f64(do), **kw)
    for i, name in enumerate(("dq", "dk", "dv")):
        got, gen, want, m = f64(fast[1 + i]), f64(generic[1 + i]), ref[i], mag[i]
        er = rel_err(got, want)
        ef = max_abs(got, want) / m.max() if m.max() > 0 else max_abs(got, want)
        assert er <= 2e-2 or ef <= 1e-4, f"{name}: rel {er:.3e} vs oracle (term scale {ef:.3e})"
        eg = rel_err(got, gen)
        efg = max_abs(got, gen) / m.max() if m.max() > 0 else max_abs(got, gen)
        assert eg <= 5e-3 or efg <= 1e-4, f"{name}: rel {eg:.3e} vs the fp32-MFMA kernel"
    for name, got, gen, want, m in (("dscale", fast[4], generic[4], ref[3], mag[3]),
                                    ("dtau", fast[5], generic[5], ref[4], mag[4])):
        got = np.atleast_1d(f64(got))
        gen = np.atleast_1d(f64(gen))
        ok = (np.abs(got - want) <= 2e-2 * np.abs(want)) | (np.abs(got - want) <= 1e-4 * m)
        assert ok.all(), f"{name}: {got} vs oracle {want} (term scale {m})"
        ok = (np.abs(got - gen) <= 5e-3 * np.abs(gen)) | (np.abs(got - gen) <= 1e-4 * m)
        assert ok.all(), f"{name}: {got} vs fp32-MFMA kernel {gen}"


def test_purified_d128_backward_many_heads(cuda_device):
    """B2 H16 T700, causal, per-head gamma and tau: every head's dgamma and
    dtau against the oracle (to the bf16 bar of their value or of the scale
    of their terms, as above), gradients on sampled heads."""
    B, H, T = 2, 16, 700
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 128), seed=31, std=0.15, n=4,
                                                              dtype=torch.bfloat16))
    scale = np.linspace(3.0, 9.0, H).astype(np.float32)
    tau = np.linspace(-0.1, 0.1, H).astype(np.float32)
    sc = torch.tensor(scale, device=cuda_device)
    ta = torch.tensor(tau, device=cuda_device)
    fast = _run(q, k, v, do, sc, ta, is_causal=True)
    dsc, dta = f64(fast[4]), f64(fast[5])
    for h in range(H):
        sl = (slice(None), slice(h, h + 1))
        args = (f64(q[sl]), f64(k[sl]), f64(v[sl]), scale[h], tau[h], f64(do[sl]))
        ref = orc.purified_backward(*args)
        mag = orc.purified_backward_magnitudes(*args)
        if h in (0, 7, 15):
            for i in range(3):
                assert rel_err(f64(fast[1 + i][sl]), ref[i]) <= 2e-2, (h, i)
        for name, got, want, m in (("dscale", dsc[h], ref[3], mag[3]), ("dtau", dta[h], ref[4], mag[4])):
            err = abs(got - float(np.squeeze(want)))
            assert err <= 2e-2 * abs(float(np.squeeze(want))) or err <= 1e-4 * float(np.squeeze(m)), (name, h, got, want, m)


def test_purified_fast_backward_full_size(cuda_device):
    """The C5 shape (B16 H16 T2048): gradients checked on sampled heads
    against the oracle; dgamma / dtau against the fp32-MFMA kernels."""
    B, H, T = 16, 16, 2048
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 64), seed=21, std=0.125, n=4,
                                                              dtype=torch.bfloat16))
    sc = torch.tensor(8.0, device=cuda_device)
    ta = torch.tensor(0.0625, device=cuda_device)
    fast = _run(q, k, v, do, sc, ta, is_causal=True)
    generic = _run(q, k, v, do, sc, ta, is_causal=True, window_size=T + 1)
    for b, h in ((0, 0), (9, 13), (15, 15)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref = orc.purified_backward(f64(q[sl]), f64(k[sl]), f64(v[sl]), 8.0, 0.0625, f64(do[sl]))
        for i in range(3):
            assert rel_err(f64(fast[1 + i][sl]), ref[i]) <= 2e-2
    for i in (4, 5):
        got, gen = float(fast[i]), float(generic[i])
        assert abs(got - gen) <= 5e-3 * abs(gen) + 1e-6, (i, got, gen)


def test_purified_fast_documents_c4_shape(cuda_device):
    """C4's shape and documents (p4b): the document kernel's purified forward
    and the document variants of the bf16-MFMA backward kernels, on two heads
    against the oracle document by document (a masked pair contributes
    nothing, so each causal document is exact on its own), and on all heads
    (output, gradients, dgamma, dtau) against the fp32-MFMA kernels reached
    through a window longer than T."""
    from util import doc_spans

    B, H, T = 4, 16, 8192
    docs = orc.geometric_doc_ids(B, T, 512.0, seed=0)
    doc_t = torch.tensor(docs, dtype=torch.int32, device=cuda_device)
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((B, H, T, 64), seed=17, std=0.125, n=4,
                                                              dtype=torch.bfloat16))
    sc = torch.tensor(8.0, device=cuda_device)
    ta = torch.tensor(-0.03, device=cuda_device)  # tau < 0: masked pairs must be zeroed explicitly
    fast = _run(q, k, v, do, sc, ta, is_causal=True, doc_ids=doc_t)
    generic = _run(q, k, v, do, sc, ta, is_causal=True, doc_ids=doc_t, window_size=T + 1)
    # The forward (the document kernel's purified mode), through the C ABI's
    # fp32 output: fp32 accumulation of split weights, held to 1e-4 against
    # the fp32-MFMA kernel and the oracle (the autograd entry's output is
    # rounded to bf16, which alone moves it by up to 2^-9).
    o32, z32 = _pur_fwd_abi(q, k, v, 8.0, -0.03, 0.05, True, 1e-8, doc=doc_t)
    o32g, z32g = _pur_fwd_abi(q, k, v, 8.0, -0.03, 0.05, True, 1e-8, doc=doc_t, window=T + 1)
    eo = rel_err(f64(o32), f64(o32g))
    print(f"p4b out: rel {eo:.3e} vs the fp32-MFMA kernel", flush=True)
    assert eo <= 1e-4, eo
    assert np.max(np.abs(f64(z32) - f64(z32g)) / f64(z32g)) <= 1e-4
    for b, h in ((0, 3), (3, 14)):
        for a, e in doc_spans(docs[b])[:6]:
            sl = (slice(b, b + 1), slice(h, h + 1), slice(a, e))
            o_ref, _ = orc.purified_forward(f64(q[sl]), f64(k[sl]), f64(v[sl]), 8.0, -0.03, 0.05, True, 1e-8)
            assert rel_err(f64(o32[sl]), o_ref) <= 1e-4, (b, h, a, e)
            ref = orc.purified_backward(f64(q[sl]), f64(k[sl]), f64(v[sl]), 8.0, -0.03, f64(do[sl]))
            mag = orc.purified_backward_magnitudes(f64(q[sl]), f64(k[sl]), f64(v[sl]), 8.0, -0.03, f64(do[sl]))
            for i, name in enumerate(("dq", "dk", "dv")):
                got = f64(fast[1 + i][sl])
                er = rel_err(got, ref[i])
                ef = max_abs(got, ref[i]) / mag[i].max() if mag[i].max() > 0 else max_abs(got, ref[i])
                assert er <= 2e-2 or ef <= 1e-4, (b, h, a, e, name, er, ef)
    for i, name in enumerate(("dq", "dk", "dv")):
        eg = rel_err(f64(fast[1 + i]), f64(generic[1 + i]))
        print(f"p4b {name}: rel {eg:.3e} vs the fp32-MFMA kernels", flush=True)
        assert eg <= 5e-3, (name, eg)
    for i in (4, 5):
        got, gen = float(fast[i]), float(generic[i])
        assert abs(got - gen) <= 5e-3 * abs(gen) + 1e-6, (i, got, gen)
