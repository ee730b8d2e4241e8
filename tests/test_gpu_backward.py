"""GPU parity of the flash-Born backward (dq, dk, dv, dscale) against the
float64 oracle's closed-form gradients on the same (dtype-rounded) inputs,
with delta = dO . O formed from the forward output the backward is handed,
as the reference does (flash_born.py:277, 302, 387).

Tolerances (normwise relative error): 2e-2 for bf16 / fp16, 1e-5 for fp32.
dscale is compared against the scale of its terms, (2/|s|) eps sum|delta/Z|,
because its value is itself a small difference.  fp16 cases default to
N(0, 0.25) inputs, inside the range where the reference's fp16 forward
weights (s q.k)^2 do not overflow at scale 8.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc
from util import TOL, doc_spans, f64, max_abs, rel_err, seeded_inputs

pytestmark = pytest.mark.gpu


def _grads(q, k, v, do, scale, **kw):
    from quantumdlblocks_amd import flash_born_attention

    q = q.detach().clone().requires_grad_(True)
    k = k.detach().clone().requires_grad_(True)
    v = v.detach().clone().requires_grad_(True)
    sc = scale.detach().clone().requires_grad_(True) if isinstance(scale, torch.Tensor) else scale
    out = flash_born_attention(q, k, v, sc, **kw)
    out.backward(do)
    torch.cuda.synchronize()
    ds = sc.grad if isinstance(sc, torch.Tensor) else None
    return out, q.grad, k.grad, v.grad, ds


# A gradient passes if its normwise relative error is within TOL, or -- for
# gradients that cancel to ~0 (a row that sees one key, a window of 1) -- if
# its error is within FLOOR of the largest magnitude of the terms it sums
# (oracle.backward_magnitudes): the rounding floor of the computation (for
# fp32, 1e-6 is ~17 ulps of the largest term).  C4's fp32 dQ passes by the
# floor: its document rows that see a few keys cancel terms of ~10^3-10^4 to
# results of ~10^-5, each row's error within ~2 ulps of its own terms.
FLOOR = {torch.float32: 1e-6, torch.bfloat16: 1e-4, torch.float16: 1e-4}


def _grad_ok(got, ref, mag, dtype, tol=None):
    """(passed, branch, normwise error, error against the term scale); branch
    names the test a passing gradient met: "rel" (normwise within TOL) or
    "floor" (only within FLOOR of its terms' scale), "FAIL" otherwise."""
    e_rel = rel_err(got, ref)
    e_floor = max_abs(got, ref) / mag.max() if mag.size and mag.max() > 0 else max_abs(got, ref)
    branch = "rel" if e_rel <= (tol or TOL[dtype]) else ("floor" if e_floor <= FLOOR[dtype] else "FAIL")
    return branch != "FAIL", branch, e_rel, e_floor


def _check_bwd(B, H, T, D, dtype, dev, *, scale=8.0, is_causal=True, eps=1e-12, window_size=0, doc=None,
               std=None, seed=0, heads=None, tol=None, check_dscale=False):
    std = (0.5 if dtype == torch.float16 else 1.0) if std is None else std
    q, k, v, do = (x.to(dev) for x in seeded_inputs((B, H, T, D), seed=seed, std=std, n=4, dtype=dtype))
    doc_t = None if doc is None else torch.as_tensor(doc, dtype=torch.int32, device=dev)
    sc_np = np.asarray(scale, dtype=np.float32)
    sc_t = torch.as_tensor(sc_np, device=dev)
    out, dq, dk, dv, ds = _grads(q, k, v, do, sc_t, is_causal=is_causal, eps=eps, window_size=window_size,
                                 doc_ids=doc_t)
    for g, x in ((dq, q), (dk, k), (dv, v)):
        assert g.dtype == x.dtype and g.shape == x.shape
    assert ds.shape == sc_t.shape and ds.dtype == sc_t.dtype
    sel = heads or [(b, h) for b in range(B) for h in range(H)]
    refs = {0: [], 1: [], 2: []}
    mags = {0: [], 1: [], 2: []}
    gots = {0: [], 1: [], 2: []}
    # Long causal rows of contiguous documents: each document's queries see
    # only its own keys and vice versa, so every gradient of a span follows
    # from that span alone (exact); the oracle runs span by span.
    spans = None
    if doc is not None and is_causal and window_size == 0 and T > 2048:
        spans = {b: doc_spans(doc[b]) for b, _ in sel}
    for b, h in sel:
        s_h = sc_np.reshape(-1)[h] if sc_np.size > 1 else sc_np.reshape(-1)[0]
        cut = [(0, T)] if spans is None else spans[b]
        part = {0: [], 1: [], 2: []}
        mpart = {0: [], 1: [], 2: []}
        for a, e in cut:
            args = (f64(q[b : b + 1, h : h + 1, a:e]), f64(k[b : b + 1, h : h + 1, a:e]),
                    f64(v[b : b + 1, h : h + 1, a:e]), s_h, f64(do[b : b + 1, h : h + 1, a:e]), is_causal, eps,
                    window_size, None if (doc is None or spans is not None) else doc[b : b + 1])
            # delta from the forward output the backward was handed (flash_born.py:277, 302)
            r = orc.backward(*args, out=f64(out[b : b + 1, h : h + 1, a:e]))
            m = orc.backward_magnitudes(*args)
            for i in range(3):
                part[i].append(r[i])
                mpart[i].append(m[i])
        for i, got_t in enumerate((dq, dk, dv)):
            refs[i].append(np.concatenate(part[i], axis=2))
            mags[i].append(np.concatenate(mpart[i], axis=2))
            gots[i].append(f64(got_t[b : b + 1, h : h + 1]))
    msgs, fails = [], []
    for i, name in enumerate(("dq", "dk", "dv")):
        got, ref, mag = (np.concatenate(x[i]) for x in (gots, refs, mags))
        assert np.isfinite(got).all(), name
        ok, branch, e_rel, e_floor = _grad_ok(got, ref, mag, dtype, tol)
        msgs.append(f"{name}:rel={e_rel:.2e}/floor={e_floor:.2e}[{branch}]")
        if not ok:
            fails.append(name)
    print(f"bwd B{B} H{H} T{T} D{D} {dtype} causal={is_causal} W={window_size} doc={doc is not None} "
          + " ".join(msgs), flush=True)
    assert not fails, fails
    if check_dscale:
        O, Z = orc.forward(f64(q), f64(k), f64(v), sc_np.astype(np.float64), is_causal, eps, window_size, doc)
        delta_n = (f64(do) * f64(out)).sum(-1) / Z
        s = sc_np.astype(np.float64).reshape(-1)
        with np.errstate(divide="ignore", invalid="ignore"):
            inv = np.where(s != 0, 2.0 / np.where(s != 0, s, 1.0), 0.0)
        if s.size > 1:
            want = inv * eps * delta_n.sum(axis=(0, 2))
            mag = np.abs(inv) * eps * np.abs(delta_n).sum(axis=(0, 2))
        else:
            want = inv * eps * np.array([delta_n.sum()])
            mag = np.abs(inv) * eps * np.array([np.abs(delta_n).sum()])
        got = f64(ds).reshape(-1)
        print(f"  dscale got={got} want={want} mag={mag}", flush=True)
        assert np.all(np.abs(got - want) <= TOL[dtype] * mag + 1e-30)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("is_causal", [True, False])
def test_bwd_c1_shape(cuda_device, dtype, is_causal):
    _check_bwd(1, 4, 256, 64, dtype, cuda_device, is_causal=is_causal)


@pytest.mark.parametrize("D, window", [(64, 0), (64, 100), (32, 0)])
@pytest.mark.parametrize("scale", [0.05, -0.3, 8.0])
def test_bwd_f16_operand_range(cuda_device, D, window, scale):
    """fp16 dot operands (p/Z and dS) stay in range for small scales with large
    overlaps, as the reference's do (the kernel's dS operand is the
    reference's 2 a dP, its p/Z operand 4 p/Z)."""
    std = 4.0 if abs(scale) < 1 else 0.5
    _check_bwd(1, 2, 300, D, torch.float16, cuda_device, scale=scale, std=std, window_size=window, seed=3)


@pytest.mark.parametrize("T", [1, 5, 33, 64, 100, 257])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bwd_ragged_lengths(cuda_device, T, dtype):
    _check_bwd(2, 3, T, 64, dtype, cuda_device, seed=T)


@pytest.mark.parametrize("D", [8, 16, 32, 48, 80, 96, 128, 160, 192, 256, 20])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bwd_head_dims(cuda_device, D, dtype):
    _check_bwd(2, 2, 96, D, dtype, cuda_device, scale=1.0 / math.sqrt(D), seed=D)


@pytest.mark.parametrize("D", [160, 224, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["causal", "dense", "window", "documents"])
def test_bwd_wide_head_dims_column_split(cuda_device, D, dtype, mode):
    """Wide head dims (16-bit): without documents the DMA-ring kernels for
    128 < D <= 256 (born_bwd_d256.h: D < 256 with zero columns); with
    documents the generic kernels (D >= 192 in two dK/dV workgroups per key
    block, each holding half of the column blocks, seven split unevenly at
    D = 224); several key blocks and query tiles, every mask mode, per-head
    scales, dscale."""
    kw = dict(is_causal=mode != "dense", window_size=90 if mode == "window" else 0,
              doc=orc.geometric_doc_ids(2, 300, 60.0, seed=D) if mode == "documents" else None)
    _check_bwd(2, 2, 300, D, dtype, cuda_device, scale=[0.2, -0.1], std=0.5, seed=D + 1, check_dscale=True, **kw)


@pytest.mark.parametrize("D", [136, 192, 224, 256])
@pytest.mark.parametrize("mode", ["causal", "dense", "window", "documents"])
def test_bwd_wide_head_dims_fp32_column_split(cuda_device, D, mode):
    """fp32 above D = 128 on the fp32-MFMA kernels, every mask mode (dense
    launches at D = 256 run the dK/dV kernel in two workgroups per key block,
    each accumulating half of the column blocks); several key blocks and
    query tiles, per-head scales.  (dscale, from the fp32 row sums of D
    products, is held to the fp32 bar at smaller head dims.)"""
    kw = dict(is_causal=mode != "dense", window_size=90 if mode == "window" else 0,
              doc=orc.geometric_doc_ids(2, 300, 60.0, seed=D) if mode == "documents" else None)
    _check_bwd(2, 2, 300, D, torch.float32, cuda_device, scale=[0.2, -0.1], std=0.5, seed=D + 2, **kw)


@pytest.mark.parametrize("D", [136, 200, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", [(True, 0, 1), (True, 0, 64), (True, 0, 129), (True, 0, 700), (False, 0, 300),
                                  (True, 1, 300), (True, 63, 300), (True, 200, 700), (False, 1, 300),
                                  (False, 64, 300), (False, 129, 700), (False, 1000, 300)])
def test_bwd_wide_dma_kernels(cuda_device, D, dtype, case):
    """128 < D <= 256 without documents: the dQ kernel (4 waves over 128
    query rows, 64-key tiles through a two-stage ring) and the dK/dV kernel
    (dV and dK of a 128-key block in two workgroups); padded head dims
    (136, 200: zero columns past D), one and several key blocks, a partial
    last tile and block, causal and dense, windows with and without
    causality shorter and longer than T; per-head scales (one negative) and
    dscale."""
    is_causal, window, T = case
    _check_bwd(1, 2, T, D, dtype, cuda_device, is_causal=is_causal, window_size=window, scale=[0.3, -0.15],
               std=0.5, seed=D + T + window, check_dscale=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [72, 96, 120])
@pytest.mark.parametrize("is_causal, window", [(True, 0), (False, 0), (True, 100)])
def test_bwd_padded_documents(cuda_device, dtype, D, is_causal, window):
    """64 < D < 128 with document ids on the D = 128 kernels' document mode
    with zero columns past D (dQ on 128-row blocks, dK/dV on 64-key blocks);
    per-head scales, dscale."""
    doc = orc.geometric_doc_ids(2, 700, 90.0, seed=D + window)
    _check_bwd(2, 2, 700, D, dtype, cuda_device, doc=doc, is_causal=is_causal, window_size=window,
               scale=[0.3, -0.15], std=0.5, seed=D + 7, check_dscale=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [136, 256])
@pytest.mark.parametrize("is_causal, window", [(True, 0), (False, 0), (True, 100)])
def test_bwd_wide_documents(cuda_device, dtype, D, is_causal, window):
    """128 < D <= 256 with document ids (dense, causal, causal window) on the
    wide-row kernels' document mode: the dQ kernel's key-tile and the dK/dV
    kernel's query-tile screening, per-wave skips and per-element tests;
    padded and unpadded head dims, per-head scales, dscale."""
    doc = orc.geometric_doc_ids(2, 700, 90.0, seed=D + window)
    _check_bwd(2, 2, 700, D, dtype, cuda_device, doc=doc, is_causal=is_causal, window_size=window,
               scale=[0.3, -0.15], std=0.5, seed=D + 3, check_dscale=True)


def test_bwd_wide_documents_many_chunks(cuda_device):
    """D = 256, sorted documents over more candidate tiles than one screening
    pass holds (256 key tiles for dQ, 256 query tiles for dK/dV): the ring
    restarts on its first stage with every chunk."""
    doc = orc.geometric_doc_ids(1, 17000, 300.0, seed=5)
    _check_bwd(1, 1, 17000, 256, torch.bfloat16, cuda_device, doc=doc, scale=0.3, std=0.5, seed=17)


def test_bwd_head_dim_above_256_takes_the_eager_path(cuda_device):
    """D > 256: autograd through the reference's eager formulation on the GPU
    (flash_born.py:670-690), gradients against the oracle."""
    _check_bwd(1, 2, 80, 272, torch.float32, cuda_device, scale=1.0 / math.sqrt(272), seed=272)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("window", [1, 7, 64, 150])
@pytest.mark.parametrize("is_causal", [True, False])
def test_bwd_sliding_window(cuda_device, dtype, window, is_causal):
    _check_bwd(2, 2, 200, 64, dtype, cuda_device, is_causal=is_causal, window_size=window, seed=window)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [1, 63, 64, 65, 127, 128, 129, 255, 256, 300, 700, 2000])
def test_bwd_sliding_window_fast_kernels(cuda_device, dtype, window):
    """Causal windows at D = 64 run the fast dQ and dK/dV kernels' window
    mode: windows on and beside the 64-row tile, 128-key and 256-row block
    edges, longer than T, a partial last block; per-head scales and dscale."""
    _check_bwd(2, 2, 1100, 64, dtype, cuda_device, window_size=window, seed=window + 3, scale=[8.0, -0.7],
               check_dscale=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [1, 63, 64, 65, 127, 128, 129, 255, 256, 300, 700, 2000])
def test_bwd_sliding_window_noncausal_fast_kernels(cuda_device, dtype, window):
    """Windows without causality at D = 64 run the fast dQ and dK/dV
    kernels' kWindowNC mode (key j is seen by queries 0 .. j + W - 1; the
    dK/dV launch takes the last key blocks first): windows on and beside the
    64-row tile, 128-key and 256-row block edges, longer than T, a partial
    last block; per-head scales and dscale."""
    _check_bwd(2, 2, 1100, 64, dtype, cuda_device, is_causal=False, window_size=window, seed=window + 5,
               scale=[8.0, -0.7], check_dscale=True)


@pytest.mark.parametrize("T", [1, 37, 64, 129, 256, 300, 513])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("window", [1, 3, 100])
def test_bwd_noncausal_window_ragged(cuda_device, T, D, window):
    """kWindowNC dQ and dK/dV on ragged lengths: a single partial tile, T on
    and beside the tile and key-block edges, windows shorter and longer than T
    (the dK/dV launch walks the key blocks from the last)."""
    _check_bwd(1, 2, T, D, torch.bfloat16, cuda_device, is_causal=False, window_size=window,
               scale=[8.0, -0.7] if D == 64 else [0.09, -0.3], std=1.0 if D == 64 else 0.7, seed=T + window,
               check_dscale=True)


@pytest.mark.parametrize("T", [1, 37, 64, 200, 256, 300, 513, 1100])
@pytest.mark.parametrize("is_causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_bwd_d128_kernels(cuda_device, T, is_causal, dtype):
    """D = 128 without documents runs its own dQ (8 waves over 256 query
    rows) and dK/dV (4 waves over 128 keys) kernels: ragged lengths, partial
    blocks and tiles, per-head scales of both signs, dscale."""
    _check_bwd(1, 2, T, 128, dtype, cuda_device, is_causal=is_causal, scale=[0.09, -0.2], std=0.7, seed=T + 5,
               check_dscale=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [1, 31, 32, 33, 64, 100, 127, 128, 129, 256, 700, 2000])
def test_bwd_d128_sliding_window(cuda_device, dtype, window):
    """Causal windows at D = 128: windows on and beside a wave's 32 rows or
    keys, the 64-row tiles, the 128-key and 256-row blocks, longer than T."""
    _check_bwd(2, 2, 1100, 128, dtype, cuda_device, window_size=window, seed=window + 13, scale=[0.09, -0.3],
               std=0.7, check_dscale=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D, window", [(128, 1), (128, 31), (128, 33), (128, 64), (128, 127), (128, 129),
                                       (128, 256), (128, 700), (128, 2000), (96, 100), (96, 257)])
def test_bwd_d128_sliding_window_noncausal(cuda_device, dtype, D, window):
    """Windows without causality at D = 128 (and D = 96 with the columns
    past D zero): the D = 128 dQ and dK/dV kernels' kWindowNC mode (dK/dV
    takes the last key blocks first); per-head scales and dscale."""
    _check_bwd(2, 2, 1100, D, dtype, cuda_device, is_causal=False, window_size=window, seed=window + 17,
               scale=[0.09, -0.3], std=0.7, check_dscale=True)


@pytest.mark.parametrize("D", [72, 96, 120])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["causal", "dense", "window"])
def test_bwd_d128_padded_head_dims(cuda_device, D, dtype, mode):
    """64 < D < 128 runs the D = 128 dQ and dK/dV kernels with the columns
    past D zero and not stored: ragged T, causal, dense, a causal window,
    dscale."""
    kw = dict(is_causal=mode != "dense", window_size=100 if mode == "window" else 0)
    _check_bwd(2, 2, 555, D, dtype, cuda_device, scale=[0.09, -0.2], std=0.7, seed=D + 3, check_dscale=True, **kw)


def test_bwd_d128_config_d5(cuda_device):
    """d5: bf16 B16 H8 T2048 D128 forward + backward (the C5 work at head dim
    128), N(0,1); 16 heads covering every batch row and block residue."""
    _check_bwd(16, 8, 2048, 128, torch.bfloat16, cuda_device, scale=0.09, heads=[(b, (3 * b + 1) % 8) for b in range(16)])


def test_bwd_sliding_window_c5_shape(cuda_device):
    """C5's shape with a 512-key window, 16 heads covering every block residue."""
    _check_bwd(16, 16, 2048, 64, torch.bfloat16, cuda_device, window_size=512, heads=[(b, b) for b in range(16)])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("is_causal", [True, False])
def test_bwd_document_mask(cuda_device, dtype, is_causal):
    doc = orc.geometric_doc_ids(3, 300, 40.0, seed=1)
    _check_bwd(3, 2, 300, 64, dtype, cuda_device, is_causal=is_causal, doc=doc)
    _check_bwd(2, 2, 257, 64, dtype, cuda_device, is_causal=is_causal, doc=doc[:2, :257], window_size=30)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 96, 128, 200, 256])
@pytest.mark.parametrize("is_causal", [True, False])
def test_bwd_unsorted_document_ids(cuda_device, dtype, D, is_causal):
    """Arbitrary (unsorted, repeating) document ids: the span of tiles a
    backward block visits, taken from document-id ranges, must stay a superset
    of the tiles holding a visible pair."""
    rng = np.random.default_rng(D + 1)
    doc = rng.integers(0, 4, size=(2, 700)).astype(np.int32)
    doc[1, 350:] = rng.integers(10, 12, size=350)
    _check_bwd(2, 2, 700, D, dtype, cuda_device, is_causal=is_causal, doc=doc, seed=D)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("is_causal", [True, False])
def test_bwd_document_tile_edges(cuda_device, dtype, D, is_causal):
    """Sorted documents whose edges fall on, just before and just after the
    32-, 64-, 128- and 256-row tile and block edges, one-token documents,
    negative ids, and a batch row sorted in descending order: the tiles a
    block's span leaves out must hold no visible pair."""
    lens = [64, 1, 63, 129, 256, 1, 1, 31, 97, 200, 65, 12, 33]
    ids = np.concatenate([np.full(n, i - 3, np.int32) for i, n in enumerate(lens)])
    doc = np.stack([ids, -ids[::-1]])
    _check_bwd(2, 2, ids.size, D, dtype, cuda_device, is_causal=is_causal, doc=doc, seed=5)


def test_bwd_documents_many_tiles(cuda_device):
    """Sorted documents over more candidate tiles than a block has threads
    (fp32, D = 256: one-wave dK/dV blocks, 32-row tiles), so the span's
    screening loop strides."""
    doc = orc.geometric_doc_ids(1, 4500, 400.0, seed=9)
    _check_bwd(1, 1, 4500, 256, torch.float32, cuda_device, doc=doc, std=0.5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("is_causal", [True, False])
def test_bwd_documents_fast_kernels(cuda_device, dtype, is_causal):
    """D = 64 with documents and no window runs the document variants of the
    DMA-ring dQ and dK/dV kernels: T not a multiple of the 64-row tile or of
    the 128- / 256-row blocks, per-head scales (one negative) and dscale."""
    doc = orc.geometric_doc_ids(2, 1100, 90.0, seed=3)
    _check_bwd(2, 3, 1100, 64, dtype, cuda_device, is_causal=is_causal, doc=doc, scale=[8.0, -0.5, 2.0],
               check_dscale=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("is_causal", [True, False])
def test_bwd_d128_documents(cuda_device, dtype, is_causal):
    """D = 128 with document ids (no window) runs the document mode of the
    D = 128 dQ and dK/dV kernels: geometric documents, per-head scales (one
    negative) and dscale; document edges on and beside the wave slices,
    tiles and blocks, one-token documents, negative ids, a descending row;
    unsorted ids."""
    doc = orc.geometric_doc_ids(2, 1100, 90.0, seed=3)
    _check_bwd(2, 3, 1100, 128, dtype, cuda_device, is_causal=is_causal, doc=doc, scale=[0.3, -0.2, 0.1],
               std=0.7, check_dscale=True)
    lens = [64, 1, 63, 129, 256, 1, 1, 31, 97, 200, 65, 12, 33, 32, 288]
    ids = np.concatenate([np.full(n, i - 3, np.int32) for i, n in enumerate(lens)])
    _check_bwd(2, 2, ids.size, 128, dtype, cuda_device, is_causal=is_causal, doc=np.stack([ids, -ids[::-1]]),
               scale=0.2, std=0.7, seed=5)
    rng = np.random.default_rng(8)
    doc = rng.integers(0, 3, size=(1, 600)).astype(np.int32)
    _check_bwd(1, 2, 600, 128, dtype, cuda_device, is_causal=is_causal, doc=doc, scale=0.2, std=0.7, seed=8)


# (A one-key window leaves each row a single weight: fp16 rounds the weights
# of tiny overlaps to zero, as the reference's kernel does, and the row's
# output with them, while the float64 oracle keeps them; so bf16 only there.)
@pytest.mark.parametrize("dtype,window", [(torch.bfloat16, 1)] + [(d, w) for d in (torch.bfloat16, torch.float16)
                                                                  for w in (33, 100, 300, 2000)])
def test_bwd_documents_and_window_fast(cuda_device, dtype, window):
    """D = 64 with document ids and a causal sliding window: the document
    variants of the DMA-ring dQ and dK/dV kernels with the window's tile
    ranges and edges; dscale."""
    # fp16: eps 1e-6.  A document's first row sees one key; when that
    # overlap is small enough for its fp16 weight to underflow, Z is eps
    # alone (the float64 oracle keeps p + eps), and with eps = 1e-12 the
    # row's fp16 gradient terms overflow (as the reference's fp16 dS would).
    eps = 1e-6 if dtype == torch.float16 else 1e-12
    doc = orc.geometric_doc_ids(2, 1100, 150.0, seed=window)
    _check_bwd(2, 3, 1100, 64, dtype, cuda_device, doc=doc, window_size=window, scale=[0.5, -0.3, 2.0], std=0.7,
               seed=window + 5, check_dscale=True, eps=eps)
    # Document edges on and beside the tiles and blocks, one-token documents
    # (bf16: in fp16 these rows of one or few weights are ill-conditioned,
    # 2.4e-2 against the oracle on these and on the register-staged kernels
    # alike).
    if dtype == torch.bfloat16:
        lens = [64, 1, 63, 129, 256, 1, 1, 31, 97, 200, 65, 12, 33, 32, 288]
        ids = np.concatenate([np.full(n, i - 3, np.int32) for i, n in enumerate(lens)])
        _check_bwd(2, 2, ids.size, 64, dtype, cuda_device, doc=np.stack([ids, -ids[::-1]]), window_size=window,
                   scale=0.5, std=0.7, seed=window + 6, eps=eps)


# (A one-key window leaves each row a single weight: fp16 rounds the weights
# of tiny overlaps to zero, as the reference's kernel does, and the row's
# output with them, while the float64 oracle keeps them; so bf16 only there.)
@pytest.mark.parametrize("dtype,window", [(torch.bfloat16, 1)] + [(d, w) for d in (torch.bfloat16, torch.float16)
                                                                  for w in (33, 100, 300, 2000)])
def test_bwd_d128_documents_and_window(cuda_device, dtype, window):
    """D = 128 with document ids and a causal sliding window: the document
    mode of the dQ and dK/dV kernels with the window's tile ranges, skips and
    per-element tests; dscale."""
    eps = 1e-6 if dtype == torch.float16 else 1e-12  # (as in the D = 64 test above)
    doc = orc.geometric_doc_ids(2, 1100, 150.0, seed=window)
    _check_bwd(2, 2, 1100, 128, dtype, cuda_device, doc=doc, window_size=window, scale=[0.2, -0.1], std=0.7,
               seed=window + 4, check_dscale=True, eps=eps)


def test_bwd_d128_documents_many_chunks(cuda_device):
    """D = 128: more candidate tiles than one screening pass holds (256 key
    tiles in dQ, 256 query tiles in dK/dV), sorted documents with one longer
    than a pass."""
    T = 17000
    doc = np.zeros((1, T), dtype=np.int32)
    doc[0, 3000:12000] = 1
    doc[0, 12000:] = 2 + orc.geometric_doc_ids(1, T - 12000, 700.0, seed=11)[0]
    _check_bwd(1, 1, T, 128, torch.bfloat16, cuda_device, doc=doc, scale=0.5, std=0.5, seed=11)


def test_bwd_d128_config_c4_documents(cuda_device):
    """C4's documents at head dim 128 with the backward (dc4b: B4 H8 T8192
    D128); 8 heads, document by document."""
    doc = orc.geometric_doc_ids(4, 8192, 512.0, seed=0)
    _check_bwd(4, 8, 8192, 128, torch.bfloat16, cuda_device, doc=doc, scale=1.0, std=0.3,
               heads=[(b, (3 * b + j) % 8) for b in range(4) for j in range(2)])


def test_bwd_documents_fast_many_chunks_causal(cuda_device):
    """More candidate tiles than one screening pass holds (256 key tiles in
    dQ, 128 query tiles in dK/dV): a 17000-token row of sorted documents, one
    of them longer than a pass."""
    T = 17000
    doc = np.zeros((1, T), dtype=np.int32)
    doc[0, 3000:12000] = 1
    doc[0, 12000:] = 2 + orc.geometric_doc_ids(1, T - 12000, 700.0, seed=11)[0]
    _check_bwd(1, 2, T, 64, torch.bfloat16, cuda_device, doc=doc, seed=11)


def test_bwd_documents_fast_many_chunks_unsorted(cuda_device):
    """Unsorted, repeating ids over more query tiles than one dK/dV screening
    pass holds, without causality: every tile is mixed and takes the
    per-element test."""
    T = 8300
    rng = np.random.default_rng(12)
    doc = rng.integers(0, 3, size=(1, T)).astype(np.int32)
    doc[0, 5000:] = rng.integers(7, 9, size=T - 5000)
    _check_bwd(1, 1, T, 64, torch.bfloat16, cuda_device, is_causal=False, doc=doc, seed=12)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bwd_scales_and_dscale(cuda_device, dtype):
    for scale in (np.array([2.5, 3.2, -0.5, 7.0]), np.array([1.0, 0.0, -8.0, 2.0])):
        _check_bwd(2, 4, 130, 64, dtype, cuda_device, scale=scale, eps=1e-3, std=0.3, check_dscale=True)
    for s in (8.0, -3.0):
        _check_bwd(2, 4, 70, 64, dtype, cuda_device, scale=s, eps=1.0, std=0.3, check_dscale=True)


def test_bwd_reference_jax_parity_case(cuda_device):
    """The reference's torch-vs-JAX gradient case (test_jax_haliax.py:74-134):
    B2 H2 T16 D8, causal, eps 1e-6, scale sqrt(8) and per-head [2.5, 3.2]; grads atol 1e-4."""
    rng = np.random.default_rng(123)
    q, k, v, do = (rng.standard_normal((2, 2, 16, 8)).astype(np.float32) for _ in range(4))
    for scale in (math.sqrt(8), np.array([2.5, 3.2], dtype=np.float32)):
        sc_t = torch.as_tensor(np.asarray(scale, dtype=np.float32), device=cuda_device)
        t = [torch.as_tensor(x, device=cuda_device) for x in (q, k, v, do)]
        out, dq, dk, dv, ds = _grads(*t, sc_t, is_causal=True, eps=1e-6)
        o_ref, _ = orc.forward(q, k, v, np.asarray(scale, np.float64), True, 1e-6)
        ref = orc.backward(q, k, v, np.asarray(scale, np.float64), do, True, 1e-6, out=f64(out))
        assert max_abs(f64(out), o_ref) <= 1e-5
        for got, want in zip((dq, dk, dv), ref[:3]):
            assert max_abs(f64(got), want) <= 1e-4
        assert max_abs(f64(ds).reshape(-1), ref[3]) <= 1e-4


def test_bwd_mixed_input_dtypes(cuda_device):
    """Compute dtype is v.dtype; grads come back in each input's own dtype."""
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((1, 2, 64, 32), seed=4, n=4))
    out, dq, dk, dv, ds = _grads(q, k.bfloat16(), v.bfloat16(), do.bfloat16(), torch.tensor(4.0, device=cuda_device))
    assert out.dtype == torch.bfloat16
    assert dq.dtype == torch.float32 and dk.dtype == torch.bfloat16 and dv.dtype == torch.bfloat16
    ref = orc.backward(f64(q.bfloat16()), f64(k.bfloat16()), f64(v.bfloat16()), 4.0, f64(do.bfloat16()),
                       out=f64(out))
    assert rel_err(f64(dq), ref[0]) <= 2e-2


def test_bwd_deterministic(cuda_device):
    q, k, v, do = (x.to(cuda_device, torch.bfloat16) for x in seeded_inputs((2, 4, 300, 64), seed=8, n=4))
    sc = torch.tensor([1.0, 2.0, 3.0, 4.0], device=cuda_device)
    a = _grads(q, k, v, do, sc, eps=1e-3)
    b = _grads(q, k, v, do, sc, eps=1e-3)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_bwd_empty(cuda_device):
    from quantumdlblocks_amd import flash_born_attention

    for shape in ((0, 2, 16, 64), (1, 2, 0, 64)):
        q = torch.zeros(shape, device=cuda_device, dtype=torch.bfloat16, requires_grad=True)
        sc = torch.tensor(2.0, device=cuda_device, requires_grad=True)
        out = flash_born_attention(q, q, q, sc)
        out.sum().backward()
        torch.cuda.synchronize()
        assert q.grad.shape == shape and sc.grad.item() == 0.0


def test_bwd_exact_oracle_end_to_end(cuda_device):
    """Well-conditioned case (non-causal, every row sees 256 keys): the GPU
    gradients also match the oracle that forms delta from its own exact O."""
    q, k, v, do = (x.to(cuda_device) for x in seeded_inputs((1, 4, 256, 64), seed=1, n=4))
    for dtype in (torch.float32, torch.bfloat16):
        t = [x.to(dtype) for x in (q, k, v, do)]
        _, dq, dk, dv, _ = _grads(*t, torch.tensor(8.0, device=cuda_device), is_causal=False)
        ref = orc.backward(f64(t[0]), f64(t[1]), f64(t[2]), 8.0, f64(t[3]), False)
        for got, want in zip((dq, dk, dv), ref[:3]):
            assert rel_err(f64(got), want) <= TOL[dtype] * (10 if dtype == torch.float32 else 1)


# Heads checked at C4 / C5 (as in test_gpu_forward.py): every batch row and
# head index, each residue of b * H + h modulo 8 twice.
C5_HEADS = [(b, (5 * b + 3) % 16) for b in range(16)]
C4_HEADS = [(b, 4 * j + (b + j) % 4) for b in range(4) for j in range(4)]


def test_bwd_config_c5(cuda_device):
    """C5: bf16 B16 H16 T2048 D64 forward + backward, N(0,1); 16 heads vs the oracle."""
    _check_bwd(16, 16, 2048, 64, torch.bfloat16, cuda_device, heads=C5_HEADS)


def test_bwd_config_c4_documents(cuda_device):
    """C4's shape with the backward (document-masked training); 16 heads,
    document by document."""
    doc = orc.geometric_doc_ids(4, 8192, 512.0, seed=0)
    _check_bwd(4, 16, 8192, 64, torch.bfloat16, cuda_device, doc=doc, heads=C4_HEADS)
