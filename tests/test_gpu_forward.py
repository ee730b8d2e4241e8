"""GPU parity of the flash-Born forward (HIP kernels via the C ABI) against the
float64 CPU oracle on the same (dtype-rounded) inputs.

Tolerances (normwise relative error max|out-ref|/max|ref|): 1e-5 for fp32,
2e-2 for bf16 / fp16, as stated for this path; max-abs error is printed.

fp16 runs the reference's own weight arithmetic (p = (s q.k)^2 in fp32,
rounded to fp16 as the P.V operand, Z from the fp32 weights), so fp16 cases
are held to the oracle that rounds the weights the same way, every row of O
to 2e-2; their default inputs are N(0, 0.25), which keeps (s q.k)^2 inside
fp16's range at scale 8 (beyond 65504 the reference's fp16 weights overflow,
and the kernel's with them).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc
from util import TOL, abi_forward, f64, max_abs, oracle_forward_heads, rel_err, row_errors, seeded_inputs

pytestmark = pytest.mark.gpu


def _run(q, k, v, scale, **kw):
    from quantumdlblocks_amd import flash_born_attention

    out = flash_born_attention(q, k, v, scale, **kw)
    torch.cuda.synchronize()
    return out


def _check_fwd(B, H, T, D, dtype, dev, *, scale=8.0, is_causal=True, eps=1e-12, window_size=0,
               doc=None, std=None, seed=0, heads=None, tol=None, inputs=None, weight_dtype="auto", row_tol="auto"):
    """Run the public entry on seeded inputs and hold O to the oracle
    (normwise relative error <= tol) and Z, read through the C ABI, to the
    oracle row by row within the rounding bound of the weights
    (util.z_row_bound).  ``heads``: the (b, h) heads to check, or "all".
    ``weight_dtype``: the oracle rounds the P.V weights as the reference's
    kernel does (oracle.forward); ``row_tol``: every row of O is also held to
    it (per-row normwise error; the worst row is printed either way).  fp16
    defaults: std 0.5, weights rounded to fp16 in the oracle, rows to 2e-2."""
    f16 = dtype == torch.float16
    std = (0.5 if f16 else 1.0) if std is None else std
    weight_dtype = ("f16" if f16 else None) if weight_dtype == "auto" else weight_dtype
    row_tol = (2e-2 if f16 else None) if row_tol == "auto" else row_tol
    if inputs is None:
        q, k, v = (x.to(dev) for x in seeded_inputs((B, H, T, D), seed=seed, std=std, dtype=dtype))
    else:
        q, k, v = inputs
    doc_t = None if doc is None else torch.as_tensor(doc, dtype=torch.int32, device=dev)
    scale_arg = scale
    if isinstance(scale, np.ndarray):
        scale_arg = torch.as_tensor(scale, dtype=torch.float32, device=dev)
    out = _run(q, k, v, scale_arg, is_causal=is_causal, eps=eps, window_size=window_size, doc_ids=doc_t)
    assert out.shape == (B, H, T, D) and out.dtype == dtype
    z = None
    if D % 8 == 0 and D <= 256:
        out2, z = abi_forward(q.contiguous(), k.contiguous(), v.contiguous(), scale, is_causal, eps,
                              window_size, doc)
        iv = torch.int32 if dtype == torch.float32 else torch.int16
        assert torch.equal(out2.view(iv), out.view(iv)), "host entry and C ABI disagree"
    sel = [(b, h) for b in range(B) for h in range(H)] if heads in (None, "all") else heads
    sc = np.asarray(scale, dtype=np.float64).reshape(-1)
    qn, kn, vn = f64(q), f64(k), f64(v)
    keys, ref, zref, zb = oracle_forward_heads(qn, kn, vn, sc, sel, is_causal, eps, window_size, doc, dtype,
                                               weight_dtype=weight_dtype)
    got = np.stack([f64(out[b, h]) for b, h in keys])
    rows = row_errors(got, ref) if eps != 0.0 else np.zeros(1)
    if eps == 0.0:
        # rows with no positive overlap are 0/0 in the reference formula: NaN
        # must appear exactly there, everything else is compared
        finite = np.isfinite(ref)
        assert np.array_equal(np.isfinite(got), finite)
        got, ref = got[finite], ref[finite]
    err = rel_err(got, ref)
    zmsg = ""
    if z is not None:
        zg = np.stack([f64(z[b, h]) for b, h in keys])
        zerr = np.abs(zg - zref)
        zratio = float((zerr / np.maximum(zb, 1e-300)).max()) if zerr.size else 0.0
        zrel = float((zerr / np.maximum(np.abs(zref), 1e-300)).max()) if zerr.size else 0.0
        zmsg = f" Z: max row rel={zrel:.3e} (max err/bound {zratio:.3f})"
    print(f"fwd B{B} H{H} T{T} D{D} {dtype} causal={is_causal} W={window_size} doc={doc is not None} "
          f"heads={len(keys)} rel={err:.3e} maxabs={max_abs(got, ref):.3e} worst row={rows.max():.3e}"
          f"{' (weights ' + weight_dtype + ')' if weight_dtype else ''}{zmsg}", flush=True)
    assert np.isfinite(got).all()
    assert err <= (tol or TOL[dtype]), err
    if row_tol is not None:
        assert rows.max() <= row_tol, f"worst row of O: {rows.max():.3e}"
    if z is not None:
        assert np.all(zerr <= zb), f"Z outside its rounding bound: {zratio}"
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("is_causal", [True, False])
def test_fwd_c1_shape(cuda_device, dtype, is_causal):
    """Config C1's shape (B1 H4 T256 D64) on the GPU, every dtype."""
    _check_fwd(1, 4, 256, 64, dtype, cuda_device, is_causal=is_causal)


@pytest.mark.parametrize("T", [1, 2, 7, 31, 64, 65, 100, 257])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fwd_ragged_lengths(cuda_device, T, dtype):
    _check_fwd(2, 3, T, 64, dtype, cuda_device, seed=T)


@pytest.mark.parametrize("T", [300, 513, 600, 777, 1100])
@pytest.mark.parametrize("is_causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [8.0, -3.0])
def test_fwd_d64_block_pairs(cuda_device, T, is_causal, dtype, scale):
    """D = 64 without masks pairs 256-row query blocks mb and nmb-1-mb in one
    workgroup: even and odd block counts, ragged last blocks, both scale signs."""
    _check_fwd(1, 2, T, 64, dtype, cuda_device, scale=scale, is_causal=is_causal, seed=T)


@pytest.mark.parametrize("T", [513, 700, 1024, 1100, 1600])
@pytest.mark.parametrize("is_causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fwd_d64_many_heads(cuda_device, T, is_causal, dtype):
    """D = 64 with enough heads for the paired launch at scale (two 256-row
    blocks per workgroup, two workgroups per CU): even and odd block counts,
    ragged last blocks, per-head scales of both signs; heads covering every
    residue of the pair index and batch row."""
    B, H = 2, 160
    sc = np.linspace(-9.0, 9.0, H).astype(np.float32)
    sc[H // 2] = 8.0
    sel = [(b, (37 * b + 11 * j) % H) for b in range(B) for j in range(4)]
    _check_fwd(B, H, T, 64, dtype, cuda_device, scale=sc, is_causal=is_causal, std=0.125, seed=T, heads=sel)


@pytest.mark.parametrize("D, window", [(64, 0), (64, 100), (32, 0), (128, 0)])
@pytest.mark.parametrize("scale", [0.05, -0.3, 8.0])
def test_fwd_f16_weight_range(cuda_device, D, window, scale):
    """fp16 weights saturate at 65504.  With |q.k| up to ~600 a small scale
    keeps the reference's (s q.k)^2 in range, and so must the kernel, whose
    fp16 weights are the reference's own (s r)^2; every row of O is held to
    the oracle that rounds the weights as the reference's kernel does."""
    std = 4.0 if abs(scale) < 1 else 0.5
    _check_fwd(1, 2, 300, D, torch.float16, cuda_device, scale=scale, std=std, window_size=window, seed=3,
               weight_dtype="f16", row_tol=2e-2)


@pytest.mark.parametrize("D", [64, 128, 48])
@pytest.mark.parametrize("scale", [8.0, -8.0, 0.5])
def test_fwd_f16_tiny_overlaps_flush_like_the_reference(cuda_device, D, scale):
    """One-key rows (causal window 1) whose single weight p = (s q.k)^2 sits
    around fp16's subnormal range: the reference's kernel rounds p to fp16 for
    P.V (flash_born.py:183), so a row keeps v (p a subnormal) or drops to 0
    (p below half the smallest subnormal, 2^-25) exactly where the rounded p
    does.  q.k is exact (one non-zero coordinate each), and every row of O is
    held to the oracle that rounds the weights the same way; the kernels that
    squared min(|s|, 1) q.k flushed rows whose weight the reference keeps."""
    from quantumdlblocks_amd import flash_born_attention

    dev = cuda_device
    T = 64
    targets = 2.0 ** -np.linspace(8, 30, T)  # weights p from 2^-8 down to 2^-30
    r = np.sqrt(targets) / abs(scale)
    q = np.zeros((1, 2, T, D), np.float32)
    k = np.zeros((1, 2, T, D), np.float32)
    q[0, :, :, 3] = r.astype(np.float16).astype(np.float32)
    k[0, :, :, 3] = 1.0
    k[0, 1, :, 3] = np.sign(scale)  # head 1: positive overlaps under either sign of the scale
    g = torch.Generator().manual_seed(D)
    v = torch.randn(1, 2, T, D, generator=g)
    qt, kt, vt = (torch.as_tensor(x).to(dev, torch.float16) for x in (q, k, v))
    out = flash_born_attention(qt, kt, vt, scale, window_size=1)
    torch.cuda.synchronize()
    ref, _ = orc.forward(f64(qt), f64(kt), f64(vt), scale, True, 1e-12, 1, weight_dtype="f16")
    exact, _ = orc.forward(f64(qt), f64(kt), f64(vt), scale, True, 1e-12, 1)
    got = f64(out)
    rows = row_errors(got, ref)
    kept = np.abs(ref).max(-1) > 0
    print(f"f16 one-key rows D{D} s={scale}: kept {int(kept.sum())} of {kept.size}, worst row {rows.max():.3e}, "
          f"rows the exact oracle keeps {int((np.abs(exact).max(-1) > 0).sum())}", flush=True)
    assert kept.sum() > 0 and (~kept).sum() > 0, "the rows must span the flush threshold"
    assert rows.max() <= 2e-3, rows.max()


@pytest.mark.parametrize("D", [8, 16, 24, 32, 40, 48, 80, 96, 112, 128, 160, 192, 256, 20, 3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fwd_head_dims(cuda_device, D, dtype):
    """Every head dim up to 256; D not a multiple of 8 is zero-padded by the host."""
    _check_fwd(2, 2, 96, D, dtype, cuda_device, scale=1.0 / math.sqrt(D), seed=D)


@pytest.mark.parametrize("D", [136, 200, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", [(True, 0, 1), (True, 0, 64), (True, 0, 129), (True, 0, 700), (False, 0, 300),
                                  (True, 1, 300), (True, 63, 300), (True, 200, 700), (False, 1, 300),
                                  (False, 64, 300), (False, 129, 700), (False, 1000, 300)])
def test_fwd_wide_dma_kernel(cuda_device, D, dtype, case):
    """128 < D <= 256 without documents: the DMA-ring forward (4 waves over
    128 query rows, 64-key tiles through a two-stage ring); padded head dims
    (136, 200: zero columns past D), one and several blocks, a partial last
    tile and block, causal and dense, windows with and without causality
    shorter and longer than T; per-head scales (one negative); O and Z."""
    is_causal, window, T = case
    _check_fwd(1, 2, T, D, dtype, cuda_device, is_causal=is_causal, window_size=window,
               scale=np.array([0.3, -0.15], dtype=np.float32), std=0.5, seed=D + T + window)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [72, 96, 120])
@pytest.mark.parametrize("is_causal, window", [(True, 0), (False, 0), (True, 100)])
def test_fwd_padded_documents(cuda_device, dtype, D, is_causal, window):
    """64 < D < 128 with document ids on the D = 128 kernel's document mode
    with zero columns past D (dense, causal, causal window); O and Z."""
    doc = orc.geometric_doc_ids(2, 700, 90.0, seed=D + window)
    _check_fwd(2, 2, 700, D, dtype, cuda_device, doc=doc, is_causal=is_causal, window_size=window,
               scale=np.array([0.3, -0.15], dtype=np.float32), std=0.5, seed=D + 9)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [136, 256])
@pytest.mark.parametrize("is_causal, window", [(True, 0), (False, 0), (True, 100)])
def test_fwd_wide_documents(cuda_device, dtype, D, is_causal, window):
    """128 < D <= 256 with document ids (dense, causal, causal window) on the
    wide-row forward's document mode; padded and unpadded head dims,
    per-head scales; O and Z."""
    doc = orc.geometric_doc_ids(2, 700, 90.0, seed=D + window)
    _check_fwd(2, 2, 700, D, dtype, cuda_device, doc=doc, is_causal=is_causal, window_size=window,
               scale=np.array([0.3, -0.15], dtype=np.float32), std=0.5, seed=D + 5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [272, 320])
def test_fwd_head_dims_above_256_take_the_eager_path(cuda_device, D, dtype):
    """Head dims the kernels do not take run the reference's eager
    formulation on the GPU, as the reference does for every head dim its
    kernel does not support (flash_born.py:670-690)."""
    _check_fwd(1, 2, 80, D, dtype, cuda_device, scale=1.0 / math.sqrt(D), seed=D)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("window", [1, 5, 64, 100, 1000])
@pytest.mark.parametrize("is_causal", [True, False])
def test_fwd_sliding_window(cuda_device, dtype, window, is_causal):
    _check_fwd(2, 2, 200, 64, dtype, cuda_device, is_causal=is_causal, window_size=window, seed=window)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [1, 63, 64, 65, 100, 255, 256, 257, 320, 512, 900])
def test_fwd_sliding_window_fast_kernel(cuda_device, dtype, window):
    """Causal windows at D = 64 run the fast kernel's window mode: windows
    that start inside, on and beside the 64-key tile and 256-row block
    edges, longer than T, over several blocks and a partial last block."""
    _check_fwd(2, 2, 1100, 64, dtype, cuda_device, window_size=window, seed=window + 7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [1, 63, 64, 65, 100, 255, 256, 257, 320, 512, 900, 2000])
def test_fwd_sliding_window_noncausal_fast_kernel(cuda_device, dtype, window):
    """Windows without causality at D = 64 (row i sees keys i - W + 1 ..
    T - 1, flash_born.py:173-174) run the fast kernel's kWindowNC mode: one
    block per workgroup, the first blocks first; windows starting inside, on
    and beside the 64-key tile and 256-row block edges, longer than T, a
    partial last tile and block."""
    _check_fwd(2, 2, 1100, 64, dtype, cuda_device, is_causal=False, window_size=window, seed=window + 9)


@pytest.mark.parametrize("T", [1, 37, 64, 255, 256, 300, 513])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("window", [1, 3, 100])
def test_fwd_noncausal_window_ragged(cuda_device, T, D, window):
    """kWindowNC on ragged lengths: a single partial tile, T on and beside
    the tile and block edges, windows shorter and longer than T."""
    _check_fwd(1, 2, T, D, torch.bfloat16, cuda_device, is_causal=False, window_size=window,
               scale=8.0 if D == 64 else 0.09, seed=T + window)


@pytest.mark.parametrize("T", [1, 37, 64, 255, 256, 300, 513, 777, 1100])
@pytest.mark.parametrize("is_causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [0.09, -0.5])
def test_fwd_d128_kernel(cuda_device, T, is_causal, dtype, scale):
    """D = 128 without documents runs its own kernel (8 waves over 256-row
    query blocks, 32 rows per wave): ragged lengths, one to five blocks,
    both scale signs (unpaired launch: too few heads to pair)."""
    _check_fwd(1, 2, T, 128, dtype, cuda_device, scale=scale, is_causal=is_causal, seed=T + 1)


@pytest.mark.parametrize("B,H,T", [(4, 32, 700), (5, 17, 1100), (2, 64, 1024), (8, 10, 1100)])
@pytest.mark.parametrize("is_causal", [True, False])
def test_fwd_d128_block_pairs(cuda_device, B, H, T, is_causal):
    """Shapes where the launch pairs blocks (mb and nmb-1-mb in one
    workgroup, the odd block count's middle block alone: every dense case,
    causal T 700, 1024 and 1100 with 85 heads) and where it does not (causal
    T 1100 with 80 heads: the pairs would run 1.25 rounds); per-head scales of
    both signs; heads covering every residue of the pair index."""
    sc = np.linspace(-0.2, 0.2, H).astype(np.float32)
    sc[H // 2] = 0.13
    sel = [(b, (7 * b + 5 * j) % H) for b in range(B) for j in range(3)]
    _check_fwd(B, H, T, 128, torch.bfloat16, cuda_device, scale=sc, is_causal=is_causal, std=0.5, seed=T,
               heads=sel)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [1, 31, 32, 33, 64, 100, 255, 256, 257, 512, 900])
def test_fwd_d128_sliding_window(cuda_device, dtype, window):
    """Causal windows at D = 128: windows starting inside, on and beside a
    wave's 32 rows, a 64-key tile and a 256-row block, longer than T."""
    _check_fwd(2, 2, 1100, 128, dtype, cuda_device, window_size=window, scale=0.09, seed=window + 11)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [1, 31, 32, 33, 64, 100, 255, 256, 257, 900, 2000])
def test_fwd_d128_sliding_window_noncausal(cuda_device, dtype, window):
    """Windows without causality at D = 128: the D = 128 kernel's kWindowNC
    mode (per-wave runs from the window's first key to T, one block per
    workgroup, the first blocks first)."""
    _check_fwd(2, 2, 1100, 128, dtype, cuda_device, is_causal=False, window_size=window, scale=0.09,
               seed=window + 15)


@pytest.mark.parametrize("D", [104, 112, 120])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["causal", "dense", "window"])
def test_fwd_d128_padded_head_dims(cuda_device, D, dtype, mode):
    """96 < D < 128 runs the D = 128 kernel with the columns past D loaded as
    zeros and not stored: ragged T, causal, dense and a causal window."""
    kw = dict(is_causal=mode != "dense", window_size=100 if mode == "window" else 0)
    _check_fwd(2, 2, 777, D, dtype, cuda_device, scale=0.11, seed=D, **kw)
    _check_fwd(4, 32, 300, D, dtype, cuda_device, scale=0.11, seed=D + 1, heads=[(0, 0), (1, 7), (3, 31)], **kw)


def test_fwd_d128_config_d3(cuda_device):
    """d3: bf16 B16 H8 T1024 D128 causal (the C3 work at head dim 128),
    N(0, 1/128); 16 heads covering every batch row and workgroup residue."""
    sel = [(b, (3 * b + 1) % 8) for b in range(16)]
    _check_fwd(16, 8, 1024, 128, torch.bfloat16, cuda_device, scale=1.0, std=128 ** -0.5, heads=sel)


def test_fwd_sliding_window_c3_shape(cuda_device):
    """C3's shape with a 256-key window, 16 heads covering every block
    residue of the launch."""
    sel = [(b, b) for b in range(16)]
    _check_fwd(16, 16, 1024, 64, torch.bfloat16, cuda_device, window_size=256, std=0.125, heads=sel)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("is_causal", [True, False])
def test_fwd_document_mask(cuda_device, dtype, is_causal):
    doc = orc.geometric_doc_ids(3, 300, 40.0, seed=1)
    _check_fwd(3, 2, 300, 64, dtype, cuda_device, is_causal=is_causal, doc=doc)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 96, 128, 200, 256])
@pytest.mark.parametrize("is_causal", [True, False])
def test_fwd_unsorted_document_ids(cuda_device, dtype, D, is_causal):
    """Arbitrary (unsorted, repeating) document ids: the kernels' tile
    screening by document-id range must stay conservative (D = 96 and 200:
    the document modes with zero columns past D)."""
    rng = np.random.default_rng(D)
    doc = rng.integers(0, 4, size=(2, 700)).astype(np.int32)
    doc[1, 350:] = rng.integers(10, 12, size=350)
    _check_fwd(2, 2, 700, D, dtype, cuda_device, is_causal=is_causal, doc=doc, seed=D)


@pytest.mark.parametrize("T, D", [(20000, 64), (9000, 256)])
def test_fwd_documents_many_tiles(cuda_device, T, D):
    """Sorted documents over more candidate key tiles than one screening pass
    holds (256 tiles): every document, checked against the oracle on its own
    span (documents do not see each other, so the span is exact)."""
    from quantumdlblocks_amd import flash_born_attention

    doc = orc.geometric_doc_ids(1, T, 300.0, seed=T)
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((1, 2, T, D), seed=7, std=0.5, dtype=torch.bfloat16))
    out = flash_born_attention(q, k, v, 8.0, doc_ids=torch.as_tensor(doc, device=cuda_device))
    got = f64(out)
    qn, kn, vn = f64(q), f64(k), f64(v)
    ids = doc[0]
    starts = np.flatnonzero(np.r_[True, ids[1:] != ids[:-1]])
    ends = np.r_[starts[1:], T]
    worst = 0.0
    for s, e in zip(starts, ends):
        ref, _ = orc.forward(qn[:, :, s:e], kn[:, :, s:e], vn[:, :, s:e], 8.0, True, 1e-12)
        worst = max(worst, rel_err(got[:, :, s:e], ref))
    print(f"documents T={T} D={D}: {len(starts)} docs, worst rel={worst:.3e}", flush=True)
    assert worst <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("is_causal", [True, False])
def test_fwd_d128_documents(cuda_device, dtype, is_causal):
    """D = 128 with document ids (no window) runs the D = 128 kernel's
    document mode: geometric documents with T not a multiple of the tile or
    block, per-head scales (one negative); documents whose edges sit on and
    beside the 32-row wave slices, 64-key tiles and 256-row blocks, one-token
    documents, negative ids and a descending batch row; unsorted ids."""
    doc = orc.geometric_doc_ids(2, 1100, 90.0, seed=3)
    _check_fwd(2, 3, 1100, 128, dtype, cuda_device, is_causal=is_causal, doc=doc,
               scale=np.array([0.3, -0.2, 0.1], np.float32), std=0.7, seed=3)
    lens = [64, 1, 63, 129, 256, 1, 1, 31, 97, 200, 65, 12, 33, 32, 288]
    ids = np.concatenate([np.full(n, i - 3, np.int32) for i, n in enumerate(lens)])
    _check_fwd(2, 2, ids.size, 128, dtype, cuda_device, is_causal=is_causal, doc=np.stack([ids, -ids[::-1]]),
               scale=0.2, std=0.7, seed=5)
    rng = np.random.default_rng(7)
    doc = rng.integers(0, 3, size=(1, 600)).astype(np.int32)
    _check_fwd(1, 2, 600, 128, dtype, cuda_device, is_causal=is_causal, doc=doc, scale=0.2, std=0.7, seed=7)


# A one-key window leaves each row a single weight, which fp16 rounds for
# P.V as the reference's kernel does (a tiny overlap's row drops to 0 with
# it): the fp16 rows are held, row by row, to the oracle that rounds the
# weights likewise (_check_fwd's fp16 default).
WINDOW_DOC_CASES = [(d, w) for d in (torch.bfloat16, torch.float16) for w in (1, 33, 100, 300, 2000)]


@pytest.mark.parametrize("dtype,window", WINDOW_DOC_CASES)
def test_fwd_documents_and_window_fast(cuda_device, dtype, window):
    """D = 64 with document ids and a causal sliding window: the document
    kernel's window mode (candidates from the block's first window, window
    edges tested per element in both column blocks)."""
    doc = orc.geometric_doc_ids(2, 1100, 150.0, seed=window)
    _check_fwd(2, 3, 1100, 64, dtype, cuda_device, doc=doc, window_size=window, scale=0.5, std=0.7,
               seed=window + 1)
    lens = [64, 1, 63, 129, 256, 1, 1, 31, 97, 200, 65, 12, 33, 32, 288]
    ids = np.concatenate([np.full(n, i - 3, np.int32) for i, n in enumerate(lens)])
    _check_fwd(2, 2, ids.size, 64, dtype, cuda_device, doc=np.stack([ids, -ids[::-1]]), window_size=window,
               scale=0.5, std=0.7, seed=window + 3)


@pytest.mark.parametrize("dtype,window", WINDOW_DOC_CASES)
def test_fwd_d128_documents_and_window(cuda_device, dtype, window):
    """D = 128 with document ids and a causal sliding window: the document
    mode's window bounds (candidate tiles from the block's first window,
    per-wave skips and per-element tests at the window edge)."""
    doc = orc.geometric_doc_ids(2, 1100, 150.0, seed=window)
    _check_fwd(2, 2, 1100, 128, dtype, cuda_device, doc=doc, window_size=window, scale=0.2, std=0.7,
               seed=window + 2)


def test_fwd_d128_documents_many_tiles(cuda_device):
    """D = 128, sorted documents over more candidate key tiles than one
    screening pass holds (256 tiles): every document against the oracle on
    its own span."""
    from quantumdlblocks_amd import flash_born_attention

    T, D = 17000, 128
    doc = np.zeros((1, T), dtype=np.int32)
    doc[0, 3000:12000] = 1
    doc[0, 12000:] = 2 + orc.geometric_doc_ids(1, T - 12000, 700.0, seed=11)[0]
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((1, 2, T, D), seed=9, std=0.3, dtype=torch.bfloat16))
    out = flash_born_attention(q, k, v, 1.0, doc_ids=torch.as_tensor(doc, device=cuda_device))
    got = f64(out)
    qn, kn, vn = f64(q), f64(k), f64(v)
    ids = doc[0]
    starts = np.flatnonzero(np.r_[True, ids[1:] != ids[:-1]])
    ends = np.r_[starts[1:], T]
    worst = 0.0
    for s, e in zip(starts, ends):
        ref, _ = orc.forward(qn[:, :, s:e], kn[:, :, s:e], vn[:, :, s:e], 1.0, True, 1e-12)
        worst = max(worst, rel_err(got[:, :, s:e], ref))
    print(f"documents T={T} D={D}: {len(starts)} docs, worst rel={worst:.3e}", flush=True)
    assert worst <= 2e-2


def test_fwd_d128_config_c4_documents(cuda_device):
    """C4's documents at head dim 128 (dc4: B4 H8 T8192 D128); 16 heads."""
    doc = orc.geometric_doc_ids(4, 8192, 512.0, seed=0)
    sel = [(b, (3 * b + j) % 8) for b in range(4) for j in range(4)]
    _check_fwd(4, 8, 8192, 128, torch.bfloat16, cuda_device, doc=doc, scale=1.0, std=128 ** -0.5, heads=sel)


def test_fwd_document_and_window(cuda_device):
    doc = orc.geometric_doc_ids(2, 333, 60.0, seed=2)
    _check_fwd(2, 4, 333, 64, torch.bfloat16, cuda_device, window_size=37, doc=doc)
    _check_fwd(2, 4, 333, 64, torch.float32, cuda_device, window_size=37, doc=doc)


def test_fwd_reference_doc_literal(cuda_device):
    """The reference's own window + document case (test_hypothesis_016:179-206):
    B2 H4 T8 D16, window 4, scale 10, doc ids from the literal EOT example."""
    from quantumdlblocks_amd import compute_document_ids, l2_normalize

    idx = torch.tensor([[10, 20, 50256, 30, 40, 50256, 50, 60], [11, 50256, 22, 33, 44, 55, 66, 77]])
    doc = compute_document_ids(idx)
    torch.manual_seed(2)
    q = l2_normalize(torch.randn(2, 4, 8, 16), dim=-1)
    k = l2_normalize(0.85 * q + 0.15 * torch.randn(2, 4, 8, 16), dim=-1)
    v = l2_normalize(torch.randn(2, 4, 8, 16), dim=-1)
    out = _run(q.to(cuda_device), k.to(cuda_device), v.to(cuda_device), 10.0, window_size=4,
               doc_ids=doc.to(cuda_device))
    ref, _ = orc.forward(f64(q), f64(k), f64(v), 10.0, True, 1e-12, 4, doc.numpy())
    assert rel_err(f64(out), ref) <= 1e-5
    assert max_abs(f64(out), ref) <= 1e-3  # the reference's own GPU-vs-CPU bound


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fwd_per_head_and_signed_scales(cuda_device, dtype):
    H = 4
    for scale in (np.array([2.5, 3.2, 0.5, 7.0]), np.array([-1.5, 2.0, -8.0, 1.0]), np.array([0.0, 1.0, 0.0, 3.0])):
        _check_fwd(2, H, 130, 64, dtype, cuda_device, scale=scale.astype(np.float32))
    for s in (-8.0, 0.0, 1e-3, 100.0):
        _check_fwd(2, H, 70, 64, dtype, cuda_device, scale=s)


def test_fwd_scale_shapes(cuda_device):
    """scale as float, 0-d, (1,), (H,), (1,H,1,1) tensors (flash_born.py:452-453, 681-683)."""
    B, H, T, D = 2, 3, 50, 32
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((B, H, T, D), seed=5))
    sc = torch.tensor([1.5, 4.0, 9.0], device=cuda_device)
    outs = [
        _run(q, k, v, sc),
        _run(q, k, v, sc.view(1, H, 1, 1)),
    ]
    ref, _ = orc.forward(f64(q), f64(k), f64(v), sc.cpu().numpy(), True, 1e-12)
    for o in outs:
        assert rel_err(f64(o), ref) <= 1e-5
    for s in (3.0, torch.tensor(3.0, device=cuda_device), torch.tensor([3.0], device=cuda_device)):
        o = _run(q, k, v, s)
        ref, _ = orc.forward(f64(q), f64(k), f64(v), 3.0, True, 1e-12)
        assert rel_err(f64(o), ref) <= 1e-5


@pytest.mark.parametrize("eps", [0.0, 1e-12, 1e-6, 1.0])
def test_fwd_eps(cuda_device, eps):
    _check_fwd(1, 2, 64, 64, torch.float32, cuda_device, eps=eps, std=0.2)
    _check_fwd(1, 2, 64, 64, torch.bfloat16, cuda_device, eps=eps, std=0.2)


def test_fwd_all_negative_overlaps_give_zero(cuda_device):
    """Keys anti-aligned with every query: every weight is relu(<0)^2 = 0, so O = 0."""
    B, H, T, D = 1, 2, 96, 64
    (base,) = seeded_inputs((1, 1, 1, D), seed=9, n=1)
    q = base.expand(B, H, T, D).abs().contiguous()
    k = -q.clone()
    (v,) = seeded_inputs((B, H, T, D), seed=10, n=1)
    for dtype in (torch.bfloat16, torch.float32):
        out = _run(q.to(cuda_device, dtype), k.to(cuda_device, dtype), v.to(cuda_device, dtype), 8.0)
        assert torch.count_nonzero(out).item() == 0


def test_fwd_empty_and_non_contiguous(cuda_device):
    for shape in ((0, 2, 16, 64), (1, 0, 16, 64), (1, 2, 0, 64)):
        q = torch.zeros(shape, device=cuda_device, dtype=torch.bfloat16)
        assert _run(q, q, q, 8.0).shape == shape
    # (B, T, H, D) storage viewed as (B, H, T, D): the host makes it contiguous.
    x = torch.randn(2, 40, 3, 64, device=cuda_device).transpose(1, 2)
    out = _run(x, x, x, 8.0)
    ref, _ = orc.forward(f64(x), f64(x), f64(x), 8.0)
    assert rel_err(f64(out), ref) <= 1e-5
    # a storage offset that breaks 16-byte alignment
    y = torch.randn(1 * 2 * 33 * 64 + 3, device=cuda_device)[3:].view(1, 2, 33, 64)
    out = _run(y, y, y, 8.0)
    ref, _ = orc.forward(f64(y), f64(y), f64(y), 8.0)
    assert rel_err(f64(out), ref) <= 1e-5


def test_fwd_autocast(cuda_device):
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((1, 2, 64, 64), seed=3))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = _run(q, k, v, 8.0)
    assert out.dtype == torch.bfloat16
    ref, _ = orc.forward(f64(q.bfloat16()), f64(k.bfloat16()), f64(v.bfloat16()), 8.0)
    assert rel_err(f64(out), ref) <= 2e-2


# ---- BASELINE.json configs at full size (subsets of heads vs the oracle) ----

# Heads checked at C4 / C5: every batch row and every head index, each
# residue of b * H + h modulo 8 (the XCD a workgroup of that head lands on)
# twice; C2 and C3 check every head.
C5_HEADS = [(b, (5 * b + 3) % 16) for b in range(16)]
C4_HEADS = [(b, 4 * j + (b + j) % 4) for b in range(4) for j in range(4)]


def test_fwd_config_c2(cuda_device):
    """C2: bf16 B32 H4 T1024 D64, Q and K L2-normalised per head vector; every head."""
    from quantumdlblocks_amd import l2_normalize

    B, H, T, D = 32, 4, 1024, 64
    q, k, v = seeded_inputs((B, H, T, D), seed=0)
    q, k = l2_normalize(q), l2_normalize(k)
    q, k, v = (x.to(cuda_device, torch.bfloat16) for x in (q, k, v))
    _check_fwd(B, H, T, D, torch.bfloat16, cuda_device, heads="all", inputs=(q, k, v))


def test_fwd_config_c2_f16_rows(cuda_device):
    """C2's shape and recipe in fp16 (L2-normalised Q and K, scale 8: many
    overlaps are small, so many weights are fp16 subnormals): every head;
    every row of O within 2e-2 of the oracle that rounds the weights as the
    reference's kernel does, Z within its bound from the reference's fp32
    weights; the worst row against the exact oracle is printed too."""
    from quantumdlblocks_amd import l2_normalize

    B, H, T, D = 32, 4, 1024, 64
    q, k, v = seeded_inputs((B, H, T, D), seed=0)
    q, k = l2_normalize(q), l2_normalize(k)
    q, k, v = (x.to(cuda_device, torch.float16) for x in (q, k, v))
    out = _check_fwd(B, H, T, D, torch.float16, cuda_device, heads="all", inputs=(q, k, v), weight_dtype="f16",
                     row_tol=2e-2)
    exact, _ = orc.forward(f64(q[:2]), f64(k[:2]), f64(v[:2]), 8.0)
    print(f"C2 fp16, batch rows 0-1 against the exact oracle: worst row {row_errors(f64(out[:2]), exact).max():.3e}, "
          f"normwise {rel_err(f64(out[:2]), exact):.3e}", flush=True)


def test_fwd_config_c3(cuda_device):
    """C3 (headline): bf16 B16 H16 T1024 D64, Q, K, V ~ N(0, 1/64); every head."""
    _check_fwd(16, 16, 1024, 64, torch.bfloat16, cuda_device, std=0.125, heads="all")


def test_fwd_config_c4(cuda_device):
    """C4: bf16 B4 H16 T8192 D64, causal within geometric(mean 512) documents;
    16 heads, document by document, and one head against the oracle's full
    document mask (which pins the span-by-span evaluation)."""
    doc = orc.geometric_doc_ids(4, 8192, 512.0, seed=0)
    out = _check_fwd(4, 16, 8192, 64, torch.bfloat16, cuda_device, doc=doc, heads=C4_HEADS)
    q, k, v = (x.to(cuda_device) for x in seeded_inputs((4, 16, 8192, 64), seed=0, dtype=torch.bfloat16))
    ref, _ = orc.forward(f64(q[1:2, 7:8]), f64(k[1:2, 7:8]), f64(v[1:2, 7:8]), 8.0, True, 1e-12, 0, doc[1:2])
    assert rel_err(f64(out[1:2, 7:8]), ref) <= 2e-2


def test_fwd_config_c5_forward(cuda_device):
    """C5's forward: bf16 B16 H16 T2048 D64, N(0,1); 16 heads."""
    _check_fwd(16, 16, 2048, 64, torch.bfloat16, cuda_device, heads=C5_HEADS)


@pytest.mark.parametrize("T", [1024, 2048])
def test_fwd_repeatable_over_stale_lds(cuda_device, T):
    """Regression: every K/V tile is read only after its own load has landed.

    A launch on decoy K/V (different values, same shape) leaves other data in
    the LDS of every CU.  A tile read before its load lands would then pick
    up decoy rows; the error (a few 1e-3 of a bf16 output) can hide inside the
    2e-2 tolerance, so the check is bitwise: the kernel is deterministic, and
    the same inputs must give identical O and Z before and after each decoy
    launch (an earlier version read its second tile's K operands during its
    first tile and failed this at T=2048).
    """
    from quantumdlblocks_amd import _native
    from quantumdlblocks_amd.kernels.flash_born import _DTYPE_CODE

    lib = _native.load()
    B, H, D = 16, 16, 64
    q, k, v = (x.to(cuda_device, torch.bfloat16).contiguous()
               for x in seeded_inputs((B, H, T, D), seed=T, std=0.125))
    kd, vd = (x.to(cuda_device, torch.bfloat16).contiguous()
              for x in seeded_inputs((B, H, T, D), seed=T + 1, std=4.0, n=2))
    scale = torch.tensor(8.0, dtype=torch.float32, device=cuda_device)
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    code = _DTYPE_CODE[torch.bfloat16]

    def fwd(kk, vv):
        out = torch.empty_like(q)
        z = torch.empty((B, H, T), dtype=torch.float32, device=cuda_device)
        rc = lib.qdl_flash_born_fwd(code, B, H, T, D, q.data_ptr(), kk.data_ptr(), vv.data_ptr(),
                                    out.data_ptr(), z.data_ptr(), scale.data_ptr(), 1, None, 1, 0,
                                    1e-12, stream)
        _native.check(rc, "qdl_flash_born_fwd")
        return out, z

    out0, z0 = fwd(k, v)
    for _ in range(5):
        fwd(kd, vd)
        out1, z1 = fwd(k, v)
        torch.cuda.synchronize()
        assert torch.equal(out1.view(torch.int16), out0.view(torch.int16))
        assert torch.equal(z1.view(torch.int32), z0.view(torch.int32))
    heads = [(0, 0), (15, 15), (7, 9)]
    got = np.concatenate([f64(out0[b : b + 1, h : h + 1]) for b, h in heads])
    ref = np.concatenate([orc.forward(f64(q[b : b + 1, h : h + 1]), f64(k[b : b + 1, h : h + 1]),
                                      f64(v[b : b + 1, h : h + 1]), 8.0)[0] for b, h in heads])
    assert rel_err(got, ref) <= 2e-2
