"""Shared helpers for the test suite (inputs, error metrics)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import born_oracle as orc


def seeded_inputs(shape, seed=0, std=1.0, n=3, dtype=torch.float32):
    """n tensors drawn N(0, std^2) in fp32 on the CPU from one generator, in order."""
    g = torch.Generator("cpu").manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype) for _ in range(n)]


def rel_err(out, ref) -> float:
    """Normwise relative error max|out - ref| / max|ref|."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.abs(ref).max() if ref.size else 0.0
    diff = np.abs(out - ref).max() if ref.size else 0.0
    return float(diff / den) if den > 0 else float(diff)


def max_abs(out, ref) -> float:
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(out - ref).max()) if ref.size else 0.0


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().double().numpy()


TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


# ---------------------------------------------------------------------------
# Direct C-ABI forward (returns Z as well as O) and the bound on Z
# ---------------------------------------------------------------------------

def abi_forward(q, k, v, scale, is_causal=True, eps=1e-12, window_size=0, doc=None):
    """qdl_flash_born_fwd on contiguous (B, H, T, D) device tensors (D a
    multiple of 8), returning (out, z) -- z = sum_j p_ij + eps per row, which
    the autograd entry keeps for the backward but does not return."""
    from quantumdlblocks_amd import _native
    from quantumdlblocks_amd.kernels.flash_born import _DTYPE_CODE

    lib = _native.load()
    B, H, T, D = q.shape
    assert D % 8 == 0 and q.is_contiguous() and k.is_contiguous() and v.is_contiguous()
    dev = q.device
    sc = torch.as_tensor(np.asarray(scale, dtype=np.float32).reshape(-1), device=dev)
    doc_t = None if doc is None else torch.as_tensor(np.asarray(doc), dtype=torch.int32, device=dev).contiguous()
    out = torch.empty_like(q)
    z = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    rc = lib.qdl_flash_born_fwd(_DTYPE_CODE[q.dtype], B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                out.data_ptr(), z.data_ptr(), sc.data_ptr(), sc.numel(),
                                None if doc_t is None else doc_t.data_ptr(), 1 if is_causal else 0,
                                int(window_size), float(eps), torch.cuda.current_stream(dev).cuda_stream)
    _native.check(rc, "qdl_flash_born_fwd")
    torch.cuda.synchronize(dev)
    return out, z


# Relative rounding of one weight p' as the kernels form it before it is
# summed into Z.  bf16 rounds p' to bf16 (unit roundoff 2^-8: the row sums are
# formed from the 16-bit weights that feed the P.V product).  fp16 keeps the
# reference's fp32 weight p = (s r)^2 (two fp32 roundings: the scale times the
# overlap, the square), as does fp32.
_Z_UNIT = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -22, torch.float32: 2.0 ** -24}


def z_row_bound(q, k, scale, z_ref, eps, dtype, mask):
    """Per-row bound on |Z_kernel - Z_ref| (float64 arrays, (B, H, T)).

    Z_ref = sum_j p_ij + eps in exact arithmetic on the dtype-rounded inputs;
    the kernel computes r_ij = q_i . k_j in fp32 (exact products of 16-bit or
    fp32 inputs, D-term fp32 sums: |dr| <= D 2^-24 sum_a |q_ia k_ja|), forms
    the weight (bf16: r|r| rounded to bf16, relative u = 2^-8, and 2^-126 s^2
    absolute below bf16's normal range; fp16 and fp32: the fp32 weight, u a
    few fp32 roundings), and sums the n_i visible weights in fp32 (relative
    n_i 2^-23), then scales by s^2 (bf16; 1 for fp16) and adds eps (two more
    roundings).  Hence
      |dZ_i| <= (u + n_i 2^-23 + 2^-22) sum_j p_ij
                + s^2 sum_j m_ij (2|r_ij| + dr_ij) dr_ij + n_i a + 2^-23 eps.
    For fp16 this is the reference's own arithmetic (Z from the fp32 weights,
    flash_born.py:180-182) up to the fp32 summation order.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    D = q.shape[-1]
    H = q.shape[1]
    s = np.asarray(scale, dtype=np.float64).reshape(-1)
    s = (s if s.size > 1 else np.full(H, s[0])).reshape(1, H, 1, 1)
    r = q @ np.swapaxes(k, -1, -2)
    dr = D * 2.0 ** -24 * (np.abs(q) @ np.swapaxes(np.abs(k), -1, -2))
    m = np.broadcast_to(mask, r.shape).astype(np.float64)
    n = m.sum(-1)
    psum = np.asarray(z_ref, dtype=np.float64) - eps
    u = _Z_UNIT[dtype]
    s2 = (s * s)[..., 0]
    term_r = (s * s * m * (2.0 * np.abs(r) + dr) * dr).sum(-1)
    absolute = (2.0 ** -126 if dtype == torch.bfloat16 else 2.0 ** -149) * s2
    return (u + n * 2.0 ** -23 + 2.0 ** -22) * np.abs(psum) + term_r + n * absolute + 2.0 ** -23 * abs(eps)


def row_errors(got, ref, floor=0.0):
    """Per-row normwise relative error of O: max_d |got - ref| / max_d |ref|
    for each row (last axis D), with rows whose reference is 0 judged by their
    absolute error against ``floor``."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    num = np.abs(got - ref).max(-1)
    den = np.abs(ref).max(-1)
    return np.where(den > 0, num / np.where(den > 0, den, 1.0), np.where(num <= floor, 0.0, np.inf))


def doc_spans(row):
    """Contiguous runs [(start, stop)] of equal ids in one batch row, checking
    that no id occurs in two runs (then causal attention within documents is
    causal attention within each run, exactly)."""
    row = np.asarray(row)
    edges = np.flatnonzero(np.diff(row)) + 1
    starts = np.concatenate([[0], edges])
    stops = np.concatenate([edges, [row.size]])
    ids = row[starts]
    assert np.unique(ids).size == ids.size, "document ids are not contiguous runs"
    return list(zip(starts.tolist(), stops.tolist()))


def oracle_forward_heads(qn, kn, vn, sc, sel, is_causal, eps, window_size, doc, dtype, chunk=16,
                         weight_dtype=None):
    """Oracle O and Z for the selected (b, h) heads, and the per-row bound on
    the kernel's Z (util.z_row_bound).  Heads of one batch row are stacked
    into one (1, n, T, D) call.  Causal rows of documents that form
    contiguous runs are computed span by span (rows of one document see only
    keys of that document, so each span is plain causal attention: exact)."""
    T = qn.shape[2]
    by_b = {}
    for b, h in sel:
        by_b.setdefault(b, []).append(h)
    refs, zrefs, bounds, keys = [], [], [], []
    spans_ok = doc is not None and is_causal and window_size == 0 and T > 2048
    for b, hs in by_b.items():
        for i in range(0, len(hs), chunk):
            hh = hs[i : i + chunk]
            s_h = sc[hh] if sc.size > 1 else sc[0]
            if spans_ok:
                o = np.empty((1, len(hh), T, qn.shape[3]))
                z = np.empty((1, len(hh), T))
                bd = np.empty((1, len(hh), T))
                for a, e in doc_spans(doc[b]):
                    qs, ks, vs = (x[b : b + 1, hh, a:e] for x in (qn, kn, vn))
                    o[..., a:e, :], z[..., a:e] = orc.forward(qs, ks, vs, s_h, True, eps, weight_dtype=weight_dtype)
                    bd[..., a:e] = z_row_bound(qs, ks, s_h, z[..., a:e], eps, dtype,
                                               orc.visible_mask(e - a, True, 0))
            else:
                dd = None if doc is None else doc[b : b + 1]
                qs, ks, vs = (x[b : b + 1, hh] for x in (qn, kn, vn))
                o, z = orc.forward(qs, ks, vs, s_h, is_causal, eps, window_size, dd, weight_dtype=weight_dtype)
                bd = z_row_bound(qs, ks, s_h, z, eps, dtype, orc.visible_mask(T, is_causal, window_size, dd))
            refs.append(o)
            zrefs.append(z)
            bounds.append(bd)
            keys += [(b, h) for h in hh]
    return keys, np.concatenate(refs, 1)[0], np.concatenate(zrefs, 1)[0], np.concatenate(bounds, 1)[0]
