"""CPU oracle for the fused Q/K prologue (unitary RoPE then L2 normalisation).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or the timed CPU
baseline).  The product path in ``quantumdlblocks_amd`` never imports it.

It restates, in numpy, what SubspaceProjectorBornAttention.forward does to Q
and K before the attention kernel (``src/qdlblocks/layers/attention.py:573-589``
in Vengo/QuantumDLBlocks), leaving out the optional wave filter and partial
key offset:

  * table padding (attention.py:574-582): with half = D / 2, a table with at
    least ``half`` columns is cut to ``half``; a shorter one is padded with
    cos = 1, sin = 0 (angle 0);
  * ``apply_unitary_rope`` (functional.py:104-121): x1 = x[..., :half],
    x2 = x[..., half:], c = cos.to(x.dtype), s = sin.to(x.dtype),
    y = cat(x1 c - x2 s, x1 s + x2 c), each tensor op in the dtype;
  * ``l2_normalize`` (functional.py:59-80, forward of ``_L2NormalizeFn`` at
    36-47): xf = y.float(), rinv = rsqrt(sum(xf * xf) + eps), out = (xf rinv) in
    the dtype;
  * backward: ``_L2NormalizeFn.backward`` (functional.py:50-57),
    g = ((gy - (gy . y) y) rinv) in the dtype, then autograd through the
    rotation: dx1 = g1 c + g2 s, dx2 = g2 c - g1 s, each product and the sum of
    the two contributions in the dtype.

Rounding model.  PyTorch computes a 16-bit elementwise op in fp32 and rounds
the result once to the dtype (round to nearest even); a product of two 16-bit
values is exact in fp32, a sum or difference is rounded to fp32 first.  The
functions below take ``dtype`` in {"bf16", "f16", "f32", "f64"}: "f64" drops
every rounding (exact arithmetic in float64, used by the mathematical pins),
"f32" rounds each op to fp32.  The row sums (sum of squares, the backward's
dot) are formed in float64 and rounded once to fp32: the reference's own
reduction order is its library's, so these two sums match it to a few fp32
ulps, not bit for bit, and the tests say so in their tolerances.  ``rinv`` is
the correctly rounded 1 / sqrt of the fp32 ``sum + eps``.

How each function is pinned (tests/test_oracle_prologue.py):
  * ``round_to``: torch's own fp32 -> bf16 / fp16 conversions on random
    values, ties, subnormals, infinities and NaN.
  * ``rope``: torch CPU evaluating the reference's expression in bf16 / fp16
    tensors (an independent implementation of the rounding model); the exact
    (f64) rotation against closed forms (a basis vector rotated by a known
    angle) and norm preservation; angle 0 is the identity.
  * ``prologue_forward``: unit norms; scale invariance of the exact map;
    rows of zeros give zeros with rinv = eps^-1/2.
  * ``eager_torch``: ``prologue_forward`` (rows within one bf16 ulp, the
    norm's summation order being torch's).
  * ``prologue_backward``: central finite differences of the exact forward
    (float64); the gradient is orthogonal to the normalised row in the
    rotated frame; the reference's own tolerance test
    (tests/test_plan041_15gb_batch24576_dyadic_scaling.py:24-44, bf16
    against fp32 within 2e-2 / 3e-2).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "round_to",
    "padded_table",
    "rope",
    "prologue_forward",
    "prologue_backward",
    "eager_torch",
]


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` (nearest even), returned as float32
    (float64 unchanged for "f64")."""
    if dtype == "f64":
        return np.asarray(x, dtype=np.float64)
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        bias = 0x7FFF + ((u >> 16) & 1)
        r = ((u + bias) & 0xFFFF0000).astype(np.uint32)
        nan = np.isnan(x)
        r = np.where(nan, (x.view(np.uint32) | 0x00400000) & 0xFFFF0000, r).astype(np.uint32)
        return r.view(np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def _op(a: np.ndarray, dtype: str) -> np.ndarray:
    """Result of one tensor op in ``dtype``: float32 -> dtype rounding, or
    float64 untouched."""
    if dtype == "f64":
        return a
    return round_to(np.asarray(a, dtype=np.float32), dtype)


def padded_table(cos: np.ndarray, sin: np.ndarray, half: int):
    """(T, n) tables -> (T, half) with the reference's cut / padding
    (attention.py:574-582)."""
    cos = np.asarray(cos)
    sin = np.asarray(sin)
    n = cos.shape[-1]
    if n >= half:
        return cos[..., :half], sin[..., :half]
    pad = [(0, 0)] * (cos.ndim - 1) + [(0, half - n)]
    return np.pad(cos, pad, constant_values=1.0), np.pad(sin, pad, constant_values=0.0)


def _ft(dtype: str):
    return np.float64 if dtype == "f64" else np.float32


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """apply_unitary_rope (functional.py:104-121) on (..., T, D) with (T, half)
    tables, every tensor op rounded to ``dtype``."""
    ft = _ft(dtype)
    x = np.asarray(x, dtype=ft)
    half = x.shape[-1] // 2
    c, s = padded_table(cos, sin, half)
    c = _op(np.asarray(c, dtype=ft), dtype)
    s = _op(np.asarray(s, dtype=ft), dtype)
    x1, x2 = x[..., :half], x[..., half:]
    y1 = _op(_op(x1 * c, dtype) - _op(x2 * s, dtype), dtype)
    y2 = _op(_op(x1 * s, dtype) + _op(x2 * c, dtype), dtype)
    return np.concatenate([y1, y2], axis=-1)


def _rinv(ss64: np.ndarray, eps: float, dtype: str) -> np.ndarray:
    if dtype == "f64":
        return 1.0 / np.sqrt(ss64 + eps)
    se = (ss64.astype(np.float32) + np.float32(eps)).astype(np.float32)
    return (1.0 / np.sqrt(se.astype(np.float64))).astype(np.float32)


def prologue_forward(x, cos, sin, eps: float, dtype: str):
    """(out, rinv) of l2_normalize(apply_unitary_rope(x)) for (..., T, D)
    rows; ``cos`` None skips the rotation.  ``rinv`` has shape (..., T)."""
    ft = _ft(dtype)
    x = np.asarray(x, dtype=ft)
    y = rope(x, cos, sin, dtype) if cos is not None else x
    ss = np.sum(np.asarray(y, dtype=np.float64) ** 2, axis=-1)
    rinv = _rinv(ss, eps, dtype)
    out = _op(y * rinv[..., None].astype(ft), dtype)
    return out, rinv


def prologue_backward(gy, out, rinv, cos, sin, dtype: str):
    """Gradient with respect to the prologue's input, given the gradient
    ``gy`` of its output ``out`` and the forward's ``rinv``."""
    ft = _ft(dtype)
    gy = np.asarray(gy, dtype=ft)
    out = np.asarray(out, dtype=ft)
    dot = np.sum(np.asarray(gy, dtype=np.float64) * np.asarray(out, dtype=np.float64), axis=-1)
    dot = dot.astype(ft)[..., None]
    r = np.asarray(rinv, dtype=ft)[..., None]
    if dtype == "f64":
        g = (gy - dot * out) * r
    else:
        g = _op(((gy - (dot * out).astype(np.float32)).astype(np.float32) * r).astype(np.float32),
                dtype)
    if cos is None:
        return g
    half = g.shape[-1] // 2
    c, s = padded_table(cos, sin, half)
    c = _op(np.asarray(c, dtype=ft), dtype)
    s = _op(np.asarray(s, dtype=ft), dtype)
    g1, g2 = g[..., :half], g[..., half:]
    d1 = _op(_op(g1 * c, dtype) + _op(g2 * s, dtype), dtype)
    d2 = _op(_op(g2 * c, dtype) - _op(g1 * s, dtype), dtype)
    return np.concatenate([d1, d2], axis=-1)


def eager_torch(x, cos, sin, eps: float):
    """The reference's eager formulation in torch, op for op, in ``x.dtype``
    (attention.py:574-589 with functional.py:104-121 and the fp32 norm of
    functional.py:78-80).  What ``bench.py`` times as the prologue's CPU
    baseline; pinned against ``prologue_forward`` (tests/test_oracle_prologue.py)."""
    import torch

    half = x.shape[-1] // 2
    if cos is not None:
        if cos.size(-1) >= half:
            c, s = cos[..., :half], sin[..., :half]
        else:
            c = torch.nn.functional.pad(cos, (0, half - cos.size(-1)), value=1.0)
            s = torch.nn.functional.pad(sin, (0, half - sin.size(-1)), value=0.0)
        c, s = c.to(x.dtype), s.to(x.dtype)
        x1, x2 = x[..., :half], x[..., half:]
        x = torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)
    xf = x.float()
    return (xf * torch.rsqrt(torch.sum(xf * xf, dim=-1, keepdim=True) + eps)).to(x.dtype)
