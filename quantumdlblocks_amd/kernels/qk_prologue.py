"""Fused Q/K prologue of the Born attention layer: unitary RoPE followed by L2
normalisation of Q and K, one HIP pass per tensor, forward and backward.

Reference: ``SubspaceProjectorBornAttention.forward``
(src/qdlblocks/layers/attention.py:573-589) applies, when rotary tables are
given,

    Q = l2_normalize(apply_unitary_rope(Q, c_use, s_use), eps)
    K = l2_normalize(apply_unitary_rope(K, c_use, s_use), eps)

with ``c_use``/``s_use`` the tables cut to, or padded up to (cos 1, sin 0),
``D // 2`` columns (attention.py:574-582), ``apply_unitary_rope`` from
functional.py:104-121 and ``l2_normalize`` with its memory-efficient autograd
function from functional.py:36-80.  The optional wave filter and partial key
offset (attention.py:560-571, 585-586) are not part of the fused op; a caller
that enables them applies them before calling it.

``fused_qk_rope_l2_normalize`` returns the normalised Q and K as contiguous
``(B, H, T, D)`` tensors.  The inputs may be strided views with unit stride on
D (for example the ``(B, T, H, D)`` projection output viewed as
``(B, H, T, D)``): the kernel reads them in place, so the ``.contiguous()``
copies before the prologue are not needed.  The backward writes the input
gradients with the inputs' own strides when those describe a dense layout
(a permuted contiguous tensor), else contiguous.
"""

from __future__ import annotations

import torch

from .. import _native
from ..functional import apply_unitary_rope, l2_normalize
from .flash_born import _DTYPE_CODE, _stream_ptr

__all__ = [
    "apply_unitary_rope",
    "flash_born_attention_qk_prologue",
    "fused_qk_rope_l2_normalize",
    "qk_prologue_backward",
    "qk_prologue_forward",
]


def _use_tables(cos: torch.Tensor, sin: torch.Tensor, half: int):
    """The reference's cut / padding of the tables to ``half`` columns
    (attention.py:574-582)."""
    if cos.size(-1) >= half:
        return cos[..., :half], sin[..., :half]
    pad = half - cos.size(-1)
    return (torch.nn.functional.pad(cos, (0, pad), value=1.0),
            torch.nn.functional.pad(sin, (0, pad), value=0.0))


def _eager(x, cos, sin, eps):
    if cos is not None:
        c, s = _use_tables(cos, sin, x.shape[-1] // 2)
        x = apply_unitary_rope(x, c, s)
    return l2_normalize(x, dim=-1, eps=eps)


def _table_2d(t: torch.Tensor, T: int, device) -> torch.Tensor:
    """(T, n) fp32 view of a table broadcastable to (..., T, n)."""
    t = t.detach()
    while t.dim() > 2:
        if t.shape[0] != 1:
            raise ValueError(
                f"rotary tables must broadcast over batch and heads, got shape {tuple(t.shape)}"
            )
        t = t[0]
    if t.dim() == 1:
        t = t.unsqueeze(0)
    if t.shape[0] != T:
        raise ValueError(f"rotary tables must have T={T} rows, got {t.shape[0]}")
    t = t.to(device=device, dtype=torch.float32)
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def _rows_ok(x: torch.Tensor) -> torch.Tensor:
    """Unit stride along D (any strides for b, h, t)."""
    return x if x.stride(-1) == 1 else x.contiguous()


def _strides(x: torch.Tensor) -> torch.Tensor:
    return torch.tensor(list(x.stride()[:3]), dtype=torch.int64)


def _launch_fwd(x: torch.Tensor, which: int, cos2, sin2, eps: float):
    """Run the forward for one tensor (``which`` 0 = q slot, 1 = k slot)."""
    lib = _native.load()
    B, H, T, D = x.shape
    out = torch.empty((B, H, T, D), dtype=x.dtype, device=x.device)
    rinv = torch.empty((B, H, T), dtype=torch.float32, device=x.device)
    st = _strides(x)
    args = [None, None, None, None]
    args[2 * which] = x.data_ptr()
    args[2 * which + 1] = st.data_ptr()
    outs = [None, None, None, None]
    outs[which] = out.data_ptr()
    outs[2 + which] = rinv.data_ptr()
    with torch.cuda.device(x.device):
        rc = lib.qdl_flash_born_qk_prologue_fwd(
            _DTYPE_CODE[x.dtype], B, H, T, D, *args,
            cos2.data_ptr() if cos2 is not None else None,
            sin2.data_ptr() if sin2 is not None else None,
            cos2.shape[1] if cos2 is not None else 0,
            cos2.stride(0) if cos2 is not None else 0,
            float(eps), *outs, _stream_ptr(x.device),
        )
    _native.check(rc, "qdl_flash_born_qk_prologue_fwd")
    return out, rinv


def _dense_layout(shape, strides) -> bool:
    """True when (shape, strides) describes a non-overlapping layout without
    gaps (a permutation of a contiguous tensor): one a gradient may take."""
    dims = sorted((st, n) for n, st in zip(shape, strides) if n != 1)
    expect = 1
    for st, n in dims:
        if st != expect:
            return False
        expect *= n
    return True


def _launch_bwd(g, out, rinv, cos2, sin2, layout, which: int):
    """Input gradient of one tensor, written with the input's (shape, strides)
    when those are dense (a permuted contiguous tensor, e.g. the projection
    layout) with unit stride along D, else contiguous.  The kernel writes each
    D row contiguously and takes only the (b, h, t) strides, so an input whose
    D stride is not 1 (e.g. a transposed (B, H, D, T) tensor) gets a
    contiguous gradient."""
    lib = _native.load()
    B, H, T, D = out.shape
    g = g.to(out.dtype).contiguous()
    shape, strides = layout
    if _dense_layout(shape, strides) and (shape[-1] == 1 or strides[-1] == 1):
        dx = torch.empty_strided(layout[0], layout[1], dtype=out.dtype, device=out.device)
    else:
        dx = torch.empty(layout[0], dtype=out.dtype, device=out.device)
    st = _strides(dx)
    gs = [None, None]
    ys = [None, None]
    rs = [None, None]
    ds = [None, None, None, None]
    gs[which] = g.data_ptr()
    ys[which] = out.data_ptr()
    rs[which] = rinv.data_ptr()
    ds[2 * which] = dx.data_ptr()
    ds[2 * which + 1] = st.data_ptr()
    with torch.cuda.device(out.device):
        rc = lib.qdl_flash_born_qk_prologue_bwd(
            _DTYPE_CODE[out.dtype], B, H, T, D, *gs, *ys, *rs,
            cos2.data_ptr() if cos2 is not None else None,
            sin2.data_ptr() if sin2 is not None else None,
            cos2.shape[1] if cos2 is not None else 0,
            cos2.stride(0) if cos2 is not None else 0,
            *ds, _stream_ptr(out.device),
        )
    _native.check(rc, "qdl_flash_born_qk_prologue_bwd")
    return dx


def _prep_tables(cos, sin, half: int, T: int, device):
    """fp32 (T, n) tables with n = min(width, half) and one row stride, or
    (None, None)."""
    if cos is None:
        return None, None
    # Columns past the table's width rotate by angle 0 inside the kernel (the
    # reference's padding, attention.py:577-582).
    n = min(cos.size(-1), half)
    cos2 = _table_2d(cos[..., :n], T, device)
    sin2 = _table_2d(sin[..., :n], T, device)
    if sin2.stride(0) != cos2.stride(0):
        cos2, sin2 = cos2.contiguous(), sin2.contiguous()
    return cos2, sin2


def qk_prologue_forward(q, k, cos=None, sin=None, eps: float = 1e-12):
    """No-autograd forward: ``(q_out, k_out, q_rinv, k_rinv)``, the normalised
    rows (contiguous, input dtypes) and 1 / sqrt(sum y^2 + eps) per row (fp32)."""
    B, H, T, D = q.shape
    cos2, sin2 = _prep_tables(cos, sin, D // 2, T, q.device)
    q_in, k_in = _rows_ok(q.detach()), _rows_ok(k.detach())
    if q_in.dtype != k_in.dtype or q_in.device != k_in.device:
        q_out, q_r = _launch_fwd(q_in, 0, cos2, sin2, eps)
        k_out, k_r = _launch_fwd(k_in, 1, cos2, sin2, eps)
        return q_out, k_out, q_r, k_r
    lib = _native.load()
    q_out = torch.empty((B, H, T, D), dtype=q.dtype, device=q.device)
    k_out = torch.empty_like(q_out)
    q_r = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    k_r = torch.empty_like(q_r)
    qs, ks = _strides(q_in), _strides(k_in)
    with torch.cuda.device(q.device):
        rc = lib.qdl_flash_born_qk_prologue_fwd(
            _DTYPE_CODE[q.dtype], B, H, T, D,
            q_in.data_ptr(), qs.data_ptr(), k_in.data_ptr(), ks.data_ptr(),
            cos2.data_ptr() if cos2 is not None else None,
            sin2.data_ptr() if sin2 is not None else None,
            cos2.shape[1] if cos2 is not None else 0,
            cos2.stride(0) if cos2 is not None else 0,
            float(eps), q_out.data_ptr(), k_out.data_ptr(), q_r.data_ptr(), k_r.data_ptr(),
            _stream_ptr(q.device),
        )
    _native.check(rc, "qdl_flash_born_qk_prologue_fwd")
    return q_out, k_out, q_r, k_r


def qk_prologue_backward(gq, gk, q_out, k_out, q_rinv, k_rinv, cos=None, sin=None,
                         q_layout=None, k_layout=None):
    """No-autograd backward: input gradients (None where the output gradient
    is None), written with ``(shape, strides)`` layouts (default contiguous)."""
    B, H, T, D = q_out.shape
    cos2, sin2 = _prep_tables(cos, sin, D // 2, T, q_out.device)
    dq = dk = None
    if gq is not None:
        lay = q_layout or (tuple(q_out.shape), tuple(q_out.stride()))
        dq = _launch_bwd(gq, q_out, q_rinv, cos2, sin2, lay, 0)
    if gk is not None:
        lay = k_layout or (tuple(k_out.shape), tuple(k_out.stride()))
        dk = _launch_bwd(gk, k_out, k_rinv, cos2, sin2, lay, 1)
    return dq, dk


class _QKPrologueFn(torch.autograd.Function):
    """Forward: normalised Q, K (contiguous, input dtypes) and 1/norm per row
    (saved).  Backward: input gradients in the inputs' dtypes and strides;
    None for the tables and eps (the reference's tables are buffers)."""

    @staticmethod
    def forward(ctx, q, k, cos, sin, eps):
        q_out, k_out, q_r, k_r = qk_prologue_forward(q, k, cos, sin, eps)
        ctx.save_for_backward(q_out, k_out, q_r, k_r)
        ctx.tables = (cos.detach(), sin.detach()) if cos is not None else (None, None)
        ctx.q_layout = (tuple(q.shape), tuple(q.stride()))
        ctx.k_layout = (tuple(k.shape), tuple(k.stride()))
        return q_out, k_out

    @staticmethod
    def backward(ctx, gq, gk):
        q_out, k_out, q_r, k_r = ctx.saved_tensors
        cos, sin = ctx.tables
        dq, dk = qk_prologue_backward(
            gq if ctx.needs_input_grad[0] else None,
            gk if ctx.needs_input_grad[1] else None,
            q_out, k_out, q_r, k_r, cos, sin, ctx.q_layout, ctx.k_layout,
        )
        return dq, dk, None, None, None


def fused_qk_rope_l2_normalize(
    q: torch.Tensor,
    k: torch.Tensor,
    cos: torch.Tensor | None = None,
    sin: torch.Tensor | None = None,
    eps: float = 1e-12,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(l2_normalize(rope(q)), l2_normalize(rope(k)))`` as the Born layer
    computes them before attention (attention.py:573-589).

    q, k: ``(B, H, T, D)`` of one shape, D even and at most 256, unit stride
    along D.  cos, sin: rotary tables broadcastable to ``(1, 1, T, n)`` (the
    reference's ``get_cos_sin`` output), or None for L2 normalisation alone.
    GPU tensors run the gfx950 HIP kernels (an error if the library is
    missing); CPU tensors take the reference's eager formulation.
    """
    if q.dim() != 4 or k.shape != q.shape:
        raise ValueError(
            f"q and k must share one (B, H, T, D) shape, got {tuple(q.shape)}, {tuple(k.shape)}"
        )
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must be given together")
    D = q.shape[-1]
    if not q.is_cuda:
        return _eager(q, cos, sin, eps), _eager(k, cos, sin, eps)
    if D % 2 or D < 2 or D > 256:
        raise NotImplementedError(f"head dim {D}: the fused prologue needs an even D in [2, 256]")
    for t in (q, k):
        if t.dtype not in _DTYPE_CODE:
            raise TypeError(f"fused_qk_rope_l2_normalize: unsupported dtype {t.dtype}")
    return _QKPrologueFn.apply(q, k, cos, sin, float(eps))


# ---------------------------------------------------------------------------
# Prologue folded into the attention kernel's loads
# ---------------------------------------------------------------------------

class _BornQKPrologueFn(torch.autograd.Function):
    """Forward: Born attention of (q', k', v) with q' = l2_normalize(rope(q)),
    k' likewise, in one call of ``qdl_flash_born_fwd_qk_prologue`` (for bf16,
    D = 64, no documents or window: the prologue kernel on K alone, then one
    attention kernel that normalises each query block as it loads it).  Saves
    q', k' and 1/norm when a gradient is needed (otherwise 1/norm and q' are
    not written).  Backward: the attention backward on (q', k', v), then the
    prologue backward into q and k (their dtypes and strides)."""

    @staticmethod
    def forward(ctx, q, k, v, scale, cos, sin, is_causal, eps, window_size, doc_ids, norm_eps):
        from .flash_born import _aligned, _autocast_dtype, _check_inputs

        lib = _native.load()
        target = _autocast_dtype(q) or v.dtype
        if target not in _DTYPE_CODE:
            raise TypeError(f"flash_born_attention_qk_prologue: unsupported dtype {target}")
        scale_flat = scale.detach().contiguous().view(-1).to(dtype=torch.float32, device=q.device)
        _check_inputs(q, k, v, scale_flat, doc_ids)
        B, H, T, D = q.shape
        q_in = _rows_ok(q.detach().to(target))
        k_in = _rows_ok(k.detach().to(target))
        v_c = _aligned(v.detach().to(target))
        cos2, sin2 = _prep_tables(cos, sin, D // 2, T, q.device)
        doc_c = None if doc_ids is None else _aligned(doc_ids.to(device=q.device, dtype=torch.int32))
        out = torch.empty((B, H, T, D), dtype=target, device=q.device)
        z = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
        q_out = torch.empty_like(out)
        k_out = torch.empty_like(out)
        grad = any(ctx.needs_input_grad[:4])
        q_r = torch.empty_like(z) if grad else None
        k_r = torch.empty_like(z) if grad else None
        qs, ks = _strides(q_in), _strides(k_in)
        window = max(int(window_size), 0)
        with torch.cuda.device(q.device):
            rc = lib.qdl_flash_born_fwd_qk_prologue(
                _DTYPE_CODE[target], B, H, T, D,
                q_in.data_ptr(), qs.data_ptr(), k_in.data_ptr(), ks.data_ptr(), v_c.data_ptr(),
                cos2.data_ptr() if cos2 is not None else None,
                sin2.data_ptr() if sin2 is not None else None,
                cos2.shape[1] if cos2 is not None else 0,
                cos2.stride(0) if cos2 is not None else 0,
                float(norm_eps), scale_flat.data_ptr(), scale_flat.numel(),
                doc_c.data_ptr() if doc_c is not None else None,
                1 if is_causal else 0, window, float(eps),
                out.data_ptr(), z.data_ptr(), q_out.data_ptr(), k_out.data_ptr(),
                q_r.data_ptr() if grad else None, k_r.data_ptr() if grad else None, _stream_ptr(q.device),
            )
        _native.check(rc, "qdl_flash_born_fwd_qk_prologue")
        if not grad:
            return out
        ctx.save_for_backward(q_out, k_out, v_c, out, z, scale_flat, q_r, k_r,
                              doc_c if doc_c is not None else torch.empty(0, dtype=torch.int32, device=q.device))
        ctx.tables = (cos.detach(), sin.detach()) if cos is not None else (None, None)
        ctx.q_layout = (tuple(q.shape), tuple(q.stride()))
        ctx.k_layout = (tuple(k.shape), tuple(k.stride()))
        ctx.is_causal, ctx.eps, ctx.window_size = bool(is_causal), float(eps), window
        ctx.has_doc_ids = doc_ids is not None
        ctx.scale_shape, ctx.scale_dtype = scale.shape, scale.dtype
        ctx.dtypes = (q.dtype, k.dtype, v.dtype)
        return out

    @staticmethod
    def backward(ctx, do):
        lib = _native.load()
        q_out, k_out, v_c, out, z, scale_flat, q_r, k_r, doc_c = ctx.saved_tensors
        B, H, T, D = q_out.shape
        from .flash_born import _aligned

        do_c = _aligned(do.to(v_c.dtype))
        dqn = torch.empty_like(q_out)
        dkn = torch.empty_like(k_out)
        dv = torch.empty_like(v_c)
        dscale = torch.empty(scale_flat.numel(), dtype=torch.float32, device=q_out.device)
        code = _DTYPE_CODE[v_c.dtype]
        ws_bytes = int(lib.qdl_flash_born_bwd_workspace_size(code, B, H, T, D, scale_flat.numel()))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q_out.device)
        with torch.cuda.device(q_out.device):
            rc = lib.qdl_flash_born_bwd(
                code, B, H, T, D,
                q_out.data_ptr(), k_out.data_ptr(), v_c.data_ptr(), out.data_ptr(), do_c.data_ptr(),
                z.data_ptr(), scale_flat.data_ptr(), scale_flat.numel(),
                doc_c.data_ptr() if ctx.has_doc_ids else None,
                1 if ctx.is_causal else 0, ctx.window_size, ctx.eps,
                dqn.data_ptr(), dkn.data_ptr(), dv.data_ptr(), dscale.data_ptr(),
                ws.data_ptr(), ws.numel(), _stream_ptr(q_out.device),
            )
        _native.check(rc, "qdl_flash_born_bwd")
        cos, sin = ctx.tables
        dq, dk = qk_prologue_backward(dqn, dkn, q_out, k_out, q_r, k_r, cos, sin, ctx.q_layout, ctx.k_layout)
        qd, kd, vd = ctx.dtypes
        return (dq.to(qd), dk.to(kd), dv.to(vd), dscale.view(ctx.scale_shape).to(ctx.scale_dtype),
                None, None, None, None, None, None, None)


def flash_born_attention_qk_prologue(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float | torch.Tensor,
    cos: torch.Tensor | None = None,
    sin: torch.Tensor | None = None,
    is_causal: bool = True,
    eps: float = 1e-12,
    window_size: int = 0,
    doc_ids: torch.Tensor | None = None,
    norm_eps: float = 1e-12,
) -> torch.Tensor:
    """The Born layer's attention data flow with the Q/K prologue folded into
    the attention kernel (attention.py:573-589 then 704-713):

        flash_born_attention(l2_normalize(rope(q)), l2_normalize(rope(k)), v, scale, ...)

    q, k: ``(B, H, T, D)`` raw projections with unit stride along D (e.g. the
    ``(B, T, H, D)`` projection output viewed as ``(B, H, T, D)``); v: any
    ``(B, H, T, D)``; cos, sin as for ``fused_qk_rope_l2_normalize`` (or None:
    normalisation only); the other arguments as for ``flash_born_attention``.
    On the GPU, bf16 with D = 64 and no documents or window runs as one
    kernel; other cases run the prologue kernel and then the attention
    kernels.  CPU tensors take the reference's eager formulation of both.
    """
    from .flash_born import MAX_HEAD_DIM, flash_born_attention

    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must share one (B, H, T, D) shape")
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must be given together")
    if not isinstance(scale, torch.Tensor):
        scale = torch.tensor(float(scale), dtype=torch.float32, device=q.device)
    D = q.shape[-1]
    if not q.is_cuda or D % 8 or D > MAX_HEAD_DIM:
        qn, kn = fused_qk_rope_l2_normalize(q, k, cos, sin, norm_eps)
        return flash_born_attention(qn, kn, v, scale, is_causal, eps, window_size, doc_ids)
    return _BornQKPrologueFn.apply(q, k, v, scale, cos, sin, bool(is_causal), float(eps), int(window_size),
                                   doc_ids, float(norm_eps))
