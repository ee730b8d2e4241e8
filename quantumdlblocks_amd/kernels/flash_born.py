"""Flash-Born attention on MI355X: host side of the gfx950 HIP kernels.

Drop-in for the reference module ``qdlblocks.kernels.flash_born`` (documented
there as ``qdlblocks.kernels.flash_born_triton``; Vengo/QuantumDLBlocks
src/qdlblocks/kernels/flash_born.py:1-690).  Same public names, call
signature, tensor layouts and autograd contract:

    flash_born_attention(q, k, v, scale, is_causal=True, eps=1e-12,
                         window_size=0, doc_ids=None) -> Tensor

computes, per (b, h) and with ``(B, H, T, D)`` inputs,

    a_ij = max(0, scale_h * q_i . k_j) * M_ij,   p_ij = a_ij ** 2
    O_i  = sum_j p_ij v_j / (sum_j p_ij + eps)
    M_ij = [causal => j <= i] & [window_size > 0 => i - j < window_size]
           & [doc_ids[b, i] == doc_ids[b, j]]

GPU tensors with head dim <= 256 always run the HIP kernels of
``libqdl_flash_born.so`` (forward, and a backward producing dq, dk, dv and
dscale).  If the library is missing the call raises: a broken install is
reported, not hidden behind a slow path.  CPU tensors, and GPU tensors with a
head dim above 256 (which the reference's kernel does not take either), run
the reference's eager formulation (flash_born.py:670-690) on their own device.
"""

from __future__ import annotations

from typing import Any

import torch

from .. import _native

# The reference exposes ``HAS_TRITON`` (flash_born.py:20-26) and callers use it
# as "the fast GPU kernel is available" (e.g. its tests' skip conditions).
# Here it means the HIP library loaded.
HAS_HIP_KERNELS: bool = _native.available()
HAS_TRITON: bool = HAS_HIP_KERNELS

IS_HIP: bool = getattr(torch.version, "hip", None) is not None

MAX_HEAD_DIM = 256

__all__ = [
    "HAS_TRITON",
    "HAS_HIP_KERNELS",
    "IS_HIP",
    "flash_born_attention",
    "flash_purified_born_attention",
    "get_flash_born_launch_meta",
    "get_rdna4_autotune_configs",
    "get_mi355x_launch_meta",
]


def _next_pow2(n: int) -> int:
    return 1 << (max(1, int(n)) - 1).bit_length()


def get_flash_born_launch_meta(
    seq_len: int,
    is_hip: bool | None = None,
    head_dim: int = 64,
) -> dict[str, int]:
    """Launch metadata of the reference's Triton kernels (flash_born.py:31-65).

    Kept for API compatibility: callers and tests read these values.  The HIP
    kernels here use their own tiling (``get_mi355x_launch_meta``).
    Tile edge: 16 for a padded head dim >= 256; 32 (16 for T < 32) for >= 128;
    otherwise 64 (32 for T < 64, 16 for T < 32).
    """
    hip = IS_HIP if is_hip is None else bool(is_hip)
    eff = _next_pow2(head_dim)
    if eff >= 256:
        edge = 16
    elif eff >= 128:
        edge = 32 if seq_len >= 32 else 16
    else:
        edge = next((e for e in (64, 32) if seq_len >= e), 16)
    meta: dict[str, int] = {"BLOCK_M": edge, "BLOCK_N": edge, "num_warps": 4}
    if hip:
        meta.update(num_stages=1, waves_per_eu=2, matrix_instr_nonkdim=16)
    else:
        meta["num_stages"] = 2 if eff < 128 else 1
    return meta


def get_rdna4_autotune_configs() -> list[dict[str, int]]:
    """The reference's four RDNA4 Triton autotune candidates (flash_born.py:68-75)."""
    rows = ((64, 64, 4, 2), (64, 32, 4, 2), (128, 64, 8, 2), (32, 32, 2, 4))
    return [
        {
            "BLOCK_M": bm,
            "BLOCK_N": bn,
            "num_warps": nw,
            "num_stages": 1,
            "waves_per_eu": wpe,
            "matrix_instr_nonkdim": 16,
        }
        for bm, bn, nw, wpe in rows
    ]


def get_mi355x_launch_meta(head_dim: int = 64, dtype: torch.dtype = torch.bfloat16) -> dict[str, int]:
    """Tiling the gfx950 forward kernel uses for this head dim and dtype."""
    dp = (max(8, head_dim) + 31) // 32 * 32
    if dtype == torch.float32:
        return {"BLOCK_M": 128, "BLOCK_N": 32, "waves": 4, "queries_per_wave": 32,
                "padded_head_dim": dp, "mfma": "32x32x2f32"}
    nqb = 2 if dp <= 64 else 1
    return {
        "BLOCK_M": 4 * 32 * nqb,
        "BLOCK_N": 64 if dp <= 128 else 32,
        "waves": 4,
        "queries_per_wave": 32 * nqb,
        "padded_head_dim": dp,
        "mfma": "32x32x16" + ("bf16" if dtype == torch.bfloat16 else "f16"),
    }


_DTYPE_CODE = {
    torch.float32: _native.DTYPE_F32,
    torch.float16: _native.DTYPE_F16,
    torch.bfloat16: _native.DTYPE_BF16,
}


def _autocast_dtype(q: torch.Tensor) -> torch.dtype | None:
    """Autocast dtype when CUDA autocast is active (flash_born.py:446)."""
    if not q.is_cuda:
        return None
    try:
        enabled = torch.is_autocast_enabled("cuda")
    except TypeError:  # older torch
        enabled = torch.is_autocast_enabled()
    if not enabled:
        return None
    try:
        return torch.get_autocast_dtype("cuda")
    except AttributeError:  # older torch
        return torch.get_autocast_gpu_dtype()


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous tensor whose base address is 16-byte aligned."""
    t = t.contiguous()
    if t.numel() and t.data_ptr() % 16:
        t = t.clone()
    return t


def _pad_head(t: torch.Tensor, dp: int) -> torch.Tensor:
    d = t.shape[-1]
    if d == dp:
        return t
    return torch.nn.functional.pad(t, (0, dp - d))


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_inputs(q, k, v, scale_flat, doc_ids):
    if q.dim() != 4:
        raise ValueError(f"q must be (B, H, T, D), got shape {tuple(q.shape)}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(
            f"q, k, v must share one (B, H, T, D) shape, got {tuple(q.shape)}, "
            f"{tuple(k.shape)}, {tuple(v.shape)}"
        )
    B, H, T, D = q.shape
    if D > MAX_HEAD_DIM:
        raise NotImplementedError(f"head_dim {D} > {MAX_HEAD_DIM} is not supported by the HIP kernels")
    n = scale_flat.numel()
    if n not in (1, H):
        raise ValueError(f"scale must hold 1 value or H={H} per-head values, got {n}")
    if doc_ids is not None and tuple(doc_ids.shape) != (B, T):
        raise ValueError(f"doc_ids must be (B, T)=({B}, {T}), got {tuple(doc_ids.shape)}")


class _FlashBornAttentionFn(torch.autograd.Function):
    """Autograd contract of the reference (flash_born.py:433-618).

    forward: computes in the autocast dtype (CUDA autocast active) else
    ``v.dtype``; saves the cast inputs, ``out``, ``Z`` (fp32, eps included),
    the flattened fp32 scale and int32 doc ids.  backward: returns dq, dk, dv
    in the original input dtypes, dscale reshaped to the scale's shape and
    dtype, and None for is_causal, eps, window_size, doc_ids.
    """

    @staticmethod
    def forward(
        ctx,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        scale: torch.Tensor,
        is_causal: bool,
        eps: float,
        window_size: int = 0,
        doc_ids: torch.Tensor | None = None,
    ) -> torch.Tensor:
        lib = _native.load()
        target = _autocast_dtype(q) or v.dtype
        if target not in _DTYPE_CODE:
            raise TypeError(f"flash_born_attention: unsupported dtype {target}")
        scale_flat = scale.detach().contiguous().view(-1).to(dtype=torch.float32, device=q.device)
        _check_inputs(q, k, v, scale_flat, doc_ids)
        B, H, T, D = q.shape
        dp = (D + 7) // 8 * 8
        q_c = _aligned(_pad_head(q.to(target), dp))
        k_c = _aligned(_pad_head(k.to(target), dp))
        v_c = _aligned(_pad_head(v.to(target), dp))
        if doc_ids is not None:
            doc_c = _aligned(doc_ids.to(device=q.device, dtype=torch.int32))
        else:
            doc_c = torch.empty(0, device=q.device, dtype=torch.int32)
        out = torch.empty_like(q_c)
        z = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
        window = int(window_size)
        if window < 0:
            window = 0
        with torch.cuda.device(q.device):
            rc = lib.qdl_flash_born_fwd(
                _DTYPE_CODE[target], B, H, T, dp,
                q_c.data_ptr(), k_c.data_ptr(), v_c.data_ptr(), out.data_ptr(), z.data_ptr(),
                scale_flat.data_ptr(), scale_flat.numel(),
                doc_c.data_ptr() if doc_ids is not None else None,
                1 if is_causal else 0, window, float(eps), _stream_ptr(q.device),
            )
        _native.check(rc, "qdl_flash_born_fwd")

        ctx.save_for_backward(q_c, k_c, v_c, out, z, scale_flat, doc_c)
        ctx.is_causal = bool(is_causal)
        ctx.window_size = window
        ctx.eps = float(eps)
        ctx.has_doc_ids = doc_ids is not None
        ctx.head_dim = D
        ctx.scale_shape = scale.shape
        ctx.scale_dtype = scale.dtype
        ctx.orig_q_dtype = q.dtype
        ctx.orig_k_dtype = k.dtype
        ctx.orig_v_dtype = v.dtype
        return out if dp == D else out[..., :D].contiguous()

    @staticmethod
    def backward(ctx, do: torch.Tensor):
        lib = _native.load()
        q_c, k_c, v_c, out, z, scale_flat, doc_c = ctx.saved_tensors
        B, H, T, dp = q_c.shape
        D = ctx.head_dim
        do_c = _aligned(_pad_head(do.to(v_c.dtype), dp))
        dq = torch.empty_like(q_c)
        dk = torch.empty_like(k_c)
        dv = torch.empty_like(v_c)
        dscale = torch.empty(scale_flat.numel(), dtype=torch.float32, device=q_c.device)
        code = _DTYPE_CODE[v_c.dtype]
        ws_bytes = int(lib.qdl_flash_born_bwd_workspace_size(code, B, H, T, dp, scale_flat.numel()))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q_c.device)
        with torch.cuda.device(q_c.device):
            rc = lib.qdl_flash_born_bwd(
                code, B, H, T, dp,
                q_c.data_ptr(), k_c.data_ptr(), v_c.data_ptr(), out.data_ptr(), do_c.data_ptr(),
                z.data_ptr(), scale_flat.data_ptr(), scale_flat.numel(),
                doc_c.data_ptr() if ctx.has_doc_ids else None,
                1 if ctx.is_causal else 0, ctx.window_size, ctx.eps,
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dscale.data_ptr(),
                ws.data_ptr(), ws.numel(), _stream_ptr(q_c.device),
            )
        _native.check(rc, "qdl_flash_born_bwd")
        if dp != D:
            dq, dk, dv = dq[..., :D], dk[..., :D], dv[..., :D]
        dq_out = dq.to(ctx.orig_q_dtype)
        dk_out = dk.to(ctx.orig_k_dtype)
        dv_out = dv.to(ctx.orig_v_dtype)
        dscale_out = dscale.view(ctx.scale_shape).to(ctx.scale_dtype)
        return dq_out, dk_out, dv_out, dscale_out, None, None, None, None


@torch.compiler.disable
def _run_triton_flash_born(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale_t: torch.Tensor,
    is_causal: bool,
    eps: float,
    window_size: int = 0,
    doc_ids: torch.Tensor | None = None,
) -> torch.Tensor:
    """Direct entry to the GPU kernels (reference name, flash_born.py:621-632)."""
    return _FlashBornAttentionFn.apply(q, k, v, scale_t, is_causal, eps, int(window_size), doc_ids)


_run_hip_flash_born = _run_triton_flash_born


def _apply_window_and_doc_mask(
    prob: torch.Tensor,
    is_causal: bool,
    window_size: int,
    doc_ids: torch.Tensor | None,
) -> torch.Tensor:
    """Zero the invisible (i, j) entries of ``prob`` (B, H, T, T) (flash_born.py:635-652)."""
    T = prob.shape[-1]
    pos = torch.arange(T, device=prob.device)
    lag = pos.view(T, 1) - pos.view(1, T)  # i - j
    keep = lag >= 0 if is_causal else torch.ones((T, T), dtype=torch.bool, device=prob.device)
    if window_size > 0:
        keep = keep & (lag < int(window_size))
    keep = keep.view(1, 1, T, T)
    if doc_ids is not None:
        same = doc_ids.unsqueeze(-1) == doc_ids.unsqueeze(-2)  # (B, T, T)
        keep = keep & same.unsqueeze(1)
    return prob * keep.to(prob.dtype)


def _eager_born(q, k, v, scale_t, is_causal, eps, window_size, doc_ids):
    """CPU formulation of the reference (flash_born.py:681-690), in ``v.dtype``."""
    s_v = scale_t.to(v.dtype)
    if s_v.ndim == 1:
        s_v = s_v.view(1, -1, 1, 1)
    scores = torch.matmul(q.to(v.dtype), k.to(v.dtype).transpose(-1, -2)) * s_v
    prob = torch.relu(scores).square()
    if is_causal or window_size > 0 or doc_ids is not None:
        prob = _apply_window_and_doc_mask(prob, is_causal, window_size, doc_ids)
    weights = prob / (prob.sum(dim=-1, keepdim=True) + eps)
    return torch.matmul(weights.to(v.dtype), v)


def flash_born_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float | torch.Tensor,
    is_causal: bool = True,
    eps: float = 1e-12,
    window_size: int = 0,
    doc_ids: torch.Tensor | None = None,
) -> torch.Tensor:
    """Born attention with the reference's signature (flash_born.py:655-690).

    ``scale`` is a float or a tensor of shape (), (1,), (H,) or (1, H, 1, 1).
    ``window_size > 0`` keeps keys with ``i - j < window_size``; ``doc_ids``
    (B, T) keeps pairs within one document.  GPU tensors run the gfx950 HIP
    kernels for any head dim up to 256; CPU tensors and larger head dims use
    the eager formulation.
    """
    if not isinstance(scale, torch.Tensor):
        scale_t = torch.tensor(float(scale), dtype=torch.float32, device=q.device)
    else:
        scale_t = scale
    if q.is_cuda and q.shape[-1] <= MAX_HEAD_DIM:
        return _run_triton_flash_born(q, k, v, scale_t, is_causal, eps, window_size=window_size, doc_ids=doc_ids)
    # CPU tensors, and head dims the kernels do not take (D > 256), run the
    # reference's eager formulation on the tensors' own device, as the
    # reference does for every shape its kernel does not support
    # (flash_born.py:670-690).
    return _eager_born(q, k, v, scale_t, is_causal, eps, window_size, doc_ids)


# ---------------------------------------------------------------------------
# Purified-Born attention (flash_born.py:693-1341)
# ---------------------------------------------------------------------------

class _FlashPurifiedBornAttentionFn(torch.autograd.Function):
    """Autograd contract of the reference (flash_born.py:1064-1270).

    forward: computes in the autocast dtype (CUDA autocast active) else
    ``v.dtype``; the kernel writes an fp32 output, saved for the backward and
    returned cast to the compute dtype; Z is fp32 with eps.  backward: returns
    dq, dk, dv in the original input dtypes, dscale and dtau in their
    parameters' shapes and dtypes, and None for eps_base, is_causal, eps,
    window_size, doc_ids.
    """

    @staticmethod
    def forward(
        ctx,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        scale: torch.Tensor,
        tau: torch.Tensor,
        eps_base: float,
        is_causal: bool,
        eps: float,
        window_size: int = 0,
        doc_ids: torch.Tensor | None = None,
    ) -> torch.Tensor:
        lib = _native.load()
        target = _autocast_dtype(q) or v.dtype
        if target not in _DTYPE_CODE:
            raise TypeError(f"flash_purified_born_attention: unsupported dtype {target}")
        scale_flat = scale.detach().contiguous().view(-1).to(dtype=torch.float32, device=q.device)
        tau_flat = tau.detach().contiguous().view(-1).to(dtype=torch.float32, device=q.device)
        _check_inputs(q, k, v, scale_flat, doc_ids)
        B, H, T, D = q.shape
        if tau_flat.numel() not in (1, H):
            raise ValueError(f"tau must hold 1 value or H={H} per-head values, got {tau_flat.numel()}")
        dp = (D + 7) // 8 * 8
        q_c = _aligned(_pad_head(q.to(target), dp))
        k_c = _aligned(_pad_head(k.to(target), dp))
        v_c = _aligned(_pad_head(v.to(target), dp))
        if doc_ids is not None:
            doc_c = _aligned(doc_ids.to(device=q.device, dtype=torch.int32))
        else:
            doc_c = torch.empty(0, device=q.device, dtype=torch.int32)
        out_f32 = torch.empty((B, H, T, dp), dtype=torch.float32, device=q.device)
        z = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
        window = max(int(window_size), 0)
        with torch.cuda.device(q.device):
            rc = lib.qdl_flash_purified_born_fwd(
                _DTYPE_CODE[target], B, H, T, dp,
                q_c.data_ptr(), k_c.data_ptr(), v_c.data_ptr(), out_f32.data_ptr(), z.data_ptr(),
                scale_flat.data_ptr(), scale_flat.numel(), tau_flat.data_ptr(), tau_flat.numel(),
                float(eps_base), doc_c.data_ptr() if doc_ids is not None else None,
                1 if is_causal else 0, window, float(eps), _stream_ptr(q.device),
            )
        _native.check(rc, "qdl_flash_purified_born_fwd")
        ctx.save_for_backward(q_c, k_c, v_c, out_f32, z, scale_flat, tau_flat, doc_c)
        ctx.is_causal = bool(is_causal)
        ctx.window_size = window
        ctx.eps_base = float(eps_base)
        ctx.has_doc_ids = doc_ids is not None
        ctx.head_dim = D
        ctx.scale_shape, ctx.scale_dtype = scale.shape, scale.dtype
        ctx.tau_shape, ctx.tau_dtype = tau.shape, tau.dtype
        ctx.orig_q_dtype, ctx.orig_k_dtype, ctx.orig_v_dtype = q.dtype, k.dtype, v.dtype
        out = out_f32 if dp == D else out_f32[..., :D]
        return out.to(target)

    @staticmethod
    def backward(ctx, do: torch.Tensor):
        lib = _native.load()
        q_c, k_c, v_c, out_f32, z, scale_flat, tau_flat, doc_c = ctx.saved_tensors
        B, H, T, dp = q_c.shape
        D = ctx.head_dim
        do_c = _aligned(_pad_head(do.to(v_c.dtype), dp))
        dq = torch.empty_like(q_c)
        dk = torch.empty_like(k_c)
        dv = torch.empty_like(v_c)
        dscale = torch.empty(scale_flat.numel(), dtype=torch.float32, device=q_c.device)
        dtau = torch.empty(tau_flat.numel(), dtype=torch.float32, device=q_c.device)
        code = _DTYPE_CODE[v_c.dtype]
        ws_bytes = int(lib.qdl_flash_purified_born_bwd_workspace_size(code, B, H, T, dp))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q_c.device)
        with torch.cuda.device(q_c.device):
            rc = lib.qdl_flash_purified_born_bwd(
                code, B, H, T, dp,
                q_c.data_ptr(), k_c.data_ptr(), v_c.data_ptr(), out_f32.data_ptr(), do_c.data_ptr(),
                z.data_ptr(), scale_flat.data_ptr(), scale_flat.numel(), tau_flat.data_ptr(), tau_flat.numel(),
                ctx.eps_base, doc_c.data_ptr() if ctx.has_doc_ids else None,
                1 if ctx.is_causal else 0, ctx.window_size,
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dscale.data_ptr(), dtau.data_ptr(),
                ws.data_ptr(), ws.numel(), _stream_ptr(q_c.device),
            )
        _native.check(rc, "qdl_flash_purified_born_bwd")
        if dp != D:
            dq, dk, dv = dq[..., :D], dk[..., :D], dv[..., :D]
        return (
            dq.to(ctx.orig_q_dtype),
            dk.to(ctx.orig_k_dtype),
            dv.to(ctx.orig_v_dtype),
            dscale.view(ctx.scale_shape).to(ctx.scale_dtype),
            dtau.view(ctx.tau_shape).to(ctx.tau_dtype),
            None,
            None,
            None,
            None,
            None,
        )


@torch.compiler.disable
def _run_triton_flash_purified_born(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale_t: torch.Tensor,
    tau_t: torch.Tensor,
    eps_base: float,
    is_causal: bool,
    eps: float,
    window_size: int = 0,
    doc_ids: torch.Tensor | None = None,
) -> torch.Tensor:
    """Direct entry to the GPU kernels (reference name, flash_born.py:1273-1287)."""
    return _FlashPurifiedBornAttentionFn.apply(
        q, k, v, scale_t, tau_t, eps_base, is_causal, eps, int(window_size), doc_ids
    )


_run_hip_flash_purified_born = _run_triton_flash_purified_born


def _eager_purified_born(q, k, v, scale_t, tau_t, eps_base, is_causal, eps, window_size, doc_ids):
    """CPU formulation of the reference (flash_born.py:1329-1341), in ``v.dtype``."""
    s = torch.matmul(q.to(v.dtype), k.to(v.dtype).transpose(-1, -2))
    g_v = scale_t.to(s.dtype)
    if g_v.ndim == 1:
        g_v = g_v.view(1, -1, 1, 1)
    t_v = tau_t.to(s.dtype)
    if t_v.ndim == 1:
        t_v = t_v.view(1, -1, 1, 1)
    u = torch.relu(g_v * (s - t_v))
    prob = u.square().square() + float(eps_base) * torch.relu(s).square()
    if is_causal or window_size > 0 or doc_ids is not None:
        prob = _apply_window_and_doc_mask(prob, is_causal, window_size, doc_ids)
    weights = prob / (prob.sum(dim=-1, keepdim=True) + eps)
    return torch.matmul(weights.to(v.dtype), v)


def flash_purified_born_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float | torch.Tensor | None = None,
    tau: float | torch.Tensor | None = None,
    eps_base: float = 0.05,
    is_causal: bool = True,
    eps: float = 1e-8,
    window_size: int = 0,
    doc_ids: torch.Tensor | None = None,
    *,
    gamma_h: float | torch.Tensor | None = None,
    tau_h: float | torch.Tensor | None = None,
    causal: bool | None = None,
) -> torch.Tensor:
    """Purified-Born attention with the reference's signature (flash_born.py:1290-1341).

    Weights ``relu(scale (q.k - tau))^4 + eps_base relu(q.k)^2`` under the
    causal / window / document masks, normalised by their sum + eps.
    ``scale`` (alias ``gamma_h``, default 8.0) and ``tau`` (alias ``tau_h``,
    default 0.0625) are floats or tensors of 1 or H values; ``causal``
    overrides ``is_causal``.  GPU tensors run the gfx950 HIP kernels for any
    head dim up to 256; CPU tensors and larger head dims use the eager
    formulation.
    """
    if scale is None:
        scale = gamma_h if gamma_h is not None else 8.0
    if tau is None:
        tau = tau_h if tau_h is not None else 0.0625
    if causal is not None:
        is_causal = bool(causal)
    scale_t = scale if isinstance(scale, torch.Tensor) else torch.tensor(float(scale), dtype=torch.float32, device=q.device)
    tau_t = tau if isinstance(tau, torch.Tensor) else torch.tensor(float(tau), dtype=torch.float32, device=q.device)
    if q.is_cuda and q.shape[-1] <= MAX_HEAD_DIM:
        return _run_triton_flash_purified_born(
            q, k, v, scale_t, tau_t, eps_base, is_causal, eps, window_size=window_size, doc_ids=doc_ids
        )
    # CPU tensors and D > 256: the reference's eager formulation on the
    # tensors' own device (flash_born.py:1318-1341).
    return _eager_purified_born(q, k, v, scale_t, tau_t, eps_base, is_causal, eps, window_size, doc_ids)
