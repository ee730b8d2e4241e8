"""CPU oracle for flash-Born attention.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline).  The product path in
``quantumdlblocks_amd`` never imports it.

It restates, from scratch, the semantics of the reference's Born attention
(``src/qdlblocks/kernels/flash_born.py`` in Vengo/QuantumDLBlocks):

    r_ij = q_i . k_j
    a_ij = max(0, scale_h * r_ij) * M_ij          (flash_born.py:166-180, 684-686)
    M_ij = [causal => j <= i] & [W > 0 => i - j < W] & [doc_i == doc_j]
                                                  (flash_born.py:169-177, 635-652)
    p_ij = a_ij ** 2
    Z_i  = sum_j p_ij + eps                       (flash_born.py:182, 185, 192)
    O_i  = sum_j p_ij v_j / Z_i                   (flash_born.py:183-186, 689-690)

and the backward pass of ``_flash_born_bwd_kernel`` /
``_flash_born_bwd_dq_kernel`` (flash_born.py:270-322, 387-427):

    delta_i = dO_i . O_i
    dP_ij   = (dO_i . v_j - delta_i) / Z_i
    dS_ij   = 2 a_ij dP_ij
    dq_i    = scale_h sum_j dS_ij k_j
    dk_j    = scale_h sum_i dS_ij q_i
    dv_j    = sum_i (p_ij / Z_i) dO_i
    dscale  = sum_{b,i,j} dS_ij r_ij   (per head when the scale is per head)

Everything is float64 numpy except ``eager_fp32_torch``, which restates the
reference's eager CPU path (flash_born.py:681-690) op for op in fp32 torch and
is what ``bench.py`` times as the CPU baseline.

How each function is pinned (tests/test_oracle.py):
  * ``compute_document_ids``: the literal golden tensor of the reference test
    tests/test_hypothesis_016_speedrun_systems_and_arch.py:163-177.
  * ``forward``: brute-force scalar loops in C (oracle/born_oracle.c, written
    independently of this file) on small shapes; hand-computed closed forms
    (T=1, T=2 with D=1); invariants (constant V, scale invariance, window=1,
    window >= T, all-equal / all-distinct doc ids, permutation equivariance,
    all-negative overlaps give O = 0, row weights sum to (Z-eps)/Z).  Its
    ``weight_dtype`` mode (the P.V weights rounded as the reference's kernel
    casts them): one-key rows whose weights sit on fp16's subnormal edges,
    worked by hand, and torch evaluating the reference kernel's arithmetic
    op by op in fp32 (fp16 and bf16).
  * ``backward``: torch.autograd of an independent float64 torch statement of
    the forward, float64 finite differences (torch.autograd.gradcheck), the
    C brute force, and the closed form dscale = (2/s) sum delta eps / Z; the
    ``out=`` path (delta from a given forward output) by perturbing ``out``
    and checking dP moves by -dO . d(out) / Z.
  * ``backward_magnitudes``: bounds |backward| elementwise, and equals |dv|
    when dO > 0 (every dv term is then non-negative).
  * ``eager_fp32_torch``: against ``forward`` at fp32 tolerance.

Purified-Born attention (flash_born.py:693-1341; the section-8 "next" row):

    u_ij = max(0, g_h (r_ij - tau_h)) M_ij, b_ij = max(0, r_ij) M_ij
                                                  (flash_born.py:782-796)
    p_ij = u_ij^4 + eps_base b_ij^2               (flash_born.py:798-799)
    Z_i  = sum_j p_ij + eps, O_i = sum_j p_ij v_j / Z_i   (801-811)
    backward (flash_born.py:905-940, 1035-1058), delta_i = dO_i . O_i:
    dP_ij = (dO_i . v_j - delta_i) / Z_i, du_ij = 4 u_ij^3 dP_ij,
    dR_ij = g_h du_ij + 2 eps_base b_ij dP_ij,
    dq = dR K, dk = dR^T Q, dv = (P / Z)^T dO,
    dg_h = sum du (r - tau), dtau_h = -g_h sum du.

How they are pinned (tests/test_oracle.py): with g = 0 the weights reduce to
eps_base b^2, i.e. Born attention with scale 1 and eps / eps_base (pinned
above); with eps_base = 0 and tau = 0 the output is invariant under g > 0;
brute-force scalar loops on tiny shapes; the gradients against
torch.autograd of ``purified_eager_fp32_torch`` run in float64 and against
float64 finite differences (gradcheck), dg and dtau included.
"""

from __future__ import annotations

import numpy as np

from .qk_prologue_oracle import round_to

__all__ = [
    "compute_document_ids",
    "visible_mask",
    "forward",
    "backward",
    "born_weights",
    "backward_magnitudes",
    "eager_fp32_torch",
    "visible_pairs",
    "geometric_doc_ids",
    "purified_forward",
    "purified_backward",
    "purified_backward_magnitudes",
    "purified_eager_fp32_torch",
]


def compute_document_ids(idx, eot_token_id: int = 50256) -> np.ndarray:
    """Per-token document ids; an EOT token belongs to the document it ends.

    Restates ``compute_document_ids`` (src/qdlblocks/layers/attention.py:308-315):
    ``cumsum(idx == eot) - (idx == eot)`` as int32.
    """
    idx = np.asarray(idx)
    is_eot = (idx == int(eot_token_id)).astype(np.int32)
    return (np.cumsum(is_eot, axis=-1, dtype=np.int32) - is_eot).astype(np.int32)


def visible_mask(T: int, is_causal: bool, window_size: int, doc_ids=None) -> np.ndarray:
    """Boolean visibility mask, shape (1 or B, 1, T, T).

    Restates ``_apply_window_and_doc_mask`` (flash_born.py:635-652): causal
    ``i - j >= 0``; window ``i - j < W`` when W > 0 (applied with or without
    causality); document equality when ``doc_ids`` (B, T) is given.
    """
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    diff = i - j
    m = (diff >= 0) if is_causal else np.ones((T, T), dtype=bool)
    if window_size > 0:
        m = m & (diff < int(window_size))
    m = m[None, None]
    if doc_ids is not None:
        d = np.asarray(doc_ids)
        m = m & (d[:, None, :, None] == d[:, None, None, :])
    return m


def _scale_bh(scale, H: int) -> np.ndarray:
    """Scale broadcast to (1, H|1, 1, 1): scalar, or exactly H per-head values.

    Mirrors flash_born.py:452-453 (``numel() > 1`` means per head, indexed by
    h) and 681-683 (a 1-D scale is viewed as (1, H, 1, 1)).
    """
    s = np.asarray(scale, dtype=np.float64).reshape(-1)
    if s.size == 1:
        return s.reshape(1, 1, 1, 1)
    if s.size != H:
        raise ValueError(f"per-head scale needs exactly H={H} values, got {s.size}")
    return s.reshape(1, H, 1, 1)


def _f64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


def born_weights(q, k, scale, is_causal=True, eps=1e-12, window_size=0, doc_ids=None):
    """Normalised Born weights p_ij / Z_i, float64, shape (B, H, T, T)."""
    q, k = _f64(q), _f64(k)
    T = q.shape[-2]
    r = q @ np.swapaxes(k, -1, -2)
    a = np.maximum(_scale_bh(scale, q.shape[1]) * r, 0.0)
    a = a * visible_mask(T, is_causal, window_size, None if doc_ids is None else _f64(doc_ids))
    p = a * a
    return p / (p.sum(-1, keepdims=True) + eps)


def forward(q, k, v, scale, is_causal=True, eps=1e-12, window_size=0, doc_ids=None, weight_dtype=None):
    """Born attention forward in float64.  Returns (O, Z), O (B,H,T,D), Z (B,H,T).

    ``weight_dtype`` ("f16" or "bf16"): the weights enter the P.V product
    rounded to that dtype from their fp32 value, as the reference's kernel
    casts them (``p.to(v.dtype)``, flash_born.py:182-183), while Z sums them
    unrounded (:182); a weight below the dtype's smallest subnormal then
    contributes nothing to O.  None: exact."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, H, T, D = q.shape
    r = q @ np.swapaxes(k, -1, -2)
    a = np.maximum(_scale_bh(scale, H) * r, 0.0)
    a = a * visible_mask(T, is_causal, window_size, None if doc_ids is None else _f64(doc_ids))
    p = a * a
    Z = p.sum(-1) + eps
    pv = p if weight_dtype is None else round_to(p.astype(np.float32), weight_dtype).astype(np.float64)
    O = (pv @ v) / Z[..., None]
    return O, Z


def backward(q, k, v, scale, do, is_causal=True, eps=1e-12, window_size=0, doc_ids=None, out=None):
    """Closed-form gradients in float64.

    Returns (dq, dk, dv, dscale) with dscale shaped like the flattened scale
    (1 value, or H values for a per-head scale).  ``out``: the forward output
    the backward is handed; as in the reference (flash_born.py:277, 302,
    387), delta_i = dO_i . out_i is formed from it.  Defaults to the exact O.
    """
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    B, H, T, D = q.shape
    s_bh = _scale_bh(scale, H)
    r = q @ np.swapaxes(k, -1, -2)
    a = np.maximum(s_bh * r, 0.0)
    a = a * visible_mask(T, is_causal, window_size, None if doc_ids is None else _f64(doc_ids))
    p = a * a
    Z = p.sum(-1) + eps
    O = (p @ v) / Z[..., None] if out is None else _f64(out)
    delta = (do * O).sum(-1)
    dP = (do @ np.swapaxes(v, -1, -2) - delta[..., None]) / Z[..., None]
    dS = 2.0 * a * dP
    dq = s_bh * (dS @ k)
    dk = s_bh * (np.swapaxes(dS, -1, -2) @ q)
    dv = np.swapaxes(p / Z[..., None], -1, -2) @ do
    per_head = np.asarray(scale).size > 1
    dsr = (dS * r).sum(axis=(0, 2, 3))  # per head
    dscale = dsr if per_head else np.array([dsr.sum()])
    return dq, dk, dv, dscale


def backward_magnitudes(q, k, v, scale, do, is_causal=True, eps=1e-12, window_size=0, doc_ids=None):
    """Size of the terms each gradient sums, float64, same shapes as
    (dq, dk, dv): the closed form of ``backward`` with every product taken in
    absolute value.  Gradients that cancel to ~0 (a row that sees one key, or
    a window of 1) are compared against a small fraction of this scale."""
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    B, H, T, D = q.shape
    s_bh = _scale_bh(scale, H)
    r = q @ np.swapaxes(k, -1, -2)
    a = np.maximum(s_bh * r, 0.0)
    a = a * visible_mask(T, is_causal, window_size, None if doc_ids is None else _f64(doc_ids))
    p = a * a
    Z = p.sum(-1) + eps
    O = (p @ v) / Z[..., None]
    delta = np.abs(do * O).sum(-1)
    dP = (np.abs(do) @ np.abs(np.swapaxes(v, -1, -2)) + delta[..., None]) / Z[..., None]
    dS = 2.0 * a * dP
    dq = np.abs(s_bh) * (dS @ np.abs(k))
    dk = np.abs(s_bh) * (np.swapaxes(dS, -1, -2) @ np.abs(q))
    dv = np.swapaxes(p / Z[..., None], -1, -2) @ np.abs(do)
    return dq, dk, dv


def visible_pairs(B: int, T: int, is_causal: bool = True, window_size: int = 0, doc_ids=None) -> int:
    """Number of visible (b, i, j) pairs summed over the batch, for one head.

    Used for the algorithmic FLOP count: fwd = 4 * D * H * pairs.
    """
    if doc_ids is None:
        if window_size <= 0:
            per_row = T * (T + 1) // 2 if is_causal else T * T
        else:
            i = np.arange(T, dtype=np.int64)
            if is_causal:
                per_row = int(np.minimum(i + 1, window_size).sum())
            else:  # keys j > i - W, i.e. j in [max(0, i-W+1), T)
                per_row = int((T - np.maximum(0, i - window_size + 1)).sum())
        return B * per_row
    total = 0
    d = np.asarray(doc_ids)
    for b in range(d.shape[0]):
        m = visible_mask(T, is_causal, window_size, d[b : b + 1])
        total += int(m.sum())
    return total


def geometric_doc_ids(B: int, T: int, mean_len: float, seed: int) -> np.ndarray:
    """Document ids for the long-context config: per row, document lengths are
    drawn from a geometric distribution with the given mean (support >= 1) from
    ``np.random.default_rng(seed)``, the last document truncated at T."""
    rng = np.random.default_rng(seed)
    out = np.empty((B, T), dtype=np.int32)
    for b in range(B):
        t = 0
        doc = 0
        while t < T:
            n = int(rng.geometric(1.0 / mean_len))
            out[b, t : t + n] = doc
            t += n
            doc += 1
    return out


def eager_fp32_torch(q, k, v, scale, is_causal=True, eps=1e-12, window_size=0, doc_ids=None):
    """The reference's eager path (flash_born.py:681-690) restated op for op.

    ``matmul(q, k^T) * scale -> relu -> square -> mask multiply ->
    prob / (sum prob + eps) -> matmul(., v)``, computed in ``v.dtype`` on the
    tensors' device.  Full T x T matmuls, no causal skipping.
    """
    import torch

    if not isinstance(scale, torch.Tensor):
        scale = torch.tensor(float(scale), dtype=torch.float32, device=q.device)
    s_v = scale.to(v.dtype)
    if s_v.ndim == 1:
        s_v = s_v.view(1, -1, 1, 1)
    scaled = torch.matmul(q.to(v.dtype), k.to(v.dtype).transpose(-1, -2)) * s_v
    prob = torch.relu(scaled).square()
    if is_causal or window_size > 0 or doc_ids is not None:
        T = prob.shape[-1]
        idx = torch.arange(T, device=prob.device)
        diff = idx[:, None] - idx[None, :]
        mask = (diff >= 0) if is_causal else torch.ones((T, T), device=prob.device, dtype=torch.bool)
        if window_size > 0:
            mask = mask & (diff < int(window_size))
        mask = mask.view(1, 1, T, T)
        if doc_ids is not None:
            mask = mask & (doc_ids[:, None, :, None] == doc_ids[:, None, None, :])
        prob = prob * mask.to(prob.dtype)
    w = prob / (torch.sum(prob, dim=-1, keepdim=True) + eps)
    return torch.matmul(w.to(v.dtype), v)


def _purified_parts(q, k, scale, tau, eps_base, is_causal, window_size, doc_ids):
    q, k = _f64(q), _f64(k)
    B, H, T, D = q.shape
    g = _scale_bh(scale, H)
    t = _scale_bh(tau, H)
    r = q @ np.swapaxes(k, -1, -2)
    m = visible_mask(T, is_causal, window_size, None if doc_ids is None else _f64(doc_ids))
    u = np.maximum(g * (r - t), 0.0) * m
    b = np.maximum(r, 0.0) * m
    p = u**4 + float(eps_base) * b * b
    return g, t, r, u, b, p


def purified_forward(q, k, v, scale, tau, eps_base=0.05, is_causal=True, eps=1e-8, window_size=0, doc_ids=None):
    """Purified-Born forward in float64 (flash_born.py:771-811).  Returns (O, Z)."""
    v = _f64(v)
    _, _, _, _, _, p = _purified_parts(q, k, scale, tau, eps_base, is_causal, window_size, doc_ids)
    Z = p.sum(-1) + eps
    return (p @ v) / Z[..., None], Z


def purified_backward(q, k, v, scale, tau, do, eps_base=0.05, is_causal=True, eps=1e-8, window_size=0,
                      doc_ids=None, out=None):
    """Purified-Born gradients in float64 (flash_born.py:905-940, 1035-1058).

    Returns (dq, dk, dv, dscale, dtau); dscale / dtau hold one value, or H
    values for a per-head parameter.  ``out``: the forward output handed to
    the backward (delta_i = dO_i . out_i, flash_born.py:928, 1014);
    defaults to the exact O.
    """
    q64, k64, v64, do = _f64(q), _f64(k), _f64(v), _f64(do)
    g, t, r, u, b, p = _purified_parts(q64, k64, scale, tau, eps_base, is_causal, window_size, doc_ids)
    Z = p.sum(-1) + eps
    O = (p @ v64) / Z[..., None] if out is None else _f64(out)
    delta = (do * O).sum(-1)
    dP = (do @ np.swapaxes(v64, -1, -2) - delta[..., None]) / Z[..., None]
    du = 4.0 * u**3 * dP
    dR = g * du + 2.0 * float(eps_base) * b * dP
    dq = dR @ k64
    dk = np.swapaxes(dR, -1, -2) @ q64
    dv = np.swapaxes(p / Z[..., None], -1, -2) @ do
    dg_h = (du * (r - t)).sum(axis=(0, 2, 3))
    dt_h = (-g * du).sum(axis=(0, 2, 3))
    dscale = dg_h if np.asarray(scale).size > 1 else np.array([dg_h.sum()])
    dtau = dt_h if np.asarray(tau).size > 1 else np.array([dt_h.sum()])
    return dq, dk, dv, dscale, dtau


def purified_backward_magnitudes(q, k, v, scale, tau, do, eps_base=0.05, is_causal=True, eps=1e-8,
                                 window_size=0, doc_ids=None):
    """Size of the terms each purified gradient sums (every product in
    absolute value): (dq, dk, dv) shaped like the gradients, then the dscale
    and dtau term sums shaped like those outputs.  The noise floor for
    gradients that cancel to ~0."""
    q64, k64, v64, do = _f64(q), _f64(k), _f64(v), _f64(do)
    g, t, r, u, b, p = _purified_parts(q64, k64, scale, tau, eps_base, is_causal, window_size, doc_ids)
    Z = p.sum(-1) + eps
    O = (p @ v64) / Z[..., None]
    delta = np.abs(do * O).sum(-1)
    dP = (np.abs(do) @ np.abs(np.swapaxes(v64, -1, -2)) + delta[..., None]) / Z[..., None]
    du = 4.0 * u**3 * dP
    dR = np.abs(g) * du + 2.0 * abs(float(eps_base)) * b * dP
    ds_h = (du * np.abs(r - t)).sum(axis=(0, 2, 3))
    dt_h = (np.abs(g) * du).sum(axis=(0, 2, 3))
    ds = ds_h if np.asarray(scale).size > 1 else np.array([ds_h.sum()])
    dt = dt_h if np.asarray(tau).size > 1 else np.array([dt_h.sum()])
    return (dR @ np.abs(k64), np.swapaxes(dR, -1, -2) @ np.abs(q64),
            np.swapaxes(p / Z[..., None], -1, -2) @ np.abs(do), ds, dt)


def purified_eager_fp32_torch(q, k, v, scale, tau, eps_base=0.05, is_causal=True, eps=1e-8, window_size=0,
                              doc_ids=None):
    """The reference's eager purified path (flash_born.py:1329-1341) restated
    op for op, in ``v.dtype`` on the tensors' device, full T x T matmuls."""
    import torch

    if not isinstance(scale, torch.Tensor):
        scale = torch.tensor(float(scale), dtype=torch.float32, device=q.device)
    if not isinstance(tau, torch.Tensor):
        tau = torch.tensor(float(tau), dtype=torch.float32, device=q.device)
    s = torch.matmul(q.to(v.dtype), k.to(v.dtype).transpose(-1, -2))
    g_v = scale.to(s.dtype)
    if g_v.ndim == 1:
        g_v = g_v.view(1, -1, 1, 1)
    t_v = tau.to(s.dtype)
    if t_v.ndim == 1:
        t_v = t_v.view(1, -1, 1, 1)
    u = torch.relu(g_v * (s - t_v))
    prob = u.square().square() + float(eps_base) * torch.relu(s).square()
    if is_causal or window_size > 0 or doc_ids is not None:
        T = prob.shape[-1]
        idx = torch.arange(T, device=prob.device)
        diff = idx[:, None] - idx[None, :]
        mask = (diff >= 0) if is_causal else torch.ones((T, T), device=prob.device, dtype=torch.bool)
        if window_size > 0:
            mask = mask & (diff < int(window_size))
        mask = mask.view(1, 1, T, T)
        if doc_ids is not None:
            mask = mask & (doc_ids[:, None, :, None] == doc_ids[:, None, None, :])
        prob = prob * mask.to(prob.dtype)
    w = prob / (torch.sum(prob, dim=-1, keepdim=True) + eps)
    return torch.matmul(w.to(v.dtype), v)
