"""GPU parity of the fused Q/K prologue (RoPE then L2 normalisation,
attention.py:573-589) against the numpy oracle, through
``fused_qk_rope_l2_normalize`` (which calls the C ABI).

Bars:
  * forward: given the kernel's 1/norm per row, the normalised rows equal the
    oracle's bit for bit (so the rotation and every rounding match the
    reference's rounding model exactly); 1/norm itself within 4 fp32 ulps of
    the oracle's (the row sum's order is the only difference), hence the rows
    within one ulp of the dtype (8 for fp32) of the oracle's own;
  * backward: given the kernel's forward outputs, the input gradient within
    the bound that the dot product's summation order allows (its only
    difference from the oracle) plus a one-ulp flip of each rounded
    intermediate, and for 16-bit dtypes at least 99% of the elements
    bit-identical;
  * end to end: the reference's own bf16 test bar (values within 2e-2,
    gradients within 3e-2 of an fp32 evaluation).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import qk_prologue_oracle as po

pytestmark = pytest.mark.gpu

NAME = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _tables(T, n, base=1024.0):
    freqs = 1.0 / base ** (torch.arange(n, dtype=torch.float32) / max(n, 1))
    ang = torch.outer(torch.arange(T, dtype=torch.float32), freqs)
    return torch.cos(ang).view(1, 1, T, n), torch.sin(ang).view(1, 1, T, n)


def _ulp(x: np.ndarray, dtype) -> np.ndarray:
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    if dtype == torch.bfloat16:
        return np.exp2(np.maximum(e, -126) - 7)
    if dtype == torch.float16:
        return np.exp2(np.maximum(e, -14) - 10)
    return np.exp2(np.maximum(e, -126) - 23)


def _np(t):
    return t.detach().float().cpu().numpy()


CASES = [
    # (B, H, T, D, dtype, n_freq or None, strided input)
    (2, 3, 33, 64, torch.bfloat16, 32, False),
    (2, 3, 33, 64, torch.bfloat16, 32, True),
    (1, 2, 100, 128, torch.bfloat16, 20, False),
    (2, 2, 65, 64, torch.float16, 40, True),
    (2, 2, 50, 64, torch.float32, 32, False),
    (1, 2, 40, 32, torch.float32, 16, True),
    (2, 2, 17, 6, torch.bfloat16, 3, False),
    (1, 3, 21, 10, torch.float32, 2, True),
    (2, 4, 64, 256, torch.bfloat16, 128, False),
    (1, 2, 70, 200, torch.float16, 100, True),
    (1, 1, 1, 64, torch.bfloat16, 32, False),
    (2, 2, 31, 64, torch.bfloat16, None, False),
    (1, 2, 9, 18, torch.float16, None, True),
]


def _inputs(B, H, T, D, dtype, strided, seed, device):
    g = torch.Generator("cpu").manual_seed(seed)
    if strided:  # the (B, T, H, D) projection output viewed as (B, H, T, D)
        q = (torch.randn(B, T, H, D, generator=g) * 0.7).to(dtype).to(device).transpose(1, 2)
        k = (torch.randn(B, T, H, D, generator=g) * 1.3).to(dtype).to(device).transpose(1, 2)
    else:
        q = (torch.randn(B, H, T, D, generator=g) * 0.7).to(dtype).to(device)
        k = (torch.randn(B, H, T, D, generator=g) * 1.3).to(dtype).to(device)
    gq = torch.randn(B, H, T, D, generator=g).to(dtype).to(device)
    gk = torch.randn(B, H, T, D, generator=g).to(dtype).to(device)
    return q, k, gq, gk


@pytest.mark.parametrize(
    "case", CASES,
    ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}D{c[3]}-{NAME[c[4]]}-n{c[5]}-{'strided' if c[6] else 'dense'}",
)
def test_prologue_forward_backward(cuda_device, case):
    from quantumdlblocks_amd.kernels.qk_prologue import (
        fused_qk_rope_l2_normalize,
        qk_prologue_backward,
        qk_prologue_forward,
    )

    B, H, T, D, dtype, nf, strided = case
    name = NAME[dtype]
    q, k, gq, gk = _inputs(B, H, T, D, dtype, strided, seed=T * 7 + D, device=cuda_device)
    if nf is None:
        cos = sin = cos_np = sin_np = None
    else:
        cos, sin = _tables(T, nf)
        cos_np, sin_np = cos[0, 0].numpy(), sin[0, 0].numpy()
        cos, sin = cos.to(cuda_device), sin.to(cuda_device)
    print(f"prologue case B{B} H{H} T{T} D{D} {name} n={nf} strided={strided}", flush=True)
    qo, ko, qr, kr = qk_prologue_forward(q, k, cos, sin, eps=1e-12)
    layouts = [(tuple(x.shape), tuple(x.stride())) for x in (q, k)]
    dq, dk = qk_prologue_backward(gq, gk, qo, ko, qr, kr, cos, sin, *layouts)
    torch.cuda.synchronize()
    assert qo.is_contiguous() and qo.dtype == dtype and ko.dtype == dtype
    assert dq.stride() == q.stride() and dk.stride() == k.stride()

    for x, out, rinv, grad_out, dx in ((q, qo, qr, gq, dq), (k, ko, kr, gk, dk)):
        x_np, out_np, k_rinv = _np(x), _np(out), _np(rinv)
        want_out, want_rinv = po.prologue_forward(x_np, cos_np, sin_np, 1e-12, name)
        np.testing.assert_allclose(k_rinv, want_rinv, rtol=4 * 2.0 ** -23, atol=0)
        # With the kernel's own 1/norm the rows match the oracle bit for bit.
        y = po.rope(x_np, cos_np, sin_np, name) if cos_np is not None else x_np
        rebuilt = po.round_to((y * k_rinv[..., None]).astype(np.float32), name)
        np.testing.assert_array_equal(out_np, rebuilt)
        mult = 8 if dtype == torch.float32 else 1
        assert np.all(np.abs(out_np - want_out) <= mult * _ulp(want_out, dtype))

        g_np = _np(grad_out)
        want_dx = po.prologue_backward(g_np, out_np, k_rinv, cos_np, sin_np, name)
        got_dx = _np(dx)
        diff = np.abs(got_dx - want_dx)
        # The row's fp32 dot product (g . y) is summed in another order than
        # the oracle's: bound its error, carry it through (g - dot y) / norm and
        # the rotation, and allow a one-ulp flip of each rounded intermediate.
        dot_err = D * 2.0 ** -24 * np.sum(np.abs(g_np * out_np), axis=-1, keepdims=True)
        l2 = (g_np - np.sum(g_np * out_np, axis=-1, keepdims=True) * out_np) * k_rinv[..., None]
        half = D // 2
        pair = np.maximum(np.abs(l2[..., :half]), np.abs(l2[..., half:]))
        pair = np.concatenate([pair, pair], axis=-1)
        bound = (mult * _ulp(want_dx, dtype) + 2 * mult * _ulp(pair, dtype)
                 + 2 * dot_err * np.abs(out_np).max(axis=-1, keepdims=True) * k_rinv[..., None])
        assert np.all(diff <= bound), float((diff - bound).max())
        if dtype != torch.float32:
            assert np.mean(diff == 0) >= 0.99

    # The autograd entry point gives the same tensors.
    qa = q.detach().requires_grad_(True)
    ka = k.detach().requires_grad_(True)
    qo2, ko2 = fused_qk_rope_l2_normalize(qa, ka, cos, sin, eps=1e-12)
    torch.autograd.backward([qo2, ko2], [gq, gk])
    torch.cuda.synchronize()
    assert torch.equal(qo2, qo) and torch.equal(ko2, ko)
    assert torch.equal(qa.grad, dq) and torch.equal(ka.grad, dk)
    assert qa.grad.stride() == q.stride()


def test_prologue_reference_bf16_bar(cuda_device):
    """The reference's bf16 L2-normalisation test bar
    (tests/test_plan041_15gb_batch24576_dyadic_scaling.py:24-44), on the whole
    fused prologue against an fp32 eager evaluation, at a C3-sized shape."""
    from quantumdlblocks_amd.kernels.qk_prologue import (
        apply_unitary_rope,
        fused_qk_rope_l2_normalize,
    )

    torch.manual_seed(101)
    B, T, H, D = 4, 1024, 16, 64
    cos, sin = _tables(T, 32)
    cos, sin = cos.to(cuda_device), sin.to(cuda_device)
    raw = torch.randn(B, T, 2 * H * D, device=cuda_device).to(torch.bfloat16)
    q = raw[..., : H * D].view(B, T, H, D).transpose(1, 2).detach().requires_grad_(True)
    k = raw[..., H * D :].view(B, T, H, D).transpose(1, 2).detach().requires_grad_(True)
    gq = torch.randn(B, H, T, D, device=cuda_device).to(torch.bfloat16)
    gk = torch.randn(B, H, T, D, device=cuda_device).to(torch.bfloat16)
    qo, ko = fused_qk_rope_l2_normalize(q, k, cos, sin, eps=1e-12)
    torch.autograd.backward([qo, ko], [gq, gk])

    def ref(x):
        xf = x.detach().float().requires_grad_(True)
        y = apply_unitary_rope(xf, cos, sin)
        y = y * torch.rsqrt(torch.sum(y * y, dim=-1, keepdim=True) + 1e-12)
        return xf, y

    qf, qy = ref(q)
    kf, ky = ref(k)
    torch.autograd.backward([qy, ky], [gq.float(), gk.float()])
    torch.cuda.synchronize()
    assert torch.allclose(qo.float(), qy, atol=2e-2, rtol=2e-2)
    assert torch.allclose(ko.float(), ky, atol=2e-2, rtol=2e-2)
    assert torch.allclose(q.grad.float(), qf.grad, atol=3e-2, rtol=3e-2)
    assert torch.allclose(k.grad.float(), kf.grad, atol=3e-2, rtol=3e-2)


def test_prologue_empty_and_single_tensor(cuda_device):
    from quantumdlblocks_amd.kernels.qk_prologue import fused_qk_rope_l2_normalize

    q = torch.zeros(2, 3, 0, 64, device=cuda_device, dtype=torch.bfloat16)
    qo, ko = fused_qk_rope_l2_normalize(q, q.clone())
    assert qo.shape == q.shape and ko.shape == q.shape
    # Only k needs a gradient: q's stays None.
    q = torch.randn(1, 2, 16, 64, device=cuda_device).to(torch.bfloat16)
    k = torch.randn(1, 2, 16, 64, device=cuda_device).to(torch.bfloat16).requires_grad_(True)
    cos, sin = _tables(16, 32)
    qo, ko = fused_qk_rope_l2_normalize(q, k, cos.to(cuda_device), sin.to(cuda_device))
    ko.float().sum().backward()
    torch.cuda.synchronize()
    assert k.grad is not None and torch.isfinite(k.grad.float()).all()
    assert qo.requires_grad is False or qo.grad_fn is not None


def test_prologue_gradients_of_sliced_and_expanded_inputs(cuda_device):
    """Q and K cut from one fused projection (rows with gaps) and an expanded
    K (stride 0 over heads): gradients equal those of contiguous copies."""
    from quantumdlblocks_amd.kernels.qk_prologue import fused_qk_rope_l2_normalize

    B, T, H, D = 2, 40, 4, 64
    g = torch.Generator("cpu").manual_seed(5)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(torch.bfloat16).to(cuda_device).requires_grad_(True)
    k1 = torch.randn(B, 1, T, D, generator=g).to(torch.bfloat16).to(cuda_device).requires_grad_(True)
    cos, sin = _tables(T, D // 2)
    cos, sin = cos.to(cuda_device), sin.to(cuda_device)
    gq = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(cuda_device)
    gk = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(cuda_device)

    q = qkv[..., : H * D].view(B, T, H, D).transpose(1, 2)
    k = k1.expand(B, H, T, D)
    qo, ko = fused_qk_rope_l2_normalize(q, k, cos, sin)
    torch.autograd.backward([qo, ko], [gq, gk])

    qkv2 = qkv.detach().clone().requires_grad_(True)
    k2 = k1.detach().clone().requires_grad_(True)
    qc = qkv2[..., : H * D].view(B, T, H, D).transpose(1, 2).contiguous()
    kc = k2.expand(B, H, T, D).contiguous()
    qo2, ko2 = fused_qk_rope_l2_normalize(qc, kc, cos, sin)
    torch.autograd.backward([qo2, ko2], [gq, gk])
    torch.cuda.synchronize()
    assert torch.equal(qo, qo2) and torch.equal(ko, ko2)
    assert torch.equal(qkv.grad, qkv2.grad)
    # The expanded K's gradient is the sum over heads, in autograd's order for both.
    assert torch.allclose(k1.grad.float(), k2.grad.float(), rtol=0, atol=0)


def test_prologue_gradients_of_transposed_inputs(cuda_device):
    """Q and K stored (B, H, D, T) and viewed as (B, H, T, D): a dense layout
    whose D stride is not 1.  The inputs are read through a contiguous copy
    and the gradients must come back equal to those of contiguous inputs (the
    kernel writes D rows contiguously, so such a gradient is allocated
    contiguous rather than with the input's strides)."""
    from quantumdlblocks_amd.kernels.qk_prologue import fused_qk_rope_l2_normalize

    B, H, T, D = 2, 3, 16, 64
    g = torch.Generator("cpu").manual_seed(11)
    qt = torch.randn(B, H, D, T, generator=g).to(torch.bfloat16).to(cuda_device).requires_grad_(True)
    kt = torch.randn(B, H, D, T, generator=g).to(torch.bfloat16).to(cuda_device).requires_grad_(True)
    cos, sin = _tables(T, D // 2)
    cos, sin = cos.to(cuda_device), sin.to(cuda_device)
    gq = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(cuda_device)
    gk = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(cuda_device)

    q, k = qt.transpose(-1, -2), kt.transpose(-1, -2)
    assert q.stride(-1) != 1
    qo, ko = fused_qk_rope_l2_normalize(q, k, cos, sin)
    torch.autograd.backward([qo, ko], [gq, gk])

    qc = qt.detach().transpose(-1, -2).contiguous().requires_grad_(True)
    kc = kt.detach().transpose(-1, -2).contiguous().requires_grad_(True)
    qo2, ko2 = fused_qk_rope_l2_normalize(qc, kc, cos, sin)
    torch.autograd.backward([qo2, ko2], [gq, gk])
    torch.cuda.synchronize()
    assert torch.equal(qo, qo2) and torch.equal(ko, ko2)
    assert torch.equal(qt.grad.transpose(-1, -2), qc.grad)
    assert torch.equal(kt.grad.transpose(-1, -2), kc.grad)
