"""The per-row bound on the kernels' Z (util.z_row_bound) holds for a CPU
emulation of how the kernels form Z, and rejects planted mistakes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc
from util import seeded_inputs, z_row_bound


def _emulate(q, k, scale, dtype, mask, eps, fp16_rounded=False):
    """Z as the 16-bit kernels form it: r in fp32; bf16: the weight r'|r'|
    rounded to bf16 after the relu, fp32 sum, times s^2, plus eps; fp16: the
    fp32 weight relu(|s| r')^2 = relu(s r)^2, fp32 sum, plus eps.
    fp16_rounded: the scheme the fp16 kernels used before, weights (c r)^2
    with c = min(|s|, 1) rounded to fp16 and summed (a planted mistake)."""
    r = q.float() @ k.float().transpose(-1, -2)
    m = torch.from_numpy(mask).float()
    if dtype == torch.float16 and not fp16_rounded:
        a = (r * abs(scale)).clamp_min(0) if scale >= 0 else (-r * abs(scale)).clamp_min(0)
        return ((a * a * m).sum(-1).double() + eps).numpy()
    c = min(abs(scale), 1.0) if dtype == torch.float16 else 1.0
    x = r * c * (1.0 if scale >= 0 else -1.0)
    w = (x * x.abs()).clamp_min(0).to(dtype).float() * m
    return (w.sum(-1).double() * (scale / c) ** 2 + eps).numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [8.0, 0.3, -2.0])
def test_bound_holds_for_the_rounded_weights(dtype, scale):
    q, k = seeded_inputs((2, 3, 200, 64), seed=4, std=0.5, n=2, dtype=dtype)
    mask = orc.visible_mask(200, True, 0)
    qd, kd = q.double().numpy(), k.double().numpy()
    _, z = orc.forward(qd, kd, kd, scale, True, 1e-12)
    zk = _emulate(q, k, scale, dtype, mask, 1e-12)
    bound = z_row_bound(qd, kd, scale, z, 1e-12, dtype, mask)
    assert np.all(np.abs(zk - z) <= bound)


def test_bound_rejects_planted_mistakes():
    dtype = torch.bfloat16
    q, k = seeded_inputs((1, 2, 256, 64), seed=5, std=0.125, n=2, dtype=dtype)
    mask = orc.visible_mask(256, True, 0)
    qd, kd = q.double().numpy(), k.double().numpy()
    _, z = orc.forward(qd, kd, kd, 8.0, True, 1e-12)
    bound = z_row_bound(qd, kd, 8.0, z, 1e-12, dtype, mask)
    good = _emulate(q, k, 8.0, dtype, mask, 1e-12)
    assert np.all(np.abs(good - z) <= bound)
    no_scale = _emulate(q, k, 1.0, dtype, mask, 1e-12)               # s^2 dropped
    assert np.any(np.abs(no_scale - z) > bound)
    half = _emulate(q, k[..., :, :], 8.0, dtype, mask * (np.arange(256) % 2 == 0), 1e-12)  # half the keys
    assert np.any(np.abs(half - z) > bound)
    no_relu_mask = _emulate(q, k, 8.0, dtype, orc.visible_mask(256, False, 0), 1e-12)  # causal mask lost
    assert np.any(np.abs(no_relu_mask - z) > bound)
    shifted = _emulate(q, torch.roll(k, 1, dims=2), 8.0, dtype, mask, 1e-12)  # keys off by one
    assert np.any(np.abs(shifted - z) > bound)


def test_fp16_bound_rejects_rounded_weight_sums():
    """C2-like rows (L2-normalised Q and K, scale 8): many overlaps are tiny,
    and fp16 weights (c r)^2 with c = min(|s|, 1) rounded before the sum flush
    or lose most of their bits; the fp16 bound, from the reference's fp32
    weights, must reject that scheme while accepting the fp32-weight sum."""
    from quantumdlblocks_amd import l2_normalize

    q, k = seeded_inputs((1, 4, 256, 64), seed=6, std=1.0, n=2, dtype=torch.float32)
    q, k = (l2_normalize(x).to(torch.float16) for x in (q, k))
    mask = orc.visible_mask(256, True, 0)
    qd, kd = q.double().numpy(), k.double().numpy()
    _, z = orc.forward(qd, kd, kd, 8.0, True, 1e-12)
    bound = z_row_bound(qd, kd, 8.0, z, 1e-12, torch.float16, mask)
    assert np.all(np.abs(_emulate(q, k, 8.0, torch.float16, mask, 1e-12) - z) <= bound)
    old = _emulate(q, k, 8.0, torch.float16, mask, 1e-12, fp16_rounded=True)
    assert np.any(np.abs(old - z) > bound)
