"""The per-row bound on the kernels' Z (util.z_row_bound) holds for a CPU
emulation of how the kernels form Z, and rejects planted mistakes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc
from util import seeded_inputs, z_row_bound


def _emulate(q, k, scale, dtype, mask, eps):
    """Z as the 16-bit kernels form it: r in fp32, weight r'|r'| (fp16: (c r)^2,
    c = min(|s|, 1)) rounded to the dtype after the relu, fp32 sum, times
    (s / c)^2, plus eps."""
    r = q.float() @ k.float().transpose(-1, -2)
    c = min(abs(scale), 1.0) if dtype == torch.float16 else 1.0
    x = r * c
    w = (x * x.abs()).clamp_min(0).to(dtype).float() * torch.from_numpy(mask).float()
    return (w.sum(-1).double() * (scale / c) ** 2 + eps).numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [8.0, 0.3])
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
