"""Pins of the Q/K prologue oracle (oracle/qk_prologue_oracle.py) against
library routines, closed forms, invariants and finite differences.  CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import qk_prologue_oracle as po

TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _tables(T, n, base=1024.0, seed=0):
    freqs = 1.0 / base ** (np.arange(n, dtype=np.float64) / max(n, 1))
    ang = np.outer(np.arange(T, dtype=np.float64), freqs).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_round_to_matches_torch_conversion(dtype):
    rng = np.random.default_rng(1)
    vals = [rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-6, 6, 4096)]
    # Ties at the 16-bit boundary, both parities, and special values.
    base = rng.standard_normal(512).astype(np.float32)
    step = 16 if dtype == "bf16" else 13
    u = base.view(np.uint32) & ~np.uint32((1 << step) - 1)
    vals.append((u | np.uint32(1 << (step - 1))).view(np.float32))
    vals.append(np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 65504.0, 65520.0,
                          6e-8, 1e-45], dtype=np.float32))
    x = np.concatenate(vals).astype(np.float32)
    if dtype == "f16":
        x = x[np.abs(x) < 1e30]
    got = po.round_to(x, dtype)
    want = torch.from_numpy(x).to(TORCH_DT[dtype]).float().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    nan = po.round_to(np.array([np.nan], dtype=np.float32), dtype)
    assert np.isnan(nan).all()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("n", [32, 20, 40])
def test_rope_rounding_matches_torch_tensor_ops(dtype, n):
    """torch CPU evaluating the reference's rotation on 16-bit tensors
    (functional.py:118-121 with the padding of attention.py:574-582) agrees
    bit for bit with the oracle's rounding model."""
    T, D = 33, 64
    rng = np.random.default_rng(2)
    x = po.round_to(rng.standard_normal((2, 3, T, D)).astype(np.float32), dtype)
    cos, sin = _tables(T, n)
    got = po.rope(x, cos, sin, dtype)

    xt = torch.from_numpy(x).to(TORCH_DT[dtype])
    ct, st = torch.from_numpy(cos), torch.from_numpy(sin)
    half = D // 2
    if ct.size(-1) >= half:
        ct, st = ct[..., :half], st[..., :half]
    else:
        ct = torch.nn.functional.pad(ct, (0, half - ct.size(-1)), value=1.0)
        st = torch.nn.functional.pad(st, (0, half - st.size(-1)), value=0.0)
    c, s = ct.to(xt.dtype), st.to(xt.dtype)
    x1, x2 = xt[..., :half], xt[..., half:]
    want = torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1).float().numpy()
    np.testing.assert_array_equal(got, want)


def test_rope_closed_form_and_norm():
    T, D = 5, 16
    half = D // 2
    theta = np.array([0.0, 0.3, -1.2, 2.5, math.pi], dtype=np.float64)
    cos = np.cos(theta)[:, None] * np.ones((1, half))
    sin = np.sin(theta)[:, None] * np.ones((1, half))
    for i in range(half):
        x = np.zeros((T, D))
        x[:, i] = 1.0
        y = po.rope(x, cos, sin, "f64")
        want = np.zeros((T, D))
        want[:, i] = np.cos(theta)
        want[:, i + half] = np.sin(theta)
        np.testing.assert_allclose(y, want, atol=1e-15)
        x = np.zeros((T, D))
        x[:, i + half] = 1.0
        y = po.rope(x, cos, sin, "f64")
        want = np.zeros((T, D))
        want[:, i] = -np.sin(theta)
        want[:, i + half] = np.cos(theta)
        np.testing.assert_allclose(y, want, atol=1e-15)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, T, D))
    y = po.rope(x, cos, sin, "f64")
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-13)
    # Angle 0 (row t = 0, and every padded pair) is the identity.
    np.testing.assert_array_equal(y[:, 0], x[:, 0])
    c2, s2 = _tables(T, 3)
    y = po.rope(x, c2.astype(np.float64), s2.astype(np.float64), "f64")
    np.testing.assert_array_equal(y[..., 3:half], x[..., 3:half])
    np.testing.assert_array_equal(y[..., half + 3:], x[..., half + 3:])


@pytest.mark.parametrize("dtype", ["f64", "f32", "bf16"])
def test_forward_unit_norm_and_zero_rows(dtype):
    rng = np.random.default_rng(4)
    T, D = 17, 64
    x = rng.standard_normal((2, 2, T, D)) * 3.0
    x[0, 1, 5] = 0.0
    x = po.round_to(x.astype(np.float32), dtype) if dtype != "f64" else x
    cos, sin = _tables(T, 32)
    out, rinv = po.prologue_forward(x, cos, sin, 1e-12, dtype)
    norms = np.linalg.norm(np.asarray(out, dtype=np.float64), axis=-1)
    tol = {"f64": 1e-12, "f32": 1e-6, "bf16": 1e-2}[dtype]
    mask = np.ones_like(norms, dtype=bool)
    mask[0, 1, 5] = False
    np.testing.assert_allclose(norms[mask], 1.0, atol=tol)
    assert np.all(out[0, 1, 5] == 0)
    np.testing.assert_allclose(rinv[0, 1, 5], 1e6, rtol=1e-6)
    # The exact map is invariant to a positive scale of the row.
    if dtype == "f64":
        with np.errstate(divide="ignore", invalid="ignore"):
            out2, _ = po.prologue_forward(x * 7.5, cos, sin, 0.0, "f64")
            out1, _ = po.prologue_forward(x, cos, sin, 0.0, "f64")
        np.testing.assert_allclose(out2[mask], out1[mask], atol=1e-14)


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(5)
    T, D = 6, 16
    x = rng.standard_normal((1, 2, T, D))
    gy = rng.standard_normal((1, 2, T, D))
    cos, sin = _tables(T, 5)
    cos, sin = cos.astype(np.float64), sin.astype(np.float64)
    eps = 1e-3
    out, rinv = po.prologue_forward(x, cos, sin, eps, "f64")
    dx = po.prologue_backward(gy, out, rinv, cos, sin, "f64")
    h = 1e-6
    num = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fp = np.sum(po.prologue_forward(xp, cos, sin, eps, "f64")[0] * gy)
        fm = np.sum(po.prologue_forward(xm, cos, sin, eps, "f64")[0] * gy)
        num[idx] = (fp - fm) / (2 * h)
    np.testing.assert_allclose(dx, num, rtol=1e-6, atol=1e-8)
    # Without the rotation as well.
    out, rinv = po.prologue_forward(x, None, None, eps, "f64")
    dx = po.prologue_backward(gy, out, rinv, None, None, "f64")
    i = (0, 1, 3, 7)
    xp, xm = x.copy(), x.copy()
    xp[i] += h
    xm[i] -= h
    fd = (np.sum(po.prologue_forward(xp, None, None, eps, "f64")[0] * gy)
          - np.sum(po.prologue_forward(xm, None, None, eps, "f64")[0] * gy)) / (2 * h)
    assert abs(dx[i] - fd) < 1e-7


def test_backward_orthogonal_to_rotated_input():
    """With eps = 0 the output is invariant to scaling the input, so the
    gradient is orthogonal to the input row: dx . x = 0."""
    rng = np.random.default_rng(6)
    T, D = 9, 32
    x = rng.standard_normal((3, T, D))
    gy = rng.standard_normal((3, T, D))
    cos, sin = _tables(T, 16)
    cos, sin = cos.astype(np.float64), sin.astype(np.float64)
    out, rinv = po.prologue_forward(x, cos, sin, 0.0, "f64")
    dx = po.prologue_backward(gy, out, rinv, cos, sin, "f64")
    np.testing.assert_allclose(np.sum(dx * x, axis=-1), 0.0, atol=1e-12)


def test_bf16_against_fp32_at_reference_tolerance():
    """The reference's test of its bf16 L2 normalisation (values within
    2e-2, gradients within 3e-2 of fp32), applied to the whole prologue."""
    rng = np.random.default_rng(101)
    T, D = 16, 64
    x = po.round_to(rng.standard_normal((4, T, D)).astype(np.float32), "bf16")
    gy = po.round_to(rng.standard_normal((4, T, D)).astype(np.float32), "bf16")
    cos, sin = _tables(T, 32)
    ob, rb = po.prologue_forward(x, cos, sin, 1e-12, "bf16")
    of, rf = po.prologue_forward(x, cos, sin, 1e-12, "f32")
    np.testing.assert_allclose(ob, of, atol=2e-2, rtol=2e-2)
    db = po.prologue_backward(gy, ob, rb, cos, sin, "bf16")
    df = po.prologue_backward(gy, of, rf, cos, sin, "f32")
    np.testing.assert_allclose(db, df, atol=3e-2, rtol=3e-2)


def test_eager_torch_against_forward():
    rng = np.random.default_rng(8)
    T, D = 40, 64
    x = po.round_to(rng.standard_normal((2, 3, T, D)).astype(np.float32), "bf16")
    cos, sin = _tables(T, 24)
    got = po.eager_torch(torch.from_numpy(x).to(torch.bfloat16), torch.from_numpy(cos),
                         torch.from_numpy(sin), 1e-12).float().numpy()
    want, _ = po.prologue_forward(x, cos, sin, 1e-12, "bf16")
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30)
    assert np.mean(got == want) > 0.99
