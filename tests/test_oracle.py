"""Pins the CPU oracle (oracle/born_oracle.py) before anything is checked against it.

Each check is independent of the formula it tests: a literal golden tensor
from the reference's own tests, a brute-force C restatement, hand-computed
closed forms, invariants of the mathematics, torch.autograd / finite
differences for the backward, and planted mistakes that the pins must catch.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLIB = os.path.join(ROOT, "oracle", "_build", "libborn_oracle.so")


# --------------------------------------------------------------------------
# brute-force C restatement (oracle/born_oracle.c)
# --------------------------------------------------------------------------

@pytest.fixture(scope="module")
def clib():
    if not os.path.exists(CLIB):
        import subprocess

        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    return ctypes.CDLL(CLIB)


_P = ctypes.c_void_p
_I = ctypes.c_int64


def _c_doc(doc):
    return None if doc is None else np.ascontiguousarray(doc, dtype=np.int32)


def c_forward(lib, q, k, v, scale, causal, eps, window, doc):
    q, k, v = (np.ascontiguousarray(x, np.float64) for x in (q, k, v))
    B, H, T, D = q.shape
    out = np.zeros_like(q)
    z = np.zeros((B, H, T))
    sc = np.ascontiguousarray(np.asarray(scale, np.float64).reshape(-1))
    d = _c_doc(doc)
    lib.born_oracle_fwd(_I(B), _I(H), _I(T), _I(D), q.ctypes.data_as(_P), k.ctypes.data_as(_P),
                        v.ctypes.data_as(_P), sc.ctypes.data_as(_P), _I(sc.size),
                        None if d is None else d.ctypes.data_as(_P), ctypes.c_int(int(causal)),
                        _I(window), ctypes.c_double(eps), out.ctypes.data_as(_P), z.ctypes.data_as(_P))
    return out, z


def c_backward(lib, q, k, v, scale, do, causal, eps, window, doc):
    q, k, v, do = (np.ascontiguousarray(x, np.float64) for x in (q, k, v, do))
    B, H, T, D = q.shape
    dq, dk, dv = (np.zeros_like(q) for _ in range(3))
    sc = np.ascontiguousarray(np.asarray(scale, np.float64).reshape(-1))
    ds = np.zeros(sc.size)
    d = _c_doc(doc)
    lib.born_oracle_bwd(_I(B), _I(H), _I(T), _I(D), q.ctypes.data_as(_P), k.ctypes.data_as(_P),
                        v.ctypes.data_as(_P), sc.ctypes.data_as(_P), _I(sc.size),
                        None if d is None else d.ctypes.data_as(_P), ctypes.c_int(int(causal)),
                        _I(window), ctypes.c_double(eps), do.ctypes.data_as(_P), dq.ctypes.data_as(_P),
                        dk.ctypes.data_as(_P), dv.ctypes.data_as(_P), ds.ctypes.data_as(_P))
    return dq, dk, dv, ds


def _rand(shape, seed, n=3):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(shape) for _ in range(n)]


CASES = [
    # (B, H, T, D, scale, causal, window, doc_mean, eps)
    (2, 3, 17, 8, 1.5, True, 0, None, 1e-12),
    (1, 2, 33, 16, [2.5, -3.0], True, 0, None, 1e-6),
    (2, 2, 29, 4, 0.7, False, 0, None, 1e-12),
    (2, 1, 40, 8, 1.0, True, 5, None, 1e-12),
    (1, 2, 40, 8, [1.0, 0.0], False, 7, None, 1e-3),
    (3, 2, 41, 8, 2.0, True, 0, 6.0, 1e-12),
    (2, 2, 37, 8, 1.0, False, 0, 4.0, 1e-12),
    (2, 2, 50, 8, 1.3, True, 9, 8.0, 1e-9),
]


@pytest.mark.parametrize("case", CASES)
def test_forward_matches_brute_force(clib, case):
    B, H, T, D, scale, causal, window, doc_mean, eps = case
    q, k, v = _rand((B, H, T, D), seed=T)
    doc = None if doc_mean is None else orc.geometric_doc_ids(B, T, doc_mean, seed=B)
    o_c, z_c = c_forward(clib, q, k, v, scale, causal, eps, window, doc)
    o_n, z_n = orc.forward(q, k, v, np.asarray(scale), causal, eps, window, doc)
    np.testing.assert_allclose(o_n, o_c, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(z_n, z_c, rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("case", CASES)
def test_backward_matches_brute_force(clib, case):
    B, H, T, D, scale, causal, window, doc_mean, eps = case
    q, k, v, do = _rand((B, H, T, D), seed=T + 1, n=4)
    doc = None if doc_mean is None else orc.geometric_doc_ids(B, T, doc_mean, seed=B)
    got = orc.backward(q, k, v, np.asarray(scale), do, causal, eps, window, doc)
    want = c_backward(clib, q, k, v, scale, do, causal, eps, window, doc)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=1e-9, atol=1e-9 * max(1.0, np.abs(w).max()))


# --------------------------------------------------------------------------
# literal golden of the reference's own test
# --------------------------------------------------------------------------

def test_compute_document_ids_literal_golden():
    """tests/test_hypothesis_016_speedrun_systems_and_arch.py:163-177 of the reference."""
    idx = np.array([[10, 20, 50256, 30, 40, 50256, 50, 60], [11, 50256, 22, 33, 44, 55, 66, 77]])
    expected = np.array([[0, 0, 0, 1, 1, 1, 2, 2], [0, 0, 1, 1, 1, 1, 1, 1]], dtype=np.int32)
    got = orc.compute_document_ids(idx, eot_token_id=50256)
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got, expected)


# --------------------------------------------------------------------------
# hand-computed closed forms
# --------------------------------------------------------------------------

def test_single_token():
    """T=1: O_0 = v_0 * p/(p+eps) with p = relu(s q.k)^2, so v_0 if q.k > 0 else 0."""
    q = np.array([[[[1.0, 2.0]]]])
    k = np.array([[[[0.5, 0.25]]]])  # q.k = 1
    v = np.array([[[[3.0, -4.0]]]])
    o, z = orc.forward(q, k, v, 2.0, eps=0.0)
    np.testing.assert_allclose(o, v)
    np.testing.assert_allclose(z, [[[4.0]]])
    o, z = orc.forward(q, -k, v, 2.0, eps=0.0)  # overlap -2 -> relu 0
    assert np.all(np.nan_to_num(o) == 0)


def test_two_tokens_by_hand():
    """D=1, T=2, causal, scale 1: r = q_i k_j.
    q = (1, 2), k = (3, -1), v = (10, 20), eps = 1:
    row 0: r00 = 3 -> p = 9; Z = 10; O = 90/10 = 9
    row 1: r10 = 6 -> 36, r11 = -2 -> 0; Z = 37; O = 360/37."""
    q = np.array([1.0, 2.0]).reshape(1, 1, 2, 1)
    k = np.array([3.0, -1.0]).reshape(1, 1, 2, 1)
    v = np.array([10.0, 20.0]).reshape(1, 1, 2, 1)
    o, z = orc.forward(q, k, v, 1.0, True, 1.0)
    np.testing.assert_allclose(o.ravel(), [9.0, 360.0 / 37.0])
    np.testing.assert_allclose(z.ravel(), [10.0, 37.0])
    # non-causal: row 0 also sees key 1: r01 = -1 -> 0; unchanged.  Row 1 unchanged.
    o2, _ = orc.forward(q, k, v, 1.0, False, 1.0)
    np.testing.assert_allclose(o2.ravel(), [9.0, 360.0 / 37.0])
    # negative scale flips which overlaps survive: row 1 keeps r11=-2 -> (2)^2 = 4
    o3, z3 = orc.forward(q, k, v, -1.0, True, 1.0)
    np.testing.assert_allclose(o3.ravel(), [0.0, 80.0 / 5.0])
    np.testing.assert_allclose(z3.ravel(), [1.0, 5.0])


def test_two_tokens_backward_by_hand():
    """Same D=1 case, dO = 1 everywhere, eps = 1, scale s = 1, causal.
    Row 1: p = (36, 0), Z = 37, O = 360/37, delta = O.
    dP_10 = (v_0 - O)/Z = (10 - 360/37)/37;  dS_10 = 2*6*dP_10
    dq_1 = s * dS_10 * k_0 = 3 dS_10; dk_0 gets s*dS_10*q_1 = 2 dS_10 from row 1
    dv_0 gets p/Z = 36/37 from row 1 and 9/10 from row 0.
    Row 0: dP_00 = (10 - 9)/10 = 0.1; dS_00 = 2*3*0.1 = 0.6; dq_0 = 0.6*3; dk_0 += 0.6*1."""
    q = np.array([1.0, 2.0]).reshape(1, 1, 2, 1)
    k = np.array([3.0, -1.0]).reshape(1, 1, 2, 1)
    v = np.array([10.0, 20.0]).reshape(1, 1, 2, 1)
    do = np.ones((1, 1, 2, 1))
    dq, dk, dv, ds = orc.backward(q, k, v, 1.0, do, True, 1.0)
    dS10 = 12.0 * (10.0 - 360.0 / 37.0) / 37.0
    np.testing.assert_allclose(dq.ravel(), [1.8, 3.0 * dS10])
    np.testing.assert_allclose(dk.ravel(), [0.6 + 2.0 * dS10, 0.0])
    np.testing.assert_allclose(dv.ravel(), [0.9 + 36.0 / 37.0, 0.0])
    # dscale = sum dS * r = 0.6*3 + dS10*6
    np.testing.assert_allclose(ds, [1.8 + 6.0 * dS10])


# --------------------------------------------------------------------------
# invariants
# --------------------------------------------------------------------------

def test_constant_values_give_scaled_constant():
    B, H, T, D = 2, 2, 30, 8
    q, k = _rand((B, H, T, D), seed=1, n=2)
    c = np.linspace(-1, 1, D)
    v = np.broadcast_to(c, (B, H, T, D)).copy()
    o, z = orc.forward(q, k, v, 1.7, True, 1e-3)
    np.testing.assert_allclose(o, c * ((z - 1e-3) / z)[..., None], rtol=1e-12, atol=1e-14)


def test_scale_invariance_and_weights():
    B, H, T, D = 1, 3, 25, 8
    q, k, v = _rand((B, H, T, D), seed=2)
    o1, _ = orc.forward(q, k, v, 1.0, True, 0.0)
    o2, _ = orc.forward(q, k, v, 37.0, True, 0.0)
    np.testing.assert_allclose(o1, o2, rtol=1e-10, atol=1e-12)
    w = orc.born_weights(q, k, 2.0, True, 1e-9)
    _, z = orc.forward(q, k, v, 2.0, True, 1e-9)
    np.testing.assert_allclose(w.sum(-1), (z - 1e-9) / z, rtol=1e-12)
    assert np.all(np.triu(w[0, 0], 1) == 0.0)  # causal upper triangle exactly zero
    assert np.all(w >= 0)


def test_window_special_cases():
    B, H, T, D = 2, 2, 21, 6
    q, k, v = _rand((B, H, T, D), seed=3)
    # window 1: only the diagonal survives
    o, z = orc.forward(q, k, v, 1.0, True, 0.0, window_size=1)
    r = (q * k).sum(-1)
    keep = (r > 0)[..., None]
    np.testing.assert_allclose(np.nan_to_num(o), np.where(keep, v, 0.0), rtol=1e-12, atol=1e-12)
    # window >= T is plain causal
    a, _ = orc.forward(q, k, v, 1.0, True, 1e-12, window_size=T)
    b, _ = orc.forward(q, k, v, 1.0, True, 1e-12)
    np.testing.assert_array_equal(a, b)


def test_document_special_cases():
    B, H, T, D = 2, 2, 19, 5
    q, k, v = _rand((B, H, T, D), seed=4)
    same = np.zeros((B, T), dtype=np.int32)
    a, _ = orc.forward(q, k, v, 1.0, True, 1e-12, doc_ids=same)
    b, _ = orc.forward(q, k, v, 1.0, True, 1e-12)
    np.testing.assert_array_equal(a, b)
    distinct = np.tile(np.arange(T, dtype=np.int32), (B, 1))
    a, _ = orc.forward(q, k, v, 1.0, False, 1e-12, doc_ids=distinct)
    b, _ = orc.forward(q, k, v, 1.0, True, 1e-12, window_size=1)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-15)


def test_weight_rounding_one_key_rows_by_hand():
    """forward(weight_dtype="f16") on one-key rows (window 1), r = q . k exact:
    the weight p = (s r)^2 enters O as fp16(p), so O_i = v_i fp16(p)/(p + eps).
    Chosen so fp16(p) is known exactly: 2^-22 and 2^-24 (subnormals, kept
    exactly), 2^-26 (below half the smallest subnormal: 0), 9 2^-28 (rounds up
    to 2^-24), 2^-10 (normal).  Z keeps the unrounded p."""
    s = 8.0
    p = np.array([2.0 ** -22, 2.0 ** -24, 2.0 ** -26, 9 * 2.0 ** -28, 2.0 ** -10])
    fp16p = np.array([2.0 ** -22, 2.0 ** -24, 0.0, 2.0 ** -24, 2.0 ** -10])
    r = np.sqrt(p) / s
    T = p.size
    q = np.zeros((1, 1, T, 4))
    k = np.zeros((1, 1, T, 4))
    q[..., 0] = r
    k[..., 0] = 1.0
    v = np.arange(1.0, 4 * T + 1).reshape(1, 1, T, 4)
    O, Z = orc.forward(q, k, v, s, True, 1e-12, 1, weight_dtype="f16")
    np.testing.assert_allclose(Z[0, 0], p + 1e-12, rtol=1e-14)
    np.testing.assert_allclose(O[0, 0], v[0, 0] * (fp16p / (p + 1e-12))[:, None], rtol=1e-12, atol=0)
    O_exact, _ = orc.forward(q, k, v, s, True, 1e-12, 1)
    np.testing.assert_allclose(O_exact[0, 0], v[0, 0] * (p / (p + 1e-12))[:, None], rtol=1e-12)


@pytest.mark.parametrize("wd,tdtype", [("f16", torch.float16), ("bf16", torch.bfloat16)])
def test_weight_rounding_matches_torch_kernel_arithmetic(wd, tdtype):
    """forward(weight_dtype=...) against torch evaluating the reference
    kernel's arithmetic op by op in fp32 (s = (q k^T) scale, a = relu(s) M,
    p = a a, z = sum p + eps, O = (p.to(dtype) @ v) / z; flash_born.py:166-186),
    on fp16-representable inputs with a wide spread of overlap magnitudes."""
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(1, 2, 48, 16, generator=g) * torch.logspace(-4, 0, 48).view(1, 1, 48, 1)).to(tdtype)
    k = torch.randn(1, 2, 48, 16, generator=g).to(tdtype)
    v = torch.randn(1, 2, 48, 16, generator=g).to(tdtype)
    scale = 6.0
    qf, kf, vf = q.float(), k.float(), v.float()
    for causal, window in ((True, 0), (True, 1), (False, 5)):
        mask = torch.from_numpy(orc.visible_mask(48, causal, window)).float()
        sc = (qf @ kf.transpose(-1, -2)) * scale
        a = sc.clamp_min(0) * mask
        pt = a * a
        zt = pt.sum(-1) + 1e-12
        ot = (pt.to(tdtype).float() @ vf) / zt[..., None]
        O, Z = orc.forward(qf.double().numpy(), kf.double().numpy(), vf.double().numpy(), scale, causal, 1e-12,
                           window, weight_dtype=wd)
        np.testing.assert_allclose(Z, zt.double().numpy(), rtol=1e-5)
        err = np.abs(O - ot.double().numpy()).max() / np.abs(ot.double().numpy()).max()
        assert err <= 2e-3, (causal, window, err)
        assert np.array_equal(O == 0, ot.double().numpy() == 0), "flushed rows differ"


def test_permutation_equivariance():
    B, H, T, D = 3, 4, 16, 8
    q, k, v = _rand((B, H, T, D), seed=5)
    sc = np.array([1.0, 2.0, 3.0, 4.0])
    o, _ = orc.forward(q, k, v, sc, True, 1e-12)
    pb, ph = np.array([2, 0, 1]), np.array([3, 1, 0, 2])
    o2, _ = orc.forward(q[pb][:, ph], k[pb][:, ph], v[pb][:, ph], sc[ph], True, 1e-12)
    np.testing.assert_allclose(o2, o[pb][:, ph], rtol=1e-13)


def test_all_negative_overlaps_give_zero():
    B, H, T, D = 1, 1, 12, 4
    q = np.abs(_rand((B, H, T, D), seed=6, n=1)[0]) + 0.1
    k = -np.abs(_rand((B, H, T, D), seed=7, n=1)[0]) - 0.1
    v = _rand((B, H, T, D), seed=8, n=1)[0]
    o, z = orc.forward(q, k, v, 3.0, False, 1e-12)
    assert np.all(o == 0.0) and np.all(z == 1e-12)
    dq, dk, dv, ds = orc.backward(q, k, v, 3.0, v, False, 1e-12)
    assert np.all(dq == 0) and np.all(dk == 0) and np.all(dv == 0) and np.all(ds == 0)


def test_visible_pairs_counts():
    T = 37
    for causal in (True, False):
        for W in (0, 1, 5, 100):
            m = orc.visible_mask(T, causal, W)
            assert orc.visible_pairs(2, T, causal, W) == 2 * int(m.sum())
    doc = orc.geometric_doc_ids(3, T, 6.0, seed=0)
    assert orc.visible_pairs(3, T, True, 0, doc) == int(orc.visible_mask(T, True, 0, doc).sum())


def test_geometric_doc_ids_properties():
    d = orc.geometric_doc_ids(4, 8192, 512.0, seed=0)
    assert d.shape == (4, 8192) and d.dtype == np.int32
    assert np.all(np.diff(d, axis=1) >= 0) and np.all(d[:, 0] == 0)
    lengths = np.concatenate([np.unique(r, return_counts=True)[1][:-1] for r in d])
    assert 300 < lengths.mean() < 800  # geometric with mean 512


# --------------------------------------------------------------------------
# backward: autograd of an independent torch statement, finite differences,
# and the closed form of dscale
# --------------------------------------------------------------------------

def _torch_forward(q, k, v, scale, causal, eps, window, doc):
    """Independent float64 torch statement of the forward (differentiable)."""
    T = q.shape[-2]
    s = scale.view(1, -1, 1, 1) if scale.dim() == 1 else scale
    r = torch.einsum("bhid,bhjd->bhij", q, k)
    a = torch.clamp(s * r, min=0.0)
    i = torch.arange(T).view(T, 1)
    j = torch.arange(T).view(1, T)
    keep = torch.ones(T, T, dtype=torch.bool)
    if causal:
        keep &= j <= i
    if window > 0:
        keep &= (i - j) < window
    keep = keep.view(1, 1, T, T)
    if doc is not None:
        dd = torch.as_tensor(doc)
        keep = keep & (dd.view(dd.shape[0], 1, T, 1) == dd.view(dd.shape[0], 1, 1, T))
    p = torch.where(keep, a * a, torch.zeros_like(a))
    return torch.einsum("bhij,bhjd->bhid", p, v) / (p.sum(-1, keepdim=True) + eps)


@pytest.mark.parametrize("case", CASES)
def test_backward_matches_autograd(case):
    B, H, T, D, scale, causal, window, doc_mean, eps = case
    q, k, v, do = _rand((B, H, T, D), seed=T + 2, n=4)
    doc = None if doc_mean is None else orc.geometric_doc_ids(B, T, doc_mean, seed=B)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    ts = torch.tensor(np.asarray(scale, dtype=np.float64), requires_grad=True)
    out = _torch_forward(tq, tk, tv, ts, causal, eps, window, doc)
    (out * torch.tensor(do)).sum().backward()
    dq, dk, dv, ds = orc.backward(q, k, v, np.asarray(scale), do, causal, eps, window, doc)
    np.testing.assert_allclose(dq, tq.grad.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(dk, tk.grad.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(dv, tv.grad.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(ds.reshape(ts.grad.shape), ts.grad.numpy(), rtol=1e-6, atol=1e-9)


def test_forward_statement_gradcheck():
    """Finite differences pin the differentiable torch statement used above."""
    q, k, v = (torch.tensor(x, requires_grad=True) for x in _rand((1, 2, 6, 3), seed=11))
    s = torch.tensor([1.3, 2.1], dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(
        lambda a, b, c, d: _torch_forward(a, b, c, d, True, 1e-3, 0, None), (q, k, v, s), eps=1e-6, atol=1e-6
    )


def test_dscale_closed_form():
    """dscale_h = (2/s_h) sum_{b,i} delta_i eps / Z_i (scale invariance)."""
    B, H, T, D = 2, 2, 24, 8
    q, k, v, do = _rand((B, H, T, D), seed=12, n=4)
    sc = np.array([1.5, -2.5])
    for eps in (1e-3, 1.0):
        o, z = orc.forward(q, k, v, sc, True, eps)
        delta = (do * o).sum(-1)
        want = (2.0 / sc) * (delta * eps / z).sum(axis=(0, 2))
        _, _, _, ds = orc.backward(q, k, v, sc, do, True, eps)
        np.testing.assert_allclose(ds, want, rtol=1e-9)


def test_backward_out_argument():
    """delta from a supplied forward output (the reference's stored O):
    identical to the default for the exact O; dv does not depend on it; the
    gradients are affine in it; a change in row i moves only row-i terms."""
    B, H, T, D = 1, 2, 20, 6
    q, k, v, do = _rand((B, H, T, D), seed=21, n=4)
    O, _ = orc.forward(q, k, v, 1.7, True, 1e-6)
    base = orc.backward(q, k, v, 1.7, do, True, 1e-6)
    same = orc.backward(q, k, v, 1.7, do, True, 1e-6, out=O)
    for x, y in zip(base, same):
        np.testing.assert_array_equal(x, y)
    rng = np.random.default_rng(0)
    dO_ = rng.standard_normal(O.shape) * 1e-3
    g1 = orc.backward(q, k, v, 1.7, do, True, 1e-6, out=O + dO_)
    g2 = orc.backward(q, k, v, 1.7, do, True, 1e-6, out=O + 2 * dO_)
    np.testing.assert_array_equal(g1[2], base[2])
    for x0, x1, x2 in zip(base, g1, g2):
        np.testing.assert_allclose(x2 - x0, 2 * (x1 - x0), rtol=1e-6, atol=1e-12)
    row = np.zeros_like(O)
    row[0, 1, 7] = 1e-3
    g3 = orc.backward(q, k, v, 1.7, do, True, 1e-6, out=O + row)
    changed = np.abs(g3[0] - base[0]).sum(-1) > 0  # dq rows
    assert changed[0, 1, 7] and changed.sum() == 1
    # dk of key j moves only where query 7 sees it (causal: j <= 7)
    moved = np.abs(g3[1] - base[1]).sum(-1)[0, 1] > 0
    assert not moved[8:].any()


def test_backward_magnitudes_bound_and_dv():
    B, H, T, D = 2, 2, 24, 8
    q, k, v, do = _rand((B, H, T, D), seed=22, n=4)
    for kw in ({}, {"is_causal": False}, {"window_size": 5}):
        g = orc.backward(q, k, v, 2.0, do, eps=1e-6, **kw)
        m = orc.backward_magnitudes(q, k, v, 2.0, do, eps=1e-6, **kw)
        for gi, mi in zip(g[:3], m):
            assert np.all(np.abs(gi) <= mi * (1 + 1e-12) + 1e-300)
    dpos = np.abs(do)
    g = orc.backward(q, k, v, 2.0, dpos, eps=1e-6)
    m = orc.backward_magnitudes(q, k, v, 2.0, dpos, eps=1e-6)
    np.testing.assert_allclose(m[2], np.abs(g[2]), rtol=1e-12)


def test_eager_fp32_restatement_matches():
    B, H, T, D = 2, 3, 40, 16
    q, k, v = (torch.tensor(x, dtype=torch.float32) for x in _rand((B, H, T, D), seed=13))
    doc = orc.geometric_doc_ids(B, T, 7.0, seed=1)
    for kw in ({}, {"is_causal": False}, {"window_size": 6}, {"doc_ids": torch.as_tensor(doc)}):
        out = orc.eager_fp32_torch(q, k, v, torch.tensor([1.0, 2.0, 3.0]), **kw)
        kw2 = dict(kw)
        if "doc_ids" in kw2:
            kw2["doc_ids"] = doc
        ref, _ = orc.forward(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                             np.array([1.0, 2.0, 3.0]), **kw2)
        assert np.abs(out.numpy() - ref).max() / np.abs(ref).max() < 1e-5


# --------------------------------------------------------------------------
# planted mistakes: each must be caught by the pins above
# --------------------------------------------------------------------------

def _mutant_forward(kind):
    def f(q, k, v, scale, is_causal=True, eps=1e-12, window_size=0, doc_ids=None):
        q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
        B, H, T, D = q.shape
        s = np.asarray(scale, np.float64).reshape(-1)
        s = s.reshape(1, -1, 1, 1) if s.size > 1 else s.reshape(1, 1, 1, 1)
        r = q @ np.swapaxes(k, -1, -2)
        if kind == "transposed":
            r = np.swapaxes(r, -1, -2)
        a = s * r if kind == "no_relu" else np.maximum(s * r, 0.0)
        m = orc.visible_mask(T, is_causal, window_size, doc_ids)
        if kind == "mask_flipped":
            m = orc.visible_mask(T, False, 0, None) & ~m if is_causal else m
        if kind == "window_off_by_one" and window_size > 0:
            i = np.arange(T)[:, None]
            j = np.arange(T)[None, :]
            m = m | ((i - j) == window_size)[None, None] & ((j <= i) if is_causal else True)
        a = a * m
        p = a * a if kind != "no_square" else a
        Z = p.sum(-1) + (0.0 if kind == "drop_eps" else eps)
        return (p @ v) / Z[..., None], Z

    return f


@pytest.mark.parametrize("kind", ["transposed", "no_relu", "mask_flipped", "window_off_by_one", "no_square", "drop_eps"])
def test_planted_mistakes_are_caught(clib, kind):
    f = _mutant_forward(kind)
    caught = False
    for case in CASES:
        B, H, T, D, scale, causal, window, doc_mean, eps = case
        q, k, v = _rand((B, H, T, D), seed=T)
        doc = None if doc_mean is None else orc.geometric_doc_ids(B, T, doc_mean, seed=B)
        with np.errstate(all="ignore"):
            o_m, z_m = f(q, k, v, np.asarray(scale), causal, eps, window, doc)
        o_c, z_c = c_forward(clib, q, k, v, scale, causal, eps, window, doc)
        if not (np.allclose(o_m, o_c, rtol=1e-12, atol=1e-12) and np.allclose(z_m, z_c, rtol=1e-12, atol=1e-15)):
            caught = True
            break
    assert caught, f"planted mistake {kind!r} was not caught by the brute-force pin"


# --------------------------------------------------------------------------
# purified-Born attention (flash_born.py:693-1341)
# --------------------------------------------------------------------------

def _pur_inputs(seed, B=2, H=3, T=7, D=4, scale=1.0):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((B, H, T, D)) * scale for _ in range(4)]


def test_purified_zero_gamma_is_born():
    # g = 0 leaves eps_base relu(r)^2: Born with scale 1 and eps / eps_base.
    q, k, v, _ = _pur_inputs(1)
    docs = np.array([[0, 0, 0, 1, 1, 2, 2], [0, 1, 1, 1, 1, 1, 2]])
    for causal, window, doc in [(True, 0, None), (False, 3, None), (True, 2, docs)]:
        O, Z = orc.purified_forward(q, k, v, 0.0, [0.3, -0.2, 0.0], 0.05, causal, 1e-6, window, doc)
        Ob, Zb = orc.forward(q, k, v, 1.0, causal, 1e-6 / 0.05, window, doc)
        np.testing.assert_allclose(O, Ob, rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(Z, 0.05 * Zb, rtol=1e-12, atol=1e-15)


def test_purified_gamma_invariance_without_base():
    # eps_base = 0, tau = 0: p = g^4 relu(r)^4, so O does not depend on g > 0.
    q, k, v, _ = _pur_inputs(2)
    O1, Z1 = orc.purified_forward(q, k, v, 2.0, 0.0, 0.0, True, 0.0)
    O2, Z2 = orc.purified_forward(q, k, v, 7.0, 0.0, 0.0, True, 0.0)
    ok = Z1 > 0
    np.testing.assert_allclose(O1[ok], O2[ok], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(Z2[ok], Z1[ok] * (7.0 / 2.0) ** 4, rtol=1e-12)


def test_purified_brute_force_loops():
    B, H, T, D = 1, 2, 5, 3
    q, k, v, _ = _pur_inputs(3, B, H, T, D)
    docs = np.array([[0, 0, 1, 1, 1]])
    g, tau, eb, eps, W = [1.5, -2.0], [0.1, -0.4], 0.3, 1e-3, 3
    O, Z = orc.purified_forward(q, k, v, g, tau, eb, True, eps, W, docs)
    for h in range(H):
        for i in range(T):
            num, den = np.zeros(D), 0.0
            for j in range(T):
                if not (j <= i and i - j < W and docs[0, i] == docs[0, j]):
                    continue
                r = sum(q[0, h, i, d] * k[0, h, j, d] for d in range(D))
                u = max(0.0, g[h] * (r - tau[h]))
                p = u ** 4 + eb * max(0.0, r) ** 2
                num += p * v[0, h, j]
                den += p
            den += eps
            assert abs(Z[0, h, i] - den) <= 1e-12 * max(1.0, den)
            np.testing.assert_allclose(O[0, h, i], num / den, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("case", [
    dict(causal=True, window=0, doc=False, per_head=False),
    dict(causal=False, window=3, doc=False, per_head=True),
    dict(causal=True, window=0, doc=True, per_head=True),
])
def test_purified_backward_matches_autograd(case):
    B, H, T, D = 2, 3, 6, 4
    q, k, v, do = _pur_inputs(4, B, H, T, D, 0.8)
    docs = np.array([[0, 0, 0, 1, 1, 1], [0, 1, 1, 2, 2, 2]]) if case["doc"] else None
    g = np.array([2.0, 1.5, 3.0]) if case["per_head"] else np.array([2.5])
    tau = np.array([0.1, -0.2, 0.05]) if case["per_head"] else np.array([0.0625])
    eb, eps = 0.05, 1e-8
    ref = orc.purified_backward(q, k, v, g, tau, do, eb, case["causal"], eps, case["window"], docs)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    tg = torch.tensor(g if case["per_head"] else g[0], requires_grad=True)
    tt = torch.tensor(tau if case["per_head"] else tau[0], requires_grad=True)
    tdoc = None if docs is None else torch.tensor(docs)
    out = orc.purified_eager_fp32_torch(tq, tk, tv, tg, tt, eb, case["causal"], eps, case["window"], tdoc)
    (out * torch.tensor(do)).sum().backward()
    for got, want in zip(ref[:3], (tq.grad, tk.grad, tv.grad)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(ref[3], np.atleast_1d(tg.grad.numpy()), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(ref[4], np.atleast_1d(tt.grad.numpy()), rtol=1e-9, atol=1e-10)


def test_purified_statement_gradcheck():
    # Finite differences pin the torch statement the backward is compared with.
    B, H, T, D = 1, 2, 4, 3
    q, k, v, _ = _pur_inputs(5, B, H, T, D, 0.9)
    args = [torch.tensor(x, requires_grad=True) for x in (q, k, v)]
    g = torch.tensor([1.7, 2.2], dtype=torch.float64, requires_grad=True)
    t = torch.tensor([0.05, -0.1], dtype=torch.float64, requires_grad=True)
    f = lambda q_, k_, v_, g_, t_: orc.purified_eager_fp32_torch(q_, k_, v_, g_, t_, 0.2, True, 1e-6)
    assert torch.autograd.gradcheck(f, (*args, g, t), eps=1e-6, atol=1e-5, rtol=1e-4)


def test_purified_backward_out_argument_and_magnitudes():
    q, k, v, do = _pur_inputs(6)
    O, _ = orc.purified_forward(q, k, v, 3.0, 0.1, 0.05, True, 1e-8)
    base = orc.purified_backward(q, k, v, 3.0, 0.1, do, 0.05, True, 1e-8)
    same = orc.purified_backward(q, k, v, 3.0, 0.1, do, 0.05, True, 1e-8, out=O)
    for a, b in zip(base, same):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-14)
    # a perturbed output changes delta and so dv stays, dq moves
    moved = orc.purified_backward(q, k, v, 3.0, 0.1, do, 0.05, True, 1e-8, out=O * 1.01)
    np.testing.assert_allclose(moved[2], base[2], rtol=1e-12)
    assert np.abs(moved[0] - base[0]).max() > 1e-6
    mags = orc.purified_backward_magnitudes(q, k, v, 3.0, 0.1, do, 0.05, True, 1e-8)
    for g_, m in zip(base, mags):
        assert np.all(np.abs(g_) <= m * (1 + 1e-12) + 1e-15)
