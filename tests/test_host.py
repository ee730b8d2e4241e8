"""Host-side logic of the drop-in module (no GPU needed)."""

from __future__ import annotations

import inspect
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_public_signature_matches_reference():
    """flash_born_attention(q, k, v, scale, is_causal=True, eps=1e-12,
    window_size=0, doc_ids=None) (reference flash_born.py:655-664)."""
    from quantumdlblocks_amd import flash_born_attention

    params = inspect.signature(flash_born_attention).parameters
    assert list(params) == ["q", "k", "v", "scale", "is_causal", "eps", "window_size", "doc_ids"]
    assert params["scale"].default is inspect.Parameter.empty
    assert params["is_causal"].default is True
    assert params["eps"].default == 1e-12
    assert params["window_size"].default == 0
    assert params["doc_ids"].default is None


def test_import_paths_expose_the_same_objects():
    import quantumdlblocks_amd as pkg
    from quantumdlblocks_amd import kernels
    from quantumdlblocks_amd.kernels import flash_born, flash_born_triton

    for name in ("flash_born_attention", "get_flash_born_launch_meta", "get_rdna4_autotune_configs",
                 "HAS_TRITON", "IS_HIP"):
        objs = {id(getattr(m, name)) for m in (pkg, kernels, flash_born, flash_born_triton)}
        assert len(objs) == 1, name
    assert flash_born_triton._run_triton_flash_born is flash_born._run_triton_flash_born
    assert pkg.IS_HIP == (torch.version.hip is not None)


def test_launch_meta_literals():
    """Literal assertions of the reference's tests: test_flash_born.py:70-83 and
    test_plan049...:309-318."""
    from quantumdlblocks_amd.kernels import get_flash_born_launch_meta, get_rdna4_autotune_configs

    hip_meta = get_flash_born_launch_meta(64, is_hip=True)
    assert hip_meta["num_warps"] == 4 and hip_meta["waves_per_eu"] == 2
    cuda_meta = get_flash_born_launch_meta(64, is_hip=False)
    assert cuda_meta["num_warps"] == 4 and "waves_per_eu" not in cuda_meta
    cfgs = get_rdna4_autotune_configs()
    assert len(cfgs) == 4
    assert all(c["matrix_instr_nonkdim"] == 16 and c["waves_per_eu"] in (2, 4) for c in cfgs)
    meta = get_flash_born_launch_meta(512, head_dim=64)
    assert meta["BLOCK_M"] == 64 and meta["BLOCK_N"] == 64
    for hd in (48, 80, 96, 112):
        assert get_flash_born_launch_meta(512, head_dim=hd)["BLOCK_M"] in (32, 64)


@pytest.mark.parametrize(
    "seq_len,head_dim,hip,expect",
    [
        (64, 64, True, {"BLOCK_M": 64, "BLOCK_N": 64, "num_warps": 4, "num_stages": 1, "waves_per_eu": 2,
                        "matrix_instr_nonkdim": 16}),
        (40, 64, False, {"BLOCK_M": 32, "BLOCK_N": 32, "num_warps": 4, "num_stages": 2}),
        (8, 32, False, {"BLOCK_M": 16, "BLOCK_N": 16, "num_warps": 4, "num_stages": 2}),
        (512, 128, False, {"BLOCK_M": 32, "BLOCK_N": 32, "num_warps": 4, "num_stages": 1}),
        (20, 96, True, {"BLOCK_M": 16, "BLOCK_N": 16, "num_warps": 4, "num_stages": 1, "waves_per_eu": 2,
                        "matrix_instr_nonkdim": 16}),
        (4096, 256, False, {"BLOCK_M": 16, "BLOCK_N": 16, "num_warps": 4, "num_stages": 1}),
        (4096, 200, True, {"BLOCK_M": 16, "BLOCK_N": 16, "num_warps": 4, "num_stages": 1, "waves_per_eu": 2,
                           "matrix_instr_nonkdim": 16}),
    ],
)
def test_launch_meta_table(seq_len, head_dim, hip, expect):
    """The reference's tile table (flash_born.py:37-65): edge by padded head dim
    and sequence length; HIP adds waves_per_eu / matrix_instr_nonkdim."""
    from quantumdlblocks_amd.kernels import get_flash_born_launch_meta

    assert get_flash_born_launch_meta(seq_len, is_hip=hip, head_dim=head_dim) == expect


def test_compute_document_ids_literal_golden():
    from quantumdlblocks_amd import compute_document_ids

    idx = torch.tensor([[10, 20, 50256, 30, 40, 50256, 50, 60], [11, 50256, 22, 33, 44, 55, 66, 77]])
    got = compute_document_ids(idx, eot_token_id=50256)
    assert got.dtype == torch.int32
    assert torch.equal(got, torch.tensor([[0, 0, 0, 1, 1, 1, 2, 2], [0, 0, 1, 1, 1, 1, 1, 1]], dtype=torch.int32))


def test_l2_normalize():
    from quantumdlblocks_amd import l2_normalize

    x = torch.randn(3, 5, 16, dtype=torch.float64)
    y = l2_normalize(x)
    torch.testing.assert_close(y.norm(dim=-1), torch.ones(3, 5, dtype=torch.float64))
    assert l2_normalize(x.bfloat16()).dtype == torch.bfloat16


def _cpu_inputs(B=2, H=3, T=20, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, T, D, generator=g) for _ in range(3)]


@pytest.mark.parametrize("kw", [{}, {"is_causal": False}, {"window_size": 5}, {"window_size": 3, "is_causal": False}])
def test_cpu_tensors_use_reference_eager_semantics(kw):
    from quantumdlblocks_amd import flash_born_attention

    q, k, v = _cpu_inputs()
    for scale in (2.0, torch.tensor(2.0), torch.tensor([1.0, 2.0, 3.0]), torch.tensor([1.0, 2.0, 3.0]).view(1, 3, 1, 1)):
        out = flash_born_attention(q, k, v, scale, **kw)
        ref, _ = orc.forward(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                             np.asarray(scale).reshape(-1), kw.get("is_causal", True), 1e-12,
                             kw.get("window_size", 0))
        assert np.abs(out.double().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


def test_reference_window_and_document_case_on_cpu():
    """The reference's CPU assertions (test_hypothesis_016:179-205): rows of the
    weights sum to 1, exact zeros outside the mask, out == weights @ v."""
    from quantumdlblocks_amd import compute_document_ids, flash_born_attention, l2_normalize

    idx = torch.tensor([[10, 20, 50256, 30, 40, 50256, 50, 60], [11, 50256, 22, 33, 44, 55, 66, 77]])
    doc = compute_document_ids(idx)
    torch.manual_seed(2)
    q = l2_normalize(torch.randn(2, 4, 8, 16), dim=-1)
    k = l2_normalize(0.85 * q + 0.15 * torch.randn(2, 4, 8, 16), dim=-1)
    v = l2_normalize(torch.randn(2, 4, 8, 16), dim=-1)
    w = torch.as_tensor(orc.born_weights(q, k, 10.0, True, 1e-8, 4, doc.numpy()))
    rows = w.sum(-1)
    assert torch.allclose(rows, torch.ones_like(rows), atol=1e-5)
    for b in range(2):
        for i in range(8):
            for j in range(8):
                if j > i or i - j >= 4 or doc[b, i] != doc[b, j]:
                    assert torch.all(w[b, :, i, j] == 0.0)
    out = flash_born_attention(q, k, v, scale=10.0, window_size=4, doc_ids=doc)
    assert torch.allclose(out.double(), torch.matmul(w, v.double()), atol=1e-4)


def test_input_validation():
    from quantumdlblocks_amd.kernels.flash_born import _check_inputs

    q = torch.zeros(2, 3, 10, 16)
    one = torch.ones(1)
    with pytest.raises(ValueError):
        _check_inputs(q, torch.zeros(2, 3, 11, 16), q, one, None)
    with pytest.raises(ValueError):
        _check_inputs(q, q, q, torch.ones(2), None)
    with pytest.raises(ValueError):
        _check_inputs(q, q, q, one, torch.zeros(2, 9, dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        big = torch.zeros(1, 1, 2, 264)
        _check_inputs(big, big, big, one, None)
    _check_inputs(q, q, q, torch.ones(3), torch.zeros(2, 10, dtype=torch.int32))


def test_head_dims_above_256_take_the_eager_path(monkeypatch):
    """The reference runs its eager formulation whenever its kernel cannot
    take the head dim (flash_born.py:670-690); so does the drop-in for GPU
    tensors with D > 256, while D <= 256 goes to the HIP kernels."""
    from quantumdlblocks_amd.kernels import flash_born as fb

    class _CudaLike(torch.Tensor):
        is_cuda = True  # routing only looks at is_cuda and the head dim

    calls = []
    monkeypatch.setattr(fb, "_run_triton_flash_born", lambda *a, **kw: calls.append("hip"))
    monkeypatch.setattr(fb, "_eager_born", lambda *a, **kw: calls.append("eager"))
    monkeypatch.setattr(fb, "_run_triton_flash_purified_born", lambda *a, **kw: calls.append("hip"))
    monkeypatch.setattr(fb, "_eager_purified_born", lambda *a, **kw: calls.append("eager"))
    for D, want in ((256, "hip"), (272, "eager"), (320, "eager"), (8, "hip")):
        x = torch.Tensor._make_subclass(_CudaLike, torch.zeros(1, 2, 4, D))
        assert x.is_cuda
        calls.clear()
        fb.flash_born_attention(x, x, x, 2.0)
        fb.flash_purified_born_attention(x, x, x)
        assert calls == [want, want], (D, calls)
    calls.clear()
    y = torch.zeros(1, 2, 4, 64)  # CPU tensors: eager
    fb.flash_born_attention(y, y, y, 2.0)
    assert calls == ["eager"]


def test_missing_library_fails_loudly():
    """With the library absent, loading raises and HAS_TRITON is False; the GPU
    path has no silent fallback."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "from quantumdlblocks_amd import _native\n"
        "import quantumdlblocks_amd as q\n"
        "assert q.HAS_TRITON is False and q.HAS_HIP_KERNELS is False\n"
        "try:\n    _native.load()\nexcept _native.NativeLibraryError as e:\n    print('raised', e)\n"
        "else:\n    raise SystemExit('no error')\n" % ROOT
    )
    env = dict(os.environ, QDL_FLASH_BORN_LIB="/nonexistent/libqdl_flash_born.so")
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    assert "raised" in res.stdout


def test_mi355x_launch_meta():
    from quantumdlblocks_amd import get_mi355x_launch_meta

    m = get_mi355x_launch_meta(64, torch.bfloat16)
    assert m["BLOCK_M"] == 256 and m["BLOCK_N"] == 64 and m["padded_head_dim"] == 64
    assert get_mi355x_launch_meta(200, torch.float16)["padded_head_dim"] == 224
    assert get_mi355x_launch_meta(64, torch.float32)["mfma"] == "32x32x2f32"


def test_integration_install_rebinds_reference_names():
    """quantumdlblocks_amd.integration.install() rebinds the names the
    reference's layers bind at import (attention.py:20) and registers the
    documented module path qdlblocks.kernels.flash_born_triton."""
    import sys
    import types

    from quantumdlblocks_amd import flash_born_attention, integration
    from quantumdlblocks_amd.kernels import flash_born_triton

    names = ["qdlblocks", "qdlblocks.kernels", "qdlblocks.kernels.flash_born", "qdlblocks.layers",
             "qdlblocks.layers.attention", "qdlblocks.kernels.flash_born_triton"]
    saved = {n: sys.modules.get(n) for n in names}
    try:
        fake = {n: types.ModuleType(n) for n in names[:-1]}
        sentinel = object()
        for n in ("qdlblocks", "qdlblocks.kernels", "qdlblocks.layers.attention"):
            fake[n].flash_born_attention = sentinel
        fake["qdlblocks.kernels"].HAS_TRITON = False
        sys.modules.update(fake)
        patched = integration.install(import_targets=False)
        assert set(patched) == {"qdlblocks", "qdlblocks.kernels", "qdlblocks.kernels.flash_born",
                                "qdlblocks.layers.attention"}
        for n in ("qdlblocks", "qdlblocks.kernels", "qdlblocks.layers.attention", "qdlblocks.kernels.flash_born"):
            assert sys.modules[n].flash_born_attention is flash_born_attention
        assert sys.modules["qdlblocks.kernels"].HAS_TRITON is flash_born_triton.HAS_TRITON
        assert sys.modules["qdlblocks.kernels.flash_born_triton"] is flash_born_triton
        assert sys.modules["qdlblocks.kernels"].flash_born_triton is flash_born_triton
        assert not hasattr(sys.modules["qdlblocks.layers.attention"], "get_rdna4_autotune_configs")
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m


def test_prologue_cpu_tensors_take_the_eager_formulation():
    """On CPU tensors the fused prologue is the reference's eager
    apply_unitary_rope + l2_normalize; it agrees with the oracle's rounding
    model (rows within one bf16 ulp: only the norm's summation order differs)."""
    import numpy as np

    from oracle import qk_prologue_oracle as po
    from quantumdlblocks_amd.kernels.qk_prologue import fused_qk_rope_l2_normalize

    g = torch.Generator().manual_seed(3)
    B, H, T, D, n = 2, 3, 20, 64, 24
    q = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    ang = torch.outer(torch.arange(T, dtype=torch.float32), 0.1 * torch.arange(1, n + 1).float())
    cos, sin = torch.cos(ang).view(1, 1, T, n), torch.sin(ang).view(1, 1, T, n)
    qo, ko = fused_qk_rope_l2_normalize(q, k, cos, sin, eps=1e-12)
    for x, o in ((q, qo), (k, ko)):
        want, _ = po.prologue_forward(x.float().numpy(), cos[0, 0].numpy(), sin[0, 0].numpy(),
                                      1e-12, "bf16")
        got = o.float().numpy()
        assert o.dtype == torch.bfloat16
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30)
    with pytest.raises(ValueError):
        fused_qk_rope_l2_normalize(q, k[:, :2])


def test_prologue_gradient_layout_rule():
    """Input gradients keep the input's strides only for dense layouts."""
    from quantumdlblocks_amd.kernels.qk_prologue import _dense_layout

    x = torch.empty(2, 8, 4, 16)  # (B, T, H, D)
    v = x.transpose(1, 2)  # (B, H, T, D) view of the projection layout
    assert _dense_layout(tuple(v.shape), v.stride())
    assert _dense_layout((2, 4, 8, 16), torch.empty(2, 4, 8, 16).stride())
    qkv = torch.empty(2, 8, 3 * 4 * 16)
    q = qkv[..., : 4 * 16].view(2, 8, 4, 16).transpose(1, 2)  # gaps between rows
    assert not _dense_layout(tuple(q.shape), q.stride())
    e = torch.empty(1, 4, 8, 16).expand(2, 4, 8, 16)  # stride 0: overlapping
    assert not _dense_layout(tuple(e.shape), e.stride())
    assert _dense_layout((1, 4, 8, 16), (999, 128, 16, 1))  # size-1 dims are free
