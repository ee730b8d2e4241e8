"""qdl_flash_born_bwd_noalloc (the backward that takes its workspace from a
fixed device array in the library) against qdl_flash_born_bwd with a caller
workspace, through the C ABI: bit-identical gradients and dscale, on two calls
in a row with the second one smaller (the array keeps the first call's
contents), and on the C5 shape.  Also: a problem too large for the array is
rejected before any HIP call."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from util import seeded_inputs


def _lib():
    from quantumdlblocks_amd import _native

    return _native.load()


def test_noalloc_rejects_problems_beyond_the_array():
    from quantumdlblocks_amd import _native

    lib = _lib()
    B, H, T, D = 16, 16, 8192, 64  # 25 MB of workspace > 16 MiB
    assert lib.qdl_flash_born_bwd_workspace_size(2, B, H, T, D, 1) > _native.BWD_SCRATCH_BYTES
    rc = lib.qdl_flash_born_bwd_noalloc(2, B, H, T, D, *([None] * 7), 1, None, 1, 0, 1e-12,
                                        None, None, None, None, None)
    assert rc == -12
    assert "16 MiB" in lib.qdl_flash_born_strerror(rc).decode()


def _run_pair(dev, B, H, T, D, dtype, *, causal=True, window=0, doc=None, scale=(8.0,), seed=0):
    from quantumdlblocks_amd import _native
    from quantumdlblocks_amd.kernels.flash_born import _DTYPE_CODE

    lib = _lib()
    code = _DTYPE_CODE[dtype]
    # fp16: N(0, 0.25), inside the range where the forward's fp16 weights
    # (s q.k)^2 do not overflow at scale 8 (they are the reference's own).
    std = 0.5 if dtype == torch.float16 else 1.0
    q, k, v, do = (x.to(dev, dtype).contiguous()
                   for x in seeded_inputs((B, H, T, D), seed=seed, std=std, n=4))
    sc = torch.tensor(scale, dtype=torch.float32, device=dev)
    out = torch.empty_like(q)
    z = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    doc_t = None if doc is None else torch.as_tensor(doc, dtype=torch.int32, device=dev)
    doc_p = None if doc_t is None else doc_t.data_ptr()
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.qdl_flash_born_fwd(code, B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                z.data_ptr(), sc.data_ptr(), sc.numel(), doc_p, int(causal), window, 1e-3, stream)
    _native.check(rc, "qdl_flash_born_fwd")
    res = []
    for noalloc in (False, True):
        dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(3))
        ds = torch.full((sc.numel(),), float("nan"), dtype=torch.float32, device=dev)
        args = [code, B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), do.data_ptr(),
                z.data_ptr(), sc.data_ptr(), sc.numel(), doc_p, int(causal), window, 1e-3,
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ds.data_ptr()]
        if noalloc:
            rc = lib.qdl_flash_born_bwd_noalloc(*args, stream)
        else:
            nbytes = int(lib.qdl_flash_born_bwd_workspace_size(code, B, H, T, D, sc.numel()))
            ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
            rc = lib.qdl_flash_born_bwd(*args, ws.data_ptr(), ws.numel(), stream)
        _native.check(rc, "qdl_flash_born_bwd" + ("_noalloc" if noalloc else ""))
        torch.cuda.synchronize(dev)
        res.append((dq, dk, dv, ds))
    iv = torch.int32 if dtype == torch.float32 else torch.int16
    for a, b in zip(res[0][:3], res[1][:3]):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a.view(iv), b.view(iv))
    assert torch.equal(res[0][3].view(torch.int32), res[1][3].view(torch.int32))


@pytest.mark.gpu
def test_noalloc_matches_caller_workspace_twice_smaller_second(cuda_device):
    # First call larger (fills more of the array), second smaller: the second
    # must not pick up anything the first left behind.
    _run_pair(cuda_device, 4, 8, 1000, 64, torch.bfloat16, scale=(8.0,), seed=1)
    _run_pair(cuda_device, 2, 4, 300, 64, torch.bfloat16, scale=(1.0, 2.0, -3.0, 4.0), seed=2)


@pytest.mark.gpu
def test_noalloc_generic_kernels_and_documents(cuda_device):
    doc = np.repeat(np.arange(10, dtype=np.int32), 50)[None].repeat(2, 0)
    _run_pair(cuda_device, 2, 3, 500, 96, torch.float16, doc=doc, seed=3)
    _run_pair(cuda_device, 1, 2, 200, 32, torch.float32, window=37, seed=4)


@pytest.mark.gpu
def test_noalloc_c5_shape(cuda_device):
    _run_pair(cuda_device, 16, 16, 2048, 64, torch.bfloat16, seed=5)


@pytest.mark.gpu
def test_noalloc_d128_kernels(cuda_device):
    # The D = 128 kernels: causal, with document ids, and a padded head dim.
    _run_pair(cuda_device, 2, 4, 1100, 128, torch.bfloat16, seed=6)
    doc = np.repeat(np.arange(11, dtype=np.int32), 100)[None].repeat(2, 0)
    _run_pair(cuda_device, 2, 2, 1100, 128, torch.bfloat16, doc=doc, seed=7)
    _run_pair(cuda_device, 1, 3, 700, 96, torch.float16, scale=(0.5, -1.0, 2.0), seed=8)
