"""The flash-Born path inside the Born attention layer's data flow.

Restates, for the test only, the default path of
``SubspaceProjectorBornAttention.forward`` (src/qdlblocks/layers/attention.py:
509-518 projections, 573-589 Q/K prologue, 691-715 flash call, 478-493 head
merge and output projection; the purified branch at 628-656) with random
weights, and runs it two ways:

  * the MI355X path: projections under bf16 autocast, the (B, T, H, D)
    projection outputs passed strided to ``fused_qk_rope_l2_normalize``, then
    ``flash_born_attention`` / ``flash_purified_born_attention`` with document
    ids computed on the device by ``compute_document_ids``;
  * the layer's eager formulation (attention.py:730-760) under the same bf16
    autocast: contiguous heads, ``apply_unitary_rope``, ``l2_normalize``, then
    the dense weights, masks and normalisation in fp32 from the bf16 Q, K, V.

Output and the gradients of the input and of every projection weight must
agree at the reference's bf16 bar (normwise relative error 2e-2; 3e-2 for
gradients, the bar of tests/test_plan041_15gb_batch24576_dyadic_scaling.py).
"""

from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double()
    b = b.detach().double()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _rope_tables(T, D, device):
    # UnitaryRoPE tables (isometric.py:105-126), base 10000, all frequencies.
    half = D // 2
    freqs = 1.0 / (10000.0 ** (torch.arange(0, half, dtype=torch.float32) / half))
    ang = torch.outer(torch.arange(T, dtype=torch.float32), freqs)
    return torch.cos(ang).view(1, 1, T, half).to(device), torch.sin(ang).view(1, 1, T, half).to(device)


def _weights(E, device, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    ws = []
    for _ in range(4):
        w = torch.empty(E, E)
        torch.nn.init.orthogonal_(w, generator=g)
        ws.append(w.to(device).requires_grad_(True))
    return ws


def _tokens(B, T, device, seed, eot=50256, p_eot=0.01):
    g = torch.Generator("cpu").manual_seed(seed)
    idx = torch.randint(0, 50000, (B, T), generator=g)
    idx[torch.rand(B, T, generator=g) < p_eot] = eot
    return idx.to(device)


def _eager_weights(Q, K, scale, purified, tau, eps_base, eps, doc):
    """The layer's dense weights in fp32: Born (attention.py:730-756) or
    purified (flash_born.py:1329-1341 with tau and gamma)."""
    T = Q.shape[-2]
    s = torch.matmul(Q, K.transpose(-1, -2))
    if purified:
        u = torch.relu(scale * (s - tau))
        prob = u.square().square() + eps_base * torch.relu(s).square()
    else:
        prob = torch.relu(s * scale).square()
    idx = torch.arange(T, device=Q.device)
    mask = (idx[:, None] - idx[None, :]) >= 0
    mask = mask.view(1, 1, T, T)
    if doc is not None:
        mask = mask & (doc[:, None, :, None] == doc[:, None, None, :])
    prob = prob * mask.to(prob.dtype)
    return prob / (prob.sum(dim=-1, keepdim=True) + eps)


@pytest.mark.parametrize("purified", [False, True], ids=["born", "purified"])
@pytest.mark.parametrize("with_docs", [False, True], ids=["causal", "documents"])
def test_layer_path_matches_eager(cuda_device, purified, with_docs):
    from quantumdlblocks_amd import (
        apply_unitary_rope,
        compute_document_ids,
        flash_born_attention,
        flash_purified_born_attention,
        fused_qk_rope_l2_normalize,
        l2_normalize,
    )

    B, T, H, D = 2, 384, 4, 64
    E = H * D
    eps = 1e-12 if not purified else 1e-8
    scale = math.sqrt(D) if not purified else 8.0
    tau, eps_base = 0.0625, 0.05
    print(f"layer case purified={purified} docs={with_docs} B{B} T{T} H{H} D{D}", flush=True)
    g = torch.Generator("cpu").manual_seed(7)
    x = torch.randn(B, T, E, generator=g).to(cuda_device)
    gout = torch.randn(B, T, E, generator=g).to(cuda_device)
    cos, sin = _rope_tables(T, D, cuda_device)
    doc = compute_document_ids(_tokens(B, T, cuda_device, 11, p_eot=0.02)) if with_docs else None
    assert doc is None or (doc.is_cuda and doc.dtype == torch.int32)

    def mi355x_path(x, ws):
        wq, wk, wv, wo = ws
        with torch.autocast("cuda", dtype=torch.bfloat16):
            psi = l2_normalize(x, dim=-1, eps=1e-12)
            Q = torch.nn.functional.linear(psi, wq).view(B, T, H, D).transpose(1, 2)
            K = torch.nn.functional.linear(psi, wk).view(B, T, H, D).transpose(1, 2)
            V = torch.nn.functional.linear(psi, wv).view(B, T, H, D).transpose(1, 2).contiguous()
            assert not Q.is_contiguous() and Q.dtype == torch.bfloat16
            Q, K = fused_qk_rope_l2_normalize(Q, K, cos, sin, eps=1e-12)
            if purified:
                heads = flash_purified_born_attention(Q, K, V, scale=scale, tau=tau, eps_base=eps_base,
                                                      is_causal=True, eps=eps, doc_ids=doc)
            else:
                heads = flash_born_attention(Q, K, V, scale=scale, is_causal=True, eps=eps, doc_ids=doc)
            out = torch.nn.functional.linear(heads.transpose(1, 2).reshape(B, T, E), wo)
        return out

    def eager_path(x, ws):
        # The layer's eager formulation under the same bf16 autocast (so both
        # paths quantise Q, K, V alike), with the attention itself in fp32.
        wq, wk, wv, wo = ws
        with torch.autocast("cuda", dtype=torch.bfloat16):
            psi = l2_normalize(x, dim=-1, eps=1e-12)
            Q = torch.nn.functional.linear(psi, wq).view(B, T, H, D).transpose(1, 2).contiguous()
            K = torch.nn.functional.linear(psi, wk).view(B, T, H, D).transpose(1, 2).contiguous()
            V = torch.nn.functional.linear(psi, wv).view(B, T, H, D).transpose(1, 2).contiguous()
            Q = l2_normalize(apply_unitary_rope(Q, cos, sin), dim=-1, eps=1e-12)
            K = l2_normalize(apply_unitary_rope(K, cos, sin), dim=-1, eps=1e-12)
        w = _eager_weights(Q.float(), K.float(), scale, purified, tau, eps_base, eps, doc)
        heads = torch.matmul(w, V.float())
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return torch.nn.functional.linear(heads.to(torch.bfloat16).transpose(1, 2).reshape(B, T, E), wo)

    ws_a = _weights(E, cuda_device, 3)
    ws_b = [w.detach().clone().requires_grad_(True) for w in ws_a]
    xa = x.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)
    out_a = mi355x_path(xa, ws_a)
    out_b = eager_path(xb, ws_b)
    out_a.backward(gout.to(out_a.dtype))
    out_b.backward(gout.to(out_b.dtype))
    torch.cuda.synchronize()
    assert out_a.dtype == torch.bfloat16
    assert _rel(out_a, out_b) < 2e-2, _rel(out_a, out_b)
    assert _rel(xa.grad, xb.grad) < 3e-2, _rel(xa.grad, xb.grad)
    for name, wa, wb in zip(("q", "k", "v", "o"), ws_a, ws_b):
        assert _rel(wa.grad, wb.grad) < 3e-2, (name, _rel(wa.grad, wb.grad))
