"""Host-side helpers on the flash-Born path's inputs.

``compute_document_ids`` builds the ``doc_ids`` argument from token ids
(reference src/qdlblocks/layers/attention.py:308-315); ``l2_normalize`` is the
per-head-vector normalisation the Born layer applies to Q and K before the
kernel (reference src/qdlblocks/functional.py:59-84); ``apply_unitary_rope``
is the rotation it applies before that (functional.py:104-121).  These are the
eager formulations; ``kernels.qk_prologue.fused_qk_rope_l2_normalize`` runs
both in one HIP pass on the GPU.
"""

from __future__ import annotations

import torch

__all__ = ["apply_unitary_rope", "compute_document_ids", "l2_normalize"]


def compute_document_ids(idx: torch.Tensor, eot_token_id: int = 50256) -> torch.Tensor:
    """Document id per token, (B, T) int32.

    Ids count the end-of-text tokens strictly before each position, so an
    end-of-text token closes (belongs to) the document it terminates.
    """
    eot = (idx == int(eot_token_id)).to(torch.int32)
    before = torch.cumsum(eot, dim=-1, dtype=torch.int32) - eot
    return before.to(torch.int32)


def l2_normalize(x: torch.Tensor, dim: int = -1, eps: float = 1e-12) -> torch.Tensor:
    """x / sqrt(sum x^2 + eps) along ``dim``, computed in fp32, returned in x.dtype."""
    xf = x.float()
    inv = torch.rsqrt(xf.square().sum(dim=dim, keepdim=True) + eps)
    return (xf * inv).to(x.dtype)


def apply_unitary_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate column pairs (i, i + D/2) of ``x`` by the tables' angles, every
    op in ``x.dtype``: cat(x1 c - x2 s, x1 s + x2 c) with c, s cast to x.dtype."""
    d = x.shape[-1]
    x1, x2 = x[..., : d // 2], x[..., d // 2 :]
    c = cos.to(x.dtype)
    s = sin.to(x.dtype)
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)
