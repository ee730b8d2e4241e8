"""Shared helpers for the test suite (inputs, error metrics)."""

from __future__ import annotations

import numpy as np
import torch


def seeded_inputs(shape, seed=0, std=1.0, n=3, dtype=torch.float32):
    """n tensors drawn N(0, std^2) in fp32 on the CPU from one generator, in order."""
    g = torch.Generator("cpu").manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype) for _ in range(n)]


def rel_err(out, ref) -> float:
    """Normwise relative error max|out - ref| / max|ref|."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.abs(ref).max() if ref.size else 0.0
    diff = np.abs(out - ref).max() if ref.size else 0.0
    return float(diff / den) if den > 0 else float(diff)


def max_abs(out, ref) -> float:
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(out - ref).max()) if ref.size else 0.0


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().double().numpy()


TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
