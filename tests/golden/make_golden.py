"""Write tests/golden/born_cases.npz: small flash-Born input/output vectors.

    python tests/golden/make_golden.py

Inputs are drawn from a fixed numpy generator and rounded to bfloat16
(stored as float32), so one fixture serves the fp32, bf16 and fp16 paths with
identical inputs.  Expected outputs (O, Z, dq, dk, dv, dscale) come from the
float64 oracle (oracle/born_oracle.py) and are stored as float32 (relative
precision ~6e-8, far inside every tolerance that reads them).

The cases cover what the reference's own tests exercise on this path
(reference tests/test_flash_born.py:19-67, tests/test_jax_haliax.py:74-134,
tests/test_hypothesis_016_speedrun_systems_and_arch.py:160-222): causal and
non-causal, window and document masks, per-head and negative scales, eps,
T = 1, and D = 8 / 16 / 32 / 64.  The reference stores no tensors of its own
for this path, so these vectors are the build's; the literal document-id
golden of the reference test is included as data (case ``docids``).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import born_oracle as orc  # noqa: E402

OUT = HERE / "born_cases.npz"

# name: (B, H, T, D, scale, is_causal, eps, window, doc kind, std)
CASES = {
    "causal_d64": (1, 1, 40, 64, 8.0, True, 1e-12, 0, None, 0.25),
    "dense_d32": (1, 2, 32, 32, 2.5, False, 1e-12, 0, None, 0.5),
    "window_doc_d16": (2, 2, 64, 16, [3.0, -2.0], True, 1e-12, 9, "geometric", 0.5),
    "negscale_eps_d64": (1, 1, 33, 64, -5.0, True, 1e-6, 0, None, 0.25),
    "perhead_d8": (2, 2, 16, 8, [2.5, 3.2], True, 1e-6, 0, None, 1.0),
    "noncausal_window_doc_d32": (1, 1, 50, 32, 4.0, False, 1e-12, 12, "geometric", 0.5),
    "single_token_d8": (1, 1, 1, 8, 1.5, True, 1e-12, 0, None, 1.0),
}


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), kept as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def make() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}
    for name, (B, H, T, D, scale, causal, eps, window, doc_kind, std) in CASES.items():
        q, k, v, do = (bf16_round(rng.standard_normal((B, H, T, D)).astype(np.float32) * std) for _ in range(4))
        sc = np.asarray(scale, dtype=np.float32).reshape(-1)
        doc = orc.geometric_doc_ids(B, T, 8.0, seed=len(name)) if doc_kind else None
        kw = dict(is_causal=causal, eps=eps, window_size=window, doc_ids=doc)
        o, z = orc.forward(q, k, v, sc if sc.size > 1 else float(sc[0]), **kw)
        dq, dk, dv, ds = orc.backward(q, k, v, sc if sc.size > 1 else float(sc[0]), do, **kw)
        p = name + "/"
        out[p + "q"], out[p + "k"], out[p + "v"], out[p + "do"] = q, k, v, do
        out[p + "scale"] = sc
        out[p + "meta"] = np.array([float(causal), eps, float(window)], dtype=np.float64)
        out[p + "doc_ids"] = doc.astype(np.int32) if doc is not None else np.zeros((0,), np.int32)
        for key, val in (("out", o), ("z", z), ("dq", dq), ("dk", dk), ("dv", dv), ("dscale", ds)):
            out[p + key] = np.asarray(val, dtype=np.float32)
    # Literal golden of the reference test (test_hypothesis_016...:163-177).
    out["docids/idx"] = np.array([[10, 20, 50256, 30, 40, 50256, 50, 60], [11, 50256, 22, 33, 44, 55, 66, 77]])
    out["docids/expected"] = np.array([[0, 0, 0, 1, 1, 1, 2, 2], [0, 0, 1, 1, 1, 1, 1, 1]], dtype=np.int32)
    return out


def cases(data) -> list[str]:
    return sorted({k.split("/")[0] for k in data.keys() if k.endswith("/q")})


if __name__ == "__main__":
    np.savez_compressed(OUT, **make())
    print(OUT, OUT.stat().st_size, "bytes")
