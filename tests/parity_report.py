"""Per-config parity table of the HIP kernels against the float64 oracle:
BASELINE.json's configs C1-C5 (C4 forward, and its document-masked training
step) in bf16, fp16 and fp32, on the configs' own seeded inputs.

    python tests/parity_report.py [--out FILE]

For each (config, dtype): O's normwise relative error max|O - O_ref| /
max|O_ref| and its max-abs error, Z's worst row-relative error and worst
error / rounding bound (util.z_row_bound; <= 1 passes), and for the configs
with a backward the same two numbers for dQ, dK and dV (delta formed from the
stored O, as the reference does).  Heads: every head at C1-C3, 16 heads at
C4 / C5 (every batch row and head index, each b * H + h residue modulo 8
twice).  Long document rows are compared document by document (exact: no
pair crosses a document).  O's worst row (per-row normwise error) is
reported too.  Needs a GPU; run by hand, not collected by pytest.

fp16 runs the reference's own weight arithmetic (p = (8 q.k)^2 in fp32,
rounded to fp16 for P.V, Z from the fp32 weights).  On the N(0, 1) inputs of
C1, C4 and C5 those weights exceed fp16's 65504 (the reference's fp16 kernel
overflows there too), so the fp16 rows of those configs draw N(0, 0.25)
instead, and every fp16 row is held to the oracle that rounds the weights as
the reference's kernel does.
"""

from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

from oracle import born_oracle as orc  # noqa: E402
from util import abi_forward, doc_spans, f64, max_abs, oracle_forward_heads, rel_err, row_errors  # noqa: E402

C5_HEADS = [(b, (5 * b + 3) % 16) for b in range(16)]
C4_HEADS = [(b, 4 * j + (b + j) % 4) for b in range(4) for j in range(4)]

# name: (B, H, T, D, std, l2-normalised q/k, document mean length, backward, heads)
CONFIGS = {
    "C1": (1, 4, 256, 64, 1.0, False, None, True, None),
    "C2": (32, 4, 1024, 64, 1.0, True, None, False, None),
    "C3": (16, 16, 1024, 64, 0.125, False, None, False, None),
    "C4": (4, 16, 8192, 64, 1.0, False, 512.0, False, C4_HEADS),
    "C4 + backward": (4, 16, 8192, 64, 1.0, False, 512.0, True, C4_HEADS),
    "C5": (16, 16, 2048, 64, 1.0, False, None, True, C5_HEADS),
}
NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _inputs(cfg, dtype, dev):
    from quantumdlblocks_amd import l2_normalize

    B, H, T, D, std, l2, doc_mean = cfg[:7]
    if dtype == torch.float16 and std >= 1.0 and not l2:
        std = 0.5  # inside the reference's fp16 weight range at scale 8
    g = torch.Generator("cpu").manual_seed(0)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g) * std for _ in range(4))
    if l2:
        q, k = l2_normalize(q), l2_normalize(k)
    doc = None if doc_mean is None else orc.geometric_doc_ids(B, T, doc_mean, seed=0)
    return [x.to(dev, dtype).contiguous() for x in (q, k, v, do)], doc


def _backward_heads(q, k, v, do, out, sel, doc, T):
    spans = None
    if doc is not None and T > 2048:
        spans = {b: doc_spans(doc[b]) for b, _ in sel}
    refs = [[], [], []]
    for b, h in sel:
        parts = [[], [], []]
        for a, e in ([(0, T)] if spans is None else spans[b]):
            args = [f64(x[b : b + 1, h : h + 1, a:e]) for x in (q, k, v)]
            r = orc.backward(*args, 8.0, f64(do[b : b + 1, h : h + 1, a:e]), True, 1e-12, 0,
                             None if (doc is None or spans is not None) else doc[b : b + 1],
                             out=f64(out[b : b + 1, h : h + 1, a:e]))
            for i in range(3):
                parts[i].append(r[i])
        for i in range(3):
            refs[i].append(np.concatenate(parts[i], axis=2)[0, 0])
    return [np.stack(r) for r in refs]


def run(name, dtype, dev):
    from quantumdlblocks_amd import flash_born_attention

    cfg = CONFIGS[name]
    B, H, T, D = cfg[:4]
    backward, heads = cfg[7], cfg[8]
    (q, k, v, do), doc = _inputs(cfg, dtype, dev)
    sel = [(b, h) for b in range(B) for h in range(H)] if heads is None else heads
    out, z = abi_forward(q, k, v, 8.0, True, 1e-12, 0, doc)
    wd = "f16" if dtype == torch.float16 else None
    keys, ref, zref, zb = oracle_forward_heads(f64(q), f64(k), f64(v), np.array([8.0]), sel, True, 1e-12, 0,
                                               doc, dtype, weight_dtype=wd)
    got = np.stack([f64(out[b, h]) for b, h in keys])
    zg = np.stack([f64(z[b, h]) for b, h in keys])
    row = {
        "config": name, "dtype": NAME[dtype] + (" (N(0, 0.25))" if dtype == torch.float16 and cfg[4] >= 1.0
                                                and not cfg[5] else ""),
        "heads": f"{len(keys)} of {B * H}",
        "O": (rel_err(got, ref), max_abs(got, ref)),
        "Orow": float(row_errors(got, ref).max()),
        "Z": (float((np.abs(zg - zref) / zref).max()), float((np.abs(zg - zref) / zb).max())),
    }
    if backward:
        qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        doc_t = None if doc is None else torch.as_tensor(doc, device=dev)
        o2 = flash_born_attention(qg, kg, vg, torch.tensor(8.0, device=dev), doc_ids=doc_t)
        o2.backward(do)
        torch.cuda.synchronize()
        refs = _backward_heads(q, k, v, do, o2.detach(), sel, doc, T)
        for name_g, t, r in zip(("dQ", "dK", "dV"), (qg.grad, kg.grad, vg.grad), refs):
            gt = np.stack([f64(t[b, h]) for b, h in sel])
            row[name_g] = (rel_err(gt, r), max_abs(gt, r))
    return row


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default="parity_report.md")
    ap.add_argument("--configs", default=",".join(CONFIGS))
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    rows = []
    for name in args.configs.split(","):
        for dtype in (torch.bfloat16, torch.float16, torch.float32):
            t0 = time.perf_counter()
            r = run(name, dtype, dev)
            rows.append(r)
            print(f"{name} {NAME[dtype]}: {r} ({time.perf_counter() - t0:.1f} s)", flush=True)
    fmt = lambda p: f"{p[0]:.2e} / {p[1]:.2e}"  # noqa: E731
    lines = [
        "| Config | dtype | heads | O rel / max-abs | O worst row | Z worst row rel / worst err÷bound "
        "| dQ rel / max-abs | dK rel / max-abs | dV rel / max-abs |",
        "|---|---|---|---|---|---|---|---|---|",
    ]
    for r in rows:
        g = [fmt(r[x]) if x in r else "—" for x in ("dQ", "dK", "dV")]
        lines.append(f"| {r['config']} | {r['dtype']} | {r['heads']} | {fmt(r['O'])} | {r['Orow']:.2e} | "
                     f"{r['Z'][0]:.2e} / {r['Z'][1]:.3f} | {' | '.join(g)} |")
    text = "\n".join(lines) + "\n"
    os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
    with open(args.out, "w") as f:
        f.write(text)
    print(text, flush=True)


if __name__ == "__main__":
    main()
