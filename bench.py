#!/usr/bin/env python
"""Flash-Born attention throughput on one MI355X.

Default (what the driver runs): config C3, the headline -- causal bf16 Born
attention forward, B=16 H=16 T=1024 D=64, Q, K, V ~ N(0, 1/64) (seeded,
synthetic), scale 8.0, eps 1e-12.  A step is one forward launch over one
input set; the timed steps rotate over several input sets (> the 256 MB
Infinity Cache) so every step reads its inputs from HBM.

Prints ONE JSON line (rank 0) with the metric of BASELINE.json: algorithmic
TFLOP/s (4*D*visible_pairs*B*H per forward) and its fraction of the MI355X
dense bf16 MFMA peak, plus ``roofline`` (the kernel's HIP-event-timed
average launch against the HBM roof) and ``cpu_baseline`` (the reference's
eager CPU path, restated in oracle/born_oracle.py, timed on a bounded sample
on this host).  The default run then times the north star's other configs
the same way (C2, C4 with its documents, the C5 forward alone and the C5
forward + backward), each with its own roofline, measured traffic and CPU
baseline, under ``detail.north_star_configs`` (``--no-extra`` skips them).

    python bench.py [--steps K] [--warmup W] [--config c3|c2|c4|c4b|c5fwd|c5|p3|p5|p4b|qk3|qk5]

p3 / p5: purified-Born attention (the reference's flash_purified_born_attention,
gamma 8, tau 0.0625, eps_base 0.05, eps 1e-8) on the C3 / C5 shapes with bf16
inputs, on bf16 MFMA: the forward splits each fp32 weight into two bf16 terms
(the reference's P V is an fp32 dot); the backward contracts the bf16-rounded
weights as the reference does.

qk3 / qk5: the fused Q/K prologue (unitary RoPE then L2 normalisation of Q
and K, attention.py:573-589), forward (qk3) or forward + backward (qk5), on the
C3 / C5 shapes, bf16, with Q and K read as the (B, T, H, D) projection output
viewed as (B, H, T, D).  It is a streaming kernel: its metric is algorithmic
GB/s against the HBM roof.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 MFMA

CONFIGS = {
    # name: (B, H, T, D, std, l2norm_qk, doc_mean, backward)
    "c2": (32, 4, 1024, 64, 1.0, True, None, False),
    "c3": (16, 16, 1024, 64, 0.125, False, None, False),
    "c4": (4, 16, 8192, 64, 1.0, False, 512.0, False),
    "c4b": (4, 16, 8192, 64, 1.0, False, 512.0, True),  # C4 with the backward (document-masked training)
    "c5fwd": (16, 16, 2048, 64, 1.0, False, None, False),
    "c5": (16, 16, 2048, 64, 1.0, False, None, True),
    # purified-Born attention on the C3 / C5 shapes
    "p3": (16, 16, 1024, 64, 0.125, False, None, False),
    "p5": (16, 16, 2048, 64, 0.125, False, None, True),
    "p4b": (4, 16, 8192, 64, 0.125, False, 512.0, True),  # C4 documents, fwd + bwd
}
PURIFIED = {"p3", "p5", "p4b"}
# Outside the D = 64 / no-window fast kernels, on the C3 work: head dim 128
# (half the heads, same flops and bytes) and sliding windows (causal, the
# reference's window_size; runtime-changed windows, born_gpt.py:594).
CONFIGS.update({
    "d3": (16, 8, 1024, 128, 0.125, False, None, False),
    "d5": (16, 8, 2048, 128, 1.0, False, None, True),
    "w3": (16, 16, 1024, 64, 0.125, False, None, False),
    "w5": (16, 16, 2048, 64, 1.0, False, None, True),
    # C4's documents at head dim 128 (half the heads, same flops and bytes)
    "dc4": (4, 8, 8192, 128, 1.0, False, 512.0, False),
    "dc4b": (4, 8, 8192, 128, 1.0, False, 512.0, True),
    # the same with a 256-key causal window (documents and window together)
    "dwc4b": (4, 8, 8192, 128, 1.0, False, 512.0, True),
    # w5's 512-key window at head dim 128 (C5 work)
    "dw5": (16, 8, 2048, 128, 1.0, False, None, True),
    "wc4b": (4, 16, 8192, 64, 1.0, False, 512.0, True),
    # purified-Born attention at head dim 128 on the same work
    "pd3": (16, 8, 1024, 128, 0.125, False, None, False),
    "pd5": (16, 8, 2048, 128, 0.125, False, None, True),
    "pdc4b": (4, 8, 8192, 128, 0.125, False, 512.0, True),  # C4 documents, fwd + bwd
    # purified with the wavelet models' 384-key causal window, C5 work, with
    # C4's documents too, and at head dim 128
    "pw5": (16, 16, 2048, 64, 0.125, False, None, True),
    "pwc4b": (4, 16, 8192, 64, 0.125, False, 512.0, True),
    "pdw5": (16, 8, 2048, 128, 0.125, False, None, True),
    # head dim 256 on the C3 / C5 work (a quarter of the heads, same flops)
    "h3": (16, 4, 1024, 256, 0.125, False, None, False),
    "h5": (16, 4, 2048, 256, 1.0, False, None, True),
})
PURIFIED |= {"pd3", "pd5", "pdc4b", "pw5", "pwc4b", "pdw5"}
WINDOW = {"w3": 256, "w5": 512, "dw5": 512, "dwc4b": 256, "wc4b": 256, "pw5": 384, "pwc4b": 384, "pdw5": 384}
PUR_GAMMA, PUR_TAU, PUR_EPS_BASE, PUR_EPS = 8.0, 0.0625, 0.05, 1e-8
# Fused Q/K prologue (RoPE + L2 normalisation) on the C3 / C5 shapes.
PROLOGUE = {"qk3": (16, 16, 1024, 64, False), "qk5": (16, 16, 2048, 64, True)}
# The prologue folded into the attention forward (one kernel), C3 / C5 / C4
# shapes (C4: its documents of mean length 512), Q and K read raw from the
# (B, T, H, D) projection layout.
FUSED = {"qkc3": (16, 16, 1024, 64, None), "qkc5": (16, 16, 2048, 64, None), "qkc4": (4, 16, 8192, 64, 512.0)}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # The defaults bring the GPU to its steady clocks first: the same launch is
    # ~15% slower over the first ~20 steps than after ~2000 (~0.1 s of load).
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS) + sorted(PROLOGUE) + sorted(FUSED))
    ap.add_argument("--sets", type=int, default=4, help="input sets rotated over the timed steps")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU-baseline leg")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="c3 only: skip the other north-star configs (C2, C4, C5 forward, C5 forward + backward) "
                         "that the default run also times under detail.north_star_configs")
    ap.add_argument("--profile", action="store_true",
                    help="run for rocprofv3: 500 warm-up steps, then 20 rotated and 20 hot steps (no CPU leg)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of known size (calibrates FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


COPY_BYTES = 512 << 20  # bytes read (and written) per calibration copy


def copy_calibration(steps):
    """A plain device-to-device copy of COPY_BYTES, `steps` times: under
    rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE per dispatch, divided into
    the known size, gives the scale factor applied to the kernel's counters."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_BYTES, "steps": steps}), flush=True)


CLOCK_RAMP_S = 0.3  # untimed load before the timed steps (clocks settle after ~0.1 s)


def clock_ramp(step, done):
    """Untimed steps after the W warm-up steps until the GPU has been loaded
    for CLOCK_RAMP_S seconds: the same launch runs ~15% slower during its
    first ~0.1 s of load than at steady clocks, so a short warm-up (the
    driver passes W=5) would otherwise time the clock ramp.  Returns the
    number of extra steps run (reported in the JSON line)."""
    import torch

    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < CLOCK_RAMP_S:
        for _ in range(50):
            step(done + n)
            n += 1
        torch.cuda.synchronize()
    return n


def load_traffic(config):
    """HBM bytes per step (every kernel of the step) measured by rocprofv3 --pmc for `config`,
    from profiles/traffic_<config>.txt (line `traffic_bytes_per_launch = N`),
    or None when no such measurement is committed."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch"):
                    return int(float(line.split("=", 1)[1]))
    except (OSError, ValueError):
        return None
    return None


def make_inputs(cfg, seed, device, dtype):
    import numpy as np
    import torch

    from quantumdlblocks_amd import l2_normalize

    B, H, T, D, std, l2, doc_mean, _ = cfg
    g = torch.Generator("cpu").manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g) * std for _ in range(4))
    if l2:
        q, k = l2_normalize(q), l2_normalize(k)
    doc = None
    if doc_mean is not None:
        doc = torch.from_numpy(doc_ids_np(B, T, doc_mean, seed)).to(device)
    return [x.to(device, dtype).contiguous() for x in (q, k, v, do)], doc


def doc_ids_np(B, T, doc_mean, seed):
    """Sorted document ids (B, T) int32: runs of geometric length with the
    given mean, as compute_document_ids produces for packed sequences."""
    import numpy as np

    rng = np.random.default_rng(seed)
    ids = np.empty((B, T), dtype=np.int32)
    for b in range(B):
        t = n_doc = 0
        while t < T:
            n = int(rng.geometric(1.0 / doc_mean))
            ids[b, t : t + n] = n_doc
            t += n
            n_doc += 1
    return ids


def visible_pairs(cfg, doc, window=0):
    """Visible (b, i, j) pairs summed over the batch, per head (causal; with a
    sliding window row i sees min(i + 1, window) keys of its run: the whole
    row, or each document's contiguous run)."""
    import numpy as np

    B, T = cfg[0], cfg[2]

    def run_pairs(n):  # causal pairs of a run of n rows
        n = np.asarray(n, dtype=np.int64)
        if window <= 0:
            return n * (n + 1) // 2
        w = np.minimum(window, n)
        return w * (w + 1) // 2 + (n - w) * w

    if doc is None:
        return B * int(run_pairs(T))
    total = 0
    for row in doc.cpu().numpy():
        _, counts = np.unique(row, return_counts=True)  # documents are contiguous runs
        total += int(run_pairs(counts).sum())
    return total


def cpu_baseline(cfg, budget_s, seed, purified=False, doc=None, window=0):
    """Time the reference's eager CPU path (fp32, full T x T) on a bounded sample
    of the same workload: n heads of batch row 0, its document mask when the
    config has documents, and the autograd backward when the config has one.
    The rate counts the flops the GPU line counts (visible pairs; 3.5x the
    forward's with the backward)."""
    import numpy as np
    import torch

    from oracle.born_oracle import eager_fp32_torch, purified_eager_fp32_torch

    backward = cfg[7]
    doc_row = None if doc is None else torch.as_tensor(np.asarray(doc)[:1], dtype=torch.int32)

    def eager(q, k, v, sc):
        if purified:
            return purified_eager_fp32_torch(q, k, v, sc, PUR_TAU, PUR_EPS_BASE, True, PUR_EPS, window_size=window,
                                             doc_ids=doc_row)
        return eager_fp32_torch(q, k, v, sc, window_size=window, doc_ids=doc_row)

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B, H, T, D, std = cfg[:5]
    g = torch.Generator("cpu").manual_seed(seed)
    per_run = max(budget_s / 8.0, 0.05)
    sc = torch.tensor(8.0)

    def sample(n):
        q, k, v, do = (torch.randn(1, n, T, D, generator=g) * std for _ in range(4))
        return [x.requires_grad_(backward) for x in (q, k, v)] + [do]

    def step(q, k, v, do):
        if backward:
            out = eager(q, k, v, sc)
            torch.autograd.grad(out, (q, k, v), do)
        else:
            with torch.no_grad():
                eager(q, k, v, sc)

    n = 1
    x = sample(n)
    t0 = time.perf_counter()
    step(*x)
    one = time.perf_counter() - t0
    n = int(max(1, min(B * H, per_run / max(one, 1e-6))))
    x = sample(n)
    for _ in range(3):
        step(*x)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        step(*x)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    pairs = visible_pairs((1, 1, T), doc_row, window)
    flops = 4.0 * D * pairs * n * (3.5 if backward else 1.0)
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    # C1 (the reference's CPU-runnable case):
    # fp32 B1 H4 T256 D64 causal forward, N(0, 1) inputs from the seed.
    g1 = torch.Generator("cpu").manual_seed(seed)
    c1 = [torch.randn(1, 4, 256, 64, generator=g1) for _ in range(3)]
    with torch.no_grad():
        for _ in range(3):
            eager_fp32_torch(*c1, sc)
        t1 = []
        for _ in range(21):
            t0 = time.perf_counter()
            eager_fp32_torch(*c1, sc)
            t1.append(time.perf_counter() - t0)
    t1.sort()
    c1_s = t1[len(t1) // 2]
    c1_flops = 4.0 * 64 * (256 * 257 // 2) * 4
    return {
        "value": flops / med / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "c1": {"value": c1_flops / c1_s / 1e12, "unit": "TFLOP/s", "seconds_per_run": c1_s,
               "sample": "C1 whole: fp32 B1 H4 T256 D64 causal forward, eager (flash_born.py:681-690 "
                         "restated), median of 21 runs after 3 warm-ups"},
        "sample": (f"{n} of the {B * H} (b,h) heads of the same config, fp32, eager "
                   f"(flash_born.py:{'1329-1341' if purified else '681-690'} restated)"
                   f"{', document mask of batch row 0' if doc_row is not None else ''}"
                   f"{', forward + autograd backward' if backward else ''}, median of 5 runs "
                   f"after 3 warm-ups, {med * 1e3:.1f} ms per run"),
        "cpu_model": cpu_model,
        "seconds_per_run": med,
        "speedup_of_gpu": None,
    }


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one GPU: this build's flash-Born path runs on a single MI355X "
            "(sharding (b, h) slices or the sequence over several GPUs is designed, not built); "
            "rerun with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration(args.steps)
        return

    if args.config in PROLOGUE:
        prologue_main(args)
        return
    if args.config in FUSED:
        fused_main(args)
        return

    steps, warmup = (20, 500) if args.profile else (args.steps, args.warmup)
    line = attention_leg(args.config, args, steps, warmup, args.cpu_seconds)
    if args.config == "c3" and not (args.no_extra or args.profile):
        # The north star's other numbers in the same run, after the headline:
        # C2, C4 (documents, visible-pair flops), C5 forward alone and C5
        # forward + backward, each with its roofline, measured traffic and a
        # bounded CPU baseline of its own.
        extra = {}
        for name in NORTH_STAR_EXTRA:
            leg = attention_leg(name, args, steps, warmup, args.cpu_seconds / 4.0)
            extra[name] = {k: leg[k] for k in ("metric", "value", "unit", "ms_per_step", "pct_of_bf16_peak",
                                              "roofline", "cpu_baseline", "config")}
            extra[name]["kernel_us_per_step_events"] = leg["detail"]["kernel_us_per_step_events"]
            extra[name]["hot_kernel_us_per_step_events"] = leg["detail"]["hot_kernel_us_per_step_events"]
            extra[name]["steps"], extra[name]["warmup"] = steps, warmup
        line["detail"]["north_star_configs"] = extra
    print(json.dumps(line), flush=True)


# Timed after the headline by the default run (config c3).
NORTH_STAR_EXTRA = ("c2", "c4", "c5fwd", "c5")


def attention_leg(config, args, steps, warmup, cpu_seconds):
    """Times `steps` steps of one attention config (after `warmup` steps and
    the clock ramp) and returns its JSON line as a dict."""
    import gc

    import torch

    from quantumdlblocks_amd import _native
    from quantumdlblocks_amd.kernels.flash_born import _DTYPE_CODE

    lib = _native.load()
    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    cfg = CONFIGS[config]
    B, H, T, D = cfg[:4]
    backward = cfg[7]
    purified = config in PURIFIED
    window = WINDOW.get(config, 0)
    gc.collect()
    torch.cuda.empty_cache()

    sets = []
    doc = None
    for i in range(max(1, args.sets)):
        (q, k, v, do), doc = make_inputs(cfg, args.seed + i, dev, dtype)
        out = torch.empty(q.shape, dtype=torch.float32, device=dev) if purified else torch.empty_like(q)
        z = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        grads = [torch.empty_like(q) for _ in range(3)] if backward else None
        sets.append((q, k, v, do, out, z, grads))
    scale = torch.tensor(8.0, dtype=torch.float32, device=dev)
    tau = torch.tensor(PUR_TAU, dtype=torch.float32, device=dev)
    dtau = torch.empty(1, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    code = _DTYPE_CODE[dtype]
    doc_ptr = doc.data_ptr() if doc is not None else None
    ws = None
    dscale = torch.empty(1, dtype=torch.float32, device=dev)
    if backward:
        if purified:
            nbytes = int(lib.qdl_flash_purified_born_bwd_workspace_size(code, B, H, T, D))
        else:
            nbytes = int(lib.qdl_flash_born_bwd_workspace_size(code, B, H, T, D, 1))
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)

    def pur_fwd(s):
        q, k, v, _, out, z, _ = s
        rc = lib.qdl_flash_purified_born_fwd(code, B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             out.data_ptr(), z.data_ptr(), scale.data_ptr(), 1, tau.data_ptr(), 1,
                                             PUR_EPS_BASE, doc_ptr, 1, window, PUR_EPS, stream)
        _native.check(rc, "qdl_flash_purified_born_fwd")

    def pur_bwd(s):
        q, k, v, do, out, z, (dq, dk, dv) = s
        rc = lib.qdl_flash_purified_born_bwd(code, B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             out.data_ptr(), do.data_ptr(), z.data_ptr(), scale.data_ptr(), 1,
                                             tau.data_ptr(), 1, PUR_EPS_BASE, doc_ptr, 1, window, dq.data_ptr(),
                                             dk.data_ptr(), dv.data_ptr(), dscale.data_ptr(), dtau.data_ptr(),
                                             ws.data_ptr(), ws.numel(), stream)
        _native.check(rc, "qdl_flash_purified_born_bwd")

    def fwd(s):
        q, k, v, _, out, z, _ = s
        rc = lib.qdl_flash_born_fwd(code, B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                    out.data_ptr(), z.data_ptr(), scale.data_ptr(), 1, doc_ptr,
                                    1, window, 1e-12, stream)
        _native.check(rc, "qdl_flash_born_fwd")

    def bwd(s):
        q, k, v, do, out, z, (dq, dk, dv) = s
        rc = lib.qdl_flash_born_bwd(code, B, H, T, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                    out.data_ptr(), do.data_ptr(), z.data_ptr(), scale.data_ptr(), 1,
                                    doc_ptr, 1, window, 1e-12, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                    dscale.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _native.check(rc, "qdl_flash_born_bwd")

    def step(i):
        s = sets[i % len(sets)]
        (pur_fwd if purified else fwd)(s)
        if backward:
            (pur_bwd if purified else bwd)(s)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ramp = clock_ramp(step, warmup)

    def timed(n_steps, rotate=True):
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        for i in range(n_steps):
            step(i if rotate else 0)
        ev1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return wall / n_steps, ev0.elapsed_time(ev1) / 1e3 / n_steps

    wall_step, ev_step = timed(steps, rotate=True)
    hot_wall, hot_ev = timed(steps, rotate=False)
    for s in sets:
        assert torch.isfinite(s[4]).all(), "non-finite output"

    pairs = visible_pairs(cfg, doc, window)
    fwd_flops = 4.0 * D * pairs * H
    flops = fwd_flops * (3.5 if backward else 1.0)
    el = 2  # bf16 bytes
    oel = 4 if purified else el  # the purified output (read back by its backward) is fp32
    fwd_bytes = B * H * T * D * (el * 3 + oel) + B * H * T * 4  # read Q, K, V; write O (+ Z fp32)
    bwd_bytes = B * H * T * D * (el * 7 + oel) + B * H * T * 4  # read Q,K,V,O,dO (+Z); write dQ,dK,dV
    nbytes = fwd_bytes + (bwd_bytes if backward else 0)

    value = flops / wall_step / 1e12
    achieved_tflops = flops / ev_step / 1e12
    achieved_gbs = nbytes / ev_step / 1e9
    ai = flops / nbytes
    # Every kernel of these configs contracts on bf16 MFMA (the purified
    # forward splits each fp32 weight into two bf16 terms).
    mfma_peak = PEAK_BF16_TFLOPS
    hbm_bound = ai * PEAK_HBM_GBS / 1e3 < mfma_peak
    if hbm_bound:
        roof = {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved_gbs / PEAK_HBM_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(achieved_tflops, 1), "peak": mfma_peak,
                "unit": "TFLOP/s", "frac": round(achieved_tflops / mfma_peak, 4)}
    # HBM bytes per step measured by rocprofv3 (all of the step's kernels).
    roof["traffic"] = load_traffic(config)

    cpu = None
    if not (args.no_cpu_baseline or args.profile):
        cpu = cpu_baseline(cfg, cpu_seconds, args.seed, purified,
                           None if doc is None else doc.cpu().numpy(), window)
        cpu["speedup_of_gpu"] = round(value / cpu["value"], 1)

    name = "fwd" if not backward else "fwd+bwd"
    kind = "Purified-Born-attn" if purified else "Born-attn"
    line = {
        "metric": f"{kind} {name} TFLOP/s + % of bf16 MFMA peak, B{B} H{H} T{T} hd{D}",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(wall_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 (fp32 weights as two bf16 terms in the forward)" if purified else "bf16",
        "data": "synthetic (seeded N(0,%g) Q, K, V; %d rotated input sets)" % (cfg[4] ** 2, len(sets)),
        "config": {
            "workload": config + (" (headline)" if config == "c3" else ""),
            "batch": B, "heads": H, "seq_len": T, "head_dim": D, "causal": True,
            "doc_mask": doc is not None, "window": window, "backward": backward, "scale": 8.0,
            "eps": PUR_EPS if purified else 1e-12,
            **({"tau": PUR_TAU, "eps_base": PUR_EPS_BASE} if purified else {}),
        },
        "pct_of_bf16_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "roofline": roof,
        "cpu_baseline": cpu,
        "detail": {
            "kernel_us_per_step_events": round(ev_step * 1e6, 3),
            "hot_kernel_us_per_step_events": round(hot_ev * 1e6, 3),
            "hot_tflops": round(flops / hot_wall / 1e12, 2),
            "untimed_clock_ramp_steps": ramp,
            "algorithmic_flops": flops,
            "algorithmic_bytes": nbytes,
            "arith_intensity": round(ai, 1),
            "achieved_tflops_events": round(achieved_tflops, 2),
            "mfma_frac_events": round(achieved_tflops / PEAK_BF16_TFLOPS, 4),
            "visible_pairs_per_head": pairs,
            "device": torch.cuda.get_device_name(dev),
            "torch": torch.__version__,
            "host": platform.node(),
        },
    }
    return line


def prologue_tables(T, n, device=None):
    """Rotary tables of the reference's UnitaryRoPE with its defaults
    (isometric.py:87-126: base 10000, every frequency active), fp32 (T, n)."""
    import torch

    freqs = 1.0 / (10000.0 ** (torch.arange(0, n, dtype=torch.float32) / n))
    ang = torch.outer(torch.arange(T, dtype=torch.float32), freqs)
    return torch.cos(ang).to(device), torch.sin(ang).to(device)


def prologue_cpu_baseline(B, H, T, D, backward, budget_s, seed):
    """The reference's eager CPU formulation (oracle/qk_prologue_oracle.py
    ``eager_torch``, bf16 tensor ops) timed on a bounded sample of heads."""
    import torch

    from oracle.qk_prologue_oracle import eager_torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator("cpu").manual_seed(seed)
    cos, sin = prologue_tables(T, D // 2)
    per_run = max(budget_s / 8.0, 0.05)

    def run(n):
        q = torch.randn(1, n, T, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, n, T, D, generator=g).to(torch.bfloat16)
        if backward:
            q.requires_grad_(True)
            k.requires_grad_(True)
        t0 = time.perf_counter()
        qo = eager_torch(q, cos, sin, 1e-12)
        ko = eager_torch(k, cos, sin, 1e-12)
        if backward:
            torch.autograd.backward([qo, ko], [torch.ones_like(qo), torch.ones_like(ko)])
        return time.perf_counter() - t0

    run(1)
    one = run(1)
    n = int(max(1, min(B * H, per_run / max(one, 1e-6))))
    for _ in range(3):
        run(n)
    times = sorted(run(n) for _ in range(5))
    med = times[len(times) // 2]
    rows = 2 * n * T
    per_row = (2 * D * 2 + 4) + ((3 * D * 2 + 4) if backward else 0)
    return {
        "value": rows * per_row / med / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"Q and K of {n} of the {B * H} (b,h) heads, bf16, eager torch "
                   f"(attention.py:574-589 restated{', with autograd backward' if backward else ''}), "
                   f"median of 5 runs after 3 warm-ups, {med * 1e3:.1f} ms per run"),
        "seconds_per_run": med,
        "speedup_of_gpu": None,
    }


def prologue_main(args):
    import torch

    from quantumdlblocks_amd import _native

    lib = _native.load()
    dev = torch.device("cuda:0")
    B, H, T, D, backward = PROLOGUE[args.config]
    steps, warmup = (20, 500) if args.profile else (args.steps, args.warmup)
    code = _native.DTYPE_BF16
    cos, sin = prologue_tables(T, D // 2, dev)
    nf, ld = cos.shape[1], cos.stride(0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    # (B, T, H, D) projection outputs viewed as (B, H, T, D): strides (T H D, D, H D).
    st = (ctypes.c_int64 * 3)(T * H * D, D, H * D)
    cst = (ctypes.c_int64 * 3)(H * T * D, T * D, D)
    sets = []
    g = torch.Generator("cpu").manual_seed(args.seed)
    for i in range(max(1, args.sets)):
        q = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(dev)
        k = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(dev)
        qo, ko = torch.empty(B, H, T, D, dtype=torch.bfloat16, device=dev), torch.empty(B, H, T, D, dtype=torch.bfloat16, device=dev)
        qr, kr = torch.empty(B, H, T, device=dev), torch.empty(B, H, T, device=dev)
        if backward:
            gq = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(dev)
            gk = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(dev)
            dq, dk = torch.empty_like(q), torch.empty_like(k)
        else:
            gq = gk = dq = dk = None
        sets.append((q, k, qo, ko, qr, kr, gq, gk, dq, dk))

    def fwd(s):
        q, k, qo, ko, qr, kr = s[:6]
        rc = lib.qdl_flash_born_qk_prologue_fwd(code, B, H, T, D, q.data_ptr(), st, k.data_ptr(), st,
                                                cos.data_ptr(), sin.data_ptr(), nf, ld, 1e-12,
                                                qo.data_ptr(), ko.data_ptr(), qr.data_ptr(), kr.data_ptr(), stream)
        _native.check(rc, "qdl_flash_born_qk_prologue_fwd")

    def bwd(s):
        q, k, qo, ko, qr, kr, gq, gk, dq, dk = s
        rc = lib.qdl_flash_born_qk_prologue_bwd(code, B, H, T, D, gq.data_ptr(), gk.data_ptr(), qo.data_ptr(),
                                                ko.data_ptr(), qr.data_ptr(), kr.data_ptr(), cos.data_ptr(),
                                                sin.data_ptr(), nf, ld, dq.data_ptr(), st, dk.data_ptr(), st, stream)
        _native.check(rc, "qdl_flash_born_qk_prologue_bwd")

    def step(i, rotate=True):
        s = sets[i % len(sets)] if rotate else sets[0]
        fwd(s)
        if backward:
            bwd(s)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ramp = clock_ramp(step, warmup)

    def timed(n_steps, rotate=True):
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        for i in range(n_steps):
            step(i, rotate)
        ev1.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n_steps, ev0.elapsed_time(ev1) / 1e3 / n_steps

    wall_step, ev_step = timed(steps, True)
    hot_wall, hot_ev = timed(steps, False)
    for s in sets:
        assert torch.isfinite(s[2].float()).all() and torch.isfinite(s[3].float()).all(), "non-finite output"
    del cst

    rows = 2 * B * H * T
    table = T * nf * 4 * 2
    fwd_bytes = rows * (2 * D * 2 + 4) + table  # read q, k; write q', k' and 1/norm; read the tables
    bwd_bytes = rows * (3 * D * 2 + 4) + table  # read dq', dk', q', k', 1/norm; write dq, dk
    nbytes = fwd_bytes + (bwd_bytes if backward else 0)
    value = nbytes / wall_step / 1e9
    achieved = nbytes / ev_step / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": load_traffic(args.config)}
    cpu = None
    if not (args.no_cpu_baseline or args.profile):
        cpu = prologue_cpu_baseline(B, H, T, D, backward, args.cpu_seconds, args.seed)
        cpu["speedup_of_gpu"] = round(value / cpu["value"], 1)
    name = "fwd+bwd" if backward else "fwd"
    line = {
        "metric": f"Q/K prologue (RoPE + L2 normalise) {name} GB/s, B{B} H{H} T{T} hd{D}",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(wall_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q, K%s; %d rotated input sets)" % (", dQ', dK'" if backward else "", len(sets)),
        "config": {"workload": args.config, "batch": B, "heads": H, "seq_len": T, "head_dim": D,
                   "rope_pairs": nf, "input_layout": "(B, T, H, D) viewed as (B, H, T, D)",
                   "backward": backward, "eps": 1e-12},
        "roofline": roof,
        "cpu_baseline": cpu,
        "detail": {
            "kernel_us_per_step_events": round(ev_step * 1e6, 3),
            "hot_kernel_us_per_step_events": round(hot_ev * 1e6, 3),
            "hot_gbs": round(nbytes / hot_wall / 1e9, 1),
            "untimed_clock_ramp_steps": ramp,
            "algorithmic_bytes": nbytes,
            "device": torch.cuda.get_device_name(dev),
            "torch": torch.__version__,
            "host": platform.node(),
        },
    }
    print(json.dumps(line), flush=True)


def fused_main(args):
    """qkc3 / qkc5 / qkc4: qdl_flash_born_fwd_qk_prologue, RoPE + L2
    normalisation of Q and K folded into the Born attention forward (C3 / C5
    / C4 shapes, C4 with its documents; bf16, causal, scale 8; Q, K the
    (B, T, H, D) projection output, rotary tables of the reference's
    UnitaryRoPE defaults).  value: the attention's
    algorithmic TFLOP/s of the whole fused step when no backward follows
    (1/norm and q' are not written); detail also times the fused step that
    writes them for a backward, and the same work as two launches (prologue
    kernel, then attention kernel), with and without 1/norm."""
    import torch

    from quantumdlblocks_amd import _native

    lib = _native.load()
    dev = torch.device("cuda:0")
    B, H, T, D, doc_mean = FUSED[args.config]
    steps, warmup = (20, 500) if args.profile else (args.steps, args.warmup)
    code = _native.DTYPE_BF16
    cos, sin = prologue_tables(T, D // 2, dev)
    nf, ld = cos.shape[1], cos.stride(0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    st = (ctypes.c_int64 * 3)(T * H * D, D, H * D)
    scale = torch.tensor(8.0, dtype=torch.float32, device=dev)
    doc = None if doc_mean is None else torch.from_numpy(doc_ids_np(B, T, doc_mean, args.seed)).to(dev)
    docp = None if doc is None else doc.data_ptr()
    g = torch.Generator("cpu").manual_seed(args.seed)
    sets = []
    for _ in range(max(1, args.sets)):
        q = (torch.randn(B, T, H, D, generator=g) * 0.125).to(torch.bfloat16).to(dev)
        k = (torch.randn(B, T, H, D, generator=g) * 0.125).to(torch.bfloat16).to(dev)
        v = (torch.randn(B, H, T, D, generator=g) * 0.125).to(torch.bfloat16).to(dev)
        out = torch.empty(B, H, T, D, dtype=torch.bfloat16, device=dev)
        z = torch.empty(B, H, T, device=dev)
        qo, ko = torch.empty_like(out), torch.empty_like(out)
        qr, kr = torch.empty_like(z), torch.empty_like(z)
        sets.append((q, k, v, out, z, qo, ko, qr, kr))

    def fused(i, rotate=True, bwd_outputs=False):
        q, k, v, out, z, qo, ko, qr, kr = sets[i % len(sets)] if rotate else sets[0]
        rc = lib.qdl_flash_born_fwd_qk_prologue(code, B, H, T, D, q.data_ptr(), st, k.data_ptr(), st, v.data_ptr(),
                                                cos.data_ptr(), sin.data_ptr(), nf, ld, 1e-12, scale.data_ptr(), 1,
                                                docp, 1, 0, 1e-12, out.data_ptr(), z.data_ptr(), qo.data_ptr(),
                                                ko.data_ptr(), qr.data_ptr() if bwd_outputs else None,
                                                kr.data_ptr() if bwd_outputs else None, stream)
        _native.check(rc, "qdl_flash_born_fwd_qk_prologue")

    def fused_train(i):
        fused(i, bwd_outputs=True)

    def separate(i, bwd_outputs=False):
        q, k, v, out, z, qo, ko, qr, kr = sets[i % len(sets)]
        rc = lib.qdl_flash_born_qk_prologue_fwd(code, B, H, T, D, q.data_ptr(), st, k.data_ptr(), st,
                                                cos.data_ptr(), sin.data_ptr(), nf, ld, 1e-12,
                                                qo.data_ptr(), ko.data_ptr(), qr.data_ptr() if bwd_outputs else None,
                                                kr.data_ptr() if bwd_outputs else None, stream)
        _native.check(rc, "qdl_flash_born_qk_prologue_fwd")
        rc = lib.qdl_flash_born_fwd(code, B, H, T, D, qo.data_ptr(), ko.data_ptr(), v.data_ptr(), out.data_ptr(),
                                    z.data_ptr(), scale.data_ptr(), 1, docp, 1, 0, 1e-12, stream)
        _native.check(rc, "qdl_flash_born_fwd")

    for i in range(warmup):
        fused(i)
    torch.cuda.synchronize()
    ramp = clock_ramp(fused, warmup)

    def timed(fn, n_steps):
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        for i in range(n_steps):
            fn(i)
        ev1.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n_steps, ev0.elapsed_time(ev1) / 1e3 / n_steps

    wall_step, ev_step = timed(fused, steps)
    for i in range(max(steps, 50)):
        fused_train(i)
    _, train_ev = timed(fused_train, steps)
    for i in range(max(steps, 50)):
        separate(i)
    sep_wall, sep_ev = timed(separate, steps)
    _, sep_train_ev = timed(lambda i: separate(i, bwd_outputs=True), steps)
    for s_ in sets:
        assert torch.isfinite(s_[3].float()).all(), "non-finite output"

    flops = 4.0 * D * visible_pairs((B, H, T), doc) * H
    rows = B * H * T
    # Algorithmic bytes of the step without a backward: read Q, K, V and the
    # tables, write O and Z.
    nbytes = rows * D * 2 * 3 + rows * D * 2 + rows * 4 + 2 * T * nf * 4
    value = flops / wall_step / 1e12
    roof = {"bound": "hbm", "achieved": round(nbytes / ev_step / 1e9, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(nbytes / ev_step / 1e9 / PEAK_HBM_GBS, 4), "traffic": None}
    line = {
        "metric": f"Born-attn fwd with fused Q/K prologue TFLOP/s, B{B} H{H} T{T} hd{D}",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(wall_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.015625) Q, K, V; %d rotated input sets)" % len(sets),
        "config": {"workload": args.config, "batch": B, "heads": H, "seq_len": T, "head_dim": D, "causal": True,
                   "doc_mask": doc_mean is not None, "doc_mean_len": doc_mean,
                   "rope_pairs": nf, "qk_layout": "(B, T, H, D) viewed as (B, H, T, D)", "scale": 8.0},
        "pct_of_bf16_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "roofline": roof,
        "cpu_baseline": None,
        "detail": {
            "flops_counted_on": "visible (causal, same-document) pairs",
            "fused_kernel_us_per_step_events": round(ev_step * 1e6, 3),
            "separate_two_launches_us_per_step_events": round(sep_ev * 1e6, 3),
            "separate_two_launches_us_per_step_wall": round(sep_wall * 1e6, 3),
            "with_backward_outputs_fused_us_per_step_events": round(train_ev * 1e6, 3),
            "with_backward_outputs_separate_us_per_step_events": round(sep_train_ev * 1e6, 3),
            "algorithmic_flops": flops,
            "algorithmic_bytes": nbytes,
            "untimed_clock_ramp_steps": ramp,
            "device": torch.cuda.get_device_name(dev),
            "torch": torch.__version__,
            "host": platform.node(),
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
