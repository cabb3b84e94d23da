#!/usr/bin/env python3
"""Benchmark of the sparse-attention forward hot path on one MI355X.

Default workload (the headline metric): causal sliding-window attention,
bf16, B=1 H=8 N=65536 D=64, window 64 (keys [i-63, i]).  A "step" is one
forward pass over that batch.  Prints ONE JSON line:

  value      queries/s (B*H*N query rows per second), whole job, 1 GPU:
             K back-to-back launches between two HIP events on the launch
             stream
  roofline   achieved algorithmic HBM GB/s of the kernel (4*B*N*H*D*elt
             bytes per launch / mean kernel duration) against the 8 TB/s
             MI355X peak (or TFLOP/s against the MFMA peak when the work is
             above the ridge).  Kernel durations come from HIP events that
             the library stamps on the kernels' own dispatches
             (ma_attn_forward_timed, hipExtLaunchKernel) in a second pass of
             K launches; traffic = measured HBM bytes per launch from the
             committed rocprofv3 counter summary (roofline.traffic_source
             names it: it is not measured in this run)
  cpu_baseline  the CPU oracle (restatement of ma_core.cpp:160-246) on this
             host, single thread, bounded sample of the same workload
  pattern_copy  sliding, Longformer and block-sparse forward: the kernel's
             access pattern without its arithmetic (ma_attn_copy_probe), timed
             the same way -- the copy speed that pattern reaches on the device;
             the 16-bit fixed-window backward: the fused kernel's pattern
             (ma_attn_backward_copy_probe)

Inputs are resident in HBM before timing; 4+ distinct input sets (>1 GB in
total) are rotated so the 256 MB MALL cannot serve a repeated set.

Workload "ticks": the tick-feature pass (TickDataset preprocessing on the
GPU, ma_tick_features) over 16M synthetic ticks; value = ticks/s, roofline =
116 algorithmic bytes per tick (the six float64 columns read by the
statistics kernel and again by the write kernel, 5 float32 written) over the
pass's stamped duration.

Workload "encoder_layer": the reference model's inference (batch 64, sequence
10, model_dim 64, 4 layers) with each encoder layer as one fused HIP kernel,
against the same weights run as the layer's separate operations; value =
sequences/s, with per-layer latencies of both forms.

With --pass backward --saved-stats (dense, block-sparse, Longformer and
index-set workloads), the backward runs from the forward's saved O and per-row
statistics (ma_attn_backward_saved), the form the autograd layer trains with;
the forward runs once per input set before timing, and the algorithmic bytes
count O and the statistics read as well.  Without --saved-stats the Longformer
backward (longformer_backward) runs a forward that writes each row's lse and
delta = sum_j P dP (no O) and then the one-pass backward, both timed; its
algorithmic bytes stay the 7 tensors of a backward.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                       [--pass forward|backward] [--saved-stats]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "ma-transformer_amd"))
sys.path.insert(0, REPO)

METRIC = "sparse-attn queries/sec + achieved HBM GB/s (% peak) at N=64K, w=64, 1 GPU"
METRIC_TICKS = "tick-feature pass ticks/sec (TickDataset preprocessing), 1 GPU"
TICKS_N = 1 << 24
TICK_BYTES = 2 * 48 + 20  # two reads of 6 float64 columns, 5 float32 written
METRIC_BWD = "sparse-attn backward queries/sec (dQ, dK, dV per query row), 1 GPU"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_F32_PEAK_TFLOPS = 157.3

# name: (B, H, N, D, dtype, pattern kwargs, description)
WORKLOADS = {
    "target": (1, 8, 65536, 64, "bf16", dict(pattern="sliding", left=63, right=0),
               "causal sliding window w=64 (keys [i-63,i]), bf16, B=1 H=8 N=65536 D=64"),
    "cfg1": (1, 4, 1024, 16, "fp32", dict(pattern="sliding", left=63, right=0),
             "causal sliding window w=64, fp32, B=1 H=4 N=1024 D=16"),
    "cfg2_fp32": (4, 8, 8192, 64, "fp32", dict(pattern="sliding", left=32, right=31),
                  "symmetric window [i-32,i+31], fp32, B=4 H=8 N=8192 D=64"),
    "cfg2_bf16": (4, 8, 8192, 64, "bf16", dict(pattern="sliding", left=32, right=31),
                  "symmetric window [i-32,i+31], bf16, B=4 H=8 N=8192 D=64"),
    "cfg3": (2, 8, 16384, 64, "bf16", dict(pattern="block_sparse", block_size=64, extra=2, seed=1234),
             "block-sparse 64x64, diag+prev+2 seeded blocks, bf16, B=2 H=8 N=16384 D=64"),
    "cfg4": (2, 12, 32768, 64, "bf16", dict(pattern="longformer", left=127, right=0, num_global=16),
             "Longformer causal w=128 + 16 globals, bf16, B=2 H=12 N=32768 D=64"),
    "cfg5_fp32": (1, 8, 65536, 64, "fp32", dict(pattern="sliding", left=63, right=0, dilation=4),
                  "dilated causal window (i-4k, k<64), fp32, B=1 H=8 N=65536 D=64"),
    "cfg5_bf16": (1, 8, 65536, 64, "bf16", dict(pattern="sliding", left=63, right=0, dilation=4),
                  "dilated causal window (i-4k, k<64), bf16, B=1 H=8 N=65536 D=64"),
    # not one of the headline configs: the dense_forward(use_causal_mask=True) path at a long sequence
    "dense_causal_bf16": (1, 8, 16384, 64, "bf16", dict(pattern="dense", causal=True),
                          "dense causal (keys [0,i]), bf16, B=1 H=8 N=16384 D=64"),
    # the reference's dense_forward dtype (fp32 only there)
    "dense_causal_fp32": (1, 8, 16384, 64, "fp32", dict(pattern="dense", causal=True),
                          "dense causal (keys [0,i]), fp32, B=1 H=8 N=16384 D=64"),
    # the generic index-set path (explicit key lists, row kernel) on the target's key sets
    "index_set": (1, 8, 65536, 64, "bf16", dict(pattern="index_set", left=63, right=0),
                  "the target's causal w=64 key sets given as an explicit index set (CSR), bf16, "
                  "B=1 H=8 N=65536 D=64"),
}


def window_csr(N: int, left: int, right: int):
    """CSR (int64 offsets [N+1], int32 keys) of the window [i-left, i+right] n [0,N)."""
    import numpy as np
    i = np.arange(N, dtype=np.int64)
    lo, hi = np.maximum(i - left, 0), np.minimum(i + right, N - 1)
    offsets = np.zeros(N + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(hi - lo + 1)
    keys = (np.repeat(lo - offsets[:-1], hi - lo + 1) + np.arange(offsets[-1])).astype(np.int32)
    return offsets, keys


def key_count(N: int, pk: dict) -> int:
    """sum_i |S_i| for one (b, h) -- closed forms of the index sets."""
    p = pk["pattern"]
    if p == "index_set":  # built as a window
        p = "sliding"
    if p == "sliding":
        dil = pk.get("dilation", 1)
        total = 0
        for rho in range(dil):
            nr = (N - rho + dil - 1) // dil
            L, R = pk["left"], pk["right"]
            # rows m in [0,nr): keys [max(0,m-L), min(nr-1,m+R)]
            total += sum(min(nr - 1, m + R) - max(0, m - L) + 1 for m in range(nr)) if nr < 4096 else \
                nr * (L + R + 1) - L * (L + 1) // 2 - R * (R + 1) // 2
        return total
    if p == "block_sparse":
        nb = (N + pk["block_size"] - 1) // pk["block_size"]
        return (nb * (2 + pk["extra"]) - 1) * pk["block_size"] * pk["block_size"]
    if p == "dense":
        return N * (N + 1) // 2 if pk.get("causal") else N * N
    if p == "longformer":
        G, L = pk["num_global"], pk["left"]
        return G * N + sum(i + 1 for i in range(G, G + L)) + (L + 1 + G) * (N - G - L)
    raise ValueError(p)


def load_traffic(workload: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (committed summary), or None."""
    path = os.path.join(REPO, "profiles", f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def load_mfma_busy(workload: str):
    """MFMA busy % of the workload's dominant forward kernel, from the
    committed rocprofv3 MfmaUtil summary, or None."""
    path = os.path.join(REPO, "profiles", "mfma_busy_by_workload.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"^mfma_busy_pct\[" + re.escape(workload) + r"\]:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(B, H, N, D, dtype, pk, budget_s=12.0):
    """Oracle (single thread) on a bounded sample: whole heads until ~budget_s."""
    import numpy as np
    from oracle import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    rng = np.random.default_rng(4321)
    q, k, v = (rng.standard_normal((B, N, H, D), dtype=np.float32) for _ in range(3))
    if dtype != "fp32":
        q, k, v = (O.round_bf16(x) for x in (q, k, v))
    table = None
    if pk["pattern"] == "block_sparse":
        nb = (N + pk["block_size"] - 1) // pk["block_size"]
        table = O.block_table(pk["seed"], nb, pk["extra"])
    offsets = keys = None
    if pk["pattern"] == "index_set":
        offsets, keys = window_csr(N, pk["left"], pk["right"])
    spec = O.Spec(B, N, H, D, pattern=pk["pattern"], left=pk.get("left", 0), right=pk.get("right", 0),
                  dilation=pk.get("dilation", 1), block_size=pk.get("block_size", 64), table=table,
                  num_global=pk.get("num_global", 0), causal=pk.get("causal", False),
                  offsets=offsets, keys=keys)
    # time one head first, then as many whole heads as fit the budget
    t0 = time.perf_counter()
    O.forward(spec, q, k, v, heads=(0, 1))
    t1 = time.perf_counter() - t0
    heads = max(1, min(H, int(budget_s / max(t1, 1e-6))))
    t0 = time.perf_counter()
    O.forward(spec, q, k, v, heads=(0, heads))
    dt = time.perf_counter() - t0
    queries = B * N * heads
    return {
        "value": queries / dt,
        "unit": "queries/s",
        "cores": 1,
        "kind": "port",
        "sample": f"oracle/oracle.c (restated ma_core.cpp:160-246, gcc -O3), {heads} of {H} heads x "
                  f"B={B} x N={N} ({queries} query rows, {dt:.2f} s) on "
                  f"{platform.processor() or platform.machine()} ({os.cpu_count()} host cpus, 1 used); "
                  f"fp32 math on {'upcast bf16' if dtype != 'fp32' else 'fp32'} inputs",
    }


def copy_bandwidth(dev, stream) -> float:
    """GB/s of a 1 GiB torch copy on this box (read + write), for comparison
    with the 8 TB/s spec; its dispatches also calibrate the rocprofv3 HBM
    counters (FETCH_SIZE / WRITE_SIZE of a known byte count)."""
    import torch
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    c0.record(stream)
    for _ in range(10):
        dst.copy_(src)
    c1.record(stream)
    torch.cuda.synchronize()
    gbps = 2 * (1 << 30) * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del src, dst
    return gbps


def cpu_baseline_ticks(n_total, budget_s=10.0):
    """Oracle (numpy float64, one thread) on 2M-tick samples until ~budget_s."""
    import numpy as np
    from oracle import features as F
    cols = F.synthetic_ticks(1 << 21, 77)
    args = [cols[c] for c in ("timestamp", "price", "bid_price", "ask_price", "bid_volume", "ask_volume")]
    reps, t0 = 0, time.perf_counter()
    while True:
        F.tick_features(*args)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            break
    ticks = reps * (1 << 21)
    return {"value": ticks / dt, "unit": "ticks/s", "cores": 1, "kind": "port",
            "sample": f"oracle/features.py (numpy restatement of data_loader.py:15-28), {reps} x 2M ticks "
                      f"({dt:.2f} s) of the {n_total}-tick workload's per-tick work on "
                      f"{platform.processor() or platform.machine()} ({os.cpu_count()} host cpus, 1 used)"}


def bench_ticks(args) -> int:
    import torch
    import tick_features as tf
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n = TICKS_N
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)

    def tick_set():
        # synthetic ticks of the reference generator's shape, built on the device
        ts = torch.sort(torch.rand(n, device=dev, dtype=torch.float64, generator=gen)).values
        mid = 100.0 * torch.exp(torch.cumsum(torch.randn(n, device=dev, dtype=torch.float64, generator=gen), 0)
                                * 1e-3)
        half = mid * 1e-4 * (0.5 + torch.rand(n, device=dev, dtype=torch.float64, generator=gen))
        side = torch.randint(-1, 2, (n,), device=dev, generator=gen).to(torch.float64)
        vol = lambda: torch.clamp(torch.round(100.0 * (1 + 0.5 * torch.randn(n, device=dev, dtype=torch.float64,
                                                                            generator=gen)).abs()), min=1.0)
        return {"timestamp": ts, "price": mid + half * side, "bid_price": mid - half, "ask_price": mid + half,
                "bid_volume": vol(), "ask_volume": vol()}

    nsets = max(2, -(-(1 << 30) // (n * 68)))  # > 1 GB of inputs and outputs in rotation
    sets = [tick_set() for _ in range(nsets)]
    args.warmup = run_warmup(args.warmup, lambda i: tf.compute_tick_features(sets[i % nsets]))
    stream = torch.cuda.current_stream(dev)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(args.steps):
        tf.compute_tick_features(sets[i % nsets])
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b in ev:
        a.record(stream)
        b.record(stream)
    torch.cuda.synchronize()
    for i in range(args.steps):
        tf.compute_tick_features(sets[i % nsets], events=ev[i])
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) for a, b in ev)
    mean_ms = sum(per) / len(per)
    alg = n * TICK_BYTES
    gbps = alg / (mean_ms * 1e-3) / 1e9
    del sets
    copy_gbps = copy_bandwidth(dev, stream)
    out = {
        "metric": METRIC_TICKS, "value": n / (ms_per_step * 1e-3), "unit": "ticks/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": f"synthetic GBM-shaped ticks built on the device, {nsets} rotated sets resident in HBM",
        "config": {"workload": "tick-feature pass (TickDataset preprocessing)", "ticks": n},
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": gbps / HBM_PEAK_GBPS, "traffic": load_traffic("ticks"),
                     "traffic_source": "profiles/traffic_ticks.txt (rocprofv3 FETCH_SIZE + WRITE_SIZE, committed)"},
        "kernel_us_mean": mean_ms * 1e3, "kernel_us_median": per[len(per) // 2] * 1e3,
        "step_us_mean": ms_per_step * 1e3, "algorithmic_bytes_per_launch": alg,
        "copy_kernel_gbps": copy_gbps, "device": torch.cuda.get_device_name(dev),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_ticks(n)
    print(json.dumps(out), flush=True)
    return 0


ENC = dict(batch=64, seq_len=10, input_dim=5, model_dim=64, num_layers=4, window=3)
METRIC_ENC = "TransformerModel inference sequences/sec (reference config, eval), 1 GPU"


def bench_encoder(args) -> int:
    """The reference model's inference at its training configuration
    (configs/default_config.yaml: batch 64, sequence 10, input_dim 5;
    model_dim 64 and 4 layers from its grid), each encoder layer as one fused
    HIP kernel (fused_layers=True) against the same weights run as the
    layer's separate operations.  value = sequences/s of the fused model;
    per-layer latencies of both forms are reported beside it.

    --layer-form fused|ops times only that form's model forward (warmup +
    steps forwards and nothing else), so a kernel trace of the run gives the
    launches of one forward: each kernel's calls / (warmup + steps)."""
    import torch
    import model as M
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    torch.manual_seed(0)
    c = ENC
    fused = M.TransformerModel(input_dim=c["input_dim"], model_dim=c["model_dim"], num_heads=2,
                               num_layers=c["num_layers"], fused_layers=True).to(dev).eval()
    ops = M.TransformerModel(input_dim=c["input_dim"], model_dim=c["model_dim"], num_heads=2,
                             num_layers=c["num_layers"], fused_layers=False).to(dev).eval()
    ops.load_state_dict(fused.state_dict())
    src = torch.randn(c["batch"], c["seq_len"], c["input_dim"], device=dev)
    x = torch.randn(c["batch"], c["seq_len"], c["model_dim"], device=dev)
    layer_f, layer_o = fused.encoder_layers[0], ops.encoder_layers[0]
    stream = torch.cuda.current_stream(dev)

    def timed(fn, steps):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(stream)
        for _ in range(steps):
            fn()
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    form = args.layer_form
    base = {"unit": "sequences/s", "n_gpus": 1, "steps": args.steps, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic N(0,1) ticks, random-init weights of the reference architecture",
            "device": torch.cuda.get_device_name(dev)}
    if form != "both":
        m = fused if form == "fused" else ops
        with torch.no_grad():
            warm = args.warmup if args.warmup is not None else 100
            for _ in range(warm):
                m(src)
            ms = timed(lambda: m(src), args.steps)
        print(json.dumps({"metric": METRIC_ENC + f" ({form} layers)", "value": c["batch"] / (ms * 1e-3),
                          "warmup": warm, "ms_per_step": ms, **base,
                          "config": {"workload": f"TransformerModel eval forward, {form} encoder layers", **c},
                          "forwards_run": warm + args.steps}), flush=True)
        return 0

    with torch.no_grad():
        err = (fused(src) - ops(src)).abs().max().item()
        for fn in (lambda: fused(src), lambda: ops(src), lambda: layer_f(x), lambda: layer_o(x)):
            args.warmup = run_warmup(args.warmup, lambda i: fn())
        ms_model_f = timed(lambda: fused(src), args.steps)
        ms_model_o = timed(lambda: ops(src), args.steps)
        ms_layer_f = timed(lambda: layer_f(x), args.steps)
        ms_layer_o = timed(lambda: layer_o(x), args.steps)
        # the kernel alone: one launch per layer, back to back on the stream
        import ma_attn as _ma
        out = torch.empty_like(x)
        L = M._layer_desc(layer_f, c["batch"], c["seq_len"], dev)
        raw = stream.cuda_stream
        ms_kernel = timed(lambda: _ma.encoder_layer_forward_raw(L, x.data_ptr(), 0, out.data_ptr(), raw),
                          args.steps)
    rows, d, f = c["batch"] * c["seq_len"], c["model_dim"], 4 * c["model_dim"]
    keys = sum(min(c["seq_len"] - 1, i + c["window"]) - max(0, i - c["window"]) + 1
               for i in range(c["seq_len"])) * c["batch"]
    flops = 4 * d * keys + 2 * rows * d * f * 2  # attention (Q.K^T, P.V) + the two Linear layers
    tflops = flops / (ms_kernel * 1e-3) / 1e12
    print(json.dumps({
        "metric": METRIC_ENC, "value": c["batch"] / (ms_model_f * 1e-3), "warmup": args.warmup,
        "ms_per_step": ms_model_f, **base,
        "config": {"workload": "TransformerModel eval forward, fused encoder layers", **c},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / MFMA_F32_PEAK_TFLOPS, "traffic": None,
                     "note": "launch-latency bound: 40 workgroups of 16 tokens"},
        "model_ms_fused": ms_model_f, "model_ms_ops": ms_model_o,
        "layer_us_fused": ms_layer_f * 1e3, "layer_us_ops": ms_layer_o * 1e3,
        "layer_kernel_us_back_to_back": ms_kernel * 1e3, "flops_per_layer": flops,
        "max_abs_diff_fused_vs_ops": err,
    }), flush=True)
    return 0


def run_warmup(warmup, step) -> int:
    """Untimed launches before the timed region; returns how many ran.

    With no --warmup, 5 first launches run, 10 more are timed, and enough
    follow to fill ~0.1 s (20..2000 in all): after a short warmup the GPU's
    clocks have not settled (target: 56.9 us per step after 20 launches,
    54.4 us after 1000).
    """
    import torch
    if warmup is not None:
        for i in range(warmup):
            step(i)
        return warmup
    for i in range(5):  # first calls: descriptors, kernel attributes
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(5, 15):
        step(i)
    torch.cuda.synchronize()
    per = max((time.perf_counter() - t0) / 10, 1e-6)
    total = max(20, min(2000, int(0.1 / per)))
    for i in range(15, total):
        step(i)
    return max(total, 15)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed launches first (default: ~0.1 s of launches, 20..2000, so the GPU's "
                         "clocks settle before the timed region)")
    ap.add_argument("--workload", default="target", choices=sorted(WORKLOADS) + ["ticks", "encoder_layer"])
    ap.add_argument("--sets", type=int, default=0, help="input sets rotated (0: enough for >1 GB)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--configs", dest="configs", action="store_true", default=None,
                    help="also measure every BASELINE config's forward (cfg1, cfg2 fp32/bf16, cfg3, cfg4, "
                         "cfg5 fp32/bf16) into the line's `configs` object (default: on for the target forward)")
    ap.add_argument("--no-configs", dest="configs", action="store_false")
    ap.add_argument("--layer-form", choices=["both", "fused", "ops"], default="both",
                    help="encoder_layer workload: time both model forms (default) or only one")
    ap.add_argument("--pass", dest="which", choices=["forward", "backward"], default="forward",
                    help="backward: dQ, dK, dV from (Q, K, V, dO) (block-sparse, Longformer and index "
                         "sets through index_set_backward over their key sets)")
    ap.add_argument("--saved-stats", action="store_true",
                    help="with --pass backward on dense, block-sparse, Longformer and index sets: the backward from "
                         "the forward's saved O and statistics (the forward runs once per input set, untimed)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        return 2
    if args.saved_stats and (args.which != "backward" or args.workload not in WORKLOADS
                             or WORKLOADS[args.workload][5]["pattern"] == "sliding"):
        print("bench.py: --saved-stats applies to --pass backward on dense, block_sparse, longformer and "
              "index_set workloads", file=sys.stderr)
        return 2
    if args.workload == "ticks":
        return bench_ticks(args)
    if args.workload == "encoder_layer":
        return bench_encoder(args)

    return bench_attention(args)


def measure(workload: str, which: str = "forward", saved: bool = False, steps: int = 200, warmup=None,
            nsets_arg: int = 0) -> dict:
    """One attention workload on cuda:0: the bench line's fields without the
    CPU baseline and the box copy rate.  Inputs are built here (enough
    rotated sets for > 1 GB, at least 4) and freed before returning."""
    import torch
    import sparse_attention_cuda as ext

    B, H, N, D, dt_name, pk, desc = WORKLOADS[workload]
    bwd = which == "backward"
    dtype = {"bf16": torch.bfloat16, "fp32": torch.float32}[dt_name]
    elt = 2 if dt_name == "bf16" else 4
    dev = torch.device("cuda", 0)

    # tensors touched per step: Q, K, V, O (forward); Q, K, V, dO, dQ, dK, dV (backward; and O from
    # saved statistics)
    tensors = 8 if saved else (7 if bwd else 4)
    set_bytes = tensors * B * N * H * D * elt
    nsets = nsets_arg or max(4, -(-(1 << 30) // set_bytes))
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    sets = []
    for _ in range(nsets):
        ts = [torch.randn(B, N, H, D, device=dev, dtype=torch.float32, generator=gen).to(dtype)
              for _ in range(4 if bwd else 3)]
        sets.append((ts[0], ts[1], ts[2], ts[3] if bwd else None))  # (Q, K, V, dO)

    iset = None  # the IndexSet of the index-set launches
    if bwd and pk["pattern"] == "sliding":
        launch = lambda s: ext.sliding_backward(s[0], s[1], s[2], s[3], pk["left"], pk["right"],
                                                pk.get("dilation", 1))
    elif bwd and pk["pattern"] == "dense":
        if saved:  # each input set's forward output and statistics, as the layer's autograd keeps them
            sets = [s_ + ext.dense_forward(s_[0], s_[1], s_[2], pk["causal"], return_lse=True) for s_ in sets]
            launch = lambda s: ext.dense_backward(s[0], s[1], s[2], s[3], pk["causal"], out=s[4], lse=s[5])
        else:
            launch = lambda s: ext.dense_backward(s[0], s[1], s[2], s[3], pk["causal"])
    elif bwd:
        # block-sparse and explicit sets train on index_set_backward over the
        # pattern's key sets as one IndexSet (built once, as the layer does);
        # Longformer on longformer_backward
        if pk["pattern"] == "index_set":
            offsets, keys = window_csr(N, pk["left"], pk["right"])
            iset = ext.IndexSet(torch.from_numpy(offsets), torch.from_numpy(keys), N, dev)
        elif pk["pattern"] == "block_sparse":
            nb = (N + pk["block_size"] - 1) // pk["block_size"]
            table = ext.BlockTable(ext.make_block_table(pk["seed"], nb, pk["extra"]), N, pk["block_size"], dev)
            iset = ext.pattern_index_set("block_sparse", N, dev, block_table=table, block_size=pk["block_size"])
        else:
            iset = ext.pattern_index_set("longformer", N, dev, left=pk["left"], right=pk["right"],
                                         num_global=pk["num_global"])
        if saved and pk["pattern"] == "longformer":
            # the layer's path: the one-pass Longformer backward from the forward's
            # output and statistics (no key-set description read)
            for n_, s_ in enumerate(sets):
                sets[n_] = s_ + ext.longformer_forward(s_[0], s_[1], s_[2], pk["left"], pk["right"],
                                                       pk["num_global"], return_lse=True)
            iset = None
            launch = lambda s: ext.longformer_backward(s[0], s[1], s[2], s[3], pk["left"], pk["right"],
                                                       pk["num_global"], out=s[4], lse=s[5])
        elif saved:
            # each input set's forward output and statistics, as the layer's autograd keeps them
            for n_, s_ in enumerate(sets):
                if pk["pattern"] == "index_set":
                    o_, l_ = ext.index_set_forward(s_[0], s_[1], s_[2], iset, return_lse=True)
                elif pk["pattern"] == "block_sparse":
                    o_, l_ = ext.block_sparse_forward(s_[0], s_[1], s_[2], table, pk["block_size"], return_lse=True)
                else:
                    o_, l_ = ext.longformer_forward(s_[0], s_[1], s_[2], pk["left"], pk["right"], pk["num_global"],
                                                    return_lse=True)
                sets[n_] = s_ + (o_, l_)
            launch = lambda s: ext.index_set_backward(s[0], s[1], s[2], s[3], iset, out=s[4], lse=s[5])
        elif pk["pattern"] == "longformer":
            # longformer_backward without saved statistics: a forward writing
            # lse and delta, then the one-pass backward (the tiled kernels
            # where the one-pass kernel does not apply), in one span
            iset = None
            launch = lambda s: ext.longformer_backward(s[0], s[1], s[2], s[3], pk["left"], pk["right"],
                                                       pk["num_global"])
        else:
            launch = lambda s: ext.index_set_backward(s[0], s[1], s[2], s[3], iset)
    elif pk["pattern"] == "sliding":
        launch = lambda s: ext.sliding_forward(s[0], s[1], s[2], pk["left"], pk["right"], pk.get("dilation", 1))
    elif pk["pattern"] == "block_sparse":
        nb = (N + pk["block_size"] - 1) // pk["block_size"]
        # checked and copied to the device once, as a model holding a fixed pattern would
        table = ext.BlockTable(ext.make_block_table(pk["seed"], nb, pk["extra"]), N, pk["block_size"], dev)
        launch = lambda s: ext.block_sparse_forward(s[0], s[1], s[2], table, pk["block_size"])
    elif pk["pattern"] == "dense":
        launch = lambda s: ext.dense_forward(s[0], s[1], s[2], pk["causal"])
    elif pk["pattern"] == "index_set":
        offsets, keys = window_csr(N, pk["left"], pk["right"])
        iset = ext.IndexSet(torch.from_numpy(offsets), torch.from_numpy(keys), N, dev)
        launch = lambda s: ext.index_set_forward(s[0], s[1], s[2], iset)
    else:
        launch = lambda s: ext.longformer_forward(s[0], s[1], s[2], pk["left"], pk["right"], pk["num_global"])

    # output buffers come from the caching allocator, so steady-state launches allocate nothing new
    warmup = run_warmup(warmup, lambda i: launch(sets[i % nsets]))
    torch.cuda.synchronize()

    # Timed region: K back-to-back launches on the launch stream between two
    # HIP events; `value` and ms_per_step come from it.
    stream = torch.cuda.current_stream(dev)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(steps):
        launch(sets[i % nsets])
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_per_step = total_ms / steps
    # Kernel durations: K more launches, each stamping its kernels' own start
    # and stop on an event pair (hipExtLaunchKernel through ma_attn_*_timed,
    # stamped on the dispatch packets).  The stamping slows the launch
    # sequence, so it stays out of the region above; the roofline uses these
    # durations.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:  # create the events before they are stamped
        a.record(stream)
        b.record(stream)
    torch.cuda.synchronize()
    for i in range(steps):
        with ext.kernel_events(*ev[i]):
            launch(sets[i % nsets])
    torch.cuda.synchronize()
    per_launch_ms = sorted(a.elapsed_time(b) for a, b in ev)
    mean_launch_ms = sum(per_launch_ms) / len(per_launch_ms)

    # The kernel's access pattern without its arithmetic (ma_attn_copy_probe),
    # timed the same way on the same rotated inputs: the copy speed this
    # pattern reaches on this device.  Sliding windows: the stream kernel's
    # workgroups, tiles and halo blocks; Longformer: the same for its window
    # (the 16 global rows each workgroup also reads are left out); block-sparse:
    # the block-row kernel's workgroups and listed blocks.
    probe_us = None
    probe_src = None
    if not bwd and pk["pattern"] in ("sliding", "longformer", "block_sparse"):
        import ma_attn as _ma
        if pk["pattern"] == "block_sparse":
            pdesc = _ma.make_desc(B, N, H, D, _ma.DTYPES[dtype], _ma.BLOCK_SPARSE, block_size=pk["block_size"],
                                  block_table_ptr=table.tensor.data_ptr(), blocks_per_row=table.width)
            probe_src = "ma_attn_copy_probe (block_row_kernel's workgroups and listed blocks, no arithmetic)"
        else:
            pdesc = _ma.make_desc(B, N, H, D, _ma.DTYPES[dtype], _ma.SLIDING, left=pk["left"], right=pk["right"],
                                  dilation=pk.get("dilation", 1))
            probe_src = ("ma_attn_copy_probe (same workgroups, tiles and halo blocks, no arithmetic)"
                         if pk["pattern"] == "sliding" else
                         "ma_attn_copy_probe (the stream kernel's window pattern without the global rows, "
                         "no arithmetic)")
        pout = torch.empty_like(sets[0][0])
        raw = stream.cuda_stream
        try:
            for i in range(20):
                s_ = sets[i % nsets]
                _ma.copy_probe_raw(pdesc, s_[0].data_ptr(), s_[1].data_ptr(), s_[2].data_ptr(), pout.data_ptr(), raw)
            pev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(steps)]
            for a_, b_ in pev:
                a_.record(stream)
                b_.record(stream)
            torch.cuda.synchronize()
            for i in range(steps):
                s_ = sets[i % nsets]
                _ma.copy_probe_raw(pdesc, s_[0].data_ptr(), s_[1].data_ptr(), s_[2].data_ptr(), pout.data_ptr(), raw,
                                   (pev[i][0].cuda_event, pev[i][1].cuda_event))
            torch.cuda.synchronize()
            probe_us = 1e3 * sum(a_.elapsed_time(b_) for a_, b_ in pev) / len(pev)
        except RuntimeError:
            probe_us = None  # the stream kernel does not take this shape
        del pout
    elif bwd and pk["pattern"] == "sliding" and dt_name != "fp32":
        # the fused backward's workgroups, chunks and steps: K, V, Q, dO rows
        # read and dQ, dK, dV rows written at the kernel's positions
        import ma_attn as _ma
        pdesc = _ma.make_desc(B, N, H, D, _ma.DTYPES[dtype], _ma.SLIDING, left=pk["left"], right=pk["right"],
                              dilation=pk.get("dilation", 1))
        probe_src = "ma_attn_backward_copy_probe (bwd_fused_kernel's workgroups, chunks and steps, no arithmetic)"
        pouts = [torch.empty_like(sets[0][0]) for _ in range(3)]
        raw = stream.cuda_stream

        def bprobe(s_, evs=None):
            _ma.backward_copy_probe_raw(pdesc, *(t_.data_ptr() for t_ in s_[:4]), *(t_.data_ptr() for t_ in pouts),
                                        raw, evs)
        try:
            for i in range(20):
                bprobe(sets[i % nsets])
            pev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(steps)]
            for a_, b_ in pev:
                a_.record(stream)
                b_.record(stream)
            torch.cuda.synchronize()
            for i in range(steps):
                bprobe(sets[i % nsets], (pev[i][0].cuda_event, pev[i][1].cuda_event))
            torch.cuda.synchronize()
            probe_us = 1e3 * sum(a_.elapsed_time(b_) for a_, b_ in pev) / len(pev)
        except RuntimeError:
            probe_us = None  # the fused backward does not take this window
        del pouts

    queries = B * H * N
    alg_bytes = tensors * B * N * H * D * elt + (4 * B * N * H if saved else 0)  # + the statistics read
    set_source = None
    if iset is not None:
        # plus the set's description, read once per pass: the tile plan the
        # kernels read when the set has one (built once on the host), else the
        # key lists (the backward: the set and its transpose)
        if iset.tile_plan is not None:
            alg_bytes += (2 if bwd else 1) * int(iset.tile_header.total_bytes)
            set_source = "tile plan (ma_attn_tile_plan), %d B" % int(iset.tile_header.total_bytes)
        else:
            alg_bytes += (2 if bwd else 1) * (8 * (N + 1) + 4 * key_count(N, pk))
            set_source = "key lists (CSR)"
    # forward: Q.K^T and P.V; backward: S, dP = dO.V^T, dV, dQ, dK (2 FLOP per MAC)
    flops = (10 if bwd else 4) * D * key_count(N, pk) * B * H
    achieved_gbps = alg_bytes / (mean_launch_ms * 1e-3) / 1e9
    tkey = workload + ("_backward_saved" if saved else ("_backward" if bwd else ""))
    traffic = load_traffic(tkey)

    # the bound is whichever peak the algorithmic work reaches first
    mfma_peak = MFMA_BF16_PEAK_TFLOPS if dt_name == "bf16" else MFMA_F32_PEAK_TFLOPS
    tflops = flops / (mean_launch_ms * 1e-3) / 1e12
    # traffic is not measured in this run: it is the committed rocprofv3 counter summary
    tsrc = f"profiles/traffic_{tkey}.txt (rocprofv3 FETCH_SIZE + WRITE_SIZE, committed)" \
        if traffic is not None else None
    if flops / alg_bytes > mfma_peak * 1e12 / (HBM_PEAK_GBPS * 1e9):
        roofline = {"bound": "mfma", "achieved": tflops, "peak": mfma_peak, "unit": "TFLOP/s",
                    "frac": tflops / mfma_peak, "traffic": traffic, "traffic_source": tsrc}
    else:
        roofline = {"bound": "hbm", "achieved": achieved_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": achieved_gbps / HBM_PEAK_GBPS, "traffic": traffic, "traffic_source": tsrc}
    out = {
        "metric": METRIC_BWD if bwd else METRIC,
        "value": queries / (ms_per_step * 1e-3),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt_name,
        "data": f"synthetic N(0,1) inputs, {nsets} rotated input sets resident in HBM",
        "config": {"workload": desc, "batch": B, "heads": H, "seq_len": N, "head_dim": D,
                   **{k_: v_ for k_, v_ in pk.items()}},
        "hbm_gbps": achieved_gbps,
        "hbm_frac_of_peak": achieved_gbps / HBM_PEAK_GBPS,
        "roofline": roofline,
        "kernel_us_mean": mean_launch_ms * 1e3,
        "kernel_us_median": per_launch_ms[len(per_launch_ms) // 2] * 1e3,
        "step_us_mean": ms_per_step * 1e3,
        "algorithmic_bytes_per_launch": alg_bytes,
        "key_set_bytes_counted": set_source,
        "flops_per_launch": flops,
        "tflops": flops / (mean_launch_ms * 1e-3) / 1e12,
        "mfma_bf16_frac_of_peak": (flops / (mean_launch_ms * 1e-3) / 1e12) / MFMA_BF16_PEAK_TFLOPS,
        # rocprofv3 MfmaUtil of the forward kernel (committed summary), not measured in this run
        "mfma_busy_pct": None if bwd else load_mfma_busy(workload),
        "mfma_busy_source": None if bwd else "profiles/mfma_busy_by_workload.md (rocprofv3 MfmaUtil, committed)",
        "device": torch.cuda.get_device_name(dev),
    }
    if probe_us is not None:
        # algorithmic bytes over the probe's mean stamped duration, and the
        # kernel's speed as a fraction of it
        out["pattern_copy"] = {"kernel_us_mean": probe_us,
                               "gbps": ((7 if bwd else 4) * B * N * H * D * elt) / (probe_us * 1e-6) / 1e9,
                               "kernel_frac_of_pattern_copy": probe_us / (mean_launch_ms * 1e3),
                               "source": probe_src}
    if bwd:
        out["pass"] = "backward_saved_statistics" if saved else "backward"
    del sets, launch
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out




# The BASELINE.json configs measured beside the headline in the default run
# (the forward pass of each; cfg2 and cfg5 in both dtypes).
CONFIG_LINES = ("cfg1", "cfg2_fp32", "cfg2_bf16", "cfg3", "cfg4", "cfg5_fp32", "cfg5_bf16")


def config_entry(r: dict) -> dict:
    """The per-config summary kept in the headline line's ``configs``."""
    pc = r.get("pattern_copy")
    traffic = r["roofline"].get("traffic")
    return {
        "workload": r["config"]["workload"], "dtype": r["dtype"],
        "kernel_us_mean": r["kernel_us_mean"], "kernel_us_median": r["kernel_us_median"],
        "step_us_mean": r["step_us_mean"], "queries_per_s": r["value"],
        "hbm_gbps": r["hbm_gbps"], "frac": r["hbm_frac_of_peak"], "tflops": r["tflops"],
        "pattern_copy": None if pc is None else {"kernel_us_mean": pc["kernel_us_mean"],
                                                 "kernel_frac_of_pattern_copy": pc["kernel_frac_of_pattern_copy"]},
        "traffic_ratio": None if traffic is None else traffic / r["algorithmic_bytes_per_launch"],
        "traffic_source": r["roofline"].get("traffic_source"),
        "steps": r["steps"], "warmup": r["warmup"],
    }


def bench_attention(args) -> int:
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    saved = args.which == "backward" and args.saved_stats
    out = measure(args.workload, args.which, saved, args.steps, args.warmup, args.sets)
    with_configs = args.configs if args.configs is not None else (
        args.workload == "target" and args.which == "forward")
    if with_configs:
        # every BASELINE config's forward under the same clock, after the
        # headline, each with its own ~0.1 s warmup and K stamped launches
        t0 = time.perf_counter()
        out["configs"] = {name: config_entry(measure(name, "forward", False, args.steps, None, 0))
                          for name in CONFIG_LINES}
        out["configs_wall_s"] = time.perf_counter() - t0
    out["copy_kernel_gbps"] = copy_bandwidth(dev, torch.cuda.current_stream(dev))
    if not args.no_cpu_baseline and args.which == "forward":
        B, H, N, D, dt_name, pk, _ = WORKLOADS[args.workload]
        out["cpu_baseline"] = cpu_baseline(B, H, N, D, dt_name, pk)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
