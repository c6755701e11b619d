"""Benchmark of the Q4_K decode GEMV hot path at Qwen2-7B shapes on one MI355X.

One step = one decode token's worth of quantized-linear work: for each of 28 layers the q, k, v, o,
gate, up and down projections ([3584,3584], [512,3584] x2, [3584,3584], [18944,3584] x2,
[3584,18944]) plus the lm_head [152064, 3584], all Q4_K with f32 activations (3.98 GB of distinct
packed weights per token, so the 256 MB Infinity Cache cannot hold them).  Per layer this is four
dependent launches, as a decoder issues them: q/k/v together (one launch, they read the same x), o,
gate/up fused with SiLU (the reference's launch_quant_swiglu), and down reading that activation;
then the lm_head.  The step is captured once into a HIP graph (torch.cuda.CUDAGraph) and replayed.
Weights and activations are synthetic and resident in HBM before the timed region.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Prints one JSON line (rank 0).  value = algorithmic GB/s over the timed steps (packed weight bytes
+ f32 x read + f32 y written), tokens_per_s = steps / s.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

LAYERS, HIDDEN, FFN, KV, VOCAB = 28, 3584, 18944, 512, 152064
PEAK_HBM_GBS = 8000.0
Q4_K = 12


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synth_q4k(torch, rows: int, cols: int, gen) -> "torch.Tensor":
    """Random Q4_K matrix [rows, cols]: uniform qs / scale bytes, d and dmin = f16(|N(0,1)| * 0.01)."""
    nsb = cols // 256
    w = torch.randint(0, 256, (rows, nsb, 144), dtype=torch.uint8, device="cuda", generator=gen)
    dd = (torch.randn((rows, nsb, 2), device="cuda", generator=gen).abs() * 0.01).to(torch.float16)
    w[:, :, 0:4] = dd.view(torch.uint8).view(rows, nsb, 4)
    return w.view(-1)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--probe-only", action="store_true",
                    help="only the gate/up SwiGLU kernel, eagerly, plus a 1 GiB copy (for rocprofv3 --pmc passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2

    import torch
    from blog_amd import qlin

    assert torch.cuda.is_available(), "needs the MI355X"
    qlin.lib()
    rb_h, rb_f = qlin.row_bytes(Q4_K, HIDDEN), qlin.row_bytes(Q4_K, FFN)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)

    if args.probe_only:
        return probe_only(torch, qlin, gen, rb_h)

    log("generating synthetic Q4_K weights (28 layers + lm_head)")
    shapes = [("q", HIDDEN, HIDDEN), ("k", KV, HIDDEN), ("v", KV, HIDDEN), ("o", HIDDEN, HIDDEN),
              ("gate", FFN, HIDDEN), ("up", FFN, HIDDEN), ("down", HIDDEN, FFN)]
    layers = [{name: synth_q4k(torch, n, k, gen) for name, n, k in shapes} for _ in range(LAYERS)]
    lm_head = synth_q4k(torch, VOCAB, HIDDEN, gen)
    x_h = torch.randn(HIDDEN, device="cuda", generator=gen)
    x_a = torch.randn(HIDDEN, device="cuda", generator=gen)
    x_f = torch.randn(FFN, device="cuda", generator=gen)
    outs = {name: torch.empty(n, device="cuda") for name, n, _ in shapes}
    act = torch.empty(FFN, device="cuda")
    logits = torch.empty(VOCAB, device="cuda")
    xin = {"q": x_h, "k": x_h, "v": x_h, "o": x_a, "gate": x_h, "up": x_h, "down": x_f}

    # algorithmic bytes: packed weights + f32 inputs read + f32 outputs written, per launch
    per_layer = (sum(layers[0][n].numel() for n in ("q", "k", "v")) + 4 * HIDDEN + 4 * (HIDDEN + 2 * KV)
                 + layers[0]["o"].numel() + 4 * HIDDEN + 4 * HIDDEN
                 + layers[0]["gate"].numel() + layers[0]["up"].numel() + 4 * HIDDEN + 4 * FFN
                 + layers[0]["down"].numel() + 4 * FFN + 4 * HIDDEN)
    bytes_per_step = LAYERS * per_layer + lm_head.numel() + 4 * HIDDEN + 4 * VOCAB
    weight_bytes = sum(t.numel() for L in layers for t in L.values()) + lm_head.numel()
    n_launches = 4 * LAYERS + 1
    log(f"{n_launches} launches per step, {weight_bytes / 1e9:.3f} GB packed weights")

    def step():
        qlin.set_stream(torch.cuda.current_stream())
        for L in layers:
            qlin.quant_gemv_multi(Q4_K, [L["q"], L["k"], L["v"]], rb_h, x_h, [outs["q"], outs["k"], outs["v"]],
                                  [HIDDEN, KV, KV], HIDDEN)
            qlin.quant_gemv(Q4_K, L["o"], rb_h, x_a, outs["o"], HIDDEN, HIDDEN, 1)
            qlin.quant_swiglu(Q4_K, L["gate"], L["up"], rb_h, rb_h, x_h, act, FFN, HIDDEN)
            qlin.quant_gemv(Q4_K, L["down"], rb_f, act, outs["down"], HIDDEN, FFN, 1)
        qlin.quant_gemv(Q4_K, lm_head, rb_h, x_h, logits, VOCAB, HIDDEN, 1)

    # eager warm-up (also initialises the library's per-device state outside capture)
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    ms_per_step = wall / args.steps * 1e3
    gbs = bytes_per_step * args.steps / wall / 1e9
    log(f"{ms_per_step:.4f} ms/step (events {gpu_s / args.steps * 1e3:.4f}), {gbs:.1f} GB/s")

    # ---- roofline probe: the dominant kernel (Q4_K gate/up + SiLU), on its own -------------------
    launch_us, achieved, gate_bytes = roofline_probe(torch, qlin, [(L["gate"], L["up"]) for L in layers], x_h, act,
                                                     rb_h, reps=20, graph=True)
    log(f"gate/up SwiGLU: {launch_us:.2f} us/launch, {achieved:.1f} GB/s")
    traffic = read_traffic()

    result = {
        "metric": "decode GEMV HBM GB/s (% of peak) + tokens/s, Qwen2-7B-shape Q4_K, 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "tokens_per_s": round(args.steps / wall, 1),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random Q4_K blocks, f32 N(0,1) activations)",
        "config": {"workload": "qwen2-7b-q4k-decode-token", "layers": LAYERS, "hidden": HIDDEN, "ffn": FFN,
                   "kv_dim": KV, "vocab": VOCAB, "weight_format": "Q4_K", "batch": 1,
                   "launches_per_step": n_launches, "algorithmic_bytes_per_step": bytes_per_step,
                   "execution": "hip graph replay"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "kernel": "mfma_gemv_kernel<12, true, 1> (Q4_K gate/up SwiGLU, 2 x [18944, 3584])",
                     "avg_launch_us": round(launch_us, 3),
                     "algorithmic_bytes_per_launch": gate_bytes},
    }

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, layers[0], shapes, xin, outs, args.cpu_seconds,
                                              bytes_per_step)
    print(json.dumps(result), flush=True)
    return 0


def roofline_probe(torch, qlin, pairs, x, act, rb, reps, graph):
    """Times launch_quant_swiglu over distinct (gate, up) pairs; returns (us/launch, GB/s, bytes/launch).

    Events are recorded on the stream the kernels run on (the graph's replay stream, or the
    current stream when eager), so the figure is the kernel's own average launch duration."""
    run = lambda: [qlin.quant_swiglu(Q4_K, wg, wu, rb, rb, x, act, FFN, HIDDEN) for wg, wu in pairs]
    qlin.set_stream(torch.cuda.current_stream())
    run()
    torch.cuda.synchronize()
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            qlin.set_stream(torch.cuda.current_stream())
            run()
        qlin.set_stream(torch.cuda.current_stream())
        body = g.replay
    else:
        body = run
    for _ in range(3):
        body()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        body()
    e1.record()
    torch.cuda.synchronize()
    launch_us = e0.elapsed_time(e1) * 1e3 / (reps * len(pairs))
    nbytes = 2 * FFN * qlin.row_bytes(Q4_K, HIDDEN) + 4 * HIDDEN + 4 * FFN
    return launch_us, nbytes / (launch_us * 1e-6) / 1e9, nbytes


def probe_only(torch, qlin, gen, rb_h) -> int:
    """Workload of the --pmc passes: 28 gate/up pairs run eagerly, then a 1 GiB device copy whose
    FETCH_SIZE / WRITE_SIZE calibrate the counters (known 1 GiB read + 1 GiB written)."""
    pairs = [(synth_q4k(torch, FFN, HIDDEN, gen), synth_q4k(torch, FFN, HIDDEN, gen)) for _ in range(LAYERS)]
    x = torch.randn(HIDDEN, device="cuda", generator=gen)
    act = torch.empty(FFN, device="cuda")
    launch_us, gbs, nbytes = roofline_probe(torch, qlin, pairs, x, act, rb_h, reps=2, graph=False)
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"probe: {launch_us:.2f} us/launch (eager, profiled), {nbytes} algorithmic bytes/launch; copy 1 GiB x 2")
    return 0


def read_traffic():
    """HBM bytes per launch of the probe kernel, from the committed rocprofv3 --pmc summary, or None.

    The summary's 'traffic_bytes_per_launch:' line is FETCH_SIZE + WRITE_SIZE of the kernel,
    each divided by what the same counter reads per byte for the 1 GiB copy."""
    path = os.path.join(ROOT, "profiles", "q4k_swiglu_pmc_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def cpu_baseline(torch, layer, shapes, xin, outs, seconds, bytes_per_step):
    """The oracle's f32 GEMV (OpenMP over rows) on this host, over layer 0's seven matrices."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    threads = min(threads, 16)
    mats = []
    for name, n, k in shapes:
        w = layer[name].cpu().numpy()
        x = xin[name].cpu().numpy()
        mats.append((name, w, orc.row_bytes(Q4_K, k), x, n, k))
    # GPU outputs of layer 0 for a parity check of the same inputs
    torch.cuda.synchronize()
    from blog_amd import qlin
    gpu_y = {}
    for name, w_dev, rb, x, n, k in [(nm, layer[nm], orc.row_bytes(Q4_K, k), xin[nm], n, k) for nm, n, k in shapes]:
        y = torch.empty(n, device="cuda")
        qlin.set_stream(torch.cuda.current_stream())
        qlin.quant_gemv(Q4_K, w_dev, rb, x, y, n, k, 1)
        gpu_y[name] = y
    torch.cuda.synchronize()
    layer_bytes = sum(w.size + 4 * k + 4 * n for _, w, _, _, n, k in mats)
    log(f"cpu baseline: oracle f32 GEMV, {threads} threads, ~{seconds:.0f} s")
    worst = 0.0
    passes, t_total = 0, 0.0
    while t_total < seconds:
        for name, w, rb, x, n, k in mats:
            t0 = time.perf_counter()
            y = orc.matmul_f32(Q4_K, w, rb, x, n, k, threads)
            t_total += time.perf_counter() - t0
            if passes == 0:
                g = gpu_y[name].cpu().numpy().astype(np.float64)
                worst = max(worst, float(np.max(np.abs(g - y[0])) / np.max(np.abs(y[0]))))
        passes += 1
    gbs = layer_bytes * passes / t_total / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "tokens_per_s": round(gbs * 1e9 / bytes_per_step, 3),
            "sample": f"layer-0 q,k,v,o,gate,up,down Q4_K GEMVs ({layer_bytes / 1e6:.1f} MB) x {passes} passes, "
                      f"{t_total:.1f} s; oracle orc_matmul_f32 (OpenMP over rows)",
            "gpu_vs_cpu_max_rel_diff": worst}


if __name__ == "__main__":
    sys.exit(main())
