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
import statistics
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
    ap.add_argument("--workload", default="qwen2-7b-q4k-decode-token", choices=sorted(WORKLOADS),
                    help="the headline decode token (default), or one of the other configurations")
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
    if args.workload != "qwen2-7b-q4k-decode-token":
        result = WORKLOADS[args.workload](args, torch, qlin, gen)
        print(json.dumps(result), flush=True)
        return 0

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
                     "kernel": "mfma_gemv_kernel<12, true, 1, false> (Q4_K gate/up SwiGLU, 2 x [18944, 3584])",
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


# ---- the other configurations (C1, C2 and C4, and DeepSeek's Q6_K lm_head) -------------------------
# Each is one JSON line like the headline one: a step is one pass of the configuration's launches
# over synthetic inputs resident in HBM, timed as HIP-graph replays on the launch stream, with the
# distinct weight copies rotated so that the 256 MB Infinity Cache cannot hold them.

BLOCK = {2: (32, 18), 6: (32, 22), 8: (32, 34), 12: (256, 144), 14: (256, 210)}
Q4_0, Q8_0, Q6_K = 2, 8, 14


def synth_blocks(torch, qtype, rows, cols, gen, scale=0.01):
    """Random blocks of any format: uniform bytes, with every f16 scale = f16(|N(0,1)| * scale)."""
    be, bb = BLOCK[qtype]
    nb = cols // be
    w = torch.randint(0, 256, (rows, nb, bb), dtype=torch.uint8, device="cuda", generator=gen)
    nsc = 2 if qtype == Q4_K else 1
    dd = (torch.randn((rows, nb, nsc), device="cuda", generator=gen).abs() * scale).to(torch.float16)
    off = 208 if qtype == Q6_K else 0
    w[:, :, off:off + 2 * nsc] = dd.view(torch.uint8).view(rows, nb, 2 * nsc)
    return w.view(-1)


def graph_us(torch, qlin, fn, reps):
    """Average microseconds of one call of fn, replayed `reps` times from a HIP graph."""
    qlin.set_stream(torch.cuda.current_stream())
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        qlin.set_stream(torch.cuda.current_stream())
        fn()
    qlin.set_stream(torch.cuda.current_stream())
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def graphs_us_interleaved(torch, qlin, fns, reps, rounds=5):
    """Median microseconds of one call of each fn: every fn captured into its own HIP graph, then
    `rounds` rounds of `reps` replays each, the graphs taking turns (alternating order), so that the
    comparison sees the same clocks and cache state."""
    graphs = []
    for fn in fns:
        qlin.set_stream(torch.cuda.current_stream())
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            qlin.set_stream(torch.cuda.current_stream())
            fn()
        qlin.set_stream(torch.cuda.current_stream())
        graphs.append(g)
    times = [[] for _ in fns]
    for rnd in range(rounds):
        order = range(len(graphs)) if rnd % 2 == 0 else reversed(range(len(graphs)))
        for i in order:
            g = graphs[i]
            for _ in range(2):
                g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            times[i].append(e0.elapsed_time(e1) * 1e3 / reps)
    return [statistics.median(t) for t in times]


def cpu_threads():
    """The process's CPU thread share: OMP_NUM_THREADS (16 per GPU job on the GPU boxes), else every
    CPU it may run on."""
    return int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or host_cpu()["cpus_allowed"]


def cpu_gemv_gbs(torch, qtype, w_dev, rb, n, k, seconds):
    """The oracle's f32 GEMV (OpenMP over rows) on one weight copy, repeated for about `seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    threads = cpu_threads()
    w = w_dev.cpu().numpy()
    x = np.random.default_rng(5).standard_normal(k).astype(np.float32)
    nbytes = n * rb + 4 * (n + k)

    def timed(nthreads, budget):
        passes, t = 0, 0.0
        while t < budget or passes == 0:
            t0 = time.perf_counter()
            orc.matmul_f32(qtype, w, rb, x, n, k, nthreads)
            t += time.perf_counter() - t0
            passes += 1
        return nbytes * passes / t / 1e9, passes, t

    gbs, passes, t = timed(threads, seconds)
    gbs1, p1, t1 = timed(1, seconds / 2)
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"[{n}, {k}] type {qtype} GEMV ({nbytes / 1e6:.1f} MB) x {passes} passes, {t:.1f} s; "
                      f"oracle orc_matmul_f32 (OpenMP over rows)",
            "one_thread_gbs": round(gbs1, 3), "one_thread_sample": f"{p1} passes, {t1:.1f} s", **host_cpu()}


def gemv_config(args, torch, qlin, gen, workload, metric, qtype, shapes, copies, scale=0.01):
    """shapes: [(name, rows, cols)] launched in order per step; `copies` distinct sets rotate; block
    scales f16(|N(0,1)| * scale)."""
    sets = [[synth_blocks(torch, qtype, n, k, gen, scale) for _, n, k in shapes] for _ in range(copies)]
    xs = {k: torch.randn(k, device="cuda", generator=gen) for _, _, k in shapes}
    ys = {n: torch.empty(n, device="cuda") for _, n, _ in shapes}
    rbs = [qlin.row_bytes(qtype, k) for _, _, k in shapes]

    def step_all():
        for ws in sets:
            for (name, n, k), w, rb in zip(shapes, ws, rbs):
                qlin.quant_gemv(qtype, w, rb, xs[k], ys[n], n, k, 1)

    reps = max(1, args.steps // copies)
    us_step = graph_us(torch, qlin, step_all, reps) / copies
    step_bytes = sum(n * rb + 4 * (n + k) for (_, n, k), rb in zip(shapes, rbs))
    # the first matrix's kernel alone, as the roofline figure
    _, n0, k0 = shapes[0]
    us0 = graph_us(torch, qlin, lambda: [qlin.quant_gemv(qtype, ws[0], rbs[0], xs[k0], ys[n0], n0, k0, 1)
                                         for ws in sets], reps) / copies
    b0 = n0 * rbs[0] + 4 * (n0 + k0)
    log(f"{workload}: {us_step:.2f} us/step, first matrix {us0:.2f} us")
    result = {
        "metric": metric, "value": round(step_bytes / us_step / 1e3, 1), "unit": "GB/s",
        "pct_of_peak": round(100.0 * step_bytes / us_step / 1e3 / PEAK_HBM_GBS, 2),
        "n_gpus": 1, "steps": reps * copies, "warmup": 3, "ms_per_step": round(us_step / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": f"synthetic (random type-{qtype} blocks, f32 N(0,1) activations), {copies} weight copies rotated",
        "config": {"workload": workload, "weight_format": qtype, "matrices": [[nm, n, k] for nm, n, k in shapes],
                   "batch": 1, "algorithmic_bytes_per_step": step_bytes, "execution": "hip graph replay"},
        "roofline": {"bound": "hbm", "achieved": round(b0 / us0 / 1e3, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(b0 / us0 / 1e3 / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": f"mfma_gemv_kernel<{qtype}, false, *, *> ({shapes[0][0]} [{n0}, {k0}])",
                     "avg_launch_us": round(us0, 3), "algorithmic_bytes_per_launch": b0},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_gemv_gbs(torch, qtype, sets[0][0], rbs[0], n0, k0, args.cpu_seconds)
    return result


def wl_c1(args, torch, qlin, gen):
    return gemv_config(args, torch, qlin, gen, "c1-q8_0-gemv-4096", "Q8_0 GEMV HBM GB/s (4096x4096, batch 1)",
                       Q8_0, [("w", 4096, 4096)], 64)


def wl_c2(args, torch, qlin, gen):
    return gemv_config(args, torch, qlin, gen, "c2-q4_0-ffn-triple",
                       "Q4_0 GEMV triple HBM GB/s (Qwen2-7B FFN gate, up, down; batch 1)", Q4_0,
                       [("gate", 18944, 3584), ("up", 18944, 3584), ("down", 3584, 18944)], 10, scale=0.02)


def wl_q6k(args, torch, qlin, gen):
    return gemv_config(args, torch, qlin, gen, "deepseek-q6_k-lm-head", "Q6_K GEMV HBM GB/s ([102400, 2048], batch 1)",
                       Q6_K, [("lm_head", 102400, 2048)], 6)


def wl_c3(args, torch, qlin, gen):
    """C3: greedy decoding of a random-init Qwen2.5-0.5B-architecture model with every linear in Q8_0
    (blog_amd/decoder.py): a 32-token uniform prompt in one batched pass, then 128 greedy tokens, one
    decode step per token (RMSNorm, q/k/v, rotary + KV store, attention, o, RMSNorm, gate/up SwiGLU,
    down, for 24 layers; final norm, tied Q8_0 head, argmax).  Prefill and decode step are each one
    captured HIP graph; the decode graph reads its token and position from device memory, so 127
    replays after the prefill are the whole generation.  The linear launches alone are timed too."""
    from blog_amd.decoder import Qwen2Config, Qwen2Decoder, make_weights
    cfg = Qwen2Config()
    L, H, KVD, F, V = cfg.layers, cfg.hidden, cfg.kv_dim, cfg.ffn, cfg.vocab
    P, NEW = 32, 128
    log("c3: random-init Q8_0 weights")
    w = make_weights(torch, cfg, seed=2024)
    dec = Qwen2Decoder(torch, cfg, w, max_seq=P + NEW, max_prompt=P)
    prompt = torch.randint(0, V, (P,), dtype=torch.int32, device="cuda", generator=gen)

    def capture(fn):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return g

    g_pre = capture(lambda: dec.prefill(prompt))
    g_step = capture(dec.step)

    def generation():
        g_pre.replay()
        for _ in range(NEW - 1):
            g_step.replay()

    for _ in range(2):
        generation()
    torch.cuda.synchronize()
    reps = max(2, args.steps // 20)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(reps):
        generation()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / reps
    gen_ms = e0.elapsed_time(e1) / reps
    us_pre = graph_replay_us(torch, g_pre, reps)
    us_step = graph_replay_us(torch, g_step, 4 * reps)
    # the quantized linears of one decode step alone (97 launches), and the gate/up SwiGLU launches
    rb_h, rb_f = qlin.row_bytes(Q8_0, H), qlin.row_bytes(Q8_0, F)
    x_h, act = dec.xn[0], dec.act[0]
    yq, yk, yv, yo, logits = (torch.empty(n, device="cuda") for n in (H, KVD, KVD, H, V))

    def linears():
        for W in w["layers"]:
            qlin.quant_gemv_multi(Q8_0, [W["wq"], W["wk"], W["wv"]], rb_h, x_h, [yq, yk, yv], [H, KVD, KVD], H)
            qlin.quant_gemv(Q8_0, W["wo"], rb_h, x_h, yo, H, H, 1)
            qlin.quant_swiglu(Q8_0, W["wg"], W["wu"], rb_h, rb_h, x_h, act, F, H)
            qlin.quant_gemv(Q8_0, W["wd"], rb_f, act, yo, H, F, 1)
        qlin.quant_gemv(Q8_0, w["table"], rb_h, x_h, logits, V, H, 1)

    us_lin = graph_us(torch, qlin, linears, reps)
    us_sw = graph_us(torch, qlin, lambda: [qlin.quant_swiglu(Q8_0, W["wg"], W["wu"], rb_h, rb_h, x_h, act, F, H)
                                           for W in w["layers"]], reps) / L
    sw_bytes = 2 * F * rb_h + 4 * (H + F)
    lin_bytes = L * ((H + 2 * KVD) * rb_h + H * rb_h + 2 * F * rb_h + H * rb_f + 4 * (3 * H + 2 * KVD + 3 * F + 2 * H)) \
        + V * rb_h + 4 * (H + V)
    log(f"c3: {gen_ms:.2f} ms per generation (32-token prompt {us_pre:.0f} us + 127 steps of {us_step:.1f} us), "
        f"{1e6 / us_step:.0f} decode tok/s; linears alone {us_lin:.1f} us/token, SwiGLU {us_sw:.2f} us")
    result = {
        "metric": "greedy decode tokens/s, Qwen2.5-0.5B-arch Q8_0 (32-token prompt + 128 tokens), 1 GPU",
        "value": round(1e6 / us_step, 1), "unit": "tokens/s", "n_gpus": 1, "steps": reps, "warmup": 2,
        "ms_per_step": round(us_step / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (Q8_0 weights)",
        "data": "synthetic (random-init N(0, 0.02) weights quantized to Q8_0; uniform random prompt ids)",
        "config": {"workload": "c3-q8_0-decode-token", "layers": L, "hidden": H, "heads": cfg.n_heads,
                   "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim, "ffn": F, "vocab": V, "weight_format": "Q8_0",
                   "prompt_tokens": P, "new_tokens": NEW, "execution": "hip graph replay (prefill graph + step graph)",
                   "generation_ms": round(gen_ms, 3), "generation_wall_ms": round(wall * 1e3, 3),
                   "prefill_us": round(us_pre, 1), "decode_step_us": round(us_step, 2),
                   "decode_step_hbm_gbs": round(lin_bytes / us_step / 1e3, 1),
                   "linear_only_us_per_token": round(us_lin, 2),
                   "linear_only_tokens_per_s": round(1e6 / us_lin, 1),
                   "linear_algorithmic_bytes_per_token": lin_bytes},
        "roofline": {"bound": "hbm", "achieved": round(sw_bytes / us_sw / 1e3, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(sw_bytes / us_sw / 1e3 / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "mfma_gemv_kernel<8, true, *, *> (Q8_0 gate/up SwiGLU, 2 x [4864, 896])",
                     "avg_launch_us": round(us_sw, 3), "algorithmic_bytes_per_launch": sw_bytes},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_decoder_tps(torch, cfg, w, prompt, args.cpu_seconds)
    return result


def cpu_decoder_tps(torch, cfg, w, prompt, seconds):
    """The oracle's decoder twin (double precision, OpenMP over each matrix's rows) on this host: the
    prompt, then as many new positions as about `seconds` allow, timed per new position."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    def bf16_values(t):
        return (t.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)

    layers = [{n: L[n].cpu().numpy() for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")} |
              {"attn_norm": bf16_values(L["attn_norm"]), "ffn_norm": bf16_values(L["ffn_norm"])} for L in w["layers"]]
    c = dict(layers=cfg.layers, hidden=cfg.hidden, n_heads=cfg.n_heads, kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
             ffn=cfg.ffn, vocab=cfg.vocab, wtype=cfg.wtype, eps=cfg.eps, theta=cfg.theta)
    final, table = bf16_values(w["final_norm"]), w["table"].cpu().numpy()
    threads = cpu_threads()
    toks = prompt.cpu().numpy().tolist()
    P = len(toks)
    # one timed pass with 2 new positions, then one sized to the budget
    t0 = time.perf_counter()
    orc.qwen2_logits(c, layers, final, table, toks + [1, 2], first=P, threads=threads)
    t_small = time.perf_counter() - t0
    n_new = max(2, min(64, int(2 * seconds / max(t_small, 1e-3))))
    t0 = time.perf_counter()
    orc.qwen2_logits(c, layers, final, table, toks + list(range(1, n_new + 1)), first=P, threads=threads)
    t = time.perf_counter() - t0
    per_new = (t - t_small) / (n_new - 2) if n_new > 2 else t / (P + n_new)
    return {"value": round(1.0 / per_new, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle orc_qwen2_logits (double precision, OpenMP over rows): the 32-token prompt plus "
                      f"{n_new} new positions in {t:.1f} s against 2 in {t_small:.1f} s; the difference per position"}


def graph_replay_us(torch, g, reps):
    """Average microseconds of one replay of a captured graph."""
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def wl_c4(args, torch, qlin, gen):
    """C4: Q4_K [14336, 4096] x activations [512, 4096] (f16 N(0,1) values) quantized to Q8_1 on the
    fly, then the matrix-core GEMM; a step is both launches."""
    M, K, N = 512, 4096, 14336
    rb = qlin.row_bytes(Q4_K, K)
    ws = [synth_blocks(torch, Q4_K, N, K, gen) for _ in range(2)]
    x = torch.randn(M, K, device="cuda", generator=gen).half().float()
    xq = torch.empty(M * qlin.lib().qlin_q8_1_row_bytes(K), dtype=torch.uint8, device="cuda")
    y = torch.empty(M, N, device="cuda")

    def step_all():
        for w in ws:
            qlin.quantize_q8_1(x, xq, K, M)
            qlin.quant_matmul_q8_1(Q4_K, w, rb, xq, y, N, K, M)

    reps = max(10, args.steps // 2)  # one replay is 2 launches of ~150 us: time enough of them
    us_step = graph_us(torch, qlin, step_all, reps) / len(ws)
    us_gemm = graph_us(torch, qlin, lambda: [qlin.quant_matmul_q8_1(Q4_K, w, rb, xq, y, N, K, M) for w in ws],
                       reps) / len(ws)
    flops = 2.0 * M * N * K
    log(f"c4: {us_step:.2f} us/step, GEMM {us_gemm:.2f} us")
    result = {
        "metric": "Q4_K x Q8_1 prefill GEMM TFLOP/s (M=512, K=4096, N=14336)",
        "value": round(flops / us_step / 1e6, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": reps * len(ws),
        "warmup": 3, "ms_per_step": round(us_step / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 (Q8_1 integers qx) x f16 (integers sc*q), f32 block sums scaled by d8",
        "data": "synthetic (random Q4_K blocks; activations f16-rounded N(0,1) quantized to Q8_1 in the step)",
        "config": {"workload": "c4-q4k-prefill-gemm", "m": M, "k": K, "n": N, "weight_format": "Q4_K",
                   "activation_format": "Q8_1", "algorithmic_flops_per_step": flops,
                   "launches_per_step": ["quantize_q8_1", "quant_matmul_q8_1"], "execution": "hip graph replay"},
        "roofline": {"bound": "mfma", "achieved": round(flops / us_gemm / 1e6, 1), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(flops / us_gemm / 1e6 / 2500.0, 4), "traffic": None,
                     "kernel": "q4k_gemm_kernel (fp16 MFMA 16x16x32; peak = dense fp16)",
                     "avg_launch_us": round(us_gemm, 3), "algorithmic_flops_per_launch": flops},
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        rows = 64
        w = ws[0].view(N, -1)[:rows].contiguous().view(-1).cpu().numpy()
        xh = x.cpu().numpy()
        xqh = orc.quantize_q8_1(xh, K)
        threads = cpu_threads()
        ps, p, t, ps1, p1, t1 = cpu_timed(lambda nt: orc.matmul_q8_1(Q4_K, w, rb, xqh, rows, K, M, threads=nt),
                                          threads, args.cpu_seconds)
        f = 2.0 * M * rows * K
        result["cpu_baseline"] = {
            "value": round(f * ps / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of the {N} weight rows x {M} tokens x {K}, {p} passes, {t:.1f} s; oracle "
                      f"orc_matmul_q8_1 (reference block-dot order, f64; OpenMP over rows)",
            "one_thread_tflops": round(f * ps1 / 1e12, 5), "one_thread_sample": f"{p1} passes, {t1:.1f} s",
            **host_cpu()}
    return result


def wl_prefill(args, torch, qlin, gen):
    """The 32-block and Q6_K formats' matrix-core prefill GEMM (Q8_1 activations, 512 tokens, f16
    N(0,1) values quantized in the step): DeepSeek-V2-Lite's Q6_K lm_head [102400, 2048] is the
    headline; its Q5_0 expert down [2048, 1408] and a Qwen2.5-0.5B Q8_0 gate [4864, 896] are timed
    alongside.  A step is quantize_q8_1 then the GEMM."""
    M = 512
    Q5_0 = 6
    shapes = [("lm_head", Q6_K, 102400, 2048), ("expert_down", Q5_0, 2048, 1408), ("ffn_gate", Q8_0, 4864, 896)]
    res = {}
    for name, qt, N, K in shapes:
        rb = qlin.row_bytes(qt, K)
        w = synth_blocks(torch, qt, N, K, gen)
        x = torch.randn(M, K, device="cuda", generator=gen).half().float()
        xq = torch.empty(M * qlin.lib().qlin_q8_1_row_bytes(K), dtype=torch.uint8, device="cuda")
        y = torch.empty(M, N, device="cuda")

        def step(qt=qt, w=w, rb=rb, x=x, xq=xq, y=y, N=N, K=K):
            qlin.quantize_q8_1(x, xq, K, M)
            qlin.quant_matmul_q8_1(qt, w, rb, xq, y, N, K, M)

        reps = max(10, args.steps // 2)
        us_step = graph_us(torch, qlin, step, reps)
        us_gemm = graph_us(torch, qlin, lambda qt=qt, w=w, rb=rb, xq=xq, y=y, N=N, K=K:
                           qlin.quant_matmul_q8_1(qt, w, rb, xq, y, N, K, M), reps)
        flops = 2.0 * M * N * K
        res[name] = {"type": qt, "n": N, "k": K, "us_step": round(us_step, 2), "us_gemm": round(us_gemm, 2),
                     "tflops_gemm": round(flops / us_gemm / 1e6, 1)}
        log(f"prefill {name}: {us_step:.2f} us/step, GEMM {us_gemm:.2f} us ({flops / us_gemm / 1e6:.1f} TFLOP/s)")
        if name == "lm_head":
            head = (w, rb, x, N, K, us_step, us_gemm, flops)
    w, rb, x, N, K, us_step, us_gemm, flops = head
    result = {
        "metric": "Q6_K x Q8_1 prefill GEMM TFLOP/s (DeepSeek-V2-Lite lm_head [102400, 2048], M=512)",
        "value": round(flops / us_step / 1e6, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": max(10, args.steps // 2),
        "warmup": 3, "ms_per_step": round(us_step / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (Q8_1 integers qx) x f16 (sc*(q-32) as two exact parts), f32 block sums scaled by d*d8",
        "data": "synthetic (random Q6_K / Q5_0 / Q8_0 blocks; activations f16-rounded N(0,1) quantized to Q8_1 "
                "in the step)",
        "config": {"workload": "deepseek-prefill-gemm", "m": M, "k": K, "n": N, "weight_format": "Q6_K",
                   "activation_format": "Q8_1", "algorithmic_flops_per_step": flops,
                   "launches_per_step": ["quantize_q8_1", "quant_matmul_q8_1"], "execution": "hip graph replay",
                   "shapes": res},
        "roofline": {"bound": "mfma", "achieved": round(flops / us_gemm / 1e6, 1), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(flops / us_gemm / 1e6 / 2500.0, 4), "traffic": None,
                     "kernel": "q6k_gemm_kernel (fp16 MFMA 16x16x32, two per block; peak = dense fp16)",
                     "avg_launch_us": round(us_gemm, 3), "algorithmic_flops_per_launch": flops},
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        rows = 64
        wh = w.view(N, -1)[:rows].contiguous().view(-1).cpu().numpy()
        xqh = orc.quantize_q8_1(x.cpu().numpy(), K)
        threads = cpu_threads()
        ps, p, t, ps1, p1, t1 = cpu_timed(lambda nt: orc.matmul_q8_1(Q6_K, wh, rb, xqh, rows, K, M, threads=nt),
                                          threads, args.cpu_seconds)
        f = 2.0 * M * rows * K
        result["cpu_baseline"] = {
            "value": round(f * ps / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of the {N} weight rows x {M} tokens x {K}, {p} passes, {t:.1f} s; oracle "
                      f"orc_matmul_q8_1 (reference block-dot order, f64; OpenMP over rows)",
            "one_thread_tflops": round(f * ps1 / 1e12, 5), "one_thread_sample": f"{p1} passes, {t1:.1f} s",
            **host_cpu()}
    return result


def cpu_timed(fn, threads, seconds):
    """Calls fn(nthreads) for about `seconds` on the process's thread share and for half as long on one
    thread; returns (passes/s on the share, passes, s, passes/s on one thread, passes, s)."""
    def timed(nthreads, budget):
        passes, t = 0, 0.0
        while t < budget or passes == 0:
            t0 = time.perf_counter()
            fn(nthreads)
            t += time.perf_counter() - t0
            passes += 1
        return passes / t, passes, t
    return (*timed(threads, seconds), *timed(1, seconds / 2))


def wl_prefill_f32(args, torch, qlin, gen):
    """The prefill entry the engine calls (TensorTool::quant_direct_gemm -> launch_quant_matmul, f32
    activations, TensorTool.cpp:163-168, kernel.cu:1254-1279): Q4_K [14336, 4096] x [512, 4096] (the
    headline) and DeepSeek-V2-Lite's Q6_K lm_head [102400, 2048] x [512, 2048], N(0,1) f32 activations.
    A step is one qlin_launch_quant_matmul; two weight copies are rotated.  Also timed: the Q4_K matrix
    at a short prompt's 64 tokens (the launch then takes the small workgroup geometry)."""
    M = 512
    shapes = [("q4k_mlp", Q4_K, 14336, 4096, M), ("q6k_lm_head", Q6_K, 102400, 2048, M),
              ("q4k_mlp_64_tokens", Q4_K, 14336, 4096, 64)]
    res, head = {}, None
    for name, qt, N, K, M in shapes:
        rb = qlin.row_bytes(qt, K)
        ws = [synth_blocks(torch, qt, N, K, gen) for _ in range(2)]
        x = torch.randn(M, K, device="cuda", generator=gen)
        y = torch.empty(M, N, device="cuda")
        reps = max(10, args.steps // 4)
        us = graph_us(torch, qlin, lambda qt=qt, ws=ws, rb=rb, x=x, y=y, N=N, K=K:
                      [qlin.quant_matmul(qt, w, rb, x, y, N, K, M) for w in ws], reps) / len(ws)
        flops = 2.0 * M * N * K
        res[name] = {"type": qt, "m": M, "n": N, "k": K, "us": round(us, 2), "tflops": round(flops / us / 1e6, 1)}
        log(f"prefill f32 {name}: {us:.2f} us ({flops / us / 1e6:.1f} TFLOP/s)")
        if head is None:
            head = (qt, ws[0], rb, x, N, K, M, us, flops, reps)
    qt, w, rb, x, N, K, M, us, flops, reps = head
    result = {
        "metric": "Q4_K x f32 prefill GEMM TFLOP/s (launch_quant_matmul, M=512, K=4096, N=14336)",
        "value": round(flops / us / 1e6, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": reps * 2, "warmup": 3,
        "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 (x 2^s as hi + lo parts) x f16 (integers sc*q), f32 accumulation",
        "data": "synthetic (random Q4_K / Q6_K blocks; f32 N(0,1) activations)",
        "config": {"workload": "prefill-f32-gemm", "m": M, "k": K, "n": N, "weight_format": "Q4_K",
                   "activation_format": "f32", "algorithmic_flops_per_step": flops,
                   "launches_per_step": ["quant_matmul"], "execution": "hip graph replay", "shapes": res},
        "roofline": {"bound": "mfma", "achieved": round(flops / us / 1e6, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(flops / us / 1e6 / 2500.0, 4), "traffic": None,
                     "kernel": "f32_gemm_kernel<12> (fp16 MFMA 16x16x32, two per block; peak = dense fp16)",
                     "avg_launch_us": round(us, 3), "algorithmic_flops_per_launch": flops},
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        rows, toks = 64, 64
        wh = w.view(N, -1)[:rows].contiguous().view(-1).cpu().numpy()
        xh = np.ascontiguousarray(x[:toks].cpu().numpy())
        threads = cpu_threads()
        ps, p, t, ps1, p1, t1 = cpu_timed(lambda nt: orc.matmul_f32(qt, wh, rb, xh, rows, K, nt), threads,
                                          args.cpu_seconds)
        f = 2.0 * rows * toks * K
        result["cpu_baseline"] = {
            "value": round(f * ps / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of the {N} weight rows x {toks} of the {M} tokens x {K}, {p} passes, {t:.1f} s; "
                      f"oracle orc_matmul_f32 (the reference's f32 dot per (token, row), OpenMP over rows)",
            "one_thread_tflops": round(f * ps1 / 1e12, 5), "one_thread_sample": f"{p1} passes, {t1:.1f} s",
            **host_cpu()}
    return result


def wl_c5(args, torch, qlin, gen):
    """C5: a DeepSeek-V2-Lite MoE FFN layer for 16 decode tokens -- 64 routed experts of Q4_K gate/up
    [1408, 2048] and Q5_0 down [2048, 1408], router logits N(0,1), top-6 with scaling 1.0, plus the 2
    shared experts (Q4_K gate/up [2816, 2048], Q4_K down [2048, 2816]).  A step is the router, the
    grouped routed decode and the shared experts (MoE.cpp:29-52 after the norm): the batched SwiGLU
    over the 16 tokens, then the batched down projection added into the same output."""
    E, ffn, hid, tokens, k = 64, 1408, 2048, 16, 6
    sffn = 2816
    Q5_0 = 6
    copies = 4  # 4 x 339 MB of expert weights rotate through the step
    mats = [(synth_blocks(torch, Q4_K, E * ffn, hid, gen), synth_blocks(torch, Q4_K, E * ffn, hid, gen),
             synth_blocks(torch, Q5_0, E * hid, ffn, gen), synth_blocks(torch, Q4_K, sffn, hid, gen),
             synth_blocks(torch, Q4_K, sffn, hid, gen), synth_blocks(torch, Q4_K, hid, sffn, gen))
            for _ in range(copies)]
    x = torch.randn(tokens, hid, device="cuda", generator=gen)
    logits = torch.randn(tokens, E, device="cuda", generator=gen)
    ids = torch.empty(tokens, k, dtype=torch.int32, device="cuda")
    rw = torch.empty(tokens, k, device="cuda")
    out = torch.zeros(tokens, hid, device="cuda")
    nws = qlin.lib().qlin_moe_ffn_workspace_bytes(tokens, k, E, ffn, hid, sffn)
    ws = torch.empty(nws + 256, dtype=torch.uint8, device="cuda")
    wsp = (ws.data_ptr() + 255) // 256 * 256
    act = torch.empty(k * ffn + sffn, device="cuda")
    sacts = torch.empty(tokens, sffn, device="cuda")
    gub, db = mats[0][0].numel(), mats[0][2].numel()
    s_rb, sd_rb = qlin.row_bytes(Q4_K, hid), qlin.row_bytes(Q4_K, sffn)

    def step_grouped():
        for wg, wu, wd, sg, su, sd in mats:
            # the whole FFN in one call: the routing and the shared SwiGLU run in the routed gate/up launch,
            # and the shared down-add launch also adds the routed sum (no combine launch)
            qlin.call("qlin_moe_ffn_decode_grouped_logits", Q4_K, wg, wu, gub, Q5_0, wd, db, E, ffn, hid, hid, Q4_K, sg,
                      su, s_rb, sd, sd_rb, sffn, x, logits, 1.0, ids, rw, wsp, nws, out, tokens, k)

    def step_three_calls():
        for wg, wu, wd, sg, su, sd in mats:
            qlin.call("qlin_moe_routed_decode_grouped_logits", Q4_K, wg, wu, gub, Q5_0, wd, db, E, ffn, hid, hid, x,
                      logits, 1.0, ids, rw, wsp, nws, out, tokens, k)
            qlin.call("qlin_launch_quant_swiglu_rows", Q4_K, sg, su, s_rb, s_rb, x, sacts, sffn, hid, tokens)
            qlin.call("qlin_launch_quant_matmul_add", Q4_K, sd, sd_rb, sacts, out, hid, sffn, tokens)

    def step_per_token():
        # each token's whole FFN in the per-token call: routing, routed and shared SwiGLU in one launch,
        # routed down, shared down-add
        for wg, wu, wd, sg, su, sd in mats:
            for t in range(tokens):
                qlin.call("qlin_moe_ffn_decode_indexed_logits", Q4_K, wg, wu, gub, Q5_0, wd, db, E, ffn, hid, hid,
                          Q4_K, sg, su, s_rb, sd, sd_rb, sffn, x[t], logits[t], 1.0, ids[t], rw[t], act, out[t], k)

    reps = max(5, args.steps // 4)
    us, us_three = (v / copies for v in graphs_us_interleaved(torch, qlin, [step_grouped, step_three_calls], reps))
    us_tok = graph_us(torch, qlin, step_per_token, max(1, reps // 4)) / copies
    distinct = int(torch.unique(ids[ids >= 0]).numel())
    per_expert = 2 * ffn * qlin.row_bytes(Q4_K, hid) + hid * qlin.row_bytes(Q5_0, ffn)
    shared = 2 * sffn * s_rb + hid * sd_rb
    nbytes = distinct * per_expert + shared + 4 * tokens * (hid + hid) + 4 * tokens * E
    log(f"c5: grouped {us:.2f} us/step (three calls {us_three:.2f} us), per-token facade {us_tok:.2f} us, "
        f"{distinct} distinct experts")
    result = {
        "metric": "MoE layer decode HBM GB/s (DeepSeek-V2-Lite shape, 16 tokens, top-6 of 64 + 2 shared)",
        "value": round(nbytes / us / 1e3, 1), "unit": "GB/s", "pct_of_peak": round(100 * nbytes / us / 1e3 / PEAK_HBM_GBS, 2),
        "n_gpus": 1, "steps": 5 * reps * copies, "warmup": 10 * copies, "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random Q4_K / Q5_0 expert blocks, f32 N(0,1) x and router logits), 4 weight copies",
        "config": {"workload": "c5-moe-grouped", "experts": E, "ffn": ffn, "hidden": hid, "tokens": tokens,
                   "top_k": k, "gate_up": "Q4_K", "down": "Q5_0", "shared_ffn": sffn, "shared": "Q4_K",
                   "distinct_experts": distinct, "algorithmic_bytes_per_step": nbytes,
                   "launches_per_step": "moe_ffn_decode_grouped_logits: stream gate/up with the routing, the "
                                        "grouping and the shared SwiGLU tiles, stream down, shared down-add with "
                                        "the routed combine (3 launches)",
                   "three_calls_us_per_step": round(us_three, 2),
                   "per_token_facade_us_per_step": round(us_tok, 2), "execution": "hip graph replay"},
        "roofline": {"bound": "hbm", "achieved": round(nbytes / us / 1e3, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "whole step (stream_kernel<Q4_K> gate/up with the router, the grouping and "
                               "the shared SwiGLU tiles, stream_kernel<Q5_0> down, q4k_dense_kernel add with "
                               "the routed combine)",
                     "avg_launch_us": round(us, 3), "algorithmic_bytes_per_launch": nbytes},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_moe_gbs(torch, mats[0], x, ids, rw, E, ffn, hid, k, args.cpu_seconds)
    return result


def cpu_moe_gbs(torch, mats, x, ids, rw, E, ffn, hid, k, seconds):
    """The oracle's per-token routed MoE (orc_swiglu_indexed, then orc_down_indexed_ordered, double-
    precision sums) over the batch's tokens for about `seconds`: on the process's thread share (one
    token per thread at a time; the oracle's calls release the interpreter) and on one thread.  GB/s of
    the expert bytes that each token's routes read."""
    import concurrent.futures as cf
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    wg, wu, wd = (t.cpu().numpy() for t in mats[:3])
    geb, deb = wg.size // E, wd.size // E
    grb, drb = geb // ffn, deb // hid
    xs, idh, rwh = x.cpu().numpy(), ids.cpu().numpy(), rw.cpu().numpy()
    per_token = k * (2 * geb + deb)

    def token(i):
        out = np.zeros(hid, np.float32)
        act = orc.swiglu_indexed(Q4_K, wg, wu, geb, geb, grb, grb, xs[i], idh[i], ffn, hid)
        orc.down_indexed_ordered(6, wd, deb, drb, act, idh[i], rwh[i], out, hid, ffn)

    def timed(nthreads, budget):
        tokens, t = 0, 0.0
        with cf.ThreadPoolExecutor(max_workers=nthreads) as ex:
            while t < budget or tokens == 0:
                batch = [(tokens + j) % xs.shape[0] for j in range(nthreads)]
                t0 = time.perf_counter()
                list(ex.map(token, batch))
                t += time.perf_counter() - t0
                tokens += nthreads
        return tokens, t

    threads = cpu_threads()
    tokens, t = timed(threads, seconds)
    tokens1, t1 = timed(1, seconds / 2)
    return {"value": round(per_token * tokens / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "tokens_per_s": round(tokens / t, 2),
            "sample": f"{tokens} tokens' routed experts ({per_token / 1e6:.1f} MB each), {t:.1f} s, {threads} "
                      f"tokens at a time; oracle orc_swiglu_indexed + orc_down_indexed_ordered",
            "one_thread_gbs": round(per_token * tokens1 / t1 / 1e9, 3),
            "one_thread_sample": f"{tokens1} tokens, {t1:.1f} s", **host_cpu()}


def wl_moe_token(args, torch, qlin, gen):
    """The engine's per-token routed MoE (TensorTool::moe_routed_decode_indexed, TensorTool.cpp:271-336)
    at DeepSeek-V2-Lite's shape: one decode token's router (top-6 of 64), then
    qlin_moe_routed_decode_indexed -- the 6 routes' Q4_K gate/up SwiGLU [1408, 2048] and their Q5_0 down
    [2048, 1408] added in route order.  A step is one token; 4 copies of the 64 experts (4 x 334 MB)
    rotate, each with its own router logits."""
    E, ffn, hid, k = 64, 1408, 2048, 6
    Q5_0 = 6
    copies = 4
    mats = [(synth_blocks(torch, Q4_K, E * ffn, hid, gen), synth_blocks(torch, Q4_K, E * ffn, hid, gen),
             synth_blocks(torch, Q5_0, E * hid, ffn, gen)) for _ in range(copies)]
    x = torch.randn(hid, device="cuda", generator=gen)
    logits = torch.randn(copies, E, device="cuda", generator=gen)
    ids = torch.empty(copies, k, dtype=torch.int32, device="cuda")
    rw = torch.empty(copies, k, device="cuda")
    act = torch.empty(k, ffn, device="cuda")
    out = torch.zeros(hid, device="cuda")
    gub, db = mats[0][0].numel(), mats[0][2].numel()
    g_rb, d_rb = qlin.row_bytes(Q4_K, hid), qlin.row_bytes(Q5_0, ffn)

    def route():
        for c in range(copies):
            qlin.call("qlin_launch_moe_router_topk", logits[c], ids[c], rw[c], 1, E, k, 1.0)

    def step():
        for c, (wg, wu, wd) in enumerate(mats):
            # the router's picks and the routed decode in one call (the routing runs in the routed
            # gate/up launch)
            qlin.call("qlin_moe_routed_decode_indexed_logits", Q4_K, wg, wu, gub, Q5_0, wd, db, E, ffn, hid, hid, x,
                      logits[c], 1.0, ids[c], rw[c], act, out, k)

    def swiglu_only():
        for c, (wg, wu, _) in enumerate(mats):
            qlin.call("qlin_launch_quant_swiglu_indexed", Q4_K, wg, wu, gub // E, gub // E, g_rb, g_rb, x, ids[c],
                      act, k, ffn, hid)

    def down_only():
        for c, (_, _, wd) in enumerate(mats):
            qlin.call("qlin_launch_quant_down_f32_indexed_accum_ordered", Q5_0, wd, db // E, d_rb, act, ids[c], rw[c],
                      out, k, hid, ffn)

    # the whole MoE FFN of a token: the routed experts plus the 2 shared experts (Q4_K gate/up
    # [2816, 2048], Q4_K down [2048, 2816]), in one call or as the separate calls
    sffn = 2816
    shared = [(synth_blocks(torch, Q4_K, sffn, hid, gen), synth_blocks(torch, Q4_K, sffn, hid, gen),
               synth_blocks(torch, Q4_K, hid, sffn, gen)) for _ in range(copies)]
    s_rb, sd_rb = qlin.row_bytes(Q4_K, hid), qlin.row_bytes(Q4_K, sffn)
    act_f = torch.empty(k * ffn + sffn, device="cuda")

    def ffn_call():
        for c, ((wg, wu, wd), (sg, su, sd)) in enumerate(zip(mats, shared)):
            qlin.call("qlin_moe_ffn_decode_indexed_logits", Q4_K, wg, wu, gub, Q5_0, wd, db, E, ffn, hid, hid, Q4_K,
                      sg, su, s_rb, sd, sd_rb, sffn, x, logits[c], 1.0, ids[c], rw[c], act_f, out, k)

    def ffn_separate():
        for c, ((wg, wu, wd), (sg, su, sd)) in enumerate(zip(mats, shared)):
            qlin.call("qlin_moe_routed_decode_indexed_logits", Q4_K, wg, wu, gub, Q5_0, wd, db, E, ffn, hid, hid, x,
                      logits[c], 1.0, ids[c], rw[c], act, out, k)
            qlin.quant_swiglu(Q4_K, sg, su, s_rb, s_rb, x, act_f[k * ffn:], sffn, hid)
            qlin.quant_gemv_add(Q4_K, sd, sd_rb, act_f[k * ffn:], out, hid, sffn)

    reps = max(1, args.steps // 4)
    us = graph_us(torch, qlin, step, reps) / copies
    us_ffn, us_ffn3 = (t / copies for t in graphs_us_interleaved(torch, qlin, [ffn_call, ffn_separate], reps))
    route()
    torch.cuda.synchronize()
    us_sw = graph_us(torch, qlin, swiglu_only, reps) / copies
    us_dn = graph_us(torch, qlin, down_only, reps) / copies
    distinct = min(int(torch.unique(ids[c][ids[c] >= 0]).numel()) for c in range(copies))
    sw_bytes = k * 2 * ffn * g_rb + 4 * hid + 4 * k * ffn
    dn_bytes = k * hid * d_rb + 4 * k * ffn + 8 * hid
    nbytes = sw_bytes + dn_bytes + 4 * E
    ffn_bytes = nbytes + 2 * sffn * s_rb + hid * sd_rb + 8 * sffn
    log(f"moe token: {us:.2f} us/token (router + routed decode), SwiGLU {us_sw:.2f} us, down {us_dn:.2f} us, "
        f"{distinct} distinct experts per token at least")
    log(f"moe ffn token (routed + shared): {us_ffn:.2f} us in one call ({ffn_bytes / us_ffn / 1e3:.0f} GB/s), "
        f"{us_ffn3:.2f} us as the separate calls")
    result = {
        "metric": "per-token routed MoE decode HBM GB/s (DeepSeek-V2-Lite shape, top-6 of 64, 1 token)",
        "value": round(nbytes / us / 1e3, 1), "unit": "GB/s", "pct_of_peak": round(100 * nbytes / us / 1e3 / PEAK_HBM_GBS, 2),
        "n_gpus": 1, "steps": reps * copies, "warmup": 3, "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random Q4_K / Q5_0 expert blocks, f32 N(0,1) x and router logits), 4 weight copies",
        "config": {"workload": "deepseek-moe-token", "experts": E, "ffn": ffn, "hidden": hid, "top_k": k,
                   "gate_up": "Q4_K", "down": "Q5_0", "algorithmic_bytes_per_step": nbytes,
                   "launches_per_step": "moe_routed_decode_indexed_logits (routed SwiGLU with the routing, "
                                        "routed down)",
                   "swiglu_us": round(us_sw, 3), "down_us": round(us_dn, 3), "execution": "hip graph replay",
                   "ffn_token_us": round(us_ffn, 3), "ffn_token_separate_calls_us": round(us_ffn3, 3),
                   "ffn_token_bytes": ffn_bytes,
                   "ffn_token": "qlin_moe_ffn_decode_indexed_logits with the 2 shared experts (Q4_K [2816, 2048] "
                                "gate/up, [2048, 2816] down): 3 launches; separate calls: 4"},
        "roofline": {"bound": "hbm", "achieved": round(sw_bytes / us_sw / 1e3, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(sw_bytes / us_sw / 1e3 / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "mfma_gemv_kernel<12, true, 1, true> (routed gate/up SwiGLU, 6 x 2 x [1408, 2048])",
                     "avg_launch_us": round(us_sw, 3), "algorithmic_bytes_per_launch": sw_bytes},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_moe_gbs(torch, mats[0], x.view(1, hid), ids[0:1], rw[0:1], E, ffn, hid, k,
                                             args.cpu_seconds)
    return result


WORKLOADS = {"qwen2-7b-q4k-decode-token": None, "c5-moe-grouped": wl_c5, "c1-q8_0-gemv-4096": wl_c1, "c2-q4_0-ffn-triple": wl_c2,
             "c3-q8_0-decode-token": wl_c3, "c4-q4k-prefill-gemm": wl_c4, "deepseek-q6_k-lm-head": wl_q6k,
             "deepseek-moe-token": wl_moe_token, "deepseek-prefill-gemm": wl_prefill,
             "prefill-f32-gemm": wl_prefill_f32}


def host_cpu() -> dict:
    """The host's CPU model, its logical CPU count, and the CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count() or 1
    return {"cpu_model": model, "nproc": os.cpu_count() or 1, "cpus_allowed": allowed}


def cpu_baseline(torch, layer, shapes, xin, outs, seconds, bytes_per_step):
    """The oracle's GEMV on this host over layer 0's seven matrices: the f32 variant (OpenMP over rows)
    on one thread and on the process's thread share (OMP_NUM_THREADS, else every allowed CPU; the GPU
    boxes give one GPU's job 16), and the double-precision variant on one thread, each for a bounded
    time.  value is the f32 figure on the thread share."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    info = host_cpu()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or info["cpus_allowed"]
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

    def timed(fn, budget):
        passes, t_total = 0, 0.0
        while t_total < budget or passes == 0:
            for name, w, rb, x, n, k in mats:
                t0 = time.perf_counter()
                fn(w, rb, x, n, k)
                t_total += time.perf_counter() - t0
            passes += 1
        return layer_bytes * passes / t_total / 1e9, passes, t_total

    log(f"cpu baseline: oracle f32 GEMV, {threads} threads and 1 thread, f64 on 1 thread ({info['cpu_model']})")
    worst = 0.0
    for name, w, rb, x, n, k in mats:
        y = orc.matmul_f32(Q4_K, w, rb, x, n, k, threads)
        g = gpu_y[name].cpu().numpy().astype(np.float64)
        worst = max(worst, float(np.max(np.abs(g - y[0])) / np.max(np.abs(y[0]))))
    gbs, passes, t_total = timed(lambda w, rb, x, n, k: orc.matmul_f32(Q4_K, w, rb, x, n, k, threads), seconds)
    gbs1, p1, t1 = timed(lambda w, rb, x, n, k: orc.matmul_f32(Q4_K, w, rb, x, n, k, 1), seconds / 2)
    gbs64, p64, t64 = timed(lambda w, rb, x, n, k: orc.matmul_f64(Q4_K, w, rb, x, n, k), seconds / 2)
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "tokens_per_s": round(gbs * 1e9 / bytes_per_step, 3),
            "sample": f"layer-0 q,k,v,o,gate,up,down Q4_K GEMVs ({layer_bytes / 1e6:.1f} MB) x {passes} passes, "
                      f"{t_total:.1f} s; oracle orc_matmul_f32 (OpenMP over rows)",
            "one_thread_gbs": round(gbs1, 3), "one_thread_sample": f"{p1} passes, {t1:.1f} s",
            "f64_one_thread_gbs": round(gbs64, 3), "f64_sample": f"orc_matmul_f64, {p64} passes, {t64:.1f} s",
            **info, "gpu_vs_cpu_max_rel_diff": worst}


if __name__ == "__main__":
    sys.exit(main())
