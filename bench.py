"""Benchmark: Qwen3-Next-80B-A3B sparse-MoE layer on one MI355X.

Headline (the JSON `value`): C2 -- one MoE-layer decode step (T=1, hidden 2048,
512 experts, top-10 renormalised, intermediate 512, shared expert 512 with its
sigmoid gate; experts and shared expert GGUF Q8_0 from seeded N(0,0.02), router
and shared gate bf16, activations bf16 N(0,1)), in microseconds per layer.

Method
  * L distinct layers (default 16, each its own 1.7 GB Q8_0 expert stack) are
    generated on the device and rotated, with a different token per step, so
    the ~37 MB a step touches is never still resident in the 256 MB Infinity
    Cache when that layer comes round again.
  * The steps are captured into one HIP graph (the library launches three
    kernels per decode step on the capturing stream) and the graph is replayed:
    warm-up replays (at least --warmup steps and at least 20 ms of replays, past
    the card's clock transient), then HIP events on the replay stream around
    exactly K steps queued right behind them (`value`); `wall_us` is the host
    clock around the same K steps with torch.cuda.synchronize() on both sides.
  * Kernel durations for the roofline come from HIP events the library has
    recorded by each kernel's own dispatch (hx_moe_timing_*, hipExtLaunchKernel)
    on the stream it launches on, over 4 x 256 steps launched eagerly behind a
    0.4 s sleep kernel. `roofline.trace_avg_us` is the same dispatches' average
    in the committed rocprofv3 trace of this command (the `timed_avg_us` column
    of profiles/c2_decode_kernels.txt); the two agree to within a few tenths of
    a percent.
  * --steps K times exactly K steps (a graph of G steps, G the largest divisor
    of K up to 256, replayed K / G times).
  * Algorithmic bytes per step are computed from the actual routing (unique
    experts touched) and the GGUF sizes of what must be read once.
  * cpu_baseline: the reference's CPU arithmetic for GGUF experts, restated in
    oracle/ (candle's activation quantisation and integer vec_dot at m <= 64
    rows, its f16 path above), on the host cores with the same weights and
    tokens: C2 per layer here; C3, the 512-token chunk and C5 full forwards in
    their lines, C4 B = 1 (one layer x 48) in the C3 line.
  * `prefill` (secondary): C3, 2048 tokens of the same layer in Q4_K_M (gate/up
    Q4_K, down Q6_K), tokens/s with its MFMA and HBM fractions (`us`: 100
    back-to-back forwards after 20 warm-up ones, timed by HIP events on the
    stream; `wall_us`: the
    host clock around the same forwards, synchronised on both sides), and a roofline
    object for the gate/up MFMA kernel (event-timed; traced average, HBM traffic
    and MFMA counters from profiles/). `prefill_512`: the same at the
    reference's production prefill chunk of 512 tokens.
  * `c5_skew` (secondary): C5, 4096 tokens with a Zipf(1.1) router bias
    calibrated so the top 8 experts take ~40% of the assignments.
  * `c4_stack` (secondary): C4, the 48-layer Q4_K_M stack with RMSNorm and
    residual (attention skipped), decode at B = 1, 4, 8, per token (one HIP
    graph of the 48 layers per B, 50 replays after 10 warm-up ones).

    python bench.py [--steps K] [--warmup W] [--layers L] [--no-cpu] [--no-prefill] [--no-c4] [--no-c5]
    python bench.py --c4-only B      (one line: the C4 stack at batch B, for profiling)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
MFMA_BF16_PEAK_TFS = 2516.6     # dense bf16: 256 CU x 4096 flop/clk x 2.4 GHz
METRIC = "MoE-layer decode µs + % HBM peak; prefill tok/s + % MFMA peak (Q4_K_M)"
KERNEL_NAMES = {"router": "k_router_dec", "gate_up": "k_gate_up_dec", "down": "k_down_dec"}
WARM_MS = 20.0                  # least warm-up of the decode headline, in ms of graph replays


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gguf_bytes(fmt, rows, cols):
    from helexa_amd import row_bytes
    return rows * row_bytes(fmt, cols)


def step_bytes(cfg, fmts, unique_experts, T):
    """Algorithmic HBM bytes of one decode forward (every touched weight byte once,
    the tokens in and out once), in total and per kernel of the decode path:
      router  -- router rows + shared-expert gate row (bf16), the tokens (and,
                 for T > 1, the shared expert's gate/up projections, which that
                 kernel computes);
      gate_up -- the routed experts' gate/up projections (and, for T = 1, the
                 shared expert's, which the single-token kernel computes while
                 it routes), the tokens;
      down    -- the routed and shared down projections, the output rows.
    The SwiGLU activations passed between kernels are intermediates and are not
    counted."""
    H, E, I, Is = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size, cfg.shared_expert_intermediate_size
    act = T * H * 2
    router_w = (E + 1) * H * 2
    shared_gu = gguf_bytes(fmts["sgate"], Is, H) + gguf_bytes(fmts["sup"], Is, H)
    routed_gu = unique_experts * (gguf_bytes(fmts["gate"], I, H) + gguf_bytes(fmts["up"], I, H))
    down_w = unique_experts * gguf_bytes(fmts["down"], H, I) + gguf_bytes(fmts["sdown"], H, Is)
    total = router_w + shared_gu + routed_gu + down_w + 2 * act
    sg_router, sg_gate_up = (0, shared_gu) if T == 1 else (shared_gu, 0)
    return total, {"router": router_w + sg_router + act, "gate_up": routed_gu + sg_gate_up + act,
                   "down": down_w + act}


def build_layers(cfg, fmts, n_layers, seed, keep_host_copy_of_first=False):
    import torch
    import helexa_amd as hx
    from helexa_amd import synth
    blocks, host0 = [], None
    for i in range(n_layers):
        w = synth.make_weights(cfg, fmts, seed + i)
        blocks.append(hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16))
        if i == 0 and keep_host_copy_of_first:
            host0 = synth.to_numpy(w)
        del w
        torch.cuda.synchronize()
    return blocks, host0


def capture(blocks, xs, ys, wss, n_steps, timing=False):
    """one HIP graph holding n_steps decode steps, step s on layer s % L"""
    import torch
    L = len(blocks)
    if timing:
        for b in blocks:
            b.timing_begin((n_steps + L - 1) // L)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n_steps):
                blocks[i % L].forward(xs[i % len(xs)], workspace=wss[i % L], stream=s, out=ys[i % len(ys)])
    torch.cuda.current_stream().wait_stream(s)
    return g


def bench_decode(args):
    import numpy as np
    import torch
    import helexa_amd as hx
    from helexa_amd import synth

    cfg, fmts = synth.A3B, synth.FMT_Q8_0
    log(f"[bench] building {args.layers} Q8_0 layers")
    t0 = time.time()
    blocks, host0 = build_layers(cfg, fmts, args.layers, 1000, keep_host_copy_of_first=not args.no_cpu)
    log(f"[bench] layers ready in {time.time() - t0:.1f}s")
    n_x = 64
    xs = [synth.make_x(cfg, 1, 50 + i) for i in range(n_x)]
    ys = [torch.empty_like(xs[0]) for _ in range(n_x)]
    wss = [torch.empty(b.workspace_size(1), dtype=torch.uint8, device="cuda") for b in blocks]

    # routing of the measured steps -> unique experts per step
    uniq = []
    for i in range(n_x):
        idx = blocks[i % len(blocks)].route(xs[i])["topk_idx"]
        uniq.append(int(torch.unique(idx).numel()))
    U = float(np.mean(uniq))
    total_bytes, kbytes = step_bytes(cfg, fmts, U, 1)

    # exactly args.steps timed steps: a graph of G steps (the largest divisor of
    # the step count up to 256) replayed steps / G times
    steps = max(1, args.steps)
    G = max(d for d in range(1, min(256, steps) + 1) if steps % d == 0)
    g = capture(blocks, xs, ys, wss, G)
    reps = steps // G
    # one replay (host clock) sizes the warm-up: at least --warmup steps and at
    # least WARM_MS of replays, which carries the card past its clock
    # transient (a chain started from idle runs slower for its first few ms)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    replay_ms = (time.perf_counter() - t0) * 1e3
    warm_reps = max(-(-args.warmup // G), int(WARM_MS / max(replay_ms, 1e-3)) + 1)
    # timed region: the warm-up replays, then a start event, the K steps and a
    # stop event, all queued on the replay stream without a synchronisation in
    # between, so the K steps run back to back behind the warm-up at the clock
    # it settled at; the events time exactly those K steps on the GPU
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    for _ in range(warm_reps):
        g.replay()
    ev0.record()
    for _ in range(reps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    us_per_layer = ev0.elapsed_time(ev1) * 1e3 / steps
    # the host clock around the same K steps, synchronised on both sides (adds
    # the host's launch of the first replay)
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - t0) / steps * 1e6

    # the graph's last write of ys[(G - 1) % 64] came from layer (G - 1) % L on
    # xs[(G - 1) % 64]: it must equal an eager forward bit for bit
    last = G - 1
    graph_ok = bool(torch.equal(blocks[last % len(blocks)].forward(xs[last % n_x]), ys[last % n_x]))

    # per-kernel durations: 256 steps launched eagerly with the library's HIP
    # events, queued behind a 0.4 s sleep kernel (long enough that every launch is
    # queued before the GPU reaches them, also under a profiler's slower host
    # side), so the GPU runs them back to back; for one token each kernel's event
    # pair is recorded by its own dispatch (hipExtLaunchKernel), the interval a
    # kernel trace reports for the same dispatches
    kern = {}
    n_t = 256
    for _ in range(4):
        for b in blocks:
            b.timing_begin((n_t + len(blocks) - 1) // len(blocks))
        torch.cuda._sleep(int(2.4e9 * 0.4))
        for i in range(n_t):
            blocks[i % len(blocks)].forward(xs[i % len(xs)], workspace=wss[i % len(blocks)], out=ys[i % len(ys)])
        torch.cuda.synchronize()
        for b in blocks:
            for name, (ms, n) in b.timing_end().items():
                if n:
                    a = kern.setdefault(name, [0.0, 0])
                    a[0] += ms
                    a[1] += n
    kern_us = {k: v[0] / v[1] * 1e3 for k, v in kern.items()}
    dominant = max(("gate_up", "down"), key=lambda k: kbytes[k])
    d_us = kern_us.get(dominant, float("nan"))
    achieved = kbytes[dominant] / (d_us * 1e-6) / 1e9
    layer_gbs = total_bytes / (us_per_layer * 1e-6) / 1e9
    from helexa_amd.profsum import read_pmc, read_stats_avg
    traffic = read_pmc(os.path.join(ROOT, "profiles", "c2_decode_pmc.txt"), KERNEL_NAMES[dominant])
    trace_us = read_stats_avg(os.path.join(ROOT, "profiles", "c2_decode_kernels.txt"), KERNEL_NAMES[dominant])

    out = {
        "metric": METRIC, "value": round(us_per_layer, 3), "unit": "us/layer (C2 decode)",
        "n_gpus": 1, "steps": steps, "warmup": warm_reps * G, "ms_per_step": round(us_per_layer / 1e3, 6),
        "wall_us": round(wall_us, 3),
        "timing": f"HIP events on the replay stream around exactly {steps} steps ({reps} replay(s) of a "
                  f"{G}-step graph), queued directly behind {warm_reps * G} warm-up steps (at least --warmup "
                  f"{args.warmup} and at least {WARM_MS:g} ms of replays); wall_us: host clock around the same "
                  f"steps, synchronised on both sides",
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "dtype_note": "expert products f16 x f16 (Q8_0 codes exact in f16, bf16 tokens converted) with f32 "
                      "accumulation; router bf16 x bf16 f32 fmaf",
        "data": "synthetic (seeded N(0,0.02) weights quantised to GGUF Q8_0 on device; bf16 N(0,1) tokens)",
        "config": {"workload": "C2: Qwen3-Next-80B-A3B MoE layer decode, T=1, Q8_0 experts, bf16 router+acts",
                   "hidden": cfg.hidden_size, "experts": cfg.num_experts, "top_k": cfg.num_experts_per_tok,
                   "moe_intermediate": cfg.moe_intermediate_size,
                   "shared_intermediate": cfg.shared_expert_intermediate_size,
                   "layers_rotated": args.layers, "unique_experts_per_step": U,
                   "graph_steps": G, "kernels_per_step": 3, "graph_replay_matches_eager": graph_ok},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": int(traffic) if traffic else None,
                     "traffic_source": "profiles/c2_decode_pmc.txt (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)"
                     if traffic else None,
                     "algorithmic_bytes_per_launch": int(kbytes[dominant]), "avg_launch_us": round(d_us, 3),
                     # the same kernel's average in the committed rocprofv3 trace (a separate,
                     # profiled run of this command; the events above cannot be read under it)
                     "trace_avg_us": trace_us, "trace_source": "profiles/c2_decode_kernels.txt" if trace_us else None},
        "layer": {"algorithmic_bytes": int(total_bytes), "achieved_GBs": round(layer_gbs, 1),
                  "hbm_frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                  "kernel_us": {k: round(v, 3) for k, v in kern_us.items()}},
    }
    return out, blocks, host0, xs


def cpu_candle(cfg, wnp, x, runs, bias=None):
    """the oracle's candle-arithmetic forward (the reference's CPU path for GGUF
    experts: Q8_0 / Q8_K activation quantisation and candle's integer vec_dot at
    m <= 64 rows, its f16 path above) on the host cores: median of `runs` after
    one warm-up; -> (seconds, threads)"""
    import numpy as np
    import torch
    from oracle import oracle as O
    orc = O.OracleMoe(cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size,
                      cfg.shared_expert_intermediate_size, cfg.norm_topk_prob, O.BF16, wnp)
    xn = x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    bn = None if bias is None else bias.detach().cpu().numpy()
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    orc.forward_candle(xn, bias=bn, nthreads=threads)
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        orc.forward_candle(xn, bias=bn, nthreads=threads)
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), threads


ARITH = ("candle CPU arithmetic restated (oracle/hx_oracle.c hxo_moe_forward_candle): per expert call of m rows, "
         "m <= 64: activations quantised to Q8_0 / Q8_K and candle's generic integer vec_dot; m > 64: f16 "
         "weights and activations, f32 accumulation, f16 output; f32 SwiGLU and combine")


def cpu_baseline_c2(cfg, host0, x0, runs=50):
    s, th = cpu_candle(cfg, host0, x0, runs)
    return {"value": round(s * 1e6, 1), "unit": "us/layer (C2 decode)", "cores": th, "kind": "port",
            "arithmetic": ARITH,
            "sample": f"one single-token decode of layer 0 (the GPU run's weights and first token), median of "
                      f"{runs} runs after a warm-up, {th} OpenMP threads"}


# the routed gate/up launch is the dominant prefill kernel; the shared expert's
# GEMMs are separate launches (template argument 2) on the handle's side stream
# prefill forwards of more tokens than this run the shared expert's GEMMs on the
# library's side stream (tile selection 1: routed, 2: shared); smaller ones fold
# the shared tiles into the routed launches (tile selection 0), as
# HX_SIDE_STREAM_T in helexa_amd/csrc/hx_internal.h
SIDE_STREAM_T = 2048


def prefill_kernels(T):
    """kernel names of a prefill forward of T tokens, per timing slot"""
    ts = "1" if T > SIDE_STREAM_T else "0"
    k = {"gate_up": f"k_gate_up_q4k<1, 4, {ts}>", "down": f"k_down_q6k<{ts}>", "router": "k_router_mfma",
         "route_tokens": "k_route_mfma"}
    if T > SIDE_STREAM_T:
        k.update({"shared_gate_up": "k_gate_up_q4k<1, 4, 2>", "shared_down": "k_down_q6k<2>"})
    return k


def prefill_work(cfg, fmts, T, U):
    """Algorithmic flops and HBM bytes of one prefill forward, in total and per
    kernel (each needed weight byte once; tokens in/out once; a kernel's own
    inputs and outputs: f16 tokens, f16 SwiGLU rows h, weighted bf16 rows):
    gate_up / down are the routed experts' launches, shared_* the shared
    expert's (on the side stream above SIDE_STREAM_T tokens; below, the shared
    tiles run in the gate_up / down launches and are counted there)."""
    H, I, Is, E, k = cfg.hidden_size, cfg.moe_intermediate_size, cfg.shared_expert_intermediate_size, \
        cfg.num_experts, cfg.num_experts_per_tok
    F = T * k
    gu_w, sgu_w = U * 2 * gguf_bytes(fmts["gate"], I, H), 2 * gguf_bytes(fmts["sgate"], Is, H)
    dn_w, sdn_w = U * gguf_bytes(fmts["down"], H, I), gguf_bytes(fmts["sdown"], H, Is)
    # router: the MFMA logits of the E routed experts over bf16 tokens, which
    # also writes the f16 copy of the tokens the expert kernels read
    flops = {"gate_up": 2 * F * 2 * H * I, "down": 2 * F * H * I, "shared_gate_up": 2 * T * 2 * H * Is,
             "shared_down": 2 * T * H * Is, "router": 2 * T * H * E}
    kbytes = {"gate_up": gu_w + T * H * 2 + F * I * 2, "down": dn_w + F * I * 2 + F * H * 2,
              "shared_gate_up": sgu_w + T * H * 2 + T * Is * 2, "shared_down": sdn_w + T * Is * 2 + T * H * 2,
              "router": E * H * 2 + T * H * 2 + T * H * 2}
    if T <= SIDE_STREAM_T:
        for kk in ("gate_up", "down"):
            flops[kk] += flops.pop("shared_" + kk)
            kbytes[kk] += kbytes.pop("shared_" + kk)
    total_flops = 2 * T * k * 3 * H * I + 2 * T * 3 * H * Is + 2 * T * H * E
    total_bytes = gu_w + sgu_w + dn_w + sdn_w + (E + 1) * H * 2 + 2 * T * H * 2
    return total_flops, total_bytes, flops, kbytes


def prefill_run(cfg, fmts, w_seed, x_seed, T, workload, reps=100, bias=None, pmc_file=None, mfma_file=None,
                trace_file=None, cpu_runs=0, c4_layer=False):
    """One prefill line: `reps` back-to-back forwards timed by HIP events on the
    stream (GPU time per forward, `us`) and by the host clock around them with a
    synchronisation on both sides (`wall_us`, which adds the host's launch of the
    first forward); then `kern_reps` forwards again with every kernel timed by
    its own dispatch's HIP events, queued behind a sleep kernel; roofline of the
    gate/up MFMA kernel (the largest)."""
    import torch
    import helexa_amd as hx
    from helexa_amd import synth
    from helexa_amd.profsum import read_pmc, read_stats_avg, read_mfma
    w = synth.make_weights(cfg, fmts, w_seed)
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16)
    wnp = synth.to_numpy(w) if cpu_runs else None
    del w
    x = synth.make_x(cfg, T, x_seed)
    ws = torch.empty(blk.workspace_size(T), dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    r = blk.route(x, router_bias=bias)
    U = int(torch.unique(r["topk_idx"]).numel())
    counts = torch.diff(r["offsets"]).cpu()
    # warm-up long enough (about 8 ms of forwards) to pass the card's clock
    # transient after idle: forwards 5-15 of a chain started from idle run up to
    # 12 % slower than the steady state that later forwards settle to
    for _ in range(20):
        blk.forward(x, router_bias=bias, workspace=ws, out=y)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    t0 = time.perf_counter()
    ev[0].record()
    for _ in range(reps):
        blk.forward(x, router_bias=bias, workspace=ws, out=y)
    ev[1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / reps
    dt = ev[0].elapsed_time(ev[1]) * 1e-3 / reps
    kern_reps = 5
    blk.timing_begin(kern_reps)
    torch.cuda._sleep(int(2.4e9 * 0.05))
    for _ in range(kern_reps):
        blk.forward(x, router_bias=bias, workspace=ws, out=y)
    torch.cuda.synchronize()
    kern = {k: v[0] / v[1] * 1e3 for k, v in blk.timing_end().items() if v[1]}
    blk.close()
    total_flops, total_bytes, kflops, kbytes = prefill_work(cfg, fmts, T, U)
    d_us = kern.get("gate_up", float("nan"))
    tfs = kflops["gate_up"] / (d_us * 1e-6) / 1e12
    kn = prefill_kernels(T)
    what = "routed gate_up" if T > SIDE_STREAM_T else "gate_up, routed and shared tiles"
    roof = {"bound": "mfma", "kernel": f"{what} ({kn['gate_up']})", "achieved": round(tfs, 1),
            "peak": MFMA_BF16_PEAK_TFS, "unit": "TFLOP/s", "frac": round(tfs / MFMA_BF16_PEAK_TFS, 4),
            "algorithmic_flops_per_launch": kflops["gate_up"], "algorithmic_bytes_per_launch": kbytes["gate_up"],
            "avg_launch_us": round(d_us, 2),
            "hbm_frac": round(kbytes["gate_up"] / (d_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}
    if pmc_file:
        tr = read_pmc(os.path.join(ROOT, "profiles", pmc_file), kn["gate_up"])
        roof["traffic"] = int(tr) if tr else None
        roof["traffic_source"] = f"profiles/{pmc_file} (FETCH_SIZE + WRITE_SIZE, copy-calibrated)" if tr else None
    if trace_file:
        roof["trace_avg_us"] = read_stats_avg(os.path.join(ROOT, "profiles", trace_file), kn["gate_up"])
        roof["trace_source"] = f"profiles/{trace_file}"
    if mfma_file:
        mf = read_mfma(os.path.join(ROOT, "profiles", mfma_file), kn["gate_up"])
        if mf:
            roof["mfma_counters"] = mf
            roof["mfma_source"] = f"profiles/{mfma_file}"
    kr = {k: {"us": round(v, 1),
              "mfma_frac": round(kflops[k] / (v * 1e-6) / (MFMA_BF16_PEAK_TFS * 1e12), 4) if k in kflops else None,
              "hbm_frac": round(kbytes[k] / (v * 1e-6) / (HBM_PEAK_GBS * 1e9), 4) if k in kbytes else None}
          for k, v in kern.items()}
    out = {"workload": workload, "tokens": T, "forwards": reps, "us": round(dt * 1e6, 1),
           "wall_us": round(wall * 1e6, 1), "tok_per_s": round(T / dt, 1),
           "mfma_frac": round(total_flops / dt / (MFMA_BF16_PEAK_TFS * 1e12), 4),
           "hbm_frac": round(total_bytes / dt / (HBM_PEAK_GBS * 1e9), 4),
           "algorithmic_flops": total_flops, "algorithmic_bytes": total_bytes, "unique_experts": U,
           "max_expert_rows": int(counts.max()), "roofline": roof, "kernels": kr}
    if cpu_runs:
        log(f"[bench] cpu baseline, {T} tokens")
        sec, th = cpu_candle(cfg, wnp, x, cpu_runs, bias)
        out["cpu_baseline"] = {"value": round(T / sec, 1), "unit": "tok/s", "us": round(sec * 1e6, 1),
                               "cores": th, "kind": "port", "arithmetic": ARITH,
                               "sample": f"the same {T} tokens and weights, full forward, median of {cpu_runs} "
                                         f"runs after a warm-up, {th} OpenMP threads"}
        if c4_layer:
            # C4 at B = 1: one Q4_K_M layer's single-token forward (RMSNorm and
            # residual add are O(H)), times the 48 layers of the stack
            sec1, th = cpu_candle(cfg, wnp, x[:1], 20)
            out["cpu_baseline_c4_b1"] = {"value": round(sec1 * 48 * 1e6, 1), "unit": "us/token (C4 B=1, 48 layers)",
                                         "cores": th, "kind": "port", "arithmetic": ARITH,
                                         "sample": "one single-token layer forward of this Q4_K_M layer, median "
                                                   "of 20 runs after a warm-up, times 48 layers"}
    return out


def bench_prefill(T=2048, reps=100, cpu_runs=0):
    """C3 (T = 2048) and the production chunk (T = 512): Q4_K_M prefill, seeded
    near-uniform routing"""
    from helexa_amd import synth
    tag = "C3" if T == 2048 else "production chunk"
    return prefill_run(synth.A3B, synth.FMT_Q4_K_M, 4242, 77, T,
                       f"{tag}: {T}-token prefill, Q4_K_M (gate/up Q4_K, down Q6_K), bf16", reps,
                       pmc_file="c3_prefill_pmc.txt" if T == 2048 else None,
                       mfma_file="c3_prefill_mfma.txt" if T == 2048 else None,
                       trace_file="c3_prefill_kernels.txt" if T == 2048 else None,
                       cpu_runs=cpu_runs, c4_layer=cpu_runs > 0 and T == 2048)


def bench_c4(n_layers=48, batches=(1, 4, 8), reps=50):
    """C4: 48-layer stack of the 80B-A3B MoE block in Q4_K_M with residual adds and
    attention skipped: per layer x <- x + moe(rmsnorm(x)) (decoder.rs:129-132), the
    RMSNorm weight stored as 1.0 with the reference's (1 + w) scaling
    (rmsnorm.rs:76-77), eps 1e-6. Each batch size's 48 layers are captured in one
    HIP graph; time per token = step time / B."""
    import torch
    import helexa_amd as hx
    from helexa_amd import synth
    cfg, fmts = synth.A3B, synth.FMT_Q4_K_M
    t0 = time.time()
    blocks, _ = build_layers(cfg, fmts, n_layers, 7000)
    log(f"[bench] C4: {n_layers} Q4_K_M layers ready in {time.time() - t0:.1f}s")
    norm_w = torch.ones(cfg.hidden_size, dtype=torch.float32, device="cuda")
    H, I, Is = cfg.hidden_size, cfg.moe_intermediate_size, cfg.shared_expert_intermediate_size
    per_expert = gguf_bytes(fmts["gate"], I, H) * 2 + gguf_bytes(fmts["down"], H, I)
    shared = gguf_bytes(fmts["sgate"], Is, H) * 2 + gguf_bytes(fmts["sdown"], H, Is)
    router = (cfg.num_experts + 1) * H * 2
    out = {"workload": f"C4: {n_layers}-layer Q4_K_M MoE stack decode (residual + RMSNorm, attention skipped), bf16",
           "layers": n_layers, "batches": {}}
    for B in batches:
        x0 = synth.make_x(cfg, B, 900 + B)
        ws = torch.empty(max(b.workspace_size(B) for b in blocks[:1]), dtype=torch.uint8, device="cuda")
        # algorithmic bytes of one step: the unique experts each layer touches on
        # this input (eager pass, layer by layer)
        x = x0.clone()
        step_bytes_ = 0
        for b in blocks:
            U = int(torch.unique(b.route(b_rms(x, norm_w))["topk_idx"]).numel())
            step_bytes_ += U * per_expert + shared + router + 2 * B * H * 2
            b.decoder_mlp_(x, norm_w, 1e-6, workspace=ws)
        eager = x.clone()
        xg = x0.clone()
        g = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            with torch.cuda.graph(g, stream=st):
                for b in blocks:
                    b.decoder_mlp_(xg, norm_w, 1e-6, workspace=ws, stream=st)
        torch.cuda.current_stream().wait_stream(st)
        xg.copy_(x0)
        g.replay()
        torch.cuda.synchronize()
        graph_ok = bool(torch.equal(xg, eager))
        # ten replays (10-40 ms) past the clock transient of the first few
        # milliseconds after idle, as for the prefill lines
        for _ in range(10):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            g.replay()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
        out["batches"][str(B)] = {"us_per_step": round(dt * 1e6, 1), "us_per_token": round(dt * 1e6 / B, 1),
                                  "us_per_layer": round(dt * 1e6 / n_layers, 2),
                                  "algorithmic_bytes_per_step": int(step_bytes_),
                                  "hbm_frac": round(step_bytes_ / dt / (HBM_PEAK_GBS * 1e9), 4),
                                  "graph_matches_eager": graph_ok}
        log(f"[bench] C4 B={B}: {out['batches'][str(B)]}")
    for b in blocks:
        b.close()
    return out


def b_rms(x, w, eps=1e-6):
    """the stack's RMSNorm on the device (f32 math, bf16 out), (1 + w) scaling --
    only used to find which experts a layer routes to for the byte count"""
    import torch
    xf = x.float()
    y = xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps) * (1.0 + w)
    return y.to(x.dtype)


def bench_c5(T=4096, target_share=0.40, reps=100, cpu_runs=0):
    """C5: 4096-token prefill of the Q4_K_M layer with a seeded Zipf(1.1) router
    bias (router_bias[e] = alpha ln p_{pi(e)}), alpha calibrated on this layer so
    the top 8 experts take about 40% of the assignments."""
    import torch
    import helexa_amd as hx
    from helexa_amd import synth
    cfg, fmts = synth.A3B, synth.FMT_Q4_K_M
    w = synth.make_weights(cfg, fmts, 4243)
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16)
    del w
    x = synth.make_x(cfg, T, 78)
    E = cfg.num_experts
    base = synth.zipf_bias(E, 1.1, 1.0, 11)
    top8 = torch.argsort(base, descending=True)[:8]

    def share(alpha):
        idx = blk.route(x, router_bias=base * alpha)["topk_idx"]
        return float(torch.isin(idx, top8).float().mean())

    lo, hi = 0.0, 2.0
    for _ in range(14):
        mid = 0.5 * (lo + hi)
        if share(mid) < target_share:
            lo = mid
        else:
            hi = mid
    alpha = 0.5 * (lo + hi)
    achieved = share(alpha)
    blk.close()
    del blk
    out = prefill_run(cfg, fmts, 4243, 78, T, f"C5: {T}-token prefill, Q4_K_M, Zipf(1.1) router bias", reps,
                      bias=base * alpha, pmc_file="c5_prefill_pmc.txt", mfma_file="c5_prefill_mfma.txt",
                      trace_file="c5_prefill_kernels.txt",
                      cpu_runs=cpu_runs)
    out.update({"alpha": round(alpha, 4), "top8_share": round(achieved, 4)})
    return out


def probe(args):
    """Workload for the rocprofv3 --pmc runs: 48 eager decode steps over 16 rotated
    layers, then the runtime's device-to-device copy of COPY_BYTES bytes (the
    counter calibration)."""
    import torch
    import helexa_amd as hx
    from helexa_amd import synth
    cfg, fmts = synth.A3B, synth.FMT_Q8_0
    blocks, _ = build_layers(cfg, fmts, 16, 1000)
    xs = [synth.make_x(cfg, 1, 50 + i) for i in range(16)]
    for i in range(48):
        blocks[i % 16].forward(xs[i % 16])
    torch.cuda.synchronize()
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "c2_decode", "steps": 48, "copy_bytes": COPY_BYTES}), flush=True)


COPY_BYTES = 256 << 20


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=512)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--probe", action="store_true", help="short workload for rocprofv3 --pmc runs")
    ap.add_argument("--prefill-only", action="store_true", help="only the C3 prefill line (for profiling)")
    ap.add_argument("--c5-only", action="store_true", help="only the C5 skewed prefill line (for profiling)")
    ap.add_argument("--no-c4", action="store_true", help="skip the 48-layer stack line")
    ap.add_argument("--no-c5", action="store_true", help="skip the skewed 4096-token prefill line")
    ap.add_argument("--c4-only", type=int, default=0, metavar="B",
                    help="only the C4 stack line at batch B (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (expert parallelism would "
              "give each GPU a contiguous range of the experts; not built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (cuda:0)", file=sys.stderr)
        sys.exit(2)
    from helexa_amd import synth
    if args.probe:
        probe(args)
        return
    if args.prefill_only:
        print(json.dumps(bench_prefill()), flush=True)
        return
    if args.c5_only:
        print(json.dumps(bench_c5()), flush=True)
        return
    if args.c4_only:
        print(json.dumps(bench_c4(batches=(args.c4_only,))), flush=True)
        return
    out, blocks, host0, xs = bench_decode(args)
    log(f"[bench] decode {out['value']} us/layer; kernels {out['layer']['kernel_us']}")
    cpu_runs = 0 if args.no_cpu else 5
    if not args.no_cpu:
        log("[bench] cpu baseline")
        out["cpu_baseline"] = cpu_baseline_c2(synth.A3B, host0, xs[0])
    else:
        out["cpu_baseline"] = None
    for b in blocks:
        b.close()
    del blocks
    torch.cuda.empty_cache()
    if not args.no_prefill:
        log("[bench] prefill")
        out["prefill"] = bench_prefill(cpu_runs=cpu_runs)
        torch.cuda.empty_cache()
        log("[bench] prefill, production chunk of 512 tokens")
        out["prefill_512"] = bench_prefill(512, cpu_runs=cpu_runs)
        torch.cuda.empty_cache()
    if not args.no_c5:
        log("[bench] C5 skewed prefill")
        out["c5_skew"] = bench_c5(cpu_runs=cpu_runs)
        torch.cuda.empty_cache()
    if not args.no_c4:
        log("[bench] C4 stack")
        out["c4_stack"] = bench_c4()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
