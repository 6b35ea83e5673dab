#!/usr/bin/env python3
"""Throughput of the qwen35moe MoE FFN block on one MI355X.

A step is one forward of one MoE layer (router, routing, dispatch, grouped
Q8_0 expert SwiGLU, shared expert, combine) over T tokens already resident in
HBM.  The headline workload is the decode-verify configuration (T = 5: one
token plus four MTP drafts); T = 1, 40 and the
T = 512 Zipf-skewed prefill chunk are reported in `sweep`.

Steps rotate over `--layers` distinct copies of the layer in HBM (16 x 856 MB
by default), so the expert weights a step reads are not left in the 256 MB
Infinity Cache by the step before: the figure is HBM-honest.

Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

E, NE, K, FF = 2048, 256, 8, 512
Q8_ROW_E = 2048 // 32 * 34   # bytes of a Q8_0 row of 2048
Q8_ROW_FF = 512 // 32 * 34   # bytes of a Q8_0 row of 512
EXPERT_BYTES = 2 * FF * Q8_ROW_E + E * Q8_ROW_FF   # 3,342,336
ROUTER_BYTES = NE * E * 4 + E * 4                  # router + gate_inp (f32)
HBM_PEAK = 8.0e12


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_bytes(U, T):
    """Algorithmic HBM bytes of one layer: the U routed experts and the shared
    expert (read once each), the router and gate_inp, h in and out out."""
    return (U + 1) * EXPERT_BYTES + ROUTER_BYTES + 2 * T * E * 4


def stage_bytes(stage, U, T):
    """Algorithmic bytes of one stage's launch (weights read once, activations
    read and written once)."""
    P = T * K
    R = P + T
    if stage == "gate_up":  # weights, Q8 h, the f32 intermediate
        return (U + 1) * 2 * FF * Q8_ROW_E + T * E * 9 // 8 + R * FF * 4
    if stage == "quant_act":
        return R * FF * 4 + R * FF * 9 // 8
    if stage == "down":  # weights, the intermediate (f32 when the kernel quantises it, T <= 16), y
        return (U + 1) * E * Q8_ROW_FF + R * FF * (4 if T <= 16 else 9 / 8) + R * E * 4
    if stage == "combine":
        return R * E * 4 + T * E * 4 + P * 8
    if stage == "router":  # router + gate_inp, h, logits, Q8 h
        return ROUTER_BYTES + T * E * 4 + T * (NE + 1) * 4 + T * E * 9 // 8
    if stage == "route_sort":
        return T * NE * 4 + P * 24
    return 0


# HBM bytes per launch of the dominant kernel, not measured in this run: the
# figures of rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over the same
# workload (scaled by a copy kernel of known size: x2.0 and x1.0), committed
# with their commands in TRAFFIC_SOURCE.  Keyed by (stage, T).
TRAFFIC_SOURCE = "profiles/moe_layer_q8_0_hbm_traffic.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)"
TRAFFIC = {
    ("gate_up", 1): 20207131, ("gate_up", 5): 91705677, ("gate_up", 40): 430113924,
    ("down", 1): 10344203, ("down", 5): 46907741, ("down", 40): 217679560,
    ("gate_up", 512): 697649152, ("down", 512): 365848576,
}


def tokens_for(layer, T, seed):
    from biv_amd import synth
    if T >= 512:
        return synth.zipf_bias_tokens(layer, seed, T)
    return synth.make_tokens(seed, T, offsets=T > 1)


def bench_gpu(eng, moes, layer, T, steps, warmup, torch):
    import numpy as np
    h = tokens_for(layer, T, 1000 + T)
    _, taps = moes[0].ffn_taps(h, dots=False)
    U = int(np.unique(taps["ids"]).size)
    h_dev = torch.from_numpy(h).cuda()
    out_dev = torch.empty_like(h_dev)
    L = len(moes)
    for i in range(warmup):
        moes[i % L].forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall = time.perf_counter()
    t0.record()
    for i in range(steps):
        moes[i % L].forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall
    ms = t0.elapsed_time(t1) / steps
    # per-step distribution: an event between consecutive steps (the launches
    # queue ahead, so each interval is one step's time on the GPU)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record()
    for i in range(steps):
        moes[i % L].forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
        evs[i + 1].record()
    torch.cuda.synchronize()
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]) * 1e3
    # each stage's launches alone, back to back over the layer copies (a
    # kernel time, as rocprof's, with no event between stages); a stage with
    # no launch at this T is null (T <= 16: the intermediate is quantised
    # inside the down + combine launch, which the "down" stage is)
    stage_us = {}
    for st in STAGE_NAMES:
        us = 1e3 * eng.time_stage(moes, h_dev.data_ptr(), T, out_dev.data_ptr(), st, steps)
        stage_us[st] = us if us >= EMPTY_STAGE_US else None
    B = layer_bytes(U, T)
    res = {
        "T": T, "U": U, "us_per_layer": round(ms * 1e3, 3), "tokens_per_s": round(T / (ms * 1e-3), 1),
        "layer_GBps": round(B / (ms * 1e-3) / 1e9, 1), "layer_hbm_frac": round(B / (ms * 1e-3) / HBM_PEAK, 4),
        "us_median": round(float(np.median(per)), 3), "us_p10": round(float(np.percentile(per, 10)), 3),
        "us_p90": round(float(np.percentile(per, 90)), 3),
        "stage_us": {k: (round(v, 3) if v is not None else None) for k, v in stage_us.items()},
        "wall_s": round(wall, 3),
    }
    if T >= 64:
        res["mfma"] = mfma_block(T, ms)
    # the dominant kernel alone: launched back to back over the layer copies
    # (the stage events above add a dispatch gap to every stage)
    dom = max(("gate_up", "down", "router"), key=lambda s: stage_us[s] or 0.0)
    kern_us = stage_us[dom]
    dbytes = stage_bytes(dom, U, T)
    ach = dbytes / (kern_us * 1e-6) / 1e9
    res["roofline"] = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK / 1e9,
                       "unit": "GB/s", "frac": round(ach * 1e9 / HBM_PEAK, 4), "traffic": TRAFFIC.get((dom, T)),
                       "traffic_source": TRAFFIC_SOURCE if (dom, T) in TRAFFIC else None,
                       "bytes_per_launch": dbytes, "avg_us": round(kern_us, 3)}
    return res


STAGE_NAMES = ("router", "route_sort", "gate_up", "quant_act", "down", "combine")
EMPTY_STAGE_US = 0.5  # an event pair around no launch measures well below this


OPS_PER_TOKEN = (K + 1) * 3 * 2 * E * FF   # int8 ops of the routed pairs and the shared row: 56,623,104
INT8_PEAK = 5.0e15


def mfma_block(T, ms, bytes_=None):
    """Algorithmic int8 ops of the layer per second against the dense int8
    MFMA peak, and the cap the HBM roofline puts on it at this arithmetic
    intensity (ops per algorithmic byte x 8 TB/s)."""
    ops = OPS_PER_TOKEN * T
    ach = ops / (ms * 1e-3)
    res = {"achieved": round(ach / 1e12, 2), "peak": INT8_PEAK / 1e12, "unit": "TOP/s",
           "frac": round(ach / INT8_PEAK, 5)}
    if bytes_ is None:
        bytes_ = layer_bytes(NE, T)
    cap = min(INT8_PEAK, ops / bytes_ * HBM_PEAK)
    res["hbm_cap"] = round(cap / 1e12, 1)
    res["frac_of_cap"] = round(ach / cap, 4)
    return res


def bench_graph_chain(eng, moes, layer, T, reps, torch):
    """The decode step as a serving loop runs it: the L layer copies' forwards
    captured into one HIP graph and replayed (a chain of L layers at T = 1),
    reported as total / L.  Each replay is checked against the eager
    result of the last layer."""
    L = len(moes)
    h_dev = torch.from_numpy(tokens_for(layer, T, 1000 + T)).cuda()
    out_dev = torch.empty_like(h_dev)
    for m in moes:
        m.forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
    torch.cuda.synchronize()
    want = out_dev.clone()
    stream = torch.cuda.current_stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for m in moes:
            m.forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
    ok = True
    for _ in range(3):
        out_dev.zero_()
        g.replay()
        torch.cuda.synchronize()
        ok &= bool(torch.equal(out_dev, want))
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / (reps * L)
    return {"T": T, "layers_in_graph": L, "replays": reps, "us_per_layer": round(ms * 1e3, 3),
            "tokens_per_s": round(T / (ms * 1e-3), 1), "replays_match_eager": ok}


def bench_config(eng, layer, copies, T, steps, warmup, torch):
    """Another layer type (configs[3]: Q4_K gate/up + Q6_K down): the same
    measurement over `copies` copies in HBM."""
    moes = [eng.moe(layer) for _ in range(copies)]
    from biv_amd import synth
    h = synth.make_tokens(1000 + T, T, offsets=T > 1)  # ~N(0,1)
    h_dev = torch.from_numpy(h).cuda()
    out_dev = torch.empty_like(h_dev)
    for i in range(warmup):
        moes[i % copies].forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        moes[i % copies].forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    res = {"T": T, "us_per_layer": round(ms * 1e3, 3), "tokens_per_s": round(T / (ms * 1e-3), 1),
           "layers_rotated": copies}
    if T >= 64:
        # Q4_K gate/up (144 B per 256) and Q6_K down (210 B per 256): 2,039,808 B per expert
        ebytes = 2 * FF * (E // 256 * 144) + E * (FF // 256 * 210)
        res["mfma"] = mfma_block(T, ms, (NE + 1) * ebytes + ROUTER_BYTES + 2 * T * E * 4)
        # the dominant kernel, the exact Q4_K gate/up, alone over the copies:
        # its algorithmic bytes are every expert's gate and up rows, the Q8 of
        # h with its scales and block sums, and the f32 intermediate written
        kern_us = 1e3 * eng.time_stage(moes, h_dev.data_ptr(), T, out_dev.data_ptr(), "gate_up", steps)
        gbytes = (NE + 1) * 2 * FF * (E // 256 * 144) + T * E * 5 // 4 + (T * K + T) * FF * 4
        ach = gbytes / (kern_us * 1e-6)
        res["roofline"] = {"kernel": "gate_up (exact Q4_K, k_gu_exact)", "bound": "hbm",
                           "achieved": round(ach / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                           "frac": round(ach / HBM_PEAK, 4), "bytes_per_launch": gbytes, "avg_us": round(kern_us, 3),
                           "traffic": KQ_TRAFFIC.get("gate_up"), "traffic_source": KQ_TRAFFIC_SOURCE}
    return res


# as TRAFFIC, for the Q4_K/Q6_K layer at T = 2048 and the BF16 layer at T = 4096
KQ_TRAFFIC_SOURCE = "profiles/prefill_hbm_traffic.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)"
KQ_TRAFFIC = {"gate_up": 688458752, "down": 585138176}
BF_TRAFFIC = {"gate_up": 1470939136, "down": 931569664}


def bench_bf16_stack(eng, T, n_layers, passes, torch):
    """n_layers BF16 MoE layers resident in HBM, a T-token chunk
    through all of them with the feed-forward half of Model::layer between
    (x += moe(rms_norm(x)), model.rs:788-790).  The layers are copies of one
    generated layer (distinct allocations, so every layer's weights come from
    HBM)."""
    import numpy as np
    from biv_amd import synth
    t = time.perf_counter()
    layer = synth.make_layer(2, types=(synth.BF16,) * 3)
    moes = [eng.moe(layer) for _ in range(n_layers)]
    log(f"bf16 stack: {n_layers} layers uploaded ({eng.device_bytes() / 1e9:.1f} GB on the device) "
        f"in {time.perf_counter() - t:.1f}s")
    rng = np.random.default_rng(3)
    norms = torch.from_numpy((1.0 + 0.02 * rng.standard_normal((n_layers, E))).astype(np.float32)).cuda()
    x0 = torch.from_numpy(synth.make_tokens(4000, T)).cuda()
    x = x0.clone()
    eps = 1e-6

    def one_pass():
        for l in range(n_layers):
            moes[l].ffn_step_device(x.data_ptr(), norms[l].data_ptr(), eps, T)

    one_pass()  # warm-up (scratch sized for T)
    torch.cuda.synchronize()
    x.copy_(x0)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(passes):
        one_pass()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / (passes * n_layers)
    # the dominant kernel, the BF16 grouped gate/up, alone over the layers
    # (on x, the last pass's output, ~N(0,1) rows): weights of every expert,
    # h's bf16 halves read, the intermediate's halves written
    kern_us = 1e3 * eng.time_stage(moes, x.data_ptr(), T, x0.data_ptr(), "gate_up", n_layers)
    gbytes = (NE + 1) * 2 * FF * E * 2 + T * E * 4 + (T * K + T) * FF * 4
    kach = gbytes / (kern_us * 1e-6)
    P = T * K
    flops = 2.0 * (P + T) * 3 * E * FF  # routed pairs and shared rows, gate + up + down
    U = NE  # every expert is routed at this T
    layer_bytes = (U + 1) * 3 * E * FF * 2 + ROUTER_BYTES + 2 * T * E * 4
    return {"T": T, "layers": n_layers, "passes": passes, "us_per_layer": round(ms * 1e3, 1),
            "tokens_per_s_per_layer": round(T / (ms * 1e-3), 1),
            "tokens_per_s_stack": round(T / (ms * 1e-3 * n_layers), 1),
            "compute": "bf16 MFMA grouped GEMM, f32 activations split into bf16 hi + lo (2 MFMAs per product)",
            # the layer is HBM-bound (128 algorithmic flop per weight byte vs
            # the bf16 ridge of ~312): bytes against 8 TB/s; the algorithmic
            # flops (routed pairs + shared rows, no hi/lo doubling) against
            # the 2.5 PFLOP/s dense bf16 peak
            "roofline": {"bound": "hbm", "achieved": round(layer_bytes / (ms * 1e-3) / 1e9, 1),
                         "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                         "frac": round(layer_bytes / (ms * 1e-3) / HBM_PEAK, 4)},
            "mfma": {"achieved": round(flops / (ms * 1e-3) / 1e12, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(flops / (ms * 1e-3) / 2.5e15, 4)},
            "kernel_roofline": {"kernel": "gate_up (BF16 grouped GEMM, k_mfma_bf16)", "bound": "hbm",
                                "achieved": round(kach / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                                "frac": round(kach / HBM_PEAK, 4), "bytes_per_launch": gbytes,
                                "avg_us": round(kern_us, 3), "traffic": BF_TRAFFIC.get("gate_up"),
                                "traffic_source": KQ_TRAFFIC_SOURCE},
            "hbm_GBps": round(layer_bytes / (ms * 1e-3) / 1e9, 1)}


def bench_dense(eng, copies, steps, warmup, torch, n_embd=4096, n_ff=12288):
    """The dense SwiGLU FFN of the qwen35 dense models (dense_ffn,
    model.rs:1118-1126) at a 9B-sized shape, Q8_0, T = 1 and 5, over `copies`
    copies in HBM: a widening beside the MoE block, not a BASELINE config."""
    from biv_amd import synth
    layer = synth.make_dense(9, n_embd=n_embd, n_ff=n_ff)
    dens = [eng.dense(layer) for _ in range(copies)]
    wbytes = 3 * n_ff * (n_embd // 32) * 34
    res = {"n_embd": n_embd, "n_ff": n_ff, "type": "Q8_0", "layers_rotated": copies, "weight_bytes": wbytes}
    for T in (1, 5):
        h_dev = torch.from_numpy(synth.make_tokens(1200 + T, T, n_embd=n_embd)).cuda()
        out_dev = torch.empty_like(h_dev)
        for i in range(warmup):
            dens[i % copies].forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(steps):
            dens[i % copies].forward_device(h_dev.data_ptr(), T, out_dev.data_ptr())
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        B = wbytes + 2 * T * n_embd * 4
        res[str(T)] = {"us_per_layer": round(ms * 1e3, 3), "tokens_per_s": round(T / (ms * 1e-3), 1),
                       "GBps": round(B / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(B / (ms * 1e-3) / HBM_PEAK, 4)}
    return res


def bench_cpu(layer, T, seconds):
    """The oracle (C restatement of biv's AVX2/AVX-VNNI CPU path) on the host cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    # every core this process may run on (the box's share of the host)
    threads = len(os.sched_getaffinity(0))
    h = tokens_for(layer, T, 1000 + T)
    oracle.moe(layer, h, threads=threads)  # warm
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.moe(layer, h, threads=threads)
        n += 1
    dt = (time.perf_counter() - t0) / n
    level = {0: "scalar", 1: "avx2", 2: "avxvnni"}[oracle.detect_level()]
    return {"value": round(T / dt, 2), "unit": "tokens/s", "cores": threads, "host_cpus": os.cpu_count(),
            "kind": "port",
            "us_per_layer": round(dt * 1e6, 1), "kernels": level,
            "sample": f"{n} forwards of the same T={T} Q8_0 layer ({seconds:.0f} s budget)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=16, help="distinct layer copies rotated in HBM")
    ap.add_argument("--T", type=int, default=5, help="tokens per step of the headline workload")
    ap.add_argument("--sweep", default="1,40,512", help="other T values to report ('' for none)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget (0 to skip)")
    ap.add_argument("--configs", default="kquant,bf16,dense",
                    help="other BASELINE configs to run: kquant (Q4_K/Q6_K at T=1, 2048), bf16 (the 40-layer BF16 "
                         "stack at T=4096), dense (the qwen35 dense FFN, 4096 x 12288 Q8_0); '' for none")
    ap.add_argument("--bf16-layers", type=int, default=40)
    ap.add_argument("--graph-reps", type=int, default=50,
                    help="replays of the graph-captured chain of --layers layers at T=1 (0 to skip)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first copy this many MiB device to device (a kernel of known traffic, to scale "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counts)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from biv_amd import hip, synth
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device="cuda")
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    t = time.perf_counter()
    layer = synth.make_layer(1)
    log(f"layer generated in {time.perf_counter() - t:.1f}s")
    eng = hip.HipEngine(0)
    # one default-priority stream for the library's kernels and the timing events
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    eng.set_stream(stream.cuda_stream)
    t = time.perf_counter()
    moes = [eng.moe(layer) for _ in range(args.layers)]
    log(f"{args.layers} layer copies uploaded ({eng.device_bytes() / 1e9:.1f} GB) in {time.perf_counter() - t:.1f}s")

    main_res = bench_gpu(eng, moes, layer, args.T, args.steps, args.warmup, torch)
    log(f"T={args.T}: {main_res}")
    sweep = {}
    for T in [int(x) for x in args.sweep.split(",") if x.strip()]:
        steps = args.steps if T <= 64 else max(20, args.steps // 4)
        sweep[str(T)] = bench_gpu(eng, moes, layer, T, steps, args.warmup, torch)
        log(f"T={T}: {sweep[str(T)]}")

    if args.graph_reps > 0:
        graph = bench_graph_chain(eng, moes, layer, 1, args.graph_reps, torch)
        log(f"graph chain T=1: {graph}")
    else:
        graph = None

    extra = {}
    todo = {c.strip() for c in args.configs.split(",") if c.strip()}
    if "kquant" in todo:
        kq = synth.make_layer(4, types=(synth.Q4K, synth.Q4K, synth.Q6K))
        extra["kquant_q4k_q6k"] = {str(T): bench_config(eng, kq, 4, T, 50 if T <= 64 else 10, 5, torch)
                                   for T in (1, 2048)}
        log(f"kquant: {extra['kquant_q4k_q6k']}")
    if "dense" in todo:
        extra["dense_ffn"] = bench_dense(eng, 8, 100, 10, torch)
        log(f"dense: {extra['dense_ffn']}")
    if "bf16" in todo:
        extra["bf16_stack"] = bench_bf16_stack(eng, 4096, args.bf16_layers, 2, torch)
        log(f"bf16 stack: {extra['bf16_stack']}")

    cpu = None
    if args.cpu_seconds > 0:
        cpu = bench_cpu(layer, args.T, args.cpu_seconds)
        log(f"cpu: {cpu}")

    ms = main_res["us_per_layer"] / 1e3
    line = {
        "metric": "MoE-layer tokens/s (qwen35moe, Q8_0, T=5 decode-verify)",
        "value": main_res["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_layer": main_res["us_per_layer"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantised to Q8_0, N(0,1) tokens)",
        "config": {"workload": "qwen35moe MoE FFN layer, Q8_0, decode-verify T=5 (configs[1])",
                   "n_embd": E, "n_expert": NE, "k": K, "n_ff": FF, "n_ff_shared": FF, "T": args.T,
                   "distinct_experts_U": main_res["U"], "layers_rotated": args.layers},
        "roofline": main_res["roofline"],
        "layer_roofline": {"bound": "hbm", "achieved": main_res["layer_GBps"], "peak": HBM_PEAK / 1e9,
                           "unit": "GB/s", "frac": main_res["layer_hbm_frac"]},
        "stage_us": main_res["stage_us"],
        "cpu_baseline": cpu,
        "sweep": sweep,
        "graph_chain_T1": graph,
        "configs": extra,
    }
    print(json.dumps(line), flush=True)
    eng.close()


if __name__ == "__main__":
    main()
