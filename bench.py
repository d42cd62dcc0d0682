#!/usr/bin/env python
"""MoE-layer throughput of the EXL3 expert path on one MI355X (bs=1 decode).

A step is one MoE layer on one token: router (softmax top-4) -> grouping -> rotated gate/up trellis GEMV -> limited
SwiGLU epilogue -> down GEMV -> epilogue -> weighted combine, with hidden 2048, 64 routed + 1 shared EXL3 expert,
intermediate 1536, K = 4 bits. Inputs are seeded synthetic tensors already resident in HBM. Steps run as HIP-graph
replays; each step uses one of `--copies` distinct copies of the layer's expert weights (16 x 308 MB; a copy comes
back after 15 other token-layers, about 356 MB of other traffic, more than the 256 MB Infinity Cache holds) and a
fresh routing, so weights stream from HBM.

Also measured in the same run:
  roofline      the dominant kernel (the layer's gate/up launch) timed inside the layer's own launch sequence with
                HIP events on its stream, its algorithmic bytes per launch / average launch time against the 8 TB/s
                HBM peak, with the down launch and the whole layer beside it;
  cpu_baseline  the scalar CPU oracle (decode + fp32 matvec of the token's 5 experts, oracle/gfr_oracle.c) on a
                bounded sample of tokens, 1 thread;
  prefill       config 4 (8192 tokens, uniform top-4) through the prefill path, against the fp16 MFMA peak;
  other_configs configs 1, 3 and 5 (decode and prefill), each against its HBM or MFMA roofline, and the reference's
                own layer geometry with its FP8 shared expert.
Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "glm-flash-rs_amd"))
sys.path.insert(1, os.path.join(ROOT, "oracle"))   # the cpu_baseline leg's checker / timed CPU path only

METRIC = "MoE-layer tok/s at bs1 decode & 8K prefill; % of HBM BW / MFMA peak"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published (no sparsity)
D, N, E, TOPK, BITS = 2048, 1536, 64, 4, 4
SLOTS = TOPK + 1


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_of(fn_steps, stream):
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for f in fn_steps:
                f()
    return g


def time_graphs(plan, stream, lead=()):
    """plan: list of graphs replayed in order; returns seconds between HIP events recorded on `stream`. lead: graphs
    replayed (untimed) right before the start event with no synchronisation in between, so that the GPU is still
    busy while the host submits the timed replays."""
    import torch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):          # a graph replays on the current stream: time on that stream
        for g in lead:
            g.replay()
        start.record(stream)
        for g in plan:
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


def ramp(graph, stream, seconds):
    """Untimed replays of `graph` for at least `seconds` of wall time: the GPU's clocks reach their steady state under
    back-to-back work (the first tens of ms of a layer loop run measurably slower on MI355X)."""
    import torch
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        while time.perf_counter() - t0 < seconds:
            for _ in range(8):
                graph.replay()
            stream.synchronize()


def decode_bench(args):
    """Config 2: `args.steps` bs=1 layer steps as the replay of one HIP graph of exactly those steps. Step j uses
    weight copy j % copies and routing j % routings. First an untimed clock ramp (`--ramp-ms` of graph replays of
    `--warmup` steps on routings the timed steps do not use, whatever --warmup is: the first tens of ms of a layer loop
    run measurably slower on MI355X); then, unsynchronised, a graph of the LEAD steps that precede step 0 in the cycle,
    still running when the timed replay is submitted, so that the first timed step meets the cache and queue state of
    any step of a long run. Both graphs are replayed once before the ramp: the first replay of a graph is several us
    slower on this stack, which a 20-step timed run would otherwise charge to its few steps. Also times the layer's first launch alone and its
    first two launches (the same steps, gfr_moe_set_launches), which gives each launch's share of a step inside the
    layer's own sequence."""
    import torch
    import gfr_moe
    import synth
    stream = torch.cuda.Stream()
    copies = [synth.experts(E + 1, D, N, BITS, seed=1000 + 17 * c) for c in range(args.copies)]
    R = args.routings
    xs = synth.activations(R, D, 5)
    logits = synth.logits(R, E, 6)
    moe = gfr_moe.Moe(D, N, E, TOPK, 1)
    lead = 32

    def step(j, r=None):
        r = j % R if r is None else r % R
        return lambda: moe.run(copies[j % len(copies)], xs[r:r + 1], logits[r:r + 1], 1, stream=stream)

    with torch.cuda.stream(stream):
        for j in range(len(copies)):
            step(j)()
    stream.synchronize()
    per_launch = {}
    for launches in (1, 2, 0):
        moe.set_launches(launches)
        nw = max(args.warmup, 1)
        warm = graph_of([step(len(copies) // 2 + j, R // 2 + j) for j in range(min(nw, 64))], stream)
        pre = graph_of([step(j) for j in range(-lead, 0)], stream)
        timed = graph_of([step(j) for j in range(args.steps)], stream)
        # the first replay of a graph is slower (its launch set-up): one untimed replay of each, before the ramp
        time_graphs([pre, timed], stream)
        ramp(warm, stream, args.ramp_ms / 1e3)
        per_launch[launches] = time_graphs([timed], stream, lead=[pre])
        del warm, pre, timed
    moe.set_launches(0)
    secs = per_launch[0]
    # the replayed layer computed what an eager run of the last timed step computes
    replayed = moe.output[0].clone()
    with torch.cuda.stream(stream):
        step(args.steps - 1)()
    stream.synchronize()
    if not (torch.isfinite(replayed).all() and torch.equal(replayed, moe.output[0])):
        raise RuntimeError("graph-replayed MoE layer differs from the eager run")
    launches_us = {"gate_up": per_launch[1] / args.steps * 1e6,
                   "down": (per_launch[2] - per_launch[1]) / args.steps * 1e6,
                   "finish": (per_launch[0] - per_launch[2]) / args.steps * 1e6}
    return secs, copies, xs, logits, stream, launches_us


def layer_bytes():
    """Algorithmic HBM bytes of one config-2 token-layer, per launch (each input read once, each output written once):
    gate/up: 5 experts' gate and up trellis, their input scales, the token, the router logits, the gate/up K-split
    partials written; down: 5 down trellis, the epilogue's scales, the partials read, the transformed k-block parts
    written, the down input xd written; finish: the parts read, y and the output written, the routing weights."""
    slots, skgu, skd = SLOTS, D // 512, N // 128
    trellis = D * N * BITS // 8
    gate_up = slots * 2 * trellis + slots * 2 * D * 2 + D * 2 + E * 4 + 2 * skgu * slots * N * 4
    down = slots * trellis + slots * (3 * N * 2 + D * 2) + 2 * skgu * slots * N * 4 + skd * slots * D * 4 + slots * N * 2
    finish = skd * slots * D * 4 + slots * D * 4 + D * 4 + slots * 4
    return {"gate_up": gate_up, "down": down, "finish": finish}


def measured_traffic():
    """HBM bytes per launch of the roofline kernel from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE per dispatch, each scaled by the same counter's reading on a plain copy of known size)."""
    path = os.path.join(ROOT, "profiles", "decode_layer_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return t.get("gate_up_hbm_bytes_per_launch")


def calibrate_copy():
    """A plain 256 MiB device copy, three times: the reference reading for the FETCH_SIZE / WRITE_SIZE counters
    (run under rocprofv3 --pmc with --calibrate-copy)."""
    import torch
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def measure_copy(nbytes=1 << 30, reps=5):
    """A plain device-to-device copy of 1 GiB (torch's copy kernel), timed with HIP events: the bytes it reads plus
    the bytes it writes over its time, the part's achievable HBM rate beside the published 8 TB/s peak."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    secs = e0.elapsed_time(e1) / 1e3 / reps
    del src, dst
    torch.cuda.empty_cache()
    return round(2 * nbytes / secs / 1e9, 1)


def prefill_bench(args, copies, stream):
    """Config 4: one MoE layer on an 8192-token prefill chunk, uniform top-4 routing (+ the shared expert)."""
    import torch
    import gfr_moe
    import synth
    rows = args.prefill_rows
    moe = gfr_moe.Moe(D, N, E, TOPK, rows)
    xs = synth.activations(rows, D, 21)
    lgs = [synth.logits(rows, E, 22 + j) for j in range(2)]
    ws = copies[:2]

    def step(j):
        return lambda: moe.run(ws[j % 2], xs, lgs[j % 2], rows, stream=stream)

    g = graph_of([step(0), step(1)], stream)
    # untimed layers first: on MI355X the layer time falls from about 1.5 to about 1.28 ms over its first ~30 back-
    # to-back layers (clock ramp), and the timed layers are the steady state after it
    time_graphs([g] * max(args.prefill_warmup // 2, 1), stream)
    n = max(args.prefill_steps // 2, 1)
    secs = time_graphs([g] * n, stream) / (2 * n)
    pairs_routed, pairs_shared = rows * TOPK, rows
    flop = (pairs_routed + pairs_shared) * 2 * (2 * D * N + N * D)
    tflops = flop / secs / 1e12
    return {"config": f"config 4: {rows} tokens x top-4 uniform + shared, one MoE layer (route, group, rotate, "
                      "gate/up + down MFMA grouped GEMMs, combine)",
            "tok_per_s": round(rows / secs, 1), "ms_per_layer": round(secs * 1e3, 4),
            "gflop": round(flop / 1e9, 1), "gflop_routed_only": round(pairs_routed * 2 * 3 * D * N / 1e9, 1),
            "achieved_tflops": round(tflops, 1), "mfma_peak_tflops": MFMA_F16_PEAK_TFLOPS,
            "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}


def other_configs(args, copies, stream):
    """The other BASELINE configs, each against its own roofline (secondary lines; `value` stays config 2):
      c1   one EXL3 linear 2048 -> 1536, K = 4, one fp16 token, cycled over >= 2 GiB of distinct weight copies;
      c3   the 32-token verify window (Zipf(1.1) top-4) through the layer's decode path, over the 8 layer copies;
      c5   the 4-layer hidden-5120 stack (160 + 1 experts, top-8, K = 2, 3, 4, 5): bs=1 decode (Zipf top-8) and
           one 16384-token prefill chunk (Zipf) per step."""
    import numpy as np
    import torch
    import gfr_moe
    import synth
    out = {}

    # ---- c1
    kin, n = 2048, 1536
    per = kin * n * BITS // 8
    ncopy = max(2 * 1024 ** 3 // per + 1, 2)
    pool = synth.trellis((ncopy, kin // 16, n // 16, 8 * BITS), 901)
    suh, svh = synth.scales((kin,), 902), synth.scales((n,), 903)
    x = torch.randn(kin, device="cuda").half()
    y = torch.empty(n, device="cuda")
    lin = gfr_moe.Linear(kin, n, BITS)
    glen = min(ncopy, 1024)
    graph = graph_of([(lambda j=j: lin.run(x, pool[j], suh, svh, y, stream=stream)) for j in range(glen)], stream)
    reps = max(args.extra_launches // glen, 1)
    time_graphs([graph], stream)
    secs = time_graphs([graph] * reps, stream) / (reps * glen)
    algo = per + kin * 2 + n * 2 + kin * 2 + n * 4
    out["c1"] = {"config": "config 1: one EXL3 linear 2048->1536, K=4, one fp16 token", "us": round(secs * 1e6, 3),
                 "bytes": algo, "gbs": round(algo / secs / 1e9, 1), "hbm_frac": round(algo / secs / 1e9 / HBM_PEAK_GBS, 4),
                 "weight_copies": ncopy}
    del pool, graph, lin
    torch.cuda.empty_cache()

    # ---- c3: 32 tokens (4 streams x 8 drafts), Zipf(1.1) top-4, the layer's decode path
    rows = 32
    moe = gfr_moe.Moe(D, N, E, TOPK, rows)
    R = 16
    xs = synth.activations(R * rows, D, 911)
    lgs = synth.zipf_logits(R * rows, E, TOPK, 1.1, 912)
    uniq = []
    for j in range(R):
        picks, _ = gfr_moe.route(lgs[j * rows:(j + 1) * rows], TOPK)
        uniq.append(len(set(picks.cpu().numpy().reshape(-1).tolist())))
    glen = R * len(copies)
    graph = graph_of([(lambda j=j: moe.run(copies[j % len(copies)], xs[(j % R) * rows:(j % R + 1) * rows],
                                           lgs[(j % R) * rows:(j % R + 1) * rows], rows, stream=stream))
                      for j in range(glen)], stream)
    time_graphs([graph], stream)
    reps = 4
    secs = time_graphs([graph] * reps, stream) / (reps * glen)
    expert_bytes = 3 * D * N * BITS // 8 + (3 * D + 3 * N) * 2     # trellis + suh_g,u,d / svh_g,u,d
    algo = float(np.mean(uniq)) * expert_bytes + rows * D * 2 + rows * D * 4
    out["c3"] = {"config": "config 3: 32-token verify window, Zipf(1.1) top-4 + shared, one MoE layer (the layer's default path for 32 rows: split-K MFMA programs)",
                 "us_per_window": round(secs * 1e6, 2), "tok_per_s": round(rows / secs, 1),
                 "distinct_experts_mean": round(float(np.mean(uniq)), 2), "bytes_per_window": int(algo),
                 "gbs": round(algo / secs / 1e9, 1), "hbm_frac": round(algo / secs / 1e9 / HBM_PEAK_GBS, 4)}
    del graph, moe
    torch.cuda.empty_cache()

    # ---- the reference's own layer geometry (experts.rs:146-156, moe.rs:132-167): hidden 4096, intermediate 512,
    # 288 routed EXL3 experts (K = 4) top-8 with GLM's gate + the FP8 shared expert, one token, Zipf(1.1) routing
    Dr, Nr, Er, Kr = 4096, 512, 288, 8
    rc = [synth.experts(Er, Dr, Nr, BITS, seed=960 + c) for c in range(4)]
    rs = [synth.fp8_shared(Dr, Nr, seed=970 + c) for c in range(4)]
    bias = torch.zeros(Er, device="cuda")
    mr = gfr_moe.Moe(Dr, Nr, Er, Kr, 1, shared_exl3=False)
    mr.set_router(bias, 2.5)
    R = 16
    xr = synth.activations(R, Dr, 971)
    lr = synth.zipf_logits(R, Er, Kr, 1.1, 972)
    glen = 4 * R
    graph = graph_of([(lambda j=j: mr.run_fp8(rc[j % 4], xr[j % R:j % R + 1], lr[j % R:j % R + 1], rs[j % 4], 1,
                                              stream=stream)) for j in range(glen)], stream)
    time_graphs([graph], stream)
    reps = 8
    secs = time_graphs([graph] * reps, stream) / (reps * glen)
    shared_bytes = 3 * Dr * Nr + 2 * (2 * Nr + Dr) + Dr * 2 + Dr * 4
    tok_bytes = Kr * (3 * Dr * Nr * BITS // 8 + (3 * Dr + 3 * Nr) * 2) + shared_bytes
    sh = gfr_moe.SharedFp8(Dr, Nr, 1)
    so = torch.empty((1, Dr), device="cuda")
    g2 = graph_of([(lambda j=j: sh.run(rs[j % 4], xr[j % R:j % R + 1], 1, out=so, stream=stream))
                   for j in range(glen)], stream)
    time_graphs([g2], stream)
    s2 = time_graphs([g2] * reps, stream) / (reps * glen)
    # the same layer on a 4096-row prefill window (the reference's FastExperts probe size), its shared expert in the
    # prefill form (bf16 copies, library GEMMs)
    rows_p = 4096
    mp = gfr_moe.Moe(Dr, Nr, Er, Kr, rows_p, shared_exl3=False)
    mp.set_router(bias, 2.5)
    for w in rs:
        w.prepare_bf16(stream)
    xp = synth.activations(rows_p, Dr, 973)
    lp = synth.zipf_logits(rows_p, Er, Kr, 1.1, 974)
    gp = graph_of([(lambda c=c: mp.run_fp8(rc[c], xp, lp, rs[c], rows_p, stream=stream)) for c in range(4)], stream)
    time_graphs([gp], stream)
    sp = time_graphs([gp] * 2, stream) / 8
    flop_p = rows_p * (Kr + 1) * 2 * 3 * Dr * Nr
    del gp, mp
    out["reference_layout"] = {
        "config": "the reference's layer geometry: hidden 4096, intermediate 512, 288 routed EXL3 experts (K=4) top-8 "
                  "(GLM gate) + the FP8 shared expert (moe.rs:132-167), one token, Zipf(1.1); the shared expert "
                  "runs inside the layer's gate/up and down launches", "us_per_token": round(secs * 1e6, 2),
        "tok_per_s": round(1 / secs, 1), "bytes_per_token": tok_bytes, "gbs": round(tok_bytes / secs / 1e9, 1),
        "hbm_frac": round(tok_bytes / secs / 1e9 / HBM_PEAK_GBS, 4),
        "shared_fp8_alone_us": round(s2 * 1e6, 2), "shared_fp8_bytes": shared_bytes,
        "prefill_4096_rows_ms": round(sp * 1e3, 3), "prefill_tflops": round(flop_p / sp / 1e12, 1),
        "prefill_mfma_frac": round(flop_p / sp / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    del graph, g2, mr, sh, rc, rs
    torch.cuda.empty_cache()

    # ---- the shared-expert fork and the routed-expert read hints (shared_expert.rs, l2_prefetch.rs)
    out["shared_branch_and_hints"] = prefetch_leg(copies, stream)
    torch.cuda.empty_cache()

    # ---- c5: 4 layers, hidden 5120, 160 routed + 1 shared, top-8, K = 2, 3, 4, 5
    D5, N5, E5, K5 = 5120, 1536, 160, 8
    bits5 = (2, 3, 4, 5)
    layers = [synth.experts(E5 + 1, D5, N5, b, seed=920 + 10 * b) for b in bits5]
    decode = gfr_moe.Moe(D5, N5, E5, K5, 1)
    R = 16
    x5 = synth.activations(R, D5, 931)
    l5 = synth.zipf_logits(R, E5, K5, 1.1, 932)
    graph = graph_of([(lambda j=j, l=l: decode.run(layers[l], x5[j:j + 1], l5[j:j + 1], 1, stream=stream))
                      for j in range(R) for l in range(4)], stream)
    time_graphs([graph], stream)
    reps = 8
    secs = time_graphs([graph] * reps, stream) / (reps * R)
    stack_bytes = sum((K5 + 1) * 3 * D5 * N5 * b // 8 for b in bits5)
    out["c5_decode"] = {"config": "config 5: 4-layer stack (K=2,3,4,5), hidden 5120, 160+1 experts, top-8, bs=1 "
                                  "decode, Zipf(1.1)", "us_per_token": round(secs * 1e6, 2),
                        "tok_per_s": round(1 / secs, 1), "bytes_per_token": stack_bytes,
                        "gbs": round(stack_bytes / secs / 1e9, 1),
                        "hbm_frac": round(stack_bytes / secs / 1e9 / HBM_PEAK_GBS, 4)}
    del graph, decode
    torch.cuda.empty_cache()
    if not args.no_prefill:
        rows5 = args.c5_prefill_rows
        pre = gfr_moe.Moe(D5, N5, E5, K5, rows5)
        xp = synth.activations(rows5, D5, 941)
        lp = synth.zipf_logits(rows5, E5, K5, 1.1, 942) if rows5 <= 4096 else _zipf_logits_gpu(rows5, E5, K5, 1.1, 943)
        graph = graph_of([(lambda l=l: pre.run(layers[l], xp, lp, rows5, stream=stream)) for l in range(4)], stream)
        time_graphs([graph], stream)
        reps = 2
        secs = time_graphs([graph] * reps, stream) / reps
        flop = 4 * rows5 * (K5 + 1) * 2 * 3 * D5 * N5
        out["c5_prefill"] = {"config": f"config 5: 4-layer stack, one {rows5}-token prefill chunk per layer, "
                                       "Zipf(1.1) top-8 + shared", "ms_per_chunk_4_layers": round(secs * 1e3, 3),
                             "tok_per_s": round(rows5 / secs, 1), "tflops": round(flop / secs / 1e12, 1),
                             "mfma_frac": round(flop / secs / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
        del graph, pre
    del layers
    torch.cuda.empty_cache()

    # ---- prepared-weight loader: config 2's 65 experts written in the reference's format, loaded with every chunk's
    # SHA-256 checked (file -> pinned staging -> HBM)
    import tempfile
    with tempfile.TemporaryDirectory() as tmp:
        chunk = 16 << 20
        path = gfr_moe.write_prepared(tmp, [copies[0]], chunk=chunk)
        prep = gfr_moe.Prepared(path)
        nbytes, secs = prep.load()
        nbytes, secs = prep.load()
        prep.close()
    nchunks = -(-nbytes // chunk)
    out["loader"] = {"config": "prepared-weight load of config 2's 65 EXL3 experts (src/prepared.rs format, 16 MiB "
                               "chunks, each SHA-256-checked, file in the page cache)",
                     "bytes": nbytes, "seconds": round(secs, 4), "gbs": round(nbytes / secs / 1e9, 3),
                     "hash_tasks_in_flight_max": min(2 * min(16, os.cpu_count() or 1), nchunks)}
    return out


def prefetch_leg(copies, stream, reps=8):
    """The shared-expert fork and the routed-expert read hints of the reference's decode round (shared_expert.rs
    Branch::run, l2_prefetch.rs Owner::experts + l2pf.cu), at config 2's shape for one token: group the routed token,
    then the shared expert's work (an FP8 shared expert of that shape, gfr_moe.SharedFp8: 9.4 MB of weights, two
    launches) and the routed experts (ExpertGpu, 4 EXL3 slots). Three forms, each a graph of 64 steps
    over the 16 cold weight copies, timed alternately:
      serial   shared work, then the routed experts, on one stream;
      branch   the shared work on a forked stream (gfr_moe.SharedBranch), joined after the routed experts;
      hinted   serial, plus the hint of the routed experts' gate/up heads forked onto a side stream right after the
               grouping (gfr_moe.Prefetch) and joined at the end."""
    import torch
    import gfr_moe
    import synth
    rows, R = 1, 16
    g = gfr_moe.Grouping(E + 1, SLOTS, rows)
    ex = gfr_moe.ExpertGpu(D, N, SLOTS, TOPK, rows)
    pf = gfr_moe.Prefetch()
    br = gfr_moe.SharedBranch()
    stride = copies[0].gt[0].numel() * 4
    T = gfr_moe.PfTensor
    for k, w in enumerate(copies):
        pf.add_experts(k, gfr_moe.pf_experts(T(w.gt.data_ptr(), E * stride), T(w.ut.data_ptr(), E * stride), E))
    plan = pf.expert_plans[0][1]
    xs = synth.activations(R, D, 951)
    picks, _ = gfr_moe.route(synth.logits(R, E, 952), TOPK)
    sw = synth.fp8_shared(D, N, seed=953)
    sh = gfr_moe.SharedFp8(D, N, rows)
    shared = torch.empty(rows, D, device="cuda")

    def step(j, form):
        def f():
            c, r = j % len(copies), j % R
            p = picks[r:r + 1]

            def shared_fn(st=None):
                sh.run(sw, xs[r:r + 1], rows, out=shared, stream=st if st is not None else stream)

            def routed(ready=None):
                ex.run_rows(copies[c], xs[r:r + 1], p, g.ids, g.count, g.members, rows, rows, stream=stream)

            g.run(p, rows, stream=stream)
            if form == "branch":
                br.run(stream, shared_fn, routed)
                return
            if form == "hinted":
                pf.experts(stream, c, rows, g.ids, g.count)
            shared_fn()
            routed()
            if form == "hinted":
                pf.join(stream)
        return f

    forms = ("serial", "branch", "hinted")
    with torch.cuda.stream(stream):
        for form in forms:
            step(0, form)()
    stream.synchronize()
    glen = 4 * len(copies)
    graphs = {form: graph_of([step(j, form) for j in range(glen)], stream) for form in forms}
    us = {form: [] for form in forms}
    for form in forms:
        time_graphs([graphs[form]] * 2, stream)
    for _ in range(reps):
        for form in forms:
            us[form].append(time_graphs([graphs[form]] * 4, stream) / (4 * glen) * 1e6)
    med = {k: round(sorted(v)[len(v) // 2], 3) for k, v in us.items()}
    return {"config": "config 2 shape, one token: grouping, an FP8 shared expert (SharedFp8, 9.4 MB), routed experts "
                      "(ExpertGpu, 4 EXL3 slots); 16 cold weight copies",
            "us_per_step_serial": med["serial"], "us_per_step_shared_branch": med["branch"],
            "us_per_step_hinted": med["hinted"], "hint_bytes_per_step": 2 * TOPK * plan.bytes}


def _zipf_logits_gpu(rows, E, topk, s, seed):
    """Zipf(s) top-k routing logits for many rows, built on the GPU (same construction as synth.zipf_logits:
    distinct experts drawn with probability 1 / (rank + 1)^s over a seeded permutation, picked logits above the
    rest and decreasing with the slot)."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    perm = torch.randperm(E, generator=g, device="cuda")
    p = 1.0 / torch.arange(1, E + 1, device="cuda", dtype=torch.float64) ** s
    chosen = torch.multinomial((p / p.sum()).float().expand(rows, E), topk, replacement=False, generator=g)
    base = torch.randn((rows, E), generator=g, device="cuda")
    vals = (8.0 - 0.25 * torch.arange(topk, device="cuda", dtype=torch.float32)).expand(rows, topk)
    base.scatter_(1, perm[chosen], vals.contiguous())
    return base


def cpu_baseline(args, copies, xs, logits):
    import numpy as np
    import torch
    import oracle
    from_refs = os.path.join(ROOT, "tests")
    sys.path.insert(0, from_refs)
    from refs import np_u16, np_u32
    w = copies[0]
    picks, _ = oracle.route(logits[:args.cpu_tokens].cpu().numpy(), TOPK, E)
    need = sorted(set(int(e) for e in picks.reshape(-1)))
    remap = {e: i for i, e in enumerate(need)}
    sub = {n: np.ascontiguousarray(np_u32(getattr(w, n)[need])) for n in ("gt", "ut", "dt")}
    vec = {n: np.ascontiguousarray(np_u16(getattr(w, n)[need])) for n in ("suh_g", "suh_u", "suh_d", "svh_g", "svh_u",
                                                                        "svh_d")}
    xb = np_u16(xs[:args.cpu_tokens])

    def token(t):
        ex = [remap[int(e)] for e in picks[t % args.cpu_tokens]]
        secs, _ = oracle.baseline_decode(xb[t % args.cpu_tokens], D, N, BITS, ex, sub["gt"], sub["ut"], sub["dt"],
                                         vec["suh_g"], vec["suh_u"], vec["suh_d"], vec["svh_g"], vec["svh_u"],
                                         vec["svh_d"])
        return secs

    total = sum(token(t) for t in range(args.cpu_tokens))
    one = {"value": round(args.cpu_tokens / total, 4), "unit": "tok/s", "cores": 1, "kind": "port",
           "cpu_model": cpu_model(),
           "sample": f"{args.cpu_tokens} tokens of config 2: per token the 5 experts' gate/up/down trellis decode "
                     f"+ fixed-order fp32 matvec + epilogues (oracle/gfr_oracle.c, scalar, 1 thread)",
           "seconds": round(total, 2)}
    # the same work on every host core the box gives this job: one token a thread (the C call drops the GIL)
    from concurrent.futures import ThreadPoolExecutor
    threads = max(1, min(args.cpu_threads, len(os.sched_getaffinity(0))))
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(token, range(threads)))
    wall = time.perf_counter() - t0
    many = {"value": round(threads / wall, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{threads} tokens of config 2 at once, one a thread, same scalar C path", "seconds": round(wall, 2)}
    return one, many


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline_c1(tokens=16, threads=16):
    """Config 1 on the host: per token the 2048 x 1536 K = 4 trellis decoded (gfro_unpack_f32) and the linear
    (gfro_linear: input scales, transform, fixed-order fp32 matvec, output transform and scales), scalar C, 1 thread,
    on seeded weights and fp16 tokens of the config's shape."""
    import numpy as np
    import oracle
    kin, n = 2048, 1536
    rng = np.random.default_rng(5)
    words = rng.integers(0, 2 ** 32, (kin // 16, n // 16, 8 * BITS), dtype=np.uint64).astype(np.uint32)
    sc = lambda k: ((rng.integers(0, 2, k) * 2 - 1) * (rng.random(k) + 0.5)).astype(np.float16).view(np.uint16)
    suh, svh = sc(kin), sc(n)
    xs = rng.standard_normal((tokens, kin)).astype(np.float16).view(np.uint16)
    def token(t):
        oracle.linear(xs[t % tokens], oracle.unpack_f32(words, kin, n, BITS), suh, svh)

    t0 = time.perf_counter()
    for t in range(tokens):
        token(t)
    secs = time.perf_counter() - t0
    one = {"value": round(tokens / secs, 3), "unit": "tok/s", "cores": 1, "kind": "port", "cpu_model": cpu_model(),
           "sample": f"{tokens} tokens of config 1: per token the trellis decode + linear (oracle/gfr_oracle.c, "
                     "scalar, 1 thread)", "seconds": round(secs, 2)}
    # every core the job may use: one token a thread (the C calls drop the GIL)
    from concurrent.futures import ThreadPoolExecutor
    nt = max(1, min(threads, len(os.sched_getaffinity(0))))
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=nt) as ex:
        list(ex.map(token, range(2 * nt)))
    wall = time.perf_counter() - t0
    many = {"value": round(2 * nt / wall, 3), "unit": "tok/s", "cores": nt, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{2 * nt} tokens of config 1 over {nt} threads, one token a thread at a time, same scalar C path",
            "seconds": round(wall, 2)}
    return one, many


def cpu_baseline_c3(copies, rows=32, threads=16):
    """Config 3 on the host, row-batched: one 32-token Zipf(1.1) window; each distinct expert's trellis decoded once
    (gfro_unpack_f32), then every member row through it (gfro_expert_row: rotation, fixed-order fp32 matvecs,
    epilogues), then the combine; scalar C, 1 thread."""
    import numpy as np
    import oracle
    import synth
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from refs import np_u16, np_u32
    w = copies[0]
    x = np_u16(synth.activations(rows, D, 961))
    picks, weights = oracle.route(synth.zipf_logits(rows, E, TOPK, 1.1, 962).cpu().numpy(), TOPK, E)
    used = sorted(set(int(e) for e in picks.reshape(-1)))
    words = {e: (np_u32(w.gt[e]), np_u32(w.ut[e]), np_u32(w.dt[e])) for e in used}
    vec = {nm: np_u16(getattr(w, nm)) for nm in ("suh_g", "suh_u", "suh_d", "svh_g", "svh_u", "svh_d")}
    y = np.empty((rows, SLOTS, D), np.float32)

    def expert(e):
        wg, wu, wd = (oracle.unpack_f32(words[e][0], D, N, BITS), oracle.unpack_f32(words[e][1], D, N, BITS),
                      oracle.unpack_f32(words[e][2], N, D, BITS))
        for r, s in zip(*np.nonzero(picks == e)):
            y[r, s] = oracle.expert_row(x[r], wg, wu, wd, *(vec[nm][e] for nm in ("suh_g", "suh_u", "suh_d", "svh_g",
                                                                                   "svh_u", "svh_d")),
                                        sk_gu=1, sk_d=1, warps=1)[0]

    t0 = time.perf_counter()
    for e in used:
        expert(e)
    oracle.combine(y, weights, rows, SLOTS)
    secs = time.perf_counter() - t0
    one = {"value": round(rows / secs, 3), "unit": "tok/s", "cores": 1, "kind": "port", "cpu_model": cpu_model(),
           "sample": f"one {rows}-token window of config 3 ({len(used)} distinct experts, each decoded once, then "
                     "its member rows; oracle/gfr_oracle.c, scalar, 1 thread)", "seconds": round(secs, 2)}
    # every core the job may use: the window's experts dealt to the threads (the C calls drop the GIL)
    from concurrent.futures import ThreadPoolExecutor
    nt = max(1, min(threads, len(os.sched_getaffinity(0))))
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=nt) as ex:
        list(ex.map(expert, used))
    oracle.combine(y, weights, rows, SLOTS)
    wall = time.perf_counter() - t0
    many = {"value": round(rows / wall, 3), "unit": "tok/s", "cores": nt, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"the same window with its {len(used)} experts dealt over {nt} threads", "seconds": round(wall, 2)}
    return one, many


def counter_summary(path):
    """Per-kernel averages of every counter in a rocprofv3 --pmc ... --output-format csv counter_collection.csv (one
    line per kernel of this library: dispatches, counter = mean value per dispatch)."""
    import csv
    import collections
    sums = collections.defaultdict(lambda: collections.defaultdict(float))
    disp = collections.defaultdict(set)
    with open(path) as f:
        for r in csv.DictReader(f):
            k = r["Kernel_Name"]
            sums[k][r["Counter_Name"]] += float(r["Counter_Value"])
            disp[k].add(r["Dispatch_Id"])
    for k in sorted(sums, key=lambda k: -len(disp[k])):
        n = len(disp[k])
        print(json.dumps({"kernel": k, "dispatches": n, **{c: round(v / n, 1) for c, v in sums[k].items()}}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--ramp-ms", type=float, default=300.0, help="untimed decode replays (wall ms) before each "
                    "timed decode replay, whatever --warmup is: the clock ramp")
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--routings", type=int, default=64)
    ap.add_argument("--cpu-tokens", type=int, default=12)
    ap.add_argument("--cpu-threads", type=int, default=16, help="threads of the all-cores CPU baseline (capped "
                    "at the cores this process may use)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-rows", type=int, default=8192)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--prefill-warmup", type=int, default=40, help="untimed prefill layers before the timed ones")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true", help="first run a 256 MiB copy (counter reference)")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary config 1 / 3 / 5 lines")
    ap.add_argument("--extra-launches", type=int, default=4096)
    ap.add_argument("--c5-prefill-rows", type=int, default=16384)
    ap.add_argument("--hints-only", action="store_true", help="run only the shared-expert fork / read-hint leg "
                    "and print its JSON (for a kernel trace of it)")
    ap.add_argument("--counter-summary", metavar="CSV", help="print per-kernel counter averages of a rocprofv3 "
                    "counter_collection.csv and exit (no GPU work)")
    args = ap.parse_args()
    if args.counter_summary:
        counter_summary(args.counter_summary)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.hints_only:
        import torch
        import synth
        copies = [synth.experts(E + 1, D, N, BITS, seed=1000 + 17 * c) for c in range(args.copies)]
        print(json.dumps(prefetch_leg(copies, torch.cuda.Stream())), flush=True)
        return
    if args.calibrate_copy:
        calibrate_copy()
    secs, copies, xs, logits, stream, launches_us = decode_bench(args)
    log(f"decode: {args.steps} steps in {secs * 1e3:.2f} ms; per launch (us): {launches_us}")
    nbytes = layer_bytes()
    layer_total = sum(nbytes.values())
    us_step = secs * 1e6 / args.steps
    gu_gbs = nbytes["gate_up"] / launches_us["gate_up"] / 1e3
    read_ahead = SLOTS * D * N * BITS // 8
    roof = {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "measured_copy_gbs": measure_copy(),
            "kernel": "expert_gemv_kernel<4,8,4,2,1,1,true> (the layer's gate/up launch: router, input rotation, "
                      "gate and up trellis GEMV)",
            "bytes_per_launch": nbytes["gate_up"], "us_per_launch": round(launches_us["gate_up"], 3),
            "timing": "HIP events on the layer's stream around graph replays of the layer cut after its first launch "
                      "(gfr_moe_set_launches(1)); includes the launch's share of the inter-kernel gaps",
            "read_ahead": {"bytes": read_ahead,
                           "what": "the gate waves also read each window expert's down trellis once into the "
                                   "memory-side cache for the down launch: in this launch's time and traffic, not in "
                                   "bytes_per_launch (they are the down launch's operand bytes)",
                           "gbs_incl": round((nbytes["gate_up"] + read_ahead) / launches_us["gate_up"] / 1e3, 1)},
            "down": {"kernel": "down_gemv_kernel<4,1,1,true,1,4> (one-wave workgroups: a slot, a 128-output block, a 128-k block)", "bytes_per_launch": nbytes["down"],
                     "us_per_launch": round(launches_us["down"], 3),
                     "gbs": round(nbytes["down"] / launches_us["down"] / 1e3, 1),
                     "frac": round(nbytes["down"] / launches_us["down"] / 1e3 / HBM_PEAK_GBS, 4)},
            "finish": {"kernel": "sum_finish_kernel", "bytes_per_launch": nbytes["finish"],
                       "us_per_launch": round(launches_us["finish"], 3)},
            "layer": {"bytes_per_step": layer_total, "us_per_step": round(us_step, 3),
                      "gbs": round(layer_total / us_step / 1e3, 1),
                      "frac": round(layer_total / us_step / 1e3 / HBM_PEAK_GBS, 4)}}
    log(f"gate/up launch: {roof['us_per_launch']} us, {roof['achieved']} GB/s; layer {roof['layer']['gbs']} GB/s")
    prefill = None
    if not args.no_prefill:
        prefill = prefill_bench(args, copies, stream)
        log(f"prefill: {prefill['ms_per_layer']} ms/layer, {prefill['achieved_tflops']} TFLOP/s")
    extra = None
    if not args.no_extra:
        extra = other_configs(args, copies, stream)
        log("other configs: " + json.dumps(extra))
    cpu = cpu_all = cpu_c1 = cpu_c3 = cpu_c1_all = cpu_c3_all = None
    if not args.no_cpu:
        cpu, cpu_all = cpu_baseline(args, copies, xs, logits)
        (cpu_c1, cpu_c1_all), (cpu_c3, cpu_c3_all) = (cpu_baseline_c1(threads=args.cpu_threads),
                                                      cpu_baseline_c3(copies, threads=args.cpu_threads))
        log(f"cpu baseline c1: {cpu_c1['value']} tok/s ({cpu_c1_all['value']} on {cpu_c1_all['cores']} threads); "
            f"c3: {cpu_c3['value']} tok/s ({cpu_c3_all['value']})")
        log(f"cpu baseline: {cpu['value']} tok/s over {cpu['seconds']} s; {cpu_all['cores']} threads "
            f"{cpu_all['value']} tok/s")
    out = {
        "metric": METRIC, "value": round(args.steps / secs, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(secs * 1e3 / args.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "config 2: one MoE layer, bs=1 decode, hidden 2048, 64 routed + 1 shared EXL3 "
                               "experts, inter 1536, top-4, K=4", "global_batch": 1, "seq_len": 1,
                   "parallelism": "single-gpu", "weight_copies": args.copies, "routings": args.routings,
                   "weight_bytes_cycled": int(args.copies * (E + 1) * 3 * D * N * BITS // 8)},
        "roofline": roof, "cpu_baseline": cpu, "cpu_baseline_all_cores": cpu_all,
        "cpu_baseline_other_configs": {"c1": cpu_c1, "c1_all_cores": cpu_c1_all, "c3": cpu_c3,
                                       "c3_all_cores": cpu_c3_all}, "prefill": prefill,
        "other_configs": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
