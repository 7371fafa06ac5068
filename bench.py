#!/usr/bin/env python3
"""Throughput of the quantized MoE expert-FFN path on one MI355X.

Headline workload (`value`): 512-token prefill of one MoE layer -- d_model 2048, 128 experts, top-8, expert
intermediate 768, Q4_K gate/up, Q6_K down, router logits biased so tokens per expert follow Zipf(1.1)
(log p_zipf + Gumbel noise added to the fp32 router GEMV).  One step = router GEMV -> softmax/top-k ->
bucketing -> Q8_K activations -> grouped int8-MFMA gate/up GEMM (SwiGLU) -> Q8_K hidden -> grouped down GEMM
-> combine, with every input already in HBM.  Each step uses a fresh (activations, routing) pair and one of
several independent weight copies, so the 256 MB MALL does not serve the weights.  Steps are replayed from a
HIP graph (captured once, checked against an eager run first).

Secondary (`decode` object): 1-token decode of the same layer shape in Q4_K/Q4_K, three launches: router GEMV +
Q8 of x -> routing + gate/up GEMV -> down GEMV + combine, cycling 4 layer copies (1.36 GB) and fresh tokens.  Its
per-kernel figures time each launch alone over the same 64 (token, copy) pairs, so they stream cold weights too.

Secondary (`workloads` object): the other configured workloads at their full shapes -- IQ4_NL / IQ4_XS (d_model
4096, 288 experts) at 1 and 4 rows, IQ2_XS (d_model 7168, 384 experts, top-6) with a shared Q4_K expert at 1 and 8
rows, one 2048-token chunk of Q5_K/Q6_K (512 experts, top-10, shared expert) and the whole 16384-token prompt as 8
such chunks (routing drawn per chunk, outputs added into the residual) -- µs per step and the HBM rate of the expert
bytes each step touches; verify batches also through the grouped GEMM path.

`roofline` reports the dominant kernel of the headline step against HBM bandwidth (8 TB/s): algorithmic bytes
per launch / its average launch duration, measured on its own stream with HIP events over graph replays of
that kernel.  `cpu_baseline` is the CPU oracle (this repository's restatement of the reference's CPU expert
path) run on a bounded sample of the same workload on this host.

`--timeline NAME ...` (a profiling mode, no headline line) replays decode steps of the named workloads on the
stamps build of the library (`python -m hyper_amd.build --stamps`: hyper_amd/libhymoe_stamps.so, whose decode
kernels stamp s_memrealtime at their phase boundaries) and prints each step's per-block phase times.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
if "--timeline" in sys.argv:   # the stamps build of the library, loaded in place of the default one
    os.environ.setdefault("HYMOE_LIB", str(ROOT / "hyper_amd" / "libhymoe_stamps.so"))

from hyper_amd import moe  # noqa: E402
from hyper_amd.formats import WORKLOADS, activations, q8_row_bytes, random_layer, row_bytes, vec_dot_type, zipf_logit_bias  # noqa: E402

METRIC = "MoE-layer µs/token decode (HBM GB/s) + prefill tokens/s (MFMA util), 1 GPU"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def graph_time(fn_list, replays: int, stream) -> float:
    """Capture fn_list (callables enqueueing work) into one HIP graph, replay `replays` times, return ms per replay."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for fn in fn_list:
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(replays):
        g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    del g
    return a.elapsed_time(b) / replays


def make_layers(w, copies, dev, seed0):
    return [random_layer(w.tg, w.td, w.E, w.ff, w.d, seed=seed0 + c, device=dev, d_range=w.d_range) for c in range(copies)]


def prefill_bench(args, dev, stream):
    w = WORKLOADS["q4k_q6k_prefill512"]
    T, k, E, d, ff = w.rows, w.k, w.E, w.d, w.ff
    g = torch.Generator(device=dev)
    g.manual_seed(1234 + 1)
    layers = make_layers(w, args.copies, dev, 100)
    devs = [moe.MoeDev(L, torch.arange(E, dtype=torch.int32, device=dev)) for L in layers]
    W_rs = [torch.randn(E, d, generator=g, device=dev) * 0.02 for _ in range(args.copies)]
    n_in = args.inputs
    xs = [activations(T, d, g, dev) for _ in range(n_in)]
    biases = [zipf_logit_bias(T, E, w.zipf, g, dev) for _ in range(n_in)]
    runners = [moe.MoeLayerRunner(devs[c], W_rs[c], k, T) for c in range(args.copies)]
    torch.cuda.synchronize()

    # eager step vs graph replay of the same step (what is timed must compute what eager computes)
    with torch.cuda.stream(stream):
        ref = runners[0].prefill(xs[0], biases[0]).clone()
        torch.cuda.synchronize()
        gg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gg, stream=stream):
            runners[0].prefill(xs[0], biases[0])
        gg.replay()
        torch.cuda.synchronize()
        if not torch.equal(runners[0].out[:T], ref):
            raise RuntimeError("graph replay of the prefill step differs from the eager step")
        del gg

    # routing statistics per input (the bytes a step must read)
    act = []
    for i in range(n_in):
        r = runners[i % args.copies]
        r.prefill(xs[i], biases[i])
        torch.cuda.synchronize()
        act.append(int(r.order_n[1].item()))
    steps = [(i % args.copies, i % n_in) for i in range(args.graph_steps)]
    fns = [lambda c=c, i=i: runners[c].prefill(xs[i], biases[i]) for c, i in steps]

    with torch.cuda.stream(stream):
        for _ in range(max(1, args.warmup)):
            for f in fns:
                f()
        torch.cuda.synchronize()
        reps = max(1, -(-args.steps // len(fns)))   # whole graphs of len(fns) steps, at least the steps asked for
        ms_graph = graph_time(fns, reps, stream)
    ms_step = ms_graph / len(fns)
    tok_s = T / (ms_step / 1e3)

    # per-kernel launch durations: each grouped GEMM alone, graph-replayed over the copies/inputs
    # (inputs of the last prefill of each (copy, input) pair are still in the runners' workspaces)
    gu_fns, dn_fns = [], []
    for c, i in steps[: 2 * args.copies]:
        r = runners[c]
        gu_fns.append(lambda r=r: moe.moe_gemm_gate_up(r.dev, r.xq, k, T * k, r.order, r.order_n, r.egrp, min(E, T * k), r.h))
        dn_fns.append(lambda r=r: moe.moe_gemm_down(r.dev, r.hq, T * k, r.order, r.order_n, r.egrp, min(E, T * k), r.wts, r.y))
    with torch.cuda.stream(stream):
        for c in range(args.copies):
            runners[c].prefill(xs[c % n_in], biases[c % n_in])
        torch.cuda.synchronize()
        ms_gu = graph_time(gu_fns, max(1, args.kernel_reps), stream) / len(gu_fns)
        ms_dn = graph_time(dn_fns, max(1, args.kernel_reps), stream) / len(dn_fns)
        act_k = [int(runners[c].order_n[1].item()) for c in range(args.copies)]
    n_act = float(np.mean(act_k))
    P = T * k
    L0 = layers[0]
    gu_bytes = n_act * 2 * L0.gate_bytes + T * q8_row_bytes(vec_dot_type(w.tg), d) + P * ff * 4
    dn_bytes = n_act * L0.down_bytes + P * q8_row_bytes(vec_dot_type(w.td), ff) + P * d * 4 + P * 4
    kern = {"gemm_gate_up": {"ms": ms_gu, "bytes": gu_bytes}, "gemm_down": {"ms": ms_dn, "bytes": dn_bytes}}
    dom = max(kern, key=lambda k_: kern[k_]["ms"])
    ach = kern[dom]["bytes"] / (kern[dom]["ms"] / 1e3) / 1e9
    step_bytes = float(np.mean(act)) * L0.expert_bytes() + E * d * 4 + T * d * 4 * 2
    ops = 2.0 * P * 3 * ff * d
    res = {
        "tok_s": tok_s, "ms_step": ms_step, "timed_steps": reps * len(fns), "active_experts_mean": float(np.mean(act)),
        "step_bytes": step_bytes, "step_hbm_gbs": step_bytes / (ms_step / 1e3) / 1e9,
        "step_int8_tops": ops / (ms_step / 1e3) / 1e12,
        "kernels": {k_: {"us": v["ms"] * 1e3, "alg_bytes": v["bytes"], "gbs": v["bytes"] / (v["ms"] / 1e3) / 1e9} for k_, v in kern.items()},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": ach / HBM_PEAK_GBS, "traffic": traffic_from_profile(dom)},
    }
    return res, layers[0], W_rs[0], xs, biases


def decode_bench(args, dev, stream):
    w = WORKLOADS["q4k_decode"]
    k, E, d, ff = w.k, w.E, w.d, w.ff
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    layers = make_layers(w, args.decode_copies, dev, 200)
    devs = [moe.MoeDev(L, torch.arange(E, dtype=torch.int32, device=dev)) for L in layers]
    W_rs = [torch.randn(E, d, generator=g, device=dev) * 0.02 for _ in layers]
    xs = activations(64, d, g, dev)
    runners = [moe.MoeLayerRunner(devs[c], W_rs[c], k, 1) for c in range(len(layers))]
    fns = [lambda c=c, i=i: runners[c].decode(xs[i:i + 1]) for i, c in zip(range(64), [j % len(layers) for j in range(64)])]
    torch.cuda.synchronize()   # the weights, slot tables and inputs come from the default stream
    with torch.cuda.stream(stream):
        for f in fns:
            f()
        torch.cuda.synchronize()
        ms = graph_time(fns, max(1, args.decode_reps), stream) / len(fns)
        # each launch alone, over the step's 64 (token, layer copy) pairs with buffers of their own: every launch
        # routes its own token to its own copy's experts, so the weights come from HBM as in the step, not from the
        # caches a repeated launch would leave them in
        bufs = [{n: getattr(runners[c], n).clone() for n in ("logits", "xq", "ids", "wts", "h", "out")}
                for c in [j % len(layers) for j in range(64)]]
        rq = [lambda r=runners[j % len(layers)], b=b, j=j: moe.moe_router_q8(r.W_r, E, d, xs[j:j + 1], d, b["logits"], E, r.vg, b["xq"], 1)
              for j, b in enumerate(bufs)]
        gu = [lambda r=runners[j % len(layers)], b=b: moe.moe_route_gate_up(r.dev, b["logits"], E, E, k, b["xq"], b["ids"], b["wts"], None, b["h"], 1)
              for j, b in enumerate(bufs)]
        dn = [lambda r=runners[j % len(layers)], b=b: moe.moe_down_reduce(r.dev, b["h"], b["ids"], b["wts"], k, None, None, b["out"], 1)
              for j, b in enumerate(bufs)]
        ms_rq = graph_time(rq, max(1, args.decode_reps), stream) / len(rq)   # (the first replay fills every buffer)
        ms_gu = graph_time(gu, max(1, args.decode_reps), stream) / len(gu)
        ms_dn = graph_time(dn, max(1, args.decode_reps), stream) / len(dn)
        # the floor of a chain of three dependent launches: three elementwise kernels a step on the token's 2048
        # floats, each reading what the one before wrote (a launch boundary and a memory round trip each), replayed
        # in a graph like the step
        sink = torch.zeros(64, d, device=dev)
        def chain(i):
            t = xs[i:i + 1] * 2.0
            t = t + 1.0
            sink[i:i + 1].copy_(t)
        ms_chain = graph_time([lambda i=i: chain(i) for i in range(64)], max(1, args.decode_reps), stream) / 64
    L0 = layers[0]
    tok_bytes = k * L0.expert_bytes() + E * d * 4 + 2 * d * 4
    us = ms * 1e3
    return ({"workload": "q4k_decode", "us_per_token": us, "hbm_gbs": tok_bytes / (us / 1e6) / 1e9,
            "hbm_frac": tok_bytes / (us / 1e6) / 1e9 / HBM_PEAK_GBS, "alg_bytes_per_token": tok_bytes,
            "chain3_floor_us": ms_chain * 1e3,
            "kernels": {"router_q8": {"us": ms_rq * 1e3, "gbs": (E * d * 4 + d * 4) / (ms_rq / 1e3) / 1e9},
                        "route_gate_up": {"us": ms_gu * 1e3, "gbs": k * 2 * L0.gate_bytes / (ms_gu / 1e3) / 1e9},
                        "down_reduce": {"us": ms_dn * 1e3, "gbs": k * L0.down_bytes / (ms_dn / 1e3) / 1e9}}}, layers)


def workloads_bench(args, dev, stream):
    """The other configured workloads at their full shapes (IQ4_NL / IQ4_XS decode and 4-row verify, IQ2_XS with a
    shared Q4_K expert at 1 and 8 rows, one 2048-token Q5_K/Q6_K chunk and the whole 16384-token prompt as 8 such
    chunks): µs per step from graph replays over `workload_copies` weight copies and fresh inputs.  Bytes per step, per
    layer call: the distinct experts its rows route to, the shared expert and the router weights; plus the activations
    in and out.  Verify batches are also timed through the grouped GEMM path (`us_per_step_grouped`)."""
    res = {}
    for name, w in WORKLOADS.items():
        if name in ("q4k_decode", "q4k_q6k_prefill512") or (args.workload and name not in args.workload):
            continue
        C = w.chunk or w.rows   # rows per layer call
        nch = w.rows // C
        copies, n_in, nsteps = args.workload_copies, 4, 8 if nch == 1 else 2
        g = torch.Generator(device=dev)
        g.manual_seed(4321)
        layers = [random_layer(w.tg, w.td, w.E, w.ff, w.d, seed=500 + c, device=dev, d_range=w.d_range, d_range_down=w.d_range_down)
                  for c in range(copies)]
        S = random_layer(w.shared[0], w.shared[1], 1, w.ff, w.d, seed=550, device=dev, d_range=w.d_range) if w.shared else None
        sdev = moe.MoeDev(S, torch.zeros(1, dtype=torch.int32, device=dev)) if S is not None else None
        runners = [moe.MoeLayerRunner(moe.MoeDev(L, torch.arange(w.E, dtype=torch.int32, device=dev)),
                                      torch.randn(w.E, w.d, generator=g, device=dev) * 0.02, w.k, C, shared=sdev) for L in layers]
        xs = [activations(w.rows, w.d, g, dev, lognormal=w.norm_lognormal) for _ in range(n_in)]
        # a chunked prompt draws its routing skew per chunk
        bs = [[zipf_logit_bias(C, w.E, w.zipf, g, dev) if w.zipf else None for _ in range(nch)] for _ in range(n_in)]
        resid = torch.zeros(w.rows, w.d, device=dev) if nch > 1 else None
        decode = w.rows <= 8

        def step(r, x, b, grouped=False):
            if nch > 1:   # the prompt's chunks in order, each chunk's output added into its residual rows
                for j in range(nch):
                    r.prefill(x[j * C:(j + 1) * C], bias=b[j], resid=resid[j * C:(j + 1) * C])
                return resid
            return r.decode(x, bias=b[0]) if decode and not grouped else r.prefill(x, bias=b[0])

        touched = []
        for i in range(n_in):
            for j in range(nch):
                runners[0].prefill(xs[i][j * C:(j + 1) * C], bias=bs[i][j]) if nch > 1 else step(runners[0], xs[i], bs[i])
                torch.cuda.synchronize()
                touched.append(int(torch.unique(runners[0].ids[: C * w.k]).numel()))

        def timed(grouped=False):
            fns = [lambda c=i % copies, i=i: step(runners[c], xs[i % n_in], bs[i % n_in], grouped) for i in range(nsteps)]
            with torch.cuda.stream(stream):
                for f in fns:
                    f()
                torch.cuda.synchronize()
                return graph_time(fns, max(1, args.decode_reps), stream) / nsteps

        ms = timed()
        L0 = layers[0]
        # per layer call: the distinct experts its rows route to, the shared expert, the router, activations in and out
        step_bytes = nch * (float(np.mean(touched)) * L0.expert_bytes() + (S.expert_bytes() if S is not None else 0) + w.E * w.d * 4) \
            + 2 * w.rows * w.d * 4
        gbs = step_bytes / (ms / 1e3) / 1e9
        res[name] = {"rows": w.rows, "us_per_step": round(ms * 1e3, 2), "tok_s": round(w.rows / (ms / 1e3), 1),
                     "experts_touched": float(np.mean(touched)), "alg_bytes": step_bytes, "hbm_gbs": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "path": "decode" if decode else "prefill"}
        if nch > 1:
            res[name].update(chunks=nch, chunk_rows=C)
        if decode and w.rows > 1:
            # the same verify batch through the grouped GEMM path (bucketing + grouped GEMMs + combine), for the choice
            res[name]["us_per_step_grouped"] = round(timed(grouped=True) * 1e3, 2)
        log(f"workload {name}: {ms * 1e3:.2f} us/step, {gbs:.0f} GB/s"
            + (f" (grouped GEMM path {res[name]['us_per_step_grouped']:.2f} us)" if "us_per_step_grouped" in res[name] else ""))
        del runners, layers, sdev, S
        torch.cuda.empty_cache()
    return res


def _resident(start, end) -> int:
    """most intervals [start, end) open at once"""
    ev = sorted([(a, 1) for a in start] + [(b, -1) for b in end])
    c = best = 0
    for _, d in ev:
        c += d
        best = max(best, c)
    return best


def _timeline_of(ts: np.ndarray) -> dict:
    """One step's stamp records (hy_stamps.cuh: router waves at [4 gw], gate/up blocks at [16384 + 8 b], down blocks
    at [32768 + 8 b], s_memrealtime at 100 MHz) -> microseconds from the router's first wave.  Per-block phases
    (medians): gate/up route = logits, slot table and Q8 row in, the token routed; wload = the first round of weight
    bytes landed; dots; fold = block-order fold and store.  Down: slots = ids, weights and slot table in; hquant = the
    hidden rows loaded and quantized (or copied); wload; dots; fold."""
    tick = 0.01
    r = ts[:16384].reshape(-1, 4)
    r = r[r[:, 2] > 0]
    g = ts[16384:32768].reshape(-1, 8)
    g = g[g[:, 7] == 1]
    d = ts[32768:].reshape(-1, 8)
    d = d[d[:, 7] == 1]
    t0 = r[:, 0].min()
    at = lambda a: float((a - t0) * tick)
    med = lambda a: float(np.median(a) * tick)
    return {
        "router": {"waves": len(r), "end": at(r[:, 1].max())},
        "gate_up": {"blocks": len(g), "first_start": at(g[:, 0].min()), "end": at(g[:, 4].max()), "resident": _resident(g[:, 0], g[:, 4]),
                    "route": med(g[:, 1] - g[:, 0]), "wload": med(g[:, 2] - g[:, 1]), "dots": med(g[:, 3] - g[:, 2]),
                    "fold": med(g[:, 4] - g[:, 3]), "block": med(g[:, 4] - g[:, 0])},
        "down": {"blocks": len(d), "first_start": at(d[:, 0].min()), "end": at(d[:, 5].max()), "resident": _resident(d[:, 0], d[:, 5]),
                 "slots": med(d[:, 1] - d[:, 0]), "hquant": med(d[:, 2] - d[:, 1]), "wload": med(d[:, 3] - d[:, 2]),
                 "dots": med(d[:, 4] - d[:, 3]), "fold": med(d[:, 5] - d[:, 4]), "block": med(d[:, 5] - d[:, 0])},
    }


def decode_timeline(name: str, dev, copies: int = 4, reps: int = 20) -> dict:
    """Per-block phase times of one decode step of workload `name` (no shared expert: the phases of the three
    routed launches), replayed as bench.py's decode measurement replays it: 64 steps over `copies` layer copies in
    one HIP graph; the stamps of the graph's last step, medians over `reps` replays."""
    import ctypes
    from hyper_amd import lib
    L = lib()
    if not hasattr(L, "hy_stamps_read"):
        raise RuntimeError(f"{os.environ.get('HYMOE_LIB')} has no stamps: build it with python -m hyper_amd.build --stamps")
    L.hy_stamps_read.argtypes, L.hy_stamps_read.restype = [ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int
    L.hy_stamps_clear.argtypes, L.hy_stamps_clear.restype = [], ctypes.c_int
    w = WORKLOADS[name]
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    layers = [random_layer(w.tg, w.td, w.E, w.ff, w.d, seed=200 + c, device=dev, d_range=w.d_range) for c in range(copies)]
    runners = [moe.MoeLayerRunner(moe.MoeDev(lay, torch.arange(w.E, dtype=torch.int32, device=dev)),
                                  torch.randn(w.E, w.d, generator=g, device=dev) * 0.02, w.k, w.rows) for lay in layers]
    xs = activations(64 * w.rows, w.d, g, dev)
    fns = [lambda c=i % copies, i=i: runners[c].decode(xs[i * w.rows:(i + 1) * w.rows]) for i in range(64)]
    torch.cuda.synchronize()   # the weights, slot tables and inputs come from the default stream
    s = torch.cuda.Stream()
    buf = np.zeros(1 << 16, dtype=np.uint64)
    steps = []
    with torch.cuda.stream(s):
        for f in fns:
            f()
        torch.cuda.synchronize()
        us_step = graph_time(fns, 1, s) * 1e3 / len(fns)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for f in fns:
                f()
        for _ in range(reps):
            if L.hy_stamps_clear() != 0:
                raise RuntimeError("hy_stamps_clear failed")
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            if L.hy_stamps_read(buf.ctypes.data, buf.nbytes) != 0:
                raise RuntimeError("hy_stamps_read failed")
            steps.append(_timeline_of(buf.astype(np.int64)))
    summary = {k: {f: round(float(np.median([st[k][f] for st in steps])), 2) for f in steps[0][k]} for k in steps[0]}
    return {"workload": name, "rows": w.rows, "us_per_step_graph": round(us_step, 2), "reps": reps, "timeline_us": summary}


def cpu_info() -> dict:
    """CPU model, physical cores and hardware threads of this host (from /proc/cpuinfo), and the CPUs this process
    may run on."""
    model, cores, hw = "unknown", set(), 0
    try:
        phys = core = None
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                hw += 1
            elif k == "model name" and model == "unknown":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
                cores.add((phys, core))
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return {"model": model, "physical_cores": len(cores) or None, "hw_threads": hw or None, "cpus_available": avail}


def cpu_baseline(layer, W_r, xs, biases, budget_s: float, dec_layers=None):
    """The CPU oracle (AVX2 integer block dots, OpenMP rows) on the headline step, on this host.
    value: whole 512-token steps on `threads` threads (the CPU share of one GPU on this machine, at most 16) until
    about 0.6 budget_s; threads_1: the first 64 tokens of a step on one thread.  decode_gbs: the 1-token Q4_K decode
    (8 experts of 2.65 MB, cycling the decode layer copies so DRAM, not the caches, serves them) as expert bytes per
    second, on one thread and on `threads` -- the quantity the reference reports for its CPU expert path."""
    import oracle as orc
    OL = orc.Layer.from_expert_layer(layer)
    Wh = W_r.cpu().numpy()
    w = WORKLOADS["q4k_q6k_prefill512"]
    threads = orc.default_threads()

    def routed(i, S):
        xh, bh = xs[i % len(xs)][:S].cpu().numpy(), biases[i % len(xs)][:S].cpu().numpy()
        logits = (orc.gemv_f32(Wh, xh) + bh).astype(np.float32)
        ids, wts, _ = orc.route(logits, w.E, w.k)
        return xh, ids, wts

    def one(i, S, th):
        xh, ids, wts = routed(i, S)
        t0 = time.perf_counter()
        orc.moe_layer(OL, xh, ids, wts, threads=th)
        return time.perf_counter() - t0

    spent, steps = 0.0, 0
    while spent < 0.6 * budget_s or steps == 0:
        spent += one(steps, w.rows, threads)
        steps += 1
    res = {"value": steps * w.rows / spent, "unit": "tokens/s", "cores": threads, "kind": "port",
           "sample": f"{steps} whole {w.rows}-token steps (routing + expert FFN + combine; same weights, fresh inputs), "
                     f"{spent:.1f} s, oracle/moe_oracle.c (AVX2 integer block dots), {threads} threads",
           "threads_1": round(64 / one(0, 64, 1), 1), "cpu": cpu_info()}
    if dec_layers:
        wd = WORKLOADS["q4k_decode"]
        OLs = [orc.Layer.from_expert_layer(L) for L in dec_layers]
        g = np.random.default_rng(7)
        tok_bytes = wd.k * dec_layers[0].expert_bytes()
        for th, key in ((1, "decode_gbs_1"), (threads, "decode_gbs")):
            n_tok, t_all = 0, 0.0
            while t_all < 0.1 * budget_s or n_tok < 8:
                Lc = OLs[n_tok % len(OLs)]
                x = g.standard_normal((1, wd.d)).astype(np.float32)
                ids = g.choice(wd.E, size=(1, wd.k), replace=False).astype(np.int32)
                wts = np.full((1, wd.k), 1.0 / wd.k, np.float32)
                t0 = time.perf_counter()
                orc.moe_layer(Lc, x, ids, wts, threads=th)
                t_all += time.perf_counter() - t0
                n_tok += 1
            res[key] = round(n_tok * tok_bytes / t_all / 1e9, 2)
        res["decode_sample"] = (f"1-token Q4_K decode, 8 experts ({tok_bytes / 1e6:.1f} MB), cycling {len(OLs)} layer copies "
                                f"({len(OLs) * dec_layers[0].expert_bytes() * wd.E / 1e9:.2f} GB)")
    return res


def copy_probe(mib: int, dev):
    """A plain copy kernel of known size (mib MiB read, mib MiB written), three launches: the yardstick that
    scales the FETCH_SIZE / WRITE_SIZE counters into bytes."""
    src = torch.randn(mib * (1 << 18), device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def traffic_from_profile(kernel: str):
    """HBM bytes per launch of `kernel` measured by counter passes (committed summary), or None."""
    f = ROOT / "profiles" / "traffic_q4k_q6k_prefill512.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 3 and parts[0] == "traffic_bytes" and parts[1] == kernel:
            return float(parts[2])
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help="timed prefill steps")
    ap.add_argument("--warmup", type=int, default=2, help="untimed passes over the step sequence")
    ap.add_argument("--copies", type=int, default=4, help="independent weight copies cycled by the prefill steps")
    ap.add_argument("--inputs", type=int, default=4, help="independent (activations, routing) sets")
    ap.add_argument("--graph-steps", type=int, default=8, help="prefill steps captured per graph")
    ap.add_argument("--kernel-reps", type=int, default=8)
    ap.add_argument("--decode-copies", type=int, default=4)
    ap.add_argument("--decode-reps", type=int, default=8)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--workload-copies", type=int, default=2, help="weight copies per workload in the `workloads` object")
    ap.add_argument("--no-workloads", action="store_true", help="skip the `workloads` object (the other configured workloads)")
    ap.add_argument("--workload", action="append", default=None, metavar="NAME",
                    help="time only these workloads in the `workloads` object (repeatable; profiling runs)")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the headline prefill (profiling runs of decode / workloads only; prints no headline line)")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU-oracle work for cpu_baseline (0: skip)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain copy kernel over MIB MiB (counter calibration under rocprofv3 --pmc)")
    ap.add_argument("--timeline", nargs="+", metavar="NAME", default=None,
                    help="print the per-block decode timeline of these workloads from the stamps build of the library, "
                         "then exit (python -m hyper_amd.build --stamps first)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: hyper_amd runs the expert path on one GPU and has no multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.timeline:
        for name in args.timeline:
            print(json.dumps(decode_timeline(name, dev)), flush=True)
        return
    stream = torch.cuda.Stream()
    if args.copy_probe:
        copy_probe(args.copy_probe, dev)
    pre = None
    if not args.no_prefill:
        log("prefill: building layers and inputs")
        pre, L0, W0, xs0, bs0 = prefill_bench(args, dev, stream)
        log(f"prefill: {pre['tok_s']:.0f} tok/s, {pre['ms_step'] * 1e3:.1f} us/step")
    dec, dec_layers = None, None
    if not args.no_decode:
        log("decode: building layers")
        dec, dec_layers = decode_bench(args, dev, stream)
        log(f"decode: {dec['us_per_token']:.2f} us/token (a chain of three dependent launches: {dec['chain3_floor_us']:.2f} us)")
    wl = None
    if not args.no_workloads:
        log("workloads: the other configured shapes")
        wl = workloads_bench(args, dev, stream)
    if pre is None:   # a profiling run: the parts it timed, no headline line
        print(json.dumps({"decode": dec, "workloads": wl}), flush=True)
        return
    cpu = None
    if args.cpu_budget > 0:
        log("cpu baseline: oracle on a sample of the prefill step")
        cpu = cpu_baseline(L0, W0, xs0, bs0, args.cpu_budget, [L.to("cpu") for L in dec_layers] if dec_layers else None)
    w = WORKLOADS["q4k_q6k_prefill512"]
    line = {
        "metric": METRIC, "value": round(pre["tok_s"], 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": pre["timed_steps"], "warmup": args.warmup,
        "ms_per_step": round(pre["ms_step"], 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": w.name, "d_model": w.d, "experts": w.E, "top_k": w.k, "ff": w.ff, "rows": w.rows,
                   "gate_up": w.tg.name, "down": w.td.name, "routing": "zipf(1.1)+gumbel logit bias",
                   "weight_copies": args.copies, "active_experts_mean": pre["active_experts_mean"]},
        "roofline": {k_: (round(v, 4) if isinstance(v, float) else v) for k_, v in pre["roofline"].items()},
        "step": {"alg_bytes": pre["step_bytes"], "hbm_gbs": round(pre["step_hbm_gbs"], 1),
                 "hbm_frac": round(pre["step_hbm_gbs"] / HBM_PEAK_GBS, 4), "int8_tops": round(pre["step_int8_tops"], 2),
                 "int8_mfma_frac": round(pre["step_int8_tops"] / INT8_PEAK_TOPS, 4),
                 "kernels": pre["kernels"]},
        "decode": dec,
        "workloads": wl,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
