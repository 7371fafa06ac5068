"""Per-block timeline of the decode step from the stamps build (libhymoe_stamps.so, -DHY_STAMPS).

    python -m hyper_amd.build --stamps
    python -m hyper_amd.stamps q4k_decode iq2xs_decode ...      # one JSON line per workload

Each workload runs as it does in bench.py's decode measurements: `copies` weight copies cycled by 64 one-token (or
one-verify-batch) decode steps captured in one HIP graph.  After a replay the device stamp array holds the last
step's three launches: every router wave's entry and exit, and for every gate/up and down block the times at its
phase boundaries (s_memrealtime, 10 ns ticks).  The medians over `reps` replays of these per-step figures are
printed, in microseconds from the router's first wave:

  router: first / last wave end; gate/up and down: first and last block start, last block end, the residency
  (most blocks running at once) and per-block phase medians (p90 where given):
    route      gate/up: logits, slot table and the Q8 row in, the token routed (every block routes its token)
    wload      gate/up: the first round of weight bytes landed (the stamp waits for them)
    dots       the item dot products of every round (gate/up), of all pairs (down)
    fold       the per-row block-order fold and the output store
    slots      down: ids, weights and the slot table in (the first barrier)
    hquant     down: the k hidden rows loaded and quantized into LDS (or copied, for the Q8_0 hand-over)
"""
import ctypes
import json
import os
import sys
from pathlib import Path

os.environ.setdefault("HYMOE_LIB", str(Path(__file__).resolve().parent / "libhymoe_stamps.so"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from . import lib, moe  # noqa: E402
from .formats import WORKLOADS, activations, random_layer  # noqa: E402

TICK_US = 0.01   # s_memrealtime runs at 100 MHz
CAP = 1 << 16


def _library():
    L = lib()
    if not hasattr(L, "hy_stamps_read"):
        raise RuntimeError(f"{os.environ['HYMOE_LIB']} has no stamps: build it with python -m hyper_amd.build --stamps")
    L.hy_stamps_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    L.hy_stamps_read.restype = ctypes.c_int
    L.hy_stamps_clear.argtypes = []
    L.hy_stamps_clear.restype = ctypes.c_int
    return L


def _resident(start, end):
    ev = sorted([(a, 1) for a in start] + [(b, -1) for b in end])
    c = best = 0
    for _, d in ev:
        c += d
        best = max(best, c)
    return best


def analyse(ts: np.ndarray) -> dict:
    """One step's records -> microseconds from the router's first wave."""
    r = ts[:16384].reshape(-1, 4)
    r = r[r[:, 2] > 0]
    g = ts[16384:32768].reshape(-1, 8)
    g = g[g[:, 7] == 1]
    d = ts[32768:].reshape(-1, 8)
    d = d[d[:, 7] == 1]
    t0 = r[:, 0].min()
    at = lambda a: float((a - t0) * TICK_US)
    med = lambda a: float(np.median(a) * TICK_US)
    p90 = lambda a: float(np.percentile(a, 90) * TICK_US)
    return {
        "router": {"waves": len(r), "first_end": at(r[:, 1].min()), "end": at(r[:, 1].max())},
        "gate_up": {"blocks": len(g), "first_start": at(g[:, 0].min()), "last_start": at(g[:, 0].max()), "end": at(g[:, 4].max()),
                    "resident": _resident(g[:, 0], g[:, 4]),
                    "route": med(g[:, 1] - g[:, 0]), "route_p90": p90(g[:, 1] - g[:, 0]),
                    "wload": med(g[:, 2] - g[:, 1]), "wload_p90": p90(g[:, 2] - g[:, 1]),
                    "dots": med(g[:, 3] - g[:, 2]), "fold": med(g[:, 4] - g[:, 3]), "block": med(g[:, 4] - g[:, 0])},
        "down": {"blocks": len(d), "first_start": at(d[:, 0].min()), "last_start": at(d[:, 0].max()), "end": at(d[:, 5].max()),
                 "resident": _resident(d[:, 0], d[:, 5]),
                 "slots": med(d[:, 1] - d[:, 0]), "hquant": med(d[:, 2] - d[:, 1]), "wload": med(d[:, 3] - d[:, 2]),
                 "dots": med(d[:, 4] - d[:, 3]), "fold": med(d[:, 5] - d[:, 4]), "block": med(d[:, 5] - d[:, 0])},
    }


def run(name: str, copies: int = 4, reps: int = 20, dev: str = "cuda:0") -> dict:
    L = _library()
    w = WORKLOADS[name]
    if w.rows > 8:
        raise ValueError(f"{name}: {w.rows} rows take the grouped GEMMs, not the decode kernels")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    layers = [random_layer(w.tg, w.td, w.E, w.ff, w.d, seed=200 + c, device=dev, d_range=w.d_range) for c in range(copies)]
    runners = [moe.MoeLayerRunner(moe.MoeDev(lay, torch.arange(w.E, dtype=torch.int32, device=dev)),
                                  torch.randn(w.E, w.d, generator=g, device=dev) * 0.02, w.k, w.rows) for lay in layers]
    xs = activations(64 * w.rows, w.d, g, dev)
    fns = [lambda c=i % copies, i=i: runners[c].decode(xs[i * w.rows:(i + 1) * w.rows]) for i in range(64)]
    torch.cuda.synchronize()   # weights, slot tables and inputs come from the default stream
    s = torch.cuda.Stream()
    buf = np.zeros(CAP, dtype=np.uint64)
    steps = []
    with torch.cuda.stream(s):
        for f in fns:
            f()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for f in fns:
                f()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        graph.replay()
        e1.record(s)
        torch.cuda.synchronize()
        us_step = e0.elapsed_time(e1) * 1e3 / len(fns)
        for _ in range(reps):
            if L.hy_stamps_clear() != 0:
                raise RuntimeError("hy_stamps_clear failed")
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            if L.hy_stamps_read(buf.ctypes.data, buf.nbytes) != 0:
                raise RuntimeError("hy_stamps_read failed")
            steps.append(analyse(buf.astype(np.int64)))
    summary = {k: {f: round(float(np.median([st[k][f] for st in steps])), 2) for f in steps[0][k]} for k in steps[0]}
    return {"workload": name, "rows": w.rows, "us_per_step_graph": round(us_step, 2), "reps": reps, "timeline_us": summary}


if __name__ == "__main__":
    for wl in sys.argv[1:] or ["q4k_decode"]:
        print(json.dumps(run(wl)), flush=True)
