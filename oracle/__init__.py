"""ctypes front of the CPU oracle (oracle/moe_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package; the
product (hyper_amd/) never does.  numpy in, numpy out.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
LIB_PATH = _DIR / "liboracle_moe.so"

(Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS,
 MXFP4) = (6, 7, 8, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 39)
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292, IQ2_XXS: 66, IQ2_XS: 74, IQ4_NL: 18, IQ4_XS: 136,
               MXFP4: 17, Q5_0: 22, Q2_K: 84, Q3_K: 110, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ1_S: 50, Q5_1: 24}
BLOCK_ELEMS = {Q8_0: 32, IQ4_NL: 32, MXFP4: 32, Q5_0: 32, Q5_1: 32}


def block_elems(t):
    return BLOCK_ELEMS.get(int(t), 256)


def vec_dot_type(t):
    return Q8_0 if int(t) in (IQ4_NL, Q8_0, MXFP4, Q5_0, Q5_1) else Q8_K


def row_bytes(t, n):
    return n // block_elems(t) * BLOCK_BYTES[int(t)]


class or_layer(ctypes.Structure):
    _fields_ = [("tg", ctypes.c_int), ("td", ctypes.c_int), ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p),
                ("down", ctypes.c_void_p), ("gate_bytes", ctypes.c_size_t), ("down_bytes", ctypes.c_size_t),
                ("ff", ctypes.c_int), ("n", ctypes.c_int), ("E", ctypes.c_int), ("clamp", ctypes.c_float)]


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sig = {
            "or_block_bytes": (ctypes.c_size_t, [I]), "or_block_elems": (I, [I]), "or_vec_dot_type": (I, [I]),
            "or_expf": (F, [F]), "or_silu": (F, [F]),
            "or_fp16_to_fp32": (F, [ctypes.c_uint16]), "or_fp32_to_fp16": (ctypes.c_uint16, [F]),
            "or_quantize_q8_K": (None, [P, P, I]), "or_quantize_q8_0": (None, [P, P, I]),
            "or_quantize_row": (I, [I, P, P, I]), "or_dequant_row": (I, [I, P, I, P]),
            "or_block_ints": (I, [I, P, P, I, P, P]), "or_block_ints_scalar": (I, [I, P, P, I, P, P]), "or_row_dot": (F, [I, P, P, I]),
            "or_gemv_f32": (None, [P, I, I, P, I, P, I, I]),
            "or_route": (I, [P, I, I, I, I, P, P, P]),
            "or_logf": (F, [F]), "or_log1pf": (F, [F]), "or_sigmoid": (F, [F]), "or_sqrt_softplus": (F, [F]),
            "or_route_sig": (I, [P, I, P, I, I, F, I, P, P, P]),
            "or_route_sqrtsp": (I, [P, I, P, I, I, F, I, P, P]),
            "or_order": (I, [P, P, I, I, P, P, P]),
            "or_moe_layer": (I, [ctypes.POINTER(or_layer), I, P, I, P, P, I, P, I, ctypes.POINTER(or_layer), P, P, P, I]),
            "or_expert_ffn": (I, [ctypes.POINTER(or_layer), I, I, P, I, P, P, I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def default_threads() -> int:
    """Oracle worker threads: ORACLE_THREADS, else OMP_NUM_THREADS, else the CPUs available to this process; at most
    16 without ORACLE_THREADS, the CPU share one GPU gets on the benchmark hosts (whatever the host's core count)."""
    if os.environ.get("ORACLE_THREADS"):
        return int(os.environ["ORACLE_THREADS"])
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        return max(1, min(16, int(os.environ["OMP_NUM_THREADS"])))
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def expf(x: float) -> float:
    return lib().or_expf(float(x))


def silu(x: float) -> float:
    return lib().or_silu(float(x))


def quantize(vtype, x) -> np.ndarray:
    x = _c(x, np.float32)
    n = x.shape[-1]
    rows = x.reshape(-1, n)
    out = np.zeros((rows.shape[0], row_bytes(vtype, n)), dtype=np.uint8)
    for i in range(rows.shape[0]):
        r = np.ascontiguousarray(rows[i])
        o = out[i]
        if lib().or_quantize_row(int(vtype), _p(r), ctypes.c_void_p(o.ctypes.data), n):
            raise ValueError("or_quantize_row failed")
    return out.reshape(x.shape[:-1] + (out.shape[-1],))


def dequant_row(t, row, n) -> np.ndarray:
    row = _c(row, np.uint8)
    out = np.zeros(n, dtype=np.float32)
    if lib().or_dequant_row(int(t), _p(row), n, _p(out)):
        raise ValueError("or_dequant_row failed")
    return out


def block_ints(t, row, xq, n, scalar=False):
    """The exact integers of every block of one weight row; scalar=True: the element-by-element restatement only."""
    row, xq = _c(row, np.uint8), _c(xq, np.uint8)
    nb = n // block_elems(t)
    si, sm = np.zeros(nb, np.int32), np.zeros(nb, np.int32)
    fn = lib().or_block_ints_scalar if scalar else lib().or_block_ints
    if fn(int(t), _p(row), _p(xq), n, _p(si), _p(sm)):
        raise ValueError("or_block_ints failed")
    return si, sm


def row_dot(t, row, xq, n) -> np.float32:
    row, xq = _c(row, np.uint8), _c(xq, np.uint8)
    return np.float32(lib().or_row_dot(int(t), _p(row), _p(xq), n))


def gemv_f32(W, x) -> np.ndarray:
    W, x = _c(W, np.float32), _c(np.atleast_2d(x), np.float32)
    rows, kdim = W.shape
    nt = x.shape[0]
    y = np.zeros((nt, rows), np.float32)
    lib().or_gemv_f32(_p(W), rows, kdim, _p(x), kdim, _p(y), rows, nt)
    return y


def route(logits, ne, k, with_sg=False):
    logits = _c(np.atleast_2d(logits), np.float32)
    nt, ls = logits.shape
    ids, wts = np.zeros((nt, k), np.int32), np.zeros((nt, k), np.float32)
    sg = np.zeros(nt, np.float32) if with_sg else None
    if lib().or_route(_p(logits), ls, ne, k, nt, _p(ids), _p(wts), _p(sg)):
        raise ValueError("or_route failed")
    return ids, wts, sg


def route_sig(logits, bias, ne, k, scale):
    """sigmoid router with selection bias (src/kernels5.cu:1090-1122): ids, wts, sg (all ones)"""
    logits = _c(np.atleast_2d(logits), np.float32)
    bias = _c(bias, np.float32)
    nt, ls = logits.shape
    ids, wts, sg = np.zeros((nt, k), np.int32), np.zeros((nt, k), np.float32), np.zeros(nt, np.float32)
    if lib().or_route_sig(_p(logits), ls, _p(bias), ne, k, float(scale), nt, _p(ids), _p(wts), _p(sg)):
        raise ValueError("or_route_sig failed")
    return ids, wts, sg


def route_sqrtsp(logits, bias, ne, k, scale):
    """sqrt-softplus router (src/kernels7.cu:816-865): ids, wts"""
    logits = _c(np.atleast_2d(logits), np.float32)
    bias = _c(bias, np.float32)
    nt, ls = logits.shape
    ids, wts = np.zeros((nt, k), np.int32), np.zeros((nt, k), np.float32)
    if lib().or_route_sqrtsp(_p(logits), ls, _p(bias), ne, k, float(scale), nt, _p(ids), _p(wts)):
        raise ValueError("or_route_sqrtsp failed")
    return ids, wts


def order(slot, ids, ne):
    slot, ids = _c(slot, np.int32), _c(ids, np.int32).ravel()
    P = ids.size
    o, on, eg = np.full(P, -1, np.int32), np.zeros(2, np.int32), np.zeros(3 * ne, np.int32)
    if lib().or_order(_p(slot), _p(ids), P, ne, _p(o), _p(on), _p(eg)):
        raise ValueError("or_order failed")
    return o[:on[0]], on, eg[:3 * on[1]].reshape(-1, 3)


class Layer:
    """numpy view of an expert layer for the oracle: gate/up [E, ff, row bytes], down [E, n, row bytes]."""

    def __init__(self, tg, td, gate, up, down, ff, n, clamp=0.0):
        self.tg, self.td, self.ff, self.n, self.clamp = int(tg), int(td), ff, n, clamp
        self.gate, self.up, self.down = _c(gate, np.uint8), _c(up, np.uint8), _c(down, np.uint8)
        self.E = self.gate.shape[0]
        c = or_layer()
        c.tg, c.td = self.tg, self.td
        c.gate, c.up, c.down = self.gate.ctypes.data, self.up.ctypes.data, self.down.ctypes.data
        c.gate_bytes, c.down_bytes = self.gate[0].nbytes, self.down[0].nbytes
        c.ff, c.n, c.E, c.clamp = ff, n, self.E, clamp
        self.c = c

    @classmethod
    def from_expert_layer(cls, L):
        """From hyper_amd.formats.ExpertLayer (torch tensors, any device)."""
        return cls(L.tg, L.td, L.gate.cpu().numpy(), L.up.cpu().numpy(), L.down.cpu().numpy(), L.ff, L.n, L.clamp)


def moe_layer(L: Layer, x, ids, wts, shared: Layer = None, sg=None, threads=None, want_hy=False):
    """CpuMoe::run_layer semantics (every expert owned): out [nt, n] (+ h [P, ff], y [P, n] in pair order)."""
    x = _c(np.atleast_2d(x), np.float32)
    ids, wts = _c(np.atleast_2d(ids), np.int32), _c(np.atleast_2d(wts), np.float32)
    nt, k = ids.shape
    out = np.zeros((nt, L.n), np.float32)
    h = np.zeros((nt * k, L.ff), np.float32) if want_hy else None
    y = np.zeros((nt * k, L.n), np.float32) if want_hy else None
    sgv = None if sg is None else _c(sg, np.float32)
    threads = threads or default_threads()
    rc = lib().or_moe_layer(ctypes.byref(L.c), nt, _p(x), x.shape[1], _p(ids), _p(wts), k, _p(out), L.n,
                            ctypes.byref(shared.c) if shared is not None else None, _p(sgv), _p(h), _p(y), threads)
    if rc:
        raise ValueError("or_moe_layer failed")
    return (out, h, y) if want_hy else out


def expert_ffn(L: Layer, e: int, x, threads=None):
    x = _c(np.atleast_2d(x), np.float32)
    nt = x.shape[0]
    h, y = np.zeros((nt, L.ff), np.float32), np.zeros((nt, L.n), np.float32)
    threads = threads or default_threads()
    if lib().or_expert_ffn(ctypes.byref(L.c), e, nt, _p(x), x.shape[1], _p(h), _p(y), threads):
        raise ValueError("or_expert_ffn failed")
    return h, y
