"""The reference's expert-compute API on torch device tensors, calling libhymoe's C ABI.

Function names, argument order and meaning follow src/kernels4.cuh:45-91 and src/experts.h:26-50
(moe_route, moe_order, moe_gate_up, moe_down, moe_gemm_gate_up, moe_gemm_down, moe_reduce,
upload_experts); errors raise HyError where the reference throws std::runtime_error.  Activations for
the grouped GEMMs are Q8 rows (q8_quantize) instead of the reference's fp16 copies.

MoeLayerRunner strings the calls together the way the reference engine does per MoE layer
(src/engine4.cu:807-888): router GEMV, route, then gate/up -> down -> combine for decode rows, or
order -> quantize -> grouped GEMMs -> combine for a prefill chunk.
"""
import ctypes
from typing import Optional

import torch

from . import check, hy_expert_tensors, hy_moe_dev, lib
from .formats import ExpertLayer, GType, q8_row_bytes, vec_dot_type


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _s(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def tile_rows(mat: torch.Tensor, in_dim: int) -> torch.Tensor:
    """GGUF rows [E, rows, row_bytes] -> the kernels' tiled layout, same shape and bytes: 16-row tiles whose 256-value
    spans lie together (span s of row r at ((r / 16) * nspan + s) * 16 * sb + (r % 16) * sb within an expert)."""
    E, rows, rb = mat.shape
    nspan = in_dim // 256
    if rows % 16 or in_dim % 256 or rb % nspan:
        raise ValueError(f"tile_rows: rows {rows} must be a multiple of 16 and in_dim {in_dim} of 256")
    sb = rb // nspan
    return mat.reshape(E, rows // 16, 16, nspan, sb).permute(0, 1, 3, 2, 4).contiguous().reshape(E, rows, rb)


class MoeDev:
    """Device expert weights + slot table (hy_moe_dev / MoeDev).  Keeps the tensors alive.

    `layer` holds GGUF rows on the device; they are re-laid into tiles (tile_rows) here, once, as the kernels read
    them.  The raw layer is not kept."""

    def __init__(self, layer: ExpertLayer, slot: torch.Tensor):
        layer = ExpertLayer(layer.tg, layer.td, layer.E, layer.ff, layer.n, tile_rows(layer.gate, layer.n),
                            tile_rows(layer.up, layer.n), tile_rows(layer.down, layer.ff), layer.clamp)
        self.layer, self.slot = layer, slot
        c = hy_moe_dev()
        c.gate, c.up, c.down = layer.gate.data_ptr(), layer.up.data_ptr(), layer.down.data_ptr()
        c.tg, c.td = int(layer.tg), int(layer.td)
        c.gate_bytes, c.down_bytes = layer.gate_bytes, layer.down_bytes
        c.slot = slot.data_ptr()
        c.ff, c.n, c.clamp, c.n_expert, c.n_local = layer.ff, layer.n, float(layer.clamp), slot.numel(), layer.E
        self.c = c
        self.ref = ctypes.byref(c)

    @property
    def tg(self):
        return self.layer.tg

    @property
    def td(self):
        return self.layer.td


def upload_experts(layer: ExpertLayer, slot=None, device="cuda") -> MoeDev:
    """Copy the experts with slot[e] >= 0 to the device at their slots (src/experts.cu:56-74).
    slot None: every expert at its own index."""
    E = layer.E
    slot_list = list(range(E)) if slot is None else [int(s) for s in slot]
    nl = max(max(slot_list) + 1, 1)
    shape_g, shape_d = (nl,) + tuple(layer.gate.shape[1:]), (nl,) + tuple(layer.down.shape[1:])
    g = torch.zeros(shape_g, dtype=torch.uint8, device=device)
    u = torch.zeros(shape_g, dtype=torch.uint8, device=device)
    d = torch.zeros(shape_d, dtype=torch.uint8, device=device)
    for e, s in enumerate(slot_list):
        if s >= 0:
            g[s].copy_(layer.gate[e]); u[s].copy_(layer.up[e]); d[s].copy_(layer.down[e])
    dev_layer = ExpertLayer(layer.tg, layer.td, nl, layer.ff, layer.n, g, u, d, layer.clamp)
    return MoeDev(dev_layer, torch.tensor(slot_list, dtype=torch.int32, device=device))


def upload_experts_c(layer: ExpertLayer, slot) -> hy_moe_dev:
    """The C ABI's own upload (hipMalloc + copies; release with free_experts)."""
    t = hy_expert_tensors()
    g, u, d = (layer.gate.contiguous().cpu(), layer.up.contiguous().cpu(), layer.down.contiguous().cpu())
    t.gate, t.up, t.down = g.data_ptr(), u.data_ptr(), d.data_ptr()
    t.gb, t.db, t.E, t.tg, t.td = layer.gate_bytes, layer.down_bytes, layer.E, int(layer.tg), int(layer.td)
    sl = torch.tensor(list(slot), dtype=torch.int32)
    out = hy_moe_dev()
    check(lib().hy_upload_experts(ctypes.byref(t), _p(sl), layer.ff, layer.n, float(layer.clamp), ctypes.byref(out)))
    return out


def free_experts(m: hy_moe_dev) -> None:
    check(lib().hy_free_experts(ctypes.byref(m)))


# ------------------------------------------------------------------ the reference API

def _bf16w(W) -> bool:
    """router weights held as bf16 (torch.bfloat16, whose storage is the uint16 bit patterns the bf16 entries take)"""
    return isinstance(W, torch.Tensor) and W.dtype == torch.bfloat16


def gemv_f32(W, rows, kdim, x, xs, y, ys, nt, stream=None, bias=None, bias_stride=0):
    """Router logits; a torch.bfloat16 W goes to gemv_bf16w (the same products and sums on the widened weights)."""
    if _bf16w(W):
        return gemv_bf16w(W, rows, kdim, x, xs, y, ys, nt, stream, bias, bias_stride)
    check(lib().hy_gemv_f32(_p(W), rows, kdim, _p(x), xs, _p(y), ys, nt, _p(bias), bias_stride, _s(stream)))


def gemv_bf16w(W, rows, kdim, x, xs, y, ys, nt, stream=None, bias=None, bias_stride=0):
    check(lib().hy_gemv_bf16w(_p(W), rows, kdim, _p(x), xs, _p(y), ys, nt, _p(bias), bias_stride, _s(stream)))


def bf16_to_f32(W, n, out, stream=None):
    check(lib().hy_bf16_to_f32(_p(W), n, _p(out), _s(stream)))


def moe_route(logits, ls, n_expert, k, ids, wts, sg, nt, stream=None):
    check(lib().hy_moe_route(_p(logits), ls, n_expert, k, _p(ids), _p(wts), _p(sg), nt, _s(stream)))


def moe_route_sig(logits, ls, bias, n_expert, k, scale, ids, wts, sg, nt, stream=None):
    """Sigmoid router with selection bias (moe_route_sig, src/kernels5.cuh:74)."""
    check(lib().hy_moe_route_sig(_p(logits), ls, _p(bias), n_expert, k, float(scale), _p(ids), _p(wts), _p(sg), nt, _s(stream)))


def moe_route_sqrtsp(logits, ls, bias, n_expert, k, scale, ids, wts, nt, stream=None):
    """sqrt-softplus router with selection bias (route7, src/kernels7.cuh:75)."""
    check(lib().hy_moe_route_sqrtsp(_p(logits), ls, _p(bias), n_expert, k, float(scale), _p(ids), _p(wts), nt, _s(stream)))


def moe_order(m: MoeDev, ids, n_pairs, n_expert, order, order_n, stream=None, egrp=None):
    check(lib().hy_moe_order(m.ref, _p(ids), n_pairs, n_expert, _p(order), _p(order_n), _s(stream), _p(egrp)))


def q8_quantize(vtype, x, xs, n, nt, q, stream=None):
    check(lib().hy_q8_quantize(int(vtype), _p(x), xs, n, nt, _p(q), _s(stream)))


def moe_gate_up(m: MoeDev, x, xs, ids, k, h, nt, stream=None, order=None, order_n=None):
    check(lib().hy_moe_gate_up(m.ref, _p(x), xs, _p(ids), k, _p(h), nt, _s(stream), _p(order), _p(order_n)))


def moe_down(m: MoeDev, h, ids, wts, k, y, nt, stream=None, order=None, order_n=None):
    check(lib().hy_moe_down(m.ref, _p(h), _p(ids), _p(wts), k, _p(y), nt, _s(stream), _p(order), _p(order_n)))


def moe_gemm_gate_up(m: MoeDev, xq, k, n_pairs, order, order_n, egrp, max_active, h, stream=None):
    check(lib().hy_moe_gemm_gate_up(m.ref, _p(xq), k, n_pairs, _p(order), _p(order_n), _p(egrp), max_active, _p(h), _s(stream)))


def moe_gemm_down(m: MoeDev, hq, n_pairs, order, order_n, egrp, max_active, wts, y, stream=None):
    check(lib().hy_moe_gemm_down(m.ref, _p(hq), n_pairs, _p(order), _p(order_n), _p(egrp), max_active, _p(wts), _p(y), _s(stream)))


def moe_reduce(shexp, sg, y, k, out, n, nt, ids, stream=None):
    check(lib().hy_moe_reduce(_p(shexp), _p(sg), _p(y), k, _p(out), n, nt, _p(ids), _s(stream)))


def moe_down_reduce(m: MoeDev, h, ids, wts, k, shexp, sg, out, nt, stream=None):
    check(lib().hy_moe_down_reduce(m.ref, _p(h), _p(ids), _p(wts), k, _p(shexp), _p(sg), _p(out), nt, _s(stream)))


def moe_reduce_residual(shexp, sg, y, k, resid, n, nt, ids, stream=None):
    """The combine added into the residual in place (resid += sg shexp + the token's y rows)."""
    check(lib().hy_moe_reduce_residual(_p(shexp), _p(sg), _p(y), k, _p(resid), n, nt, _p(ids), _s(stream)))


def moe_down_reduce_residual(m: MoeDev, h, ids, wts, k, shexp, sg, resid, nt, stream=None):
    check(lib().hy_moe_down_reduce_residual(m.ref, _p(h), _p(ids), _p(wts), k, _p(shexp), _p(sg), _p(resid), nt, _s(stream)))


def moe_router_q8(W_r, rows, kdim, x, xs, logits, ls, vtype, xq, nt, stream=None, bias=None, bias_stride=0):
    """gemv_f32 and the Q8 rows of x in one launch (a torch.bfloat16 W_r: the bf16-weight router)."""
    fn = lib().hy_moe_router_q8_bf16w if _bf16w(W_r) else lib().hy_moe_router_q8
    check(fn(_p(W_r), rows, kdim, _p(x), xs, _p(bias), bias_stride, _p(logits), ls, int(vtype), _p(xq), nt, _s(stream)))


def moe_route_gate_up(m: MoeDev, logits, ls, n_expert, k, xq, ids, wts, sg, h, nt, stream=None):
    """moe_route and moe_gate_up (on Q8 rows) in one launch."""
    check(lib().hy_moe_route_gate_up(m.ref, _p(logits), ls, n_expert, k, _p(xq), _p(ids), _p(wts), _p(sg), _p(h), nt, _s(stream)))


def moe_shared_gate_up(m: MoeDev, xq, h, nt, stream=None):
    """The shared expert's decode gate/up (local expert 0, k = 1) from the Q8 rows of x."""
    check(lib().hy_moe_shared_gate_up(m.ref, _p(xq), _p(h), nt, _s(stream)))


def moe_shared_down(m: MoeDev, h, out, nt, stream=None):
    """The shared expert's decode down (local expert 0, weight 1) for nt rows, each row's value alone."""
    check(lib().hy_moe_shared_down(m.ref, _p(h), _p(out), nt, _s(stream)))


def moe_route_gate_up_q8(m: MoeDev, logits, ls, n_expert, k, xq, ids, wts, sg, h, hq, nt, stream=None):
    """moe_route_gate_up that also writes the hidden rows as Q8_0 blocks (down types with a Q8_0 partner)."""
    check(lib().hy_moe_route_gate_up_q8(m.ref, _p(logits), ls, n_expert, k, _p(xq), _p(ids), _p(wts), _p(sg), _p(h), _p(hq), nt,
                                        _s(stream)))


def moe_down_reduce_q8(m: MoeDev, hq, ids, wts, k, shexp, sg, out, residual, nt, stream=None):
    """moe_down_reduce (or its residual form) from the Q8_0 hidden rows of moe_route_gate_up_q8."""
    check(lib().hy_moe_down_reduce_q8(m.ref, _p(hq), _p(ids), _p(wts), k, _p(shexp), _p(sg), _p(out), int(bool(residual)), nt,
                                      _s(stream)))


def dequant_row(type_, row, n, out, stream=None):
    check(lib().hy_dequant_row(int(type_), _p(row), n, _p(out), _s(stream)))


def block_ints(type_, rows, row_bytes, nrows, xq, n, sumi, summ, stream=None):
    check(lib().hy_block_ints(int(type_), _p(rows), row_bytes, nrows, _p(xq), n, _p(sumi), _p(summ), _s(stream)))


# ------------------------------------------------------------------ one MoE layer, engine-style

class MoeLayerRunner:
    """Workspace + call sequence for one MoE layer on one GPU.

    decode(x): rows <= decode_rows use gate/up GEMV -> fused down+combine (src/engine4.cu:880-888);
    prefill(x): bucketing + grouped int8-MFMA GEMMs (src/engine4.cu:851-854, :887).
    The router is W_r [E, d], fp32 (src/engine4.cu:807) or bf16 (the router16 path, src/engine4.cu:808: the same
    logits as the widened fp32 matrix, half the bytes); `bias` adds per-token logits (skewed routing).
    `router` picks the routing on the logits: "softmax" (moe_route, src/kernels4.cu:297-344), or, with `router_bias`
    (E floats, selection only) and `router_scale`: "sigmoid" (moe_route_sig, src/kernels5.cu:1090-1122; sg = 1) or
    "sqrt_softplus" (route7, src/kernels7.cu:816-865).
    """

    def __init__(self, dev: MoeDev, W_r: torch.Tensor, k: int, max_rows: int, shared: Optional[MoeDev] = None,
                 sg_logit: bool = False, router: str = "softmax", router_bias: Optional[torch.Tensor] = None,
                 router_scale: float = 1.0):
        if router not in ("softmax", "sigmoid", "sqrt_softplus"):
            raise ValueError(f"unknown router {router!r}")
        if router != "softmax" and (router_bias is None or sg_logit):
            raise ValueError(f"the {router} router takes router_bias and no shared-gate logit")
        self.router, self.router_bias, self.router_scale = router, router_bias, float(router_scale)
        L = dev.layer
        if W_r.dtype not in (torch.float32, torch.bfloat16) or W_r.dim() != 2 or W_r.shape[1] != L.n or not W_r.is_contiguous():
            raise ValueError(f"W_r must be a contiguous fp32 or bf16 [rows, {L.n}] matrix, got {W_r.dtype} {tuple(W_r.shape)}")
        self.dev, self.W_r, self.k, self.E, self.d, self.ff = dev, W_r, k, dev.slot.numel(), L.n, L.ff
        self.shared = shared
        self.sg_logit = sg_logit
        device = W_r.device
        self.device, self.max_rows = device, int(max_rows)
        T, P = max_rows, max_rows * k
        f32, i32 = dict(dtype=torch.float32, device=device), dict(dtype=torch.int32, device=device)
        self.ls = self.E + (1 if sg_logit else 0)
        self.logits = torch.empty(T, self.ls, **f32)
        self.ids = torch.empty(P, **i32)
        self.wts = torch.empty(P, **f32)
        self.sg = torch.empty(T, **f32) if sg_logit or router == "sigmoid" else None
        self.order = torch.empty(P, **i32)
        self.order_n = torch.zeros(2, **i32)
        self.egrp = torch.empty(3 * self.E, **i32)
        self.h = torch.empty(P, self.ff, **f32)
        self.y = torch.empty(P, self.d, **f32)
        self.out = torch.empty(T, self.d, **f32)
        self.vg, self.vd = vec_dot_type(L.tg), vec_dot_type(L.td)
        self.xq = torch.empty(T * q8_row_bytes(self.vg, self.d), dtype=torch.uint8, device=device)
        self.hq = torch.empty(P * q8_row_bytes(self.vd, self.ff), dtype=torch.uint8, device=device)
        # decode hands the hidden over as Q8_0 rows where the down type's partner is Q8_0, within the kernels' limits
        # (n <= 4096; k * ff / 32 <= 512 blocks and k * ff / 32 * 34 bytes <= 32 KiB per token)
        nbh = self.ff // 32
        self.dec_hq = (router == "softmax" and vec_dot_type(L.tg) == GType.Q8_0 and vec_dot_type(L.td) == GType.Q8_0
                       and self.d <= 4096 and self.k * nbh <= 512
                       and self.k * nbh * 34 <= 32768 and self.E <= 1024)
        self._side = None   # the shared expert's second stream, made on first use
        # decode's shared expert on a second stream: None = beyond 8 rows (up to 8 rows its gate/up and down read the
        # weights once for several rows and are shortest in order, ahead of the routed kernels: the 8-row IQ2_XS
        # verify with a Q4_K shared expert 332 us in order against 344-347 beside them; one row runs in order as well),
        # True / False = always / never
        self.shared_stream: Optional[bool] = None
        # prefill's shared expert on a second stream, beside the routing and the routed GEMMs
        self.prefill_shared_stream = True
        if shared is not None:
            S = shared.layer
            self.sh_ids = torch.zeros(T, **i32)
            self.sh_ones = torch.ones(T, **f32)
            self.sh_h = torch.empty(T, S.ff, **f32)
            self.sh_y = torch.empty(T, self.d, **f32)
            self.sh_order = torch.arange(T, **i32)
            # order_n = (nt, 1) and egrp = (expert 0, start 0, nt) in one buffer, so one strided fill writes both counts
            self.sh_cnt = torch.tensor([0, 1, 0, 0, 0], **i32)
            self.sh_order_n, self.sh_egrp = self.sh_cnt[0:2], self.sh_cnt[2:5]
            self.sh_xq = (None if vec_dot_type(S.tg) == self.vg
                          else torch.empty(T * q8_row_bytes(vec_dot_type(S.tg), self.d), dtype=torch.uint8, device=device))
            self.sh_hq = torch.empty(T * q8_row_bytes(vec_dot_type(S.td), S.ff), dtype=torch.uint8, device=device)

    def _route_logits(self, nt: int, stream=None):
        if self.router == "softmax":
            moe_route(self.logits, self.ls, self.E, self.k, self.ids, self.wts, self.sg, nt, stream)
        elif self.router == "sigmoid":
            moe_route_sig(self.logits, self.ls, self.router_bias, self.E, self.k, self.router_scale, self.ids, self.wts, self.sg,
                          nt, stream)
        else:
            moe_route_sqrtsp(self.logits, self.ls, self.router_bias, self.E, self.k, self.router_scale, self.ids, self.wts, nt,
                             stream)

    def route(self, x: torch.Tensor, nt: int, bias: Optional[torch.Tensor] = None, stream=None):
        rows = self.W_r.shape[0]
        gemv_f32(self.W_r, rows, self.d, x, x.stride(0), self.logits, self.ls, nt, stream,
                 bias=bias, bias_stride=0 if bias is None else bias.stride(0))
        self._route_logits(nt, stream)

    def _fork_side(self, stream):
        """the shared expert's second stream (default priority), made to wait for `stream`'s work so far"""
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.device)
            self._fork, self._join = torch.cuda.Event(), torch.cuda.Event()
        self._fork.record(stream if stream is not None else torch.cuda.current_stream())
        self._side.wait_event(self._fork)
        return self._side

    def _shared_decode(self, x, nt, stream):
        S = self.shared
        if vec_dot_type(S.layer.tg) == self.vg:   # the routed gate's Q8 rows of x serve the shared expert too
            moe_shared_gate_up(S, self.xq, self.sh_h, nt, stream)
        else:
            moe_gate_up(S, x, x.stride(0), self.sh_ids, 1, self.sh_h, nt, stream)
        moe_shared_down(S, self.sh_h, self.sh_y, nt, stream)

    def _shared_decode_legacy(self, x, nt, stream):
        S = self.shared
        moe_gate_up(S, x, x.stride(0), self.sh_ids, 1, self.sh_h, nt, stream)
        moe_down(S, self.sh_h, self.sh_ids, self.sh_ones, 1, self.sh_y, nt, stream)

    def _shared_prefill(self, x, nt, stream):
        S = self.shared
        # one active "expert" holding every token: (0, 0, nt).  The count is written on `stream` at every step (a fill
        # kernel, which a captured graph records with this step's nt), so an eager step or another capture of a
        # different nt in between never leaves a stale count behind.
        with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
            self.sh_cnt[0::4].fill_(nt)
        xq = self.xq   # the routed gate's Q8 rows of x, where the shared gate takes the same activation type
        if self.sh_xq is not None:
            q8_quantize(vec_dot_type(S.tg), x, x.stride(0), self.d, nt, self.sh_xq, stream)
            xq = self.sh_xq
        moe_gemm_gate_up(S, xq, 1, nt, self.sh_order, self.sh_order_n, self.sh_egrp, 1, self.sh_h, stream)
        q8_quantize(vec_dot_type(S.td), self.sh_h, S.layer.ff, S.layer.ff, nt, self.sh_hq, stream)
        moe_gemm_down(S, self.sh_hq, nt, self.sh_order, self.sh_order_n, self.sh_egrp, 1, self.sh_ones, self.sh_y, stream)

    def _check_rows(self, x: torch.Tensor, bias=None, resid: Optional[torch.Tensor] = None) -> int:
        """The kernels index every workspace buffer by token: x must fit the rows the runner was built for, and be
        float32 rows of d contiguous values on the runner's device (as must bias and resid)."""
        if x.dim() != 2 or x.shape[1] != self.d:
            raise ValueError(f"x must be [nt, {self.d}], got {tuple(x.shape)}")
        nt = x.shape[0]
        if nt > self.max_rows:
            raise ValueError(f"{nt} rows exceed the runner's max_rows {self.max_rows}")
        for name, t in (("x", x), ("bias", bias), ("resid", resid)):
            if t is None:
                continue
            if t.dtype != torch.float32 or t.device != self.device:
                raise ValueError(f"{name} must be float32 on {self.device}, got {t.dtype} on {t.device}")
            if t.dim() != 2 or t.shape[0] < nt or t.stride(1) != 1:
                raise ValueError(f"{name} must be 2-D with contiguous rows and at least {nt} of them")
            if name != "bias" and (t.stride(0) % 4 or t.data_ptr() % 16):
                raise ValueError(f"{name} rows must be 16-byte aligned")
        if bias is not None and bias.shape[1] < self.W_r.shape[0]:
            raise ValueError(f"bias rows must hold {self.W_r.shape[0]} logits")
        if resid is not None and resid.shape[1] != self.d:
            raise ValueError(f"resid must be [nt, {self.d}]")
        return nt

    def decode(self, x: torch.Tensor, bias=None, stream=None, resid: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Decode / short verify: router + Q8 of x, route + gate/up, down + combine (two more for a shared expert).
        With `resid` ([nt, d] fp32) the combine is added into it in place and resid is returned."""
        nt = self._check_rows(x, bias, resid)
        moe_router_q8(self.W_r, self.W_r.shape[0], self.d, x, x.stride(0), self.logits, self.ls, self.vg, self.xq, nt, stream,
                      bias=bias, bias_stride=0 if bias is None else bias.stride(0))
        shexp, joined = None, None
        side = self.shared_stream if self.shared_stream is not None else nt > 8
        if self.shared is not None and not side:
            self._shared_decode(x, nt, stream)
            shexp = self.sh_y
        elif self.shared is not None:
            # the shared expert does not depend on the routing: its two launches run on a second stream (default
            # priority), forked after the Q8 rows of x and joined before the combine
            self._shared_decode(x, nt, self._fork_side(stream))
            self._join.record(self._side)
            shexp, joined = self.sh_y, (stream if stream is not None else torch.cuda.current_stream())
        if self.dec_hq:
            moe_route_gate_up_q8(self.dev, self.logits, self.ls, self.E, self.k, self.xq, self.ids, self.wts, self.sg, self.h, self.hq,
                                 nt, stream)
            out = self.out if resid is None else resid
            if joined is not None:
                joined.wait_event(self._join)
            moe_down_reduce_q8(self.dev, self.hq, self.ids, self.wts, self.k, shexp, self.sg, out, resid is not None, nt, stream)
            return out[:nt]
        if self.router == "softmax":
            moe_route_gate_up(self.dev, self.logits, self.ls, self.E, self.k, self.xq, self.ids, self.wts, self.sg, self.h, nt, stream)
        else:   # the fused route + gate/up kernel routes by softmax: route first, then the gate/up GEMV by ids
            self._route_logits(nt, stream)
            moe_gate_up(self.dev, x, x.stride(0), self.ids, self.k, self.h, nt, stream)
        if joined is not None:
            joined.wait_event(self._join)
        if resid is not None:
            moe_down_reduce_residual(self.dev, self.h, self.ids, self.wts, self.k, shexp, self.sg, resid, nt, stream)
            return resid[:nt]
        moe_down_reduce(self.dev, self.h, self.ids, self.wts, self.k, shexp, self.sg, self.out, nt, stream)
        return self.out[:nt]

    def decode_legacy(self, x: torch.Tensor, bias=None, stream=None) -> torch.Tensor:
        """The same step through the reference-signature entry points (fp32 x and h in, quantized inside)."""
        nt = self._check_rows(x, bias)
        self.route(x, nt, bias, stream)
        shexp = None
        if self.shared is not None:
            self._shared_decode_legacy(x, nt, stream)
            shexp = self.sh_y
        moe_gate_up(self.dev, x, x.stride(0), self.ids, self.k, self.h, nt, stream)
        moe_down_reduce(self.dev, self.h, self.ids, self.wts, self.k, shexp, self.sg, self.out, nt, stream)
        return self.out[:nt]

    def prefill(self, x: torch.Tensor, bias=None, stream=None, resid: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Prefill: the grouped GEMM path.  With `resid` ([nt, d] fp32) the combine is added into it in place."""
        nt, k = self._check_rows(x, bias, resid), self.k
        P = nt * k
        moe_router_q8(self.W_r, self.W_r.shape[0], self.d, x, x.stride(0), self.logits, self.ls, self.vg, self.xq, nt, stream,
                      bias=bias, bias_stride=0 if bias is None else bias.stride(0))
        side = None
        if self.shared is not None and self.prefill_shared_stream:
            # the shared expert needs only the Q8 rows of x: its launches run beside the routing and the routed GEMMs
            side = self._fork_side(stream)
            self._shared_prefill(x, nt, side)
            self._join.record(side)
        self._route_logits(nt, stream)
        moe_order(self.dev, self.ids, P, self.E, self.order, self.order_n, stream, self.egrp)
        max_active = min(self.E, P)
        moe_gemm_gate_up(self.dev, self.xq, k, P, self.order, self.order_n, self.egrp, max_active, self.h, stream)
        q8_quantize(self.vd, self.h, self.ff, self.ff, P, self.hq, stream)
        moe_gemm_down(self.dev, self.hq, P, self.order, self.order_n, self.egrp, max_active, self.wts, self.y, stream)
        shexp = None
        if self.shared is not None:
            if side is None:
                self._shared_prefill(x, nt, stream)
            else:
                (stream if stream is not None else torch.cuda.current_stream()).wait_event(self._join)
            shexp = self.sh_y
        if resid is not None:
            moe_reduce_residual(shexp, self.sg, self.y, k, resid, self.d, nt, self.ids, stream)
            return resid[:nt]
        moe_reduce(shexp, self.sg, self.y, k, self.out, self.d, nt, self.ids, stream)
        return self.out[:nt]
