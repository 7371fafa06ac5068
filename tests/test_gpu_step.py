"""hy_moe_decode: one MoE layer's decode step in one C call, its intermediates in a caller workspace.  Checked bit for
bit against the CPU oracle and against MoeLayerRunner.decode (the same launches through the separate entry points),
with and without a shared expert and its sigmoid gate, as a residual add, and with a router bias."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import HY_EINVAL, HY_EBAD_SHAPE, lib, moe
from hyper_amd.formats import GType
from tests.helpers import assert_bits_equal, gen, layer, oracle_layer

pytestmark = pytest.mark.gpu


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def decode_c(m, W_r, x, k, shared=None, out=None, residual=False, bias=None, ws=None):
    L = lib()
    nt, d = x.shape
    rows = W_r.shape[0]
    sref = shared.ref if shared is not None else None
    need = L.hy_moe_decode_ws_bytes(m.ref, rows, k, sref, nt)
    if ws is None:
        ws = torch.empty(need + 256, dtype=torch.uint8, device=x.device)
    base = (ws.data_ptr() + 255) & ~255
    if out is None:
        out = torch.full((nt, d), float("nan"), device=x.device)
    rc = L.hy_moe_decode(m.ref, _p(W_r), rows, _p(x), x.stride(0), _p(bias), 0 if bias is None else bias.stride(0), k, sref,
                         _p(out), int(residual), nt, ctypes.c_void_p(base), need, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, L.hy_last_error()
    return out, ws, base


@pytest.mark.parametrize("tg,td,E,d,ff,k,nt,shared,gate,bias", [
    (GType.Q4_K, GType.Q4_K, 128, 2048, 768, 8, 1, False, False, False),
    (GType.Q4_K, GType.Q6_K, 128, 2048, 768, 8, 4, False, False, True),
    (GType.IQ4_NL, GType.IQ4_NL, 96, 1024, 512, 8, 3, False, False, False),
    (GType.Q8_0, GType.Q8_0, 64, 1024, 512, 8, 2, True, False, False),        # the Q8_0 hidden hand-over, shared expert
    (GType.IQ2_XXS, GType.IQ2_XXS, 48, 1024, 512, 6, 4, True, True, False),   # IQ2_XXS layer, shared expert, its gate
    (GType.MXFP4, GType.MXFP4, 32, 2048, 768, 4, 3, False, False, True),      # MXFP4 layer: the Q8_0 hand-over, a bias
    (GType.Q5_0, GType.Q5_0, 40, 1024, 512, 8, 2, True, False, False),        # Q5_0 layer with a shared expert
    (GType.Q2_K, GType.Q2_K, 64, 2048, 768, 8, 1, False, False, False),
    (GType.Q3_K, GType.Q3_K, 32, 1024, 512, 4, 5, True, True, True),
    (GType.IQ3_XXS, GType.IQ3_XXS, 48, 1024, 512, 6, 4, True, True, False),
    (GType.IQ3_S, GType.IQ3_S, 64, 2048, 768, 8, 2, True, False, True),
    (GType.IQ2_S, GType.IQ2_S, 48, 1024, 512, 6, 3, True, True, False),
    (GType.IQ1_S, GType.IQ1_S, 48, 2048, 512, 6, 2, True, False, True),
    (GType.Q5_1, GType.Q5_1, 40, 1024, 512, 8, 3, True, True, False),      # Q5_1: the Q8_0 hand-over with the sum term
    (GType.IQ2_XS, GType.IQ2_XS, 64, 1024, 512, 6, 2, True, True, False),
    (GType.Q5_K, GType.Q6_K, 48, 512, 512, 4, 8, True, False, True),
    (GType.IQ4_XS, GType.IQ4_XS, 32, 512, 256, 4, 12, True, True, False),   # more than 8 rows: batched router
    # up to the 64-row limit: the batched router on d 2048 and 7168, 256-512 pair columns of route_gate_up, the
    # down kernel's rows per wave at 32-64 tokens, and the shared expert's fixed-expert launches at 32-64 rows
    (GType.Q4_K, GType.Q6_K, 128, 2048, 768, 8, 32, False, False, True),
    (GType.Q4_K, GType.Q6_K, 128, 2048, 768, 8, 64, True, True, False),
    (GType.IQ2_XS, GType.IQ2_XS, 64, 7168, 512, 6, 64, True, True, False),
])
def test_decode_step_matches_oracle_and_runner(cuda, tg, td, E, d, ff, k, nt, shared, gate, bias):
    seed = 3000 + E + nt
    L = layer(tg, td, E, ff, d, seed=seed)
    S = layer(GType.Q4_K, td if td != GType.IQ4_NL else GType.Q4_K, 1, ff, d, seed=seed + 1) if shared else None
    g = gen(seed + 2)
    rows = E + (1 if gate else 0)
    W_r = torch.randn(rows, d, generator=g) * 0.02
    x = torch.randn(nt, d, generator=g)
    b = torch.randn(nt, rows, generator=g) if bias else None
    logits = orc.gemv_f32(W_r.numpy(), x.numpy())
    if b is not None:
        logits = (logits + b.numpy()).astype(np.float32)
    ids, wts, sgv = orc.route(logits, E, k, with_sg=gate)
    ref = orc.moe_layer(oracle_layer(L), x.numpy(), ids, wts, shared=oracle_layer(S) if S is not None else None,
                        sg=sgv if gate else None)
    m = moe.upload_experts(L, device=cuda)
    sm = moe.upload_experts(S, device=cuda) if S is not None else None
    xd, Wd, bd = x.to(cuda), W_r.to(cuda), b.to(cuda) if b is not None else None
    out, ws, base = decode_c(m, Wd, xd, k, sm, bias=bd)
    torch.cuda.synchronize()
    assert_bits_equal(out.cpu().numpy(), ref, "hy_moe_decode")
    r = moe.MoeLayerRunner(m, Wd, k, nt, shared=sm, sg_logit=gate)
    assert_bits_equal(r.decode(xd, bias=bd).cpu().numpy(), ref, "runner")
    # the routing is left in the workspace: ids right after the logits
    off = ((nt * rows * 4 + 255) // 256) * 256
    ids_dev = ws[base - ws.data_ptr() + off: base - ws.data_ptr() + off + 4 * nt * k].view(torch.int32)
    assert_bits_equal(ids_dev.cpu().numpy().reshape(nt, k), ids, "ids")
    # residual: resid + out, one fp32 add
    res0 = torch.randn(nt, d, generator=g)
    res = res0.to(cuda)
    decode_c(m, Wd, xd, k, sm, out=res, residual=True, bias=bd)
    torch.cuda.synchronize()
    assert_bits_equal(res.cpu().numpy(), (res0.numpy() + ref).astype(np.float32), "residual")


def test_decode_step_rejects_bad_workspace_and_rows(cuda):
    L = lib()
    Lr = layer(GType.Q4_K, GType.Q4_K, 16, 256, 256, seed=77)
    m = moe.upload_experts(Lr, device=cuda)
    W = torch.zeros(16, 256, device=cuda)
    x = torch.zeros(1, 256, device=cuda)
    out = torch.zeros(1, 256, device=cuda)
    need = L.hy_moe_decode_ws_bytes(m.ref, 16, 4, None, 1)
    ws = torch.empty(need + 512, dtype=torch.uint8, device=cuda)
    base = (ws.data_ptr() + 255) & ~255
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.hy_moe_decode(m.ref, _p(W), 16, _p(x), 256, None, 0, 4, None, _p(out), 0, 1, ctypes.c_void_p(base), need - 1, s) == HY_EINVAL
    assert L.hy_moe_decode(m.ref, _p(W), 16, _p(x), 256, None, 0, 4, None, _p(out), 0, 1, ctypes.c_void_p(base + 4), need, s) == HY_EINVAL
    assert L.hy_moe_decode(m.ref, _p(W), 17 + 1, _p(x), 256, None, 0, 4, None, _p(out), 0, 1, ctypes.c_void_p(base), need, s) == HY_EBAD_SHAPE
    assert L.hy_moe_decode(m.ref, _p(W), 16, _p(x), 256, None, 0, 4, None, _p(out), 0, 65, ctypes.c_void_p(base), need, s) == HY_EBAD_SHAPE
