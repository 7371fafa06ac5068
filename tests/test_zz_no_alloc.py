"""hy_moe_decode_noalloc (the decode step on the library's own scratch array, no allocation) against hy_moe_decode (the
same step on a caller workspace): bit for bit, on two calls in a row whose second is smaller, with a shared expert and
its gate, then as a residual add; and against the CPU oracle.  Also at the largest row count whose intermediates fit
the 1 MiB array, and the refusal one row beyond it."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import HY_EBAD_SHAPE, lib, moe
from hyper_amd.formats import GType
from tests.helpers import assert_bits_equal, gen, layer, oracle_layer

pytestmark = pytest.mark.gpu


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_noalloc_decode_matches_workspace_entry(cuda):
    L = lib()
    E, d, ff, k = 64, 2048, 768, 8
    Lr = layer(GType.Q4_K, GType.Q6_K, E, ff, d, seed=4100)
    S = layer(GType.Q4_K, GType.Q6_K, 1, ff, d, seed=4101)
    m, sm = moe.upload_experts(Lr, device=cuda), moe.upload_experts(S, device=cuda)
    g = gen(4102)
    rows = E + 1
    W = (torch.randn(rows, d, generator=g) * 0.02).to(cuda)
    for nt in (8, 3):   # two calls in a row, the second smaller
        x = torch.randn(nt, d, generator=g).to(cuda)
        need = L.hy_moe_decode_ws_bytes(m.ref, rows, k, sm.ref, nt)
        ws = torch.empty(need + 256, dtype=torch.uint8, device=cuda)
        base = ctypes.c_void_p((ws.data_ptr() + 255) & ~255)
        a = torch.full((nt, d), float("nan"), device=cuda)
        b = torch.full((nt, d), float("nan"), device=cuda)
        assert L.hy_moe_decode(m.ref, _p(W), rows, _p(x), d, None, 0, k, sm.ref, _p(a), 0, nt, base, need, _stream()) == 0, L.hy_last_error()
        assert L.hy_moe_decode_noalloc(m.ref, _p(W), rows, _p(x), d, None, 0, k, sm.ref, _p(b), 0, nt, _stream()) == 0, L.hy_last_error()
        torch.cuda.synchronize()
        assert_bits_equal(b.cpu().numpy(), a.cpu().numpy(), f"noalloc vs workspace, {nt} rows")
        logits = orc.gemv_f32(W.cpu().numpy(), x.cpu().numpy())
        ids, wts, sgv = orc.route(logits, E, k, with_sg=True)
        ref = orc.moe_layer(oracle_layer(Lr), x.cpu().numpy(), ids, wts, shared=oracle_layer(S), sg=sgv)
        assert_bits_equal(b.cpu().numpy(), ref, f"noalloc vs oracle, {nt} rows")
        res0 = torch.randn(nt, d, generator=g)
        res = res0.to(cuda)
        assert L.hy_moe_decode_noalloc(m.ref, _p(W), rows, _p(x), d, None, 0, k, sm.ref, _p(res), 1, nt, _stream()) == 0, L.hy_last_error()
        torch.cuda.synchronize()
        assert_bits_equal(res.cpu().numpy(), (res0.numpy() + ref).astype(np.float32), f"noalloc residual, {nt} rows")


def test_noalloc_decode_at_its_scratch_limit(cuda):
    L = lib()
    E, d, ff, k = 128, 2048, 768, 8
    Lr = layer(GType.Q4_K, GType.Q6_K, E, ff, d, seed=4110)
    S = layer(GType.Q4_K, GType.Q6_K, 1, ff, d, seed=4111)
    m, sm = moe.upload_experts(Lr, device=cuda), moe.upload_experts(S, device=cuda)
    rows = E + 1
    need = {nt: L.hy_moe_decode_ws_bytes(m.ref, rows, k, sm.ref, nt) for nt in range(1, 65)}
    nt = max(n for n, b in need.items() if b <= 1 << 20)
    assert nt < 64 and need[nt + 1] > 1 << 20, "the layer's rows must reach past the scratch array"
    g = gen(4112)
    W = (torch.randn(rows, d, generator=g) * 0.02).to(cuda)
    x = torch.randn(nt + 1, d, generator=g).to(cuda)
    ws = torch.empty(need[nt] + 256, dtype=torch.uint8, device=cuda)
    base = ctypes.c_void_p((ws.data_ptr() + 255) & ~255)
    a = torch.full((nt, d), float("nan"), device=cuda)
    b = torch.full((nt + 1, d), float("nan"), device=cuda)
    assert L.hy_moe_decode(m.ref, _p(W), rows, _p(x), d, None, 0, k, sm.ref, _p(a), 0, nt, base, need[nt], _stream()) == 0, L.hy_last_error()
    assert L.hy_moe_decode_noalloc(m.ref, _p(W), rows, _p(x), d, None, 0, k, sm.ref, _p(b), 0, nt, _stream()) == 0, L.hy_last_error()
    torch.cuda.synchronize()
    assert_bits_equal(b[:nt].cpu().numpy(), a.cpu().numpy(), f"noalloc vs workspace, {nt} rows ({need[nt]} bytes)")
    assert torch.isnan(b[nt]).all(), "a row past nt was written"
    # one row more needs more than the array holds: refused before any launch
    assert L.hy_moe_decode_noalloc(m.ref, _p(W), rows, _p(x), d, None, 0, k, sm.ref, _p(b), 0, nt + 1, _stream()) == HY_EBAD_SHAPE
    assert b"scratch" in L.hy_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(b[nt]).all()
