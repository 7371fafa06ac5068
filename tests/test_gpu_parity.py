"""GPU parity: every kernel of the path through the C ABI against the CPU oracle on the same seeded inputs.

Integer and index results (Q8 blocks, block integers, ids, order) must be identical; fp32 results are
bit-identical under the shared numeric contract (each test also states the 2e-3 relative-L2
bound on fp32 expert outputs, which bit-identity implies).
"""
import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import HyError, moe
from hyper_amd.formats import GType, block_bytes, block_elems, q8_row_bytes, random_blocks, vec_dot_type
from tests.helpers import (ALL_TYPES, D_RANGE, TYPES_256, assert_bits_equal, gen, layer, oracle_layer, rel_l2, routing,
                           x_distributions)

pytestmark = pytest.mark.gpu
TOL = 2e-3   # final fp32 expert outputs within 2e-3 relative L2 of the CPU path


def _sync():
    torch.cuda.synchronize()


# ------------------------------------------------------------------ A4: activation quantizers

@pytest.mark.parametrize("vt", [GType.Q8_K, GType.Q8_0])
def test_q8_quantize_bitexact(cuda, vt):
    n = 2048
    for name, x in x_distributions(4 * n, seed=11).items():
        x2 = x.reshape(4, n)
        ref = orc.quantize(vt, x2)
        xd = torch.from_numpy(x2).to(cuda)
        q = torch.zeros(4 * q8_row_bytes(vt, n), dtype=torch.uint8, device=cuda)
        moe.q8_quantize(vt, xd, n, n, 4, q)
        _sync()
        assert_bits_equal(q.cpu().numpy().reshape(ref.shape), ref, f"{vt.name} {name}")


# ------------------------------------------------------------------ A11: block decoding

@pytest.mark.parametrize("t", ALL_TYPES)
def test_dequant_row_bitexact(cuda, t):
    n = 4096
    nb = n // block_elems(t)
    blk = random_blocks(t, nb, gen(21 + int(t)), "cpu", D_RANGE.get(t, (1e-3, 1e-2)))
    row = blk.reshape(-1).numpy()
    ref = orc.dequant_row(t, row, n)
    out = torch.zeros(n, dtype=torch.float32, device=cuda)
    moe.dequant_row(t, blk.reshape(-1).to(cuda), n, out)
    _sync()
    assert_bits_equal(out.cpu().numpy(), ref, f"dequant {t.name}")


@pytest.mark.parametrize("t", ALL_TYPES)
def test_block_ints_bitexact(cuda, t):
    """The per-block int32 dot products (sumi, summ) of the decode kernels' item code."""
    n, nrows = 2048, 24
    rb = n // block_elems(t) * block_bytes(t)
    rows = random_blocks(t, nrows * n // block_elems(t), gen(31 + int(t)), "cpu", D_RANGE[t]).reshape(nrows, rb)
    vt = vec_dot_type(t)
    x = x_distributions(n, seed=7)["heavy"]
    xq = orc.quantize(vt, x)
    ref_si = np.stack([orc.block_ints(t, rows[i].numpy(), xq, n)[0] for i in range(nrows)])
    ref_sm = np.stack([orc.block_ints(t, rows[i].numpy(), xq, n)[1] for i in range(nrows)])
    nb = n // block_elems(t)
    si = torch.zeros(nrows * nb, dtype=torch.int32, device=cuda)
    sm = torch.zeros(nrows * nb, dtype=torch.int32, device=cuda)
    moe.block_ints(t, rows.reshape(-1).to(cuda), rb, nrows, torch.from_numpy(xq).to(cuda), n, si, sm)
    _sync()
    assert_bits_equal(si.cpu().numpy().reshape(nrows, nb), ref_si, f"sumi {t.name}")
    assert_bits_equal(sm.cpu().numpy().reshape(nrows, nb), ref_sm, f"summ {t.name}")


def test_block_ints_rejects_row_strides_that_break_span_alignment(cuda):
    """Row strides must keep each row's 256-value spans at the alignment they have in the uploaded layout (the largest
    power of two dividing the span, at most 16), which the 17- and 18-byte block types' reads count on: rejected
    before any launch, with the output left untouched; a padded stride that keeps the alignment is accepted."""
    n = 256
    for t, bad, good in ((GType.MXFP4, 136 + 4, 136 + 8), (GType.IQ4_NL, 144 + 2, 144 + 16), (GType.Q6_K, 211, 212)):
        rows = torch.zeros(2 * good, dtype=torch.uint8, device=cuda)
        xq = torch.from_numpy(orc.quantize(vec_dot_type(t), np.ones(n, np.float32))).to(cuda)
        nb = n // block_elems(t)
        si = torch.full((2 * nb,), 7, dtype=torch.int32, device=cuda)
        sm = torch.full((2 * nb,), 7, dtype=torch.int32, device=cuda)
        with pytest.raises(HyError, match="row_bytes"):
            moe.block_ints(t, rows, bad, 2, xq, n, si, sm)
        _sync()
        assert (si.cpu() == 7).all() and (sm.cpu() == 7).all()
        moe.block_ints(t, rows, good, 2, xq, n, si, sm)
        _sync()


# ------------------------------------------------------------------ A1-A3: router and bucketing

@pytest.mark.parametrize("rows,kdim,nt", [(128, 2048, 1), (129, 2048, 3), (288, 4096, 4), (128, 2048, 37)])
def test_router_gemv_bitexact(cuda, rows, kdim, nt):
    g = gen(41)
    W = torch.randn(rows, kdim, generator=g) * 0.02
    x = torch.randn(nt, kdim, generator=g)
    bias = torch.randn(nt, rows, generator=g)
    ref = orc.gemv_f32(W.numpy(), x.numpy())
    y = torch.zeros(nt, rows, device=cuda)
    moe.gemv_f32(W.to(cuda), rows, kdim, x.to(cuda), kdim, y, rows, nt)
    yb = torch.zeros(nt, rows, device=cuda)
    moe.gemv_f32(W.to(cuda), rows, kdim, x.to(cuda), kdim, yb, rows, nt, bias=bias.to(cuda), bias_stride=rows)
    _sync()
    assert_bits_equal(y.cpu().numpy(), ref, "logits")
    assert_bits_equal(yb.cpu().numpy(), (ref + bias.numpy()).astype(np.float32), "logits + bias")


@pytest.mark.parametrize("E,k,nt", [(128, 8, 7), (288, 8, 5), (384, 6, 9), (512, 10, 33), (1000, 14, 3), (64, 64, 2)])
def test_route_bitexact(cuda, E, k, nt):
    g = gen(51 + E)
    logits = torch.randn(nt, E + 1, generator=g) * 2
    logits[0, :E] = 0.25                  # all equal: ids 0..k-1 (tools/routebench.cu:20 tie test)
    if nt > 1:
        logits[1, 5] = logits[1, 9]       # an exact tie between two experts
    ids_r, wts_r, sg_r = orc.route(logits.numpy(), E, k, with_sg=True)
    ids = torch.zeros(nt * k, dtype=torch.int32, device=cuda)
    wts = torch.zeros(nt * k, device=cuda)
    sg = torch.zeros(nt, device=cuda)
    moe.moe_route(logits.to(cuda), E + 1, E, k, ids, wts, sg, nt)
    _sync()
    assert_bits_equal(ids.cpu().numpy().reshape(nt, k), ids_r, "ids")
    assert_bits_equal(wts.cpu().numpy().reshape(nt, k), wts_r, "wts")
    assert_bits_equal(sg.cpu().numpy(), sg_r, "sg")
    assert list(ids_r[0]) == list(range(k))


@pytest.mark.parametrize("E,P,absent,skew", [(128, 4096, 0, False), (512, 20480, 0, False), (288, 32, 5, False), (1024, 3000, 100, False),
                                              (16, 0, 0, False), (8, 333, 3, False), (1, 1500, 0, False), (128, 4096, 3, True),
                                              (128, 131072, 0, True)])
def test_order_bitexact(cuda, E, P, absent, skew):
    """Blocks of 1024 pairs each place their own range; ragged ends, one expert, Zipf-skewed ids (most pairs on a
    few experts) and 128 blocks."""
    rng = np.random.default_rng(E + P)
    slot = np.arange(E, dtype=np.int32)
    if absent:
        slot[rng.choice(E, absent, replace=False)] = -1
    if skew:
        ids = np.minimum(rng.zipf(1.3, P) - 1, E + 1).astype(np.int32)
    else:
        ids = rng.integers(-2, E + 2, P).astype(np.int32)   # includes out-of-range ids (skipped)
    o_r, on_r, eg_r = orc.order(slot, ids, E)
    dev = moe.MoeDev.__new__(moe.MoeDev)
    from hyper_amd import hy_moe_dev
    import ctypes
    sl = torch.from_numpy(slot).to(cuda)
    c = hy_moe_dev(); c.slot = sl.data_ptr(); c.n_expert = E; c.n_local = E
    dev.c, dev.ref, dev.slot = c, ctypes.byref(c), sl
    order = torch.full((max(P, 1),), -7, dtype=torch.int32, device=cuda)
    order_n = torch.zeros(2, dtype=torch.int32, device=cuda)
    egrp = torch.zeros(3 * E, dtype=torch.int32, device=cuda)
    moe.moe_order(dev, torch.from_numpy(ids).to(cuda) if P else order, P, E, order, order_n, egrp=egrp)
    _sync()
    on = order_n.cpu().numpy()
    assert_bits_equal(on, on_r, "order_n")
    assert_bits_equal(order.cpu().numpy()[:on[0]], o_r, "order")
    assert_bits_equal(egrp.cpu().numpy()[:3 * on[1]].reshape(-1, 3), eg_r, "egrp")


# ------------------------------------------------------------------ A5/A6/A9: decode GEMVs + combine

DECODE_CASES = [
    (GType.Q4_K, GType.Q4_K, 2048, 768, 8, 1),
    (GType.Q4_K, GType.Q6_K, 2048, 768, 8, 3),
    (GType.Q5_K, GType.Q6_K, 2048, 512, 10, 2),
    (GType.IQ4_NL, GType.IQ4_NL, 4096, 1536, 8, 1),
    (GType.IQ4_XS, GType.IQ4_XS, 4096, 1536, 8, 4),
    (GType.IQ2_XS, GType.IQ2_XS, 7168, 2048, 6, 2),
    (GType.Q8_0, GType.Q8_0, 2048, 768, 8, 2),
    (GType.Q8_0, GType.Q6_K, 2048, 512, 4, 3),
    (GType.IQ2_XXS, GType.IQ2_XXS, 7168, 2048, 6, 2),
    (GType.IQ2_XXS, GType.IQ2_XS, 2048, 768, 8, 3),
    (GType.MXFP4, GType.MXFP4, 2048, 768, 8, 2),
    (GType.MXFP4, GType.Q8_0, 4096, 1536, 4, 3),
    (GType.Q5_0, GType.Q5_0, 2048, 768, 8, 2),
    (GType.Q5_0, GType.Q4_K, 1024, 512, 6, 3),
    (GType.Q2_K, GType.Q2_K, 2048, 768, 8, 2),
    (GType.Q2_K, GType.Q6_K, 4096, 1536, 6, 3),
    (GType.Q3_K, GType.Q3_K, 2048, 768, 8, 2),
    (GType.Q3_K, GType.Q4_K, 2560, 512, 4, 3),
    (GType.IQ3_XXS, GType.IQ3_XXS, 7168, 2048, 6, 2),
    (GType.IQ3_XXS, GType.Q4_K, 2048, 768, 8, 3),
    (GType.IQ3_S, GType.IQ3_S, 4096, 1536, 8, 2),
    (GType.IQ3_S, GType.IQ4_XS, 2048, 768, 6, 3),
    (GType.IQ2_S, GType.IQ2_S, 7168, 2048, 6, 2),
    (GType.IQ2_S, GType.Q4_K, 2048, 768, 8, 3),
    (GType.IQ1_S, GType.IQ1_S, 7168, 2048, 6, 2),
    (GType.IQ1_S, GType.Q2_K, 2048, 768, 8, 3),
    (GType.Q5_1, GType.Q5_1, 2048, 768, 8, 2),
    (GType.Q5_1, GType.Q6_K, 4096, 1536, 4, 3),
]


@pytest.mark.parametrize("tg,td,d,ff,k,nt", DECODE_CASES)
def test_decode_gemv_bitexact(cuda, tg, td, d, ff, k, nt):
    E = 12
    L = layer(tg, td, E, ff, d, seed=61 + int(tg), clamp=0.0)
    OL = oracle_layer(L)
    ids, wts = routing(nt, E, k, seed=62)
    x = torch.randn(nt, d, generator=gen(63))
    out_r, h_r, y_r = orc.moe_layer(OL, x.numpy(), ids, wts, want_hy=True)
    dev = moe.upload_experts(L, device=cuda)
    xd, idsd, wtsd = x.to(cuda), torch.from_numpy(ids).reshape(-1).to(cuda), torch.from_numpy(wts).reshape(-1).to(cuda)
    h = torch.zeros(nt * k, ff, device=cuda)
    y = torch.zeros(nt * k, d, device=cuda)
    out = torch.zeros(nt, d, device=cuda)
    out2 = torch.zeros(nt, d, device=cuda)
    moe.moe_gate_up(dev, xd, d, idsd, k, h, nt)
    moe.moe_down(dev, h, idsd, wtsd, k, y, nt)
    moe.moe_reduce(None, None, y, k, out, d, nt, idsd)
    moe.moe_down_reduce(dev, h, idsd, wtsd, k, None, None, out2, nt)
    _sync()
    assert_bits_equal(h.cpu().numpy(), h_r, "h")
    assert_bits_equal(y.cpu().numpy(), (wts.reshape(-1, 1) * y_r).astype(np.float32), "y = w * down . q8(h)")
    assert_bits_equal(out.cpu().numpy(), out_r, "out (reduce)")
    assert_bits_equal(out2.cpu().numpy(), out_r, "out (fused down + reduce)")
    assert rel_l2(out.cpu().numpy(), out_r) <= TOL


def test_decode_clamp_and_order(cuda):
    """SwiGLU limit (src/cpu_moe.cpp:891-892) and the ordered pair list (skips non-local experts)."""
    tg = td = GType.Q4_K
    E, d, ff, k, nt = 10, 2048, 512, 4, 3
    L = layer(tg, td, E, ff, d, seed=71, clamp=3.0)
    OL = oracle_layer(L)
    ids, wts = routing(nt, E, k, seed=72)
    x = torch.randn(nt, d, generator=gen(73)) * 3
    _, h_r, y_r = orc.moe_layer(OL, x.numpy(), ids, wts, want_hy=True)
    dev = moe.upload_experts(L, device=cuda)
    idsd, wtsd = torch.from_numpy(ids).reshape(-1).to(cuda), torch.from_numpy(wts).reshape(-1).to(cuda)
    order = torch.zeros(nt * k, dtype=torch.int32, device=cuda)
    order_n = torch.zeros(2, dtype=torch.int32, device=cuda)
    moe.moe_order(dev, idsd, nt * k, E, order, order_n)
    h = torch.full((nt * k, ff), float("nan"), device=cuda)
    y = torch.full((nt * k, d), float("nan"), device=cuda)
    moe.moe_gate_up(dev, x.to(cuda), d, idsd, k, h, nt, order=order, order_n=order_n)
    moe.moe_down(dev, h, idsd, wtsd, k, y, nt, order=order, order_n=order_n)
    _sync()
    assert_bits_equal(h.cpu().numpy(), h_r, "h (clamped)")
    assert_bits_equal(y.cpu().numpy(), (wts.reshape(-1, 1) * y_r).astype(np.float32), "y")


# ------------------------------------------------------------------ A7/A8: grouped GEMMs

GEMM_CASES = [
    (GType.Q4_K, GType.Q6_K, 2048, 768, 8, 40),
    (GType.Q4_K, GType.Q4_K, 2048, 768, 8, 70),
    (GType.Q5_K, GType.Q6_K, 2048, 512, 10, 33),
    (GType.Q5_K, GType.Q6_K, 2048, 768, 10, 600),   # enough items for the 16-wave Q5_K gate/up (6 row blocks)
    (GType.IQ4_XS, GType.IQ4_XS, 4096, 1536, 8, 4),
    (GType.IQ2_XS, GType.IQ2_XS, 7168, 2048, 6, 8),
    (GType.IQ4_NL, GType.IQ4_NL, 4096, 1536, 8, 4),
    (GType.IQ4_NL, GType.IQ4_NL, 2048, 512, 8, 50),
    (GType.Q8_0, GType.Q8_0, 2048, 768, 8, 40),
    (GType.IQ2_XXS, GType.IQ2_XXS, 7168, 2048, 6, 8),
    (GType.IQ2_XXS, GType.Q6_K, 2048, 768, 8, 60),
    (GType.Q4_K, GType.Q8_0, 1024, 512, 4, 30),     # a K-quant gate/up with a Q8_0 down (Q8_K x, Q8_0 hidden)
    (GType.MXFP4, GType.MXFP4, 2048, 768, 8, 40),
    (GType.MXFP4, GType.Q6_K, 2048, 512, 4, 30),    # Q8_0 x for gate/up, a Q8_K hidden for the down
    (GType.Q5_0, GType.Q5_0, 2048, 768, 8, 40),
    (GType.Q4_K, GType.Q5_0, 1024, 512, 4, 30),
    (GType.Q2_K, GType.Q2_K, 2048, 768, 8, 40),
    (GType.Q2_K, GType.Q4_K, 2048, 1024, 6, 120),
    (GType.Q3_K, GType.Q3_K, 2048, 768, 8, 40),
    (GType.Q3_K, GType.Q6_K, 1024, 512, 4, 70),
    (GType.IQ3_XXS, GType.IQ3_XXS, 7168, 2048, 6, 8),
    (GType.IQ3_XXS, GType.Q6_K, 2048, 768, 8, 60),
    (GType.IQ3_S, GType.IQ3_S, 4096, 1536, 8, 12),
    (GType.IQ3_S, GType.Q4_K, 2048, 512, 6, 90),
    (GType.IQ2_S, GType.IQ2_S, 7168, 2048, 6, 8),
    (GType.IQ2_S, GType.Q6_K, 2048, 768, 8, 60),
    (GType.IQ1_S, GType.IQ1_S, 7168, 2048, 6, 8),
    (GType.IQ1_S, GType.Q4_K, 2048, 768, 8, 60),
    (GType.Q5_1, GType.Q5_1, 2048, 768, 8, 40),
    (GType.Q4_K, GType.Q5_1, 1024, 512, 4, 30),
    (GType.Q4_K, GType.Q6_K, 2048, 768, 1, 100),    # k = 1: the pair is the token (reciprocal 2^32)
    (GType.Q4_K, GType.Q6_K, 1024, 512, 3, 90),     # odd k: the pair-to-token multiply-high
    (GType.Q4_K, GType.Q6_K, 1024, 256, 16, 12),    # k = E: every expert active, every token in each
]


@pytest.mark.parametrize("tg,td,d,ff,k,nt", GEMM_CASES)
def test_grouped_gemm_bitexact(cuda, tg, td, d, ff, k, nt):
    E = 16
    L = layer(tg, td, E, ff, d, seed=81 + int(tg))
    OL = oracle_layer(L)
    ids, wts = routing(nt, E, k, seed=82, zipf=1.1)
    x = torch.randn(nt, d, generator=gen(83))
    out_r, h_r, y_r = orc.moe_layer(OL, x.numpy(), ids, wts, want_hy=True)
    dev = moe.upload_experts(L, device=cuda)
    P = nt * k
    idsd, wtsd = torch.from_numpy(ids).reshape(-1).to(cuda), torch.from_numpy(wts).reshape(-1).to(cuda)
    order = torch.zeros(P, dtype=torch.int32, device=cuda)
    order_n = torch.zeros(2, dtype=torch.int32, device=cuda)
    egrp = torch.zeros(3 * E, dtype=torch.int32, device=cuda)
    moe.moe_order(dev, idsd, P, E, order, order_n, egrp=egrp)
    xq = torch.zeros(nt * q8_row_bytes(vec_dot_type(tg), d), dtype=torch.uint8, device=cuda)
    moe.q8_quantize(vec_dot_type(tg), x.to(cuda), d, d, nt, xq)
    h = torch.full((P, ff), float("nan"), device=cuda)
    moe.moe_gemm_gate_up(dev, xq, k, P, order, order_n, egrp, E, h)
    hq = torch.zeros(P * q8_row_bytes(vec_dot_type(td), ff), dtype=torch.uint8, device=cuda)
    moe.q8_quantize(vec_dot_type(td), h, ff, ff, P, hq)
    y = torch.full((P, d), float("nan"), device=cuda)
    moe.moe_gemm_down(dev, hq, P, order, order_n, egrp, E, wtsd, y)
    out = torch.zeros(nt, d, device=cuda)
    moe.moe_reduce(None, None, y, k, out, d, nt, idsd)
    _sync()
    assert_bits_equal(h.cpu().numpy(), h_r, "h (grouped gate/up)")
    assert_bits_equal(y.cpu().numpy(), (wts.reshape(-1, 1) * y_r).astype(np.float32), "y (grouped down)")
    assert_bits_equal(out.cpu().numpy(), out_r, "out")
    assert rel_l2(out.cpu().numpy(), out_r) <= TOL


@pytest.mark.parametrize("tg,td,E,d,ff,k,nt,sh,sg_logit", [
    (GType.Q4_K, GType.Q6_K, 32, 2048, 768, 8, 40, GType.Q4_K, True),
    (GType.IQ4_XS, GType.IQ4_XS, 24, 4096, 1536, 8, 24, GType.IQ4_XS, False),
    # a shared gate whose activation type differs from the routed gate's (Q8_K against Q8_0): the shared expert's own
    # Q8 rows of x, quantized on its stream
    (GType.IQ4_NL, GType.IQ4_NL, 24, 2048, 512, 4, 40, GType.Q4_K, True),
    # a Q5_K shared expert: a single expert's gate/up in 16-wave blocks, here one item (the routed one in 8-wave blocks)
    (GType.Q5_K, GType.Q6_K, 16, 2048, 512, 4, 40, GType.Q5_K, True),
])
def test_runner_prefill_shared_matches_oracle(cuda, tg, td, E, d, ff, k, nt, sh, sg_logit):
    """Prefill through the runner with an always-on shared expert (and its sigmoid gate): the combine's shared
    term and the pairs' order against the oracle's layer."""
    L = layer(tg, td, E, ff, d, seed=900 + nt)
    S = layer(sh, td, 1, ff, d, seed=901)
    g = gen(902)
    W_r = torch.randn(E + (1 if sg_logit else 0), d, generator=g) * 0.02
    x = torch.randn(nt, d, generator=g)
    logits = orc.gemv_f32(W_r.numpy(), x.numpy())
    ids, wts, sgv = orc.route(logits, E, k, with_sg=sg_logit)
    out_r = orc.moe_layer(oracle_layer(L), x.numpy(), ids, wts, shared=oracle_layer(S), sg=sgv if sg_logit else None)
    r = moe.MoeLayerRunner(moe.upload_experts(L, device=cuda), W_r.to(cuda), k, max_rows=nt,
                           shared=moe.upload_experts(S, device=cuda), sg_logit=sg_logit)
    out = r.prefill(x.to(cuda)).clone()
    _sync()
    assert_bits_equal(out.cpu().numpy(), out_r, "runner.prefill")


def test_runner_prefill_shared_graph_replays(cuda):
    """The prefill step with a shared expert (and its sigmoid gate) captured into a HIP graph: every replay, with
    eager work and synchronizations between them, equals the eager step and the oracle, for two inputs in turn.  The
    eager steps in between take fewer rows than the captured one, so a shared-expert count left behind by them would
    show in the next replay."""
    tg, td, E, d, ff, k, nt = GType.Q4_K, GType.Q6_K, 32, 2048, 768, 8, 48
    L = layer(tg, td, E, ff, d, seed=920)
    S = layer(GType.Q4_K, td, 1, ff, d, seed=921)
    g = gen(922)
    W_r = torch.randn(E + 1, d, generator=g) * 0.02
    xs = [torch.randn(nt, d, generator=g) for _ in range(2)]
    refs = []
    for x in xs:
        logits = orc.gemv_f32(W_r.numpy(), x.numpy())
        ids, wts, sgv = orc.route(logits, E, k, with_sg=True)
        refs.append(orc.moe_layer(oracle_layer(L), x.numpy(), ids, wts, shared=oracle_layer(S), sg=sgv))
    r = moe.MoeLayerRunner(moe.upload_experts(L, device=cuda), W_r.to(cuda), k, max_rows=nt,
                           shared=moe.upload_experts(S, device=cuda), sg_logit=True)
    xin = torch.empty(nt, d, device=cuda)
    torch.cuda.synchronize()   # the uploads ran on the default stream; the step runs on another
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        xin.copy_(xs[0])
        eager = r.prefill(xin).clone()   # also the warm-up before capture
        torch.cuda.synchronize()
        assert_bits_equal(eager.cpu().numpy(), refs[0], "eager prefill")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = r.prefill(xin)
    for rep in range(4):
        i = rep % 2
        xin.copy_(xs[i].to(cuda))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_bits_equal(out.cpu().numpy(), refs[i], f"graph replay {rep}")
        nt2 = nt - 8 * (rep + 1)
        small = r.prefill(xin[:nt2].clone()).clone()   # eager work of another row count between replays
        torch.cuda.synchronize()
        if rep == 0:
            x2 = xs[i][:nt2].numpy()
            ids2, wts2, sg2 = orc.route(orc.gemv_f32(W_r.numpy(), x2), E, k, with_sg=True)
            ref2 = orc.moe_layer(oracle_layer(L), x2, ids2, wts2, shared=oracle_layer(S), sg=sg2)
            assert_bits_equal(small.cpu().numpy(), ref2, "eager prefill of fewer rows")

def test_reduce_unaligned_rows(cuda):
    """The combine with rows that are not a multiple of 4 (the scalar path): sg * shexp, then the valid pairs in
    ascending expert id, ties by position; ids < 0 are skipped and a token without pairs keeps sg * shexp."""
    nt, k, n = 5, 6, 257
    g = gen(910)
    y = torch.randn(nt * k, n, generator=g)
    shexp = torch.randn(nt, n, generator=g)
    sg = torch.rand(nt, generator=g)
    ids = torch.tensor([[5, 1, -1, 9, 3, 2], [0, 0, 4, -1, -1, 7], [-1] * 6, [12, 11, 10, 9, 8, 7], [3, -1, 3, 1, 2, 0]],
                       dtype=torch.int32)
    want = np.zeros((nt, n), dtype=np.float32)
    for t in range(nt):
        acc = (np.float32(sg[t]) * shexp[t].numpy()).astype(np.float32)
        for j in sorted((j for j in range(k) if ids[t, j] >= 0), key=lambda j: (int(ids[t, j]), j)):
            acc = (acc + y[t * k + j].numpy()).astype(np.float32)
        want[t] = acc
    out = torch.full((nt, n), float("nan"), device=cuda)
    moe.moe_reduce(shexp.to(cuda), sg.to(cuda), y.to(cuda), k, out, n, nt, ids.reshape(-1).to(cuda))
    _sync()
    assert_bits_equal(out.cpu().numpy(), want, "out")
