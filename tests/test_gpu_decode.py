"""GPU parity of the three-launch decode path -- router + Q8 of x, route + gate/up, down + combine -- against the
CPU oracle, through the C ABI.  Everything is compared bit for bit (the fp32 results share the oracle's
expression order); the 2e-3 relative-L2 bound on fp32 expert outputs is asserted as well."""
import ctypes
import types

import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import moe
from hyper_amd.formats import GType, q8_row_bytes, vec_dot_type
from tests.helpers import assert_bits_equal, assert_logits_close, gen, layer, oracle_layer, rel_l2, router_on_matrix_cores

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.mark.parametrize("E,d,nt,vt,with_sg,with_bias", [
    (128, 2048, 1, GType.Q8_K, False, False),
    (128, 2048, 8, GType.Q8_K, False, True),
    (288, 4096, 4, GType.Q8_0, False, False),
    (384, 7168, 8, GType.Q8_K, True, False),
    (512, 2048, 3, GType.Q8_K, True, True),
    # more than 8 rows: the batched routers.  The fmaf chain (logits bit for bit) where the matrix cores' 64 x 64 tiles
    # would leave CUs idle: LDS tiles of 8 tokens (64 x 512 x 12, 48 x 4096 x 300) or 16 (256 x 768 x 1024, 288 x 4096
    # x 512), register tiles for d % 256 != 0 (64 x 544 x 40), register rows (513 x 512 x 256 -- 17 row groups x 32
    # chunks --, 128 x 2048 x 512, one chunk a block, 199 x 2048 x 333, partial groups, chunks and token ranges, and
    # 16 x 2048 x 2048 below)
    (64, 512, 12, GType.Q8_0, True, False),
    (48, 4096, 300, GType.Q8_0, False, True),
    (256, 768, 1024, GType.Q8_K, True, False),
    (64, 544, 40, GType.Q8_0, False, True),     # an odd Q8_0 block count
    (512, 512, 256, GType.Q8_K, True, True),
    (128, 2048, 512, GType.Q8_K, False, True),  # the 512-token batch's shape
    (199, 2048, 333, GType.Q8_0, True, True),
    (288, 4096, 512, GType.Q8_K, False, False),
    # the matrix cores (logits within the fp32 bound, Q8 rows bit for bit): 64 x 64 tiles when they fill every CU
    (512, 2048, 2048, GType.Q8_K, False, True),   # the 2048-token chunk's shape, no rows past the tiles
    (512, 2048, 2040, GType.Q8_K, True, True),    # a shared-gate row past the tiles, a partial last token tile
    (600, 1024, 2048, GType.Q8_0, False, False),  # 24 rows past the tiles (a wave each), Q8_0 rows of x
    # K chunks of 64 that are no multiple of the four-chunk ring: 1 and 3 (every round partly past the end), 21
    (512, 64, 2048, GType.Q8_0, False, True),
    (512, 192, 2048, GType.Q8_0, True, False),
    (512, 1344, 2048, GType.Q8_0, False, True),
    (16, 2048, 2048, GType.Q8_K, False, True),    # too few rows for either: the register-row kernel
])
def test_router_q8_bitexact(cuda, E, d, nt, vt, with_sg, with_bias):
    g = gen(1000 + E + nt)
    rows = E + (1 if with_sg else 0)
    W = torch.randn(rows, d, generator=g) * 0.02
    x = torch.randn(nt, d, generator=g)
    bias = torch.randn(nt, rows, generator=g) if with_bias else None
    ref_log = orc.gemv_f32(W.numpy(), x.numpy())
    if bias is not None:
        ref_log = (ref_log + bias.numpy()).astype(np.float32)
    ref_q = orc.quantize(vt, x.numpy())
    logits = torch.full((nt, rows), float("nan"), device=cuda)
    xq = torch.zeros(nt * q8_row_bytes(vt, d), dtype=torch.uint8, device=cuda)
    moe.moe_router_q8(W.to(cuda), rows, d, x.to(cuda), d, logits, rows, vt, xq, nt,
                      bias=bias.to(cuda) if bias is not None else None, bias_stride=rows if bias is not None else 0)
    torch.cuda.synchronize()
    if router_on_matrix_cores(rows, d, nt):   # the matrix cores' sum order
        assert_logits_close(logits.cpu().numpy(), W.numpy(), x.numpy(), bias.numpy() if bias is not None else None)
    else:
        assert_bits_equal(logits.cpu().numpy(), ref_log, "logits")
    assert_bits_equal(xq.cpu().numpy().reshape(ref_q.shape), ref_q, "xq")


ROUTE_GU_CASES = [
    # tg, td, E, d, ff, k, nt, sg
    (GType.Q4_K, GType.Q4_K, 128, 2048, 768, 8, 1, False),
    (GType.Q4_K, GType.Q6_K, 128, 2048, 768, 8, 3, True),
    (GType.Q5_K, GType.Q6_K, 40, 2048, 512, 10, 2, False),
    (GType.IQ4_NL, GType.IQ4_NL, 24, 4096, 1536, 8, 1, False),
    (GType.IQ4_XS, GType.IQ4_XS, 24, 4096, 1536, 8, 4, False),
    (GType.IQ2_XS, GType.IQ2_XS, 16, 7168, 2048, 6, 2, True),
    (GType.IQ4_NL, GType.IQ4_NL, 16, 2048, 4096, 8, 2, False),   # k * ff / 32 > 512: down falls back to the R-row kernel
    (GType.Q4_K, GType.Q6_K, 64, 2560, 512, 8, 4, False),         # down: 3 rows a wave, the last block's rows past n
    (GType.Q8_0, GType.Q8_0, 32, 2048, 768, 8, 2, True),
    (GType.Q8_0, GType.Q4_K, 24, 1024, 512, 6, 3, False),
    (GType.IQ2_XXS, GType.IQ2_XXS, 16, 7168, 2048, 6, 2, True),
    (GType.IQ2_XXS, GType.IQ2_XS, 20, 2048, 768, 8, 3, False),
    (GType.MXFP4, GType.MXFP4, 32, 2048, 768, 8, 2, True),
    (GType.MXFP4, GType.Q4_K, 24, 1024, 512, 6, 3, False),
    (GType.Q5_0, GType.Q5_0, 32, 2048, 768, 8, 2, True),
    (GType.Q2_K, GType.Q2_K, 64, 2048, 1024, 8, 3, False),
    (GType.Q3_K, GType.Q3_K, 48, 2048, 768, 6, 2, True),
    (GType.IQ3_XXS, GType.IQ3_XXS, 16, 7168, 2048, 6, 2, True),
    (GType.IQ3_XXS, GType.IQ2_XXS, 20, 2048, 768, 8, 3, False),
    (GType.IQ3_S, GType.IQ3_S, 24, 4096, 1536, 8, 2, True),
    (GType.IQ3_S, GType.IQ2_XS, 16, 7168, 2048, 6, 1, False),
    (GType.IQ2_S, GType.IQ2_S, 16, 7168, 2048, 6, 2, True),
    (GType.IQ2_S, GType.IQ3_S, 24, 2048, 768, 8, 3, False),
    (GType.IQ1_S, GType.IQ1_S, 16, 7168, 2048, 6, 2, True),
    (GType.IQ1_S, GType.IQ2_XXS, 24, 2048, 768, 8, 3, False),
    (GType.Q5_1, GType.Q5_1, 32, 2048, 768, 8, 2, True),
    (GType.Q5_1, GType.Q4_K, 24, 1024, 512, 6, 3, False),
]


def _logits(E, nt, sg, seed):
    g = gen(seed)
    return (torch.randn(nt, E + (1 if sg else 0), generator=g) * 1.5).numpy().astype(np.float32)


@pytest.mark.parametrize("tg,td,E,d,ff,k,nt,sg", ROUTE_GU_CASES)
def test_route_gate_up_and_down_bitexact(cuda, tg, td, E, d, ff, k, nt, sg):
    L = layer(tg, td, E, ff, d, seed=700 + int(tg) + nt)
    OL = oracle_layer(L)
    dev = moe.upload_experts(L, device=cuda)
    vg = vec_dot_type(tg)
    for rep, rows in enumerate((nt, max(1, nt - 1))):
        lg = _logits(E, rows, sg, 710 + rep)
        ls = lg.shape[1]
        ids_r, wts_r, sg_r = orc.route(lg, E, k, with_sg=sg)
        x = torch.randn(rows, d, generator=gen(720 + rep))
        out_r, h_r, _ = orc.moe_layer(OL, x.numpy(), ids_r, wts_r, want_hy=True)
        xq = torch.from_numpy(orc.quantize(vg, x.numpy())).reshape(-1).to(cuda)
        ids = torch.full((rows * k,), -5, dtype=torch.int32, device=cuda)
        wts = torch.zeros(rows * k, device=cuda)
        sgd = torch.zeros(rows, device=cuda) if sg else None
        h = torch.full((rows * k, ff), float("nan"), device=cuda)
        out = torch.full((rows, d), float("nan"), device=cuda)
        moe.moe_route_gate_up(dev, torch.from_numpy(lg).to(cuda), ls, E, k, xq, ids, wts, sgd, h, rows)
        moe.moe_down_reduce(dev, h, ids, wts, k, None, None, out, rows)
        torch.cuda.synchronize()
        assert_bits_equal(ids.cpu().numpy().reshape(rows, k), ids_r, f"ids rep {rep}")
        assert_bits_equal(wts.cpu().numpy().reshape(rows, k), wts_r, f"wts rep {rep}")
        if sg:
            assert_bits_equal(sgd.cpu().numpy(), sg_r, f"sg rep {rep}")
        assert_bits_equal(h.cpu().numpy(), h_r, f"h rep {rep}")
        assert_bits_equal(out.cpu().numpy(), out_r, f"out rep {rep}")
        assert rel_l2(out.cpu().numpy(), out_r) <= TOL


def _tie_logits(E, seed):
    """Three tokens whose routing leans on the tie rules: equal top logits, top logits a few ulps apart (their
    probabilities can round to one value), and all logits equal (the selection is the k lowest ids)."""
    rng = np.random.default_rng(seed)
    lg = (rng.standard_normal((3, E)) * 0.5).astype(np.float32)
    top = rng.permutation(E)[:6]
    lg[0, top] = 2.0
    lg[1] -= 2.0
    lg[1, top] = np.float32(0.25) - np.arange(6, dtype=np.float32) * np.float32(2.0 ** -26)   # one ulp apart
    lg[2, :] = 0.25
    return lg


# up to 128 experts: the eight-wave ranks; more: one wave
@pytest.mark.parametrize("E,k", [(40, 8), (128, 8), (8, 8), (64, 64), (288, 8), (384, 6), (512, 16), (300, 17), (129, 1)])
def test_route_gate_up_tie_rules(cuda, E, k):
    """The fused routing (logit ranks, checked against the probabilities, else ranks of the probabilities)
    selects, orders and weights the experts exactly as the oracle's router on ties."""
    tg = td = GType.Q4_K
    d, ff = (2048, 256) if E <= 128 else (256, 256)
    L = layer(tg, td, E, ff, d, seed=760 + E)
    OL = oracle_layer(L)
    dev = moe.upload_experts(L, device=cuda)
    lg = _tie_logits(E, 761 + k)
    nt = lg.shape[0]
    ids_r, wts_r, _ = orc.route(lg, E, k)
    x = torch.randn(nt, d, generator=gen(762))
    _, h_r, _ = orc.moe_layer(OL, x.numpy(), ids_r, wts_r, want_hy=True)
    xq = torch.from_numpy(orc.quantize(GType.Q8_K, x.numpy())).reshape(-1).to(cuda)
    ids = torch.full((nt * k,), -5, dtype=torch.int32, device=cuda)
    wts = torch.zeros(nt * k, device=cuda)
    h = torch.full((nt * k, ff), float("nan"), device=cuda)
    moe.moe_route_gate_up(dev, torch.from_numpy(lg).to(cuda), E, E, k, xq, ids, wts, None, h, nt)
    torch.cuda.synchronize()
    assert_bits_equal(ids.cpu().numpy().reshape(nt, k), ids_r, "ids")
    assert_bits_equal(wts.cpu().numpy().reshape(nt, k), wts_r, "wts")
    assert_bits_equal(h.cpu().numpy(), h_r, "h")
    assert list(ids_r[2]) == list(range(k)), "all-equal logits select the k lowest ids"


@pytest.mark.parametrize("E,k,sg", [(288, 8, False), (384, 6, True), (512, 10, True), (200, 16, False)])
def test_route_gate_up_many_experts(cuda, E, k, sg):
    """Random logits over 129-512 experts (one wave routes them), four tokens: ids, weights, the shared gate and h
    equal the oracle's."""
    tg = td = GType.Q4_K
    d, ff, nt = 256, 256, 4
    L = layer(tg, td, E, ff, d, seed=780 + E)
    OL = oracle_layer(L)
    dev = moe.upload_experts(L, device=cuda)
    lg = _logits(E, nt, sg, 781 + k)
    ids_r, wts_r, sg_r = orc.route(lg, E, k, with_sg=sg)
    x = torch.randn(nt, d, generator=gen(782))
    _, h_r, _ = orc.moe_layer(OL, x.numpy(), ids_r, wts_r, want_hy=True)
    xq = torch.from_numpy(orc.quantize(GType.Q8_K, x.numpy())).reshape(-1).to(cuda)
    ids = torch.full((nt * k,), -5, dtype=torch.int32, device=cuda)
    wts = torch.zeros(nt * k, device=cuda)
    sgd = torch.zeros(nt, device=cuda) if sg else None
    h = torch.full((nt * k, ff), float("nan"), device=cuda)
    moe.moe_route_gate_up(dev, torch.from_numpy(lg).to(cuda), lg.shape[1], E, k, xq, ids, wts, sgd, h, nt)
    torch.cuda.synchronize()
    assert_bits_equal(ids.cpu().numpy().reshape(nt, k), ids_r, "ids")
    assert_bits_equal(wts.cpu().numpy().reshape(nt, k), wts_r, "wts")
    if sg:
        assert_bits_equal(sgd.cpu().numpy(), sg_r, "sg")
    assert_bits_equal(h.cpu().numpy(), h_r, "h")


def test_decode_skips_non_local_experts(cuda):
    """Experts without a slot leave their h rows unwritten and drop out of the sum, as on the CPU."""
    tg = td = GType.Q4_K
    E, d, ff, k, nt = 12, 2048, 512, 4, 3
    L = layer(tg, td, E, ff, d, seed=730)
    slot = [(-1 if e in (2, 5, 7) else e) for e in range(E)]
    dev = moe.upload_experts(L, slot=slot, device=cuda)
    lg = _logits(E, nt, False, 731)
    ids_r, wts_r, _ = orc.route(lg, E, k)
    x = torch.randn(nt, d, generator=gen(732))
    local = np.array([slot[e] >= 0 for e in ids_r.reshape(-1)]).reshape(ids_r.shape)
    assert not local.all(), "the case must route some pairs to non-local experts"
    ids_cpu = np.where(local, ids_r, -1).astype(np.int32)
    out_r, h_r, _ = orc.moe_layer(oracle_layer(L), x.numpy(), ids_cpu, wts_r, want_hy=True)
    xq = torch.from_numpy(orc.quantize(GType.Q8_K, x.numpy())).reshape(-1).to(cuda)
    ids = torch.zeros(nt * k, dtype=torch.int32, device=cuda)
    wts = torch.zeros(nt * k, device=cuda)
    h = torch.full((nt * k, ff), float("nan"), device=cuda)
    out = torch.zeros(nt, d, device=cuda)
    moe.moe_route_gate_up(dev, torch.from_numpy(lg).to(cuda), E, E, k, xq, ids, wts, None, h, nt)
    moe.moe_down_reduce(dev, h, ids, wts, k, None, None, out, nt)
    torch.cuda.synchronize()
    hv = h.cpu().numpy()
    lv = local.reshape(-1)
    assert_bits_equal(hv[lv], h_r[lv], "h of local pairs")
    assert np.isnan(hv[~lv]).all()
    assert_bits_equal(out.cpu().numpy(), out_r, "out")


def test_slot_entries_outside_n_local_are_absent(cuda):
    """A slot-table entry outside [0, n_local) (a stale or corrupt table) makes its expert absent in every kernel
    that reads the table -- routed gate/up, down + combine, the separate gate/up and down GEMVs, the fused GEMV down
    + combine and the bucketing -- instead of forming a weight address past the allocation."""
    tg = td = GType.Q4_K
    E, d, ff, k, nt = 12, 2048, 512, 4, 3
    L = layer(tg, td, E, ff, d, seed=740)
    dev = moe.upload_experts(L, device=cuda)
    assert dev.c.n_local == E
    bad = {1: E, 4: E + 1000, 6: 1 << 30, 9: -5}
    for e, v in bad.items():
        dev.slot[e] = v
    torch.cuda.synchronize()
    lg = _logits(E, nt, False, 741)
    ids_r, wts_r, _ = orc.route(lg, E, k)
    local = np.array([e not in bad for e in ids_r.reshape(-1)]).reshape(ids_r.shape)
    assert not local.all(), "the case must route some pairs to the corrupted entries"
    ids_cpu = np.where(local, ids_r, -1).astype(np.int32)
    x = torch.randn(nt, d, generator=gen(742))
    out_r, h_r, _ = orc.moe_layer(oracle_layer(L), x.numpy(), ids_cpu, wts_r, want_hy=True)
    xq = torch.from_numpy(orc.quantize(GType.Q8_K, x.numpy())).reshape(-1).to(cuda)
    ids = torch.zeros(nt * k, dtype=torch.int32, device=cuda)
    wts = torch.zeros(nt * k, device=cuda)
    h = torch.full((nt * k, ff), float("nan"), device=cuda)
    out = torch.zeros(nt, d, device=cuda)
    moe.moe_route_gate_up(dev, torch.from_numpy(lg).to(cuda), E, E, k, xq, ids, wts, None, h, nt)
    moe.moe_down_reduce(dev, h, ids, wts, k, None, None, out, nt)
    torch.cuda.synchronize()
    lv = local.reshape(-1)
    hv = h.cpu().numpy()
    assert_bits_equal(hv[lv], h_r[lv], "h of local pairs")
    assert np.isnan(hv[~lv]).all()
    assert_bits_equal(out.cpu().numpy(), out_r, "out (route + gate/up, down + combine)")
    # the reference-signature GEMVs on the same routing
    xd = x.to(cuda)
    h2 = torch.full((nt * k, ff), float("nan"), device=cuda)
    y2 = torch.full((nt * k, d), float("nan"), device=cuda)
    moe.moe_gate_up(dev, xd, d, ids, k, h2, nt)
    moe.moe_down(dev, h2, ids, wts, k, y2, nt)
    torch.cuda.synchronize()
    assert_bits_equal(h2.cpu().numpy()[lv], h_r[lv], "moe_gate_up h of local pairs")
    assert np.isnan(h2.cpu().numpy()[~lv]).all()
    assert (y2.cpu().numpy()[~lv] == 0).all(), "moe_down writes zeros for pairs without a local expert"
    # bucketing drops the corrupted experts' pairs
    P = nt * k
    order = torch.full((P,), -7, dtype=torch.int32, device=cuda)
    order_n = torch.zeros(2, dtype=torch.int32, device=cuda)
    egrp = torch.zeros(3 * E, dtype=torch.int32, device=cuda)
    moe.moe_order(dev, ids, P, E, order, order_n, egrp=egrp)
    torch.cuda.synchronize()
    slot_eff = np.array([-1 if e in bad else e for e in range(E)], np.int32)
    o_r, on_r, eg_r = orc.order(slot_eff, ids_r.reshape(-1).astype(np.int32), E)
    on = order_n.cpu().numpy()
    assert_bits_equal(on, on_r, "order_n")
    assert_bits_equal(order.cpu().numpy()[:on[0]], o_r, "order")
    assert_bits_equal(egrp.cpu().numpy()[:3 * on[1]].reshape(-1, 3), eg_r, "egrp")


RUNNER_CASES = [
    # tg, td, E, d, ff, k, nt, shared (type or None), sg_logit
    (GType.Q4_K, GType.Q4_K, 128, 2048, 768, 8, 1, None, False),
    (GType.IQ4_NL, GType.IQ4_NL, 24, 4096, 1536, 8, 4, None, False),
    (GType.IQ4_XS, GType.IQ4_XS, 24, 4096, 1536, 8, 1, None, False),
    (GType.IQ2_XS, GType.IQ2_XS, 16, 7168, 2048, 6, 1, GType.Q4_K, True),
    (GType.IQ2_XS, GType.IQ2_XS, 16, 7168, 2048, 6, 8, GType.Q4_K, True),
    (GType.Q5_K, GType.Q6_K, 32, 2048, 512, 10, 2, GType.Q5_K, False),
]


@pytest.mark.parametrize("tg,td,E,d,ff,k,nt,sh,sg_logit", RUNNER_CASES)
def test_runner_decode_matches_oracle(cuda, tg, td, E, d, ff, k, nt, sh, sg_logit):
    L = layer(tg, td, E, ff, d, seed=600 + E + nt)
    S = layer(sh, GType.Q6_K if sh == GType.Q5_K else sh, 1, ff, d, seed=601) if sh is not None else None
    g = gen(602)
    W_r = torch.randn(E + (1 if sg_logit else 0), d, generator=g) * 0.02
    x = torch.randn(nt, d, generator=g)
    logits = orc.gemv_f32(W_r.numpy(), x.numpy())
    ids, wts, sgv = orc.route(logits, E, k, with_sg=sg_logit)
    out_r = orc.moe_layer(oracle_layer(L), x.numpy(), ids, wts, shared=oracle_layer(S) if S is not None else None,
                          sg=sgv if sg_logit else None)
    dev = moe.upload_experts(L, device=cuda)
    sdev = moe.upload_experts(S, device=cuda) if S is not None else None
    r = moe.MoeLayerRunner(dev, W_r.to(cuda), k, max_rows=8, shared=sdev, sg_logit=sg_logit)
    xd = x.to(cuda)
    out = r.decode(xd).clone()
    out_legacy = r.decode_legacy(xd).clone()
    torch.cuda.synchronize()
    assert_bits_equal(out.cpu().numpy(), out_r, "runner.decode")
    assert_bits_equal(out_legacy.cpu().numpy(), out_r, "runner.decode_legacy")
    assert rel_l2(out.cpu().numpy(), out_r) <= TOL


@pytest.mark.parametrize("tg,td", [(GType.Q4_K, GType.Q6_K), (GType.IQ4_NL, GType.IQ4_NL)])
def test_c_abi_upload_matches_python_upload(cuda, tg, td):
    """hy_upload_experts (host-side tiling) and the Python upload (device-side tiling) hand the kernels the same
    bytes: the decode through either matches the oracle bit for bit."""
    E, d, ff, k, nt = 12, 2048, 512, 4, 2
    L = layer(tg, td, E, ff, d, seed=740 + int(tg))
    slot = [(-1 if e == 3 else (E + 2 - e if e > 3 else e)) for e in range(E)]   # 0 1 2 -1 10 9 ... 3: unique
    c = moe.upload_experts_c(L, slot)
    try:
        py = moe.upload_experts(L, slot=slot, device=cuda)
        cd = types.SimpleNamespace(c=c, ref=ctypes.byref(c))
        lg = _logits(E, nt, False, 741)
        ids_r, wts_r, _ = orc.route(lg, E, k)
        x = torch.randn(nt, d, generator=gen(742))
        local = np.array([slot[e] >= 0 for e in ids_r.reshape(-1)]).reshape(ids_r.shape)
        out_r = orc.moe_layer(oracle_layer(L), x.numpy(), np.where(local, ids_r, -1).astype(np.int32), wts_r)
        xq = torch.from_numpy(orc.quantize(vec_dot_type(tg), x.numpy())).reshape(-1).to(cuda)
        for dev in (cd, py):
            ids = torch.zeros(nt * k, dtype=torch.int32, device=cuda)
            wts = torch.zeros(nt * k, device=cuda)
            h = torch.zeros(nt * k, ff, device=cuda)
            out = torch.full((nt, d), float("nan"), device=cuda)
            moe.moe_route_gate_up(dev, torch.from_numpy(lg).to(cuda), E, E, k, xq, ids, wts, None, h, nt)
            moe.moe_down_reduce(dev, h, ids, wts, k, None, None, out, nt)
            torch.cuda.synchronize()
            assert_bits_equal(out.cpu().numpy(), out_r, "out")
    finally:
        moe.free_experts(c)


@pytest.mark.parametrize("side", [True, False])
def test_runner_decode_shared_graph_replays(cuda, side):
    """Decode with a shared expert (its launches on a second stream forked and joined inside the step, or in order)
    captured into a HIP graph: every replay, with eager steps (fewer rows) and synchronizations in between, equals the
    oracle."""
    tg, td, E, d, ff, k, nt = GType.Q4_K, GType.Q6_K, 32, 2048, 512, 6, 3
    L = layer(tg, td, E, ff, d, seed=940)
    S = layer(GType.Q4_K, GType.Q6_K, 1, ff, d, seed=941)
    g = gen(942)
    W_r = torch.randn(E + 1, d, generator=g) * 0.02
    xs = [torch.randn(nt, d, generator=g) for _ in range(2)]

    def ref(x):
        logits = orc.gemv_f32(W_r.numpy(), x.numpy())
        ids, wts, sgv = orc.route(logits, E, k, with_sg=True)
        return orc.moe_layer(oracle_layer(L), x.numpy(), ids, wts, shared=oracle_layer(S), sg=sgv)

    refs = [ref(x) for x in xs]
    r = moe.MoeLayerRunner(moe.upload_experts(L, device=cuda), W_r.to(cuda), k, max_rows=nt,
                           shared=moe.upload_experts(S, device=cuda), sg_logit=True)
    r.shared_stream = side
    xin = torch.empty(nt, d, device=cuda)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        xin.copy_(xs[0])
        eager = r.decode(xin).clone()
        torch.cuda.synchronize()
        assert_bits_equal(eager.cpu().numpy(), refs[0], "eager decode")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = r.decode(xin)
    for rep in range(4):
        i = rep % 2
        xin.copy_(xs[i].to(cuda))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_bits_equal(out.cpu().numpy(), refs[i], f"replay {rep}")
        one = r.decode(xs[1 - i][:1].to(cuda)).clone()   # an eager step of one row in between
        torch.cuda.synchronize()
        assert_bits_equal(one.cpu().numpy(), ref(xs[1 - i][:1]), f"eager one-row step {rep}")


SHARED_CASES = [
    # tg, td, d, ff, nt: 1 row (the per-token kernels), 2..8 rows (one pass over the weights for every row), more
    # than 8 or beyond the one-pass kernels' LDS (the per-token kernels again)
    (GType.Q4_K, GType.Q4_K, 7168, 2048, 1), (GType.Q4_K, GType.Q4_K, 7168, 2048, 4), (GType.Q4_K, GType.Q4_K, 7168, 2048, 8),
    (GType.Q5_K, GType.Q6_K, 2048, 512, 5), (GType.IQ2_XS, GType.IQ2_XS, 7168, 2048, 8), (GType.IQ4_NL, GType.IQ4_NL, 4096, 1536, 2),
    (GType.IQ4_NL, GType.IQ4_NL, 4096, 1536, 8), (GType.Q4_K, GType.Q6_K, 2048, 768, 12), (GType.IQ4_XS, GType.IQ4_XS, 4096, 1536, 3),
    (GType.Q8_0, GType.Q8_0, 2048, 768, 6), (GType.MXFP4, GType.MXFP4, 2048, 768, 7), (GType.Q5_0, GType.Q5_1, 2048, 768, 2),
    (GType.Q5_1, GType.Q5_0, 1024, 512, 8), (GType.Q2_K, GType.Q3_K, 2048, 1024, 4), (GType.Q3_K, GType.Q2_K, 2048, 768, 3),
    (GType.IQ1_S, GType.IQ2_S, 7168, 2048, 5), (GType.IQ2_S, GType.IQ1_S, 2048, 768, 8), (GType.IQ3_S, GType.IQ3_XXS, 4096, 1536, 4),
    (GType.IQ3_XXS, GType.IQ2_XXS, 2048, 768, 6), (GType.IQ2_XXS, GType.IQ3_S, 2048, 768, 2), (GType.Q6_K, GType.Q4_K, 2048, 512, 8),
]


@pytest.mark.parametrize("tg,td,d,ff,nt", SHARED_CASES)
def test_shared_gate_up_and_down_bitexact(cuda, tg, td, d, ff, nt):
    """hy_moe_shared_gate_up / hy_moe_shared_down: local expert 0 for every row from the Q8 rows of x, then its
    down for every row, bit for bit the oracle's h and output with every id 0, weight 1 and k = 1 (the shared
    expert), twice in a row (the second call with fewer rows)."""
    L = layer(tg, td, 1, ff, d, seed=960 + int(tg) + nt)
    dev = moe.upload_experts(L, device=cuda)
    OL = oracle_layer(L)
    for rep, rows in enumerate((nt, max(1, nt - 3))):
        x = torch.randn(rows, d, generator=gen(961 + rep))
        ids = np.zeros((rows, 1), dtype=np.int32)
        wts = np.ones((rows, 1), dtype=np.float32)
        out_r, h_r, _ = orc.moe_layer(OL, x.numpy(), ids, wts, want_hy=True)
        xq = torch.from_numpy(orc.quantize(vec_dot_type(tg), x.numpy())).reshape(-1).to(cuda)
        h = torch.full((rows, ff), float("nan"), device=cuda)
        y = torch.full((rows, d), float("nan"), device=cuda)
        moe.moe_shared_gate_up(dev, xq, h, rows)
        moe.moe_shared_down(dev, h, y, rows)
        torch.cuda.synchronize()
        assert_bits_equal(h.cpu().numpy(), h_r, f"h rep {rep}")
        assert_bits_equal(y.cpu().numpy(), out_r, f"shared down rep {rep}")
