"""GPU: the decode hand-over of the hidden as Q8_0 rows for layers whose gate/up and down both take Q8_0 activations
(IQ4_NL, Q8_0, MXFP4).  hy_moe_route_gate_up_q8 writes h and the
Q8_0 rows of h; hy_moe_down_reduce_q8 reads those rows in place of quantizing h in every block.  Checked bit for bit
against the oracle: h, the rows (the oracle's Q8_0 quantizer on h, src/kernels4.cu:2007-2022 quantizes h the same way
before the down dot), and out, plain and added into a residual; with experts that are not local (their rows stay
unwritten and drop out of the sum) and two calls in a row, the second with fewer rows.  Other types refuse."""
import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import HyError, moe
from hyper_amd.formats import GType, q8_row_bytes

from .helpers import assert_bits_equal, gen, layer, oracle_layer, rel_l2

pytestmark = pytest.mark.gpu
TOL = 2e-3   # final fp32 outputs within 2e-3 relative L2 of the CPU path (bit-identity implies it)

CASES = [
    # E, d, ff, k, nt, non-local experts
    (24, 4096, 1536, 8, 1, ()),
    (24, 4096, 1536, 8, 4, ()),
    (16, 2048, 512, 8, 3, (1, 4, 9)),
    (32, 1024, 256, 4, 8, (0, 31)),
]


@pytest.mark.parametrize("E,d,ff,k,nt,absent", CASES)
def test_hidden_q8_handover_bitexact(cuda, E, d, ff, k, nt, absent):
    print(f"hidden q8 E={E} d={d} ff={ff} k={k} nt={nt} absent={absent}", flush=True)
    tg = {3: GType.Q8_0, 4: GType.MXFP4}.get(nt, GType.IQ4_NL)
    td = {3: GType.IQ4_NL, 4: GType.MXFP4, 8: GType.Q8_0}.get(nt, GType.IQ4_NL)
    L = layer(tg, td, E, ff, d, seed=740 + nt)   # IQ4_NL both ways, a Q8_0 gate/up (3 rows), MXFP4 both ways (4 rows), a Q8_0 down (8 rows)
    slot = [(-1 if e in absent else e) for e in range(E)]
    dev = moe.upload_experts(L, slot=slot, device=cuda)
    OL = oracle_layer(L)
    row_q = q8_row_bytes(GType.Q8_0, ff)
    for rep, rows in enumerate((nt, max(1, nt - 2))):
        lg = (torch.randn(rows, E, generator=gen(741 + rep)) * 1.5).numpy().astype(np.float32)
        lg[0, list(absent)] += np.float32(4.0)   # row 0 picks the non-local experts
        ids_r, wts_r, _ = orc.route(lg, E, k)
        local = np.array([slot[e] >= 0 for e in ids_r.reshape(-1)]).reshape(ids_r.shape)
        if absent:
            assert not local.all(), "the case must route some pairs to non-local experts"
        ids_cpu = np.where(local, ids_r, -1).astype(np.int32)
        x = torch.randn(rows, d, generator=gen(742 + rep))
        out_r, h_r, _ = orc.moe_layer(OL, x.numpy(), ids_cpu, wts_r, want_hy=True)
        # the oracle's Q8_0 blocks of h, in the hand-over's layout: per token, the k rows' block values, then scales
        nbh = ff // 32
        raw = orc.quantize(GType.Q8_0, h_r).reshape(rows, k, nbh, 34)
        hq_r = np.concatenate([raw[..., 2:].reshape(rows, -1), raw[..., :2].reshape(rows, -1)], axis=1).reshape(-1)
        xq = torch.from_numpy(orc.quantize(GType.Q8_0, x.numpy())).reshape(-1).to(cuda)
        ids = torch.full((rows * k,), -5, dtype=torch.int32, device=cuda)
        wts = torch.zeros(rows * k, device=cuda)
        h = torch.full((rows * k, ff), float("nan"), device=cuda)
        hq = torch.full((rows * k * row_q,), 0xAB, dtype=torch.uint8, device=cuda)
        out = torch.full((rows, d), float("nan"), device=cuda)
        resid0 = torch.randn(rows, d, generator=gen(743 + rep))
        resid = resid0.to(cuda)
        moe.moe_route_gate_up_q8(dev, torch.from_numpy(lg).to(cuda), E, E, k, xq, ids, wts, None, h, hq, rows)
        moe.moe_down_reduce_q8(dev, hq, ids, wts, k, None, None, out, False, rows)
        moe.moe_down_reduce_q8(dev, hq, ids, wts, k, None, None, resid, True, rows)
        torch.cuda.synchronize()
        lv = local.reshape(-1)
        assert_bits_equal(ids.cpu().numpy().reshape(rows, k), ids_r, f"ids rep {rep}")
        assert_bits_equal(wts.cpu().numpy().reshape(rows, k), wts_r, f"wts rep {rep}")
        hv, hqv = h.cpu().numpy(), hq.cpu().numpy()
        assert_bits_equal(hv[lv], h_r[lv], f"h of local pairs rep {rep}")
        assert np.isnan(hv[~lv]).all(), "non-local pairs leave h unwritten"
        # byte masks of each pair's values and scales in the layout
        pair = np.arange(rows * k).reshape(rows, k)
        sel = np.zeros((rows * k, rows * k * nbh * 34), dtype=bool)
        for t_ in range(rows):
            base = t_ * k * nbh * 34
            for j_ in range(k):
                sel[pair[t_, j_], base + j_ * nbh * 32: base + (j_ + 1) * nbh * 32] = True
                sel[pair[t_, j_], base + k * nbh * 32 + j_ * nbh * 2: base + k * nbh * 32 + (j_ + 1) * nbh * 2] = True
        mine = sel[lv].any(axis=0)
        assert_bits_equal(hqv[mine], hq_r[mine], f"Q8_0 blocks of h rep {rep}")
        assert (hqv[sel[~lv].any(axis=0)] == 0xAB).all(), "non-local pairs leave their Q8_0 blocks unwritten"
        assert_bits_equal(out.cpu().numpy(), out_r, f"out rep {rep}")
        assert_bits_equal(resid.cpu().numpy(), (resid0.numpy() + out_r).astype(np.float32), f"resid + out rep {rep}")
        assert rel_l2(out.cpu().numpy(), out_r) <= TOL


def test_hidden_q8_refuses_other_types(cuda):
    E, d, ff, k, nt = 8, 2048, 512, 4, 1
    cases = [(GType.Q4_K, GType.Q6_K, d), (GType.IQ4_NL, GType.IQ4_NL, 8192)]   # K-quant down; n beyond 4096
    for tg, td, n in cases:
        L = layer(tg, td, E, ff, n, seed=750)
        dev = moe.upload_experts(L, device=cuda)
        lg = torch.zeros(nt, E, device=cuda)
        xq = torch.zeros(4 * nt * n, dtype=torch.uint8, device=cuda)
        ids = torch.zeros(nt * k, dtype=torch.int32, device=cuda)
        wts = torch.zeros(nt * k, device=cuda)
        h = torch.zeros(nt * k, ff, device=cuda)
        hq = torch.zeros(nt * k * q8_row_bytes(GType.Q8_0, ff), dtype=torch.uint8, device=cuda)
        out = torch.zeros(nt, n, device=cuda)
        with pytest.raises(HyError, match="route_gate_up_q8"):
            moe.moe_route_gate_up_q8(dev, lg, E, E, k, xq, ids, wts, None, h, hq, nt)
        if td != GType.IQ4_NL:
            with pytest.raises(HyError, match="down_reduce_q8"):
                moe.moe_down_reduce_q8(dev, hq, ids, wts, k, None, None, out, False, nt)
    torch.cuda.synchronize()
