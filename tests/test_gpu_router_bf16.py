"""bf16 router weights (gemv_bf16w, src/kernels4.cu:181-197, :1914-1917; bf16_to_f32, :198-201, :1918-1920): bf16 bit
patterns widened on load give the same products and sums as the fp32 router on the widened matrix, so every launch
shape's logits must equal the fp32 entry's -- and the oracle's gemv on the widened weights -- bit for bit."""
import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import moe
from hyper_amd.formats import GType, q8_row_bytes, vec_dot_type
from tests.helpers import assert_bits_equal, assert_logits_close, gen, layer, oracle_layer, router_on_matrix_cores

pytestmark = pytest.mark.gpu


def _bf16_weights(rows, kdim, seed):
    """router weights rounded to bf16, and their exact fp32 values"""
    W16 = (torch.randn(rows, kdim, generator=gen(seed)) * 0.02).to(torch.bfloat16)
    return W16, W16.float()


# nt 1 / 3 / 4: a wave per row; 5 / 37: 4 x 8 register tiles; kdim 1000: the tail of a 256-value step
@pytest.mark.parametrize("rows,kdim,nt", [(128, 2048, 1), (129, 2048, 3), (288, 4096, 4), (513, 2048, 5), (128, 1000, 37)])
def test_gemv_bf16w_bitexact(cuda, rows, kdim, nt):
    W16, W32 = _bf16_weights(rows, kdim, 141 + nt)
    g = gen(142)
    x = torch.randn(nt, kdim, generator=g)
    bias = torch.randn(nt, rows, generator=g)
    ref = orc.gemv_f32(W32.numpy(), x.numpy())
    y16 = torch.zeros(nt, rows, device=cuda)
    y32 = torch.zeros(nt, rows, device=cuda)
    yb = torch.zeros(nt, rows, device=cuda)
    xd = x.to(cuda)
    moe.gemv_bf16w(W16.to(cuda), rows, kdim, xd, kdim, y16, rows, nt)
    moe.gemv_f32(W32.to(cuda), rows, kdim, xd, kdim, y32, rows, nt)
    moe.gemv_f32(W16.to(cuda), rows, kdim, xd, kdim, yb, rows, nt, bias=bias.to(cuda), bias_stride=rows)   # dispatches on dtype
    torch.cuda.synchronize()
    assert_bits_equal(y16.cpu().numpy(), ref, "bf16 logits vs oracle on the widened weights")
    assert_bits_equal(y16.cpu().numpy(), y32.cpu().numpy(), "bf16 vs fp32 entry")
    assert_bits_equal(yb.cpu().numpy(), (ref + bias.numpy()).astype(np.float32), "bf16 logits + bias")


# nt <= 8: the decode router (a wave per row); 9 and 40 tokens: the batched router's 8-token LDS tiles; 256 tokens x
# 513 rows, 512 x 129 and 2048 x 16: the register-row kernel (a partial row group too); 512 x 288 at kdim 4096: 16-token
# LDS tiles; 2048 x 577: 64 x 64 matrix-core tiles and a row past them; kdim 992 (not a multiple of 256): the register
# tiles
@pytest.mark.parametrize("rows,kdim,nt,vt", [(129, 2048, 1, GType.Q8_K), (288, 4096, 8, GType.Q8_0), (513, 2048, 9, GType.Q8_K),
                                              (128, 2048, 40, GType.Q8_K), (513, 1024, 256, GType.Q8_0), (129, 2048, 512, GType.Q8_K),
                                              (288, 4096, 512, GType.Q8_0), (128, 992, 20, GType.Q8_0),
                                              (577, 2048, 2048, GType.Q8_K), (16, 2048, 2048, GType.Q8_K)])
def test_router_q8_bf16w_bitexact(cuda, rows, kdim, nt, vt):
    W16, W32 = _bf16_weights(rows, kdim, 151 + nt)
    g = gen(152)
    x = torch.randn(nt, kdim, generator=g)
    bias = torch.randn(nt, rows, generator=g)
    ref = (orc.gemv_f32(W32.numpy(), x.numpy()) + bias.numpy()).astype(np.float32)
    xd, bd = x.to(cuda), bias.to(cuda)
    outs = []
    for W in (W16, W32):
        lg = torch.zeros(nt, rows, device=cuda)
        xq = torch.zeros(nt * q8_row_bytes(vt, kdim), dtype=torch.uint8, device=cuda)
        moe.moe_router_q8(W.to(cuda), rows, kdim, xd, kdim, lg, rows, vt, xq, nt, bias=bd, bias_stride=rows)
        outs.append((lg, xq))
    torch.cuda.synchronize()
    if router_on_matrix_cores(rows, kdim, nt):   # the matrix cores' sum order: within the fp32 bound of the oracle
        assert_logits_close(outs[0][0].cpu().numpy(), W32.numpy(), x.numpy(), bias.numpy(), "bf16 router logits vs oracle")
    else:
        assert_bits_equal(outs[0][0].cpu().numpy(), ref, "bf16 router logits vs oracle")
    assert_bits_equal(outs[0][0].cpu().numpy(), outs[1][0].cpu().numpy(), "bf16 vs fp32 router logits")
    assert_bits_equal(outs[0][1].cpu().numpy(), orc.quantize(vt, x.numpy()).reshape(-1), "Q8 rows of x")


@pytest.mark.parametrize("n", [1, 4, 1027, 1 << 20])
def test_bf16_to_f32_exact(cuda, n):
    bits = torch.randint(0, 1 << 16, (n,), generator=gen(160 + n % 97), dtype=torch.int32).to(torch.int16)
    out = torch.full((n,), float("nan"), device=cuda)
    moe.bf16_to_f32(bits.to(cuda), n, out)
    torch.cuda.synchronize()
    want = bits.numpy().view(np.uint16).astype(np.uint32) << 16
    assert_bits_equal(out.cpu().numpy().view(np.uint32), want, "widened bits")


@pytest.mark.parametrize("nt", [1, 4, 40])
def test_runner_bf16_router_matches_fp32(cuda, nt):
    """MoeLayerRunner with a bf16 W_r (the router16 path) against the same runner on the widened fp32 matrix: decode
    (up to 8 rows) and prefill outputs identical."""
    tg = td = GType.Q4_K
    E, d, ff, k = 16, 2048, 512, 4
    L = layer(tg, td, E, ff, d, seed=171)
    dev = moe.upload_experts(L, device=cuda)
    W16, W32 = _bf16_weights(E, d, 172)
    x = torch.randn(nt, d, generator=gen(173)).to(cuda)
    outs = []
    for W in (W16, W32):
        r = moe.MoeLayerRunner(dev, W.to(cuda), k, max_rows=nt)
        o1 = (r.decode(x) if nt <= 8 else r.prefill(x)).clone()
        o2 = r.prefill(x).clone()
        outs.append((o1, o2))
    torch.cuda.synchronize()
    assert_bits_equal(outs[0][0].cpu().numpy(), outs[1][0].cpu().numpy(), "decode / first path")
    assert_bits_equal(outs[0][1].cpu().numpy(), outs[1][1].cpu().numpy(), "prefill")
    logits = orc.gemv_f32(W32.numpy(), x.cpu().numpy())
    ids, wts, _ = orc.route(logits, E, k)
    ref = orc.moe_layer(oracle_layer(L), x.cpu().numpy(), ids, wts)
    assert_bits_equal(outs[0][1].cpu().numpy(), ref, "prefill vs oracle")
