"""The alternative routers on the GPU (hy_moe_route_sig: sigmoid + selection bias, src/kernels5.cu:1090-1122;
hy_moe_route_sqrtsp: sqrt-softplus + selection bias, src/kernels7.cu:816-865), bit for bit against the oracle: every
expert count shape the path meets (16 .. 1024 experts), k up to 16, logits across both branches of softplus and
far into the sigmoid's tails, ties, and the 2^-14 floor of the sigmoid router's weight sum."""
import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import moe

from .helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


def _run(mode, logits, bias, E, k, scale, cuda):
    nt, ls = logits.shape
    lg, bs = torch.from_numpy(logits).to(cuda), torch.from_numpy(bias).to(cuda)
    ids = torch.full((nt * k,), -1, dtype=torch.int32, device=cuda)
    wts = torch.full((nt * k,), float("nan"), device=cuda)
    if mode == "sig":
        sg = torch.zeros(nt, device=cuda)
        moe.moe_route_sig(lg, ls, bs, E, k, scale, ids, wts, sg, nt)
        torch.cuda.synchronize()
        assert torch.all(sg == 1.0)
        ref_ids, ref_wts, _ = orc.route_sig(logits, bias, E, k, scale)
    else:
        moe.moe_route_sqrtsp(lg, ls, bs, E, k, scale, ids, wts, nt)
        torch.cuda.synchronize()
        ref_ids, ref_wts = orc.route_sqrtsp(logits, bias, E, k, scale)
    assert_bits_equal(ids.cpu().numpy().reshape(nt, k), ref_ids, f"{mode} ids")
    assert_bits_equal(wts.cpu().numpy().reshape(nt, k), ref_wts, f"{mode} wts")


@pytest.mark.parametrize("mode", ["sig", "sqrtsp"])
@pytest.mark.parametrize("E,k", [(16, 4), (128, 8), (288, 8), (384, 6), (513, 16), (1024, 16)])
def test_router_bits(cuda, mode, E, k):
    print(f"router {mode} E {E} k {k}", flush=True)
    rng = np.random.default_rng(E * 31 + k)
    nt = 96
    logits = (rng.standard_normal((nt, E + 3)) * 2.0).astype(np.float32)   # a stride wider than E
    logits[:8] = rng.uniform(-95.0, 45.0, (8, E + 3)).astype(np.float32)    # tails: exp underflow, softplus above 20
    logits[8:12] = 0.5                                                       # ties: every key equal
    bias = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    _run(mode, logits, bias, E, k, 2.5, cuda)
    _run(mode, logits, np.zeros(E, np.float32), E, k, 1.0, cuda)


def test_sigmoid_weight_floor_bits(cuda):
    E, k = 64, 8
    logits = np.full((4, E), -40.0, np.float32)
    logits[:, :k] = -30.0
    _run("sig", logits, np.zeros(E, np.float32), E, k, 1.0, cuda)


@pytest.mark.parametrize("router", ["sigmoid", "sqrt_softplus"])
def test_layer_with_router(cuda, router):
    """MoeLayerRunner with the router: decode (1 and 4 rows) and prefill (96 rows) equal the oracle layer on the
    oracle router's ids and weights, bit for bit."""
    from hyper_amd.formats import GType, activations, random_layer
    from .helpers import oracle_layer
    print(f"layer with router {router}", flush=True)
    E, d, ff, k, scale = 64, 1024, 512, 6, 2.5
    L = random_layer(GType.Q4_K, GType.Q6_K, E, ff, d, seed=61)
    rng = np.random.default_rng(62)
    W_r = (rng.standard_normal((E, d)) * 0.05).astype(np.float32)
    rb = rng.uniform(-0.05, 0.05, E).astype(np.float32)
    dev = moe.MoeDev(L.to(cuda), torch.arange(E, dtype=torch.int32, device=cuda))
    r = moe.MoeLayerRunner(dev, torch.from_numpy(W_r).to(cuda), k, max_rows=96, router=router,
                           router_bias=torch.from_numpy(rb).to(cuda), router_scale=scale)
    for nt, fn in ((1, r.decode), (4, r.decode), (96, r.prefill)):
        g = torch.Generator(device=cuda)
        g.manual_seed(63 + nt)
        x = activations(nt, d, g, cuda)
        out = fn(x).clone()
        torch.cuda.synchronize()
        logits = orc.gemv_f32(W_r, x.cpu().numpy())
        if router == "sigmoid":
            ids, wts, _ = orc.route_sig(logits, rb, E, k, scale)
        else:
            ids, wts = orc.route_sqrtsp(logits, rb, E, k, scale)
        assert_bits_equal(r.ids.cpu().numpy()[: nt * k].reshape(nt, k), ids, f"ids nt={nt}")
        ref = orc.moe_layer(oracle_layer(L), x.cpu().numpy(), ids, wts)
        assert_bits_equal(out.cpu().numpy(), ref, f"out nt={nt}")
