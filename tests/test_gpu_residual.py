"""The combine written into the residual (hy_moe_reduce_residual, hy_moe_down_reduce_residual): for decode and
prefill, with a shared expert and its sigmoid gate, the residual afterwards equals residual + the oracle's layer
output, one fp32 addition, bit for bit; and the plain entry points are unchanged beside them."""
import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import moe
from hyper_amd.formats import GType, activations, random_layer

from .helpers import assert_bits_equal, oracle_layer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tg,td", [(GType.Q4_K, GType.Q6_K), (GType.IQ4_NL, GType.IQ4_NL)])
def test_combine_into_residual(cuda, tg, td):
    print(f"residual combine {tg.name}/{td.name}", flush=True)
    E, d, ff, k = 32, 1024, 512, 4
    L = random_layer(tg, td, E, ff, d, seed=81)
    S = random_layer(tg, td, 1, ff, d, seed=82)
    rng = np.random.default_rng(83)
    W_r = (rng.standard_normal((E + 1, d)) * 0.05).astype(np.float32)   # row E: the shared-expert gate logit
    dev = moe.MoeDev(L.to(cuda), torch.arange(E, dtype=torch.int32, device=cuda))
    sdev = moe.MoeDev(S.to(cuda), torch.zeros(1, dtype=torch.int32, device=cuda))
    r = moe.MoeLayerRunner(dev, torch.from_numpy(W_r).to(cuda), k, max_rows=80, shared=sdev, sg_logit=True)
    for nt, fn in ((1, r.decode), (5, r.decode), (80, r.prefill)):
        g = torch.Generator(device=cuda)
        g.manual_seed(84 + nt)
        x = activations(nt, d, g, cuda)
        resid0 = torch.randn(nt, d, generator=g, device=cuda)
        plain = fn(x).clone()
        resid = resid0.clone()
        got = fn(x, resid=resid)
        torch.cuda.synchronize()
        assert got.data_ptr() == resid.data_ptr()
        logits = orc.gemv_f32(W_r, x.cpu().numpy())
        ids, wts, sg = orc.route(logits, E, k, with_sg=True)
        ref = orc.moe_layer(oracle_layer(L), x.cpu().numpy(), ids, wts, shared=oracle_layer(S), sg=sg)
        assert_bits_equal(plain.cpu().numpy(), ref, f"plain out nt={nt}")
        want = (resid0.cpu().numpy() + ref).astype(np.float32)
        assert_bits_equal(resid.cpu().numpy(), want, f"residual nt={nt}")
