"""Every configured workload at its real shapes (expert count, d_model, ff, k, rows, types, shared expert, Zipf routing
and log-normal token norms) through MoeLayerRunner on the GPU: decode / verify rows through the three-launch decode,
longer batches through the prefill path.  The layers are generated on the device at full size; the oracle checks a
sample of the tokens on a sub-layer holding only the experts they route to (ids remapped in ascending order, so the
combine order is unchanged).  Logits are checked against the oracle's fmaf chain (bit for bit on the fmaf-chain
routers; within the fp32 summation bound where the 2048-token chunk's router runs on the matrix cores); routing and
outputs are then compared bit for bit to the oracle's given the GPU's logits; the 2e-3 relative-L2 bound on fp32
expert outputs is asserted as well."""
import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import moe
from hyper_amd.formats import WORKLOADS, activations, random_layer, zipf_logit_bias
from tests.helpers import assert_bits_equal, assert_logits_close, rel_l2, router_on_matrix_cores

pytestmark = pytest.mark.gpu
SAMPLE = 24   # tokens checked against the oracle in batches longer than that


def _sub_layer(L, used):
    """oracle layer of the experts `used` (ascending) of the device layer L"""
    idx = torch.as_tensor(used, dtype=torch.long, device=L.gate.device)
    return orc.Layer(L.tg, L.td, L.gate[idx].cpu().numpy(), L.up[idx].cpu().numpy(), L.down[idx].cpu().numpy(), L.ff, L.n, L.clamp)


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_workload_full_size(cuda, name):
    w = WORKLOADS[name]
    seed = 900 + sum(map(ord, name))
    L = random_layer(w.tg, w.td, w.E, w.ff, w.d, seed=seed, device=cuda, d_range=w.d_range, d_range_down=w.d_range_down)
    S = random_layer(w.shared[0], w.shared[1], 1, w.ff, w.d, seed=seed + 1, device=cuda, d_range=w.d_range) if w.shared else None
    g = torch.Generator(device=cuda)
    g.manual_seed(seed + 2)
    W_r = torch.randn(w.E, w.d, generator=g, device=cuda) * 0.02
    x = activations(w.rows, w.d, g, cuda, lognormal=w.norm_lognormal)
    bias = zipf_logit_bias(w.rows, w.E, w.zipf, g, cuda) if w.zipf and not w.chunk else None
    dev = moe.MoeDev(L, torch.arange(w.E, dtype=torch.int32, device=cuda))
    sdev = moe.MoeDev(S, torch.zeros(1, dtype=torch.int32, device=cuda)) if S is not None else None
    if w.chunk:
        _prompt_in_chunks(w, L, S, W_r, x, g, dev, sdev, seed)
        return
    r = moe.MoeLayerRunner(dev, W_r, w.k, max_rows=w.rows, shared=sdev)
    out = (r.decode(x, bias=bias) if w.rows <= 8 else r.prefill(x, bias=bias)).clone()
    torch.cuda.synchronize()

    rng = np.random.default_rng(seed)
    tok = np.arange(w.rows) if w.rows <= SAMPLE else np.sort(rng.choice(w.rows, SAMPLE, replace=False))
    xs = x.cpu().numpy()[tok]
    logits = r.logits.cpu().numpy()[tok, :w.E]
    assert_logits_close(logits, W_r.cpu().numpy(), xs, bias.cpu().numpy()[tok] if bias is not None else None)
    if not router_on_matrix_cores(w.E, w.d, w.rows):   # the fmaf-chain routers: the oracle's bits
        ref_l = orc.gemv_f32(W_r.cpu().numpy(), xs)
        assert_bits_equal(logits, (ref_l + bias.cpu().numpy()[tok]).astype(np.float32) if bias is not None else ref_l, "logits")
    ids, wts, _ = orc.route(logits, w.E, w.k)   # routing given the GPU's logits
    assert_bits_equal(r.ids.cpu().numpy().reshape(-1, w.k)[tok], ids, "ids")
    assert_bits_equal(r.wts.cpu().numpy().reshape(-1, w.k)[tok], wts, "wts")
    used = np.unique(ids)
    ids_sub = np.searchsorted(used, ids).astype(np.int32)
    ref = orc.moe_layer(_sub_layer(L, used), xs, ids_sub, wts, shared=orc.Layer.from_expert_layer(S) if S is not None else None)
    got = out.cpu().numpy()[tok]
    assert_bits_equal(got, ref, "out")
    assert rel_l2(got, ref) <= 2e-3


def _prompt_in_chunks(w, L, S, W_r, x, g, dev, sdev, seed):
    """A long prompt through one runner of chunk rows: each chunk draws its own routing skew and adds its output into
    its rows of a random residual.  Checked: every chunk's logits and routing on its sampled tokens, and the residual
    rows of all sampled tokens (the oracle's layer output plus one fp32 add to the residual they started from)."""
    C, nch = w.chunk, w.rows // w.chunk
    r = moe.MoeLayerRunner(dev, W_r, w.k, max_rows=C, shared=sdev)
    resid = torch.randn(w.rows, w.d, generator=g, device=x.device)
    resid0 = resid.cpu().numpy()
    rng = np.random.default_rng(seed)
    tok = np.sort(rng.choice(w.rows, SAMPLE, replace=False))
    Wh, xs_all = W_r.cpu().numpy(), x.cpu().numpy()
    ids_all, wts_all = np.zeros((w.rows, w.k), np.int32), np.zeros((w.rows, w.k), np.float32)
    for j in range(nch):
        b = zipf_logit_bias(C, w.E, w.zipf, g, x.device)
        r.prefill(x[j * C:(j + 1) * C], bias=b, resid=resid[j * C:(j + 1) * C])
        torch.cuda.synchronize()
        t = tok[(tok >= j * C) & (tok < (j + 1) * C)] - j * C
        if t.size == 0:
            continue
        logits = r.logits.cpu().numpy()[t, :w.E]
        assert_logits_close(logits, Wh, xs_all[j * C + t], b.cpu().numpy()[t], f"chunk {j} logits")
        ids, wts, _ = orc.route(logits, w.E, w.k)   # routing given the GPU's logits
        assert_bits_equal(r.ids.cpu().numpy().reshape(-1, w.k)[t], ids, f"chunk {j} ids")
        assert_bits_equal(r.wts.cpu().numpy().reshape(-1, w.k)[t], wts, f"chunk {j} wts")
        ids_all[j * C + t], wts_all[j * C + t] = ids, wts
    ids, wts = ids_all[tok], wts_all[tok]
    used = np.unique(ids)
    ids_sub = np.searchsorted(used, ids).astype(np.int32)
    ref = orc.moe_layer(_sub_layer(L, used), xs_all[tok], ids_sub, wts, shared=orc.Layer.from_expert_layer(S) if S is not None else None)
    got = resid.cpu().numpy()[tok]
    assert_bits_equal(got, (resid0[tok] + ref).astype(np.float32), "residual rows")
    assert rel_l2(got - resid0[tok], ref) <= 2e-3
