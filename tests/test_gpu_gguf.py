"""GGUF expert loading end to end on the GPU: a layer written to a GGUF file, read back through libhymoe's reader
(hy_gguf_*), placed on the device both ways -- the Python upload (moe.MoeDev over gguf.expert_layer) and the C ABI's
hy_gguf_expert_tensors + hy_upload_experts -- then run through MoeLayerRunner (decode and prefill) and the
separate decode entries: every output is bit-identical to the CPU oracle on the bytes that were written."""
import ctypes
import types

import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd import check, hy_moe_dev, lib, moe
from hyper_amd.formats import GType, activations, random_layer, vec_dot_type
from hyper_amd.gguf import GGUF, expert_layer

from .gguf_writer import STR, U32, write_gguf
from .helpers import assert_bits_equal, oracle_layer, rel_l2

pytestmark = pytest.mark.gpu

E, D, FF, K = 16, 1024, 512, 4


def _write(path, L):
    kv = [("general.architecture", STR, "qwen3moe"), ("general.alignment", U32, 32), ("qwen3moe.expert_count", U32, E)]
    ts = [("blk.3.ffn_gate_exps.weight", int(L.tg), [D, FF, E], L.gate.numpy().tobytes()),
          ("blk.3.ffn_up_exps.weight", int(L.tg), [D, FF, E], L.up.numpy().tobytes()),
          ("blk.3.ffn_down_exps.weight", int(L.td), [FF, D, E], L.down.numpy().tobytes())]
    write_gguf(path, kv, ts)


def _reference(L, W_r, x):
    logits = orc.gemv_f32(W_r, x)
    ids, wts, _ = orc.route(logits, E, K)
    return logits, ids, wts, orc.moe_layer(oracle_layer(L), x, ids, wts)


@pytest.mark.parametrize("tg,td", [(GType.Q4_K, GType.Q6_K), (GType.IQ4_XS, GType.IQ4_XS), (GType.IQ1_S, GType.Q2_K),
                                   (GType.MXFP4, GType.Q5_1), (GType.IQ3_S, GType.Q3_K)])
def test_gguf_layer_runs_bit_exact(cuda, tmp_path, tg, td):
    print(f"gguf layer {tg.name}/{td.name}: E {E} d {D} ff {FF}", flush=True)
    L = random_layer(tg, td, E, FF, D, seed=31 + int(tg))
    path = tmp_path / "layer.gguf"
    _write(path, L)
    rng = np.random.default_rng(32)
    W_r = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)
    with GGUF(path) as g:
        assert g.get_int("qwen3moe.expert_count") == E
        X = expert_layer(g, 3)
        dev = moe.MoeDev(X.to(cuda), torch.arange(E, dtype=torch.int32, device=cuda))
        r = moe.MoeLayerRunner(dev, torch.from_numpy(W_r).to(cuda), K, max_rows=64)
        for nt, fn in ((1, r.decode), (64, r.prefill)):
            gx = torch.Generator(device=cuda)
            gx.manual_seed(33 + nt)
            x = activations(nt, D, gx, cuda)
            out = fn(x).clone()
            torch.cuda.synchronize()
            logits, ids, wts, ref = _reference(L, W_r, x.cpu().numpy())
            assert_bits_equal(r.ids.cpu().numpy().reshape(-1, K)[:nt], ids, f"ids nt={nt}")
            assert_bits_equal(out.cpu().numpy(), ref, f"out nt={nt}")
            assert rel_l2(out.cpu().numpy(), ref) <= 2e-3

        # the C ABI's path: hy_gguf_expert_tensors -> hy_upload_experts (host-side tiling), experts 0..E-1 at slots
        # E-1..0, then the two decode launches
        t = g.expert_tensors(3, E)
        slot = torch.tensor([E - 1 - e for e in range(E)], dtype=torch.int32)
        c = hy_moe_dev()
        check(lib().hy_upload_experts(ctypes.byref(t), ctypes.c_void_p(slot.data_ptr()), FF, D, 0.0, ctypes.byref(c)))
        try:
            cd = types.SimpleNamespace(c=c, ref=ctypes.byref(c))
            nt = 2
            x = torch.from_numpy(rng.standard_normal((nt, D)).astype(np.float32))
            logits, ids, wts, ref = _reference(L, W_r, x.numpy())
            xq = torch.from_numpy(orc.quantize(vec_dot_type(tg), x.numpy())).reshape(-1).to(cuda)
            ids_d = torch.zeros(nt * K, dtype=torch.int32, device=cuda)
            wts_d = torch.zeros(nt * K, device=cuda)
            h = torch.zeros(nt * K, FF, device=cuda)
            out = torch.full((nt, D), float("nan"), device=cuda)
            moe.moe_route_gate_up(cd, torch.from_numpy(logits).to(cuda), E, E, K, xq, ids_d, wts_d, None, h, nt)
            moe.moe_down_reduce(cd, h, ids_d, wts_d, K, None, None, out, nt)
            torch.cuda.synchronize()
            assert_bits_equal(out.cpu().numpy(), ref, "C ABI upload: out")
        finally:
            moe.free_experts(c)
