"""Committed golden fixtures (tests/golden/oracle_fixtures.npz, written by tests/golden/make_fixtures.py).

CPU: the seeded inputs still hash to what was recorded and the oracle still produces the recorded outputs, so a
change to the oracle (or to the generators) cannot silently move the reference every GPU test compares with.
GPU: the kernels reproduce the recorded outputs without the oracle running at all.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd.formats import q8_row_bytes, vec_dot_type
from tests.golden.fixture_inputs import CASES, digest, inputs
from tests.helpers import assert_bits_equal

FIX = np.load(Path(__file__).parent / "golden" / "oracle_fixtures.npz")


def _fix(name, key):
    return FIX[f"{name}/{key}"]


@pytest.mark.parametrize("name", list(CASES))
def test_inputs_unchanged(name):
    assert digest(inputs(name)) == bytes(_fix(name, "sha")).hex(), f"{name}: seeded inputs changed"


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_reproduces_fixtures(name):
    c, inp = CASES[name], inputs(name)
    if c["kind"] == "quant":
        assert_bits_equal(orc.quantize(c["vt"], inp["x"]), _fix(name, "q"), name)
    elif c["kind"] == "blocks":
        t, n, w = c["t"], c["n"], inp["w"]
        assert_bits_equal(orc.dequant_row(t, w.reshape(-1), n * w.shape[0]), _fix(name, "deq"), name)
        for r in range(w.shape[0]):
            si, sm = orc.block_ints(t, w[r], inp["xq"], n)
            assert_bits_equal(si, _fix(name, "sumi")[r], f"{name} sumi {r}")
            assert_bits_equal(sm, _fix(name, "summ")[r], f"{name} summ {r}")
            assert orc.row_dot(t, w[r], inp["xq"], n) == _fix(name, "dot")[r]
    elif c["kind"] == "route":
        ids, wts, sg = orc.route(inp["logits"], c["E"], c["k"], with_sg=True)
        assert_bits_equal(ids, _fix(name, "ids"))
        assert_bits_equal(wts, _fix(name, "wts"))
        assert_bits_equal(sg, _fix(name, "sg"))
    else:
        L = orc.Layer(**inp["layer"])
        o, h, _ = orc.moe_layer(L, inp["x"], inp["ids"], inp["wts"], want_hy=True)
        assert_bits_equal(o, _fix(name, "out"))
        assert_bits_equal(h, _fix(name, "h"))


# ------------------------------------------------------------------ kernels against the stored outputs

@pytest.mark.gpu
@pytest.mark.parametrize("name", [n for n, c in CASES.items() if c["kind"] in ("quant", "route", "blocks")])
def test_gpu_matches_fixture(cuda, name):
    from hyper_amd import moe
    c, inp = CASES[name], inputs(name)
    if c["kind"] == "quant":
        x = torch.from_numpy(inp["x"]).to(cuda)
        nt, n = x.shape
        q = torch.zeros(nt * q8_row_bytes(c["vt"], n), dtype=torch.uint8, device=cuda)
        moe.q8_quantize(c["vt"], x, n, n, nt, q)
        torch.cuda.synchronize()
        assert_bits_equal(q.cpu().numpy().reshape(_fix(name, "q").shape), _fix(name, "q"), name)
    elif c["kind"] == "route":
        lg = torch.from_numpy(inp["logits"]).to(cuda)
        nt, ls = lg.shape
        ids = torch.zeros(nt * c["k"], dtype=torch.int32, device=cuda)
        wts = torch.zeros(nt * c["k"], dtype=torch.float32, device=cuda)
        sg = torch.zeros(nt, dtype=torch.float32, device=cuda)
        moe.moe_route(lg, ls, c["E"], c["k"], ids, wts, sg, nt)
        torch.cuda.synchronize()
        assert_bits_equal(ids.cpu().numpy().reshape(nt, -1), _fix(name, "ids"))
        assert_bits_equal(wts.cpu().numpy().reshape(nt, -1), _fix(name, "wts"))
        assert_bits_equal(sg.cpu().numpy(), _fix(name, "sg"))
    else:
        t, n, w = c["t"], c["n"], inp["w"]
        rows = w.shape[0]
        out = torch.zeros(rows * n, dtype=torch.float32, device=cuda)
        moe.dequant_row(t, torch.from_numpy(w.reshape(-1)).to(cuda), rows * n, out)
        sumi = torch.zeros(_fix(name, "sumi").shape, dtype=torch.int32, device=cuda)
        summ = torch.zeros(_fix(name, "summ").shape, dtype=torch.int32, device=cuda)
        moe.block_ints(t, torch.from_numpy(w).to(cuda), w.shape[1], rows, torch.from_numpy(inp["xq"]).to(cuda), n, sumi, summ)
        torch.cuda.synchronize()
        assert_bits_equal(out.cpu().numpy(), _fix(name, "deq"), f"{name} dequant")
        assert_bits_equal(sumi.cpu().numpy(), _fix(name, "sumi"), f"{name} sumi")
        assert_bits_equal(summ.cpu().numpy(), _fix(name, "summ"), f"{name} summ")


@pytest.mark.gpu
@pytest.mark.parametrize("name", [n for n, c in CASES.items() if c["kind"] == "layer"])
@pytest.mark.parametrize("path", ["decode", "grouped"])
def test_gpu_layer_matches_fixture(cuda, name, path):
    from hyper_amd import moe
    from hyper_amd.formats import ExpertLayer
    c, inp = CASES[name], inputs(name)
    Ld = inp["layer"]
    L = ExpertLayer(tg=Ld["tg"], td=Ld["td"], E=c["E"], gate=torch.from_numpy(Ld["gate"]), up=torch.from_numpy(Ld["up"]),
                    down=torch.from_numpy(Ld["down"]), ff=Ld["ff"], n=Ld["n"])
    dev = moe.upload_experts(L, device=cuda)
    nt, k, d, ff, E = c["nt"], c["k"], c["d"], c["ff"], c["E"]
    P = nt * k
    x = torch.from_numpy(inp["x"]).to(cuda)
    ids = torch.from_numpy(inp["ids"]).reshape(-1).to(cuda)
    wts = torch.from_numpy(inp["wts"]).reshape(-1).to(cuda)
    h = torch.full((P, ff), float("nan"), device=cuda)
    out = torch.zeros(nt, d, device=cuda)
    if path == "decode":
        moe.moe_gate_up(dev, x, d, ids, k, h, nt)
        moe.moe_down_reduce(dev, h, ids, wts, k, None, None, out, nt)
    else:
        order = torch.zeros(P, dtype=torch.int32, device=cuda)
        order_n = torch.zeros(2, dtype=torch.int32, device=cuda)
        egrp = torch.zeros(3 * E, dtype=torch.int32, device=cuda)
        moe.moe_order(dev, ids, P, E, order, order_n, egrp=egrp)
        vg, vd = vec_dot_type(c["tg"]), vec_dot_type(c["td"])
        xq = torch.zeros(nt * q8_row_bytes(vg, d), dtype=torch.uint8, device=cuda)
        moe.q8_quantize(vg, x, d, d, nt, xq)
        moe.moe_gemm_gate_up(dev, xq, k, P, order, order_n, egrp, E, h)
        hq = torch.zeros(P * q8_row_bytes(vd, ff), dtype=torch.uint8, device=cuda)
        moe.q8_quantize(vd, h, ff, ff, P, hq)
        y = torch.full((P, d), float("nan"), device=cuda)
        moe.moe_gemm_down(dev, hq, P, order, order_n, egrp, E, wts, y)
        moe.moe_reduce(None, None, y, k, out, d, nt, ids)
    torch.cuda.synchronize()
    assert_bits_equal(h.cpu().numpy(), _fix(name, "h"), f"{name} {path} h")
    assert_bits_equal(out.cpu().numpy(), _fix(name, "out"), f"{name} {path} out")
