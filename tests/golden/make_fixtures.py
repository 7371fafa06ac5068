"""Write tests/golden/oracle_fixtures.npz: expected outputs of the CPU oracle on seeded inputs.

Inputs are regenerated from their seeds by tests/golden/fixture_inputs.py (a SHA-256 of every input is stored
and checked, so a change of generator is caught); only outputs are stored.  The CPU suite checks that the
oracle still produces them, the GPU suite checks the kernels against them.

    python tests/golden/make_fixtures.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle as orc  # noqa: E402
from tests.golden.fixture_inputs import CASES, digest, inputs  # noqa: E402


def main():
    out = {}
    for name in CASES:
        inp = inputs(name)
        out[f"{name}/sha"] = np.frombuffer(bytes.fromhex(digest(inp)), np.uint8)
        kind = CASES[name]["kind"]
        if kind == "quant":
            out[f"{name}/q"] = orc.quantize(CASES[name]["vt"], inp["x"])
        elif kind == "blocks":
            t, n = CASES[name]["t"], CASES[name]["n"]
            out[f"{name}/deq"] = orc.dequant_row(t, inp["w"].reshape(-1), n * inp["w"].shape[0])
            si, sm = zip(*(orc.block_ints(t, inp["w"][r], inp["xq"], n) for r in range(inp["w"].shape[0])))
            out[f"{name}/sumi"], out[f"{name}/summ"] = np.stack(si), np.stack(sm)
            out[f"{name}/dot"] = np.float32([orc.row_dot(t, inp["w"][r], inp["xq"], n) for r in range(inp["w"].shape[0])])
        elif kind == "route":
            ids, wts, sg = orc.route(inp["logits"], CASES[name]["E"], CASES[name]["k"], with_sg=True)
            out[f"{name}/ids"], out[f"{name}/wts"], out[f"{name}/sg"] = ids, wts, sg
        elif kind == "layer":
            L = orc.Layer(**inp["layer"])
            o, h, y = orc.moe_layer(L, inp["x"], inp["ids"], inp["wts"], want_hy=True)
            out[f"{name}/out"], out[f"{name}/h"] = o, h
    np.savez_compressed(Path(__file__).with_name("oracle_fixtures.npz"), **out)
    print(f"{len(out)} arrays")


if __name__ == "__main__":
    main()
