"""Seeded inputs of the golden fixtures (outputs live in oracle_fixtures.npz)."""
import hashlib

import numpy as np
import torch

from hyper_amd.formats import GType, block_elems, random_blocks, random_layer, vec_dot_type

CASES = {
    "q8k_heavy": {"kind": "quant", "vt": GType.Q8_K, "seed": 1},
    "q8_0_heavy": {"kind": "quant", "vt": GType.Q8_0, "seed": 2},
    **{f"blocks_{t.name}": {"kind": "blocks", "t": t, "n": 1024, "seed": 10 + int(t)}
       for t in (GType.Q4_K, GType.Q5_K, GType.Q6_K, GType.IQ4_XS, GType.IQ2_XS, GType.IQ4_NL,
                 GType.Q8_0, GType.IQ2_XXS, GType.MXFP4, GType.Q5_0, GType.Q5_1, GType.Q2_K, GType.Q3_K, GType.IQ3_XXS,
                 GType.IQ3_S, GType.IQ2_S, GType.IQ1_S)},
    "route_288_8": {"kind": "route", "E": 288, "k": 8, "seed": 3},
    "layer_q4k_q6k": {"kind": "layer", "tg": GType.Q4_K, "td": GType.Q6_K, "E": 3, "ff": 256, "d": 512, "k": 2, "nt": 2, "seed": 4},
    "layer_iq4nl": {"kind": "layer", "tg": GType.IQ4_NL, "td": GType.IQ4_NL, "E": 3, "ff": 256, "d": 512, "k": 2, "nt": 2, "seed": 5},
    "layer_iq3s_q3k": {"kind": "layer", "tg": GType.IQ3_S, "td": GType.Q3_K, "E": 3, "ff": 256, "d": 512, "k": 2, "nt": 2, "seed": 6},
    "layer_mxfp4_q5_1": {"kind": "layer", "tg": GType.MXFP4, "td": GType.Q5_1, "E": 3, "ff": 256, "d": 512, "k": 2, "nt": 2, "seed": 7},
}


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def inputs(name: str) -> dict:
    c = CASES[name]
    g = _gen(c["seed"])
    if c["kind"] == "quant":
        z = torch.randn(2, 512, generator=g)
        return {"x": (z ** 3 * 30).numpy().astype(np.float32)}
    if c["kind"] == "blocks":
        import oracle as orc
        t, n = c["t"], c["n"]
        nb = n // block_elems(t)
        w = random_blocks(t, 3 * nb, g, "cpu", (1e-3, 1e-2)).numpy().reshape(3, -1)
        x = torch.randn(n, generator=g).numpy().astype(np.float32)
        vt = vec_dot_type(t)
        return {"w": w, "x": x, "xq": orc.quantize(vt, x)}
    if c["kind"] == "route":
        return {"logits": (torch.randn(5, c["E"] + 1, generator=g) * 2).numpy().astype(np.float32)}
    if c["kind"] == "layer":
        L = random_layer(c["tg"], c["td"], c["E"], c["ff"], c["d"], seed=c["seed"], d_range=(1e-3, 1e-2))
        x = torch.randn(c["nt"], c["d"], generator=g).numpy().astype(np.float32)
        ids = np.stack([np.random.default_rng(c["seed"] + t).permutation(c["E"])[:c["k"]] for t in range(c["nt"])]).astype(np.int32)
        wts = np.full((c["nt"], c["k"]), 1.0 / c["k"], np.float32)
        return {"layer": dict(tg=c["tg"], td=c["td"], gate=L.gate.numpy(), up=L.up.numpy(), down=L.down.numpy(), ff=c["ff"], n=c["d"]),
                "x": x, "ids": ids, "wts": wts}
    raise ValueError(name)


def digest(inp: dict) -> str:
    h = hashlib.sha256()
    def add(v):
        if isinstance(v, dict):
            for k in sorted(v):
                add(v[k])
        elif isinstance(v, np.ndarray):
            h.update(np.ascontiguousarray(v).tobytes())
        else:
            h.update(repr(v).encode())
    add(inp)
    return h.hexdigest()
