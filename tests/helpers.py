"""Shared test utilities: seeded inputs, the oracle's view of a layer, exact comparisons."""
import numpy as np
import torch

import oracle as orc
from hyper_amd.formats import GType, activations, random_layer, zipf_logit_bias

TYPES_256 = [GType.Q4_K, GType.Q5_K, GType.Q6_K, GType.IQ4_XS, GType.IQ2_XS, GType.IQ2_XXS, GType.Q2_K, GType.Q3_K, GType.IQ3_XXS, GType.IQ3_S, GType.IQ2_S, GType.IQ1_S]
ALL_TYPES = TYPES_256 + [GType.IQ4_NL, GType.Q8_0, GType.MXFP4, GType.Q5_0, GType.Q5_1]
D_RANGE = {GType.Q4_K: (1e-4, 4e-3), GType.Q5_K: (1e-4, 4e-3), GType.Q6_K: (1e-4, 4e-3),
           GType.IQ4_XS: (1e-3, 1e-2), GType.IQ2_XS: (1e-3, 1e-2), GType.IQ2_XXS: (1e-3, 1e-2), GType.IQ4_NL: (1e-3, 1e-2),
           GType.Q8_0: (1e-4, 1e-3), GType.MXFP4: (1e-2, 1e-1),
           GType.Q5_0: (1e-3, 1e-2), GType.Q2_K: (1e-3, 1e-2), GType.Q3_K: (1e-4, 1e-3), GType.IQ3_XXS: (1e-3, 1e-2), GType.IQ3_S: (1e-3, 1e-2), GType.IQ2_S: (1e-3, 1e-2), GType.IQ1_S: (1e-2, 1e-1), GType.Q5_1: (1e-3, 1e-2)}   # MXFP4: power-of-two scales, codebook values up to 12


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def x_distributions(n: int, seed: int) -> dict:
    """The activation distributions of the reference's quantizer test (tools/cpumoebench.cu:53-86): normal,
    heavy-tailed x^3 * 30, values on a 1/8 grid (exact ties), sparse large outliers; plus all-zero and
    negative-maximum blocks, and a block whose largest |x| occurs twice with opposite signs."""
    rng = np.random.default_rng(seed)
    z = rng.standard_normal(n).astype(np.float32)
    d = {
        "normal": z,
        "heavy": (z ** 3 * 30).astype(np.float32),
        "ties": (np.round(z * 8) / 8).astype(np.float32),
        "sparse": np.where(rng.random(n) < 0.01, z * 1000, z * 0.01).astype(np.float32),
    }
    zero = z.copy()
    zero[:256] = 0
    d["zero_block"] = zero
    neg = z.copy()
    neg[37] = -50.0
    neg[300] = 50.0     # equal magnitude in the next 256-value block
    d["neg_max"] = neg
    tie = z.copy()
    tie[20] = -60.0
    tie[66] = 60.0      # equal magnitude later in the same 256-value block: the first occurrence (negative) wins
    d["lane_tie"] = tie
    return d


def layer(tg, td, E, ff, n, seed, clamp=0.0):
    return random_layer(tg, td, E, ff, n, seed, d_range=D_RANGE[GType(tg)], d_range_down=D_RANGE[GType(td)], clamp=clamp)


def oracle_layer(L) -> "orc.Layer":
    return orc.Layer.from_expert_layer(L)


def routing(T, E, k, seed, zipf=None):
    """ids/wts [T, k] from the oracle's router on seeded logits (Zipf-biased when zipf is set)."""
    g = gen(seed)
    logits = torch.randn(T, E, generator=g) * 0.5
    if zipf:
        logits = logits + zipf_logit_bias(T, E, zipf, g)
    ids, wts, _ = orc.route(logits.numpy(), E, k)
    return ids, wts


def assert_bits_equal(a, b, what=""):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    if a.dtype.kind == "f":
        ok = (a == b) | (np.isnan(a) & np.isnan(b))
    else:
        ok = a == b
    if not ok.all():
        idx = np.argwhere(~ok)
        i = tuple(idx[0])
        raise AssertionError(f"{what}: {int((~ok).sum())} of {a.size} differ; first at {i}: {a[i]!r} vs {b[i]!r}")


def rel_l2(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_logits_close(got, W, x, bias=None, what="logits"):
    """Router logits from the matrix cores against the oracle's fmaf chain (orc.gemv_f32): any two fp32 evaluations of
    a d-term dot product lie within 2 d u sum|w x| of each other (u = 2^-24, the worst-case bound of recursive fp32
    summation, twice), plus half an ulp of the bias add.  A mistake in the operand layout (a transposed or shifted
    tile) is off by O(sum|w x|) and fails it."""
    W = np.asarray(W, np.float32)
    x = np.asarray(x, np.float32)
    ref = orc.gemv_f32(W, x).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(W.astype(np.float64)).T
    bound = 2 * W.shape[1] * 2.0 ** -24 * mag
    if bias is not None:
        b = np.asarray(bias, np.float32)
        ref = ref + b
        bound = bound + np.abs(ref) * 2.0 ** -23
    err = np.abs(np.asarray(got, np.float64) - ref)
    bad = ~(err <= bound)
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside the fp32 bound; first at {i}: {got[i]!r} vs {ref[i]!r} "
                             f"(bound {bound[i]:.3g})")


def router_on_matrix_cores(rows: int, kdim: int, nt: int) -> bool:
    """Whether hy_moe_router_q8 computes these logits on the matrix cores (their own sum order) rather than the fmaf
    chain of gemv_f32: more than 8 tokens and enough full 64 x 64 tiles for every CU -- the library's dispatch
    (router_pre_any, hy_route.hip)."""
    return nt > 8 and kdim % 64 == 0 and (rows // 64) * ((nt + 63) // 64) >= 256
