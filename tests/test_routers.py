"""The oracle's alternative routers (src/kernels5.cu:1090-1122 sigmoid + selection bias, src/kernels7.cu:816-865
sqrt-softplus + selection bias) and their scalar functions, pinned without retyping them: or_logf / or_log1pf /
the two scores against fp64 numpy within 2-2.5 ulp over their ranges plus special values; the selections against an fp64
brute force on keys spaced far beyond rounding; the tie rule, the bias-only-selects rule, the weight formulas' sums
and the 2^-14 floor."""
import numpy as np
import pytest

import oracle as orc


def ulp_err(got, ref):
    got = np.asarray(got, np.float64)
    ref64 = np.asarray(ref, np.float64)
    sp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(got - ref64) / sp


def _vec(fn, xs):
    return np.array([fn(float(x)) for x in xs], np.float32)


def test_logf_within_2_ulp_and_special_values():
    rng = np.random.default_rng(1)
    xs = np.concatenate([np.exp(rng.uniform(np.log(1e-44), np.log(3e38), 40000)), rng.uniform(0.5, 2.0, 20000),
                         np.array([1.0, 2.0, 0.5, np.sqrt(0.5), 1.17549435e-38, 1.4e-45])]).astype(np.float32)
    got = _vec(orc.lib().or_logf, xs)
    assert ulp_err(got, np.log(xs.astype(np.float64))).max() <= 2.0
    L = orc.lib().or_logf
    assert L(1.0) == 0.0 and L(0.0) == -np.inf and L(np.inf) == np.inf
    assert np.isnan(L(-1.0)) and np.isnan(L(float("nan")))


def test_log1pf_within_2_ulp():
    rng = np.random.default_rng(2)
    xs = np.concatenate([np.exp(rng.uniform(np.log(1e-30), np.log(5e8), 40000)), -np.exp(rng.uniform(np.log(1e-30), np.log(0.99), 20000)),
                         np.array([0.0, 1e-38, 1.0, -0.5])]).astype(np.float32)
    got = _vec(orc.lib().or_log1pf, xs)
    assert ulp_err(got, np.log1p(xs.astype(np.float64))).max() <= 2.5   # log's error plus about one ulp of the correction
    assert orc.lib().or_log1pf(-1.0) == -np.inf


def test_router_scores_within_2_ulp():
    rng = np.random.default_rng(3)
    ls = np.concatenate([rng.uniform(-86, 30, 40000), np.array([20.0, 20.000002, 19.999998, 0.0, -86.0])]).astype(np.float32)
    l64 = ls.astype(np.float64)
    sig = _vec(orc.lib().or_sigmoid, ls)
    assert ulp_err(sig, 1.0 / (1.0 + np.exp(-l64))).max() <= 2.5   # expf's error carried through 1 / (1 + e)
    sp = _vec(orc.lib().or_sqrt_softplus, ls)
    ref = np.sqrt(np.where(l64 > 20.0, l64, np.log1p(np.exp(l64))))
    assert ulp_err(sp, ref).max() <= 2.5
    big = ls[ls > 20.0]   # above 20 the score is sqrt(l) itself, correctly rounded
    assert np.array_equal(_vec(orc.lib().or_sqrt_softplus, big), np.sqrt(big))


def _spaced(nt, E, rng, lo=-4.0, hi=4.0):
    """logits and bias whose keys (score + bias) are far apart: distinct multiples of 1e-2 on a shuffled grid"""
    logits = np.stack([rng.permutation(np.linspace(lo, hi, E)) for _ in range(nt)]).astype(np.float32)
    bias = (rng.permutation(E) * 1e-1 / E).astype(np.float32)
    return logits, bias


@pytest.mark.parametrize("mode", ["sig", "sqrtsp"])
@pytest.mark.parametrize("E,k", [(16, 4), (288, 8), (384, 6), (1024, 16)])
def test_selection_matches_fp64_brute_force(mode, E, k):
    rng = np.random.default_rng(E + k)
    nt, scale = 5, 2.5
    logits, bias = _spaced(nt, E, rng)
    l64 = logits.astype(np.float64)
    score = 1.0 / (1.0 + np.exp(-l64)) if mode == "sig" else np.sqrt(np.log1p(np.exp(l64)))
    key = score + bias
    want = np.argsort(-key, axis=1, kind="stable")[:, :k]
    if mode == "sig":
        ids, wts, sg = orc.route_sig(logits, bias, E, k, scale)
        assert np.all(sg == 1.0)
    else:
        ids, wts = orc.route_sqrtsp(logits, bias, E, k, scale)
    assert np.array_equal(ids, want)
    sel = np.take_along_axis(score, want, axis=1)
    # the weights follow the scores alone (not the bias) and sum to scale
    np.testing.assert_allclose(wts, sel / sel.sum(1, keepdims=True) * scale, rtol=2e-6)


@pytest.mark.parametrize("mode", ["sig", "sqrtsp"])
def test_ties_go_to_the_lower_index(mode):
    E, k = 40, 8
    logits = np.full((2, E), 0.25, np.float32)
    bias = np.zeros(E, np.float32)
    ids = orc.route_sig(logits, bias, E, k, 1.0)[0] if mode == "sig" else orc.route_sqrtsp(logits, bias, E, k, 1.0)[0]
    assert np.array_equal(ids, np.tile(np.arange(k), (2, 1)))
    bias[[3, 30]] = 1.0    # equal keys again among the two boosted experts: 3 before 30, then 0, 1, ...
    ids = orc.route_sig(logits, bias, E, k, 1.0)[0] if mode == "sig" else orc.route_sqrtsp(logits, bias, E, k, 1.0)[0]
    assert list(ids[0]) == [3, 30, 0, 1, 2, 4, 5, 6]


def test_bias_selects_but_does_not_weigh():
    E, k = 64, 4
    rng = np.random.default_rng(7)
    logits = rng.uniform(-1, 1, (1, E)).astype(np.float32)
    lowest = int(np.argmin(logits[0]))
    bias = np.zeros(E, np.float32)
    bias[lowest] = 100.0
    for mode in ("sig", "sqrtsp"):
        if mode == "sig":
            ids, wts, _ = orc.route_sig(logits, bias, E, k, 1.0)
            s = 1.0 / (1.0 + np.exp(-logits[0].astype(np.float64)))
        else:
            ids, wts = orc.route_sqrtsp(logits, bias, E, k, 1.0)
            s = np.sqrt(np.log1p(np.exp(logits[0].astype(np.float64))))
        assert ids[0, 0] == lowest
        np.testing.assert_allclose(wts[0, 0], s[lowest] / s[ids[0]].sum(), rtol=2e-6)


def test_sigmoid_weight_floor():
    """Tiny selected probabilities: the sum is floored at 2^-14, so the weights are p scale 2^14 and sum below scale."""
    E, k = 32, 4
    logits = np.full((1, E), -40.0, np.float32)
    logits[0, :k] = -30.0
    ids, wts, _ = orc.route_sig(logits, np.zeros(E, np.float32), E, k, 1.0)
    assert list(ids[0]) == list(range(k))
    p = np.float32(orc.lib().or_sigmoid(-30.0))
    assert np.all(wts[0] == np.float32(p * np.float32(1.0 / 6.103515625e-5)))


def test_c_abi_rejects_bad_router_arguments():
    """The entry points check their limits before any launch (no GPU needed): k 1..16, n_expert 1..1024, a stride
    of at least n_expert, non-null buffers."""
    import ctypes
    from hyper_amd import HY_EBAD_SHAPE, HY_EINVAL, lib
    L = lib()
    buf = (ctypes.c_float * 4)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    for fn, extra in ((L.hy_moe_route_sig, (p,)), (L.hy_moe_route_sqrtsp, ())):
        def call(ls, ne, k, bias=p):
            return fn(p, ls, bias, ne, k, 1.0, p, p, *extra, 1, None)
        assert call(64, 64, 17) == HY_EBAD_SHAPE
        assert call(2000, 1025, 8) == HY_EBAD_SHAPE
        assert call(32, 64, 8) == HY_EBAD_SHAPE
        assert call(64, 64, 8, bias=None) == HY_EINVAL
