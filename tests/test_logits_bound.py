"""The fp32 bound the matrix-core router's logits are held to (tests/helpers.py assert_logits_close): it admits any
summation order of the same products (numpy's blocked matmul, a reversed fp32 chain, the exact value rounded once)
and rejects a mistake in the operand layout (a token's logits shifted by one expert, a transposed 16 x 16 tile)."""
import numpy as np
import pytest

import oracle as orc
from tests.helpers import assert_logits_close


def _case(seed, rows=48, d=512, nt=9):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, d)) * 0.02).astype(np.float32), rng.standard_normal((nt, d)).astype(np.float32)


def test_other_summation_orders_pass():
    W, x = _case(1)
    assert_logits_close(orc.gemv_f32(W, x), W, x)
    assert_logits_close((x @ W.T).astype(np.float32), W, x)
    rev = np.zeros((x.shape[0], W.shape[0]), np.float32)
    for k in reversed(range(W.shape[1])):
        rev = (rev + x[:, k:k + 1] * W[:, k]).astype(np.float32)
    assert_logits_close(rev, W, x)
    assert_logits_close((x.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32), W, x)
    b = np.random.default_rng(2).standard_normal((x.shape[0], W.shape[0])).astype(np.float32)
    assert_logits_close(((x @ W.T) + b).astype(np.float32), W, x, b)


def test_layout_mistakes_fail():
    W, x = _case(3, rows=32, nt=16)
    good = orc.gemv_f32(W, x)
    with pytest.raises(AssertionError):
        assert_logits_close(np.roll(good, 1, axis=1), W, x)
    t = good.copy()
    t[:16, :16] = t[:16, :16].T.copy()
    with pytest.raises(AssertionError):
        assert_logits_close(t, W, x)
