"""The library's host Q8_K quantizer (hy_q8k_quantize_host, the C++ face's hymoe::q8k_test_quantize -- the
reference's src/cpu_moe.h:46, host buffers in and out) against the oracle's quantizer, bit for bit, over the
distributions of the reference's own quantizer test (tools/cpumoebench.cu:53-86) and the known-answer blocks.
No GPU: the entry point makes no HIP call."""
import ctypes

import numpy as np
import pytest

import hyper_amd
import oracle as orc
from hyper_amd import lib
from hyper_amd.formats import GType
from tests.helpers import x_distributions


def host_q8k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.full(x.size // 256 * 292, 0xA5, np.uint8)   # poison: every byte must be written
    rc = lib().hy_q8k_quantize_host(ctypes.c_void_p(x.ctypes.data), ctypes.c_void_p(y.ctypes.data), x.size)
    assert rc == hyper_amd.HY_OK, lib().hy_last_error()
    return y.reshape(-1, 292)


@pytest.mark.parametrize("name", ["normal", "heavy", "ties", "sparse", "zero_block", "neg_max", "lane_tie"])
@pytest.mark.parametrize("seed", [3, 11, 29])
def test_host_q8k_matches_oracle(name, seed):
    x = x_distributions(4096, seed=seed)[name]
    assert (host_q8k(x) == orc.quantize(GType.Q8_K, x).reshape(-1, 292)).all()


def test_host_q8k_known_answers():
    x = np.zeros(512, np.float32)
    x[:8] = [2.5, 3.5, -0.5, -127.0, 1.5, -2.5, 0.49999997, 126.5]   # iscale = 1: q = round-half-even(x)
    x[256 + 10], x[256 + 20] = 5.0, -5.0                             # first of two equal magnitudes is positive
    q = host_q8k(x)
    d0 = q[0, :4].view(np.float32)[0]
    qs0 = q[0, 4:260].view(np.int8)
    assert d0 == np.float32(1.0)
    assert list(qs0[:8]) == [2, 4, 0, -127, 2, -2, 0, 126]
    assert q[0, 260:].view(np.int16)[0] == 2 + 4 + 0 - 127 + 2 - 2 + 0 + 126
    qs1 = q[1, 4:260].view(np.int8)
    assert qs1[10] == -127 and qs1[20] == 127
    assert q[1, :4].view(np.float32)[0] == np.float32(1.0) / np.float32(np.float32(-127.0) / np.float32(5.0))


def test_host_q8k_zero_block_and_shapes():
    L = lib()
    q = host_q8k(np.zeros(256, np.float32))
    assert (q == 0).all(), "an all-zero block: d = 0, q = 0, zero sums"
    x = np.ones(300, np.float32)
    y = np.zeros(292 * 2, np.uint8)
    assert L.hy_q8k_quantize_host(ctypes.c_void_p(x.ctypes.data), ctypes.c_void_p(y.ctypes.data), 300) == hyper_amd.HY_EBAD_SHAPE
    assert L.hy_q8k_quantize_host(None, ctypes.c_void_p(y.ctypes.data), 256) == hyper_amd.HY_EINVAL
    assert L.hy_q8k_quantize_host(ctypes.c_void_p(x.ctypes.data), ctypes.c_void_p(y.ctypes.data), 0) == hyper_amd.HY_OK
