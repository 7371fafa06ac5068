"""MoeLayerRunner refuses inputs its workspace cannot hold before any kernel runs (CPU tensors, no GPU needed)."""
import pytest
import torch

from hyper_amd import moe
from hyper_amd.formats import GType, random_layer


@pytest.fixture(scope="module")
def runner():
    L = random_layer(GType.Q4_K, GType.Q4_K, 4, 256, 256, seed=3)
    dev = moe.MoeDev(L, torch.arange(4, dtype=torch.int32))
    return moe.MoeLayerRunner(dev, torch.zeros(4, 256), k=2, max_rows=2)


def test_rows_beyond_max_rows_raise(runner):
    with pytest.raises(ValueError, match="max_rows"):
        runner.decode(torch.zeros(3, 256))
    with pytest.raises(ValueError, match="max_rows"):
        runner.prefill(torch.zeros(3, 256))
    with pytest.raises(ValueError, match="max_rows"):
        runner.decode_legacy(torch.zeros(3, 256))


def test_bad_activation_layouts_raise(runner):
    with pytest.raises(ValueError, match="float32"):
        runner.decode(torch.zeros(1, 256, dtype=torch.float16))
    with pytest.raises(ValueError, match=r"\[nt, 256\]"):
        runner.decode(torch.zeros(1, 512))
    with pytest.raises(ValueError, match="contiguous"):
        runner.prefill(torch.zeros(256, 2).t())
    with pytest.raises(ValueError, match="resid"):
        runner.decode(torch.zeros(1, 256), resid=torch.zeros(1, 128))
    with pytest.raises(ValueError, match="bias"):
        runner.decode(torch.zeros(1, 256), bias=torch.zeros(1, 2))
