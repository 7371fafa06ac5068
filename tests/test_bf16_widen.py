"""The bf16 router weights' widening (the bf16 entries and their tests shift the 16-bit pattern into the high half of
an fp32) against torch's own bfloat16 -> float32 conversion, on all 65,536 patterns (NaN payloads included)."""
import numpy as np
import torch


def test_bf16_widening_matches_torch():
    u16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = u16.astype(np.uint32) << 16
    theirs = torch.from_numpy(u16.view(np.int16)).view(torch.bfloat16).float().numpy().view(np.uint32)
    assert np.array_equal(ours, theirs)
