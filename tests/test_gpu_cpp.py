"""A C++ program built against include/hymoe.hpp and linked with libhymoe.so (tests/cpp/moe_step, built by
tests/cpp/Makefile) runs one decode step -- moe_decode on a workspace and moe_decode_noalloc -- and one prefill step
through the reference-signature calls, on experts it uploads itself from GGUF-layout bytes, and calls the host quantizer
hymoe::q8k_test_quantize on std::vector data.  Its outputs must equal the CPU oracle's bit for bit."""
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd.formats import GType
from tests.helpers import assert_bits_equal, gen, layer, oracle_layer

pytestmark = pytest.mark.gpu
EXE = Path(__file__).resolve().parent / "cpp" / "moe_step"


@pytest.mark.parametrize("tg,td,E,d,ff,k,ntd,ntp", [
    (GType.Q4_K, GType.Q4_K, 32, 2048, 768, 8, 1, 96),
    (GType.Q4_K, GType.Q6_K, 24, 1024, 512, 4, 3, 40),
])
def test_cpp_caller_matches_oracle(cuda, tmp_path, tg, td, E, d, ff, k, ntd, ntp):
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built (make -C tests/cpp)")
    L = layer(tg, td, E, ff, d, seed=5100 + E)
    g = gen(5101 + E)
    W = (torch.randn(E, d, generator=g) * 0.02).numpy()
    xd = torch.randn(ntd, d, generator=g).numpy()
    xp = torch.randn(ntp, d, generator=g).numpy()
    gate, up, down = (t.cpu().numpy() for t in (L.gate, L.up, L.down))
    hdr = np.array([E, d, ff, k, ntd, ntp, int(tg), int(td)], np.int32).tobytes() + np.array([L.gate_bytes, L.down_bytes], np.uint64).tobytes()
    inp, out = tmp_path / "in.bin", tmp_path / "out.bin"
    inp.write_bytes(hdr + gate.tobytes() + up.tobytes() + down.tobytes() + W.astype(np.float32).tobytes()
                    + xd.astype(np.float32).tobytes() + xp.astype(np.float32).tobytes())
    r = subprocess.run([str(EXE), str(inp), str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    raw = out.read_bytes()
    f32 = np.frombuffer(raw[: 4 * d * (2 * ntd + ntp)], np.float32)
    dec, dec_na, pre = f32[: ntd * d].reshape(ntd, d), f32[ntd * d: 2 * ntd * d].reshape(ntd, d), f32[2 * ntd * d:].reshape(ntp, d)
    o_ids = 4 * d * (2 * ntd + ntp)
    ids_pre = np.frombuffer(raw[o_ids: o_ids + 4 * ntp * k], np.int32).reshape(ntp, k)
    xq_host = np.frombuffer(raw[o_ids + 4 * ntp * k:], np.uint8).reshape(ntp * d // 256, 292)
    assert_bits_equal(xq_host, orc.quantize(GType.Q8_K, xp).reshape(-1, 292), "q8k_test_quantize")
    OL = oracle_layer(L)
    for x, got, what in ((xd, dec, "moe_decode"), (xd, dec_na, "moe_decode_noalloc"), (xp, pre, "prefill")):
        ids, wts, _ = orc.route(orc.gemv_f32(W, x), E, k)
        if what == "prefill":
            assert_bits_equal(ids_pre, ids, "prefill ids")
        assert_bits_equal(got, orc.moe_layer(OL, x, ids, wts), what)
