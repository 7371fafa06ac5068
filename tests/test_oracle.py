"""CPU tests that pin the oracle (oracle/moe_oracle.c) without a GPU.

The reference ships no golden vectors for this path and its CPU dot products come from ggml, which is not
vendored; the oracle is pinned instead by
  - the reference's codebooks (digests in tests/golden/reference_tables.json, made from the reference sources),
  - known-answer blocks built by hand from the layouts of the reference's deq8<T> (src/kernels4.cu:421-714),
  - a second, independent numpy decoder of every format (tests/np_formats.py),
  - brute-force integer dot products and an fp64 recomputation of the whole layer,
  - the reference's quantizer-test distributions (tools/cpumoebench.cu:53-86) against numpy restatements of
    ggml's scalar quantize_row_q8_K and x86 quantize_row_q8_0,
  - closed forms and properties for exp, routing and bucketing.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as orc
from hyper_amd.formats import GType, block_bytes, block_elems, random_blocks, row_bytes, vec_dot_type
from tests import np_formats as nf
from tests.helpers import D_RANGE, gen, layer, oracle_layer, routing, x_distributions

GOLDEN = Path(__file__).resolve().parent / "golden"
TABLES = json.loads((GOLDEN / "reference_tables.json").read_text())


# ------------------------------------------------------------------ codebooks

def iq2xs_rows() -> np.ndarray:
    """The IQ2_XS codebook as the kernels and the oracle expand it from iq2xs_grid.inc."""
    text = (Path(__file__).resolve().parents[1] / "hyper_amd/csrc/iq2xs_grid.inc").read_text()
    body = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))
    codes = [int(v) for v in body.replace(",", " ").split() if v.isdigit()]
    assert len(codes) == 512
    lv = np.array([8, 25, 43], np.uint8)
    rows = np.zeros((512, 8), np.uint8)
    for i, c in enumerate(codes):
        for j in range(8):
            rows[i, j] = lv[c % 3]
            c //= 3
    return rows


def iq2xxs_rows() -> np.ndarray:
    """The IQ2_XXS codebook as the kernels and the oracle expand it from iq2xxs_grid.inc."""
    text = (Path(__file__).resolve().parents[1] / "hyper_amd/csrc/iq2xxs_grid.inc").read_text()
    body = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))
    codes = [int(v) for v in body.replace(",", " ").split() if v.isdigit()]
    assert len(codes) == 256
    lv = np.array([8, 25, 43], np.uint8)
    rows = np.zeros((256, 8), np.uint8)
    for i, c in enumerate(codes):
        for j in range(8):
            rows[i, j] = lv[c % 3]
            c //= 3
    return rows


def iq3xxs_rows() -> np.ndarray:
    """The IQ3_XXS codebook as the kernels and the oracle expand it from iq3xxs_grid.inc (base-8 digits: byte i's
    level 4 + 8 d, 62 for d = 7)."""
    text = (Path(__file__).resolve().parents[1] / "hyper_amd/csrc/iq3xxs_grid.inc").read_text()
    body = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))
    codes = [int(v) for v in body.replace(",", " ").split() if v.isdigit()]
    assert len(codes) == 256
    lv = np.array([4, 12, 20, 28, 36, 44, 52, 62], np.uint8)
    rows = np.zeros((256, 4), np.uint8)
    for i, c in enumerate(codes):
        for j in range(4):
            rows[i, j] = lv[c % 8]
            c //= 8
    return rows


def iq3s_rows() -> np.ndarray:
    """The IQ3_S codebook as the kernels and the oracle expand it from iq3s_grid.inc (base-8 digits: 2 d + 1)."""
    text = (Path(__file__).resolve().parents[1] / "hyper_amd/csrc/iq3s_grid.inc").read_text()
    body = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))
    codes = [int(v) for v in body.replace(",", " ").split() if v.isdigit()]
    assert len(codes) == 512
    rows = np.zeros((512, 4), np.uint8)
    for i, c in enumerate(codes):
        for j in range(4):
            rows[i, j] = 2 * (c % 8) + 1
            c //= 8
    return rows


def iq2s_rows() -> np.ndarray:
    """The IQ2_S codebook as the kernels and the oracle expand it from iq2s_grid.inc (base-3 as IQ2_XS's)."""
    text = (Path(__file__).resolve().parents[1] / "hyper_amd/csrc/iq2s_grid.inc").read_text()
    body = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))
    codes = [int(v) for v in body.replace(",", " ").split() if v.isdigit()]
    assert len(codes) == 1024
    lv = np.array([8, 25, 43], np.uint8)
    rows = np.zeros((1024, 8), np.uint8)
    for i, c in enumerate(codes):
        for j in range(8):
            rows[i, j] = lv[c % 3]
            c //= 3
    return rows


def iq1s_rows() -> np.ndarray:
    """The IQ1_S codebook as the kernels and the oracle expand it from iq1s_grid.inc (base-3, digit = value + 1)."""
    text = (Path(__file__).resolve().parents[1] / "hyper_amd/csrc/iq1s_grid.inc").read_text()
    body = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))
    codes = [int(v) for v in body.replace(",", " ").split() if v.isdigit()]
    assert len(codes) == 2048
    rows = np.zeros((2048, 8), np.int8)
    for i, c in enumerate(codes):
        for j in range(8):
            rows[i, j] = c % 3 - 1
            c //= 3
    return rows


def grid_for(t):
    t = GType(t)
    return {GType.IQ2_XXS: iq2xxs_rows, GType.IQ3_XXS: iq3xxs_rows, GType.IQ3_S: iq3s_rows,
            GType.IQ2_S: iq2s_rows, GType.IQ1_S: iq1s_rows}.get(t, iq2xs_rows)()


def ksigns() -> np.ndarray:
    return np.array([i | ((bin(i).count("1") & 1) << 7) for i in range(128)], np.uint8)


def test_codebooks_match_reference():
    rows = iq2xs_rows()
    assert hashlib.sha256(rows.tobytes()).hexdigest() == TABLES["iq2xs_grid_sha256"]
    assert hashlib.sha256(iq2xxs_rows().tobytes()).hexdigest() == TABLES["iq2xxs_grid_sha256"]
    assert hashlib.sha256(iq3xxs_rows().tobytes()).hexdigest() == TABLES["iq3xxs_grid_sha256"]
    assert hashlib.sha256(iq3s_rows().tobytes()).hexdigest() == TABLES["iq3s_grid_sha256"]
    assert hashlib.sha256(iq2s_rows().tobytes()).hexdigest() == TABLES["iq2s_grid_sha256"]
    assert hashlib.sha256(iq1s_rows().tobytes()).hexdigest() == TABLES["iq1s_grid_sha256"]
    assert hashlib.sha256(ksigns().tobytes()).hexdigest() == TABLES["ksigns_sha256"]
    assert hashlib.sha256(nf.KV_IQ4NL.astype(np.int8).tobytes()).hexdigest() == TABLES["iq4nl_sha256"]
    assert all(bin(int(s)).count("1") % 2 == 0 for s in ksigns())   # every sign byte has an even bit count


# ------------------------------------------------------------------ scalar helpers

def test_expf_accuracy_and_special_values():
    x = np.concatenate([np.linspace(-87.0, 88.7, 200001, dtype=np.float32),
                        np.float32([0.0, -0.0, 1e-30, -1e-30, 0.5, -0.5, 1.0, 10.0, -10.0])])
    got = np.array([orc.expf(v) for v in x[::7]], np.float64)
    ref = np.exp(x[::7].astype(np.float64))
    ulp = np.abs(got - ref) / np.spacing(np.float32(ref).astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 2.0, f"max {ulp.max()} ulp"
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-87.5) == 0.0 and orc.expf(-1e30) == 0.0             # below exp(-87): flushed, no subnormals
    assert np.isinf(orc.expf(88.8)) and np.isnan(orc.expf(float("nan")))
    assert orc.expf(-87.0) >= np.finfo(np.float32).tiny                  # the smallest non-zero result is normal
    for v in (-30.0, -1.5, 0.0, 2.0, 40.0):                               # silu(x) = x / (1 + exp(-x))
        assert orc.silu(v) == np.float32(np.float32(v) / (np.float32(1.0) + np.float32(orc.expf(-v))))


def test_fp16_conversions_match_numpy():
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().or_fp16_to_fp32(int(h)) for h in allh[::3]], np.float32)
    ok = (got == ref[::3]) | (np.isnan(got) & np.isnan(ref[::3]))
    assert ok.all()
    rng = np.random.default_rng(3)
    f = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 3000),
                        np.float32([65504.0, 65520.0, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8, 1e-9, -0.0, np.inf])])
    got = np.array([orc.lib().or_fp32_to_fp16(float(v)) for v in f], np.uint16)
    with np.errstate(over="ignore"):
        assert (got == f.astype(np.float16).view(np.uint16)).all()


# ------------------------------------------------------------------ activation quantizers

def np_quantize_q8_K(x: np.ndarray) -> np.ndarray:
    """ggml's quantize_row_q8_K (scalar reference) in float32 numpy: first-occurrence signed max,
    iscale = -127/max, nearest_int(iscale * x) by the 1.5 * 2^23 trick, min(127, .), int16 sums of 16."""
    out = np.zeros((x.size // 256, 292), np.uint8)
    for i, blk in enumerate(x.astype(np.float32).reshape(-1, 256)):
        ax = np.abs(blk)
        amax = ax.max()
        if amax == 0:
            continue
        mx = blk[int(np.argmax(ax))]                          # argmax returns the first occurrence
        iscale = np.float32(-127.0) / mx
        v = (iscale * blk).astype(np.float32) + np.float32(12582912.0)
        q = (v.view(np.int32) & 0x007FFFFF) - 0x00400000
        q = np.minimum(q, 127).astype(np.int8)
        out[i, 0:4] = np.frombuffer(np.float32(np.float32(1.0) / iscale).tobytes(), np.uint8)
        out[i, 4:260] = q.view(np.uint8)
        out[i, 260:292] = q.astype(np.int16).reshape(16, 16).sum(axis=1).astype(np.int16).view(np.uint8)
    return out


def np_quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """ggml's x86 quantize_row_q8_0 in float32 numpy: d = amax/127 (fp16), id = 127/amax, round-half-even."""
    out = np.zeros((x.size // 32, 34), np.uint8)
    for i, blk in enumerate(x.astype(np.float32).reshape(-1, 32)):
        amax = np.abs(blk).max()
        d = np.float32(amax / np.float32(127.0))
        idv = np.float32(np.float32(127.0) / amax) if amax != 0 else np.float32(0.0)
        out[i, 0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
        out[i, 2:34] = np.rint((blk * idv).astype(np.float32)).astype(np.int8).view(np.uint8)
    return out


@pytest.mark.parametrize("name", ["normal", "heavy", "ties", "sparse", "zero_block", "neg_max", "lane_tie"])
def test_q8k_matches_ggml_scalar_restatement(name):
    x = x_distributions(4096, seed=17)[name]
    got = orc.quantize(GType.Q8_K, x.reshape(2, 2048)).reshape(-1, 292)
    assert (got == np_quantize_q8_K(x)).all()


@pytest.mark.parametrize("name", ["normal", "heavy", "ties", "sparse", "zero_block"])
def test_q8_0_matches_ggml_x86_restatement(name):
    x = x_distributions(4096, seed=19)[name]
    got = orc.quantize(GType.Q8_0, x.reshape(2, 2048)).reshape(-1, 34)
    assert (got == np_quantize_q8_0(x)).all()


def test_q8_0_known_answers_round_half_even():
    """Q8_0 at exact .5 ties.  The reference links ggml built for its AVX2 host (Makefile:1 names the
    Threadripper/AVX2 target, Makefile:6 compiles with -march=native, and llama.cpp's own build defaults to the
    native ISA), so from_float for IQ4_NL activations is ggml's AVX2 quantize_row_q8_0, whose
    _mm256_round_ps(_MM_ROUND_NEAREST) rounds half to even; the scalar fallback's roundf would give the
    away-from-zero column below instead.  amax = 127 makes id = 127/amax = 1 exactly and d = 1 (fp16 0x3C00),
    so every q is the rounding of x itself."""
    x = np.zeros(64, np.float32)
    ties = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5, 126.5, -126.5, 0.25, -0.75]
    x[0:len(ties)] = ties
    x[31] = -127.0                                                   # amax of block 0
    even = [0, 2, 2, 0, -2, -2, 4, -4, 126, -126, 0, -1]
    away = [1, 2, 3, -1, -2, -3, 4, -4, 127, -127, 0, -1]
    x[32:40] = [63.5, -63.5, 0.5, 127.0, 1.5, 64.5, -0.5, 2.5]      # block 1: amax 127 again
    got = orc.quantize(GType.Q8_0, x).reshape(2, 34)
    assert bytes(got[0, 0:2]) == b"\x00\x3c" and bytes(got[1, 0:2]) == b"\x00\x3c"   # d = 1.0 in fp16
    q0 = got[0, 2:34].view(np.int8)
    assert list(q0[:len(ties)]) == even and list(q0[:len(ties)]) != away
    assert q0[31] == -127 and not q0[len(ties):31].any()
    assert list(got[1, 2:10].view(np.int8)) == [64, -64, 0, 127, 2, 64, 0, 2]


def test_q5k_known_answer_positions():
    """Q5_K element e of sub-block j = e / 32, l = e % 32: low 4 bits in qs[32 (j / 2) + l] at byte 48 (high nibble
    for odd j), bit 4 = bit j of qh[l] at byte 16; value (d sc_j) q5 - dmin m_j (src/kernels4.cu:437-448)."""
    want = np.array([(7 * e + 3 * (e // 32) + e // 64) % 32 for e in range(256)], np.int64)
    assert len(set(want[0:32])) == 32 and (want >= 16).sum() > 100      # every sub-block uses the fifth bit
    blk = np.zeros(176, np.uint8)
    blk[0:2], blk[2:4] = _f16b(1.0), _f16b(0.0)
    blk[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]                  # sc = 1, m = 0 for all eight sub-blocks
    for e in range(256):
        j, l = divmod(e, 32)
        blk[48 + 32 * (j // 2) + l] |= (want[e] & 15) << (4 * (j % 2))
        blk[16 + l] |= (want[e] >> 4) << j
    assert (orc.dequant_row(GType.Q5_K, blk, 256) == want.astype(np.float32)).all()
    # scales and mins through the j >= 4 branch: sub-block 6 gets sc = 37 (low 4 bits 5 in byte 10, high 2 bits 2
    # in byte 2's top bits), m = 3 (byte 10's high nibble)
    blk[2:4] = _f16b(0.5)
    blk[4 + 10] = 5 | (3 << 4)
    blk[4 + 2] = 1 | (2 << 6)
    j6 = np.arange(256) // 32 == 6
    exp = np.where(j6, np.float32(37) * want.astype(np.float32) - np.float32(1.5), want.astype(np.float32)).astype(np.float32)
    assert (orc.dequant_row(GType.Q5_K, blk, 256) == exp).all()


def test_iq4xs_known_answer_positions():
    """IQ4_XS 32-group ib: 6-bit scale ls = nibble (ib & 1) of scales_l[ib / 2] | bits 2 ib of scales_h << 4; element
    l < 16 is the low nibble of qs[16 ib + l], l >= 16 the high nibble of qs[16 ib + l - 16]; value
    (d (ls - 32)) kv[nibble] (src/kernels4.cu:660-670)."""
    kv = nf.KV_IQ4NL
    ls = np.array([33, 40, 1, 63, 17, 37, 50, 9], np.int64)             # every value of the two high bits occurs
    idx = np.array([(5 * e + e // 32 + 3 * ((e // 16) % 2)) % 16 for e in range(256)], np.int64)
    blk = np.zeros(136, np.uint8)
    blk[0:2] = _f16b(1.0)
    sh = 0
    for ib in range(8):
        blk[4 + ib // 2] |= (ls[ib] & 15) << (4 * (ib % 2))
        sh |= int(ls[ib] >> 4) << (2 * ib)
    blk[2:4] = np.frombuffer(np.uint16(sh).tobytes(), np.uint8)
    for e in range(256):
        ib, l = divmod(e, 32)
        blk[8 + 16 * ib + (l % 16)] |= idx[e] << (4 if l >= 16 else 0)
    want = ((ls[np.arange(256) // 32] - 32) * kv[idx]).astype(np.float32)
    assert (orc.dequant_row(GType.IQ4_XS, blk, 256) == want).all()


def test_iq4nl_known_answer_positions():
    """IQ4_NL block of 32: value j < 16 is kv[qs[j] & 15] d, value 16 + j is kv[qs[j] >> 4] d (src/kernels4.cu:629-636)."""
    kv = nf.KV_IQ4NL
    idx = np.array([[(3 * j + 7 * b + (j >= 16)) % 16 for j in range(32)] for b in range(2)], np.int64)
    blk = np.zeros((2, 18), np.uint8)
    for b, dv in enumerate((2.0, -0.5)):
        blk[b, 0:2] = _f16b(dv)
        for j in range(32):
            blk[b, 2 + (j % 16)] |= idx[b, j] << (4 if j >= 16 else 0)
    want = np.concatenate([kv[idx[0]] * 2.0, kv[idx[1]] * -0.5]).astype(np.float32)
    assert (orc.dequant_row(GType.IQ4_NL, blk.reshape(-1), 64) == want).all()


def test_iq2xxs_known_answer_positions():
    """IQ2_XXS (src/kernels4.cu:578-589): 32-group ib's grid rows are bytes 2 + 8 ib + l, its word at 6 + 8 ib holds the
    four 7-bit sign indices (bits 7 l ..) and the 4-bit scale (bits 28 ..); value = d (0.5 + sc) / 4 * grid * sign.
    Rows fixed by the reference's table: row 0 is all 8s, row 1 = 0x080808080808082b (byte 0 = 43).  With d = 1:
    group 0 takes rows 0, 1, 0, 0 and sign index 1 on 8-group 1 (ksign(1) = 0x81: elements 0 and 7 negated),
    scale 0 (db = 1/8); group 1 takes row 0 with scale 15 (db = 3.875); the rest row 0, scale 0."""
    rows = iq2xxs_rows()
    assert list(rows[0]) == [8] * 8 and list(rows[1]) == [43] + [8] * 7
    blk = np.zeros(66, np.uint8)
    blk[0:2] = _f16b(1.0)
    blk[2 + 1] = 1                                             # group 0, 8-group 1: grid row 1
    blk[6:10] = np.frombuffer(np.uint32(1 << 7).tobytes(), np.uint8)     # group 0: sign index 1 on 8-group 1
    blk[14:18] = np.frombuffer(np.uint32(15 << 28).tobytes(), np.uint8)  # group 1: scale 15
    want = np.ones(256, np.float32)
    want[8:16] = [-43 / 8, 1, 1, 1, 1, 1, 1, -1]
    want[32:64] = 31.0
    got = orc.dequant_row(GType.IQ2_XXS, blk, 256)
    assert (got == want).all(), np.nonzero(got != want)
    x = np.arange(256, dtype=np.float32) % 7 - 3.0            # small integers: Q8_K of x is exact up to its scale
    xq = orc.quantize(GType.Q8_K, x)
    q8 = xq[4:260].view(np.int8).astype(np.int64)
    ints = (want * 8).astype(np.int64)                          # grid * sign at scale 0; group 1's rows stay 8s
    ints[32:64] = 8
    scale = np.array([1] + [31] + [1] * 6, np.int64)            # 2 sc + 1 per 32-group
    si, sm = orc.block_ints(GType.IQ2_XXS, blk, xq, 256)
    assert int(si[0]) == int(sum(scale[g] * (ints[32 * g:32 * g + 32] @ q8[32 * g:32 * g + 32]) for g in range(8)))
    assert not sm.any()


def test_iq3xxs_known_answer_positions():
    """IQ3_XXS (src/kernels4.cu:613-627): 32-group ib's grid indices are bytes 2 + 8 ib .. (8-group l: rows 2 l, 2 l + 1
    of 4 bytes each), its word at 66 + 4 ib holds the four 7-bit sign indices (bits 7 l ..) and the 4-bit scale (bits
    28 ..); value = d (0.5 + sc) / 2 * grid * sign.  Rows fixed by the reference's table: row 0 is all 4s, row 1 =
    0x04040414 (byte 0 = 20).  With d = 1: group 0's 8-group 1 takes rows 1, 0 and sign index 1 (ksign(1) = 0x81:
    elements 0 and 7 negated), scale 0 (db = 1/4); group 1 has scale 15 (db = 7.75); the rest row 0, scale 0."""
    rows = iq3xxs_rows()
    assert list(rows[0]) == [4] * 4 and list(rows[1]) == [20, 4, 4, 4]
    blk = np.zeros(98, np.uint8)
    blk[0:2] = _f16b(1.0)
    blk[2 + 2] = 1                                                         # group 0, 8-group 1, first row: 1
    blk[66:70] = np.frombuffer(np.uint32(1 << 7).tobytes(), np.uint8)     # group 0: sign index 1 on 8-group 1
    blk[70:74] = np.frombuffer(np.uint32(15 << 28).tobytes(), np.uint8)   # group 1: scale 15
    want = np.ones(256, np.float32)
    want[8:16] = [-5, 1, 1, 1, 1, 1, 1, -1]
    want[32:64] = 31.0
    got = orc.dequant_row(GType.IQ3_XXS, blk, 256)
    assert (got == want).all(), np.nonzero(got != want)
    x = np.arange(256, dtype=np.float32) % 7 - 3.0
    xq = orc.quantize(GType.Q8_K, x)
    q8 = xq[4:260].view(np.int8).astype(np.int64)
    ints = (want * 4).astype(np.int64)                          # grid * sign at scale 0; group 1's rows stay 4s
    ints[32:64] = 4
    scale = np.array([1] + [31] + [1] * 6, np.int64)            # 2 sc + 1 per 32-group
    si, sm = orc.block_ints(GType.IQ3_XXS, blk, xq, 256)
    assert int(si[0]) == int(sum(scale[g] * (ints[32 * g:32 * g + 32] @ q8[32 * g:32 * g + 32]) for g in range(8)))
    assert not sm.any()


def test_iq3s_known_answer_positions():
    """IQ3_S (src/kernels4.cu:682-695): 32-group ib's 8-group l takes rows qs[8 ib + 2 l] and qs[8 ib + 2 l + 1], each with
    a 9th index bit from qh[ib] (bits 2 l, 2 l + 1); bit j of the literal byte signs[4 ib + l] negates value j; value =
    d (1 + 2 sc) * grid.  Rows fixed by the reference's table: row 0 = 0x01010101, row 1 = 0x01010103 (byte 0 = 3),
    row 256 (the 9th bit) = its own first entry.  Placed by hand: group 0, 8-group 1 takes row 1 then row 256 (9th
    bit of the second index), sign byte 0x81; group 3 has scale 7 (factor 15)."""
    rows = iq3s_rows()
    assert list(rows[0]) == [1, 1, 1, 1] and list(rows[1]) == [3, 1, 1, 1]
    r256 = [int(v) for v in rows[256]]
    assert r256 != [1, 1, 1, 1]   # so a dropped 9th index bit (row 0 in its place) shows
    blk = np.zeros(110, np.uint8)
    blk[0:2] = _f16b(1.0)
    blk[2 + 2] = 1                # group 0, 8-group 1, first index: row 1
    blk[66] = 1 << 3              # group 0: 9th bit of index 3 (8-group 1's second): row 256
    blk[74 + 1] = 0x81            # group 0, 8-group 1: values 0 and 7 negated
    blk[106 + 1] = 7 << 4         # group 3: scale 7
    want = np.ones(256, np.float32)
    want[8:16] = [-3, 1, 1, 1] + [r256[0], r256[1], r256[2], -r256[3]]
    want[96:128] = 15.0
    got = orc.dequant_row(GType.IQ3_S, blk, 256)
    assert (got == want).all(), np.nonzero(got != want)
    x = np.arange(256, dtype=np.float32) % 5 - 2.0
    xq = orc.quantize(GType.Q8_K, x)
    q8 = xq[4:260].view(np.int8).astype(np.int64)
    ints = want.astype(np.int64)
    ints[96:128] = 1
    scale = np.array([1, 1, 1, 15, 1, 1, 1, 1], np.int64)
    si, sm = orc.block_ints(GType.IQ3_S, blk, xq, 256)
    assert int(si[0]) == int(sum(scale[g] * (ints[32 * g:32 * g + 32] @ q8[32 * g:32 * g + 32]) for g in range(8)))
    assert not sm.any()


def test_iq2s_known_answer_positions():
    """IQ2_S (src/kernels4.cu:602-613): 32-group ib's 8-group l takes grid row qs[4 ib + l] with bits 2 l, 2 l + 1 of
    qh[ib] as index bits 8-9; bit j of the literal byte signs[4 ib + l] negates value j; value = d (0.5 + sc) / 4 * grid,
    sc the nibble l / 2 of scales[ib].  Rows fixed by the reference's table: row 0 all 8s, row 1 = byte 0 43, the rest 8;
    row 768 (both high bits) differs from row 0.  Placed by hand: group 0's 8-group 1 takes row 1 with sign byte 0x81,
    its 8-group 2 row 768; group 2's second 16-group has scale 15."""
    rows = iq2s_rows()
    assert list(rows[0]) == [8] * 8 and list(rows[1]) == [43] + [8] * 7
    r768 = [int(v) for v in rows[768]]
    assert r768 != [8] * 8
    blk = np.zeros(82, np.uint8)
    blk[0:2] = _f16b(1.0)
    blk[2 + 1] = 1                 # group 0, 8-group 1: row 1
    blk[34 + 1] = 0x81             # its sign byte: values 0 and 7 negated
    blk[66] = 3 << 4               # group 0, 8-group 2: index bits 8-9 set (row 768)
    blk[74 + 2] = 15 << 4          # group 2, second 16-group: scale 15
    want = np.ones(256, np.float32)                                # d (0.5 + 0) / 4 * 8 = 1
    want[8:16] = [-43 / 8, 1, 1, 1, 1, 1, 1, -1]
    want[16:24] = np.array(r768, np.float32) / 8
    want[80:96] = 31.0                                             # (0.5 + 15) / 4 * 8
    got = orc.dequant_row(GType.IQ2_S, blk, 256)
    assert (got == want).all(), np.nonzero(got != want)
    x = np.arange(256, dtype=np.float32) % 7 - 3.0
    xq = orc.quantize(GType.Q8_K, x)
    q8 = xq[4:260].view(np.int8).astype(np.int64)
    ints = (want * 8).astype(np.int64)
    ints[80:96] = 8
    scale = np.ones(16, np.int64)
    scale[5] = 31                                                  # 16-group 5 = group 2's second half
    si, sm = orc.block_ints(GType.IQ2_S, blk, xq, 256)
    assert int(si[0]) == int(sum(scale[g] * (ints[16 * g:16 * g + 16] @ q8[16 * g:16 * g + 16]) for g in range(16)))
    assert not sm.any()


def test_iq1s_known_answer_positions():
    """IQ1_S (src/kernels4.cu:650-659): 32-group ib's 8-group l takes grid row qs[4 ib + l] with bits 3 l .. 3 l + 2 of
    qh[ib] as index bits 8-10; value = d (2 s + 1) (grid + delta), s = qh bits 12-14, delta = -1/8 if qh bit 15 else
    +1/8.  Rows fixed by the reference's table: row 0 = all -1, row 1 = -1 except byte 0 = +1 (0xffffffffffffff01 read
    little-endian); row 1792 (index bits 8-10 all set) differs from row 0.  Placed by hand: group 0's 8-group 1 takes
    row 1, group 1's 8-group 2 row 1792 with scale 5 (factor 11) and the negative delta."""
    rows = iq1s_rows()
    assert list(rows[0]) == [-1] * 8
    r1, r1792 = [int(v) for v in rows[1]], [int(v) for v in rows[1792]]
    assert r1 == [1] + [-1] * 7 and r1792 != [-1] * 8
    blk = np.zeros(50, np.uint8)
    blk[0:2] = _f16b(0.5)
    blk[2 + 1] = 1                                                        # group 0, 8-group 1: row 1
    qh1 = (7 << 6) | (5 << 12) | 0x8000                                   # group 1: 8-group 2 high bits, scale 5, -delta
    blk[34 + 2:34 + 4] = np.frombuffer(np.uint16(qh1).tobytes(), np.uint8)
    grid = np.full(256, -1.0)
    grid[8:16] = r1
    grid[48:56] = r1792
    dl = np.array([0.5] * 32 + [0.5 * 11] * 32 + [0.5] * 192)
    delta = np.array([0.125] * 32 + [-0.125] * 32 + [0.125] * 192)
    want = (dl.astype(np.float32) * (grid.astype(np.float32) + delta.astype(np.float32))).astype(np.float32)
    got = orc.dequant_row(GType.IQ1_S, blk, 256)
    assert (got == want).all(), np.nonzero(got != want)
    x = np.arange(256, dtype=np.float32) % 9 - 4.0
    xq = orc.quantize(GType.Q8_K, x)
    q8 = xq[4:260].view(np.int8).astype(np.int64)
    ls = np.array([1, 11, 1, 1, 1, 1, 1, 1], np.int64)
    sg = np.array([1, -1, 1, 1, 1, 1, 1, 1], np.int64)
    g = grid.astype(np.int64)
    si, sm = orc.block_ints(GType.IQ1_S, blk, xq, 256)
    assert int(si[0]) == int(sum(ls[k] * (g[32 * k:32 * k + 32] @ q8[32 * k:32 * k + 32]) for k in range(8)))
    assert int(sm[0]) == int(sum(ls[k] * sg[k] * q8[32 * k:32 * k + 32].sum() for k in range(8)))


def test_q8_0_weight_known_answers():
    """Q8_0 weights (src/kernels4.cu:421-714, deq8: d * qs[j]): value j of a block is d * (int8) qs[j] in place, and
    against a Q8_0 activation block the integer is sum_j qs[j] y[j] (ggml's vec_dot_q8_0_q8_0), folded as
    x_d * (d * sumi)."""
    q = np.array([[(5 * j + 3 * b) % 256 - 128 for j in range(32)] for b in range(2)], np.int64)   # -128 .. 127
    blk = np.zeros((2, 34), np.uint8)
    for b, dv in enumerate((0.5, -0.25)):
        blk[b, 0:2] = _f16b(dv)
        blk[b, 2:34] = q[b].astype(np.int8).view(np.uint8)
    want = np.concatenate([q[0] * 0.5, q[1] * -0.25]).astype(np.float32)
    assert (orc.dequant_row(GType.Q8_0, blk.reshape(-1), 64) == want).all()
    y = np.array([(-7 * j) % 255 - 127 for j in range(64)], np.int64)   # the activation's int8 values
    ya = np.zeros((2, 34), np.uint8)
    for b, yd in enumerate((2.0, 0.125)):
        ya[b, 0:2] = _f16b(yd)
        ya[b, 2:34] = y[32 * b:32 * b + 32].astype(np.int8).view(np.uint8)
    si, sm = orc.block_ints(GType.Q8_0, blk.reshape(-1), ya.reshape(-1), 64)
    assert list(si) == [int(q[0] @ y[:32]), int(q[1] @ y[32:])] and not sm.any()
    t0, t1 = np.float32(0.5) * np.float32(si[0]), np.float32(-0.25) * np.float32(si[1])
    acc = np.float32(np.float64(2.0) * np.float64(t0))
    want_dot = np.float32(np.float64(np.float32(0.125)) * np.float64(t1) + np.float64(acc))   # one rounding: fmaf
    assert orc.row_dot(GType.Q8_0, blk.reshape(-1), ya.reshape(-1), 64) == want_dot


def test_mxfp4_known_answers():
    """MXFP4 (src/kernels4.cu:550-577): byte 0 is an E8M0 exponent, value j < 16 = kv[qs[j] & 15] * 2^(e - 128) and
    16 + j = kv[qs[j] >> 4] * 2^(e - 128), kv the E2M1 codes doubled (OCP MX: code 7 = 6.0 -> 12, code 9 = -0.5 -> -1,
    code 8 = -0 -> 0).  The scale's edge exponents: 0 and 1 give the fp32 subnormals 2^-128, 2^-127; 255 gives 2^127
    (no NaN code).  Against Q8_0 the integer is sum kv y, folded as x_d * (2^(e - 128) * sumi)."""
    assert list(nf.e2m1_doubled(np.arange(16))) == [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    exps = (128, 0, 1, 255, 127)
    idx = np.array([[(5 * j + 3 * b + (j >= 16)) % 16 for j in range(32)] for b in range(len(exps))], np.int64)
    blk = np.zeros((len(exps), 17), np.uint8)
    for b, e in enumerate(exps):
        blk[b, 0] = e
        for j in range(32):
            blk[b, 1 + (j % 16)] |= idx[b, j] << (4 if j >= 16 else 0)
    kv = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.float64)
    with np.errstate(over="ignore"):   # e = 255: kv 2^127 past fp32's range for |kv| >= 2 is inf, as the product is there
        want = np.concatenate([kv[idx[b]] * np.ldexp(1.0, e - 128) for b, e in enumerate(exps)]).astype(np.float32)
    assert np.isinf(want[96:128]).any()
    assert np.float32(np.ldexp(1.0, -128)) != 0 and np.float32(np.ldexp(1.0, 127)) == np.float32(2.0 ** 127)
    got = orc.dequant_row(GType.MXFP4, blk.reshape(-1), 32 * len(exps))
    assert (got == want).all(), np.nonzero(got != want)
    y = np.array([(11 * j) % 255 - 127 for j in range(64)], np.int64)
    ya = np.zeros((2, 34), np.uint8)
    for b, yd in enumerate((0.25, 3.0)):
        ya[b, 0:2] = _f16b(yd)
        ya[b, 2:34] = y[32 * b:32 * b + 32].astype(np.int8).view(np.uint8)
    wb = blk[[0, 4]].reshape(-1)                                  # exponents 128 and 127: scales 1 and 1/2
    si, sm = orc.block_ints(GType.MXFP4, wb, ya.reshape(-1), 64)
    ints = [int(kv[idx[0]].astype(np.int64) @ y[:32]), int(kv[idx[4]].astype(np.int64) @ y[32:])]
    assert list(si) == ints and not sm.any()
    t0, t1 = np.float32(si[0]), np.float32(0.5) * np.float32(si[1])
    acc = np.float32(np.float64(0.25) * np.float64(t0))
    want_dot = np.float32(np.float64(3.0) * np.float64(t1) + np.float64(acc))    # one rounding: fmaf
    assert orc.row_dot(GType.MXFP4, wb, ya.reshape(-1), 64) == want_dot


def test_q5_0_known_answers():
    """Q5_0 (src/kernels4.cu:464-478): value j = (nibble j | bit j of qh << 4) - 16, nibble j the low one of qs[j] for
    j < 16 and the high one of qs[j - 16] above; qh a little-endian u32 at byte 2.  Blocks built value by value (each
    x in 0..31 placed by hand), so a swapped nibble half, a qh bit read from the wrong end, or a dropped -16 fails;
    against Q8_0 the integer is sum (x - 16) y, folded as x_d * (d * sumi)."""
    x = np.array([[(7 * j + 11 * b) % 32 for j in range(32)] for b in range(2)], np.int64)   # 0 .. 31
    blk = np.zeros((2, 22), np.uint8)
    for b, dv in enumerate((0.5, -2.0)):
        blk[b, 0:2] = _f16b(dv)
        qh = 0
        for j in range(32):
            blk[b, 6 + (j % 16)] |= (x[b, j] & 15) << (4 if j >= 16 else 0)
            qh |= int(x[b, j] >> 4) << j
        blk[b, 2:6] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    want = np.concatenate([(x[0] - 16) * 0.5, (x[1] - 16) * -2.0]).astype(np.float32)
    assert (orc.dequant_row(GType.Q5_0, blk.reshape(-1), 64) == want).all()
    y = np.array([(13 * j) % 255 - 127 for j in range(64)], np.int64)
    ya = np.zeros((2, 34), np.uint8)
    for b, yd in enumerate((0.75, 0.125)):
        ya[b, 0:2] = _f16b(yd)
        ya[b, 2:34] = y[32 * b:32 * b + 32].astype(np.int8).view(np.uint8)
    si, sm = orc.block_ints(GType.Q5_0, blk.reshape(-1), ya.reshape(-1), 64)
    assert list(si) == [int((x[0] - 16) @ y[:32]), int((x[1] - 16) @ y[32:])] and not sm.any()
    t0, t1 = np.float32(0.5) * np.float32(si[0]), np.float32(-2.0) * np.float32(si[1])
    acc = np.float32(np.float64(0.75) * np.float64(t0))
    want_dot = np.float32(np.float64(0.125) * np.float64(t1) + np.float64(acc))    # one rounding: fmaf
    assert orc.row_dot(GType.Q5_0, blk.reshape(-1), ya.reshape(-1), 64) == want_dot


def test_q2k_known_answer_positions():
    """Q2_K (src/kernels4.cu:639-647): value 128 h + 32 j + l is bits 2 j of qs byte 32 h + l (qs at 16), scaled by
    d * (scale nibble) minus dmin * (min nibble) of its 16-group's scale byte (index value // 16).  Every value's
    2-bit field is placed by hand, and each group gets its own scale and min, so a wrong byte, shift, group or nibble
    fails; the block integers (sum sc sum q y, sum m bsum) are checked the same way."""
    q = np.array([(3 * e + e // 37) % 4 for e in range(256)], np.int64)
    sc = np.array([(5 * g + 1) % 16 for g in range(16)], np.int64)
    mn = np.array([(7 * g + 3) % 16 for g in range(16)], np.int64)
    blk = np.zeros(84, np.uint8)
    blk[0:16] = sc | (mn << 4)
    for e in range(256):
        h, j, l = e // 128, (e // 32) % 4, e % 32
        blk[16 + 32 * h + l] |= q[e] << (2 * j)
    blk[80:82] = _f16b(0.5)
    blk[82:84] = _f16b(0.25)
    g = np.arange(256) // 16
    dl = (np.float32(0.5) * sc[g].astype(np.float32)).astype(np.float32)
    ml = (np.float32(0.25) * mn[g].astype(np.float32)).astype(np.float32)
    want = (dl * q.astype(np.float32) - ml).astype(np.float32)
    assert (orc.dequant_row(GType.Q2_K, blk, 256) == want).all()
    x = np.arange(256, dtype=np.float32) % 9 - 4.0
    xq = orc.quantize(GType.Q8_K, x)
    q8 = xq[4:260].view(np.int8).astype(np.int64)
    si, sm = orc.block_ints(GType.Q2_K, blk, xq, 256)
    assert int(si[0]) == int(sum(sc[k] * (q[16 * k:16 * k + 16] @ q8[16 * k:16 * k + 16]) for k in range(16)))
    assert int(sm[0]) == int(sum(mn[k] * q8[16 * k:16 * k + 16].sum() for k in range(16)))


def test_q3k_known_answer_positions():
    """Q3_K (src/kernels4.cu:698-707): value 128 hf + 32 j + l = (bits 2 j of qs byte 32 hf + l) - 4 unless bit 4 hf + j
    of hmask[l] is set, times d * (scale - 32) of its 16-group; the 16 scales are 6-bit values split into a nibble and
    two high bits.  Every 2-bit field, hmask bit and scale is placed by hand (scales 0..63 all distinct per group), so a
    wrong byte, shift, nibble half or high-bit position fails; the block integer is checked against the hand values."""
    q2 = np.array([(5 * e + e // 29) % 4 for e in range(256)], np.int64)
    hb = np.array([(e * 7 + e // 11) % 3 != 0 for e in range(256)], np.int64)
    sc6 = np.array([(11 * g + 5) % 64 for g in range(16)], np.int64)
    blk = np.zeros(110, np.uint8)
    for e in range(256):
        hf, j, l = e // 128, (e // 32) % 4, e % 32
        blk[32 + 32 * hf + l] |= q2[e] << (2 * j)
        blk[l] |= hb[e] << (4 * hf + j)
    for g in range(16):
        blk[96 + g % 8] |= (sc6[g] & 15) << (4 * (g // 8))
        blk[104 + g % 4] |= (sc6[g] >> 4) << (2 * (g // 4))
    blk[108:110] = _f16b(0.25)
    val = q2 - 4 * (1 - hb)
    dl = (np.float32(0.25) * (sc6 - 32).astype(np.float32)).astype(np.float32)
    want = (dl[np.arange(256) // 16] * val.astype(np.float32)).astype(np.float32)
    assert (orc.dequant_row(GType.Q3_K, blk, 256) == want).all()
    x = np.arange(256, dtype=np.float32) % 11 - 5.0
    xq = orc.quantize(GType.Q8_K, x)
    q8 = xq[4:260].view(np.int8).astype(np.int64)
    si, sm = orc.block_ints(GType.Q3_K, blk, xq, 256)
    assert int(si[0]) == int(sum((sc6[g] - 32) * (val[16 * g:16 * g + 16] @ q8[16 * g:16 * g + 16]) for g in range(16)))
    assert not sm.any()


def test_q5_1_known_answers():
    """Q5_1 (src/kernels4.cu:449-462): value j = x d + m with x = nibble j | bit j of qh << 4 (0..31).  Blocks built value
    by value; against a Q8_0 activation block the integers are sum x y and sum y (the min's partner: the Q8_1 row's d
    and q are Q8_0's, and sum y stands for its s / d), folded as x_d * fma(d, sumi, m * sum y)."""
    x = np.array([[(9 * j + 5 * b) % 32 for j in range(32)] for b in range(2)], np.int64)
    blk = np.zeros((2, 24), np.uint8)
    for b, (dv, mv) in enumerate(((0.5, -3.0), (-0.25, 1.5))):
        blk[b, 0:2] = _f16b(dv)
        blk[b, 2:4] = _f16b(mv)
        qh = 0
        for j in range(32):
            blk[b, 8 + (j % 16)] |= (x[b, j] & 15) << (4 if j >= 16 else 0)
            qh |= int(x[b, j] >> 4) << j
        blk[b, 4:8] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    want = np.concatenate([(x[0] * np.float32(0.5)).astype(np.float32) + np.float32(-3.0),
                           (x[1] * np.float32(-0.25)).astype(np.float32) + np.float32(1.5)]).astype(np.float32)
    assert (orc.dequant_row(GType.Q5_1, blk.reshape(-1), 64) == want).all()
    y = np.array([(17 * j) % 255 - 127 for j in range(64)], np.int64)
    ya = np.zeros((2, 34), np.uint8)
    for b, yd in enumerate((0.5, 2.0)):
        ya[b, 0:2] = _f16b(yd)
        ya[b, 2:34] = y[32 * b:32 * b + 32].astype(np.int8).view(np.uint8)
    si, sm = orc.block_ints(GType.Q5_1, blk.reshape(-1), ya.reshape(-1), 64)
    assert list(si) == [int(x[0] @ y[:32]), int(x[1] @ y[32:])]
    assert list(sm) == [int(y[:32].sum()), int(y[32:].sum())]
    t0 = np.float32(np.float64(0.5) * np.float64(si[0]) + np.float64(np.float32(-3.0) * np.float32(sm[0])))
    t1 = np.float32(np.float64(-0.25) * np.float64(si[1]) + np.float64(np.float32(1.5) * np.float32(sm[1])))
    acc = np.float32(np.float64(0.5) * np.float64(t0))
    want_dot = np.float32(np.float64(2.0) * np.float64(t1) + np.float64(acc))   # fmaf: one rounding each
    assert orc.row_dot(GType.Q5_1, blk.reshape(-1), ya.reshape(-1), 64) == want_dot


def test_q8k_known_answers():
    x = np.zeros(512, np.float32)
    # block 0: max -127 at index 3 -> iscale = 1, q = round-half-even(x)
    x[:8] = [2.5, 3.5, -0.5, -127.0, 1.5, -2.5, 0.49999997, 126.5]
    # block 1: |x| equal at 10 (positive, first) and 20 (negative): max = +5, iscale = -25.4
    x[256 + 10], x[256 + 20], x[256 + 30] = 5.0, -5.0, 0.1
    q = orc.quantize(GType.Q8_K, x).reshape(2, 292)
    d0, qs0 = q[0, 0:4].view(np.float32)[0], q[0, 4:260].view(np.int8)
    assert d0 == 1.0
    assert list(qs0[:8]) == [2, 4, 0, -127, 2, -2, 0, 126]
    assert (q[0, 260:292].view(np.int16) == qs0.astype(np.int16).reshape(16, 16).sum(1)).all()
    d1, qs1 = q[1, 0:4].view(np.float32)[0], q[1, 4:260].view(np.int8)
    assert qs1[10] == -127 and qs1[20] == 127 and qs1[30] == -3      # -25.4 * 0.1 = -2.54 -> -3
    assert d1 == np.float32(1.0) / (np.float32(-127.0) / np.float32(5.0))
    z = orc.quantize(GType.Q8_K, np.zeros(256, np.float32))          # all zero: d = 0, qs = 0, bsums = 0
    assert not z.any()


# ------------------------------------------------------------------ block decoding

ALL = [GType.Q4_K, GType.Q5_K, GType.Q6_K, GType.IQ4_XS, GType.IQ2_XS, GType.IQ2_XXS, GType.IQ4_NL, GType.Q8_0, GType.MXFP4,
       GType.Q5_0, GType.Q2_K, GType.Q3_K, GType.IQ3_XXS, GType.IQ3_S, GType.IQ2_S, GType.IQ1_S, GType.Q5_1]


def blocks(t, nb, seed):
    return random_blocks(t, nb, gen(seed), "cpu", D_RANGE.get(GType(t), (1e-3, 1e-2))).numpy()


@pytest.mark.parametrize("t", ALL)
def test_dequant_matches_numpy_decoder(t):
    b = blocks(t, 64, 100 + int(t))
    n = 64 * block_elems(t)
    got = orc.dequant_row(t, b.reshape(-1), n)
    ref = nf.dequant(t, b, grid_for(t), ksigns()).reshape(-1)
    assert (got == ref).all(), f"{int((got != ref).sum())} values differ"


def _f16b(v):
    return list(np.frombuffer(np.float16(v).tobytes(), np.uint8))


def test_q4k_known_answer_positions():
    """d = 1, dmin = 0, every sub-block scale 1: value e must be the nibble placed for element e by the
    reference's layout (byte 16 + 32 (j/2) + l, low nibble for even sub-block j; src/kernels4.cu:427-436)."""
    want = np.array([(7 * e + e // 32) % 16 for e in range(256)], np.int64)
    blk = np.zeros(144, np.uint8)
    blk[0:2], blk[2:4] = _f16b(1.0), _f16b(0.0)
    blk[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]              # sc = 1, m = 0 for all eight sub-blocks
    for e in range(256):
        j, l = divmod(e, 32)
        blk[16 + 32 * (j // 2) + l] |= want[e] << (4 * (j % 2))
    assert (orc.dequant_row(GType.Q4_K, blk, 256) == want.astype(np.float32)).all()
    blk[2:4] = _f16b(0.5)                                          # mins: sub-block 5 gets m = 3
    blk[4 + 9] = 1 | (3 << 4)                                      # scale byte 9: sc_5 = 1, m_5 = 3 (j >= 4 branch)
    exp = want.astype(np.float32) - np.where(np.arange(256) // 32 == 5, np.float32(1.5), np.float32(0))
    assert (orc.dequant_row(GType.Q4_K, blk, 256) == exp).all()


def test_q6k_known_answer_positions():
    """Q6_K element e = 128 hf + 32 qt + l: low 4 bits in ql[64 hf + 32 (qt & 1) + l] (high nibble for qt >= 2),
    bits 4-5 in qh[32 hf + l] >> 2 qt, int8 scale e // 16, value d * sc * (q6 - 32) (src/kernels4.cu:671-681)."""
    want = np.array([(11 * e) % 64 for e in range(256)], np.int64)
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        hf, qt, l = e // 128, (e // 32) % 4, e % 32
        blk[64 * hf + 32 * (qt & 1) + l] |= (want[e] & 15) << (4 if qt >= 2 else 0)
        blk[128 + 32 * hf + l] |= (want[e] >> 4) << (2 * qt)
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8) * np.where(np.arange(16) % 2, -1, 1).astype(np.int8).view(np.uint8)
    blk[208:210] = _f16b(1.0)
    sc = blk[192:208].view(np.int8).astype(np.float32)
    exp = (np.repeat(sc, 16) * (want - 32).astype(np.float32)).astype(np.float32)
    assert (orc.dequant_row(GType.Q6_K, blk, 256) == exp).all()


def test_iq2xs_known_answer():
    """IQ2_XS 8-group l of 32-group ib: grid row qs[4 ib + l] & 511, signs ksigns[qs >> 9], scale nibble (l / 2) of
    scales[ib]; value d (0.5 + sc) / 4 grid sign (src/kernels4.cu:592-601)."""
    rows, ks = iq2xs_rows(), ksigns()
    blk = np.zeros(74, np.uint8)
    blk[0:2] = _f16b(4.0)
    qs = np.array([(37 * i) % 512 | (((5 * i) % 128) << 9) for i in range(32)], np.uint16)
    blk[2:66] = qs.view(np.uint8)
    blk[66:74] = [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]
    got = orc.dequant_row(GType.IQ2_XS, blk, 256)
    for e in range(256):
        ib, l, j = e // 32, (e // 8) % 4, e % 8
        q = int(qs[4 * ib + l])
        sc = (blk[66 + ib] >> (4 * (l // 2))) & 15
        v = np.float32(4.0) * (np.float32(0.5) + np.float32(sc)) * np.float32(0.25) * np.float32(rows[q & 511, j])
        assert got[e] == (-v if (ks[q >> 9] >> j) & 1 else v)


# ------------------------------------------------------------------ integer block dots

@pytest.mark.parametrize("t", ALL)
def test_block_ints_brute_force(t):
    n = 2048
    vt = vec_dot_type(t)
    rows = blocks(t, 6 * n // block_elems(t), 200 + int(t)).reshape(6, -1)
    for name, x in list(x_distributions(n, seed=23).items())[:4]:
        xq = orc.quantize(vt, x)
        for r in range(rows.shape[0]):
            si, sm = orc.block_ints(t, rows[r], xq, n)
            bsi, bsm = nf.block_ints(t, rows[r], xq, grid_for(t), ksigns())
            assert (si == bsi).all() and (sm == bsm).all(), f"{t.name} {name} row {r}"


@pytest.mark.parametrize("t", [GType.Q4_K, GType.Q5_K, GType.Q6_K])
def test_vector_block_ints_equal_scalar_restatement(t):
    """The K-quants' AVX2 integers (the CPU baseline's path) equal the element-by-element restatement on every block,
    for all the quantizer-test activation distributions, including blocks with extreme scales."""
    n = 4096
    rows = blocks(t, 16 * n // 256, 400 + int(t)).reshape(16, -1)
    rows[0, :] = 0xFF            # every quant, scale and min at its maximum (the fp16 fields become NaN: ints only)
    if t == GType.Q6_K:
        rows[1].reshape(-1, 210)[:, 192:208] = 0x80   # int8 scales at -128
    for name, x in x_distributions(n, seed=29).items():
        xq = orc.quantize(GType.Q8_K, x)
        for r in range(rows.shape[0]):
            a = orc.block_ints(t, rows[r], xq, n)
            b = orc.block_ints(t, rows[r], xq, n, scalar=True)
            assert (a[0] == b[0]).all() and (a[1] == b[1]).all(), f"{t.name} {name} row {r}"


@pytest.mark.parametrize("t", ALL)
def test_row_dot_equals_fp64_of_dequantized_operands(t):
    """The block integers and their fp32 fold agree with sum(dequant(w) * dequant(q8(x))) in fp64 up to fp32 rounding."""
    n = 4096
    vt = vec_dot_type(t)
    rows = blocks(t, 8 * n // block_elems(t), 300 + int(t)).reshape(8, -1)
    x = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    xq = orc.quantize(vt, x)
    xd = orc.dequant_row(vt, xq, n).astype(np.float64)
    for r in range(8):
        w = nf.dequant(t, rows[r], grid_for(t), ksigns()).reshape(-1).astype(np.float64)
        ref = float(w @ xd)
        got = float(orc.row_dot(t, rows[r], xq, n))
        scale = float(np.abs(w).dot(np.abs(xd)))
        assert abs(got - ref) <= 1e-6 * scale + 1e-30, (t, r, got, ref)


# ------------------------------------------------------------------ router and bucketing

def test_router_gemv_sum_order_and_value():
    rng = np.random.default_rng(7)
    W = (rng.standard_normal((9, 2048)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, 2048)).astype(np.float32)
    y = orc.gemv_f32(W, x)
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(x).max() * np.abs(W).max() * 2048 ** 0.5
    # the contract's order, restated: 64 fma chains over e = 256 i + 4 L + j, then the xor butterfly 1 .. 32
    w, xv = W[0], x[0]
    part = []
    for L in range(64):
        a = np.float32(0)
        for i in range(8):
            for j in range(4):
                e = 256 * i + 4 * L + j
                a = np.float32(np.float64(w[e]) * np.float64(xv[e]) + np.float64(a))   # fma: exact product, one rounding
        part.append(a)
    part = np.array(part, np.float32)
    for off in (1, 2, 4, 8, 16, 32):
        part = (part + part[np.arange(64) ^ off]).astype(np.float32)
    assert part[0] == y[0, 0]


@pytest.mark.parametrize("E,k", [(128, 8), (288, 8), (384, 6), (512, 10), (1024, 16)])
def test_route_topk_properties(E, k):
    rng = np.random.default_rng(E)
    logits = (rng.standard_normal((20, E + 1)) * 3).astype(np.float32)
    ids, wts, sg = orc.route(logits, E, k, with_sg=True)
    for t in range(20):
        l = logits[t, :E].astype(np.float64)
        order = np.lexsort((np.arange(E), -l))          # exact selection on logits (softmax is monotonic)
        gap = l[order[k - 1]] - l[order[k]]
        if gap > 1e-5:
            assert list(ids[t]) == list(order[:k])
        p = np.exp(l[ids[t]] - l.max())
        assert np.allclose(wts[t], p / p.sum(), rtol=2e-6, atol=1e-12)
        assert abs(sg[t] - 1.0 / (1.0 + np.exp(-float(logits[t, E])))) <= 2e-7
    eq = np.full((1, E), 0.3, np.float32)                  # all ties: the lowest indices (tools/routebench.cu:20)
    ids, wts, _ = orc.route(eq, E, k)
    assert list(ids[0]) == list(range(k)) and np.all(wts == wts[0, 0])


def test_order_matches_stable_sort():
    rng = np.random.default_rng(9)
    E, P = 300, 5000
    slot = np.arange(E, dtype=np.int32)
    slot[rng.choice(E, 40, replace=False)] = -1
    ids = rng.integers(-3, E + 3, P).astype(np.int32)
    order, on, eg = orc.order(slot, ids, E)
    valid = (ids >= 0) & (ids < E)
    valid[valid] &= slot[ids[valid]] >= 0
    p = np.nonzero(valid)[0]
    ref = p[np.argsort(ids[p], kind="stable")]
    assert (order == ref).all() and on[0] == ref.size
    e_act, counts = np.unique(ids[p], return_counts=True)
    assert on[1] == e_act.size and (eg[:, 0] == e_act).all() and (eg[:, 2] == counts).all()
    assert (eg[:, 1] == np.concatenate([[0], np.cumsum(counts)[:-1]])).all()


# ------------------------------------------------------------------ the layer

@pytest.mark.parametrize("tg,td,d,ff,k", [(GType.Q4_K, GType.Q6_K, 2048, 512, 4), (GType.IQ4_NL, GType.IQ4_NL, 1024, 512, 3),
                                          (GType.IQ2_XS, GType.Q4_K, 1024, 256, 2), (GType.Q5_K, GType.IQ4_XS, 512, 512, 5)])
def test_layer_matches_fp64_recomputation(tg, td, d, ff, k):
    """CpuMoe::run_layer semantics (src/cpu_moe.cpp:668-1008): pairs in expert order, quantized activations,
    SwiGLU, re-quantized hidden, down, weighted sum -- recomputed in fp64 from the numpy decoders."""
    E, nt = 6, 3
    L = layer(tg, td, E, ff, d, seed=400 + int(tg), clamp=0.0)
    OL = oracle_layer(L)
    ids, wts = routing(nt, E, k, seed=401)
    x = torch.randn(nt, d, generator=gen(402)).numpy()
    out, h, y = orc.moe_layer(OL, x, ids, wts, want_hy=True)
    vg, vd = vec_dot_type(tg), vec_dot_type(td)
    rows_g, ks = iq2xs_rows(), ksigns()
    ref = np.zeros((nt, d))
    for t in range(nt):
        xd = orc.dequant_row(vg, orc.quantize(vg, x[t]), d).astype(np.float64)
        for j in np.argsort(ids[t], kind="stable"):
            e = ids[t, j]
            G = nf.dequant(tg, OL.gate[e], rows_g, ks).reshape(ff, d).astype(np.float64)
            U = nf.dequant(tg, OL.up[e], rows_g, ks).reshape(ff, d).astype(np.float64)
            g, u = G @ xd, U @ xd
            hh = g / (1 + np.exp(-g)) * u
            p = t * k + j
            assert np.allclose(hh, h[p], rtol=1e-5, atol=1e-5 * np.abs(hh).max())
            hd = orc.dequant_row(vd, orc.quantize(vd, h[p]), ff).astype(np.float64)   # the oracle's own h
            D = nf.dequant(td, OL.down[e], rows_g, ks).reshape(d, ff).astype(np.float64)
            yy = D @ hd
            assert np.allclose(yy, y[p], rtol=1e-5, atol=1e-5 * np.abs(yy).max())
            ref[t] += wts[t, j] * yy
    assert np.linalg.norm(out - ref) <= 1e-5 * np.linalg.norm(ref)
    # the weighted sum itself: first pair assigns w*y, later pairs add w*y, in ascending expert id
    for t in range(nt):
        acc = None
        for j in np.argsort(ids[t], kind="stable"):
            v = (wts[t, j] * y[t * k + j]).astype(np.float32)
            acc = v if acc is None else (acc + v).astype(np.float32)
        assert (acc == out[t]).all()


def test_layer_close_to_unquantized_math():
    """Q8 activations cost well under 3 % relative L2 against fp64 math on fp32 activations."""
    E, d, ff, k, nt = 4, 2048, 512, 2, 2
    L = layer(GType.Q4_K, GType.Q4_K, E, ff, d, seed=500)
    OL = oracle_layer(L)
    ids, wts = routing(nt, E, k, seed=501)
    x = torch.randn(nt, d, generator=gen(502)).numpy()
    out = orc.moe_layer(OL, x, ids, wts)
    ref = np.zeros((nt, d))
    for t in range(nt):
        for j in range(k):
            e = ids[t, j]
            G = nf.dequant(GType.Q4_K, OL.gate[e]).reshape(ff, d).astype(np.float64)
            U = nf.dequant(GType.Q4_K, OL.up[e]).reshape(ff, d).astype(np.float64)
            D = nf.dequant(GType.Q4_K, OL.down[e]).reshape(d, ff).astype(np.float64)
            g, u = G @ x[t], U @ x[t]
            ref[t] += wts[t, j] * (D @ (g / (1 + np.exp(-g)) * u))
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 0.03


def test_shared_expert_and_garbage_ids():
    E, d, ff, k, nt = 5, 512, 256, 2, 3
    L = layer(GType.Q4_K, GType.Q4_K, E, ff, d, seed=600)
    S = layer(GType.Q4_K, GType.Q4_K, 1, ff, d, seed=601)
    OL, OS = oracle_layer(L), oracle_layer(S)
    ids = np.array([[0, 3], [4, -1], [7, 2]], np.int32)          # -1 and 7 (>= E) are skipped
    wts = np.full((nt, k), 0.5, np.float32)
    x = torch.randn(nt, d, generator=gen(602)).numpy()
    sg = np.float32([0.25, 1.0, 0.75])
    out = orc.moe_layer(OL, x, ids, wts, shared=OS, sg=sg)
    _, ysh = orc.expert_ffn(OS, 0, x)
    _, _, y = orc.moe_layer(OL, x, ids, wts, want_hy=True)
    for t in range(nt):
        acc = (sg[t] * ysh[t]).astype(np.float32)
        for j in np.argsort(ids[t], kind="stable"):
            if 0 <= ids[t, j] < E:
                acc = (acc + (wts[t, j] * y[t * k + j]).astype(np.float32)).astype(np.float32)
        assert (acc == out[t]).all()
