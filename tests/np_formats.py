"""Independent numpy decoders of the GGUF block formats, written from the reference's deq8<T> layouts
(src/kernels4.cu:421-714) in vectorised numpy -- a second implementation the C oracle is checked against.

Each decoder returns the block's integer structure: quant values q [nb, 256 or 32] as the dot products use
them (Q6_K: q6 - 32; IQ4: codebook values; IQ2_XS: signed grid values), the per-group integer scales
(group size 32 or 16) and mins, and the fp16 scale fields as float32.
"""
import numpy as np

KV_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int64)


def f16(b2):
    return np.ascontiguousarray(b2).view(np.float16).astype(np.float32).reshape(-1)


def _scale_min_k4(s):      # s: [nb, 12] -> sc, m [nb, 8] (src/kernels4.cu:423-426)
    s = s.astype(np.int64)
    sc, m = np.zeros((s.shape[0], 8), np.int64), np.zeros((s.shape[0], 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def q4k(b):
    b = b.reshape(-1, 144)
    sc, m = _scale_min_k4(b[:, 4:16])
    qs = b[:, 16:144].astype(np.int64).reshape(-1, 4, 32)          # 4 pairs of sub-blocks
    q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 256)       # sub-block 2p: low, 2p+1: high
    return dict(q=q, sc=sc, m=m, gsize=32, d=f16(b[:, 0:2]), dmin=f16(b[:, 2:4]))


def q5k(b):
    b = b.reshape(-1, 176)
    sc, m = _scale_min_k4(b[:, 4:16])
    qh = b[:, 16:48].astype(np.int64)                                 # [nb, 32]: bit j -> sub-block j
    qs = b[:, 48:176].astype(np.int64).reshape(-1, 4, 32)
    lo = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32)
    hb = np.stack([(qh >> j) & 1 for j in range(8)], axis=1)          # [nb, 8, 32]
    q = (lo | (hb << 4)).reshape(-1, 256)
    return dict(q=q, sc=sc, m=m, gsize=32, d=f16(b[:, 0:2]), dmin=f16(b[:, 2:4]))


def q6k(b):
    b = b.reshape(-1, 210)
    ql = b[:, 0:128].astype(np.int64).reshape(-1, 2, 2, 32)           # [half][qt & 1][l]
    qh = b[:, 128:192].astype(np.int64).reshape(-1, 2, 32)            # [half][l]
    q = np.zeros((b.shape[0], 2, 4, 32), np.int64)                    # [half][qt][l]
    for qt in range(4):
        lo = (ql[:, :, qt & 1, :] >> (4 if qt >= 2 else 0)) & 0xF
        q[:, :, qt, :] = lo | (((qh >> (2 * qt)) & 3) << 4)
    q = q.reshape(-1, 256) - 32
    sc = b[:, 192:208].view(np.int8).astype(np.int64)                  # group e // 16
    return dict(q=q, sc=sc, m=None, gsize=16, d=f16(b[:, 208:210]))


def iq4xs(b):
    b = b.reshape(-1, 136)
    sh = b[:, 2].astype(np.int64) | (b[:, 3].astype(np.int64) << 8)
    sl = b[:, 4:8].astype(np.int64)
    ls = np.stack([((sl[:, ib // 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4) for ib in range(8)], axis=1)
    qs = b[:, 8:136].astype(np.int64).reshape(-1, 8, 16)
    idx = np.concatenate([qs & 0xF, qs >> 4], axis=2).reshape(-1, 256)
    return dict(q=KV_IQ4NL[idx], sc=ls - 32, m=None, gsize=32, d=f16(b[:, 0:2]))


def iq4nl(b):
    b = b.reshape(-1, 18)
    qs = b[:, 2:18].astype(np.int64)
    idx = np.concatenate([qs & 0xF, qs >> 4], axis=1)
    return dict(q=KV_IQ4NL[idx], sc=np.ones((b.shape[0], 1), np.int64), m=None, gsize=32, d=f16(b[:, 0:2]))


def q8_0w(b):
    """Q8_0 weights: d f16 @0, qs int8[32] @2 (deq8: d * qs[j])."""
    b = b.reshape(-1, 34)
    return dict(q=b[:, 2:34].view(np.int8).astype(np.int64), sc=np.ones((b.shape[0], 1), np.int64), m=None, gsize=32,
                d=f16(b[:, 0:2]))


def e2m1_doubled(idx):
    """Twice the value of an E2M1 (OCP MX fp4) code: sign bit 3, exponent bits 2-1 (bias 1), mantissa bit 0;
    exponent 0 is subnormal (m / 2), else 2^(e - 1) (1 + m / 2)."""
    idx = np.asarray(idx, np.int64)
    s, e, m = (idx >> 3) & 1, (idx >> 1) & 3, idx & 1
    mag = np.where(e == 0, m * 0.5, np.ldexp(1.0 + m * 0.5, (e - 1).astype(np.int32)))
    return (np.where(s == 1, -1, 1) * 2 * mag).astype(np.int64)


def e8m0_half(e):
    """Half of the E8M0 (OCP MX) scale 2^(e - 127), as float32 (2^-128 and 2^-127 are fp32 subnormals)."""
    return np.ldexp(np.float64(1.0), np.asarray(e, np.int32) - 128).astype(np.float32)


def mxfp4(b):
    """MXFP4 weights: E8M0 exponent @0, qs[16] @1; value j < 16 from the low nibble of qs[j], 16 + j from its high
    nibble; scale e8m0_half(e), values the doubled E2M1 codes."""
    b = b.reshape(-1, 17)
    qs = b[:, 1:17].astype(np.int64)
    idx = np.concatenate([qs & 0xF, qs >> 4], axis=1)
    return dict(q=e2m1_doubled(idx), sc=np.ones((b.shape[0], 1), np.int64), m=None, gsize=32, d=e8m0_half(b[:, 0]))


def q2k(b):
    """Q2_K: scales[16] @0 (16-group g: scale = low nibble, min = high nibble), qs[64] @16, d @80, dmin @82.  Value
    128 h + 32 j + l (h < 2, j < 4, l < 32) is bits 2 j .. 2 j + 1 of qs byte 32 h + l."""
    b = b.reshape(-1, 84)
    qs = b[:, 16:80].astype(np.int64).reshape(-1, 2, 1, 32)                       # [h][.][l]
    q = ((qs >> (2 * np.arange(4)).reshape(1, 1, 4, 1)) & 3).reshape(-1, 256)      # [h][j][l] -> value order
    s = b[:, 0:16].astype(np.int64)
    return dict(q=q, sc=s & 15, m=s >> 4, gsize=16, d=f16(b[:, 80:82]), dmin=f16(b[:, 82:84]))


def q3k(b):
    """Q3_K in ggml's block_q3_K terms: hmask[32], qs[64], scales[12], d.  Sub-block s = 0..7 of 32 values uses bit s
    of hmask[l] and bits 2 (s % 4) of qs[32 (s // 4) + l]; value = q - (4 if the hmask bit is clear); 16-group i's
    scale is the low (i < 8) or high (i >= 8) nibble of scales[i % 8] with bits 2 (i // 4) of scales[8 + i % 4] on top,
    less 32."""
    b = b.reshape(-1, 110)
    hm = b[:, 0:32].astype(np.int64)
    qs = b[:, 32:96].astype(np.int64).reshape(-1, 2, 32)
    vals = []
    for s in range(8):
        q = (qs[:, s // 4, :] >> (2 * (s % 4))) & 3
        vals.append(q - 4 * (1 - ((hm >> s) & 1)))
    s = b[:, 96:108].astype(np.int64)
    sc = np.stack([((s[:, i % 8] >> (4 * (i // 8))) & 15) | (((s[:, 8 + i % 4] >> (2 * (i // 4))) & 3) << 4)
                   for i in range(16)], axis=1) - 32
    return dict(q=np.concatenate(vals, axis=1), sc=sc, m=None, gsize=16, d=f16(b[:, 108:110]))


def iq3xxs(b, grid_rows, ksigns):
    """grid_rows: [256, 4] codebook bytes, ksigns: [128] sign bytes.  32-group ib: eight grid indices at 2 + 8 ib
    (8-group l: rows 2 l and 2 l + 1, four values each), then a little-endian word at 66 + 4 ib with the four 7-bit sign
    indices (bits 7 l ..) and the 4-bit scale (bits 28 ..)."""
    b = b.reshape(-1, 98)
    idx = b[:, 2:66].astype(np.int64).reshape(-1, 8, 4, 2)                       # [ib][l][half]
    g = grid_rows[idx].astype(np.int64).reshape(-1, 8, 4, 8)                     # [ib][l][8 values]
    a = np.ascontiguousarray(b[:, 66:98]).view(np.uint32).astype(np.int64).reshape(-1, 8)
    sgn = ksigns[np.stack([(a >> (7 * l)) & 127 for l in range(4)], axis=2)].astype(np.int64)
    bits = (sgn[..., None] >> np.arange(8)) & 1
    q = np.where(bits == 1, -g, g).reshape(-1, 256)
    return dict(q=q, sc=2 * (a >> 28) + 1, m=None, gsize=32, d=f16(b[:, 0:2]))


def iq3s(b, grid_rows):
    """grid_rows: [512, 4] codebook bytes.  32-group ib: eight indices at 2 + 8 ib, their 9th bits in qh[ib] (@66, bit
    k for index k), four literal sign bytes at 74 + 4 ib (bit j negates value j of the 8-group), scale nibble ib % 2 of
    scales[ib // 2] (@106), the group's factor 2 sc + 1."""
    b = b.reshape(-1, 110)
    qh = b[:, 66:74].astype(np.int64)                                           # [ib]
    idx = b[:, 2:66].astype(np.int64).reshape(-1, 8, 8) | (((qh[:, :, None] >> np.arange(8)) & 1) << 8)
    g = grid_rows[idx].astype(np.int64).reshape(-1, 8, 4, 8)                    # [ib][l][8 values]
    sgn = b[:, 74:106].astype(np.int64).reshape(-1, 8, 4)
    bits = (sgn[..., None] >> np.arange(8)) & 1
    q = np.where(bits == 1, -g, g).reshape(-1, 256)
    s = b[:, 106:110].astype(np.int64)
    sc = np.stack([(s[:, ib // 2] >> (4 * (ib % 2))) & 15 for ib in range(8)], axis=1)
    return dict(q=q, sc=2 * sc + 1, m=None, gsize=32, d=f16(b[:, 0:2]))


def iq2s(b, grid_rows):
    """grid_rows: [1024, 8] codebook bytes.  32-group ib: four index bytes at 2 + 4 ib with two more bits each in
    qh[ib] (@66, bits 2 l, 2 l + 1 for 8-group l), four literal sign bytes at 34 + 4 ib, scale nibbles of scales[ib]
    (@74) for its two 16-groups, each 2 sc + 1."""
    b = b.reshape(-1, 82)
    qh = b[:, 66:74].astype(np.int64)
    idx = b[:, 2:34].astype(np.int64).reshape(-1, 8, 4) | (((qh[:, :, None] >> (2 * np.arange(4))) & 3) << 8)
    g = grid_rows[idx].astype(np.int64)                                           # [ib][l][8]
    sgn = b[:, 34:66].astype(np.int64).reshape(-1, 8, 4)
    bits = (sgn[..., None] >> np.arange(8)) & 1
    q = np.where(bits == 1, -g, g).reshape(-1, 256)
    s = b[:, 74:82].astype(np.int64)
    sc = np.stack([s & 15, s >> 4], axis=2).reshape(-1, 16)
    return dict(q=q, sc=2 * sc + 1, m=None, gsize=16, d=f16(b[:, 0:2]))


def iq1s(b, grid_rows):
    """grid_rows: [2048, 8] int8 codebook values.  32-group ib: four index bytes at 2 + 4 ib, the little-endian qh[ib]
    at 34 + 2 ib: bits 3 l .. 3 l + 2 are index bits 8-10 of 8-group l, bits 12-14 the scale s (factor 2 s + 1), bit 15
    the delta's sign (-1/8 if set).  m carries factor * sign, the weight of the group's activation sum."""
    b = b.reshape(-1, 50)
    qh = np.ascontiguousarray(b[:, 34:50]).view(np.uint16).astype(np.int64).reshape(-1, 8)
    idx = b[:, 2:34].astype(np.int64).reshape(-1, 8, 4) | (((qh[:, :, None] >> (3 * np.arange(4))) & 7) << 8)
    q = grid_rows[idx].astype(np.int64).reshape(-1, 256)
    ls = 2 * ((qh >> 12) & 7) + 1
    sgn = np.where(qh & 0x8000, -1, 1)
    return dict(q=q, sc=ls, m=ls * sgn, gsize=32, d=f16(b[:, 0:2]), delta=np.where(qh & 0x8000, -0.125, 0.125))


def q5_1w(b):
    """Q5_1 weights: d f16 @0, m f16 @2, qh little-endian u32 @4, qs[16] @8; value j = d (nibble j + 16 bit j) + m."""
    b = b.reshape(-1, 24)
    qh = np.ascontiguousarray(b[:, 4:8]).view(np.uint32).astype(np.int64).reshape(-1)
    qs = b[:, 8:24].astype(np.int64)
    x = np.concatenate([qs & 0xF, qs >> 4], axis=1) + 16 * ((qh[:, None] >> np.arange(32)) & 1)
    return dict(q=x, sc=np.ones((b.shape[0], 1), np.int64), m=np.ones((b.shape[0], 1), np.int64), gsize=32,
                d=f16(b[:, 0:2]), dmin=f16(b[:, 2:4]))


def q5_0w(b):
    """Q5_0 weights: d f16 @0, qh little-endian u32 @2, qs[16] @6; value j = (nibble j + 16 * bit j of qh) - 16, the
    nibbles in qs order, low halves first (values 0..15), then high halves (16..31)."""
    b = b.reshape(-1, 22)
    qh = np.ascontiguousarray(b[:, 2:6]).view(np.uint32).astype(np.int64).reshape(-1)
    qs = b[:, 6:22].astype(np.int64)
    nib = np.concatenate([qs & 0xF, qs >> 4], axis=1)
    hi = (qh[:, None] >> np.arange(32)) & 1
    return dict(q=nib + 16 * hi - 16, sc=np.ones((b.shape[0], 1), np.int64), m=None, gsize=32, d=f16(b[:, 0:2]))


def iq2xs(b, grid_rows, ksigns):
    """grid_rows: [512, 8] codebook bytes, ksigns: [128] sign bytes."""
    b = b.reshape(-1, 74)
    qs = b[:, 2:66].copy().view(np.uint16).astype(np.int64).reshape(-1, 8, 4)     # [ib][l]
    g = grid_rows[qs & 511].astype(np.int64)                                       # [nb, 8, 4, 8]
    sgn = ksigns[qs >> 9].astype(np.int64)
    bits = (sgn[..., None] >> np.arange(8)) & 1
    q = np.where(bits == 1, -g, g).reshape(-1, 256)
    s = b[:, 66:74].astype(np.int64)
    sc = np.stack([s & 0xF, s >> 4], axis=2).reshape(-1, 16)                       # 16-groups
    return dict(q=q, sc=2 * sc + 1, m=None, gsize=16, d=f16(b[:, 0:2]))


def iq2xxs(b, grid_rows, ksigns):
    """grid_rows: [256, 8] codebook bytes, ksigns: [128] sign bytes.  32-group ib: grid rows at bytes 2 + 8 ib + l,
    then a little-endian word with the four 7-bit sign indices (bits 7 l ..) and the 4-bit scale (bits 28 ..)."""
    b = b.reshape(-1, 66)
    w = b[:, 2:66].reshape(-1, 8, 8)
    g = grid_rows[w[:, :, 0:4].astype(np.int64)].astype(np.int64)                   # [nb, 8, 4, 8]
    a1 = np.ascontiguousarray(w[:, :, 4:8]).view(np.uint32).astype(np.int64).reshape(-1, 8)
    sgn = ksigns[np.stack([(a1 >> (7 * l)) & 127 for l in range(4)], axis=2)].astype(np.int64)
    bits = (sgn[..., None] >> np.arange(8)) & 1
    q = np.where(bits == 1, -g, g).reshape(-1, 256)
    return dict(q=q, sc=2 * (a1 >> 28) + 1, m=None, gsize=32, d=f16(b[:, 0:2]))


def q8k(b):
    b = b.reshape(-1, 292)
    return dict(d=b[:, 0:4].copy().view(np.float32).reshape(-1), qs=b[:, 4:260].view(np.int8).astype(np.int64),
                bsums=b[:, 260:292].copy().view(np.int16).astype(np.int64))


def q8_0(b):
    b = b.reshape(-1, 34)
    return dict(d=f16(b[:, 0:2]), qs=b[:, 2:34].view(np.int8).astype(np.int64))


def decode(t, b, grid_rows=None, ksigns=None):
    t = int(t)
    if t == 12: return q4k(b)
    if t == 13: return q5k(b)
    if t == 14: return q6k(b)
    if t == 23: return iq4xs(b)
    if t == 20: return iq4nl(b)
    if t == 8: return q8_0w(b)
    if t == 39: return mxfp4(b)
    if t == 6: return q5_0w(b)
    if t == 7: return q5_1w(b)
    if t == 10: return q2k(b)
    if t == 11: return q3k(b)
    if t == 18: return iq3xxs(b, grid_rows, ksigns)
    if t == 21: return iq3s(b, grid_rows)
    if t == 22: return iq2s(b, grid_rows)
    if t == 19: return iq1s(b, grid_rows)
    if t == 17: return iq2xs(b, grid_rows, ksigns)
    if t == 16: return iq2xxs(b, grid_rows, ksigns)
    raise ValueError(t)


def dequant(t, b, grid_rows=None, ksigns=None):
    """float32 values with the deq8 expression order (each product rounded on its own)."""
    f = decode(t, b, grid_rows, ksigns)
    q, gs = f["q"], f["gsize"]
    n = q.shape[1]
    sc = np.repeat(f["sc"], gs, axis=1)[:, :n].astype(np.float32)
    d = f["d"][:, None]
    t = int(t)
    if t in (12, 13, 10):
        m = np.repeat(f["m"], gs, axis=1).astype(np.float32)
        return ((d * sc) * q.astype(np.float32) - f["dmin"][:, None] * m).astype(np.float32)
    if t in (14, 11):
        return ((d * sc) * q.astype(np.float32)).astype(np.float32)
    if t == 23:
        return ((d * sc) * q.astype(np.float32)).astype(np.float32)
    if t == 7:
        return (q.astype(np.float32) * d + f["dmin"][:, None]).astype(np.float32)
    if t in (20, 39, 6):
        return (q.astype(np.float32) * d).astype(np.float32)
    if t == 8:
        return (d * q.astype(np.float32)).astype(np.float32)
    if t == 19:   # d (2 s + 1) (grid + delta)
        dl = (d * sc).astype(np.float32)
        delta = np.repeat(f["delta"], gs, axis=1).astype(np.float32)
        return (dl * (q.astype(np.float32) + delta)).astype(np.float32)
    if t == 21:   # d (2 sc + 1), then times the grid byte, then the sign
        db = (d * sc.astype(np.float32)).astype(np.float32)
        return ((db * np.abs(q).astype(np.float32)) * np.where(q < 0, np.float32(-1), np.float32(1))).astype(np.float32)
    if t in (16, 17, 18, 22):
        db = (d * (np.float32(0.5) + ((sc - 1) / 2).astype(np.float32))) * np.float32(0.5 if t == 18 else 0.25)
        return ((db * np.abs(q).astype(np.float32)) * np.where(q < 0, np.float32(-1), np.float32(1))).astype(np.float32)
    raise ValueError(t)


def block_ints(t, b, xq, grid_rows=None, ksigns=None):
    """Brute-force integers per block: sumi = sum over groups of scale * sum(q * y), summ = sum_j m_j * sum(y_j)."""
    f = decode(t, b, grid_rows, ksigns)
    q, gs = f["q"], f["gsize"]
    if int(t) in (20, 8, 39, 6, 7):
        y = q8_0(xq)["qs"]
    else:
        y = q8k(xq)["qs"]
    prod = (q * y).reshape(q.shape[0], -1, gs).sum(axis=2)            # per group
    sumi = (prod * f["sc"]).sum(axis=1)
    if f["m"] is not None:
        summ = (f["m"] * y.reshape(y.shape[0], -1, gs).sum(axis=2)).sum(axis=1)
    else:
        summ = np.zeros_like(sumi)
    return sumi, summ
