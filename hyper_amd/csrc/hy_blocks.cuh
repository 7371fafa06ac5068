// Per-type block decoding for the integer dot products.
//
// Decode GEMV mapping: a 256-value item of a weight row (one super-block, or eight IQ4_NL / Q8_0 blocks) is
// handled by 8 lanes; lane L loads a 16-byte slice of the quant bytes (coalesced: the group reads the
// item's quant bytes contiguously) and returns exact integer partial sums (sumi, summ) against the
// matching Q8 activation bytes; the 8 partials are summed exactly in integers.  Layouts follow the
// reference's deq8<T> (src/kernels4.cu:421-714).
#pragma once
#include "hy_common.cuh"

namespace hy {

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int) a, (int) b, c, false); }
__device__ __forceinline__ uint32_t byte_of(uint4 v, int i) {   // byte i (0..15) of a 16-byte vector
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xff;
}
// 6-bit scale and min of sub-block j from the 12 scale bytes held in words s0..s2 (src/kernels4.cu:423-426)
__device__ __forceinline__ void scale_min_k4(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &sc, int &mn) {
    const uint4 v = make_uint4(s0, s1, s2, 0);
    if (j < 4) { sc = byte_of(v, j) & 63; mn = byte_of(v, j + 4) & 63; }
    else { sc = (byte_of(v, j + 4) & 0xF) | ((byte_of(v, j - 4) >> 6) << 4); mn = (byte_of(v, j + 4) >> 4) | ((byte_of(v, j) >> 6) << 4); }
}
// four packed nibble indices (bytes 0..15) -> entries of a 16-byte int8 codebook T0..T3 as packed int8
__device__ __forceinline__ uint32_t kv16(uint32_t idx, uint32_t T0, uint32_t T1, uint32_t T2, uint32_t T3) {
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    // 0xFF in the bytes whose index is 8..15: selector idx >> 1 picks a byte of 0xFFFFFFFF (4..7) or of 0 (0..3)
    const uint32_t m = __builtin_amdgcn_perm(0xFFFFFFFFu, 0u, (idx >> 1) & 0x07070707u);
    return (hi & m) | (lo & ~m);
}
// the IQ4_NL codebook (bytes: -127 -104 -83 -65 | -49 -35 -22 -10 | 1 13 25 38 | 53 69 89 113)
__device__ __forceinline__ uint32_t kv4(uint32_t idx) { return kv16(idx, 0xBFAD9881u, 0xF6EADDCFu, 0x26190D01u, 0x71594535u); }
// the MXFP4 codebook, E2M1 values doubled (src/kernels4.cu:551; bytes: 0 1 2 3 | 4 6 8 12 | 0 -1 -2 -3 | -4 -6 -8 -12)
__device__ __forceinline__ uint32_t kvfp4(uint32_t idx) { return kv16(idx, 0x03020100u, 0x0C080604u, 0xFDFEFF00u, 0xF4F8FAFCu); }
// IQ2 signs: 8 sign bits -> two words whose bytes are 0xFF where negated; value = (g ^ M) + (M & 1)
__device__ __forceinline__ uint32_t spread4(uint32_t b4) { return (b4 * 0x00204081u) & 0x01010101u; }
// 0xFC in the bytes holding 1 (the others 0): OR-ed onto a 2-bit value it makes the int8 value - 4
__device__ __forceinline__ uint32_t fill_fc(uint32_t s) { return (s << 8) - (s << 2); }
// 0xF0 in the bytes whose bit is set in b4 (4 bits): OR-ed onto a nibble it makes the int8 nibble - 16
__device__ __forceinline__ uint32_t fill_f0(uint32_t b4) {
    const uint32_t s = spread4(b4);
    return (s << 8) - (s << 4);
}
__device__ __forceinline__ uint32_t apply_sign(uint32_t g, uint32_t b4) {
    const uint32_t one = spread4(b4);
    return (g ^ (one * 0xFFu)) + one;
}
// the same with the byte mask given (0xFF per negated byte): -g = ~g + 1 per byte, no carry (codebook bytes are not 0)
__device__ __forceinline__ uint32_t apply_mask(uint32_t g, uint32_t m) { return (g ^ m) + (m & 0x01010101u); }
// LDS entries of an expanded IQ2_XS codebook: 512 rows, then 128 sign masks (IQ2_XXS: 256 rows, then the masks)
__host__ __device__ constexpr int iq2_rows(int t) { return t == IQ1_S ? 2048 : t == IQ2_S ? 1024 : t == IQ2_XS || t == IQ3_S ? 512 : 256; }
// sign masks after the rows: the 128 ksign patterns, or for IQ3_S and IQ2_S (literal sign bytes) all 256 bytes
__host__ __device__ constexpr bool literal_signs(int t) { return t == IQ3_S || t == IQ2_S; }
__host__ __device__ constexpr int iq2_masks(int t) { return t == IQ1_S ? 0 : literal_signs(t) ? 256 : 128; }   // IQ1_S: no signs
__host__ __device__ constexpr int iq2_lds(int t) { return iq2_type(t) ? iq2_rows(t) + iq2_masks(t) : 1; }   // uint2 entries
constexpr int GRID_LDS = 2048;   // the largest of them (IQ1_S; IQ2_S 1024 + 256)
// Q6_K: q6 bytes (0..63) -> q6 - 32 as int8: per byte (q + 96) ^ 128 = q - 32 mod 256 (q + 96 < 256: no carry)
__device__ __forceinline__ uint32_t q6_signed(uint32_t q) { return (q + 0x60606060u) ^ 0x80808080u; }

// ---------------------------------------------------------------- decode-GEMV items (8 lanes)
template <int T> struct Item;

// Q4_K (144 B: d, dmin, scales[12], qs[128]).  Lane L: qs bytes 16 L .. 16 L + 15 = values 16 (L & 1) ..
// of sub-blocks 2 (L >> 1) (low nibbles) and 2 (L >> 1) + 1 (high nibbles).
template <> struct Item<Q4_K> {
    uint4 hd, qs;
    __device__ __forceinline__ void load(const uint8_t *b, int L) { hd = load16_a4(b); qs = load16_a4(b + 16 + 16 * L); }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const int c = L >> 1, hh = L & 1;
        int sc0, m0, sc1, m1;
        scale_min_k4(hd.y, hd.z, hd.w, 2 * c, sc0, m0);
        scale_min_k4(hd.y, hd.z, hd.w, 2 * c + 1, sc1, m1);
        const uint32_t *ya = (const uint32_t *) (y + 4 + 64 * c + 16 * hh), *yb = (const uint32_t *) (y + 4 + 64 * c + 32 + 16 * hh);
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) { sa = sdot4(q[i] & 0x0F0F0F0Fu, ya[i], sa); sb = sdot4((q[i] >> 4) & 0x0F0F0F0Fu, yb[i], sb); }
        const int16_t *bs = (const int16_t *) (y + 260);
        si = __mul24(sc0, sa) + __mul24(sc1, sb);   // 24-bit products, exact here: |sa| < 2^16, scales 6-bit
        sm = __mul24(m0, bs[4 * c + hh]) + __mul24(m1, bs[4 * c + 2 + hh]);
    }
    __device__ __forceinline__ float tval(int si, int sm) const {
        return __builtin_fmaf(h2f(hd.x & 0xffff), (float) si, -(h2f(hd.x >> 16) * (float) sm));
    }
};
// Q5_K (176 B: d, dmin, scales[12], qh[32], qs[128]): as Q4_K, bit j of qh[l] is bit 4 of sub-block j's value l.
template <> struct Item<Q5_K> {
    uint4 hd, qh, qs;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        hd = load16_a4(b); qh = load16_a4(b + 16 + 16 * (L & 1)); qs = load16_a4(b + 48 + 16 * L);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const int c = L >> 1, hh = L & 1;
        int sc0, m0, sc1, m1;
        scale_min_k4(hd.y, hd.z, hd.w, 2 * c, sc0, m0);
        scale_min_k4(hd.y, hd.z, hd.w, 2 * c + 1, sc1, m1);
        const uint32_t *ya = (const uint32_t *) (y + 4 + 64 * c + 16 * hh), *yb = (const uint32_t *) (y + 4 + 64 * c + 32 + 16 * hh);
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w}, h[4] = {qh.x, qh.y, qh.z, qh.w};
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (((h[i] >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            sa = sdot4(lo, ya[i], sa); sb = sdot4(hi, yb[i], sb);
        }
        const int16_t *bs = (const int16_t *) (y + 260);
        si = __mul24(sc0, sa) + __mul24(sc1, sb);   // 24-bit products, exact here: |sa| < 2^16, scales 6-bit
        sm = __mul24(m0, bs[4 * c + hh]) + __mul24(m1, bs[4 * c + 2 + hh]);
    }
    __device__ __forceinline__ float tval(int si, int sm) const {
        return __builtin_fmaf(h2f(hd.x & 0xffff), (float) si, -(h2f(hd.x >> 16) * (float) sm));
    }
};
// Q2_K (84 B: scales[16] @0, qs[64] @16, d @80, dmin @82), src/kernels4.cu:639-647.  Value e is the 2-bit field
// 2 ((e >> 5) & 3) of qs byte 32 (e >> 7) + (e & 31); 16-group g = e >> 4 has scale byte g (low nibble the scale, high
// nibble the min).  Lane L = 32-group L: 32 qs bytes at 16 + 32 (L >> 2), shift 2 (L & 3), 16-groups 2 L and 2 L + 1
// (ggml's vec_dot_q2_K_q8_K integers: sumi = sum_g sc_g sum_16 q y, summ = sum_g m_g bsum_g).  Blocks are 4-byte
// aligned (84-byte rows).
template <> struct Item<Q2_K> {
    uint4 q0, q1;
    uint32_t dm, scm;   // d | dmin << 16; the lane's two scale bytes
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        q0 = load16_a4(b + 16 + 32 * (L >> 2));
        q1 = load16_a4(b + 32 + 32 * (L >> 2));
        dm = *(const uint32_t *) (b + 80);
        scm = ld_u16(b + 2 * L);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const int sh = 2 * (L & 3);
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sa = sdot4((q[i] >> sh) & 0x03030303u, ya[i], sa);
            sb = sdot4((q[4 + i] >> sh) & 0x03030303u, ya[4 + i], sb);
        }
        const int16_t *bs = (const int16_t *) (y + 260);
        si = (int) (scm & 15) * sa + (int) ((scm >> 8) & 15) * sb;
        sm = (int) ((scm >> 4) & 15) * bs[2 * L] + (int) (scm >> 12) * bs[2 * L + 1];
    }
    __device__ __forceinline__ float tval(int si, int sm) const {
        return __builtin_fmaf(h2f(dm & 0xffff), (float) si, -(h2f(dm >> 16) * (float) sm));
    }
};
// IQ3_XXS (98 B: d, qs[64] @2, scales_and_signs u32[8] @66), src/kernels4.cu:613-627.  Lane L = 32-group L: grid
// indices qs[8 L + 2 l], qs[8 L + 2 l + 1] (4-byte rows, values 0-3 and 4-7 of 8-group l), the word at 66 + 4 L holding
// the four 7-bit sign indices (bits 7 l ..) and the 4-bit scale (bits 28 ..); value d (2 sc + 1) / 4 grid sign
// (ggml's vec_dot_iq3_xxs_q8_K integers: sumi = sum_ib (2 sc + 1) sum_32 grid sign y).  Blocks are 2-byte aligned.
template <> struct Item<IQ3_XXS> {
    uint32_t g0, g1, a;   // the lane's 8 index bytes; its scale/sign word
    uint16_t d;
    const uint2 *grid;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        const uint8_t *p = b + 2 + 8 * L;
        g0 = (uint32_t) ld_u16(p) | ((uint32_t) ld_u16(p + 2) << 16);
        g1 = (uint32_t) ld_u16(p + 4) | ((uint32_t) ld_u16(p + 6) << 16);
        a = (uint32_t) ld_u16(b + 66 + 4 * L) | ((uint32_t) ld_u16(b + 68 + 4 * L) << 16);
        d = ld_u16(b);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        int s = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t gw = l < 2 ? g0 : g1, sh = 16 * (l & 1);
            const uint2 m = grid[256 + ((a >> (7 * l)) & 127)];
            s = sdot4(apply_mask(grid[(gw >> sh) & 255].x, m.x), ya[2 * l], s);
            s = sdot4(apply_mask(grid[(gw >> (sh + 8)) & 255].x, m.y), ya[2 * l + 1], s);
        }
        si = (2 * (int) (a >> 28) + 1) * s;
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return (h2f(d) * 0.25f) * (float) si; }
};
// IQ1_S (50 B: d, qs[32] @2, qh u16[8] @34), src/kernels4.cu:650-659.  Lane L = 32-group L: 8-group l takes grid row
// qs[4 L + l] | 3 bits (3 l) of qh[L] << 8 (8 int8 values in {-1, 0, 1}), scale ls = 2 ((qh >> 12) & 7) + 1 and delta
// +-1/8 by qh's top bit: value d ls (grid + delta).  The integers of the reference's own IQ1_S x Q8_K dot
// (src/iq1s_dot.h:26-64): sumi = sum_ib ls sum_32 grid y, summ = sum_ib ls (-1 if the top bit) (bsum pair of ib);
// folded as (d / 8) (8 sumi + summ), an exact integer times a power-of-two scaled d.  Blocks are 2-byte aligned.
template <> struct Item<IQ1_S> {
    uint32_t gq, qh;   // the lane's 4 index bytes; its qh halfword
    uint16_t d;
    const uint2 *grid;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        gq = (uint32_t) ld_u16(b + 2 + 4 * L) | ((uint32_t) ld_u16(b + 4 + 4 * L) << 16);
        qh = ld_u16(b + 34 + 2 * L);
        d = ld_u16(b);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        int s = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint2 g = grid[((gq >> (8 * l)) & 255) | (((qh >> (3 * l)) & 7) << 8)];
            s = sdot4(g.y, ya[2 * l + 1], sdot4(g.x, ya[2 * l], s));
        }
        const int ls = 2 * (int) ((qh >> 12) & 7) + 1;
        const int16_t *bs = (const int16_t *) (y + 260);
        si = ls * s;
        sm = (qh & 0x8000 ? -ls : ls) * (bs[2 * L] + bs[2 * L + 1]);
    }
    __device__ __forceinline__ float tval(int si, int sm) const { return (h2f(d) * 0.125f) * (float) (8 * si + sm); }
};
// IQ2_S (82 B: d, qs[32] @2, signs[32] @34, qh[8] @66, scales[8] @74), src/kernels4.cu:602-613.  Lane L = 32-group
// L: 8-group l takes grid row qs[4 L + l] | bits 2 l, 2 l + 1 of qh[L] << 8 (8-byte rows of the 1024-row codebook),
// sign byte signs[4 L + l] (bit j negates value j), the scale nibble l / 2 of scales[L] (16-groups) (ggml's
// vec_dot_iq2_s_q8_K integers: sumi = sum over 16-groups (2 sc + 1) sum_16 grid sign y).  Blocks are 2-byte aligned.
template <> struct Item<IQ2_S> {
    uint32_t gq, sg, hs;   // the lane's 4 index bytes; its 4 sign bytes; qh byte | scale byte << 8
    uint16_t d;
    const uint2 *grid;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        gq = (uint32_t) ld_u16(b + 2 + 4 * L) | ((uint32_t) ld_u16(b + 4 + 4 * L) << 16);
        sg = (uint32_t) ld_u16(b + 34 + 4 * L) | ((uint32_t) ld_u16(b + 36 + 4 * L) << 16);
        hs = (uint32_t) b[66 + L] | ((uint32_t) b[74 + L] << 8);
        d = ld_u16(b);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        int s[4];
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint2 g = grid[((gq >> (8 * l)) & 255) | (((hs >> (2 * l)) & 3) << 8)], m = grid[1024 + ((sg >> (8 * l)) & 255)];
            s[l] = sdot4(apply_mask(g.y, m.y), ya[2 * l + 1], sdot4(apply_mask(g.x, m.x), ya[2 * l], 0));
        }
        si = (2 * (int) ((hs >> 8) & 15) + 1) * (s[0] + s[1]) + (2 * (int) ((hs >> 12) & 15) + 1) * (s[2] + s[3]);
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return (h2f(d) * 0.125f) * (float) si; }
};
// IQ3_S (110 B: d, qs[64] @2, qh[8] @66, signs[32] @74, scales[4] @106), src/kernels4.cu:682-695.  Lane L = 32-group
// L: 8-group l takes grid rows qs[8 L + 2 l] | bit 2 l of qh[L] << 8 and qs[8 L + 2 l + 1] | bit 2 l + 1 << 8 (4-byte
// rows of the 512-row codebook), sign byte signs[4 L + l] (bit j negates value j), scale 2 sc + 1 with sc nibble L & 1
// of scales[L / 2] (the integers of the reference's own IQ3_S x Q8_K dot, src/iq3s_dot.h:48-76: sumi = sum_ib
// (2 sc + 1) sum_32 grid sign y).  Blocks are 2-byte aligned (110-byte rows).
template <> struct Item<IQ3_S> {
    uint32_t g0, g1, sg, hs;   // the lane's 8 index bytes; its 4 sign bytes; qh byte | scale nibble << 8
    uint16_t d;
    const uint2 *grid;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        const uint8_t *p = b + 2 + 8 * L;
        g0 = (uint32_t) ld_u16(p) | ((uint32_t) ld_u16(p + 2) << 16);
        g1 = (uint32_t) ld_u16(p + 4) | ((uint32_t) ld_u16(p + 6) << 16);
        sg = (uint32_t) ld_u16(b + 74 + 4 * L) | ((uint32_t) ld_u16(b + 76 + 4 * L) << 16);
        hs = (uint32_t) b[66 + L] | ((uint32_t) ((b[106 + (L >> 1)] >> (4 * (L & 1))) & 15) << 8);
        d = ld_u16(b);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        int s = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t gw = l < 2 ? g0 : g1, sh = 16 * (l & 1);
            const uint32_t i1 = ((gw >> sh) & 255) | (((hs >> (2 * l)) & 1) << 8), i2 = ((gw >> (sh + 8)) & 255) | (((hs >> (2 * l + 1)) & 1) << 8);
            const uint2 m = grid[512 + ((sg >> (8 * l)) & 255)];
            s = sdot4(apply_mask(grid[i1].x, m.x), ya[2 * l], s);
            s = sdot4(apply_mask(grid[i2].x, m.y), ya[2 * l + 1], s);
        }
        si = (2 * (int) (hs >> 8) + 1) * s;
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return h2f(d) * (float) si; }
};
// Q3_K (110 B: hmask[32] @0, qs[64] @32, scales[12] @96, d @108), src/kernels4.cu:698-707.  Value e = 128 hf + 32 j + l
// is the 2-bit field 2 j of qs byte 32 hf + l, less 4 where bit 4 hf + j of hmask[l] is clear; 16-group is = e >> 4
// has the signed 6-bit scale (scales[is & 7] >> 4 (is >> 3) & 15 | (scales[8 + (is & 3)] >> 2 (is >> 2) & 3) << 4) - 32.
// Lane L = 32-group L (hf = L >> 2, j = L & 3), 16-groups 2 L and 2 L + 1: sum (q | h << 2) y less 4 bsum per group
// (ggml's vec_dot_q3_K_q8_K integers: sumi = sum_g sc_g sum_16 (q - 4 (1 - h)) y).  Blocks are 2-byte aligned
// (110-byte rows); every 16-byte read ends by byte 97.
template <> struct Item<Q3_K> {
    Raw32 qr, hr;      // the lane's 32 quant bytes and the block's 32 high-bit bytes
    uint32_t sl, sh;   // the two 16-groups' low-nibble bytes and high-bit bytes
    uint16_t d;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        const int hf = L >> 2, grp = L >> 1, k = 2 * (L & 1);
        qr.load(b + 32 + 32 * hf);
        hr.load(b);
        sl = ld_u16(b + 96 + 4 * (grp & 1) + k);
        sh = ld_u16(b + 104 + k);
        d = ld_u16(b + 108);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const int hf = L >> 2, j = L & 3, grp = L >> 1, s2 = 2 * j, hb = 4 * hf + j;
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        const uint4 q0 = qr.lo(), q1 = qr.hi(), h0 = hr.lo(), h1 = hr.hi();
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w}, h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sa = sdot4(((q[i] >> s2) & 0x03030303u) | (((h[i] >> hb) & 0x01010101u) << 2), ya[i], sa);
            sb = sdot4(((q[4 + i] >> s2) & 0x03030303u) | (((h[4 + i] >> hb) & 0x01010101u) << 2), ya[4 + i], sb);
        }
        const int16_t *bs = (const int16_t *) (y + 260);
        const int sc0 = (int) (((sl >> (4 * (grp >> 1))) & 15) | (((sh >> (2 * grp)) & 3) << 4)) - 32;
        const int sc1 = (int) (((sl >> (8 + 4 * (grp >> 1))) & 15) | (((sh >> (8 + 2 * grp)) & 3) << 4)) - 32;
        si = __mul24(sc0, sa - 4 * bs[2 * L]) + __mul24(sc1, sb - 4 * bs[2 * L + 1]);   // exact: operands well inside 24 bits
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return h2f(d) * (float) si; }
};
// Q6_K (210 B: ql[128], qh[64], scales int8[16], d).  Lane L: ql bytes 64 hf + 32 qt0 + 16 hl .. (+16) with
// hf = L >> 2, qt0 = (L >> 1) & 1, hl = L & 1: low nibbles are the 16-group g = 8 hf + 2 qt0 + hl, high nibbles
// group g + 4; bits 2 qt of qh[32 hf + l] are bits 4-5.  (q6 - 32) . y = q6 . y - 32 bsum_g.
template <> struct Item<Q6_K> {
    Raw16 qlr, qhr;
    int sc_lo, sc_hi;
    uint16_t d;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        const int hf = L >> 2, qt0 = (L >> 1) & 1, hl = L & 1, g = 8 * hf + 2 * qt0 + hl;
        qlr.load(b + 64 * hf + 32 * qt0 + 16 * hl);   // (both end well inside the 210-byte block)
        qhr.load(b + 128 + 32 * hf + 16 * hl);
        sc_lo = (int8_t) b[192 + g]; sc_hi = (int8_t) b[192 + g + 4];
        d = ld_u16(b + 208);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const int hf = L >> 2, qt0 = (L >> 1) & 1, hl = L & 1, g = 8 * hf + 2 * qt0 + hl;
        const uint32_t *ya = (const uint32_t *) (y + 4 + 16 * g), *yb = (const uint32_t *) (y + 4 + 16 * (g + 4));
        const uint4 ql = qlr.bytes(), qh = qhr.bytes();
        const uint32_t q[4] = {ql.x, ql.y, ql.z, ql.w}, h[4] = {qh.x, qh.y, qh.z, qh.w};
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (((h[i] >> (2 * qt0)) & 0x03030303u) << 4);
            const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (2 * qt0 + 4)) & 0x03030303u) << 4);
            sa = sdot4(lo, ya[i], sa); sb = sdot4(hi, yb[i], sb);
        }
        const int16_t *bs = (const int16_t *) (y + 260);
        si = __mul24(sc_lo, sa - 32 * bs[g]) + __mul24(sc_hi, sb - 32 * bs[g + 4]);   // exact: |sa - 32 bs| < 2^18
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return h2f(d) * (float) si; }
};
// IQ4_XS (136 B: d, scales_h u16, scales_l[4], qs[128]).  Lane L = 32-group L: qs bytes 16 L .. (+16), low
// nibbles values 0..15, high nibbles 16..31; scale ls - 32 (src/iq3s_dot.h:136-166).
template <> struct Item<IQ4_XS> {
    uint4 qs;
    uint32_t dsh;   // d | scales_h << 16
    uint32_t sl;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        qs = load16_a4(b + 8 + 16 * L);
        dsh = *(const uint32_t *) b;
        sl = b[4 + (L >> 1)];
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) { s = sdot4(kv4(q[i] & 0x0F0F0F0Fu), ya[i], s); s = sdot4(kv4((q[i] >> 4) & 0x0F0F0F0Fu), ya[4 + i], s); }
        const int ls = ((sl >> (4 * (L & 1))) & 0xF) | ((((dsh >> 16) >> (2 * L)) & 3) << 4);
        si = (ls - 32) * s;
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return h2f(dsh & 0xffff) * (float) si; }
};
// IQ2_XS (74 B: d, qs u16[32], scales[8]).  Lane L = 32-group L: 8-groups l = 0..3 use qs[4 L + l]: grid row
// q & 511, signs ksigns[q >> 9]; scale nibble l >> 1 of scales[L]; value d (2 sc + 1) / 8 grid sign.
// `grid`: the codebook rows expanded to 8 bytes each and the sign masks (LDS, expand_iq2_grid).
template <> struct Item<IQ2_XS> {
    uint16_t q[4];
    uint16_t d;
    uint8_t sc;
    const uint2 *grid;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
#pragma unroll
        for (int l = 0; l < 4; ++l) q[l] = ld_u16(b + 2 + 2 * (4 * L + l));
        d = ld_u16(b);
        sc = b[66 + L];
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        int s[4];
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint2 g = grid[q[l] & 511], sm = grid[512 + (q[l] >> 9)];
            s[l] = sdot4(apply_mask(g.y, sm.y), ya[2 * l + 1], sdot4(apply_mask(g.x, sm.x), ya[2 * l], 0));
        }
        si = (2 * (sc & 15) + 1) * (s[0] + s[1]) + (2 * (sc >> 4) + 1) * (s[2] + s[3]);
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return (h2f(d) * 0.125f) * (float) si; }
};
// IQ2_XXS (66 B: d, qs u16[32]), src/kernels4.cu:578-589.  Lane L = 32-group L, two words at 2 + 8 L: a0 holds the
// four 8-groups' grid rows (byte l), a1 their 7-bit sign indices (bits 7 l ..) and the group's 4-bit scale (bits 28..);
// value d (2 sc + 1) / 8 grid sign (ggml's vec_dot_iq2_xxs_q8_K integers: sumi = (2 sc + 1) sum grid sign y per group).
template <> struct Item<IQ2_XXS> {
    uint32_t a0, a1;
    uint16_t d;
    const uint2 *grid;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {   // b is 2-byte aligned (66-byte rows)
        const uint8_t *p = b + 2 + 8 * L;
        a0 = (uint32_t) ld_u16(p) | ((uint32_t) ld_u16(p + 2) << 16);
        a1 = (uint32_t) ld_u16(p + 4) | ((uint32_t) ld_u16(p + 6) << 16);
        d = ld_u16(b);
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int L, int &si, int &sm) const {
        const uint32_t *ya = (const uint32_t *) (y + 4 + 32 * L);
        int s = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint2 g = grid[(a0 >> (8 * l)) & 255], m = grid[256 + ((a1 >> (7 * l)) & 127)];
            s = sdot4(apply_mask(g.y, m.y), ya[2 * l + 1], sdot4(apply_mask(g.x, m.x), ya[2 * l], s));
        }
        si = (2 * (int) (a1 >> 28) + 1) * s;
        sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return (h2f(d) * 0.125f) * (float) si; }
};
// IQ4_NL (18 B: d, qs[16]) against Q8_0: lane L takes the item's block L (32 values) whole; `y` is that
// block's Q8_0 data in the padded layout (d at 0, qs at 4).
template <> struct Item<IQ4_NL> {
    Raw16 qr;
    uint16_t d;
    // qs of block L: 2 mod 4 for even L (spans are 16-byte aligned), where the 2 bytes read past them are the next
    // block's d (L < 7)
    __device__ __forceinline__ void load(const uint8_t *b, int L) { qr.load(b + 18 * L + 2); d = ld_u16(b + 18 * L); }
    // the block's integer dot against the 32 activation values ya (4 a word)
    __device__ __forceinline__ int dot32(const uint32_t (&ya)[8]) const {
        const uint4 qs = qr.bytes();
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) { s = sdot4(kv4(q[i] & 0x0F0F0F0Fu), ya[i], s); s = sdot4(kv4((q[i] >> 4) & 0x0F0F0F0Fu), ya[4 + i], s); }
        return s;
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int, int &si, int &sm) const {
        const uint32_t *yw = (const uint32_t *) (y + 4);
        const uint32_t ya[8] = {yw[0], yw[1], yw[2], yw[3], yw[4], yw[5], yw[6], yw[7]};
        si = dot32(ya); sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return h2f(d) * (float) si; }
};
// Q8_0 weights (34 B: d, qs[32] int8) against Q8_0, src/kernels4.cu:421-714 (deq8: d * qs[j]): lane L takes the
// item's block L whole.  Its qs start at 34 L + 2: 2 mod 4 for even L, where the second 16-byte load reads the 2 bytes
// past the block (the next block's d, L < 7); aligned for odd L.
template <> struct Item<Q8_0> {
    Raw32 qr;
    uint16_t d;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        qr.load(b + 34 * L + 2);
        d = ld_u16(b + 34 * L);
    }
    __device__ __forceinline__ int dot32(const uint32_t (&ya)[8]) const {
        const uint4 q0 = qr.lo(), q1 = qr.hi();
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = sdot4(q[i], ya[i], s);
        return s;
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int, int &si, int &sm) const {
        const uint32_t *yw = (const uint32_t *) (y + 4);
        const uint32_t ya[8] = {yw[0], yw[1], yw[2], yw[3], yw[4], yw[5], yw[6], yw[7]};
        si = dot32(ya); sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return h2f(d) * (float) si; }
};
// MXFP4 (17 B: e, qs[16]) against Q8_0, src/kernels4.cu:569-577: lane L takes the item's block L whole, value j < 16 =
// kv[qs[j] & 15], 16 + j = kv[qs[j] >> 4], scaled by e8m0_half(e) (ggml's vec_dot_mxfp4_q8_0 integers:
// sumi = sum_32 kv q8).  Block L's qs start at 17 L + 1, at every offset mod 4; the spans are 8-byte aligned
// (136 bytes), so the misaligned loads end within the block or at most 3 bytes into the next (L < 7; for L = 7 the
// qs end the span, dword-aligned).
template <> struct Item<MXFP4> {
    Raw16 qr;
    uint32_t e;
    __device__ __forceinline__ void load(const uint8_t *b, int L) { qr.load(b + 17 * L + 1); e = b[17 * L]; }
    __device__ __forceinline__ int dot32(const uint32_t (&ya)[8]) const {
        const uint4 qs = qr.bytes();
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) { s = sdot4(kvfp4(q[i] & 0x0F0F0F0Fu), ya[i], s); s = sdot4(kvfp4((q[i] >> 4) & 0x0F0F0F0Fu), ya[4 + i], s); }
        return s;
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int, int &si, int &sm) const {
        const uint32_t *yw = (const uint32_t *) (y + 4);
        const uint32_t ya[8] = {yw[0], yw[1], yw[2], yw[3], yw[4], yw[5], yw[6], yw[7]};
        si = dot32(ya); sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return e8m0_half(e) * (float) si; }
};
// the integer sum of a 32-value activation block (4 values a word)
__device__ __forceinline__ int ysum32(const uint32_t (&ya)[8]) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = sdot4(ya[i], 0x01010101u, s);
    return s;
}
// Q5_1 (24 B: d, m, qh u32 @4, qs[16] @8), src/kernels4.cu:449-462: value j = d x + m, x = nibble j | qh bit j << 4
// (0..31; nibble j the low one of qs[j] for j < 16, the high one of qs[j - 16] above).  The reference's CPU path pairs
// it with Q8_1 rows, whose d and q are Q8_0's and whose s is fp16(d sum q); here the partner is the Q8_0 row and the
// min's term takes the exact integer sum q: sumi = sum_32 x q8 (ints' si), the block's activation sum (sm), folded as
// t = fma(d, sumi, m * sum).  Block L sits at 24 L of the 16-byte aligned 192-byte span: every field is dword-aligned.
template <> struct Item<Q5_1> {
    uint4 qs;
    uint32_t qh, dm;   // qh; d | m << 16
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        qs = load16_a4(b + 24 * L + 8);
        qh = *(const uint32_t *) (b + 24 * L + 4);
        dm = *(const uint32_t *) (b + 24 * L);
    }
    __device__ __forceinline__ int dot32(const uint32_t (&ya)[8]) const {
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s = sdot4((q[i] & 0x0F0F0F0Fu) | (spread4((qh >> (4 * i)) & 15) << 4), ya[i], s);
            s = sdot4(((q[i] >> 4) & 0x0F0F0F0Fu) | (spread4((qh >> (16 + 4 * i)) & 15) << 4), ya[4 + i], s);
        }
        return s;
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int, int &si, int &sm) const {
        const uint32_t *yw = (const uint32_t *) (y + 4);
        const uint32_t ya[8] = {yw[0], yw[1], yw[2], yw[3], yw[4], yw[5], yw[6], yw[7]};
        si = dot32(ya); sm = ysum32(ya);
    }
    __device__ __forceinline__ float tval(int si, int sm) const {
        return __builtin_fmaf(h2f(dm & 0xffff), (float) si, h2f(dm >> 16) * (float) sm);
    }
};
// Q5_0 (22 B: d, qh u32, qs[16]) against Q8_0, src/kernels4.cu:464-478: lane L takes the item's block L whole, value
// j = (nibble j | qh bit j << 4) - 16, nibble j the low one of qs[j] for j < 16, the high one of qs[j - 16] above; as
// an int8 byte that is the nibble, OR 0xF0 where the qh bit is clear (ggml's vec_dot_q5_0_q8_0 integers:
// sumi = sum_32 (x - 16) q8).  Block L sits at 22 L of the 16-byte aligned 176-byte span: its qs (22 L + 6) and qh
// (22 L + 2) are 2 mod 4 for even L, where the 16-byte read takes 2 bytes of block L + 1 (L < 7), and dword-aligned
// for odd L.
template <> struct Item<Q5_0> {
    Raw16 qr;
    uint32_t qh;
    uint16_t d;
    __device__ __forceinline__ void load(const uint8_t *b, int L) {
        qr.load(b + 22 * L + 6);
        qh = (uint32_t) ld_u16(b + 22 * L + 2) | ((uint32_t) ld_u16(b + 22 * L + 4) << 16);
        d = ld_u16(b + 22 * L);
    }
    __device__ __forceinline__ int dot32(const uint32_t (&ya)[8]) const {
        const uint4 qs = qr.bytes();
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w}, nh = ~qh;
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s = sdot4((q[i] & 0x0F0F0F0Fu) | fill_f0((nh >> (4 * i)) & 15), ya[i], s);
            s = sdot4(((q[i] >> 4) & 0x0F0F0F0Fu) | fill_f0((nh >> (16 + 4 * i)) & 15), ya[4 + i], s);
        }
        return s;
    }
    __device__ __forceinline__ void ints(const uint8_t *y, int, int &si, int &sm) const {
        const uint32_t *yw = (const uint32_t *) (y + 4);
        const uint32_t ya[8] = {yw[0], yw[1], yw[2], yw[3], yw[4], yw[5], yw[6], yw[7]};
        si = dot32(ya); sm = 0;
    }
    __device__ __forceinline__ float tval(int si, int) const { return h2f(d) * (float) si; }
};

// expand a grid codebook (base-3 codes: IQ2_XS 512 rows, IQ2_XXS 256, IQ2_S 1024; base-8 codes: IQ3_XXS 256 and IQ3_S
// 512 rows of 4 bytes, in .x) into rows x 8 bytes of LDS, followed by the sign patterns as byte masks (entry rows + i:
// byte j = 0xFF where bit j of ksign(i) is set, the parity bit giving byte 7; for the literal-sign types, IQ3_S and
// IQ2_S, bit j of i itself, i < 256; IQ1_S has no signs: its 2048 rows hold int8 -1 / 0 / 1)
template <int T>
__device__ __forceinline__ void expand_iq2_grid(uint2 *grid) {
    static_assert(iq2_type(T), "an IQ2 codebook");
    constexpr int R = iq2_rows(T);
    for (int i = threadIdx.x; i < R + iq2_masks(T); i += blockDim.x) {
        if (i >= R) {
            const uint32_t ks = literal_signs(T) ? (uint32_t) i - R : ksign((uint32_t) i - R);
            grid[i] = make_uint2(spread4(ks & 15) * 0xFFu, spread4(ks >> 4) * 0xFFu);
            continue;
        }
        if constexpr (T == IQ3_XXS) {
            uint32_t c = c_iq3xxs_code[i], lo = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j, c >>= 3) lo |= ((c & 7) == 7 ? 62u : 4u + 8u * (c & 7)) << (8 * j);
            grid[i] = make_uint2(lo, 0u);
            continue;
        }
        if constexpr (T == IQ3_S) {
            uint32_t c = c_iq3s_code[i], lo = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j, c >>= 3) lo |= (2u * (c & 7) + 1u) << (8 * j);
            grid[i] = make_uint2(lo, 0u);
            continue;
        }
        if constexpr (T == IQ1_S) {
            uint32_t c = c_iq1s_code[i], lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t v = (uint32_t) (int) ((c % 3) - 1) & 0xFFu;   // digit d -> int8 d - 1
                c /= 3;
                if (j < 4) lo |= v << (8 * j); else hi |= v << (8 * (j - 4));
            }
            grid[i] = make_uint2(lo, hi);
            continue;
        }
        uint32_t c = T == IQ2_XS ? c_iq2xs_code[i] : T == IQ2_S ? c_iq2s_code[i] : c_iq2xxs_code[i], lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t dgt = c % 3; c /= 3;
            const uint32_t v = dgt == 0 ? 8u : dgt == 1 ? 25u : 43u;
            if (j < 4) lo |= v << (8 * j); else hi |= v << (8 * (j - 4));
        }
        grid[i] = make_uint2(lo, hi);
    }
}

} // namespace hy
