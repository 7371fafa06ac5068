// Prefill / speculative-verify grouped expert GEMMs on int8 MFMA (gfx950 v_mfma_i32_16x16x32_i8).
//
// Work item = (active expert, chunk of up to 64 of its tokens, 64 weight rows); the block's 4 waves take 16
// rows each (gate/up: 32 output rows, waves 0-1 in gate and waves 2-3 in up, SwiGLU after an LDS exchange).
// Items are numbered expert by expert; a block finds its (expert, chunk) from egrp with a block-wide prefix
// of the experts' chunk counts (replaces k_moe_gemm /
// k_moe_gemm2, src/kernels4.cu:1354-1467, :1521-1631, which dequantize to fp16 and run fp16 MMA).
// Per 256-value block b of the K dimension:
//   A (16 tokens x 32 k): the tokens' Q8_K bytes, staged through LDS (double-buffered) for the 4 waves;
//   B (32 k x 16 rows):   one weight row per lane group, decoded to int8 in registers chunk by chunk;
//   D = A B per 32-value chunk, exact int32; sumi += scale * D (one 24-bit v_mad per value and chunk: |D| < 2^23,
//   |scale| < 2^8); the mins
//   term of Q4_K / Q5_K is a second, chained MFMA against a B that holds the chunk's min; after the 8 chunks
//   the block's integers fold into the fp32 accumulator with the contract's formula.
// The next block's weight bytes and activation bytes are loaded while this block computes.
// Operand layouts (16x16x32 i8): A lane l holds token l % 16, k = 8 (l / 16) .. + 7; B lane l holds weight row
// l % 16 with the same k; D lane l holds row l % 16 for tokens 4 (l / 16) + v, v = 0..3.
// Types with 16-value scale groups (Q6_K, IQ2_XS) run each chunk as two MFMAs with B zeroed in the lanes of
// the other group (lanes 0-31 hold k 0..15, lanes 32-63 k 16..31).
#include "hy_internal.h"
#include "hy_blocks.cuh"

#include <algorithm>
#include <type_traits>

namespace hy {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma16(long a, long b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0); }
__device__ __forceinline__ long mk_long(uint32_t lo, uint32_t hi) { return (long) (((unsigned long long) hi << 32) | lo); }
__device__ __forceinline__ uint2 load8_a2(const uint8_t *p) {   // 8 bytes from a 2-byte aligned address, no overread
    if (((uintptr_t) p & 3) == 0) { const uint32_t *w = (const uint32_t *) p; return make_uint2(w[0], w[1]); }
    const uint32_t h0 = *(const uint16_t *) p, d1 = *(const uint32_t *) (p + 2), h2 = *(const uint16_t *) (p + 6);
    return make_uint2(h0 | (d1 << 16), (d1 >> 16) | (h2 << 16));
}

// Branch-free loads from 2-byte aligned addresses (a fixed instruction count per step lets the compiler count
// the loads in flight): whole dwords from the aligned-down address, joined with v_alignbyte.
__device__ __forceinline__ uint32_t join_b(uint32_t hi, uint32_t lo, uint32_t sb) { return __builtin_amdgcn_alignbyte(hi, lo, sb); }
// 8 bytes at p (2-byte aligned); reads the dwords at p & ~3 .. + 11, all of which must lie in the buffer
// (the aligned-down pointer is formed by pointer arithmetic on p, so that an LDS pointer stays an LDS pointer)
__device__ __forceinline__ uint2 ld8_2a(const uint8_t *p) {
    const uint32_t *w = (const uint32_t *) (p - ((uintptr_t) p & 3));
    const uint32_t sb = (uint32_t) ((uintptr_t) p & 3);
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2];
    return make_uint2(join_b(d1, d0, sb), join_b(d2, d1, sb));
}
// 16 bytes at p (2-byte aligned), with p + 18 the end of the block: the fifth dword is read only when p is
// misaligned (else the fourth is read again), so nothing past p + 18 is touched
__device__ __forceinline__ uint4 ld16_2a_tail(const uint8_t *p) {
    const uint32_t *w = (const uint32_t *) (p - ((uintptr_t) p & 3));
    const uint32_t sb = (uint32_t) ((uintptr_t) p & 3);
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2], d3 = w[3], d4 = w[sb ? 4 : 3];
    return make_uint4(join_b(d1, d0, sb), join_b(d2, d1, sb), join_b(d3, d2, sb), join_b(d4, d3, sb));
}

// The raw bytes of one weight row's 256-value block that lane quarter q needs, and their decoding per 32-value
// chunk c: B operand words b0/b1 (8 int8 values), scale(s), min.
template <int T> struct Raw;

template <> struct Raw<Q4_K> {   // 144 B: d, dmin, scales[12], qs[128]; chunk c: nibbles (c & 1) of qs[32 (c / 2) + 8 q ..]
    static constexpr bool mins = true, g16 = false, per_chunk = false;
    uint4 hd; uint2 qv[4];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        hd = load16_a4(blk);
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) qv[jp] = *(const uint2 *) (blk + 16 + 32 * jp + 8 * q);
    }
    __device__ __forceinline__ void chunk(int c, int, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int sh = 4 * (c & 1);
        b0 = (qv[c >> 1].x >> sh) & 0x0F0F0F0Fu; b1 = (qv[c >> 1].y >> sh) & 0x0F0F0F0Fu;
        scale_min_k4(hd.y, hd.z, hd.w, c, s0, mn);
        s1 = 0;
    }
    __device__ __forceinline__ float fold(int si, int sm) const {
        return __builtin_fmaf(h2f(hd.x & 0xffff), (float) si, -(h2f(hd.x >> 16) * (float) sm));
    }
};
template <> struct Raw<Q5_K> {   // 176 B: + qh[32] @16 (bit c of qh[l] is bit 4 of chunk c's value l), qs @48
    static constexpr bool mins = true, g16 = false, per_chunk = false;
    uint4 hd; uint2 qv[4], qh;
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        hd = load16_a4(blk);
        qh = *(const uint2 *) (blk + 16 + 8 * q);
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) qv[jp] = *(const uint2 *) (blk + 48 + 32 * jp + 8 * q);
    }
    __device__ __forceinline__ void chunk(int c, int, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int sh = 4 * (c & 1);
        b0 = ((qv[c >> 1].x >> sh) & 0x0F0F0F0Fu) | (((qh.x >> c) & 0x01010101u) << 4);
        b1 = ((qv[c >> 1].y >> sh) & 0x0F0F0F0Fu) | (((qh.y >> c) & 0x01010101u) << 4);
        scale_min_k4(hd.y, hd.z, hd.w, c, s0, mn);
        s1 = 0;
    }
    __device__ __forceinline__ float fold(int si, int sm) const {
        return __builtin_fmaf(h2f(hd.x & 0xffff), (float) si, -(h2f(hd.x >> 16) * (float) sm));
    }
};
// Q2_K (84 B: scales[16], qs[64] @16, d @80, dmin @82): chunk c = values 32 c ..: 2-bit fields 2 (c & 3) of qs bytes
// 32 (c >> 2) + 8 q ..; the chunk's 16-groups 2 c (lanes q < 2) and 2 c + 1 (q >= 2): scales s0 / s1, and the lane's
// own group's min (the mins MFMA takes each lane quarter's bytes, so each 8-value piece carries its group's min).
template <> struct Raw<Q2_K> {
    static constexpr bool mins = true, g16 = true, per_chunk = false;
    uint4 scv; uint2 qv[2]; uint32_t dm;
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        scv = load16_a4(blk);
        qv[0] = *(const uint2 *) (blk + 16 + 8 * q);
        qv[1] = *(const uint2 *) (blk + 48 + 8 * q);
        dm = *(const uint32_t *) (blk + 80);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int sh = 2 * (c & 3);
        b0 = (qv[c >> 2].x >> sh) & 0x03030303u;
        b1 = (qv[c >> 2].y >> sh) & 0x03030303u;
        const uint32_t w = (c < 2 ? scv.x : c < 4 ? scv.y : c < 6 ? scv.z : scv.w) >> (16 * (c & 1));   // bytes 2 c, 2 c + 1
        s0 = (int) (w & 15);
        s1 = (int) ((w >> 8) & 15);
        mn = (int) ((w >> (q < 2 ? 4 : 12)) & 15);
    }
    __device__ __forceinline__ float fold(int si, int sm) const {
        return __builtin_fmaf(h2f(dm & 0xffff), (float) si, -(h2f(dm >> 16) * (float) sm));
    }
};
// IQ3_XXS (98 B): chunk c = 32-group c; lane q takes 8-group q: grid indices qs[8 c + 2 q], qs[8 c + 2 q + 1] (a
// halfword at 2 + 8 c + 2 q), sign index bits 7 q .. of the word at 66 + 4 c, the chunk's scale 2 sc + 1 (bits 28 ..)
// (src/kernels4.cu:613-627; ggml's vec_dot_iq3_xxs_q8_K integers).
template <> struct Raw<IQ3_XXS> {
    static constexpr bool mins = false, g16 = false, per_chunk = false;
    uint32_t gi[4], a[8], d;   // gi: the lane's index pair of chunk c in halfword c % 2 of gi[c / 2]
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; c += 2)
            gi[c >> 1] = (uint32_t) ld_u16(blk + 2 + 8 * c + 2 * q) | ((uint32_t) ld_u16(blk + 10 + 8 * c + 2 * q) << 16);
#pragma unroll
        for (int c = 0; c < 8; ++c) a[c] = (uint32_t) ld_u16(blk + 66 + 4 * c) | ((uint32_t) ld_u16(blk + 68 + 4 * c) << 16);
        d = ld_u16(blk);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *grid, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const uint32_t ip = gi[c >> 1] >> (16 * (c & 1));
        const uint2 m = grid[256 + ((a[c] >> (7 * q)) & 127)];
        b0 = apply_mask(grid[ip & 255].x, m.x);
        b1 = apply_mask(grid[(ip >> 8) & 255].x, m.y);
        s0 = 2 * (int) (a[c] >> 28) + 1;
        s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return (h2f(d) * 0.25f) * (float) si; }
};
// IQ1_S (50 B): chunk c = 32-group c; lane q takes 8-group q: grid row qs[4 c + q] | 3 bits (3 q) of qh[c] << 8 (int8
// -1 / 0 / 1), the chunk's scale ls; the delta term rides on the mins MFMA with the chunk's ls * (+-1) as its "min", so
// sm = sum_ib ls sign sum_32 y and the fold is (d / 8) (8 si + sm) (src/kernels4.cu:650-659; src/iq1s_dot.h:26-64).
template <> struct Raw<IQ1_S> {
    static constexpr bool mins = true, g16 = false, per_chunk = false;
    uint32_t gq[2], qh[4], d;   // gq: the lane's index byte of chunk c in byte c % 4 of gq[c / 4]; qh[c] in halfwords
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        gq[0] = gq[1] = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) gq[c >> 2] |= (uint32_t) blk[2 + 4 * c + q] << (8 * (c & 3));
#pragma unroll
        for (int i = 0; i < 4; ++i) qh[i] = (uint32_t) ld_u16(blk + 34 + 4 * i) | ((uint32_t) ld_u16(blk + 36 + 4 * i) << 16);
        d = ld_u16(blk);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *grid, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const uint32_t h = (qh[c >> 1] >> (16 * (c & 1))) & 0xffff;
        const uint2 g = grid[((gq[c >> 2] >> (8 * (c & 3))) & 255) | (((h >> (3 * q)) & 7) << 8)];
        b0 = g.x; b1 = g.y;
        s0 = 2 * (int) ((h >> 12) & 7) + 1;
        s1 = 0;
        mn = h & 0x8000 ? -s0 : s0;
    }
    __device__ __forceinline__ float fold(int si, int sm) const { return (h2f(d) * 0.125f) * (float) (8 * si + sm); }
};
// IQ2_S (82 B): chunk c = 32-group c; lane q takes 8-group q: grid row qs[4 c + q] | bits 2 q, 2 q + 1 of qh[c] << 8,
// sign byte signs[4 c + q], the chunk's 16-group scales 2 sc + 1 from the nibbles of scales[c] (s0 for lanes q < 2)
// (src/kernels4.cu:602-613; ggml's vec_dot_iq2_s_q8_K integers).
template <> struct Raw<IQ2_S> {
    static constexpr bool mins = false, g16 = true, per_chunk = false;
    uint32_t gq[2], sg[2], qh[2], sc[2], d;   // byte c % 4 of [c / 4]: the lane's index byte, its sign byte, qh[c], scales[c]
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        gq[0] = gq[1] = sg[0] = sg[1] = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            gq[c >> 2] |= (uint32_t) blk[2 + 4 * c + q] << (8 * (c & 3));
            sg[c >> 2] |= (uint32_t) blk[34 + 4 * c + q] << (8 * (c & 3));
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            qh[i] = (uint32_t) ld_u16(blk + 66 + 4 * i) | ((uint32_t) ld_u16(blk + 68 + 4 * i) << 16);
            sc[i] = (uint32_t) ld_u16(blk + 74 + 4 * i) | ((uint32_t) ld_u16(blk + 76 + 4 * i) << 16);
        }
        d = ld_u16(blk);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *grid, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int sh = 8 * (c & 3);
        const uint32_t idx = ((gq[c >> 2] >> sh) & 255) | (((qh[c >> 2] >> (sh + 2 * q)) & 3) << 8);
        const uint2 g = grid[idx], m = grid[1024 + ((sg[c >> 2] >> sh) & 255)];
        b0 = apply_mask(g.x, m.x);
        b1 = apply_mask(g.y, m.y);
        const uint32_t s = (sc[c >> 2] >> sh) & 255;
        s0 = 2 * (int) (s & 15) + 1;
        s1 = 2 * (int) (s >> 4) + 1;
        mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return (h2f(d) * 0.125f) * (float) si; }
};
// IQ3_S (110 B): chunk c = 32-group c; lane q takes 8-group q: grid indices qs[8 c + 2 q], qs[8 c + 2 q + 1] with bits
// 2 q, 2 q + 1 of qh[c] as their 9th bits, sign byte signs[4 c + q], the chunk's scale 2 sc + 1 (nibble c & 1 of
// scales[c / 2]) (src/kernels4.cu:682-695; src/iq3s_dot.h:48-76 integers).
template <> struct Raw<IQ3_S> {
    static constexpr bool mins = false, g16 = false, per_chunk = false;
    uint32_t gi[4], qh[2], sg[2], sc, d;   // gi: index pairs (halfword c % 2 of gi[c / 2]); qh, sg: byte c % 4 of [c / 4]
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; c += 2)
            gi[c >> 1] = (uint32_t) ld_u16(blk + 2 + 8 * c + 2 * q) | ((uint32_t) ld_u16(blk + 10 + 8 * c + 2 * q) << 16);
        qh[0] = (uint32_t) ld_u16(blk + 66) | ((uint32_t) ld_u16(blk + 68) << 16);
        qh[1] = (uint32_t) ld_u16(blk + 70) | ((uint32_t) ld_u16(blk + 72) << 16);
        sg[0] = sg[1] = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) sg[c >> 2] |= (uint32_t) blk[74 + 4 * c + q] << (8 * (c & 3));
        sc = (uint32_t) ld_u16(blk + 106) | ((uint32_t) ld_u16(blk + 108) << 16);
        d = ld_u16(blk);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *grid, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const uint32_t ip = gi[c >> 1] >> (16 * (c & 1)), h = qh[c >> 2] >> (8 * (c & 3));
        const uint32_t i1 = (ip & 255) | (((h >> (2 * q)) & 1) << 8), i2 = ((ip >> 8) & 255) | (((h >> (2 * q + 1)) & 1) << 8);
        const uint2 m = grid[512 + ((sg[c >> 2] >> (8 * (c & 3))) & 255)];
        b0 = apply_mask(grid[i1].x, m.x);
        b1 = apply_mask(grid[i2].x, m.y);
        s0 = 2 * (int) ((sc >> (4 * c)) & 15) + 1;
        s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return h2f(d) * (float) si; }
};
// Q3_K (110 B: hmask[32], qs[64] @32, scales[12] @96, d @108): chunk c = values 32 c .., hf = c >> 2, j = c & 3; lane
// values l = 8 q .. + 7: 2-bit fields 2 j of qs bytes 32 + 32 hf + l, each byte OR 0xFC where bit 4 hf + j of hmask[l]
// is clear (q - 4 as int8); 16-groups 2 c (lanes q < 2) and 2 c + 1 with their signed 6-bit scales.  Blocks are 2-byte
// aligned: ld8_2a's 12-byte reads end by byte 99.
__device__ __forceinline__ int q3k_scale(const uint32_t (&s)[3], int is) {
    auto byte = [&](int i) { return (int) ((s[i >> 2] >> (8 * (i & 3))) & 255); };
    return (((byte(is & 7) >> (4 * (is >> 3))) & 15) | (((byte(8 + (is & 3)) >> (2 * (is >> 2))) & 3) << 4)) - 32;
}
template <> struct Raw<Q3_K> {
    static constexpr bool mins = false, g16 = true, per_chunk = false;
    uint2 qv[2], hm; uint32_t sc[3], d;
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        qv[0] = ld8_2a(blk + 32 + 8 * q);
        qv[1] = ld8_2a(blk + 64 + 8 * q);
        hm = ld8_2a(blk + 8 * q);
#pragma unroll
        for (int i = 0; i < 3; ++i) sc[i] = (uint32_t) ld_u16(blk + 96 + 4 * i) | ((uint32_t) ld_u16(blk + 98 + 4 * i) << 16);
        d = ld_u16(blk + 108);
    }
    __device__ __forceinline__ void chunk(int c, int, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int s2 = 2 * (c & 3), hb = 4 * (c >> 2) + (c & 3);
        b0 = ((qv[c >> 2].x >> s2) & 0x03030303u) | fill_fc((~hm.x >> hb) & 0x01010101u);
        b1 = ((qv[c >> 2].y >> s2) & 0x03030303u) | fill_fc((~hm.y >> hb) & 0x01010101u);
        s0 = q3k_scale(sc, 2 * c);
        s1 = q3k_scale(sc, 2 * c + 1);
        mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return h2f(d) * (float) si; }
};
// Q6_K (210 B): chunk c = elements 32 c ..: hf = c >> 2, qt = c & 3; lane values l = 8 q .. + 7 from
// ql[64 hf + 32 (qt & 1) + l] (high nibble when qt >= 2) and bits 2 qt of qh[32 hf + l]; groups 2 c, 2 c + 1.
template <> struct Raw<Q6_K> {
    static constexpr bool mins = false, g16 = true, per_chunk = false;
    uint2 ql[4], qh[2]; uint4 scv; uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ql[i] = ld8_2a(blk + 64 * (i >> 1) + 32 * (i & 1) + 8 * q);   // reads up to blk + 132
#pragma unroll
        for (int i = 0; i < 2; ++i) qh[i] = ld8_2a(blk + 128 + 32 * i + 8 * q);                     // up to blk + 196
        scv = ld16_2a_tail(blk + 192);                                                                // up to blk + 210
        d = ld_u16(blk + 208);
    }
    __device__ __forceinline__ void chunk(int c, int, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int hf = c >> 2, qt = c & 3, sh = qt >= 2 ? 4 : 0;
        const uint2 l = ql[2 * hf + (qt & 1)], h = qh[hf];
        b0 = q6_signed(((l.x >> sh) & 0x0F0F0F0Fu) | (((h.x >> (2 * qt)) & 0x03030303u) << 4));
        b1 = q6_signed(((l.y >> sh) & 0x0F0F0F0Fu) | (((h.y >> (2 * qt)) & 0x03030303u) << 4));
        s0 = (int) (int8_t) byte_of(scv, 2 * c);
        s1 = (int) (int8_t) byte_of(scv, 2 * c + 1);
        mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return h2f(d) * (float) si; }
};
// IQ4_XS (136 B): chunk c = 32-group c; lane values 8 q .. + 7 are nibbles (q >> 1) of qs[16 c + 8 (q & 1) ..]
template <> struct Raw<IQ4_XS> {
    static constexpr bool mins = false, g16 = false, per_chunk = false;
    uint2 qv[8]; uint32_t dsh, sl;
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; ++c) qv[c] = *(const uint2 *) (blk + 8 + 16 * c + 8 * (q & 1));
        dsh = *(const uint32_t *) blk;
        sl = *(const uint32_t *) (blk + 4);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int s = 4 * (q >> 1);
        b0 = kv4((qv[c].x >> s) & 0x0F0F0F0Fu);
        b1 = kv4((qv[c].y >> s) & 0x0F0F0F0Fu);
        s0 = (((sl >> (8 * (c >> 1) + 4 * (c & 1))) & 0xF) | ((((dsh >> 16) >> (2 * c)) & 3) << 4)) - 32;
        s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return h2f(dsh & 0xffff) * (float) si; }
};
// IQ2_XS (74 B): chunk c = 32-group c; lane q takes 8-group q (grid row qs[4 c + q], signs); scales
// 2 (scales[c] & 15) + 1 for k 0..15 (lanes q < 2) and 2 (scales[c] >> 4) + 1 for k 16..31.
template <> struct Raw<IQ2_XS> {
    static constexpr bool mins = false, g16 = true, per_chunk = false;
    uint32_t qq[4]; uint2 scv; uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; c += 2) qq[c >> 1] = (uint32_t) ld_u16(blk + 2 + 2 * (4 * c + q)) | ((uint32_t) ld_u16(blk + 2 + 2 * (4 * c + 4 + q)) << 16);
        scv = make_uint2((uint32_t) ld_u16(blk + 66) | ((uint32_t) ld_u16(blk + 68) << 16),
                         (uint32_t) ld_u16(blk + 70) | ((uint32_t) ld_u16(blk + 72) << 16));
        d = ld_u16(blk);
    }
    __device__ __forceinline__ void chunk(int c, int, const uint2 *grid, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const uint32_t qv = (qq[c >> 1] >> (16 * (c & 1))) & 0xffff;
        const uint2 g = grid[qv & 511], sm = grid[512 + (qv >> 9)];
        b0 = apply_mask(g.x, sm.x);
        b1 = apply_mask(g.y, sm.y);
        const uint32_t s = ((c < 4 ? scv.x : scv.y) >> (8 * (c & 3))) & 0xff;
        s0 = 2 * (int) (s & 15) + 1;
        s1 = 2 * (int) (s >> 4) + 1;
        mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return (h2f(d) * 0.125f) * (float) si; }
};

// IQ2_XXS (66 B): chunk c = 32-group c, two words at 2 + 8 c (grid rows a byte each, then 4 x 7 sign bits and the
// 4-bit scale); lane q takes 8-group q: grid row byte q of the first word, signs bits 7 q .. of the second, the chunk's
// scale 2 sc + 1 (src/kernels4.cu:578-589; ggml's vec_dot_iq2_xxs_q8_K integers).
template <> struct Raw<IQ2_XXS> {
    static constexpr bool mins = false, g16 = false, per_chunk = false;
    uint32_t gi[2], a1[8], d;   // gi: the lane's grid row of chunk c in byte c % 4 of gi[c / 4]
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        gi[0] = gi[1] = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint8_t *p = blk + 2 + 8 * c;
            a1[c] = (uint32_t) ld_u16(p + 4) | ((uint32_t) ld_u16(p + 6) << 16);
            gi[c >> 2] |= (uint32_t) p[q] << (8 * (c & 3));
        }
        d = ld_u16(blk);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *grid, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const uint2 g = grid[(gi[c >> 2] >> (8 * (c & 3))) & 255], m = grid[256 + ((a1[c] >> (7 * q)) & 127)];
        b0 = apply_mask(g.x, m.x);
        b1 = apply_mask(g.y, m.y);
        s0 = 2 * (int) (a1[c] >> 28) + 1;
        s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float fold(int si, int) const { return (h2f(d) * 0.125f) * (float) si; }
};

// IQ4_NL (8 blocks of 18 B per 256 values, Q8_0 activations): chunk c = block c; lane values 8 q .. + 7 are
// nibbles (q >> 1) of qs[8 (q & 1) ..]; every block folds on its own: acc = fma(x_d, fp16(d_c) * D, acc).
template <> struct Raw<IQ4_NL> {
    static constexpr bool mins = false, g16 = false, per_chunk = true;
    uint2 qv[8]; uint32_t dd[4];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        // the span is 16-byte aligned (rows of 144 n / 256 bytes), so block c's qs sit at 2 mod 4 for even c and
        // at 0 mod 4 for odd c
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint8_t *p = blk + 18 * c + 2 + 8 * (q & 1);
            if (c & 1) qv[c] = *(const uint2 *) p;
            else {
                const uint32_t *w = (const uint32_t *) (p - 2);
                const uint32_t d0 = w[0], d1 = w[1], d2 = w[2];
                qv[c] = make_uint2(join_b(d1, d0, 2), join_b(d2, d1, 2));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) dd[i] = (uint32_t) ld_u16(blk + 36 * i) | ((uint32_t) ld_u16(blk + 36 * i + 18) << 16);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int s = 4 * (q >> 1);
        b0 = kv4((qv[c].x >> s) & 0x0F0F0F0Fu);
        b1 = kv4((qv[c].y >> s) & 0x0F0F0F0Fu);
        s0 = 1; s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float cfold(int c, int d) const { return h2f((dd[c >> 1] >> (16 * (c & 1))) & 0xffff) * (float) d; }
    __device__ __forceinline__ float fold(int si, int) const { return (float) si; }
};
// Q8_0 weights (8 blocks of 34 B per 256 values, Q8_0 activations): chunk c = block c; lane values 8 q .. + 7 are
// qs[8 q ..] of block c as they are (int8); block c's qs sit at 34 c + 2 (2 mod 4 for even c, where the 8-byte read
// takes 2 bytes of block c + 1, c < 7); every block folds on its own, as IQ4_NL's.
template <> struct Raw<Q8_0> {
    static constexpr bool mins = false, g16 = false, per_chunk = true;
    uint2 qv[8]; uint32_t dd[4];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; ++c) qv[c] = ld8_2a(blk + 34 * c + 2 + 8 * q);
#pragma unroll
        for (int i = 0; i < 4; ++i) dd[i] = (uint32_t) ld_u16(blk + 68 * i) | ((uint32_t) ld_u16(blk + 68 * i + 34) << 16);
    }
    __device__ __forceinline__ void chunk(int c, int, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        b0 = qv[c].x; b1 = qv[c].y;
        s0 = 1; s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float cfold(int c, int d) const { return h2f((dd[c >> 1] >> (16 * (c & 1))) & 0xffff) * (float) d; }
    __device__ __forceinline__ float fold(int si, int) const { return (float) si; }
};
// MXFP4 (8 blocks of 17 B per 256 values, Q8_0 activations): chunk c = block c, lane values as IQ4_NL's (nibbles
// (q >> 1) of qs[8 (q & 1) ..]), the MXFP4 codebook, the fold e8m0_half(e_c) * D.  Spans of 136 bytes are 8-byte
// aligned, so block c's qs at 17 c + 1 sit at offset (17 c + 1) mod 4 = 1 2 3 0 1 2 3 0: the dword-aligned ones
// (c = 3, 7) are read as they are, the others by ld8_2a, whose 12 bytes end at most at blk + 119.
template <> struct Raw<MXFP4> {
    static constexpr bool mins = false, g16 = false, per_chunk = true;
    uint2 qv[8]; uint32_t ee[2];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint8_t *p = blk + 17 * c + 1 + 8 * (q & 1);
            qv[c] = (c & 3) == 3 ? *(const uint2 *) p : ld8_2a(p);
        }
        ee[0] = ee[1] = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) ee[c >> 2] |= (uint32_t) blk[17 * c] << (8 * (c & 3));
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int s = 4 * (q >> 1);
        b0 = kvfp4((qv[c].x >> s) & 0x0F0F0F0Fu);
        b1 = kvfp4((qv[c].y >> s) & 0x0F0F0F0Fu);
        s0 = 1; s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float cfold(int c, int d) const { return e8m0_half((ee[c >> 2] >> (8 * (c & 3))) & 255) * (float) d; }
    __device__ __forceinline__ float fold(int si, int) const { return (float) si; }
};
// Q5_1 (8 blocks of 24 B per 256 values, Q8_0 activations): chunk c = block c, lane values as IQ4_NL's with the fifth
// bits in qh byte q of the block (x = nibble | bit << 4, 0..31); every field dword-aligned (24-byte blocks in a 192-byte
// span).  The min's term needs each token's block sum q: chunk_fold takes it from one more MFMA against ones
// (ysum), and the fold is fma(d_c, D, m_c * S) (the integers of Item<Q5_1>).
template <> struct Raw<Q5_1> {
    static constexpr bool mins = false, g16 = false, per_chunk = true;
    uint2 qv[8]; uint32_t hb[2], dm[8];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            qv[c] = *(const uint2 *) (blk + 24 * c + 8 + 8 * (q & 1));
            dm[c] = *(const uint32_t *) (blk + 24 * c);
        }
        hb[0] = hb[1] = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) hb[c >> 2] |= (uint32_t) blk[24 * c + 4 + q] << (8 * (c & 3));
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int s = 4 * (q >> 1);
        const uint32_t h = hb[c >> 2] >> (8 * (c & 3));
        b0 = ((qv[c].x >> s) & 0x0F0F0F0Fu) | (spread4(h & 15) << 4);
        b1 = ((qv[c].y >> s) & 0x0F0F0F0Fu) | (spread4((h >> 4) & 15) << 4);
        s0 = 1; s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float cfold2(int c, int d, int ys) const {
        return __builtin_fmaf(h2f(dm[c] & 0xffff), (float) d, h2f(dm[c] >> 16) * (float) ys);
    }
    __device__ __forceinline__ float cfold(int c, int d) const { return cfold2(c, d, 0); }
    __device__ __forceinline__ float fold(int si, int) const { return (float) si; }
};
// Q5_0 (8 blocks of 22 B per 256 values, Q8_0 activations): chunk c = block c, lane values as IQ4_NL's (nibbles
// (q >> 1) of qs[8 (q & 1) ..]) with their fifth bits in qh byte q (bits 8 q .. 8 q + 7), each byte nibble | 0xF0
// where the bit is clear (x - 16 as int8).  Block c's qs (22 c + 6) and qh (22 c + 2) are 2 mod 4 for even c, read by
// ld8_2a whose 12 bytes end at most at blk + 155, and dword-aligned for odd c, read as they are.
template <> struct Raw<Q5_0> {
    static constexpr bool mins = false, g16 = false, per_chunk = true;
    uint2 qv[8]; uint32_t hb[2], dd[4];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint8_t *p = blk + 22 * c + 6 + 8 * (q & 1);
            qv[c] = (c & 1) ? *(const uint2 *) p : ld8_2a(p);
        }
        hb[0] = hb[1] = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) hb[c >> 2] |= (uint32_t) blk[22 * c + 2 + q] << (8 * (c & 3));
#pragma unroll
        for (int i = 0; i < 4; ++i) dd[i] = (uint32_t) ld_u16(blk + 44 * i) | ((uint32_t) ld_u16(blk + 44 * i + 22) << 16);
    }
    __device__ __forceinline__ void chunk(int c, int q, const uint2 *, uint32_t &b0, uint32_t &b1, int &s0, int &s1, int &mn) const {
        const int s = 4 * (q >> 1);
        const uint32_t nh = ~(hb[c >> 2] >> (8 * (c & 3)));
        b0 = ((qv[c].x >> s) & 0x0F0F0F0Fu) | fill_f0(nh & 15);
        b1 = ((qv[c].y >> s) & 0x0F0F0F0Fu) | fill_f0((nh >> 4) & 15);
        s0 = 1; s1 = 0; mn = 0;
    }
    __device__ __forceinline__ float cfold(int c, int d) const { return h2f((dd[c >> 1] >> (16 * (c & 1))) & 0xffff) * (float) d; }
    __device__ __forceinline__ float fold(int si, int) const { return (float) si; }
};

constexpr int GM_TOK = 64, GM_TILES = GM_TOK / 16, GM_ROWS = 64, GM_LD = 264;   // LDS row stride of staged activations

// one chunk's integers for the tiles: si[tile][v] += scale * D; sm[tile] chained for the mins
// A-operand bytes of token row t (tile * 16 + rr), k = 32 c + 8 q .. + 7: padded rows (GM_LD bytes), or rows of 256
// bytes whose 16-byte pieces are stored at piece ^ (t % 16) (the LDS-DMA layout; conflict-free MFMA operand reads)
template <bool SWZ>
__device__ __forceinline__ long a_frag(const int8_t *As, int tile, int rr, int c, int q) {
    if constexpr (SWZ) return *(const long *) (As + (tile * 16 + rr) * 256 + 16 * ((2 * c + (q >> 1)) ^ rr) + 8 * (q & 1));
    else return *(const long *) (As + (tile * 16 + rr) * GM_LD + 32 * c + 8 * q);
}

// (NT: a compile-time bound on the tiles; ntile, the run-time count, is NT itself where the caller specializes)
template <int T, bool SWZ = false, int NT = GM_TILES>
__device__ __forceinline__ void chunk_ints(const Raw<T> &w, int c, int q, const uint2 *grid, const int8_t *As, int rr, int ntile,
                                           int (&si)[GM_TILES][4], v4i (&sm)[GM_TILES], const long (*af)[8] = nullptr) {
    const v4i z = {0, 0, 0, 0};
    uint32_t b0, b1;
    int s0, s1, mn;
    w.chunk(c, q, grid, b0, b1, s0, s1, mn);
    const uint32_t mb = __builtin_amdgcn_perm(0u, (uint32_t) mn, 0u);   // the min in all four bytes (selector 0-3: bytes of the 2nd operand)
#pragma unroll
    for (int tile = 0; tile < NT; ++tile) {
        if (tile >= ntile) break;
        const long a = af ? af[tile][c] : a_frag<SWZ>(As, tile, rr, c, q);   // af: read up front by the caller
        if constexpr (Raw<T>::g16) {
            const bool lo = q < 2;
            const v4i d0 = mfma16(a, mk_long(lo ? b0 : 0u, lo ? b1 : 0u), z);
            const v4i d1 = mfma16(a, mk_long(lo ? 0u : b0, lo ? 0u : b1), z);
#pragma unroll
            for (int v = 0; v < 4; ++v) si[tile][v] += __mul24(s0, d0[v]) + __mul24(s1, d1[v]);
            if constexpr (Raw<T>::mins) sm[tile] = mfma16(a, mk_long(mb, mb), sm[tile]);   // mb: the lane's group's min
        } else {
            const v4i d0 = mfma16(a, mk_long(b0, b1), z);
#pragma unroll
            for (int v = 0; v < 4; ++v) si[tile][v] += __mul24(s0, d0[v]);
            if constexpr (Raw<T>::mins) sm[tile] = mfma16(a, mk_long(mb, mb), sm[tile]);
        }
    }
}


// each Raw<T> register set: wait until its loads have landed (every register is an input of an empty asm)
template <class R> __device__ __forceinline__ void touch_regs(const R &r) {
    static_assert(sizeof(R) % 4 == 0, "register set of whole dwords");
    const uint32_t *w = (const uint32_t *) &r;
#pragma unroll
    for (int i = 0; i < (int) (sizeof(R) / 4); ++i) asm volatile("" ::"v"(w[i]));
}

// Direct global -> LDS loads and the epilogue's stores, issued from inline asm so that the compiler's wait
// bookkeeping sees only the weight loads of the stream.  (Its bookkeeping treats LDS loads, register loads and
// stores as possibly completing out of order and would then wait for all of them at every step.)  Vector memory
// operations of a wave complete in issue order, so waiting for a step's weight registers also covers every DMA
// issued before them.  M0 holds the LDS address of a DMA; it is saved and restored around it.
__device__ __forceinline__ void dma_lds_b32(const void *g, uint32_t lds) {
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
__device__ __forceinline__ void dma_lds_b128(const void *g, uint32_t lds) {
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
__device__ __forceinline__ void store_f32(float *g, float v) { asm volatile("global_store_dword %0, %1, off" ::"v"(g), "v"(v) : "memory"); }

// ------------------------------------------------------------------ the grouped GEMM stream
// A block (8 waves, 512 threads, one per CU) owns 128 weight rows -- gate/up: 64 gate rows (waves 0-3) and the 64
// up rows of the same outputs (waves 4-7); down: 128 rows -- and the work items blockIdx.y, + gridDim.y, ... (numbered
// expert by expert, up to 64 tokens each).  Its steps, (item, 256-value span b) in order, form one stream.  Every
// operand reaches LDS by DMA: a stage holds the 8 waves' 16-row weight tiles of span b (each one contiguous run of
// the tiled layout) and the item's 64 activation rows of span b.  D stages rotate: step s computes from stage s % D
// while the DMAs of steps s + 1 .. s + D - 1 are in flight.
//
// Waits are explicit.  Each wave issues the same L DMA instructions per step, and loads complete in issue order, so
// "vmcnt <= (D - 2) L" right before issuing step s + D - 1 means this wave's step-s DMAs have landed; a barrier
// then makes the whole stage visible and frees stage (s - 1) % D for the next issue.  Nothing in the stream is a
// compiler-visible global load, so the compiler adds no waits of its own.  The epilogue's stores are not counted:
// a store still in flight only makes a later wait stricter (loads cannot overtake the loads before them).
// Geometry of the stream kernel for weight type T, W waves (8 or 16) per block and B blocks per CU (1 or 2): the
// stages get what is left of the CU's 160 KB LDS after the item tables.
template <int T, int W, int B> struct G5 {
    static constexpr int WAVES = W, THREADS = 64 * W, ROWS = 16 * W;   // a wave owns 16 weight rows
    static constexpr int HALF = W / 2;                          // gate/up: waves 0 .. HALF - 1 in gate, the rest in up
    static constexpr int TPW = GM_TOK / W;                      // activation rows each wave fetches per step
    static constexpr int NA = TPW / 4;                          // their 1 KB DMA instructions
    static constexpr int PER = 1024 / THREADS;                  // expert groups per thread in the item scan
    static constexpr int ITEMS = B == 1 ? 16 : 8;               // items per segment (their tables live in LDS)
    static constexpr int LDS_STAGES = B == 1 ? 150 * 1024 : 72 * 1024;
    static constexpr int BB = block_bytes(T);                   // weight bytes per row and 256 values
    static constexpr int TB = 16 * BB;                          // one wave's 16-row tile of a span
    static constexpr int WB = W * TB;                           // weights of a stage
    static constexpr int AB = GM_TOK * 256;                     // activation values of a stage (64 rows of 256)
    static constexpr int SB = WB + AB + 4 * GM_TOK;             // + the rows' Q8_K d
    static constexpr int D = 4 * SB <= LDS_STAGES ? 4 : 3 * SB <= LDS_STAGES ? 3 : 2;   // stages
    static constexpr int N4 = TB / 1024, NR = TB - 1024 * N4, N1 = (NR + 255) / 256;   // tile DMAs: 1 KB, then 256 B
    static constexpr int L = N4 + N1 + NA + 1;                  // DMA instructions per wave and step
    static_assert(W == 8 || W == 16, "8 or 16 waves");
    static_assert(TB % 16 == 0 && NR % 4 == 0 && SB % 16 == 0, "DMA granules");
    static_assert(D * SB <= LDS_STAGES, "stages fit");
    static_assert((D - 2) * L <= 63, "vmcnt range");
};
// Q4_K and IQ4_XS gate/up (whose step fits 128 registers): two blocks of 8 waves per CU, each block's stream
// running independently of the other's; the rest: one block of 8 waves (up to 256 registers, deeper rings)
template <int T, bool GU> constexpr int g5_blocks() { return GU && (T == Q4_K || T == IQ4_XS) ? 2 : 1; }

__device__ __forceinline__ v4i mfma64(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
// byte `b` of x in both 16-bit halves / in all four bytes
__device__ __forceinline__ uint32_t bcast16(uint32_t x, int b) { return __builtin_amdgcn_perm(0u, x, 0x0C000C00u | (uint32_t) b | ((uint32_t) b << 16)); }
__device__ __forceinline__ uint32_t bcast8(uint32_t x, int b) { return __builtin_amdgcn_perm(0u, x, 0x01010101u * (uint32_t) b); }
// four bytes of q (each < 16) times the small factor f (< 8) held in both 16-bit halves: products < 128 stay in their bytes
__device__ __forceinline__ int mul_bytes(uint32_t q, uint32_t f) {
    const v2u16 r = __builtin_bit_cast(v2u16, q) * __builtin_bit_cast(v2u16, f);
    return (int) __builtin_bit_cast(uint32_t, r);
}

// Q4_K step on the 16x16x64 MFMA.  The dot products are exact integers, so the K order inside an MFMA is free: in MFMA
// j (values 64 j .. 64 j + 63 of the span) lane quarter q holds values 64 j + 16 q .. + 15, one contiguous 16-byte
// piece of the token row (A: a single LDS read straight into the operand registers) and, for B, the same values of the
// weight row: the low nibbles of qs[32 j + 16 q ..] (chunk 2j) for q < 2, the high nibbles of qs[32 j + 16 (q - 2) ..]
// (chunk 2j + 1) for q >= 2.  Every lane's 16 values lie in one chunk, so its 6-bit scale s = 8 a + b (a, b < 8) is
// applied inside B: D1 = sum a_c dot_c and D2 = sum b_c dot_c (a q, b q < 128 fit int8), sum_c s_c dot_c = 8 D1 + D2
// exactly; a third MFMA against the chunk mins gives sum_c m_c sum(x_c).
// Token tiles T0 .. T0 + NT - 1 (compile-time: straight-line code, accumulators only for the tiles present)
// The lane's constants (quarter, row, offsets, selectors) are derived in the step from a lane id the compiler cannot
// hoist: recomputing them costs a few instructions, keeping them live across the stream would cost registers.
__device__ __forceinline__ int lane_id_here() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}
template <int NT, int T0, bool FIRST>
__device__ __forceinline__ void step_q4k(const uint8_t *wl0, const int8_t *as, const float *yd, float (&acc)[GM_TILES][4]) {
    // the tiles past NT hold nothing this item reads (a tile count is fixed for an item, and an item's first span
    // writes its tiles without reading them): marking them redefined frees their registers in this step
#pragma unroll
    for (int t = T0 + NT; t < GM_TILES; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) asm volatile("" : "=v"(acc[t][v]));
    const int lid = lane_id_here(), q = lid >> 4, rr = lid & 15;
    const uint8_t *wl = wl0 + rr * block_bytes(Q4_K);
    const uint4 hd = *(const uint4 *) wl;   // d | dmin, scales[12]
    const uint32_t s_lo = hd.y & 0x3F3F3F3Fu, m_lo = hd.z & 0x3F3F3F3Fu;   // chunks 0..3, one per byte
    const uint32_t s_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);         // chunks 4..7
    const uint32_t m_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    const int hs = q >> 1;                   // 1: this lane takes the odd chunk of each pair (the high nibbles)
    const uint32_t nsh = 4u * (uint32_t) hs;
    const int8_t *arow = as + rr * 256;      // token row rr of tile 0; piece p of row t sits at p ^ (t % 16)
    const v4i z = {0, 0, 0, 0};
    v4i d1[NT], d2[NT], dm[NT];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 w = *(const uint4 *) (wl + 16 + 32 * j + 16 * (q & 1));
        const uint32_t sp = j < 2 ? s_lo : s_hi, mp = j < 2 ? m_lo : m_hi;
        const int c = ((2 * j) & 3) + hs;    // this lane's chunk, as a byte of sp / mp
        const uint32_t a = bcast16((sp >> 3) & 0x07070707u, c), b = bcast16(sp & 0x07070707u, c);
        const uint32_t n0 = (w.x >> nsh) & 0x0F0F0F0Fu, n1 = (w.y >> nsh) & 0x0F0F0F0Fu;
        const uint32_t n2 = (w.z >> nsh) & 0x0F0F0F0Fu, n3 = (w.w >> nsh) & 0x0F0F0F0Fu;
        const v4i B1 = {mul_bytes(n0, a), mul_bytes(n1, a), mul_bytes(n2, a), mul_bytes(n3, a)};
        const v4i B2 = {mul_bytes(n0, b), mul_bytes(n1, b), mul_bytes(n2, b), mul_bytes(n3, b)};
        const int mm = (int) bcast8(mp, c);
        const v4i Bm = {mm, mm, mm, mm};
        const int po = 16 * ((4 * j + q) ^ rr);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const v4i A = *(const v4i *) (arow + (T0 + t) * 16 * 256 + po);
            d1[t] = mfma64(A, B1, j ? d1[t] : z);
            d2[t] = mfma64(A, B2, j ? d2[t] : z);
            dm[t] = mfma64(A, Bm, j ? dm[t] : z);
            asm volatile("");   // a scheduling-region boundary: operands are not hoisted across tiles (register pressure)
        }
    }
    const float d = h2f(hd.x & 0xffff), dmin = h2f(hd.x >> 16);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int si = (d1[t][v] << 3) + d2[t][v];
            acc[T0 + t][v] = __builtin_fmaf(yd[(T0 + t) * 16 + 4 * q + v], __builtin_fmaf(d, (float) si, -(dmin * (float) dm[t][v])), FIRST ? 0.0f : acc[T0 + t][v]);
        }
    }
}

// 16 bytes at p, which is 2-byte aligned (sb = p & 3 is 0 or 2, the same for every call of a lane): five dwords from
// p - sb, joined; reads at most p + 18
__device__ __forceinline__ uint4 ld16_u2(const uint8_t *p, uint32_t sb) {
    const uint32_t *w = (const uint32_t *) (p - sb);
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2], d3 = w[3], d4 = w[4];
    return make_uint4(__builtin_amdgcn_alignbyte(d1, d0, sb), __builtin_amdgcn_alignbyte(d2, d1, sb),
                      __builtin_amdgcn_alignbyte(d3, d2, sb), __builtin_amdgcn_alignbyte(d4, d3, sb));
}
typedef short v2i16 __attribute__((ext_vector_type(2)));

// Q6_K step on the 16x16x64 MFMA.  In MFMA j (values 64 j .. + 63 of the span) lane quarter q holds values
// 64 j + 16 q .. + 15, which are exactly scale group g = 4 j + q: A is one contiguous 16-byte piece of the token row,
// B carries the group's scale, B = sc_g (q6 - 32) in [-4064, 4096], as two int8 planes B = 64 H + L (H = B >> 6 in
// [-64, 64], L = B & 63): D_H = X.H and D_L = X.L give sum_g sc_g dot_g = 64 D_H + D_L exactly.  The lane's values sit
// in ql[64 (j / 2) + 16 q ..] (nibble j % 2) and qh[32 (j / 2) + 16 (q % 2) ..] (bits 4 (j % 2) + 2 (q / 2)); rows of
// the 210-byte blocks are 2-byte aligned in LDS, so 16-byte reads go through ld16_u2.
template <int NT, int T0, bool FIRST>
__device__ __forceinline__ void step_q6k(const uint8_t *wt0, const int8_t *as, const float *yd, float (&acc)[GM_TILES][4]) {
    // the tiles past NT hold nothing this item reads (a tile count is fixed for an item, and an item's first span
    // writes its tiles without reading them): marking them redefined frees their registers in this step
#pragma unroll
    for (int t = T0 + NT; t < GM_TILES; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) asm volatile("" : "=v"(acc[t][v]));
    const int lid = lane_id_here(), q = lid >> 4, rr = lid & 15;
    const uint8_t *blk = wt0 + rr * block_bytes(Q6_K);
    const uint32_t sb = 2u * (uint32_t) (rr & 1);   // the tile starts dword-aligned; a 210-byte row shifts by 2
    const uint4 scq = ld16_u2(blk + 192, sb);       // the 16 group scales (int8)
    const float d = h2f(ld_u16(blk + 208));
    const int8_t *arow = as + rr * 256;
    const v4i z = {0, 0, 0, 0};
    v4i dh[NT], dl[NT];
    uint4 ql, qh;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if ((j & 1) == 0) {
            ql = ld16_u2(blk + 64 * (j >> 1) + 16 * q, sb);
            qh = ld16_u2(blk + 128 + 32 * (j >> 1) + 16 * (q & 1), sb);
        }
        const uint32_t scw = j == 0 ? scq.x : j == 1 ? scq.y : j == 2 ? scq.z : scq.w;
        const int sc = __builtin_amdgcn_sbfe((int) scw, 8 * q, 8);   // scale of group 4 j + q
        const uint32_t sc16 = ((uint32_t) sc & 0xffffu) * 0x10001u, off16 = ((uint32_t) (-32 * sc) & 0xffffu) * 0x10001u;
        const uint32_t hsh = 4u * (uint32_t) (j & 1) + 2u * (uint32_t) (q >> 1);
        const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w}, qhw[4] = {qh.x, qh.y, qh.z, qh.w};
        int H[4], L[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t nib = ((j & 1) ? qlw[i] >> 4 : qlw[i]) & 0x0F0F0F0Fu;
            const uint32_t qv = nib | (((qhw[i] >> hsh) & 0x03030303u) << 4);   // four 6-bit values, one per byte
            // values 0, 1 and 2, 3 in 16-bit lanes: B = q sc - 32 sc, exact in 16 bits
            const v2u16 e = __builtin_bit_cast(v2u16, __builtin_amdgcn_perm(0u, qv, 0x0C010C00u));
            const v2u16 o = __builtin_bit_cast(v2u16, __builtin_amdgcn_perm(0u, qv, 0x0C030C02u));
            const v2u16 s2 = __builtin_bit_cast(v2u16, sc16), c2 = __builtin_bit_cast(v2u16, off16);
            const v2u16 be = e * s2 + c2, bo = o * s2 + c2;
            const uint32_t ube = __builtin_bit_cast(uint32_t, be), ubo = __builtin_bit_cast(uint32_t, bo);
            L[i] = (int) (__builtin_amdgcn_perm(ubo, ube, 0x06040200u) & 0x3F3F3F3Fu);
            const v2i16 he = __builtin_bit_cast(v2i16, be) >> (short) 6, ho = __builtin_bit_cast(v2i16, bo) >> (short) 6;
            H[i] = (int) __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ho), __builtin_bit_cast(uint32_t, he), 0x06040200u);
        }
        const v4i Bh = {H[0], H[1], H[2], H[3]}, Bl = {L[0], L[1], L[2], L[3]};
        const int po = 16 * ((4 * j + q) ^ rr);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const v4i A = *(const v4i *) (arow + (T0 + t) * 16 * 256 + po);
            dh[t] = mfma64(A, Bh, j ? dh[t] : z);
            dl[t] = mfma64(A, Bl, j ? dl[t] : z);
            asm volatile("");   // a scheduling-region boundary: operands are not hoisted across tiles (register pressure)
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int si = (dh[t][v] << 6) + dl[t][v];
            acc[T0 + t][v] = __builtin_fmaf(yd[(T0 + t) * 16 + 4 * q + v], d * (float) si, FIRST ? 0.0f : acc[T0 + t][v]);
        }
    }
    asm volatile("");   // keeps the tile-count variants from being merged (which moved the accumulators to memory)
}

__host__ __device__ constexpr int xcd_gcd8(int n) { return (n & 7) == 0 ? 8 : (n & 3) == 0 ? 4 : (n & 1) == 0 ? 2 : 1; }


// floor(p / a) as a multiply-high, with a_mul = ceil(2^32 / a): exact while p * (a_mul * a - 2^32) < 2^32, which
// p * a < 2^32 guarantees (the launchers check it)
__device__ __forceinline__ uint32_t div_by_mul(uint32_t p, uint64_t a_mul) { return (uint32_t) (((uint64_t) p * a_mul) >> 32); }
static inline uint64_t div_mul_of(int a) { return ((1ull << 32) + (uint64_t) a - 1) / (uint64_t) a; }

template <int T, bool GU, int W, int B>
__global__ __launch_bounds__(64 * W, B * W / 4) void k_gemm(hy_moe_dev m, const uint8_t *__restrict__ aq, uint64_t a_mul, const int *__restrict__ order,
                                                        const int *__restrict__ order_n, const int *__restrict__ egrp, const float *__restrict__ wts,
                                                        float *__restrict__ out) {
    static_assert(vec_dot_type(T) != Q8_0, "the Q8_0-activation types run k_gemm_nl");
    using C = G5<T, W, B>;
    constexpr int D = C::D, AQ = Q8K_BYTES;
    __shared__ __align__(16) uint8_t smem[D * C::SB];   // stage s at s * SB: weights [wave][TB], activations [64][256], d [64]
    __shared__ uint64_t s_scan[1024 + C::WAVES];                // per expert group: exclusive prefix of its items per tile class
    __shared__ int s_item[C::ITEMS][3];                  // first pair in order, tokens, weight slot
    __shared__ int s_pair[C::ITEMS][GM_TOK];             // pair index of each token of the segment's items
    __shared__ float s_wt[GU ? 1 : C::ITEMS][GM_TOK];    // down: their route weights
    __shared__ uint2 grid[iq2_lds(T)];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, rr = lane & 15, q = lane >> 4;
    const int na = order_n[1];
    // ---- items.  Expert group g (cnt tokens) owns ceil(cnt / 64) items: full ones of 4 token tiles and a last one of
    // ceil(rem / 16) tiles.  Items are ordered by tile count (class 4: full items and last items of 4 tiles, expert by
    // expert; then the last items of 3, 2 and 1 tiles) and dealt to the gridDim.y item slots in snake order (slot y
    // takes positions k S + y for even k and k S + S - 1 - y for odd k), which evens out the slots' work.
    // s_scan holds each group's exclusive prefix of the four class counts, 16 bits each (item totals stay below 2^16).
    {
        uint64_t c2[C::PER], loc = 0;
#pragma unroll
        for (int i = 0; i < C::PER; ++i) {
            const int g = C::PER * tid + i;
            uint64_t c = 0;
            if (g < na) {
                const int cnt = egrp[3 * g + 2], n = (cnt + GM_TOK - 1) / GM_TOK, cl = (cnt - GM_TOK * (n - 1) + 15) >> 4;
                c = (uint64_t) (n - 1 + (cl == 4)) | ((uint64_t) (cl == 3) << 16) | ((uint64_t) (cl == 2) << 32) | ((uint64_t) (cl == 1) << 48);
            }
            c2[i] = c;
            loc += c;
        }
        uint64_t inc = loc;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) { const uint64_t t = __shfl_up(inc, o); if (lane >= o) inc += t; }
        if (lane == 63) s_scan[1024 + wave] = inc;
        __syncthreads();
        uint64_t base = 0;
        for (int w = 0; w < wave; ++w) base += s_scan[1024 + w];
        uint64_t ex = base + inc - loc;
#pragma unroll
        for (int i = 0; i < C::PER; ++i) { s_scan[C::PER * tid + i] = ex; ex += c2[i]; }
        if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
        __syncthreads();
    }
    uint64_t tot = 0;
    for (int w = 0; w < C::WAVES; ++w) tot += s_scan[1024 + w];
    const int n4 = (int) (tot & 0xffff), n3 = (int) ((tot >> 16) & 0xffff), n2 = (int) ((tot >> 32) & 0xffff), n1 = (int) (tot >> 48);
    const int total = n4 + n3 + n2 + n1;
    // Block (x, y) runs on XCD (x + gridDim.x y) % 8, and each XCD has its own L2.  This block's logical row block
    // bx and item slot y0: with gridDim.y a multiple of 8 (the host's choice from 8 slots up), XCD c takes the slots
    // c ys / 8 .. (c + 1) ys / 8 - 1, each with all its row blocks -- an item's activation rows are fetched into one
    // L2 and read there by every row block, and runs of consecutive item positions (mostly one expert's items) share
    // their weight tiles there.  Fewer slots: logical slots l, l + 1, ... sit P = 8 / gcd(gridDim.x, 8) physical
    // slots apart (P = 1 unless gridDim.y is a multiple of it): the same XCD for every row block, the weights shared.
    const int ys = gridDim.y;
    int bx, y0;
    if (ys % 8 == 0) {
        const int b = (int) blockIdx.x + (int) gridDim.x * (int) blockIdx.y;
        bx = (b >> 3) % (int) gridDim.x;
        y0 = (b & 7) * (ys / 8) + (b >> 3) / (int) gridDim.x;
    } else {
        const int P0 = 8 / xcd_gcd8((int) gridDim.x), P = ys % P0 == 0 ? P0 : 1;
        bx = blockIdx.x;
        y0 = ((int) blockIdx.y % P) * (ys / P) + (int) blockIdx.y / P;
    }
    const int rounds = total / ys, rem_items = total - rounds * ys;
    const int my_items = rounds + (((rounds & 1) ? ys - 1 - y0 : y0) < rem_items ? 1 : 0);
    if (my_items == 0) return;   // uniform over the block
    const int in_dim = GU ? m.n : m.ff, nsb = in_dim / 256;
    const size_t mbytes = GU ? m.gate_bytes : m.down_bytes;
    // this wave's 16 rows: tile index (rows / 16) in its matrix, and the output row of each lane
    const int tile_row = GU ? bx * C::HALF + wave % C::HALF : bx * C::WAVES + wave;
    const int row = 16 * tile_row + rr;
    const uint8_t *Wmat = (GU ? (wave < C::HALF ? m.gate : m.up) : m.down) + (size_t) tile_row * nsb * C::TB;
    const size_t arow = (size_t) nsb * AQ;
    auto stage_w = [&](int s) { return smem + s * C::SB; };
    auto stage_a = [&](int s) { return (int8_t *) (smem + s * C::SB + C::WB); };
    auto stage_d = [&](int s) { return (const float *) (smem + s * C::SB + C::WB + C::AB); };

    for (int seg = 0; seg < my_items; seg += C::ITEMS) {
        const int nit = min(C::ITEMS, my_items - seg);
        __syncthreads();   // readers of the previous segment's tables are done
        for (int i = tid; i < nit; i += C::THREADS) {
            const int k = seg + i;
            int pos = k * ys + ((k & 1) ? ys - 1 - y0 : y0);   // position in the class order
            int cls = 0;                                        // field of s_scan: 0 = 4 tiles, 1 = 3, 2 = 2, 3 = 1
            if (pos >= n4) { pos -= n4; cls = 1; if (pos >= n3) { pos -= n3; cls = 2; if (pos >= n2) { pos -= n2; cls = 3; } } }
            int lo = 0, hi = na - 1;   // last group whose prefix in the class <= pos: the group that owns the item
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if ((int) ((s_scan[mid] >> (16 * cls)) & 0xffff) <= pos) lo = mid; else hi = mid - 1;
            }
            const int cnt = egrp[3 * lo + 2];
            const int chunk = cls == 0 ? pos - (int) (s_scan[lo] & 0xffff) : (cnt - 1) / GM_TOK;
            const int tok0 = chunk * GM_TOK;
            s_item[i][0] = egrp[3 * lo + 1] + tok0;
            s_item[i][1] = min(GM_TOK, cnt - tok0);
            s_item[i][2] = m.slot[egrp[3 * lo]];
        }
        __syncthreads();
        for (int i = tid; i < nit * GM_TOK; i += C::THREADS) {
            const int it = i / GM_TOK, tk = i - it * GM_TOK;
            const int pr = tk < s_item[it][1] ? order[s_item[it][0] + tk] : -1;
            s_pair[it][tk] = pr;
            if (!GU) s_wt[GU ? 0 : it][tk] = pr >= 0 ? wts[pr] : 0.0f;
        }
        __syncthreads();
        const int nsteps = nit * nsb;

        // ---- issue: the DMAs of step (iss_it, iss_b) into stage iss_stage, then advance (staying on the last step
        // once there).  Activation rows: this wave's tokens 8 wave + 4 i + lane / 16 (lane l fetches 16-byte piece
        // (l % 16) ^ (t % 16) of token t, the conflict-free layout the MFMA reads use) and, on lanes 0-7, the d of
        // tokens 8 wave + lane.  Absent tokens are not fetched (their LDS rows keep stale bytes, whose MFMA columns
        // are never stored); lane 0 of an instruction fetches from the item's first row when its token is absent.
        // Offsets are bytes from aq (the caller's activations stay below 4 GB).
        uint32_t aoff[C::NA], doff;
        int iss_it = 0, iss_b = 0, iss_stage = 0, iss_step = 0, iss_ntok = 0;
        const uint32_t lane16 = 16 * lane, lane4 = 4 * lane;
        auto issue = [&]() {
            const int it = iss_it, b = iss_b;
            if (b == 0) {
                const int ntok = __builtin_amdgcn_readfirstlane(s_item[it][1]);   // uniform: a scalar register
                iss_ntok = ntok;
                const int p0 = s_pair[it][0];
#pragma unroll
                for (int i = 0; i < C::NA; ++i) {
                    const int t = C::TPW * wave + 4 * i + (lane >> 4);
                    const int pr = t < ntok ? s_pair[it][t] : p0;
                    aoff[i] = (GU ? div_by_mul((uint32_t) pr, a_mul) : (uint32_t) pr) * (uint32_t) arow + 4 + 16 * ((lane & 15) ^ (t & 15));
                }
                const int td = C::TPW * wave + (lane & (C::TPW - 1));
                const int prd = td < ntok ? s_pair[it][td] : p0;
                doff = (GU ? div_by_mul((uint32_t) prd, a_mul) : (uint32_t) prd) * (uint32_t) arow;
            }
            const int stage = iss_stage;
            const uint8_t *wsrc = Wmat + (size_t) __builtin_amdgcn_readfirstlane(s_item[it][2]) * mbytes + (size_t) b * C::TB;
            const uint32_t wdst = lds_addr(stage_w(stage) + wave * C::TB);
#pragma unroll
            for (int i = 0; i < C::N4; ++i) dma_s128(wsrc + 1024 * i, lane16, wdst + 1024 * i);
#pragma unroll
            for (int j = 0; j < C::N1; ++j)
                if (256 * j + 4 * lane < C::NR) dma_s32(wsrc + 1024 * C::N4 + 256 * j, lane4, wdst + 1024 * C::N4 + 256 * j);
            const uint32_t bo = (uint32_t) b * AQ;
            const uint32_t adst = lds_addr(stage_a(stage) + C::TPW * wave * 256);
            // lanes of absent tokens sit out, except lane 0, so that every instruction issues (the waits count them)
#pragma unroll
            for (int i = 0; i < C::NA; ++i)
                if (C::TPW * wave + 4 * i + (lane >> 4) < iss_ntok || lane == 0) dma_s128(aq, aoff[i] + bo, adst + 1024 * i);
            if (lane < C::TPW && (C::TPW * wave + lane < iss_ntok || lane == 0)) dma_s32(aq, doff + bo, lds_addr(stage_d(stage) + C::TPW * wave));
            if (iss_step < nsteps - 1) {
                ++iss_step;
                if (++iss_b == nsb) { iss_b = 0; ++iss_it; }
            }
            iss_stage = iss_stage == D - 1 ? 0 : iss_stage + 1;
            // uniform counters: kept in scalar registers (the compiler cannot prove them uniform by itself)
            iss_it = __builtin_amdgcn_readfirstlane(iss_it);
            iss_b = __builtin_amdgcn_readfirstlane(iss_b);
            iss_step = __builtin_amdgcn_readfirstlane(iss_step);
            iss_stage = __builtin_amdgcn_readfirstlane(iss_stage);
        };

        float acc[GM_TILES][4];
#pragma unroll
        for (int i = 0; i < GM_TILES; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i][v] = 0.0f;
        auto compute = [&](int it, int b, int stage) {
            const int ntok = __builtin_amdgcn_readfirstlane(s_item[it][1]), ntile = (ntok + 15) >> 4;   // uniform
            const int8_t *as = stage_a(stage);
            const float *yd = stage_d(stage);
            if constexpr (T == Q4_K) {
                // straight-line code per tile count
                const uint8_t *wt = stage_w(stage) + wave * C::TB;
                static_assert(GM_TILES == 4, "one case per tile count");
                // an item's first span starts its accumulators (fmaf with +0, the bits of a sum begun at 0): no reset
                // after the epilogue, so the accumulators stay in the same registers on every path through the loop
                if (b == 0) {
                    switch (ntile) {
                    case 1: step_q4k<1, 0, true>(wt, as, yd, acc); break;
                    case 2: step_q4k<2, 0, true>(wt, as, yd, acc); break;
                    case 3: step_q4k<3, 0, true>(wt, as, yd, acc); break;
                    default: step_q4k<4, 0, true>(wt, as, yd, acc); break;
                    }
                } else {
                    switch (ntile) {
                    case 1: step_q4k<1, 0, false>(wt, as, yd, acc); break;
                    case 2: step_q4k<2, 0, false>(wt, as, yd, acc); break;
                    case 3: step_q4k<3, 0, false>(wt, as, yd, acc); break;
                    default: step_q4k<4, 0, false>(wt, as, yd, acc); break;
                    }
                }
            } else if constexpr (T == Q6_K) {
                const uint8_t *wt = stage_w(stage) + wave * C::TB;
                if (b == 0) {
                    switch (ntile) {
                    case 1: step_q6k<1, 0, true>(wt, as, yd, acc); break;
                    case 2: step_q6k<2, 0, true>(wt, as, yd, acc); break;
                    case 3: step_q6k<3, 0, true>(wt, as, yd, acc); break;
                    default: step_q6k<4, 0, true>(wt, as, yd, acc); break;
                    }
                } else {
                    switch (ntile) {
                    case 1: step_q6k<1, 0, false>(wt, as, yd, acc); break;
                    case 2: step_q6k<2, 0, false>(wt, as, yd, acc); break;
                    case 3: step_q6k<3, 0, false>(wt, as, yd, acc); break;
                    default: step_q6k<4, 0, false>(wt, as, yd, acc); break;
                    }
                }
            } else {
            Raw<T> wr;
            wr.load(stage_w(stage) + wave * C::TB + rr * C::BB, q);
            int si[GM_TILES][4];
            v4i sm[GM_TILES];
#pragma unroll
            for (int i = 0; i < GM_TILES; ++i) {
#pragma unroll
                for (int v = 0; v < 4; ++v) si[i][v] = 0;
                sm[i] = v4i{0, 0, 0, 0};
            }
            if constexpr (B == 1 && W == 8) {
                // the step's activation fragments (tile, chunk) read from LDS up front: one LDS round trip a step
                // instead of one per chunk and tile (the register budget of one 8-wave block per CU has room for them)
                long af[GM_TILES][8];
#pragma unroll
                for (int tile = 0; tile < GM_TILES; ++tile) {
                    if (tile >= ntile) break;
#pragma unroll
                    for (int c = 0; c < 8; ++c) af[tile][c] = a_frag<true>(as, tile, rr, c, q);
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) chunk_ints<T, true>(wr, c, q, grid, as, rr, ntile, si, sm, af);
            } else {
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    chunk_ints<T, true>(wr, c, q, grid, as, rr, ntile, si, sm);
                    // 16 waves (128 registers): a scheduling-region boundary per chunk, so that the next chunks'
                    // operand reads are not hoisted into this one (which spilled)
                    if constexpr (W == 16) asm volatile("");
                }
            }
#pragma unroll
            for (int tile = 0; tile < GM_TILES; ++tile) {
                if (tile >= ntile) break;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[tile][v] = __builtin_fmaf(yd[tile * 16 + 4 * q + v], wr.fold(si[tile][v], sm[tile][v]), acc[tile][v]);
            }
            }
            if (b != nsb - 1) return;
            // ---- the item's outputs, through this stage (every wave has finished reading it after a barrier), TOKP
            // tokens a pass: the waves' accumulators go there token-major -- rows padded by one float against bank
            // conflicts -- and wave w finishes tokens w, w + WAVES, ... of the pass: one output row per lane (SwiGLU
            // of the gate and up values, or the route weight times the down value), stored as whole rows.
            constexpr int OR = GU ? 16 * C::HALF : C::ROWS;   // output rows of the block
            constexpr int LD = OR + 1;                         // floats per token in LDS
            constexpr int NCOPY = GU ? 2 : 1;
            constexpr int TOKP = NCOPY * 64 * LD * 4 <= C::WB + C::AB ? 64 : NCOPY * 32 * LD * 4 <= C::WB + C::AB ? 32 : 16;
            static_assert(NCOPY * TOKP * LD * 4 <= C::WB + C::AB, "the exchange fits in a stage");
            float *s_o = (float *) stage_w(stage);             // gate (or down) values
            float *s_u = s_o + TOKP * LD;                      // up values
            const int row0 = bx * OR;
            for (int p0 = 0; p0 < ntok; p0 += TOKP) {
                lds_barrier();   // the stage (or the previous pass) is no longer read
                {
                    float *dst = GU && wave >= C::HALF ? s_u : s_o;
                    const int orow = (GU ? wave % C::HALF : wave) * 16 + rr;
#pragma unroll
                    for (int tile = 0; tile < GM_TILES; ++tile) {
                        if (tile >= ntile) break;
                        if (tile * 16 < p0 || tile * 16 >= p0 + TOKP) continue;
#pragma unroll
                        for (int v = 0; v < 4; ++v) dst[(tile * 16 - p0 + 4 * q + v) * LD + orow] = acc[tile][v];
                    }
                }
                lds_barrier();
                for (int tok = p0 + wave; tok < min(ntok, p0 + TOKP); tok += C::WAVES) {
                    float *o = out + (size_t) s_pair[it][tok] * (GU ? m.ff : m.n) + row0;
                    const float wt = GU ? 0.0f : s_wt[GU ? 0 : it][tok];
                    const float *so = s_o + (tok - p0) * LD, *su = s_u + (tok - p0) * LD;
#pragma unroll
                    for (int r = lane; r < OR; r += 64) store_f32(o + r, GU ? hy_swiglu(so[r], su[r], m.clamp) : wt * so[r]);
                }
            }
            if constexpr (T != Q4_K && T != Q6_K) {   // (the Q4_K / Q6_K steps start the next item's sums themselves)
#pragma unroll
                for (int tile = 0; tile < GM_TILES; ++tile)
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[tile][v] = 0.0f;
            }
        };

        // the stream: steps 0 .. D - 2 issued ahead; past the end, the last step is issued again (into the stage
        // of step s - 1, which nobody reads any more) so that every wait counts the same instructions
#pragma unroll
        for (int s = 0; s < D - 1; ++s) issue();
        for (int st = 0, it = 0, b = 0, stage = 0; st < nsteps; ++st) {
            wait_vm<(D - 2) * C::L>();
            lds_barrier();
            issue();
            compute(it, b, stage);
            if (++b == nsb) { b = 0; ++it; }
            stage = stage == D - 1 ? 0 : stage + 1;
        }
        wait_vm<0>();   // no DMA into this block's LDS may outlive the segment
    }
}

// IQ4_NL / Q8_0 / MXFP4 / Q5_0 / Q5_1: one chunk's MFMA per tile folded straight into the fp32 accumulators (Yc: 8 block scales per token)
template <int T>
__device__ __forceinline__ void chunk_fold(const Raw<T> &w, int c, int q, const int8_t *As, const float *Yc, int rr, int ntile,
                                           float (&acc)[GM_TILES][4]) {
    const v4i z = {0, 0, 0, 0};
    uint32_t b0, b1;
    int s0, s1, mn;
    w.chunk(c, q, nullptr, b0, b1, s0, s1, mn);
#pragma unroll
    for (int tile = 0; tile < GM_TILES; ++tile) {
        if (tile >= ntile) break;
        const long a = *(const long *) (As + (tile * 16 + rr) * GM_LD + 32 * c + 8 * q);
        const v4i d0 = mfma16(a, mk_long(b0, b1), z);
        if constexpr (ysum_type(T)) {   // each token's block sum: the same A against ones
            const v4i d1 = mfma16(a, mk_long(0x01010101u, 0x01010101u), z);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[tile][v] = __builtin_fmaf(Yc[(tile * 16 + 4 * q + v) * 8 + c], w.cfold2(c, d0[v], d1[v]), acc[tile][v]);
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[tile][v] = __builtin_fmaf(Yc[(tile * 16 + 4 * q + v) * 8 + c], w.cfold(c, d0[v]), acc[tile][v]);
        }
    }
}

// IQ4_NL, Q8_0, MXFP4, Q5_0 and Q5_1 weights (Q8_0 activations, whose 2-byte aligned blocks the LDS DMA above cannot stage): register-staged
// stream, one step ahead.  A block walks the work items it, it + gridDim.y, ...; the (item, block) steps form one stream in which the
// next step's weight and activation bytes are loaded while the current step computes, across item boundaries.
template <int T, bool GU>
__global__ __launch_bounds__(256) void k_gemm_nl(hy_moe_dev m, const uint8_t *__restrict__ aq, int a_div, const int *__restrict__ order,
                                              const int *__restrict__ order_n, const int *__restrict__ egrp, const float *__restrict__ wts,
                                              float *__restrict__ out) {
    __shared__ __align__(16) int8_t As[2][GM_TOK * GM_LD];
    constexpr bool NL = vec_dot_type(T) == Q8_0;     // Q8_0 activations, per-block fold (IQ4_NL, Q8_0, MXFP4, Q5_0, Q5_1)
    __shared__ float Yd[2][GM_TOK * (NL ? 8 : 1)];
    __shared__ int s_scan[1024 + 8];
    __shared__ float s_up[GU ? 32 * GM_TOK : 1];
    __shared__ uint2 grid[iq2_lds(T)];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, rr = lane & 15, q = lane >> 4;
    const int na = order_n[1];
    // ---- items: expert group g owns ceil(cnt_g / GM_TOK) of them; s_scan = exclusive prefix (block-wide)
    {
        int c4[4], loc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = 4 * tid + i;
            c4[i] = g < na ? (egrp[3 * g + 2] + GM_TOK - 1) / GM_TOK : 0;
            loc += c4[i];
        }
        int inc = loc;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) { const int t = __shfl_up(inc, o); if (lane >= o) inc += t; }
        if (lane == 63) s_scan[1024 + wave] = inc;
        __syncthreads();
        int base = 0;
        for (int w = 0; w < wave; ++w) base += s_scan[1024 + w];
        int ex = base + inc - loc;
#pragma unroll
        for (int i = 0; i < 4; ++i) { s_scan[4 * tid + i] = ex; ex += c4[i]; }
        if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
        __syncthreads();
    }
    const int total = s_scan[1024] + s_scan[1025] + s_scan[1026] + s_scan[1027];
    int it = blockIdx.y;
    if (it >= total) return;
    const int rows = GU ? m.ff : m.n, in_dim = GU ? m.n : m.ff, nsb = in_dim / 256;
    const int orows = GU ? 32 : GM_ROWS;
    const int row = blockIdx.x * orows + (GU ? (wave & 1) : wave) * 16 + rr;
    const bool row_ok = row < rows;
    const size_t mbytes = GU ? m.gate_bytes : m.down_bytes;
    const uint8_t *Wbase = (GU ? (wave < 2 ? m.gate : m.up) : m.down) + tiled_off(row_ok ? row : rows - 1, 0, nsb, span_bytes(T));
    constexpr int AB = NL ? 8 * Q8_0_BYTES : Q8K_BYTES;   // activation bytes per 256 values
    const size_t arow = (size_t) nsb * AB;
    constexpr int BB = NL ? 8 * block_bytes(T) : block_bytes(T);   // weight bytes per 256 values
    const int st_tok = tid >> 2, st_part = tid & 3;   // staging: 64 bytes of token st_tok per thread

    // item -> (first pair in order, tokens, weight pointer); the staging thread's activation row
    struct ItemState { int start, ntok; const uint8_t *W; const uint8_t *src; };
    auto locate = [&](int item) {
        int lo = 0, hi = na - 1;   // last group whose prefix <= item
        while (lo < hi) { const int mid = (lo + hi + 1) >> 1; if (s_scan[mid] <= item) lo = mid; else hi = mid - 1; }
        const int tok0 = (item - s_scan[lo]) * GM_TOK;
        ItemState st;
        st.start = egrp[3 * lo + 1] + tok0;
        st.ntok = min(GM_TOK, egrp[3 * lo + 2] - tok0);
        st.W = Wbase + (size_t) m.slot[egrp[3 * lo]] * mbytes;
        st.src = nullptr;
        if (st_tok < st.ntok) {
            const int p = order[st.start + st_tok];
            st.src = aq + (size_t) (GU ? p / a_div : p) * arow;
        }
        return st;
    };
    auto load_a = [&](const uint8_t *src, int b, uint4 (&a)[4], float (&yd)[2]) {
        if (src) {
            const uint8_t *s = src + (size_t) b * AB;
            if constexpr (NL) {   // Q8_0 blocks 2 st_part, 2 st_part + 1: qs at 68 p + 2 (2 mod 4) and 68 p + 36
                const uint8_t *p0 = s + 2 * Q8_0_BYTES * st_part;
                a[0] = load16_a2(p0 + 2); a[1] = load16_a2(p0 + 18);
                a[2] = load16_a4(p0 + 36); a[3] = load16_a4(p0 + 52);
                yd[0] = h2f(ld_u16(p0)); yd[1] = h2f(ld_u16(p0 + Q8_0_BYTES));
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = load16_a4(s + 4 + 64 * st_part + 16 * i);
                yd[0] = *(const float *) s; yd[1] = 0.0f;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = make_uint4(0, 0, 0, 0);
            yd[0] = yd[1] = 0.0f;
        }
    };

    ItemState cur = locate(it);
    Raw<T> w;
    w.load(cur.W, q);
    uint4 a[4];
    float yd[2];
    load_a(cur.src, 0, a, yd);
    float acc[GM_TILES][4];
#pragma unroll
    for (int i = 0; i < GM_TILES; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][v] = 0.0f;
    int b = 0, buf = 0;
    for (;;) {
        {
            uint4 *dst = (uint4 *) (As[buf] + st_tok * GM_LD + 64 * st_part);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = a[i];
            if constexpr (NL) { Yd[buf][st_tok * 8 + 2 * st_part] = yd[0]; Yd[buf][st_tok * 8 + 2 * st_part + 1] = yd[1]; }
            else if (st_part == 0) Yd[buf][st_tok] = yd[0];
        }
        // the next step: block b + 1 of this item, or block 0 of the next item
        const bool last_b = b + 1 == nsb;
        const int nit = last_b ? it + (int) gridDim.y : it;
        const bool more = nit < total;
        ItemState nxt = cur;
        Raw<T> nw;
        if (more) {
            if (last_b) nxt = locate(nit);
            const int nb = last_b ? 0 : b + 1;
            nw.load(nxt.W + (size_t) nb * (HY_TILE * BB), q);
            load_a(nxt.src, nb, a, yd);
        }
        __syncthreads();
        const int ntile = (cur.ntok + 15) / 16;
        if constexpr (NL) {
#pragma unroll
            for (int c = 0; c < 8; ++c) chunk_fold<T>(w, c, q, As[buf], Yd[buf], rr, ntile, acc);
        } else {
            int si[GM_TILES][4];
            v4i sm[GM_TILES];
#pragma unroll
            for (int i = 0; i < GM_TILES; ++i) {
#pragma unroll
                for (int v = 0; v < 4; ++v) si[i][v] = 0;
                sm[i] = v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) chunk_ints<T>(w, c, q, grid, As[buf], rr, ntile, si, sm);
#pragma unroll
            for (int tile = 0; tile < GM_TILES; ++tile) {
                if (tile >= ntile) break;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[tile][v] = __builtin_fmaf(Yd[buf][tile * 16 + 4 * q + v], w.fold(si[tile][v], sm[tile][v]), acc[tile][v]);
            }
        }
        if (last_b) {   // the item's outputs
            if (GU && wave >= 2) {
#pragma unroll
                for (int tile = 0; tile < GM_TILES; ++tile)
#pragma unroll
                    for (int v = 0; v < 4; ++v) s_up[((wave & 1) * 16 + rr) * GM_TOK + tile * 16 + 4 * q + v] = acc[tile][v];
            }
            if (GU) __syncthreads();
            if (!GU || wave < 2) {
#pragma unroll
                for (int tile = 0; tile < GM_TILES; ++tile) {
                    if (tile >= ntile) break;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int tok = tile * 16 + 4 * q + v;
                        if (tok < cur.ntok && row_ok) {
                            const int p = order[cur.start + tok];
                            if (GU) out[(size_t) p * m.ff + row] = hy_swiglu(acc[tile][v], s_up[((wave & 1) * 16 + rr) * GM_TOK + tok], m.clamp);
                            else out[(size_t) p * m.n + row] = wts[p] * acc[tile][v];
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < GM_TILES; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[i][v] = 0.0f;
        }
        if (!more) break;
        cur = nxt;
        it = nit;
        b = last_b ? 0 : b + 1;
        buf ^= 1;
        w = nw;
    }
}

#define HY_GEMM_SWITCH(T, ...)                                                                    \
    switch (T) {                                                                                   \
    case Q4_K: { constexpr int TT = Q4_K; __VA_ARGS__; }                                                 \
    case Q5_K: { constexpr int TT = Q5_K; __VA_ARGS__; }                                                 \
    case Q6_K: { constexpr int TT = Q6_K; __VA_ARGS__; }                                                 \
    case IQ4_XS: { constexpr int TT = IQ4_XS; __VA_ARGS__; }                                             \
    case IQ2_XS: { constexpr int TT = IQ2_XS; __VA_ARGS__; }                                             \
    case IQ2_XXS: { constexpr int TT = IQ2_XXS; __VA_ARGS__; }                                           \
    case Q2_K: { constexpr int TT = Q2_K; __VA_ARGS__; }                                                 \
    case Q3_K: { constexpr int TT = Q3_K; __VA_ARGS__; }                                                 \
    case IQ3_XXS: { constexpr int TT = IQ3_XXS; __VA_ARGS__; }                                           \
    case IQ3_S: { constexpr int TT = IQ3_S; __VA_ARGS__; }                                               \
    case IQ2_S: { constexpr int TT = IQ2_S; __VA_ARGS__; }                                               \
    case IQ1_S: { constexpr int TT = IQ1_S; __VA_ARGS__; }                                               \
    default: set_error("grouped GEMM: unsupported expert type %d", (int) (T)); return HY_EUNSUPPORTED_TYPE; \
    }

// k_gemm keeps each expert group's item prefix per tile class in a 16-bit field of s_scan: the item total of a launch
// must stay below 2^16 (checked against the upper bound below, from the host)
constexpr int GM_MAX_ITEMS = 1 << 16;
// upper bound of the work items: sum over active experts of ceil(cnt / GM_TOK) <= ceil(P / GM_TOK) + active
static int max_items(int n_pairs, int max_active) { return (n_pairs + GM_TOK - 1) / GM_TOK + max_active; }
// the current device's CU count (an attribute query: cheap, thread-safe, and right for each device)
static int cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    return cus;
}
// item slots per row tile: enough blocks for about `per_cu` resident blocks on every CU.  k_gemm (`xcd`) groups its
// slots by XCD when they are a multiple of 8, else places consecutive items P slots apart: from 8 slots up a
// multiple of 8, else of P where there are that many.
static int item_slots(int row_tiles, int n_pairs, int max_active, int per_cu, bool xcd = false) {
    const int want = cu_count() * per_cu / row_tiles;   // every block resident at once
    const int n = std::max(1, std::min(max_items(n_pairs, max_active), want));
    if (xcd && n >= 8) return n / 8 * 8;
    const int P = 8 / xcd_gcd8(row_tiles);
    return n >= P ? n / P * P : n;
}

int launch_gemm_gate_up(const hy_moe_dev &m, const void *xq, int k, int n_pairs, const int *order, const int *order_n, const int *egrp,
                        int max_active, float *h, hipStream_t s) {
    if (max_active <= 0 || n_pairs <= 0) return HY_OK;
    const int rt = (m.ff + 31) / 32;
    if (vec_dot_type(m.tg) == Q8_0) {
        dim3 grid(rt, item_slots(rt, n_pairs, max_active, 3));
        if (m.tg == IQ4_NL) hipLaunchKernelGGL((k_gemm_nl<IQ4_NL, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp, nullptr, h);
        else if (m.tg == MXFP4) hipLaunchKernelGGL((k_gemm_nl<MXFP4, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp, nullptr, h);
        else if (m.tg == Q5_0) hipLaunchKernelGGL((k_gemm_nl<Q5_0, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp, nullptr, h);
        else if (m.tg == Q5_1) hipLaunchKernelGGL((k_gemm_nl<Q5_1, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp, nullptr, h);
        else hipLaunchKernelGGL((k_gemm_nl<Q8_0, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp, nullptr, h);
        return check_launch("hy_moe_gemm_gate_up");
    }
    if ((size_t) n_pairs * (m.n / 256) * Q8K_BYTES >= (1ull << 32)) { set_error("hy_moe_gemm_gate_up: activations of 4 GB or more"); return HY_EBAD_SHAPE; }
    if (k <= 0 || (uint64_t) n_pairs * (uint64_t) k >= (1ull << 32)) { set_error("hy_moe_gemm_gate_up: k out of range for the pair count"); return HY_EBAD_SHAPE; }
    if (max_items(n_pairs, max_active) >= GM_MAX_ITEMS) { set_error("hy_moe_gemm_gate_up: %d pairs make more than %d work items", n_pairs, GM_MAX_ITEMS - 1); return HY_EBAD_SHAPE; }
    // Q5_K: 16-wave blocks (256 weight rows, so every item's activations are read by half as many row blocks, and
    // four waves a SIMD) while that grid still has a block for every CU, and for a single expert: a shared expert's
    // GEMM, which runs beside the routing and the routed GEMMs on a second stream, then takes half the CUs and leaves
    // the rest to them (the 2048-token Q5_K/Q6_K chunk 690 -> 683 us; alone it takes 46 us against 32 at 8 waves and
    // twice the blocks).  Other small grids keep 8 waves.  ff is a multiple of 256, so either size tiles it.
    if (m.tg == Q5_K && (max_items(n_pairs, max_active) * (m.ff / 128) >= cu_count() || max_active == 1)) {
        const int rb = m.ff / 128;
        dim3 grid(rb, item_slots(rb, n_pairs, max_active, 1, true));
        hipLaunchKernelGGL((k_gemm<Q5_K, true, 16, 1>), grid, dim3(1024), 0, s, m, (const uint8_t *) xq, div_mul_of(k), order, order_n, egrp, nullptr, h);
        return check_launch("hy_moe_gemm_gate_up");
    }
    HY_GEMM_SWITCH(m.tg, {
        constexpr int W = 8, B = g5_blocks<TT, true>();
        const int rb = m.ff / (8 * W);   // 8 W output rows a block
        dim3 grid(rb, item_slots(rb, n_pairs, max_active, B, B == 1));   // two blocks a CU: every slot counts
        hipLaunchKernelGGL((k_gemm<TT, true, W, B>), grid, dim3(64 * W), 0, s, m, (const uint8_t *) xq, div_mul_of(k), order, order_n, egrp, nullptr, h);
        return check_launch("hy_moe_gemm_gate_up");
    });
}
int launch_gemm_down(const hy_moe_dev &m, const void *hq, int n_pairs, const int *order, const int *order_n, const int *egrp, int max_active,
                     const float *wts, float *y, hipStream_t s) {
    if (max_active <= 0 || n_pairs <= 0) return HY_OK;
    const int rt = (m.n + GM_ROWS - 1) / GM_ROWS;
    if (vec_dot_type(m.td) == Q8_0) {
        dim3 grid(rt, item_slots(rt, n_pairs, max_active, 3));
        if (m.td == IQ4_NL) hipLaunchKernelGGL((k_gemm_nl<IQ4_NL, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp, wts, y);
        else if (m.td == MXFP4) hipLaunchKernelGGL((k_gemm_nl<MXFP4, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp, wts, y);
        else if (m.td == Q5_0) hipLaunchKernelGGL((k_gemm_nl<Q5_0, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp, wts, y);
        else if (m.td == Q5_1) hipLaunchKernelGGL((k_gemm_nl<Q5_1, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp, wts, y);
        else hipLaunchKernelGGL((k_gemm_nl<Q8_0, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp, wts, y);
        return check_launch("hy_moe_gemm_down");
    }
    if ((size_t) n_pairs * (m.ff / 256) * Q8K_BYTES >= (1ull << 32)) { set_error("hy_moe_gemm_down: activations of 4 GB or more"); return HY_EBAD_SHAPE; }
    if (max_items(n_pairs, max_active) >= GM_MAX_ITEMS) { set_error("hy_moe_gemm_down: %d pairs make more than %d work items", n_pairs, GM_MAX_ITEMS - 1); return HY_EBAD_SHAPE; }
    HY_GEMM_SWITCH(m.td, {
        constexpr int W = TT == Q6_K ? 16 : 8, B = g5_blocks<TT, false>();   // Q6_K: 16 waves (fits 128 registers)
        const int rb = m.n / (16 * W);   // 16 W output rows a block
        dim3 grid(rb, item_slots(rb, n_pairs, max_active, B, true));
        hipLaunchKernelGGL((k_gemm<TT, false, W, B>), grid, dim3(64 * W), 0, s, m, (const uint8_t *) hq, div_mul_of(1), order, order_n, egrp, wts, y);
        return check_launch("hy_moe_gemm_down");
    });
}

} // namespace hy
