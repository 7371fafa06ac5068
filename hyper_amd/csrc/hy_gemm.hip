// Prefill / speculative-verify grouped expert GEMMs on int8 MFMA (gfx950 v_mfma_i32_16x16x32_i8).
//
// A block takes one active expert (blockIdx.y < order_n[1]) and 64 weight rows (16 per wave; gate/up: the
// same 16 rows of gate and of up), and walks the expert's tokens in passes of up to 64 (four 16-token tiles)
// (replaces k_moe_gemm / k_moe_gemm2, src/kernels4.cu:1354-1467, :1521-1631, which dequantize to fp16 and use
// fp16 MMA).  Per 256-value block b:
//   A (16 tokens x 32 k): the tokens' Q8_K bytes, staged through LDS for all four waves;
//   B (32 k x 16 rows):   the weight rows' quant values decoded to int8 in registers, per 32-value chunk;
//   D = A B (exact int32 per chunk); each chunk's D is scaled by its scale group's integer scale (one
//   v_mad per value) into sumi, the mins term of Q4_K / Q5_K is a second chained MFMA against a B holding the
//   chunk's min, and the block's integers fold into the fp32 accumulator with the contract's formula.
// Operand layouts (CDNA3/4 16x16x32 i8): A lane l holds token l % 16, k = 8 (l / 16) .. + 7; B lane l holds
// weight row l % 16 with the same k; D lane l holds row l % 16 for tokens 4 (l / 16) + v, v = 0..3.
// Types with 16-value scale groups (Q6_K, IQ2_XS) run each chunk as two MFMAs with B zeroed in the lanes of
// the other group (lanes 0-31 hold k 0..15, lanes 32-63 k 16..31).
#include "hy_internal.h"
#include "hy_blocks.cuh"

namespace hy {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma16(long a, long b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0); }
__device__ __forceinline__ long mk_long(uint32_t lo, uint32_t hi) { return (long) (((unsigned long long) hi << 32) | lo); }
__device__ __forceinline__ uint2 load8_a2(const uint8_t *p) {   // 8 bytes from a 2-byte aligned address, no overread
    if (((uintptr_t) p & 3) == 0) { const uint32_t *w = (const uint32_t *) p; return make_uint2(w[0], w[1]); }
    const uint32_t h0 = *(const uint16_t *) p, d1 = *(const uint32_t *) (p + 2), h2 = *(const uint16_t *) (p + 6);
    return make_uint2(h0 | (d1 << 16), (d1 >> 16) | (h2 << 16));
}

// B fragments of one weight row's 256-value block for the lane's k quarter q: b[c] (8 int8 values of chunk c),
// integer scales, and the fold.
template <int T> struct Frag;

template <> struct Frag<Q4_K> {
    static constexpr bool mins = true, g16 = false;
    uint4 hd; uint2 qv[4];
    uint32_t b[8][2]; int sc[8], mn[8];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        hd = load16_a4(blk);
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) qv[jp] = *(const uint2 *) (blk + 16 + 32 * jp + 8 * q);
    }
    __device__ __forceinline__ void prep(int, const uint2 *) {
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
            b[2 * jp][0] = qv[jp].x & 0x0F0F0F0Fu; b[2 * jp][1] = qv[jp].y & 0x0F0F0F0Fu;
            b[2 * jp + 1][0] = (qv[jp].x >> 4) & 0x0F0F0F0Fu; b[2 * jp + 1][1] = (qv[jp].y >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) scale_min_k4(hd.y, hd.z, hd.w, c, sc[c], mn[c]);
    }
    __device__ __forceinline__ float fold(int si, int sm) const {
        return __builtin_fmaf(h2f(hd.x & 0xffff), (float) si, -(h2f(hd.x >> 16) * (float) sm));
    }
};
template <> struct Frag<Q5_K> {
    static constexpr bool mins = true, g16 = false;
    uint4 hd; uint2 qv[4], qh;
    uint32_t b[8][2]; int sc[8], mn[8];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
        hd = load16_a4(blk);
        qh = *(const uint2 *) (blk + 16 + 8 * q);
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) qv[jp] = *(const uint2 *) (blk + 48 + 32 * jp + 8 * q);
    }
    __device__ __forceinline__ void prep(int, const uint2 *) {
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
            const int j0 = 2 * jp, j1 = 2 * jp + 1;
            b[j0][0] = (qv[jp].x & 0x0F0F0F0Fu) | (((qh.x >> j0) & 0x01010101u) << 4);
            b[j0][1] = (qv[jp].y & 0x0F0F0F0Fu) | (((qh.y >> j0) & 0x01010101u) << 4);
            b[j1][0] = ((qv[jp].x >> 4) & 0x0F0F0F0Fu) | (((qh.x >> j1) & 0x01010101u) << 4);
            b[j1][1] = ((qv[jp].y >> 4) & 0x0F0F0F0Fu) | (((qh.y >> j1) & 0x01010101u) << 4);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) scale_min_k4(hd.y, hd.z, hd.w, c, sc[c], mn[c]);
    }
    __device__ __forceinline__ float fold(int si, int sm) const {
        return __builtin_fmaf(h2f(hd.x & 0xffff), (float) si, -(h2f(hd.x >> 16) * (float) sm));
    }
};
// Q6_K: chunk c = elements 32 c ..: hf = c >> 2, qt = c & 3; lane values l = 8 q .. + 7 from ql[64 hf + 32 (qt & 1) + l]
// (high nibble when qt >= 2) and bits 2 qt of qh[32 hf + l]; 16-groups 2 c (lanes q < 2) and 2 c + 1.
template <> struct Frag<Q6_K> {
    static constexpr bool mins = false, g16 = true;
    uint2 ql[4], qh[2]; uint4 scv; uint16_t d;
    uint32_t b[8][2]; int sc[16], mn[8];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ql[i] = load8_a2(blk + 64 * (i >> 1) + 32 * (i & 1) + 8 * q);
#pragma unroll
        for (int i = 0; i < 2; ++i) qh[i] = load8_a2(blk + 128 + 32 * i + 8 * q);
        scv = load16_a2(blk + 192);
        d = ld_u16(blk + 208);
    }
    __device__ __forceinline__ void prep(int, const uint2 *) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int hf = c >> 2, qt = c & 3;
            const uint2 l = ql[2 * hf + (qt & 1)], h = qh[hf];
            const int s1 = qt >= 2 ? 4 : 0;
            b[c][0] = q6_signed(((l.x >> s1) & 0x0F0F0F0Fu) | (((h.x >> (2 * qt)) & 0x03030303u) << 4));
            b[c][1] = q6_signed(((l.y >> s1) & 0x0F0F0F0Fu) | (((h.y >> (2 * qt)) & 0x03030303u) << 4));
        }
#pragma unroll
        for (int g = 0; g < 16; ++g) sc[g] = (int) (int8_t) byte_of(scv, g);
    }
    __device__ __forceinline__ float fold(int si, int) const { return h2f(d) * (float) si; }
};
// IQ4_XS: chunk c = 32-group c: lane values 8 q .. + 7 are nibbles (q >> 1) of qs[16 c + 8 (q & 1) ..]
template <> struct Frag<IQ4_XS> {
    static constexpr bool mins = false, g16 = false;
    uint2 qv[8]; uint32_t dsh, sl;
    uint32_t b[8][2]; int sc[8], mn[8];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; ++c) qv[c] = *(const uint2 *) (blk + 8 + 16 * c + 8 * (q & 1));
        dsh = *(const uint32_t *) blk;
        sl = *(const uint32_t *) (blk + 4);
    }
    __device__ __forceinline__ void prep(int q, const uint2 *) {
        const int s = 4 * (q >> 1);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            b[c][0] = kv4((qv[c].x >> s) & 0x0F0F0F0Fu);
            b[c][1] = kv4((qv[c].y >> s) & 0x0F0F0F0Fu);
            const int ls = ((sl >> (8 * (c >> 1) + 4 * (c & 1))) & 0xF) | ((((dsh >> 16) >> (2 * c)) & 3) << 4);
            sc[c] = ls - 32;
        }
    }
    __device__ __forceinline__ float fold(int si, int) const { return h2f(dsh & 0xffff) * (float) si; }
};
// IQ2_XS: chunk c = 32-group c; lane q takes its 8-group q (grid row qs[4 c + q], signs); scale nibbles:
// (scales[c] & 15) for lanes q < 2, (scales[c] >> 4) for q >= 2, as 2 sc + 1.
template <> struct Frag<IQ2_XS> {
    static constexpr bool mins = false, g16 = true;
    uint16_t qq[8]; uint2 scv; uint16_t d;
    uint32_t b[8][2]; int sc[16], mn[8];
    __device__ __forceinline__ void load(const uint8_t *blk, int q) {
#pragma unroll
        for (int c = 0; c < 8; ++c) qq[c] = ld_u16(blk + 2 + 2 * (4 * c + q));
        scv = load8_a2(blk + 66);
        d = ld_u16(blk);
    }
    __device__ __forceinline__ void prep(int, const uint2 *grid) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint2 g = grid[qq[c] & 511];
            const uint32_t sg = ksign(qq[c] >> 9);
            b[c][0] = apply_sign(g.x, sg & 15);
            b[c][1] = apply_sign(g.y, sg >> 4);
            const uint32_t s = ((c < 4 ? scv.x : scv.y) >> (8 * (c & 3))) & 0xff;
            sc[2 * c] = 2 * (int) (s & 15) + 1;
            sc[2 * c + 1] = 2 * (int) (s >> 4) + 1;
        }
    }
    __device__ __forceinline__ float fold(int si, int) const { return (h2f(d) * 0.125f) * (float) si; }
};

constexpr int GM_TOK = 64, GM_LD = 264;   // tokens per pass, LDS row stride of the staged activations

// sumi / summ of one 16-token tile against one prepared row block
template <int T>
__device__ __forceinline__ void tile_ints(const Frag<T> &f, const int8_t *As, int tile, int rr, int q, int si[4], v4i &sm) {
    const v4i z = {0, 0, 0, 0};
#pragma unroll
    for (int v = 0; v < 4; ++v) si[v] = 0;
    sm = z;
    const int8_t *arow = As + (tile * 16 + rr) * GM_LD + 8 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const long a = *(const long *) (arow + 32 * c);
        if constexpr (Frag<T>::g16) {
            const bool lo = q < 2;
            const long bl = mk_long(lo ? f.b[c][0] : 0u, lo ? f.b[c][1] : 0u), bh = mk_long(lo ? 0u : f.b[c][0], lo ? 0u : f.b[c][1]);
            const v4i s0 = mfma16(a, bl, z), s1 = mfma16(a, bh, z);
#pragma unroll
            for (int v = 0; v < 4; ++v) si[v] += f.sc[2 * c] * s0[v] + f.sc[2 * c + 1] * s1[v];
        } else {
            const v4i s0 = mfma16(a, mk_long(f.b[c][0], f.b[c][1]), z);
#pragma unroll
            for (int v = 0; v < 4; ++v) si[v] += f.sc[c] * s0[v];
            if constexpr (Frag<T>::mins) {
                const uint32_t mb = (uint32_t) f.mn[c] * 0x01010101u;
                sm = mfma16(a, mk_long(mb, mb), sm);
            }
        }
    }
}

template <int T, bool GU>
__global__ __launch_bounds__(256) void k_gemm(hy_moe_dev m, const uint8_t *__restrict__ aq, int a_div, const int *__restrict__ order,
                                              const int *__restrict__ order_n, const int *__restrict__ egrp, const float *__restrict__ wts,
                                              float *__restrict__ out) {
    __shared__ __align__(16) int8_t As[GM_TOK * GM_LD];
    __shared__ float Yd[GM_TOK];
    __shared__ uint2 grid[T == IQ2_XS ? 512 : 1];
    if ((int) blockIdx.y >= order_n[1]) return;
    const int e = egrp[3 * blockIdx.y], start = egrp[3 * blockIdx.y + 1], cnt = egrp[3 * blockIdx.y + 2];
    const int slot = m.slot[e];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, rr = lane & 15, q = lane >> 4;
    const int rows = GU ? m.ff : m.n, in_dim = GU ? m.n : m.ff, nsb = in_dim / 256;
    const int row = blockIdx.x * 64 + wave * 16 + rr;
    const bool row_ok = row < rows;
    const size_t mbytes = GU ? m.gate_bytes : m.down_bytes, rb = mbytes / rows;
    const uint8_t *W0 = (GU ? m.gate : m.down) + (size_t) slot * mbytes + (size_t) (row_ok ? row : rows - 1) * rb;
    const uint8_t *W1 = GU ? m.up + (size_t) slot * mbytes + (size_t) (row_ok ? row : rows - 1) * rb : nullptr;
    const size_t arow = (size_t) nsb * Q8K_BYTES;
    if (T == IQ2_XS) expand_iq2xs_grid(grid);
    constexpr int BB = block_bytes(T);
    for (int tb = 0; tb < cnt; tb += GM_TOK) {
        const int ntile = min(4, (cnt - tb + 15) / 16);
        float ag[4][4], au[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) ag[i][v] = au[i][v] = 0.0f;
        // the staging thread's token row (fixed over k)
        const int st_tok = tid >> 2, st_part = tid & 3;
        const uint8_t *st_src = nullptr;
        if (tb + st_tok < cnt) {
            const int p = order[start + tb + st_tok];
            st_src = aq + (size_t) (GU ? p / a_div : p) * arow;
        }
        for (int b = 0; b < nsb; ++b) {
            Frag<T> fg, fu;
            fg.load(W0 + (size_t) b * BB, q);
            if (GU) fu.load(W1 + (size_t) b * BB, q);
            __syncthreads();
            {
                uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0, v2 = v0, v3 = v0;
                float yd = 0.0f;
                if (st_src) {
                    const uint8_t *s = st_src + (size_t) b * Q8K_BYTES;
                    v0 = load16_a4(s + 4 + 64 * st_part); v1 = load16_a4(s + 20 + 64 * st_part);
                    v2 = load16_a4(s + 36 + 64 * st_part); v3 = load16_a4(s + 52 + 64 * st_part);
                    yd = *(const float *) s;
                }
                uint4 *dst = (uint4 *) (As + st_tok * GM_LD + 64 * st_part);
                dst[0] = v0; dst[1] = v1; dst[2] = v2; dst[3] = v3;
                if (st_part == 0) Yd[st_tok] = yd;
            }
            __syncthreads();
            fg.prep(q, grid);
            if (GU) fu.prep(q, grid);
#pragma unroll
            for (int tile = 0; tile < 4; ++tile) {
                if (tile >= ntile) break;
                int si[4];
                v4i sm;
                tile_ints<T>(fg, As, tile, rr, q, si, sm);
#pragma unroll
                for (int v = 0; v < 4; ++v) ag[tile][v] = __builtin_fmaf(Yd[tile * 16 + 4 * q + v], fg.fold(si[v], sm[v]), ag[tile][v]);
                if (GU) {
                    tile_ints<T>(fu, As, tile, rr, q, si, sm);
#pragma unroll
                    for (int v = 0; v < 4; ++v) au[tile][v] = __builtin_fmaf(Yd[tile * 16 + 4 * q + v], fu.fold(si[v], sm[v]), au[tile][v]);
                }
            }
        }
#pragma unroll
        for (int tile = 0; tile < 4; ++tile) {
            if (tile >= ntile) break;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int tok = tb + tile * 16 + 4 * q + v;
                if (tok < cnt && row_ok) {
                    const int p = order[start + tok];
                    if (GU) out[(size_t) p * m.ff + row] = hy_swiglu(ag[tile][v], au[tile][v], m.clamp);
                    else out[(size_t) p * m.n + row] = wts[p] * ag[tile][v];
                }
            }
        }
    }
}

#define HY_GEMM_SWITCH(T, CALL)                                                                    \
    switch (T) {                                                                                   \
    case Q4_K: { constexpr int TT = Q4_K; CALL; }                                                 \
    case Q5_K: { constexpr int TT = Q5_K; CALL; }                                                 \
    case Q6_K: { constexpr int TT = Q6_K; CALL; }                                                 \
    case IQ4_XS: { constexpr int TT = IQ4_XS; CALL; }                                             \
    case IQ2_XS: { constexpr int TT = IQ2_XS; CALL; }                                             \
    default: set_error("grouped GEMM: unsupported expert type %d", (int) (T)); return HY_EUNSUPPORTED_TYPE; \
    }

int launch_gemm_gate_up(const hy_moe_dev &m, const void *xq, int k, const int *order, const int *order_n, const int *egrp, int max_active,
                        float *h, hipStream_t s) {
    if (max_active <= 0) return HY_OK;
    dim3 grid((m.ff + 63) / 64, max_active);
    HY_GEMM_SWITCH(m.tg, hipLaunchKernelGGL((k_gemm<TT, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp,
                                            nullptr, h);
                   return check_launch("hy_moe_gemm_gate_up"));
}
int launch_gemm_down(const hy_moe_dev &m, const void *hq, const int *order, const int *order_n, const int *egrp, int max_active,
                     const float *wts, float *y, hipStream_t s) {
    if (max_active <= 0) return HY_OK;
    dim3 grid((m.n + 63) / 64, max_active);
    HY_GEMM_SWITCH(m.td, hipLaunchKernelGGL((k_gemm<TT, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp,
                                            wts, y);
                   return check_launch("hy_moe_gemm_down"));
}

} // namespace hy
