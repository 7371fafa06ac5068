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
__device__ __forceinline__ uint2 ld8_2a(const uint8_t *p) {
    const uint32_t *w = (const uint32_t *) ((uintptr_t) p & ~(uintptr_t) 3);
    const uint32_t sb = (uint32_t) ((uintptr_t) p & 3);
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2];
    return make_uint2(join_b(d1, d0, sb), join_b(d2, d1, sb));
}
// 16 bytes at p (2-byte aligned), with p + 18 the end of the block: the fifth dword is read only when p is
// misaligned (else the fourth is read again), so nothing past p + 18 is touched
__device__ __forceinline__ uint4 ld16_2a_tail(const uint8_t *p) {
    const uint32_t *w = (const uint32_t *) ((uintptr_t) p & ~(uintptr_t) 3);
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
        const uint2 g = grid[qv & 511];
        const uint32_t sg = ksign(qv >> 9);
        b0 = apply_sign(g.x, sg & 15);
        b1 = apply_sign(g.y, sg >> 4);
        const uint32_t s = ((c < 4 ? scv.x : scv.y) >> (8 * (c & 3))) & 0xff;
        s0 = 2 * (int) (s & 15) + 1;
        s1 = 2 * (int) (s >> 4) + 1;
        mn = 0;
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

constexpr int GM_TOK = 64, GM_TILES = GM_TOK / 16, GM_ROWS = 64, GM_LD = 264;   // LDS row stride of staged activations

// one chunk's integers for the tiles: si[tile][v] += scale * D; sm[tile] chained for the mins
// A-operand bytes of token row t (tile * 16 + rr), k = 32 c + 8 q .. + 7: padded rows (GM_LD bytes), or rows of 256
// bytes whose 16-byte pieces are stored at piece ^ (t % 16) (the LDS-DMA layout; conflict-free MFMA operand reads)
template <bool SWZ>
__device__ __forceinline__ long a_frag(const int8_t *As, int tile, int rr, int c, int q) {
    if constexpr (SWZ) return *(const long *) (As + (tile * 16 + rr) * 256 + 16 * ((2 * c + (q >> 1)) ^ rr) + 8 * (q & 1));
    else return *(const long *) (As + (tile * 16 + rr) * GM_LD + 32 * c + 8 * q);
}

template <int T, bool SWZ = false>
__device__ __forceinline__ void chunk_ints(const Raw<T> &w, int c, int q, const uint2 *grid, const int8_t *As, int rr, int ntile,
                                           int (&si)[GM_TILES][4], v4i (&sm)[GM_TILES]) {
    const v4i z = {0, 0, 0, 0};
    uint32_t b0, b1;
    int s0, s1, mn;
    w.chunk(c, q, grid, b0, b1, s0, s1, mn);
    const uint32_t mb = __builtin_amdgcn_perm(0u, (uint32_t) mn, 0u);   // the min in all four bytes (selector 0-3: bytes of the 2nd operand)
#pragma unroll
    for (int tile = 0; tile < GM_TILES; ++tile) {
        if (tile >= ntile) break;
        const long a = a_frag<SWZ>(As, tile, rr, c, q);
        if constexpr (Raw<T>::g16) {
            const bool lo = q < 2;
            const v4i d0 = mfma16(a, mk_long(lo ? b0 : 0u, lo ? b1 : 0u), z);
            const v4i d1 = mfma16(a, mk_long(lo ? 0u : b0, lo ? 0u : b1), z);
#pragma unroll
            for (int v = 0; v < 4; ++v) si[tile][v] += __mul24(s0, d0[v]) + __mul24(s1, d1[v]);
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

// Block barrier for LDS hand-offs that leaves global loads in flight: waits for this wave's LDS operations only
// (s_waitcnt lgkmcnt(0); vmcnt and expcnt left at their maxima), no memory fence -- __syncthreads() would also
// wait for every outstanding global load, which would drain the prefetch stream at every step.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Direct global -> LDS loads and the epilogue's stores, issued from inline asm so that the compiler's wait
// bookkeeping sees only the weight loads of the stream.  (Its bookkeeping treats LDS loads, register loads and
// stores as possibly completing out of order and would then wait for all of them at every step.)  Vector memory
// operations of a wave complete in issue order, so waiting for a step's weight registers also covers every DMA
// issued before them.  M0 holds the LDS address of a DMA; it is saved and restored around it.
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t) (uintptr_t) p; }
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

constexpr int GM_STAGES = 3;         // activation stages in LDS, filled by DMA two steps ahead of their use
constexpr int GM_MAX_ITEMS = 32;     // items per segment: their tables live in LDS (more items: one segment after another)

// A block owns the items blockIdx.y, + gridDim.y, ... (numbered expert by expert, up to 64 tokens each) for its 64
// weight rows (blockIdx.x).  Its steps -- (item, 256-value block b) in order -- form one stream: step s computes
// from activation stage s % 3 and weight registers w[s % 3] while the DMA and the weight loads of step s + 2 are in
// flight.  In every step the activation DMA is issued before the weight loads (a scheduling barrier keeps them
// apart) and loads complete in order, so once w[s % 3] has landed this wave's stage-s DMA has too; a block
// barrier then makes every wave's stage-s bytes visible and frees stage (s - 1) % 3 for the DMA of step s + 2.
template <int T, bool GU>
__global__ __launch_bounds__(256, 2) void k_gemm(hy_moe_dev m, const uint8_t *__restrict__ aq, int a_div, const int *__restrict__ order,
                                                 const int *__restrict__ order_n, const int *__restrict__ egrp, const float *__restrict__ wts,
                                                 float *__restrict__ out) {
    static_assert(T != IQ4_NL, "IQ4_NL runs k_gemm_nl");
    constexpr int AB = Q8K_BYTES;                                // activation bytes per 256 values (Q8_K)
    constexpr int BB = block_bytes(T);                           // weight bytes per 256 values
    // the three stages are separate objects, so that the compiler can tell a stage being read from the stages
    // the DMA is filling (else it would wait for every outstanding DMA before each LDS read)
    __shared__ __align__(16) int8_t As0[GM_TOK * 256], As1[GM_TOK * 256], As2[GM_TOK * 256];   // swizzled token rows
    __shared__ __align__(16) uint32_t Ys0[GM_TOK], Ys1[GM_TOK], Ys2[GM_TOK];   // the Q8_K d (fp32) of each token
    auto As = [&](int stage) -> int8_t * { return stage == 0 ? As0 : stage == 1 ? As1 : As2; };
    auto Ys = [&](int stage) -> uint32_t * { return stage == 0 ? Ys0 : stage == 1 ? Ys1 : Ys2; };
    __shared__ int s_scan[1024 + 8];
    __shared__ int s_item[GM_MAX_ITEMS][3];                       // first pair in order, tokens, weight slot
    __shared__ int s_pair[GM_MAX_ITEMS][GM_TOK];                  // pair index of each token of the segment's items
    __shared__ float s_wt[GU ? 1 : GM_MAX_ITEMS][GM_TOK];         // down: their route weights
    __shared__ float s_up[GU ? 32 * GM_TOK : 1];
    __shared__ uint2 grid[T == IQ2_XS ? 512 : 1];
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
        if (T == IQ2_XS) expand_iq2xs_grid(grid);
        __syncthreads();
    }
    const int total = s_scan[1024] + s_scan[1025] + s_scan[1026] + s_scan[1027];
    const int y0 = blockIdx.y, ys = gridDim.y;
    const int my_items = total > y0 ? (total - 1 - y0) / ys + 1 : 0;
    if (my_items == 0) return;   // uniform over the block
    const int rows = GU ? m.ff : m.n, in_dim = GU ? m.n : m.ff, nsb = in_dim / 256;
    const int row = blockIdx.x * (GU ? 32 : GM_ROWS) + (GU ? (wave & 1) : wave) * 16 + rr;
    const bool row_ok = row < rows;
    const size_t mbytes = GU ? m.gate_bytes : m.down_bytes;
    // span b of this lane's row sits at Wrow + b * HY_TILE * BB (tiled weight layout)
    const uint8_t *Wrow = (GU ? (wave < 2 ? m.gate : m.up) : m.down) + tiled_off(row_ok ? row : rows - 1, 0, nsb, BB);
    const size_t arow = (size_t) nsb * AB;
    const int my_tok = wave * 16 + (lane & 15);   // the token whose row pointer this lane carries (lanes 0..15)

    for (int seg = 0; seg < my_items; seg += GM_MAX_ITEMS) {
        const int nit = min(GM_MAX_ITEMS, my_items - seg);
        __syncthreads();   // readers of the previous segment's table are done
        for (int i = tid; i < nit; i += 256) {
            const int item = y0 + (seg + i) * ys;
            int lo = 0, hi = na - 1;   // last group whose prefix <= item
            while (lo < hi) { const int mid = (lo + hi + 1) >> 1; if (s_scan[mid] <= item) lo = mid; else hi = mid - 1; }
            const int tok0 = (item - s_scan[lo]) * GM_TOK;
            s_item[i][0] = egrp[3 * lo + 1] + tok0;
            s_item[i][1] = min(GM_TOK, egrp[3 * lo + 2] - tok0);
            s_item[i][2] = m.slot[egrp[3 * lo]];
        }
        __syncthreads();
        // the segment's pair indices (and down: route weights), with ordinary loads, before its stream starts
        for (int i = tid; i < nit * GM_TOK; i += 256) {
            const int it = i / GM_TOK, tk = i - it * GM_TOK;
            const int pr = tk < s_item[it][1] ? order[s_item[it][0] + tk] : -1;
            s_pair[it][tk] = pr;
            if (!GU) s_wt[GU ? 0 : it][tk] = pr >= 0 ? wts[pr] : 0.0f;
        }
        __syncthreads();
        const int nsteps = nit * nsb;
        const uint8_t *src_cur = nullptr;
        Raw<T> w[3];
        auto issue = [&](int st, int stage, Raw<T> &wr) {
            const int it = st / nsb, b = st - it * nsb;
            const int ntok = s_item[it][1];
            if (b == 0) {
                const int pr = my_tok < ntok ? s_pair[it][my_tok] : -1;
                src_cur = pr >= 0 ? aq + (size_t) (GU ? pr / a_div : pr) * arow : aq;
            }
            // activations of step st -> stage: one DMA per token row of this wave, then the scales.  Every step issues
            // the same instructions (rows of absent tokens point at row 0 of the activations: harmless reads into LDS
            // rows nobody uses), so the compiler can count the loads in flight and wait for exactly one step.
            int8_t *as = As(stage);
            const uint64_t sp = (uint64_t) src_cur;
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {   // tokens wave*16 + 4 i4 .. + 3: lane l takes piece (l % 16) ^ (t % 16) of token l / 16
                const int t16 = 4 * i4 + (lane >> 4), tk = wave * 16 + t16;
                const uint8_t *rowp = (const uint8_t *) __shfl(sp, t16);
                const int piece = (lane & 15) ^ (tk & 15);
                dma_lds_b128(rowp + (size_t) b * AB + 4 + 16 * piece, lds_addr(as + (wave * 16 + 4 * i4) * 256));
            }
            if (lane < 16) dma_lds_b32(src_cur + (size_t) b * AB, lds_addr(Ys(stage) + wave * 16));
            __builtin_amdgcn_sched_barrier(0);
            wr.load(Wrow + (size_t) s_item[it][2] * mbytes + (size_t) b * (HY_TILE * BB), q);
            __builtin_amdgcn_sched_barrier(0);
        };

        // compute side
        float acc[GM_TILES][4], ep_val[GM_TILES][4];
        int ep_it = -1;
#pragma unroll
        for (int i = 0; i < GM_TILES; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i][v] = 0.0f;
        auto compute = [&](int st, int stage, const Raw<T> &wr) {
            const int it = st / nsb, b = st - it * nsb;
            const int ntok = s_item[it][1], ntile = (ntok + 15) / 16;
            const int8_t *as = As(stage);
            {
                int si[GM_TILES][4];
                v4i sm[GM_TILES];
#pragma unroll
                for (int i = 0; i < GM_TILES; ++i) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) si[i][v] = 0;
                    sm[i] = v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) chunk_ints<T, true>(wr, c, q, grid, as, rr, ntile, si, sm);
                const float *yd = (const float *) Ys(stage);
#pragma unroll
                for (int tile = 0; tile < GM_TILES; ++tile) {
                    if (tile >= ntile) break;
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[tile][v] = __builtin_fmaf(yd[tile * 16 + 4 * q + v], wr.fold(si[tile][v], sm[tile][v]), acc[tile][v]);
                }
            }
            if (b == nsb - 1) {   // the item's outputs: into ep_val now, to memory at the start of the next step
                if (GU && wave >= 2) {
#pragma unroll
                    for (int tile = 0; tile < GM_TILES; ++tile)
#pragma unroll
                        for (int v = 0; v < 4; ++v) s_up[((wave & 1) * 16 + rr) * GM_TOK + tile * 16 + 4 * q + v] = acc[tile][v];
                }
                if (GU) lds_barrier();
#pragma unroll
                for (int tile = 0; tile < GM_TILES; ++tile)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int tok = tile * 16 + 4 * q + v;
                        if (GU) ep_val[tile][v] = wave < 2 && tile < ntile ? hy_swiglu(acc[tile][v], s_up[((wave & 1) * 16 + rr) * GM_TOK + tok], m.clamp) : 0.0f;
                        else ep_val[tile][v] = tile < ntile ? s_wt[GU ? 0 : it][tok] * acc[tile][v] : 0.0f;
                        acc[tile][v] = 0.0f;
                    }
                ep_it = it;
            }
        };
        // the stored item's outputs (rows of this wave that exist, tokens of the item)
        auto flush_ep = [&]() {
            if (ep_it < 0) return;
            const int ntok = s_item[ep_it][1];
            if (row_ok && (!GU || wave < 2)) {
#pragma unroll
                for (int tile = 0; tile < GM_TILES; ++tile)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int tok = tile * 16 + 4 * q + v;
                        if (tok < ntok) store_f32(out + (size_t) s_pair[ep_it][tok] * (GU ? m.ff : m.n) + row, ep_val[tile][v]);
                    }
            }
            ep_it = -1;
        };

        // the stream: steps 0 and 1 issued ahead, then per step: wait for its bytes, barrier, issue step + 2, compute
        issue(0, 0, w[0]);
        issue(min(1, nsteps - 1), 1, w[1]);
#define HY_GM_STEP(U)                                                                          \
        {                                                                                      \
            const int st = s0 + U;                                                             \
            if (st >= nsteps) break;                                                           \
            touch_regs(w[U]);                                                                  \
            lds_barrier();                                                                     \
            flush_ep();                                                                        \
            issue(min(st + 2, nsteps - 1), (U + 2) % 3, w[(U + 2) % 3]);   /* past the end: a harmless repeat */ \
            compute(st, U, w[U]);                                                              \
        }
        for (int s0 = 0; s0 < nsteps; s0 += 3) {
            HY_GM_STEP(0)
            HY_GM_STEP(1)
            HY_GM_STEP(2)
        }
#undef HY_GM_STEP
        flush_ep();
    }
    __builtin_amdgcn_s_waitcnt(0);   // no DMA into this block's LDS may outlive it
}

// IQ4_NL: one chunk's MFMA per tile folded straight into the fp32 accumulators (Yc: 8 block scales per token)
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
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[tile][v] = __builtin_fmaf(Yc[(tile * 16 + 4 * q + v) * 8 + c], w.cfold(c, d0[v]), acc[tile][v]);
    }
}

// IQ4_NL (Q8_0 activations, whose 2-byte aligned blocks the LDS DMA above cannot stage): register-staged
// stream, one step ahead.  A block walks the work items it, it + gridDim.y, ...; the (item, block) steps form one stream in which the
// next step's weight and activation bytes are loaded while the current step computes, across item boundaries.
template <int T, bool GU>
__global__ __launch_bounds__(256) void k_gemm_nl(hy_moe_dev m, const uint8_t *__restrict__ aq, int a_div, const int *__restrict__ order,
                                              const int *__restrict__ order_n, const int *__restrict__ egrp, const float *__restrict__ wts,
                                              float *__restrict__ out) {
    __shared__ __align__(16) int8_t As[2][GM_TOK * GM_LD];
    constexpr bool NL = T == IQ4_NL;                 // Q8_0 activations, per-block fold
    __shared__ float Yd[2][GM_TOK * (NL ? 8 : 1)];
    __shared__ int s_scan[1024 + 8];
    __shared__ float s_up[GU ? 32 * GM_TOK : 1];
    __shared__ uint2 grid[T == IQ2_XS ? 512 : 1];
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
        if (T == IQ2_XS) expand_iq2xs_grid(grid);
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

#define HY_GEMM_SWITCH(T, CALL)                                                                    \
    switch (T) {                                                                                   \
    case Q4_K: { constexpr int TT = Q4_K; CALL; }                                                 \
    case Q5_K: { constexpr int TT = Q5_K; CALL; }                                                 \
    case Q6_K: { constexpr int TT = Q6_K; CALL; }                                                 \
    case IQ4_XS: { constexpr int TT = IQ4_XS; CALL; }                                             \
    case IQ2_XS: { constexpr int TT = IQ2_XS; CALL; }                                             \
    default: set_error("grouped GEMM: unsupported expert type %d", (int) (T)); return HY_EUNSUPPORTED_TYPE; \
    }

// upper bound of the work items: sum over active experts of ceil(cnt / GM_TOK) <= ceil(P / GM_TOK) + active
static int max_items(int n_pairs, int max_active) { return (n_pairs + GM_TOK - 1) / GM_TOK + max_active; }
// item slots per row tile: enough blocks for about `per_cu` resident blocks on every CU
static int item_slots(int row_tiles, int n_pairs, int max_active, int per_cu) {
    static int cus = 0;
    if (!cus) { int dev = 0; hipDeviceProp_t pr; if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&pr, dev) == hipSuccess) cus = pr.multiProcessorCount; if (cus <= 0) cus = 256; }
    const int want = (cus * per_cu + row_tiles - 1) / row_tiles;
    return std::max(1, std::min(max_items(n_pairs, max_active), want));
}

int launch_gemm_gate_up(const hy_moe_dev &m, const void *xq, int k, int n_pairs, const int *order, const int *order_n, const int *egrp,
                        int max_active, float *h, hipStream_t s) {
    if (max_active <= 0 || n_pairs <= 0) return HY_OK;
    const int rt = (m.ff + 31) / 32;
    if (m.tg == IQ4_NL) {
        dim3 grid(rt, item_slots(rt, n_pairs, max_active, 3));
        hipLaunchKernelGGL((k_gemm_nl<IQ4_NL, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp, nullptr, h);
        return check_launch("hy_moe_gemm_gate_up");
    }
    dim3 grid(rt, item_slots(rt, n_pairs, max_active, 2));
    HY_GEMM_SWITCH(m.tg, hipLaunchKernelGGL((k_gemm<TT, true>), grid, dim3(256), 0, s, m, (const uint8_t *) xq, k, order, order_n, egrp,
                                            nullptr, h);
                   return check_launch("hy_moe_gemm_gate_up"));
}
int launch_gemm_down(const hy_moe_dev &m, const void *hq, int n_pairs, const int *order, const int *order_n, const int *egrp, int max_active,
                     const float *wts, float *y, hipStream_t s) {
    if (max_active <= 0 || n_pairs <= 0) return HY_OK;
    const int rt = (m.n + GM_ROWS - 1) / GM_ROWS;
    if (m.td == IQ4_NL) {
        dim3 grid(rt, item_slots(rt, n_pairs, max_active, 3));
        hipLaunchKernelGGL((k_gemm_nl<IQ4_NL, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp, wts, y);
        return check_launch("hy_moe_gemm_down");
    }
    dim3 grid(rt, item_slots(rt, n_pairs, max_active, 2));
    HY_GEMM_SWITCH(m.td, hipLaunchKernelGGL((k_gemm<TT, false>), grid, dim3(256), 0, s, m, (const uint8_t *) hq, 1, order, order_n, egrp,
                                            wts, y);
                   return check_launch("hy_moe_gemm_down"));
}

} // namespace hy
