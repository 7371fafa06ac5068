// Shared device code of the MoE expert-FFN kernels (gfx950, wave64).
//
// Numeric contract (shared with the CPU oracle, which restates src/cpu_moe.cpp:668-1008):
//  * activations are quantized to ggml's vec_dot partner of the weight type: Q8_K (K-quants, IQ4_XS,
//    IQ2_XS; src/cpu_moe.cpp:35-78) or Q8_0 (IQ4_NL);
//  * each weight block against its activation block yields exact integers sumi (and summ for the types
//    with mins); a row dot product folds block b's integers into t_b with one fp32 formula and
//    accumulates acc = fmaf(xd_b, t_b, acc) over b = 0, 1, ... in order;
//  * SwiGLU uses hy_expf below (Cody-Waite reduction + the Cephes degree-5 polynomial);
//  * the library is compiled with -ffp-contract=off: every product and sum not written as fmaf is
//    rounded on its own, so results are bit-identical to the oracle's.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace hy {

// GGUF type ids (src/gguf.h:13-18)
enum GT : int { Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15, IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19, IQ4_NL = 20, IQ3_S = 21, IQ2_S = 22, IQ4_XS = 23, MXFP4 = 39 };

constexpr int Q8K_BYTES = 292;   // float d; int8 qs[256]; int16 bsums[16]
constexpr int Q8_0_BYTES = 34;   // fp16 d; int8 qs[32]

__host__ __device__ constexpr int block_bytes(int t) {
    return t == Q4_K ? 144 : t == Q5_K ? 176 : t == Q6_K ? 210 : t == IQ4_XS ? 136 : t == IQ2_XS ? 74 : t == IQ2_XXS ? 66
         : t == IQ4_NL ? 18 : t == Q8_0 ? 34 : t == MXFP4 ? 17 : t == Q5_0 ? 22 : t == Q2_K ? 84 : t == Q3_K ? 110 : t == IQ3_XXS ? 98 : t == IQ3_S ? 110 : t == IQ2_S ? 82 : t == IQ1_S ? 50 : t == Q5_1 ? 24 : t == Q8_K ? 292 : 0;
}
__host__ __device__ constexpr int block_elems(int t) {
    return (t == IQ4_NL || t == Q8_0 || t == MXFP4 || t == Q5_0 || t == Q5_1) ? 32
         : (t == Q4_K || t == Q5_K || t == Q6_K || t == IQ4_XS || t == IQ2_XS || t == IQ2_XXS || t == Q2_K || t == Q3_K || t == IQ3_XXS || t == IQ3_S || t == IQ2_S || t == IQ1_S || t == Q8_K) ? 256 : 0;
}
// the grid types (IQ2_XS, IQ2_XXS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S): codebook rows and sign masks in LDS (expand_iq2_grid)
__host__ __device__ constexpr bool iq2_type(int t) {
    return t == IQ2_XS || t == IQ2_XXS || t == IQ2_S || t == IQ3_XXS || t == IQ3_S || t == IQ1_S;
}
__host__ __device__ constexpr int vec_dot_type(int t) { return t == IQ4_NL || t == Q8_0 || t == MXFP4 || t == Q5_0 || t == Q5_1 ? Q8_0 : Q8_K; }
// 32-value block types whose fold also takes the activation block's integer sum (Q5_1's min: m * sum q)
__host__ __device__ constexpr bool ysum_type(int t) { return t == Q5_1; }

// ------------------------------------------------------------------ scalar helpers

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }
// four router weights at p as fp32: fp32 rows as they are; bf16 rows (uint16 bit patterns, p 8-byte aligned) widened,
// which is exact (a bf16 value is the fp32 value with the low 16 bits zero), so both give the same products and sums
__device__ __forceinline__ float4 ld_w4(const float *p) { return *(const float4 *) p; }
__device__ __forceinline__ float4 ld_w4(const uint16_t *p) {
    const uint2 v = *(const uint2 *) p;
    return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                       __uint_as_float(v.y & 0xffff0000u));
}

// exp(x) of the contract: x = n ln2 + r (ln2 = 0.693359375 - 2.12194440e-4, the first part exact in
// 9 bits), exp(r) by the Cephes expf polynomial (S. L. Moshier), 2^n applied as two exact scalings.
// Below exp(-87) the result is 0: no subnormal is ever produced.
__device__ __forceinline__ float hy_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_huge_valf();
    if (x < -87.0f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(n, -0.693359375f, x);
    r = __builtin_fmaf(n, 2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    const float z = r * r;
    float y = __builtin_fmaf(p, z, r);
    y = y + 1.0f;
    const int ni = (int) n, n1 = ni / 2, n2 = ni - n1;
    const float s1 = __uint_as_float((uint32_t) (n1 + 127) << 23), s2 = __uint_as_float((uint32_t) (n2 + 127) << 23);
    return (y * s1) * s2;
}
__device__ __forceinline__ float hy_silu(float x) { return x / (1.0f + hy_expf(-x)); }
// log(x), x > 0: x = 2^e m with m in [sqrt(1/2), sqrt(2)), log(m) by the Cephes single-precision polynomial in
// f = m - 1 (S. L. Moshier, Cephes Math Library, logf.c) with fmaf, e ln2 added as e C2 + e C1 (C1 = 0.693359375);
// subnormal x scaled by 2^23 first.  The same operations as the oracle's or_logf.
__device__ __forceinline__ float hy_logf(float x) {
    if (x != x || x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_huge_valf();
    if (x == __builtin_huge_valf()) return x;
    int e = 0;
    if (x < 1.17549435e-38f) { x = x * 8388608.0f; e = -23; }
    const uint32_t b = __float_as_uint(x);
    e += (int) ((b >> 23) & 0xffu) - 126;
    const float m = __uint_as_float((b & 0x007fffffu) | 0x3f000000u);
    float f;
    if (m < 0.70710678118654752f) { e -= 1; f = m + m - 1.0f; } else { f = m - 1.0f; }
    const float z = f * f;
    float y = 7.0376836292e-2f;
    y = __builtin_fmaf(y, f, -1.1514610310e-1f);
    y = __builtin_fmaf(y, f, 1.1676998740e-1f);
    y = __builtin_fmaf(y, f, -1.2420140846e-1f);
    y = __builtin_fmaf(y, f, 1.4249322787e-1f);
    y = __builtin_fmaf(y, f, -1.6668057665e-1f);
    y = __builtin_fmaf(y, f, 2.0000714765e-1f);
    y = __builtin_fmaf(y, f, -2.4999993993e-1f);
    y = __builtin_fmaf(y, f, 3.3333331174e-1f);
    y = (y * f) * z;
    const float fe = (float) e;
    y = __builtin_fmaf(fe, -2.12194440e-4f, y);
    y = __builtin_fmaf(-0.5f, z, y);
    return __builtin_fmaf(fe, 0.693359375f, f + y);
}
// log(1 + x), x >= -1: log(u) x / (u - 1) with u = 1 + x rounded (D. Goldberg, 1991, theorem 4); x when u == 1
__device__ __forceinline__ float hy_log1pf(float x) {
    if (x != x) return x;
    const float u = 1.0f + x;
    if (u == 1.0f) return x;
    if (u == __builtin_huge_valf()) return u;
    return hy_logf(u) * (x / (u - 1.0f));
}
// the routers' scores: sigmoid (src/kernels5.cu:35) and sqrt(softplus) (src/kernels7.cu:823-826)
__device__ __forceinline__ float hy_sigmoid(float l) { return 1.0f / (1.0f + hy_expf(-l)); }
__device__ __forceinline__ float hy_sqrt_softplus(float l) { return sqrtf(l > 20.0f ? l : hy_log1pf(hy_expf(l))); }
// silu(g) * u, with a limit L > 0: silu(min(g, L)) * clamp(u, -L, L) (src/cpu_moe.cpp:891-892)
__device__ __forceinline__ float hy_swiglu(float g, float u, float L) {
    if (L > 0.0f) { g = fminf(g, L); u = fminf(fmaxf(u, -L), L); }
    return hy_silu(g) * u;
}

// ------------------------------------------------------------------ weight layout in HBM
// Expert matrices are stored as 16-row tiles whose 256-value spans lie together: span s of row r at byte
// ((r / 16) * nspan + s) * 16 * sb + (r % 16) * sb  (sb: bytes per 256 values, nspan = values per row / 256).
// One K step of 16 rows is then one contiguous run (2304 bytes for Q4_K) instead of 16 pieces a row apart; the
// GGUF block bytes themselves are unchanged.  hy_upload_experts writes this layout.
constexpr int HY_TILE = 16;
__host__ __device__ constexpr size_t tiled_off(int row, int span, int nspan, int sb) {
    return ((size_t) (row >> 4) * nspan + span) * (size_t) (HY_TILE * sb) + (size_t) (row & 15) * sb;
}
// the same within one expert matrix of under 4 GiB (the launchers check), as a 32-bit offset
__device__ __forceinline__ uint32_t tiled_off32(int row, int span, int nspan, int sb) {
    return ((uint32_t) (row >> 4) * (uint32_t) nspan + (uint32_t) span) * (uint32_t) (HY_TILE * sb) + (uint32_t) (row & 15) * (uint32_t) sb;
}
__host__ __device__ constexpr int span_bytes(int t) { return block_bytes(t) * (256 / block_elems(t)); }
// a slot-table entry as every kernel takes it: a local expert index below n_local, else -1 (absent)
__device__ __forceinline__ int bound_slot(int raw, int n_local) { return (unsigned) raw < (unsigned) n_local ? raw : -1; }

// ------------------------------------------------------------------ wave helpers

__device__ __forceinline__ int lane_id() { return __lane_id(); }
// DPP lane exchange (GFX9 dpp_ctrl): quad_perm [1,0,3,2] = lane ^ 1, quad_perm [2,3,0,1] = lane ^ 2,
// row_half_mirror = lane i <-> 7 - i within 8, row_mirror = lane i <-> 15 - i within 16
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
template <int CTRL> __device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
__device__ __forceinline__ float readlane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// The contract's wave sum: the xor butterfly 1, 2, 4, ..., 32 (lane i adds lane i ^ o), every lane gets the
// result.  Steps 1 and 2 are exact xor exchanges; after them each quad holds one value, so pairing lane i with
// 7 - i adds the same two quad values as xor 4 does (and i <-> 15 - i the same two half-rows as xor 8); the
// row values then meet as (r0 + r1) + (r2 + r3), as xor 16 then xor 32 add them.  fp32 addition is
// commutative, so every step produces the butterfly's bits.
__device__ __forceinline__ float wave_sum_xor(float v) {
    v = v + dpp_f<DPP_XOR1>(v);
    v = v + dpp_f<DPP_XOR2>(v);
    v = v + dpp_f<DPP_HALF_MIRROR>(v);
    v = v + dpp_f<DPP_MIRROR>(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
// exact integer sum over each aligned group of 8 lanes (every lane of the group gets it)
__device__ __forceinline__ int group8_isum(int v) {
    v += dpp_i<DPP_XOR1>(v);
    v += dpp_i<DPP_XOR2>(v);
    v += dpp_i<DPP_HALF_MIRROR>(v);
    return v;
}
// wave-wide best (value, index) under `better` (a strict total order: the result does not depend on how the
// lanes are paired); every lane gets it (uniform)
template <class Better>
__device__ __forceinline__ void wave_best(float &v, int &i, Better better) {
#define HY_BEST_STEP(CTRL) { const float ov = dpp_f<CTRL>(v); const int oi = dpp_i<CTRL>(i); if (better(ov, oi, v, i)) { v = ov; i = oi; } }
    HY_BEST_STEP(DPP_XOR1) HY_BEST_STEP(DPP_XOR2) HY_BEST_STEP(DPP_HALF_MIRROR) HY_BEST_STEP(DPP_MIRROR)
#undef HY_BEST_STEP
    float bv = readlane_f(v, 0);
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float ov = readlane_f(v, r);
        const int oi = __builtin_amdgcn_readlane(i, r);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    v = bv; i = bi;
}
// Block barrier for LDS hand-offs that leaves global loads in flight: waits for this wave's LDS operations only
// (s_waitcnt lgkmcnt(0); vmcnt and expcnt left at their maxima), no memory fence -- __syncthreads() would also
// wait for every outstanding global load, which would drain every prefetch in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Direct global -> LDS loads (global_load_lds_dword / _dwordx4) from inline asm: a wave-uniform base address in SGPRs,
// a per-lane 32-bit byte offset, and the LDS address of the instruction's first lane in M0 (saved and restored around
// it); lane l's bytes land at M0 + 4 l (dword) or M0 + 16 l (dwordx4).  The compiler does not count them: a kernel that
// issues them waits for them itself (wait_vm; vector memory loads of a wave complete in issue order).
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t) (uintptr_t) p; }
// The same with a wave-uniform base address in SGPRs and a per-lane 32-bit byte offset (no 64-bit address math per lane)
__device__ __forceinline__ uint64_t sgpr_ptr(const void *p) {   // p is uniform; this makes the compiler keep it in SGPRs
    const uint64_t v = (uint64_t) p;
    // readfirstlane returns int: each half goes through uint32_t so that the low half does not sign-extend
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (v >> 32));
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    return ((uint64_t) hi << 32) | lo;
}
__device__ __forceinline__ void dma_s32(const void *base, uint32_t voff, uint32_t lds) {
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(voff), "s"(sgpr_ptr(base)), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
__device__ __forceinline__ void dma_s128(const void *base, uint32_t voff, uint32_t lds) {
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(voff), "s"(sgpr_ptr(base)), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
template <int N> __device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

template <int W> __device__ __forceinline__ int group_isum(int v) {   // sum over aligned groups of W lanes
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// 16 bytes from a 2-byte aligned address (GGUF blocks of 18, 74, 210 bytes): when the address is 2 mod 4,
// a halfword, three dwords and a halfword -- exactly the 16 bytes, nothing past them
__device__ __forceinline__ uint4 load16_a2(const uint8_t *p) {
    uint4 v;
    if (((uintptr_t) p & 3) == 0) {
        const uint32_t *q = (const uint32_t *) p;
        v.x = q[0]; v.y = q[1]; v.z = q[2]; v.w = q[3];
        return v;
    }
    const uint32_t h0 = *(const uint16_t *) p, h4 = *(const uint16_t *) (p + 14);
    const uint32_t *q = (const uint32_t *) (p + 2);
    const uint32_t d1 = q[0], d2 = q[1], d3 = q[2];
    v.x = h0 | (d1 << 16); v.y = (d1 >> 16) | (d2 << 16); v.z = (d2 >> 16) | (d3 << 16); v.w = (d3 >> 16) | (h4 << 16);
    return v;
}
// 16 bytes at any byte offset (MXFP4's 17-byte blocks), without a branch for lanes whose alignments differ: the four
// dwords from p & ~3 and a fifth when p is not dword-aligned (else the fourth again), kept as loaded and joined with
// v_alignbyte where they are used.  The reads end with the dword holding p + 15, at most 3 bytes past the 16, which
// the callers keep inside the buffer.  Joined at the load, they would make the compiler wait for the load right
// there, so that one item's loads land before the next item's go out; kept raw, a load's wait falls at its first
// use, after the round's other loads.
struct Raw16 {
    uint32_t w0, w1, w2, w3, w4, sb;
    __device__ __forceinline__ void load(const uint8_t *p) {
        sb = (uint32_t) ((uintptr_t) p & 3);
        const uint32_t *w = (const uint32_t *) (p - sb);
        w0 = w[0]; w1 = w[1]; w2 = w[2]; w3 = w[3]; w4 = w[sb ? 4 : 3];
    }
    __device__ __forceinline__ uint4 bytes() const {
        return make_uint4(__builtin_amdgcn_alignbyte(w1, w0, sb), __builtin_amdgcn_alignbyte(w2, w1, sb),
                          __builtin_amdgcn_alignbyte(w3, w2, sb), __builtin_amdgcn_alignbyte(w4, w3, sb));
    }
};
// 32 bytes the same way: nine dwords (eight when aligned), joined at use as two 16-byte halves
struct Raw32 {
    uint32_t w0, w1, w2, w3, w4, w5, w6, w7, w8, sb;
    __device__ __forceinline__ void load(const uint8_t *p) {
        sb = (uint32_t) ((uintptr_t) p & 3);
        const uint32_t *w = (const uint32_t *) (p - sb);
        w0 = w[0]; w1 = w[1]; w2 = w[2]; w3 = w[3]; w4 = w[4]; w5 = w[5]; w6 = w[6]; w7 = w[7]; w8 = w[sb ? 8 : 7];
    }
    __device__ __forceinline__ uint4 lo() const {
        return make_uint4(__builtin_amdgcn_alignbyte(w1, w0, sb), __builtin_amdgcn_alignbyte(w2, w1, sb),
                          __builtin_amdgcn_alignbyte(w3, w2, sb), __builtin_amdgcn_alignbyte(w4, w3, sb));
    }
    __device__ __forceinline__ uint4 hi() const {
        return make_uint4(__builtin_amdgcn_alignbyte(w5, w4, sb), __builtin_amdgcn_alignbyte(w6, w5, sb),
                          __builtin_amdgcn_alignbyte(w7, w6, sb), __builtin_amdgcn_alignbyte(w8, w7, sb));
    }
};
__device__ __forceinline__ uint4 load16_a4(const uint8_t *p) {   // dword-aligned 16 bytes
    const uint32_t *q = (const uint32_t *) p;
    uint4 v; v.x = q[0]; v.y = q[1]; v.z = q[2]; v.w = q[3];
    return v;
}
__device__ __forceinline__ uint16_t ld_u16(const uint8_t *p) { return *(const uint16_t *) p; }

// ------------------------------------------------------------------ codebooks

// IQ4_NL / IQ4_XS values (src/kernels4.cu:546)
__device__ __constant__ const int8_t c_kv_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
// IQ2_XS codebook rows, base-3 coded (digit i = byte i: 0 -> 8, 1 -> 25, 2 -> 43)
__device__ __constant__ const uint16_t c_iq2xs_code[512] = {
#include "iq2xs_grid.inc"
};
// MXFP4 block scale: an E8M0 exponent as 2^(e - 128), the half of 2^(e - 127) that pairs with the doubled fp4
// codebook (ggml_e8m0_to_fp32_half; src/kernels4.cu:567-568): e < 2 gives the subnormals 2^-128, 2^-127
__host__ __device__ inline float e8m0_half(uint32_t e) {
    const uint32_t bits = e < 2 ? 0x00200000u << e : (e - 1) << 23;
    float f;
    __builtin_memcpy(&f, &bits, 4);
    return f;
}
// IQ2_XXS codebook rows, the same coding (g_iq2xxs_grid, src/iq_grids.h:14-79)
__device__ __constant__ const uint16_t c_iq2xxs_code[256] = {
#include "iq2xxs_grid.inc"
};
// IQ2_S codebook rows, the same coding (g_iq2s_grid, src/iq_grids.h:210-467)
__device__ __constant__ const uint16_t c_iq2s_code[1024] = {
#include "iq2s_grid.inc"
};
// IQ1_S codebook rows of 8 int8 values in {-1, 0, 1}, base-3 coded with digit = value + 1 (g_iq1s_grid,
// src/iq_grids.h:504-1017)
__device__ __constant__ const uint16_t c_iq1s_code[2048] = {
#include "iq1s_grid.inc"
};
// IQ3_XXS codebook rows of 4 bytes, base-8 coded: digit i = byte i's level, 4 + 8 d (62 for d = 7) (g_iq3xxs_grid,
// src/iq_grids.h:468-503)
__device__ __constant__ const uint16_t c_iq3xxs_code[256] = {
#include "iq3xxs_grid.inc"
};
// IQ3_S codebook rows of 4 bytes, base-8 coded: digit i = byte i's level, 2 d + 1 (g_iq3s_grid, src/kernels4.cu:480-545)
__device__ __constant__ const uint16_t c_iq3s_code[512] = {
#include "iq3s_grid.inc"
};
// the IQ2 sign table: 7 sign bits plus an 8th that makes the count even (src/iq_grids.h:4-13)
__device__ __forceinline__ uint32_t ksign(uint32_t i) { return i | ((uint32_t) (__builtin_popcount(i) & 1) << 7); }

// ------------------------------------------------------------------ activation quantizers

__device__ __forceinline__ int nearest_int(float f) {   // the 1.5 * 2^23 trick of ggml's nearest_int
    const float v = f + 12582912.f;
    return (__float_as_int(v) & 0x007fffff) - 0x00400000;
}

// one Q8_K block of 256 values by one wave (lane: values 4 lane .. 4 lane + 3): first-occurrence signed
// max, iscale = -127/max, q = min(127, nearest_int(iscale * x)), int16 sums of 16, d = 1/iscale.
// An all-zero block writes d = 0, qs = 0, bsums = 0. `out` may be global or LDS (4-byte aligned).
// q8k_block_vals: the block from the lane's four values xv (values 4 lane .. 4 lane + 3)
__device__ __forceinline__ void q8k_block_vals(const float (&xv)[4], uint8_t *out) {
    const int lane = lane_id();
    float am = fabsf(xv[0]);
    int ix = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i) { const float a = fabsf(xv[i]); if (a > am) { am = a; ix = i; } }
    int gi = 4 * lane + ix;
    wave_best(am, gi, [](float a, int ia, float b, int ib) { return (a > b) | ((a == b) & (ia < ib)); });
    uint32_t packed = 0;
    int s = 0;
    float d = 0.0f;
    if (am > 0.0f) {
        const int src = gi >> 2, c = gi & 3;   // uniform
        const float mx = readlane_f(c == 0 ? xv[0] : c == 1 ? xv[1] : c == 2 ? xv[2] : xv[3], src);
        const float iscale = -127.f / mx;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pr = iscale * xv[i];
            int q = nearest_int(pr);
            q = q < 127 ? q : 127;
            s += q;
            packed |= (uint32_t) (q & 0xff) << (8 * i);
        }
        d = 1.0f / iscale;
    }
    s += dpp_i<DPP_XOR1>(s);
    s += dpp_i<DPP_XOR2>(s);
    ((uint32_t *) (out + 4))[lane] = packed;
    if ((lane & 3) == 0) ((int16_t *) (out + 260))[lane >> 2] = (int16_t) s;
    if (lane == 0) *(float *) out = d;
}
// The same Q8_K block by 16 lanes (an aligned DPP row; row lane l holds values 16 l .. 16 l + 15): each lane's
// values are one int16 sum, and the signed max travels with the (|x|, index) winner of the row.
__device__ __forceinline__ void q8k_block16(const float (&xv)[16], uint8_t *out) {
    const int l = lane_id() & 15;
    float am = fabsf(xv[0]), sv = xv[0];
    int gi = 16 * l;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        const float a = fabsf(xv[i]);
        if (a > am) { am = a; sv = xv[i]; gi = 16 * l + i; }
    }
#define HY_B16_STEP(CTRL)                                                                                      \
    {                                                                                                          \
        const float oa = dpp_f<CTRL>(am), os = dpp_f<CTRL>(sv);                                                \
        const int oi = dpp_i<CTRL>(gi);                                                                        \
        if ((oa > am) | ((oa == am) & (oi < gi))) { am = oa; sv = os; gi = oi; }                                   \
    }
    HY_B16_STEP(DPP_XOR1) HY_B16_STEP(DPP_XOR2) HY_B16_STEP(DPP_HALF_MIRROR) HY_B16_STEP(DPP_MIRROR)
#undef HY_B16_STEP
    uint32_t pk[4] = {0u, 0u, 0u, 0u};
    int s = 0;
    float d = 0.0f;
    if (am > 0.0f) {   // uniform over the row
        const float iscale = -127.f / sv;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float pr = iscale * xv[i];
            int q = nearest_int(pr);
            q = q < 127 ? q : 127;
            s += q;
            pk[i >> 2] |= (uint32_t) (q & 0xff) << (8 * (i & 3));
        }
        d = 1.0f / iscale;
    }
    uint32_t *qs = (uint32_t *) (out + 4 + 16 * l);
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[i] = pk[i];
    ((int16_t *) (out + 260))[l] = (int16_t) s;
    if (l == 0) *(float *) out = d;
}
// q8k_block16 from memory: the row's lane l loads values 16 l .. 16 l + 15 of the block at x (16-byte aligned)
__device__ __forceinline__ void q8k_block16_load(const float *x, uint8_t *out) {
    const float4 *src = (const float4 *) (x + 16 * (lane_id() & 15));
    float xv[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = src[i];
        xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
    }
    q8k_block16(xv, out);
}
__device__ __forceinline__ void q8k_block_wave(const float *x, uint8_t *out) {
    const float4 v = *(const float4 *) (x + 4 * lane_id());
    const float xv[4] = {v.x, v.y, v.z, v.w};
    q8k_block_vals(xv, out);
}

// two Q8_0 blocks (64 values) by one wave into blocks of `stride` bytes with qs at `qoff`, as ggml's x86
// quantize_row_q8_0: d = amax / 127 (stored fp16), id = 127 / amax (0 if amax == 0), q = rint(x * id)
// from the lane's value v (value `lane` of the pair; lanes 32-63 ignored when !valid2)
// (the arithmetic: the lane's q and its block's d)
__device__ __forceinline__ int q8_0_pair_q(float v, bool on, float &d) {
    const int lane = lane_id();
    if (!on) v = 0.0f;
    float am = fabsf(v);
    am = fmaxf(am, dpp_f<DPP_XOR1>(am));
    am = fmaxf(am, dpp_f<DPP_XOR2>(am));
    am = fmaxf(am, dpp_f<DPP_HALF_MIRROR>(am));
    am = fmaxf(am, dpp_f<DPP_MIRROR>(am));
    am = lane < 32 ? fmaxf(readlane_f(am, 0), readlane_f(am, 16)) : fmaxf(readlane_f(am, 32), readlane_f(am, 48));
    d = am / 127.f;
    const float id = am != 0.0f ? 127.f / am : 0.0f;
    return (int) __builtin_rintf(v * id);
}
__device__ __forceinline__ void q8_0_pair_vals(float v, uint8_t *out, bool valid2, int stride, int qoff) {
    const int lane = lane_id();
    const bool on = lane < 32 || valid2;
    float d;
    const int q = q8_0_pair_q(v, on, d);
    if (on) {
        uint8_t *b = out + (lane >> 5) * stride;
        b[qoff + (lane & 31)] = (uint8_t) (int8_t) q;
        if ((lane & 31) == 0) *(uint16_t *) b = f2h(d);
    }
}
// the same pair into split storage: the blocks' qs at qs + 32 i, their fp16 d at dq[i]
__device__ __forceinline__ void q8_0_pair_split(float v, uint8_t *qs, uint16_t *dq, bool valid2) {
    const int lane = lane_id();
    const bool on = lane < 32 || valid2;
    float d;
    const int q = q8_0_pair_q(v, on, d);
    if (on) {
        qs[32 * (lane >> 5) + (lane & 31)] = (uint8_t) (int8_t) q;
        if ((lane & 31) == 0) dq[lane >> 5] = f2h(d);
    }
}
__device__ __forceinline__ void q8_0_pair_wave(const float *x, uint8_t *out, bool valid2, int stride, int qoff) {
    const int lane = lane_id();
    q8_0_pair_vals(lane < 32 || valid2 ? x[lane] : 0.0f, out, valid2, stride, qoff);
}

} // namespace hy
