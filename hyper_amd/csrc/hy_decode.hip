// Decode / short-verify path in three launches per MoE layer, with no hand-off between blocks of a launch
// (device-scope fences and contended atomics cost more than a launch boundary on MI355X):
//   k_router_q8      router GEMV, a wave per logit row, plus the Q8 blocks of x (gemv_f32, src/kernels4.cu:163-180);
//   k_route_gate_up  every block routes its own token from the logits (one wave: softmax / top-k / renormalise /
//                    shared gate, src/kernels4.cu:297-344), then a wave per ff row of its pair computes gate and up
//                    against the Q8 x and SwiGLU (moe_gate_up, src/kernels4.cu:1973-2006);
//   k_dec_down       each block quantizes the k hidden rows of its token into LDS once, then a wave per output row
//                    computes the down dots of all k pairs and the combine in ascending expert id (moe_down +
//                    moe_reduce, src/kernels4.cu:2007-2022, :1182-1206).
// Inside a wave the 8-lane groups take 256-value items (Item<T>, exact integers), the group's integers are summed
// with DPP, and each row's blocks are folded in block order by one lane: the same contract as the oracle.
#include "hy_internal.h"
#include "hy_blocks.cuh"

#include <algorithm>

namespace hy {

constexpr int DEC_MAXP = 8;        // passes of 8 items per wave: up to 64 items (256-value spans) per wave
constexpr int DEC_ROUTE_NT = 8;    // tokens the fused router takes (more: the separate kernels)

// ---------------------------------------------------------------- k_router

__device__ __forceinline__ bool rt_better2(float a, int ia, float b, int ib) { return a > b || (a == b && ia < ib); }

// softmax / top-k of one token by one wave (expert e in lane e % 64, slot e / 64), the contract of k_route
template <int V>
__device__ void route_wave(const float *l, int ne, int k, int *ids, float *wts, float *sg) {
    const int lane = threadIdx.x & 63;
    float v[V];
    int vi[V];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int e = lane + 64 * i;
        v[i] = e < ne ? l[e] : -__builtin_huge_valf();
        vi[i] = e < ne ? e : 0x7fffffff;
        mx = fmaxf(mx, v[i]);
    }
    mx = wave_max(mx);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i)
        if (vi[i] < ne) { v[i] = hy_expf(v[i] - mx); acc = acc + v[i]; }
    const float s = wave_sum_xor(acc);
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = vi[i] < ne ? v[i] / s : -1.0f;
#pragma unroll
    for (int i = 1; i < V; ++i)
#pragma unroll
        for (int j = i; j > 0; --j)
            if (rt_better2(v[j], vi[j], v[j - 1], vi[j - 1])) {
                const float tv = v[j]; v[j] = v[j - 1]; v[j - 1] = tv;
                const int ti = vi[j]; vi[j] = vi[j - 1]; vi[j - 1] = ti;
            }
    float selw = 0.0f, tot = 0.0f;
    int seli = 0;
    for (int j = 0; j < k; ++j) {
        float bv = v[0];
        int bi = vi[0];
        wave_best(bv, bi, rt_better2);
        if (lane == j) { selw = bv; seli = bi; }
        tot = tot + bv;
        if (vi[0] == bi) {
#pragma unroll
            for (int i = 0; i < V - 1; ++i) { v[i] = v[i + 1]; vi[i] = vi[i + 1]; }
            v[V - 1] = -1.0f; vi[V - 1] = 0x7fffffff;
        }
    }
    if (lane < k) { ids[lane] = seli; wts[lane] = selw / tot; }
    if (lane == 0 && sg) sg[0] = 1.0f / (1.0f + hy_expf(-l[ne]));
}

template <int VT>
__global__ __launch_bounds__(256) void k_router_q8(const float *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                                   const float *__restrict__ bias, int bs, float *__restrict__ logits, int ls,
                                                   uint8_t *__restrict__ xq, int nt) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + wave, r = gw;
    // Q8 of x: global wave gw quantizes Q8_K block gw (token gw / nb) or the Q8_0 pair 2 gw ..
    if (VT == Q8_K) {
        const int nb = kdim / 256;
        if (gw < nt * nb) {
            const int t = gw / nb, b = gw % nb;
            q8k_block_wave(x + (size_t) t * xs + 256 * b, xq + ((size_t) t * nb + b) * Q8K_BYTES);
        }
    } else {
        const int nb = kdim / 32, npair = (nb + 1) / 2;
        if (gw < nt * npair) {
            const int t = gw / npair, b = 2 * (gw % npair);
            q8_0_pair_wave(x + (size_t) t * xs + 32 * b, xq + ((size_t) t * nb + b) * Q8_0_BYTES, b + 1 < nb, Q8_0_BYTES, 2);
        }
    }
    // logits of row r for every token: lane L sums elements 256 i + 4 L + j with fmaf, then the butterfly
    if (r >= rows) return;
    float acc[DEC_ROUTE_NT];
#pragma unroll
    for (int t = 0; t < DEC_ROUTE_NT; ++t) acc[t] = 0.0f;
    for (int e = 4 * lane; e < kdim; e += 256) {
        const float4 w = *(const float4 *) (W + (size_t) r * kdim + e);
#pragma unroll
        for (int t = 0; t < DEC_ROUTE_NT; ++t) {
            if (t < nt) {
                const float4 xv = *(const float4 *) (x + (size_t) t * xs + e);
                acc[t] = __builtin_fmaf(w.x, xv.x, acc[t]);
                acc[t] = __builtin_fmaf(w.y, xv.y, acc[t]);
                acc[t] = __builtin_fmaf(w.z, xv.z, acc[t]);
                acc[t] = __builtin_fmaf(w.w, xv.w, acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < DEC_ROUTE_NT; ++t) {
        if (t < nt) {
            float v = wave_sum_xor(acc[t]);
            if (bias) v = v + bias[(size_t) t * bs + r];
            if (lane == 0) logits[(size_t) t * ls + r] = v;
        }
    }
}

// ---------------------------------------------------------------- item dots against global Q8 rows

// the integers of item `it` (256 values, span gi of a row) against the Q8 row `y` (global); K-quants: summed
// over the 8 lanes (every lane of the group gets them)
template <int T>
__device__ __forceinline__ float item_t(const Item<T> &it, const uint8_t *y, int gi, int L, bool valid, float *tv_out, int tv_idx) {
    if constexpr (T == IQ4_NL) {
        // lane L takes block 8 gi + L whole: Q8_0 qs at 34 b + 2
        const uint8_t *yb = y + (size_t) (8 * gi + L) * Q8_0_BYTES;
        int s = 0;
        if (valid) {
            const uint4 y0 = load16_a2(yb + 2), y1 = load16_a2(yb + 18);
            const uint32_t q[4] = {it.qs.x, it.qs.y, it.qs.z, it.qs.w}, ya[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) { s = sdot4(kv4(q[i] & 0x0F0F0F0Fu), ya[i], s); s = sdot4(kv4((q[i] >> 4) & 0x0F0F0F0Fu), ya[4 + i], s); }
            tv_out[tv_idx + L] = it.tval(s, 0);
        }
        return 0.0f;
    } else {
        int si = 0, sm = 0;
        if (valid) it.ints(y + (size_t) gi * Q8K_BYTES, L, si, sm);
        si = group8_isum(si);
        sm = group8_isum(sm);
        if (valid && L == 0) tv_out[tv_idx] = it.tval(si, sm);
        return 0.0f;
    }
}
// activation scale of block b of a Q8 row
template <int VT> __device__ __forceinline__ float q8_scale(const uint8_t *y, int b) {
    if constexpr (VT == Q8_K) return *(const float *) (y + (size_t) b * Q8K_BYTES);
    else return h2f(ld_u16(y + (size_t) b * Q8_0_BYTES));
}

// ---------------------------------------------------------------- k_dec_gate_up

constexpr int DEC_GU_TV = 2 * 256;   // fold inputs per wave: 2 matrices x up to 256 blocks (IQ4_NL, n <= 8192)
constexpr int DEC_GU_WAVES = 8;      // ff rows per block (a wave each)

template <int T, int V, int NP>
__global__ __launch_bounds__(64 * DEC_GU_WAVES) void k_route_gate_up(hy_moe_dev m, const float *__restrict__ logits, int ls, int ne, int k,
                                                                   const uint8_t *__restrict__ xq, int *__restrict__ ids,
                                                                   float *__restrict__ wts, float *__restrict__ sg, float *__restrict__ h) {
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    constexpr int SPAN_W = 256 / BE * block_bytes(T);
    constexpr int SPAN_Y = VT == Q8_K ? Q8K_BYTES : 8 * Q8_0_BYTES;
    __shared__ float tv[DEC_GU_WAVES][DEC_GU_TV];
    __shared__ int s_ids[64];
    __shared__ float s_wts[64], s_sg;
    __shared__ int s_slot[64 * V];
    __shared__ uint2 grid[T == IQ2_XS ? 512 : 1];
    const int p = blockIdx.y, t = p / k, j = p - t * k;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 3, L = lane & 7;
    // the slot table comes in alongside the logits; the token's routing (every block of the token computes the
    // same bits); the first block of each token publishes it for the down projection
    for (int e = (int) threadIdx.x; e < ne; e += 64 * DEC_GU_WAVES) s_slot[e] = m.slot[e];
    if (wave == 0) route_wave<V>(logits + (size_t) t * ls, ne, k, s_ids, s_wts, sg ? &s_sg : nullptr);
    if constexpr (T == IQ2_XS) expand_iq2xs_grid(grid);
    __syncthreads();
    if (blockIdx.x == 0 && j == 0 && wave == 0) {
        if (lane < k) { ids[(size_t) t * k + lane] = s_ids[lane]; wts[(size_t) t * k + lane] = s_wts[lane]; }
        if (lane == 0 && sg) sg[t] = s_sg;
    }
    const int e = s_ids[j];
    const int slot = (e >= 0 && e < ne) ? s_slot[e] : -1;
    if (slot < 0) return;   // uniform over the block: the pair's h rows are not written
    const int ff = m.ff, ng = m.n / 256, nb = m.n / BE, items = 2 * ng;
    const int row = blockIdx.x * DEC_GU_WAVES + wave;
    if (row >= ff) return;  // wave-uniform; no block barrier follows
    const uint8_t *Wg = m.gate + (size_t) slot * m.gate_bytes + tiled_off(row, 0, ng, SPAN_W);
    const uint8_t *Wu = m.up + (size_t) slot * m.gate_bytes + tiled_off(row, 0, ng, SPAN_W);
    const uint8_t *y = xq + (size_t) t * ng * SPAN_Y;
    Item<T> it[NP];
#pragma unroll
    for (int ps = 0; ps < NP; ++ps) {
        const int i = g + 8 * ps;
        if (i < items) {
            const int mat = i >= ng, gi = i - mat * ng;
            it[ps].load((mat ? Wu : Wg) + (size_t) gi * HY_TILE * SPAN_W, L);
        }
    }
    float *tw = tv[wave];
#pragma unroll
    for (int ps = 0; ps < NP; ++ps) {
        const int i = g + 8 * ps;
        if (8 * ps >= items) break;   // wave-uniform
        const bool valid = i < items;
        const int mat = i >= ng, gi = i - mat * ng;
        if constexpr (T == IQ2_XS) it[ps].grid = grid;
        item_t<T>(it[ps], y, gi, L, valid, tw, mat * nb + (T == IQ4_NL ? 8 * gi : gi));
    }
    // the wave's own LDS writes, read back by its lane 0 (LDS operations of a wave complete in order)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) {
        float ag = 0.0f, au = 0.0f;
        for (int b = 0; b < nb; ++b) {
            const float xd = q8_scale<VT>(y, b);
            ag = __builtin_fmaf(xd, tw[b], ag);
            au = __builtin_fmaf(xd, tw[nb + b], au);
        }
        h[(size_t) p * ff + row] = hy_swiglu(ag, au, m.clamp);
    }
}

// ---------------------------------------------------------------- k_dec_down

constexpr int DEC_DN_WAVES = 8;       // output rows per block (a wave each)
constexpr int DEC_DN_TV = 512;        // fold inputs per wave: k pairs x blocks of ff (k * nb <= 512)
constexpr int DEC_DN_HQ = 32768;      // LDS bytes for the token's k quantized hidden rows

__device__ __forceinline__ void wave_lds_sync() {   // a wave's own LDS writes, visible to its other lanes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int T, int NP>
__global__ __launch_bounds__(64 * DEC_DN_WAVES) void k_dec_down(hy_moe_dev m, const float *__restrict__ h, const int *__restrict__ ids,
                                                               const float *__restrict__ wts, int k, const float *__restrict__ shexp,
                                                               const float *__restrict__ sg, float *__restrict__ out) {
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    constexpr int SPAN_W = 256 / BE * block_bytes(T);
    constexpr int SPAN_Y = VT == Q8_K ? Q8K_BYTES : 8 * Q8_0_BYTES;
    __shared__ __align__(16) uint8_t hq[DEC_DN_HQ];
    __shared__ float tv[DEC_DN_WAVES][DEC_DN_TV];
    __shared__ float fo[DEC_DN_WAVES][64];
    __shared__ int ordw[DEC_DN_WAVES][64];
    __shared__ uint2 grid[T == IQ2_XS ? 512 : 1];
    const int t = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 3, L = lane & 7;
    const int n = m.n, ff = m.ff, ng = ff / 256, nb = ff / BE, items = k * ng;
    const int row = blockIdx.x * DEC_DN_WAVES + wave;
    const bool row_ok = row < n;
    // lane j < k: pair j's expert and slot (-1: skipped); `okm`: the valid pairs as a wave-uniform bit mask
    const int my_e = lane < k ? ids[t * k + lane] : -1;
    const int my_slot = (my_e >= 0 && my_e < m.n_expert) ? m.slot[my_e] : -1;
    const uint64_t okm = __ballot(my_slot >= 0);
    auto pair_ok = [&](int j) { return (okm >> j) & 1; };
    Item<T> it[NP];
    auto load_round = [&](int base) {
#pragma unroll
        for (int ps = 0; ps < NP; ++ps) {
            const int i = base + g + 8 * ps;
            const int j = i / ng, gi = i - j * ng;
            const int sl = __shfl(my_slot, j < 64 ? j : 0);
            if (i < items && row_ok && sl >= 0) it[ps].load(m.down + (size_t) sl * m.down_bytes + tiled_off(row, gi, ng, SPAN_W), L);
        }
    };
    // the first round of weight bytes goes out before the hidden rows are quantized
    load_round(0);
    {
        const float *hp = h + (size_t) t * k * ff;
        // a wave's units: all their loads first, then the quantization (one memory round trip)
        constexpr int QU = 4;   // units per wave per batch
        if constexpr (VT == Q8_K) {
            const int units = k * ng;
            for (int u0 = wave; u0 < units; u0 += QU * DEC_DN_WAVES) {
                float xv[QU][4];
#pragma unroll
                for (int q = 0; q < QU; ++q) {
                    const int u = u0 + q * DEC_DN_WAVES;
                    if (u < units && pair_ok(u / ng)) {
                        const float4 v = *(const float4 *) (hp + (size_t) u * 256 + 4 * lane);
                        xv[q][0] = v.x; xv[q][1] = v.y; xv[q][2] = v.z; xv[q][3] = v.w;
                    }
                }
#pragma unroll
                for (int q = 0; q < QU; ++q) {
                    const int u = u0 + q * DEC_DN_WAVES;
                    if (u < units && pair_ok(u / ng)) q8k_block_vals(xv[q], hq + (size_t) u * Q8K_BYTES);   // wave-uniform
                }
            }
        } else {
            const int npair = (nb + 1) / 2, units = k * npair;
            for (int u0 = wave; u0 < units; u0 += QU * DEC_DN_WAVES) {
                float xv[QU];
#pragma unroll
                for (int q = 0; q < QU; ++q) {
                    const int u = u0 + q * DEC_DN_WAVES;
                    xv[q] = 0.0f;
                    if (u < units) {
                        const int j = u / npair, b = 2 * (u - j * npair);
                        if (pair_ok(j) && (lane < 32 || b + 1 < nb)) xv[q] = hp[(size_t) j * ff + 32 * b + lane];
                    }
                }
#pragma unroll
                for (int q = 0; q < QU; ++q) {
                    const int u = u0 + q * DEC_DN_WAVES;
                    if (u < units) {
                        const int j = u / npair, b = 2 * (u - j * npair);
                        if (pair_ok(j))   // wave-uniform
                            q8_0_pair_vals(xv[q], hq + (size_t) j * ng * SPAN_Y + (size_t) b * Q8_0_BYTES, b + 1 < nb, Q8_0_BYTES, 2);
                    }
                }
            }
        }
    }
    if constexpr (T == IQ2_XS) expand_iq2xs_grid(grid);
    __syncthreads();
    if (!row_ok) return;   // wave-uniform; no block barrier follows
    float *tw = tv[wave];
    for (int base = 0; base < items; base += 8 * NP) {   // wave-uniform rounds of up to 8 NP items
        if (base) load_round(base);
#pragma unroll
        for (int ps = 0; ps < NP; ++ps) {
            const int i = base + g + 8 * ps;
            if (base + 8 * ps >= items) break;   // wave-uniform
            const int j = i / ng, gi = i - j * ng;
            const bool valid = i < items && pair_ok(j);
            if constexpr (T == IQ2_XS) it[ps].grid = grid;
            item_t<T>(it[ps], hq + (size_t) j * ng * SPAN_Y, gi, L, valid, tw, j * nb + (T == IQ4_NL ? 8 * gi : gi));
        }
    }
    wave_lds_sync();
    // lane j folds pair j in block order; its rank among the valid pairs by (expert id, j) is its place in the sum
    int rank = 0;
    for (int i = 0; i < k; ++i) {   // uniform trip count; the other lanes' experts by lane read
        const int ei = __shfl(my_e, i);
        if (pair_ok(i) && (ei < my_e || (ei == my_e && i < lane))) ++rank;
    }
    if (lane < k && pair_ok(lane)) {
        const uint8_t *yj = hq + (size_t) lane * ng * SPAN_Y;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) acc = __builtin_fmaf(q8_scale<VT>(yj, b), tw[lane * nb + b], acc);
        fo[wave][lane] = wts[t * k + lane] * acc;
        ordw[wave][rank] = lane;
    }
    wave_lds_sync();
    if (lane == 0) {
        const int nv = __builtin_popcountll(okm);
        float acc = 0.0f;
        bool first = true;
        if (shexp) { acc = (sg ? sg[t] : 1.0f) * shexp[(size_t) t * n + row]; first = false; }
        for (int r = 0; r < nv; ++r) {
            const float v = fo[wave][ordw[wave][r]];
            if (first) { acc = v; first = false; } else acc = acc + v;
        }
        out[(size_t) t * n + row] = acc;
    }
}

// ---------------------------------------------------------------- launchers

#define HY_DEC_SWITCH(T, CALL)                                                                   \
    switch (T) {                                                                                 \
    case Q4_K: { constexpr int TT = Q4_K; CALL; }                                               \
    case Q5_K: { constexpr int TT = Q5_K; CALL; }                                               \
    case Q6_K: { constexpr int TT = Q6_K; CALL; }                                               \
    case IQ4_XS: { constexpr int TT = IQ4_XS; CALL; }                                           \
    case IQ2_XS: { constexpr int TT = IQ2_XS; CALL; }                                           \
    case IQ4_NL: { constexpr int TT = IQ4_NL; CALL; }                                           \
    default: set_error("unsupported expert type %d", (int) (T)); return HY_EUNSUPPORTED_TYPE;   \
    }

int launch_router_q8(const float *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                     int vtype, void *xq, int nt, hipStream_t s) {
    if (nt == 0) return HY_OK;
    if (nt > DEC_ROUTE_NT) {   // batched rows: the separate kernels
        int rc = launch_q8(vtype, x, xs, kdim, nt, xq, s);
        if (!rc) rc = launch_gemv_f32(W, rows, kdim, x, xs, logits, ls, nt, bias, bs, s);
        return rc;
    }
    const int qwaves = vtype == Q8_K ? nt * (kdim / 256) : nt * ((kdim / 32 + 1) / 2);
    const int blocks = (std::max(rows, qwaves) + 3) / 4;
    if (vtype == Q8_K)
        hipLaunchKernelGGL((k_router_q8<Q8_K>), dim3(blocks), dim3(256), 0, s, W, rows, kdim, x, xs, bias, bs, logits, ls, (uint8_t *) xq, nt);
    else
        hipLaunchKernelGGL((k_router_q8<Q8_0>), dim3(blocks), dim3(256), 0, s, W, rows, kdim, x, xs, bias, bs, logits, ls, (uint8_t *) xq, nt);
    return check_launch("hy_moe_router_q8");
}

int launch_route_gate_up(const hy_moe_dev &m, const float *logits, int ls, int ne, int k, const void *xq, int *ids, float *wts, float *sg,
                         float *h, int nt, hipStream_t s) {
    const int ng = m.n / 256, nb = m.n / block_elems(m.tg);
    if (2 * ng > 8 * DEC_MAXP || 2 * nb > DEC_GU_TV) { set_error("hy_moe_route_gate_up: n = %d exceeds %d", m.n, 256 * 4 * DEC_MAXP); return HY_EBAD_SHAPE; }
    if (nt == 0) return HY_OK;
    dim3 grid((m.ff + DEC_GU_WAVES - 1) / DEC_GU_WAVES, nt * k);
    const int V = (ne + 63) / 64;
    const int np = (2 * ng + 7) / 8;   // passes of 8 items
#define HY_RGU(VV, NN) hipLaunchKernelGGL((k_route_gate_up<TT, VV, NN>), grid, dim3(64 * DEC_GU_WAVES), 0, s, m, logits, ls, ne, k, (const uint8_t *) xq, ids, wts, sg, h)
#define HY_RGU_V(NN) if (V <= 1) HY_RGU(1, NN); else if (V <= 2) HY_RGU(2, NN); else if (V <= 4) HY_RGU(4, NN); else if (V <= 8) HY_RGU(8, NN); else HY_RGU(16, NN);
    HY_DEC_SWITCH(m.tg, {
        if (np <= 2) { HY_RGU_V(2) } else if (np <= 4) { HY_RGU_V(4) } else { HY_RGU_V(8) }
        return check_launch("hy_moe_route_gate_up");
    });
#undef HY_RGU_V
#undef HY_RGU
}

// the fused decode down + combine; shapes beyond its LDS budget return HY_EUNSUPPORTED_TYPE (caller falls back)
int launch_dec_down(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp, const float *sg,
                    float *out, int nt, hipStream_t s) {
    const int vt = vec_dot_type(m.td), ng = m.ff / 256, nb = m.ff / block_elems(m.td);
    const int span_y = vt == Q8_K ? Q8K_BYTES : 8 * Q8_0_BYTES;
    if (k > 64 || k * nb > DEC_DN_TV || (size_t) k * ng * span_y > (size_t) DEC_DN_HQ) return HY_EUNSUPPORTED_TYPE;
    if (nt == 0) return HY_OK;
    dim3 grid((m.n + DEC_DN_WAVES - 1) / DEC_DN_WAVES, nt);
    const int np = (k * ng + 7) / 8;   // passes of 8 items (more than 8: rounds)
#define HY_DN(NN) hipLaunchKernelGGL((k_dec_down<TT, NN>), grid, dim3(64 * DEC_DN_WAVES), 0, s, m, h, ids, wts, k, shexp, sg, out)
    HY_DEC_SWITCH(m.td, {
        if (np <= 2) HY_DN(2); else if (np <= 4) HY_DN(4); else HY_DN(8);
        return check_launch("hy_moe_down_reduce");
    });
#undef HY_DN
}

} // namespace hy
