// Decode path: activation quantizers, dequant-fused gate/up (SwiGLU) and down GEMVs, the combine, and the
// test hooks.  One block (4 waves) takes one (token, expert) pair and R rows; 8-lane groups take 256-value
// items of the rows (src/kernels4.cu:730-770 k_moe_gate_up, :994-1035 k_moe_down, :1070-1116 k_moe_gu_q4k).
#include "hy_internal.h"
#include "hy_blocks.cuh"

namespace hy {

// ---------------------------------------------------------------- Q8 quantizers (A4)
// the padded Q8_0 layout used in LDS: d at 0, qs at 4 (36 bytes: the qs words stay 4-byte aligned)
constexpr int Q8_0_LDS = 36;

// Q8_K: 16 blocks of 256 values per block of 256 threads, 16 lanes each (block u = token u / nb, block u % nb)
__global__ __launch_bounds__(256) void k_q8k(const float *__restrict__ x, int xs, int n, int nt, uint8_t *__restrict__ q) {
    const int nb = n / 256, u = blockIdx.x * 16 + (threadIdx.x >> 4);
    if (u >= nt * nb) return;   // uniform over the 16-lane row
    const int t = u / nb, b = u - t * nb;
    q8k_block16_load(x + (size_t) t * xs + 256 * b, q + ((size_t) t * nb + b) * Q8K_BYTES);
}
__global__ __launch_bounds__(256) void k_q8_0(const float *__restrict__ x, int xs, int n, uint8_t *__restrict__ q) {
    const int t = blockIdx.y, b = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2, nb = n / 32;
    if (b >= nb) return;
    q8_0_pair_wave(x + (size_t) t * xs + 32 * b, q + ((size_t) t * nb + b) * Q8_0_BYTES, b + 1 < nb, Q8_0_BYTES, 2);
}
int launch_q8(int vtype, const float *x, int xs, int n, int nt, void *q, hipStream_t s) {
    if (nt == 0) return HY_OK;
    if (vtype == Q8_K) hipLaunchKernelGGL(k_q8k, dim3((nt * (n / 256) + 15) / 16), dim3(256), 0, s, x, xs, n, nt, (uint8_t *) q);
    else hipLaunchKernelGGL(k_q8_0, dim3((n / 32 + 7) / 8, nt), dim3(256), 0, s, x, xs, n, (uint8_t *) q);
    return check_launch("hy_q8_quantize");
}

// quantize one fp32 row of `len` values into LDS (Q8_K: 292-byte blocks; Q8_0: padded 36-byte blocks)
template <int VT> __device__ __forceinline__ void quantize_row_lds(const float *x, int len, uint8_t *lds) {
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (VT == Q8_K) {
        for (int b = w; b < len / 256; b += nw) q8k_block_wave(x + 256 * b, lds + Q8K_BYTES * b);
    } else {
        const int nb = len / 32;
        for (int b = 2 * w; b < nb; b += 2 * nw) q8_0_pair_wave(x + 32 * b, lds + Q8_0_LDS * b, b + 1 < nb, Q8_0_LDS, 4);
    }
}

// ---------------------------------------------------------------- the GEMVs (A5, A6)
constexpr int GEMV_MAXI = 8;   // items per 8-lane group (R is chosen so that nmat * R * ng <= 32 * GEMV_MAXI)
__host__ __device__ constexpr int lds16(int bytes) { return (bytes + 15) / 16 * 16; }

// GU: h[p][r0 + i] = swiglu(gate . x, up . x); else y[p][r0 + i] = w[p] * (down . q8(h[p])).
// LDS: [quantized input][t values: nmat x R x nb][fold results 2 x R][IQ2_XS grid]
template <int T, bool GU>
__global__ __launch_bounds__(256) void k_gemv(hy_moe_dev m, int n_expert, const float *__restrict__ src, int ss, const int *__restrict__ ids,
                                              int k, const float *__restrict__ wts, float *__restrict__ dst, int R,
                                              const int *__restrict__ order, const int *__restrict__ order_n) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    int p;
    if (order) { if ((int) blockIdx.x >= *order_n) return; p = order[blockIdx.x]; }
    else p = blockIdx.x;
    const int e = ids[p];
    const int slot = (e >= 0 && e < n_expert) ? bound_slot(m.slot[e], m.n_local) : -1;
    const int in_dim = GU ? m.n : m.ff, rows = GU ? m.ff : m.n;
    const int r0 = blockIdx.y * R, nr = min(R, rows - r0);
    if (slot < 0) {
        if (!GU && !order)
            for (int i = threadIdx.x; i < nr; i += blockDim.x) dst[(size_t) p * m.n + r0 + i] = 0.0f;
        return;
    }
    const int nb = in_dim / BE, ng = in_dim / 256;
    const int nmat = GU ? 2 : 1;
    const size_t mbytes = GU ? m.gate_bytes : m.down_bytes;
    const uint8_t *W0 = (GU ? m.gate : m.down) + (size_t) slot * mbytes;
    const uint8_t *W1 = GU ? m.up + (size_t) slot * mbytes : nullptr;
    const float *xin = src + (size_t) (GU ? p / k : p) * ss;

    uint8_t *xq = smem;
    const int xq_bytes = lds16(VT == Q8_K ? ng * Q8K_BYTES : nb * Q8_0_LDS);
    float *tv = (float *) (smem + xq_bytes);
    float *fo = (float *) (smem + xq_bytes + lds16(4 * nmat * R * nb));
    uint2 *grid = (uint2 *) (smem + xq_bytes + lds16(4 * nmat * R * nb) + lds16(4 * 2 * R));

    const int g = threadIdx.x >> 3, L = threadIdx.x & 7;
    const int items = nmat * nr * ng;
    Item<T> it[GEMV_MAXI];
#pragma unroll
    for (int i = 0; i < GEMV_MAXI; ++i) {
        const int id = g + 32 * i;
        if (id < items) {
            const int mat = id / (nr * ng), rem = id % (nr * ng), row = rem / ng, gi = rem % ng;
            const uint8_t *base = (mat ? W1 : W0) + tiled_off(r0 + row, gi, ng, span_bytes(T));
            it[i].load(base, L);
        }
    }
    quantize_row_lds<VT>(xin, in_dim, xq);
    if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < GEMV_MAXI; ++i) {
        const int id = g + 32 * i;
        if (id < items) {
            const int mat = id / (nr * ng), rem = id % (nr * ng), row = rem / ng, gi = rem % ng;
            if constexpr (iq2_type(T)) it[i].grid = grid;
            int si, sm;
            if constexpr (block_elems(T) == 32) {
                it[i].ints(xq + (8 * gi + L) * Q8_0_LDS, L, si, sm);
                tv[(mat * R + row) * nb + 8 * gi + L] = it[i].tval(si, sm);
            } else {
                it[i].ints(xq + gi * Q8K_BYTES, L, si, sm);
                si = group8_isum(si);
                sm = group8_isum(sm);
                if (L == 0) tv[(mat * R + row) * nb + gi] = it[i].tval(si, sm);
            }
        }
    }
    __syncthreads();
    for (int f = threadIdx.x; f < nmat * nr; f += blockDim.x) {
        const int mat = f / nr, row = f % nr;
        const float *t = tv + (mat * R + row) * nb;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) {
            const float xd = VT == Q8_K ? *(const float *) (xq + b * Q8K_BYTES) : h2f(*(const uint16_t *) (xq + b * Q8_0_LDS));
            acc = __builtin_fmaf(xd, t[b], acc);
        }
        fo[mat * R + row] = acc;
    }
    __syncthreads();
    for (int f = threadIdx.x; f < nr; f += blockDim.x) {
        if (GU) dst[(size_t) p * m.ff + r0 + f] = hy_swiglu(fo[f], fo[R + f], m.clamp);
        else dst[(size_t) p * m.n + r0 + f] = wts[p] * fo[f];
    }
}

template <int T, bool GU> static size_t gemv_lds(int in_dim, int R) {
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    const int nb = in_dim / BE, ng = in_dim / 256, nmat = GU ? 2 : 1;
    return lds16(VT == Q8_K ? ng * Q8K_BYTES : nb * Q8_0_LDS) + lds16(4 * nmat * R * nb) + lds16(4 * 2 * R) + (iq2_type(T) ? iq2_lds(T) * 8 : 0);
}

template <int T, bool GU>
static int launch_gemv_t(const hy_moe_dev &m, const float *src, int ss, const int *ids, int k, const float *wts, float *dst, int nt,
                         hipStream_t s, const int *order, const int *order_n) {
    const int in_dim = GU ? m.n : m.ff, rows = GU ? m.ff : m.n, ng = in_dim / 256, nmat = GU ? 2 : 1;
    int R = 32 * GEMV_MAXI / (nmat * ng);
    if (R < 1) { set_error("%s: input dimension %d exceeds %d", GU ? "hy_moe_gate_up" : "hy_moe_down", in_dim, 256 * 32 * GEMV_MAXI / nmat); return HY_EBAD_SHAPE; }
    if (R > rows) R = rows;
    if (R > 128) R = 128;
    const size_t lds = gemv_lds<T, GU>(in_dim, R);
    if (lds > 64 * 1024) { set_error("%s: %zu bytes of LDS needed", GU ? "hy_moe_gate_up" : "hy_moe_down", lds); return HY_EBAD_SHAPE; }
    dim3 grid(nt * k, (rows + R - 1) / R);
    if (grid.x == 0) return HY_OK;
    hipLaunchKernelGGL((k_gemv<T, GU>), grid, dim3(256), lds, s, m, m.n_expert, src, ss, ids, k, wts, dst, R, order, order_n);
    return check_launch(GU ? "hy_moe_gate_up" : "hy_moe_down");
}

#define HY_TYPE_SWITCH(T, CALL)                                                           \
    switch (T) {                                                                          \
    case Q4_K: { constexpr int TT = Q4_K; CALL; }                                        \
    case Q5_K: { constexpr int TT = Q5_K; CALL; }                                        \
    case Q6_K: { constexpr int TT = Q6_K; CALL; }                                        \
    case IQ4_XS: { constexpr int TT = IQ4_XS; CALL; }                                    \
    case IQ2_XS: { constexpr int TT = IQ2_XS; CALL; }                                    \
    case IQ2_XXS: { constexpr int TT = IQ2_XXS; CALL; }                                  \
    case IQ4_NL: { constexpr int TT = IQ4_NL; CALL; }                                    \
    case Q8_0: { constexpr int TT = Q8_0; CALL; }                                        \
    case MXFP4: { constexpr int TT = MXFP4; CALL; }                                      \
    case Q5_0: { constexpr int TT = Q5_0; CALL; }                                        \
    case Q5_1: { constexpr int TT = Q5_1; CALL; }                                        \
    case Q2_K: { constexpr int TT = Q2_K; CALL; }                                        \
    case Q3_K: { constexpr int TT = Q3_K; CALL; }                                        \
    case IQ3_XXS: { constexpr int TT = IQ3_XXS; CALL; }                                  \
    case IQ3_S: { constexpr int TT = IQ3_S; CALL; }                                      \
    case IQ2_S: { constexpr int TT = IQ2_S; CALL; }                                      \
    case IQ1_S: { constexpr int TT = IQ1_S; CALL; }                                      \
    default: set_error("unsupported expert type %d", (int) (T)); return HY_EUNSUPPORTED_TYPE; \
    }

int launch_gate_up(const hy_moe_dev &m, const float *x, int xs, const int *ids, int k, float *h, int nt, hipStream_t s, const int *order,
                   const int *order_n) {
    HY_TYPE_SWITCH(m.tg, return (launch_gemv_t<TT, true>(m, x, xs, ids, k, nullptr, h, nt, s, order, order_n)));
}
int launch_down(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, float *y, int nt, hipStream_t s,
                const int *order, const int *order_n) {
    HY_TYPE_SWITCH(m.td, return (launch_gemv_t<TT, false>(m, h, m.ff, ids, k, wts, y, nt, s, order, order_n)));
}

// ---------------------------------------------------------------- combine (A9)
// out[t][r] = sg * shexp (if shexp) then + y of the token's pairs in ascending expert id (src/cpu_moe.cpp:863-874
// order; the first pair is the start value when there is no shared expert); negative ids are skipped.  One block
// per token: wave 0 ranks the token's pairs (rank = valid pairs with a smaller id, ties by position), then every
// thread sums VW consecutive columns per pass (VW = 4: 16-byte loads when n and the rows allow it).
template <int VW>
__global__ __launch_bounds__(256) void k_reduce(const float *__restrict__ shexp, const float *__restrict__ sg, const float *__restrict__ y,
                                                int k, float *__restrict__ out, int n, const int *__restrict__ ids, int res) {
    __shared__ int ord[64];
    __shared__ int s_cnt;
    const int t = blockIdx.x, tid = threadIdx.x;
    if (tid < 64) {
        const int e = tid < k ? ids[(size_t) t * k + tid] : -1;
        int rank = 0;
        for (int i = 0; i < k; ++i) {
            const int o = __shfl(e, i);
            rank += (o >= 0 && (o < e || (o == e && i < tid))) ? 1 : 0;
        }
        if (e >= 0) ord[rank] = tid;
        const int c = __popcll(__ballot(e >= 0));
        if (tid == 0) s_cnt = c;
    }
    __syncthreads();
    const int c = s_cnt;
    const float g = shexp ? (sg ? sg[t] : 1.0f) : 0.0f;
    for (int r = VW * tid; r < n; r += VW * (int) blockDim.x) {
        float acc[VW] = {}, v[VW];   // a token with no shared expert and no valid pair gets zeros
        bool first = true;
        if (shexp) {
            if constexpr (VW == 4) { const float4 x = *(const float4 *) (shexp + (size_t) t * n + r); v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; }
            else v[0] = shexp[(size_t) t * n + r];
#pragma unroll
            for (int j = 0; j < VW; ++j) acc[j] = g * v[j];
            first = false;
        }
        // the pairs' rows in batches of 8 whose loads are all in flight before the first add; the adds keep the
        // ascending expert-id order
        for (int i0 = 0; i0 < c; i0 += 8) {
            float b[8][VW];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + u < c) {
                    const float *yp = y + ((size_t) t * k + ord[i0 + u]) * n + r;
                    if constexpr (VW == 4) { const float4 x = *(const float4 *) yp; b[u][0] = x.x; b[u][1] = x.y; b[u][2] = x.z; b[u][3] = x.w; }
                    else b[u][0] = *yp;
                }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + u < c) {
#pragma unroll
                    for (int j = 0; j < VW; ++j) acc[j] = first ? b[u][j] : acc[j] + b[u][j];
                    first = false;
                }
        }
        if (res) {   // the residual add: out (the residual) + the part, as a separate rounding
            if constexpr (VW == 4) { const float4 o = *(const float4 *) (out + (size_t) t * n + r); acc[0] = o.x + acc[0]; acc[1] = o.y + acc[1]; acc[2] = o.z + acc[2]; acc[3] = o.w + acc[3]; }
            else acc[0] = out[(size_t) t * n + r] + acc[0];
        }
        if constexpr (VW == 4) *(float4 *) (out + (size_t) t * n + r) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        else out[(size_t) t * n + r] = acc[0];
    }
}
int launch_reduce(const float *shexp, const float *sg, const float *y, int k, float *out, int n, int nt, const int *ids, hipStream_t s, int res) {
    if (nt == 0) return HY_OK;
    const bool vec = n % 4 == 0 && ((uintptr_t) y & 15) == 0 && ((uintptr_t) out & 15) == 0 && ((uintptr_t) shexp & 15) == 0;
    if (vec) hipLaunchKernelGGL(k_reduce<4>, dim3(nt), dim3(256), 0, s, shexp, sg, y, k, out, n, ids, res);
    else hipLaunchKernelGGL(k_reduce<1>, dim3(nt), dim3(256), 0, s, shexp, sg, y, k, out, n, ids, res);
    return check_launch("hy_moe_reduce");
}

// ---------------------------------------------------------------- fused decode down + combine
// A block takes token t and R output rows for all k pairs: h of the k pairs quantized into LDS, pairs visited in
// ascending expert id, out = sg * shexp (if shexp) then + w * (down . q8(h)), the first pair starting the sum.
template <int T>
__global__ __launch_bounds__(256) void k_down_reduce(hy_moe_dev m, int n_expert, const float *__restrict__ h, const int *__restrict__ ids,
                                                     int k, const float *__restrict__ wts, const float *__restrict__ shexp,
                                                     const float *__restrict__ sg, float *__restrict__ out, int R, int res) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    const int t = blockIdx.x, in_dim = m.ff, rows = m.n;
    const int r0 = blockIdx.y * R, nr = min(R, rows - r0);
    const int nb = in_dim / BE, ng = in_dim / 256;
    const int xq_row = VT == Q8_K ? ng * Q8K_BYTES : nb * Q8_0_LDS;
    const int o_tv = lds16(k * xq_row), o_fo = o_tv + lds16(4 * k * R * nb), o_ord = o_fo + lds16(4 * k * R), o_grid = o_ord + lds16(4 * k);
    uint8_t *xq = smem;
    float *tv = (float *) (smem + o_tv);     // [k][R][nb]
    float *fo = (float *) (smem + o_fo);     // [k][R]
    int *ord = (int *) (smem + o_ord);       // [k]: pair order by expert, -1 past the valid ones
    uint2 *grid = (uint2 *) (smem + o_grid);
    if (threadIdx.x == 0) {
        int c = 0;
        for (int j = 0; j < k; ++j) {
            const int e = ids[t * k + j];
            if (e < 0 || e >= n_expert || bound_slot(m.slot[e], m.n_local) < 0) continue;
            int i = c++;
            while (i > 0 && ids[t * k + ord[i - 1]] > e) { ord[i] = ord[i - 1]; --i; }
            ord[i] = j;
        }
        for (int i = c; i < k; ++i) ord[i] = -1;
    }
    const int g = threadIdx.x >> 3, L = threadIdx.x & 7;
    const int items = k * nr * ng;
    // pairs are indexed by j here (route rank); ord gives the summation order
    Item<T> it[GEMV_MAXI];
#pragma unroll
    for (int i = 0; i < GEMV_MAXI; ++i) {
        const int id = g + 32 * i;
        if (id < items) {
            const int j = id / (nr * ng), rem = id % (nr * ng), row = rem / ng, gi = rem % ng;
            const int e = ids[t * k + j];
            const int sl = (e >= 0 && e < n_expert) ? bound_slot(m.slot[e], m.n_local) : -1;
            if (sl >= 0) {
                const uint8_t *base = m.down + (size_t) sl * m.down_bytes + tiled_off(r0 + row, gi, ng, span_bytes(T));
                it[i].load(base, L);
            }
        }
    }
    for (int j = 0; j < k; ++j) quantize_row_lds<VT>(h + ((size_t) t * k + j) * in_dim, in_dim, xq + j * xq_row);
    if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < GEMV_MAXI; ++i) {
        const int id = g + 32 * i;
        if (id < items) {
            const int j = id / (nr * ng), rem = id % (nr * ng), row = rem / ng, gi = rem % ng;
            if constexpr (iq2_type(T)) it[i].grid = grid;
            int si, sm;
            if constexpr (block_elems(T) == 32) {
                it[i].ints(xq + j * xq_row + (8 * gi + L) * Q8_0_LDS, L, si, sm);
                tv[(j * R + row) * nb + 8 * gi + L] = it[i].tval(si, sm);
            } else {
                it[i].ints(xq + j * xq_row + gi * Q8K_BYTES, L, si, sm);
                si = group8_isum(si);
                sm = group8_isum(sm);
                if (L == 0) tv[(j * R + row) * nb + gi] = it[i].tval(si, sm);
            }
        }
    }
    __syncthreads();
    for (int f = threadIdx.x; f < k * nr; f += blockDim.x) {
        const int j = f / nr, row = f % nr;
        const float *tt = tv + (j * R + row) * nb;
        const uint8_t *xj = xq + j * xq_row;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) {
            const float xd = VT == Q8_K ? *(const float *) (xj + b * Q8K_BYTES) : h2f(*(const uint16_t *) (xj + b * Q8_0_LDS));
            acc = __builtin_fmaf(xd, tt[b], acc);
        }
        fo[j * R + row] = acc;
    }
    __syncthreads();
    for (int f = threadIdx.x; f < nr; f += blockDim.x) {
        float acc = 0.0f;
        bool first = true;
        if (shexp) { acc = (sg ? sg[t] : 1.0f) * shexp[(size_t) t * rows + r0 + f]; first = false; }
        for (int i = 0; i < k && ord[i] >= 0; ++i) {
            const int j = ord[i];
            const float v = wts[t * k + j] * fo[j * R + f];
            if (first) { acc = v; first = false; } else acc = acc + v;
        }
        out[(size_t) t * rows + r0 + f] = res ? out[(size_t) t * rows + r0 + f] + acc : acc;
    }
}

template <int T>
static int launch_down_reduce_t(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp,
                                const float *sg, float *out, int nt, hipStream_t s, int res) {
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    const int in_dim = m.ff, rows = m.n, ng = in_dim / 256, nb = in_dim / BE;
    int R = 32 * GEMV_MAXI / (k * ng);
    if (R < 1) { set_error("hy_moe_down_reduce: k * ff / 256 = %d exceeds %d", k * ng, 32 * GEMV_MAXI); return HY_EBAD_SHAPE; }
    if (R > rows) R = rows;
    const int xq_row = VT == Q8_K ? ng * Q8K_BYTES : nb * Q8_0_LDS;
    const size_t lds = lds16(k * xq_row) + lds16(4 * k * R * nb) + lds16(4 * k * R) + lds16(4 * k) + (iq2_type(T) ? iq2_lds(T) * 8 : 0);
    if (lds > 64 * 1024) { set_error("hy_moe_down_reduce: %zu bytes of LDS needed", lds); return HY_EBAD_SHAPE; }
    if (nt == 0) return HY_OK;
    dim3 grid(nt, (rows + R - 1) / R);
    hipLaunchKernelGGL((k_down_reduce<T>), grid, dim3(256), lds, s, m, m.n_expert, h, ids, k, wts, shexp, sg, out, R, res);
    return check_launch("hy_moe_down_reduce");
}
int launch_down_reduce(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp, const float *sg,
                       float *out, int nt, hipStream_t s, int res) {
    HY_TYPE_SWITCH(m.td, return (launch_down_reduce_t<TT>(m, h, ids, wts, k, shexp, sg, out, nt, s, res)));
}

// ---------------------------------------------------------------- test hooks
// one row dequantized with the deq8 expressions (src/kernels4.cu:421-714): thread per value
__global__ void k_dequant(int type, const uint8_t *__restrict__ row, int n, float *__restrict__ out) {
    __shared__ uint2 grid[GRID_LDS];
    if (type == IQ2_XS) expand_iq2_grid<IQ2_XS>(grid);
    else if (type == IQ2_XXS) expand_iq2_grid<IQ2_XXS>(grid);
    else if (type == IQ3_XXS) expand_iq2_grid<IQ3_XXS>(grid);
    else if (type == IQ3_S) expand_iq2_grid<IQ3_S>(grid);
    else if (type == IQ2_S) expand_iq2_grid<IQ2_S>(grid);
    else if (type == IQ1_S) expand_iq2_grid<IQ1_S>(grid);
    __syncthreads();
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = 0.0f;
    if (type == Q4_K || type == Q5_K) {
        const int bb = type == Q4_K ? 144 : 176;
        const uint8_t *b = row + (size_t) (i >> 8) * bb;
        const int e = i & 255, j = e >> 5, l = e & 31;
        int sc, mn;
        scale_min_k4(*(const uint32_t *) (b + 4), *(const uint32_t *) (b + 8), *(const uint32_t *) (b + 12), j, sc, mn);
        const float d = h2f(ld_u16(b)) * (float) sc, m = h2f(ld_u16(b + 2)) * (float) mn;
        int q;
        if (type == Q4_K) q = (b[16 + 32 * (j >> 1) + l] >> (4 * (j & 1))) & 0xF;
        else q = ((b[48 + 32 * (j >> 1) + l] >> (4 * (j & 1))) & 0xF) | (((b[16 + l] >> j) & 1) << 4);
        v = d * (float) q - m;
    } else if (type == Q6_K) {
        const uint8_t *b = row + (size_t) (i >> 8) * 210;
        const int e = i & 255, hf = e >> 7, qt = (e >> 5) & 3, l = e & 31;
        const int q = (((b[hf * 64 + (qt & 1) * 32 + l] >> (qt >= 2 ? 4 : 0)) & 0xF) | (((b[128 + hf * 32 + l] >> (2 * qt)) & 3) << 4)) - 32;
        const float d = h2f(ld_u16(b + 208)) * (float) (int8_t) b[192 + hf * 8 + (l >> 4) + 2 * qt];
        v = d * (float) q;
    } else if (type == IQ4_XS) {
        const uint8_t *b = row + (size_t) (i >> 8) * 136;
        const int e = i & 255, ib = e >> 5, l = e & 31;
        const int sh = ld_u16(b + 2);
        const int ls = ((b[4 + (ib >> 1)] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
        const float dl = h2f(ld_u16(b)) * (float) (ls - 32);
        v = dl * (float) c_kv_iq4nl[(b[8 + 16 * ib + (l & 15)] >> (l >= 16 ? 4 : 0)) & 0xF];
    } else if (type == IQ4_NL) {
        const uint8_t *b = row + (size_t) (i >> 5) * 18;
        const int e = i & 31;
        v = (float) c_kv_iq4nl[(b[2 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF] * h2f(ld_u16(b));
    } else if (type == IQ2_XS) {
        const uint8_t *b = row + (size_t) (i >> 8) * 74;
        const int e = i & 255, ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
        const float db = h2f(ld_u16(b)) * (0.5f + (float) ((b[66 + ib] >> (4 * (l >> 1))) & 0xF)) * 0.25f;
        const int q = ld_u16(b + 2 + 2 * (4 * ib + l));
        const uint2 gr = grid[q & 511];
        const float gv = (float) (((j < 4 ? gr.x : gr.y) >> (8 * (j & 3))) & 0xff);
        v = (db * gv) * ((ksign(q >> 9) >> j) & 1 ? -1.0f : 1.0f);
    } else if (type == IQ2_XXS) {
        const uint8_t *b = row + (size_t) (i >> 8) * 66;
        const int e = i & 255, ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
        const uint32_t a1 = (uint32_t) ld_u16(b + 6 + 8 * ib) | ((uint32_t) ld_u16(b + 8 + 8 * ib) << 16);
        const float db = h2f(ld_u16(b)) * (0.5f + (float) (a1 >> 28)) * 0.25f;
        const uint2 gr = grid[b[2 + 8 * ib + l]];
        const float gv = (float) (((j < 4 ? gr.x : gr.y) >> (8 * (j & 3))) & 0xff);
        v = (db * gv) * ((ksign((a1 >> (7 * l)) & 127) >> j) & 1 ? -1.0f : 1.0f);
    } else if (type == MXFP4) {   // src/kernels4.cu:569-577
        const uint8_t *b = row + (size_t) (i >> 5) * 17;
        const int e = i & 31;
        v = (float) (int8_t) (kvfp4((b[1 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF) & 0xff) * e8m0_half(b[0]);
    } else if (type == IQ1_S) {   // src/kernels4.cu:650-659
        const uint8_t *b = row + (size_t) (i >> 8) * 50;
        const int e = i & 255, ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
        const int qh = ld_u16(b + 34 + 2 * ib);
        const float dl = h2f(ld_u16(b)) * (float) (2 * ((qh >> 12) & 7) + 1);
        const float delta = qh & 0x8000 ? -0.125f : 0.125f;
        const uint2 gr = grid[b[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7) << 8)];
        v = dl * ((float) (int8_t) (((j < 4 ? gr.x : gr.y) >> (8 * (j & 3))) & 0xff) + delta);
    } else if (type == IQ2_S) {   // src/kernels4.cu:602-613
        const uint8_t *b = row + (size_t) (i >> 8) * 82;
        const int e = i & 255, ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
        const float db = h2f(ld_u16(b)) * (0.5f + (float) ((b[74 + ib] >> (4 * (l >> 1))) & 0xf)) * 0.25f;
        const uint2 gr = grid[b[2 + 4 * ib + l] | (((b[66 + ib] >> (2 * l)) & 3) << 8)];
        const float gv = (float) (((j < 4 ? gr.x : gr.y) >> (8 * (j & 3))) & 0xff);
        v = (db * gv) * ((b[34 + 4 * ib + l] >> j) & 1 ? -1.0f : 1.0f);
    } else if (type == IQ3_S) {   // src/kernels4.cu:682-695
        const uint8_t *b = row + (size_t) (i >> 8) * 110;
        const int e = i & 255, ib = e >> 5, l = (e >> 3) & 3, j = e & 7, hb = 2 * l + (j >> 2);
        const float db = h2f(ld_u16(b)) * (float) (1 + 2 * ((b[106 + (ib >> 1)] >> (4 * (ib & 1))) & 15));
        const uint32_t gr = grid[b[2 + 8 * ib + hb] | (((b[66 + ib] >> hb) & 1) << 8)].x;
        const float gv = (float) ((gr >> (8 * (j & 3))) & 0xff);
        v = (db * gv) * ((b[74 + 4 * ib + l] >> j) & 1 ? -1.0f : 1.0f);
    } else if (type == IQ3_XXS) {   // src/kernels4.cu:613-627
        const uint8_t *b = row + (size_t) (i >> 8) * 98;
        const int e = i & 255, ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
        const uint32_t a = (uint32_t) ld_u16(b + 66 + 4 * ib) | ((uint32_t) ld_u16(b + 68 + 4 * ib) << 16);
        const float db = h2f(ld_u16(b)) * (0.5f + (float) (a >> 28)) * 0.5f;
        const uint32_t gr = grid[b[2 + 8 * ib + 2 * l + (j >> 2)]].x;
        const float gv = (float) ((gr >> (8 * (j & 3))) & 0xff);
        v = (db * gv) * ((ksign((a >> (7 * l)) & 127) >> j) & 1 ? -1.0f : 1.0f);
    } else if (type == Q3_K) {   // src/kernels4.cu:698-707
        const uint8_t *b = row + (size_t) (i >> 8) * 110;
        const int e = i & 255, is = e >> 4, hf = e >> 7, j = (e >> 5) & 3, l = e & 31;
        const int sc = (((b[96 + (is & 7)] >> (4 * (is >> 3))) & 15) | (((b[104 + (is & 3)] >> (2 * (is >> 2))) & 3) << 4)) - 32;
        const float dl = h2f(ld_u16(b + 108)) * (float) sc;
        v = dl * (float) (((b[32 + 32 * hf + l] >> (2 * j)) & 3) - (((b[l] >> (4 * hf + j)) & 1) ? 0 : 4));
    } else if (type == Q2_K) {   // src/kernels4.cu:639-647
        const uint8_t *b = row + (size_t) (i >> 8) * 84;
        const int e = i & 255, sc = b[e >> 4];
        const int q = (b[16 + 32 * (e >> 7) + (e & 31)] >> (2 * ((e >> 5) & 3))) & 3;
        const float dl = h2f(ld_u16(b + 80)) * (float) (sc & 15), ml = h2f(ld_u16(b + 82)) * (float) (sc >> 4);
        v = dl * (float) q - ml;
    } else if (type == Q5_1) {   // src/kernels4.cu:449-462
        const uint8_t *b = row + (size_t) (i >> 5) * 24;
        const int e = i & 31;
        const uint32_t qh = (uint32_t) ld_u16(b + 4) | ((uint32_t) ld_u16(b + 6) << 16);
        const int x = ((b[8 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF) | (((qh >> e) & 1) << 4);
        v = (float) x * h2f(ld_u16(b)) + h2f(ld_u16(b + 2));
    } else if (type == Q5_0) {   // src/kernels4.cu:464-478
        const uint8_t *b = row + (size_t) (i >> 5) * 22;
        const int e = i & 31;
        const uint32_t qh = (uint32_t) ld_u16(b + 2) | ((uint32_t) ld_u16(b + 4) << 16);
        const int x = ((b[6 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF) | (((qh >> e) & 1) << 4);
        v = (float) (x - 16) * h2f(ld_u16(b));
    } else if (type == Q8_0) {
        const uint8_t *b = row + (size_t) (i >> 5) * 34;
        v = h2f(ld_u16(b)) * (float) (int8_t) b[2 + (i & 31)];
    } else if (type == Q8_K) {
        const uint8_t *b = row + (size_t) (i >> 8) * 292;
        v = *(const float *) b * (float) (int8_t) b[4 + (i & 255)];
    }
    out[i] = v;
}
int launch_dequant_row(int type, const uint8_t *row, int n, float *out, hipStream_t s) {
    if (n == 0) return HY_OK;
    hipLaunchKernelGGL(k_dequant, dim3((n + 255) / 256), dim3(256), 0, s, type, row, n, out);
    return check_launch("hy_dequant_row");
}

// every block's exact integers through the decode kernels' item code: a group of 8 lanes per (row, 256-value
// item); Q8 activations read from global memory (Q8_0 repacked into the padded LDS layout first)
template <int T>
__global__ __launch_bounds__(256) void k_block_ints(const uint8_t *__restrict__ rows, size_t row_bytes, int nrows, const uint8_t *__restrict__ xq,
                                                    int n, int *__restrict__ sumi, int *__restrict__ summ) {
    __shared__ uint2 grid[GRID_LDS];
    __shared__ __align__(16) uint8_t y0[8 * Q8_0_LDS * 32];
    constexpr int BE = block_elems(T), VT = vec_dot_type(T);
    const int ng = n / 256, nb = n / BE;
    if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
    if (VT == Q8_0)   // repack up to 256 Q8_0 blocks of the activation row into the padded layout
        for (int i = threadIdx.x; i < nb && i < 256; i += blockDim.x) {
            const uint8_t *s = xq + i * Q8_0_BYTES;
            uint8_t *d = y0 + i * Q8_0_LDS;
            *(uint16_t *) d = ld_u16(s);
            for (int j = 0; j < 32; ++j) d[4 + j] = s[2 + j];
        }
    __syncthreads();
    const int g = blockIdx.x * 32 + (threadIdx.x >> 3), L = threadIdx.x & 7;
    if (g >= nrows * ng) return;
    const int row = g / ng, gi = g % ng;
    Item<T> it;
    it.load(rows + row * row_bytes + (size_t) gi * (256 / BE) * block_bytes(T), L);
    if constexpr (iq2_type(T)) it.grid = grid;
    int si, sm;
    if constexpr (block_elems(T) == 32) {
        it.ints(y0 + (8 * gi + L) * Q8_0_LDS, L, si, sm);
        sumi[row * nb + 8 * gi + L] = si;
        summ[row * nb + 8 * gi + L] = sm;   // (Q5_1: the activation block's sum; the others 0)
    } else {
        it.ints(xq + gi * Q8K_BYTES, L, si, sm);
        si = group8_isum(si);
        sm = group8_isum(sm);
        if (L == 0) { sumi[row * nb + gi] = si; summ[row * nb + gi] = sm; }
    }
}
int launch_block_ints(int type, const uint8_t *rows, size_t row_bytes, int nrows, const void *xq, int n, int *sumi, int *summ,
                      hipStream_t s) {
    const int groups = nrows * (n / 256);
    if (groups == 0) return HY_OK;
    if (vec_dot_type(type) == Q8_0 && n / 32 > 256) { set_error("hy_block_ints: rows of 32-value blocks longer than 8192"); return HY_EBAD_SHAPE; }
    dim3 grid((groups + 31) / 32);
    HY_TYPE_SWITCH(type, hipLaunchKernelGGL((k_block_ints<TT>), grid, dim3(256), 0, s, rows, row_bytes, nrows, (const uint8_t *) xq, n,
                                            sumi, summ);
                   return check_launch("hy_block_ints"));
}

} // namespace hy
