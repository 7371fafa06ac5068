// Router GEMV, softmax/top-k routing and token->expert bucketing.
#include "hy_internal.h"

namespace hy {

// ---------------------------------------------------------------- router logits (A1)
// y[t][r] = W[r] . x[t] (+ bias[t][r]): src/kernels4.cu:163-180 (gemv_f32).  Summation order of the contract:
// lane L of a wave accumulates elements 256 i + 4 L + j (j = 0..3) with fmaf in index order, then the
// 64 partial sums meet in an xor butterfly (1, 2, ..., 32).  A wave computes RW rows x TW tokens.
template <int RW, int TW>
__global__ __launch_bounds__(256) void k_gemv_f32(const float *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                                  float *__restrict__ y, int ys, int nt, const float *__restrict__ bias, int bs) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = (blockIdx.x * 4 + wave) * RW, t0 = blockIdx.y * TW;
    if (r0 >= rows) return;
    float acc[RW][TW];
#pragma unroll
    for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int b = 0; b < TW; ++b) acc[a][b] = 0.0f;
    for (int e = 4 * lane; e < kdim; e += 256) {
        float4 w[RW], xv[TW];
#pragma unroll
        for (int a = 0; a < RW; ++a) w[a] = r0 + a < rows ? *(const float4 *) (W + (size_t) (r0 + a) * kdim + e) : make_float4(0, 0, 0, 0);
#pragma unroll
        for (int b = 0; b < TW; ++b) xv[b] = t0 + b < nt ? *(const float4 *) (x + (size_t) (t0 + b) * xs + e) : make_float4(0, 0, 0, 0);
#pragma unroll
        for (int a = 0; a < RW; ++a)
#pragma unroll
            for (int b = 0; b < TW; ++b) {
                float s = acc[a][b];
                s = __builtin_fmaf(w[a].x, xv[b].x, s);
                s = __builtin_fmaf(w[a].y, xv[b].y, s);
                s = __builtin_fmaf(w[a].z, xv[b].z, s);
                s = __builtin_fmaf(w[a].w, xv[b].w, s);
                acc[a][b] = s;
            }
    }
#pragma unroll
    for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int b = 0; b < TW; ++b) {
            float s = wave_sum_xor(acc[a][b]);
            if (lane == 0 && r0 + a < rows && t0 + b < nt) {
                if (bias) s = s + bias[(size_t) (t0 + b) * bs + r0 + a];
                y[(size_t) (t0 + b) * ys + r0 + a] = s;
            }
        }
}

int launch_gemv_f32(const float *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bs,
                    hipStream_t s) {
    if (nt <= 4) {
        dim3 g((rows + 3) / 4, nt);
        hipLaunchKernelGGL((k_gemv_f32<1, 1>), g, dim3(256), 0, s, W, rows, kdim, x, xs, y, ys, nt, bias, bs);
    } else {
        dim3 g((rows + 15) / 16, (nt + 7) / 8);
        hipLaunchKernelGGL((k_gemv_f32<4, 8>), g, dim3(256), 0, s, W, rows, kdim, x, xs, y, ys, nt, bias, bs);
    }
    return check_launch("hy_gemv_f32");
}

// ---------------------------------------------------------------- routing (A2)
__device__ __forceinline__ bool rt_better(float a, int ia, float b, int ib) { return (a > b) | ((a == b) & (ia < ib)); }   // no short circuit: no branches

// a wave per token, expert e in lane e % 64 slot e / 64 (V slots): max, exp, the contract's sum (lane L adds
// its experts in slot order, then the xor butterfly), p = v / s; each lane sorts its V candidates
// (descending, ties to the lower index), then k rounds of wave argmax; weights p_j / sum of the selected
// (summed in selection order); sg = sigmoid(logit ne).  src/kernels4.cu:297-344.
template <int V>
__global__ __launch_bounds__(64) void k_route(const float *__restrict__ logits, int ls, int ne, int k, int *__restrict__ ids,
                                              float *__restrict__ wts, float *__restrict__ sg) {
    const int t = blockIdx.x, lane = threadIdx.x;
    const float *l = logits + (size_t) t * ls;
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
            if (rt_better(v[j], vi[j], v[j - 1], vi[j - 1])) {
                const float tv = v[j]; v[j] = v[j - 1]; v[j - 1] = tv;
                const int ti = vi[j]; vi[j] = vi[j - 1]; vi[j - 1] = ti;
            }
    float selw = 0.0f, tot = 0.0f;
    int seli = 0;
    for (int j = 0; j < k; ++j) {
        float bv = v[0];
        int bi = vi[0];
        wave_best(bv, bi, rt_better);
        if (lane == j) { selw = bv; seli = bi; }
        tot = tot + bv;
        if (vi[0] == bi) {
#pragma unroll
            for (int i = 0; i < V - 1; ++i) { v[i] = v[i + 1]; vi[i] = vi[i + 1]; }
            v[V - 1] = -1.0f; vi[V - 1] = 0x7fffffff;
        }
    }
    if (lane < k) { ids[(size_t) t * k + lane] = seli; wts[(size_t) t * k + lane] = selw / tot; }
    if (lane == 0 && sg) sg[t] = 1.0f / (1.0f + hy_expf(-l[ne]));
}

int launch_route(const float *logits, int ls, int ne, int k, int *ids, float *wts, float *sg, int nt, hipStream_t s) {
    if (nt == 0) return HY_OK;
    const int V = (ne + 63) / 64;
    dim3 g(nt);
    if (V <= 1) hipLaunchKernelGGL((k_route<1>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    else if (V <= 2) hipLaunchKernelGGL((k_route<2>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    else if (V <= 4) hipLaunchKernelGGL((k_route<4>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    else if (V <= 8) hipLaunchKernelGGL((k_route<8>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    else hipLaunchKernelGGL((k_route<16>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    return check_launch("hy_moe_route");
}

// ---------------------------------------------------------------- bucketing (A3)
// One block of 16 waves.  Pairs p with slot[ids[p]] >= 0, grouped by expert, stable by pair index
// (src/cpu_moe.cpp:672-687 order; the GPU reference src/kernels4.cu:1275-1295 is unordered within an
// expert).  Wave w owns a contiguous segment of pairs: (1) per-wave histograms, (2) prefix over experts
// and waves, egrp/order_n, (3) each wave walks its segment 64 pairs at a time: a lane finds the lanes that hold its
// expert from ten ballots (one per bit of the id, ids < 1024), its rank is the number of those below it, and the
// highest of them advances the wave's running counter for the expert.
constexpr int ORD_WAVES = 16;
__global__ __launch_bounds__(64 * ORD_WAVES) void k_order(const int *__restrict__ slot, const int *__restrict__ ids, int P, int ne,
                                                          int *__restrict__ order, int *__restrict__ order_n, int *__restrict__ egrp) {
    __shared__ int c[ORD_WAVES * 1024];
    __shared__ int tot[1024];
    __shared__ int wsum[2][ORD_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int seg = ((P + ORD_WAVES - 1) / ORD_WAVES + 63) / 64 * 64;
    const int p0 = w * seg, p1 = min(P, p0 + seg);
    for (int i = tid; i < ORD_WAVES * ne; i += blockDim.x) c[i] = 0;
    __syncthreads();
    for (int p = p0 + lane; p < p1; p += 64) {
        const int e = ids[p];
        if (e >= 0 && e < ne && slot[e] >= 0) atomicAdd(&c[w * ne + e], 1);
    }
    __syncthreads();
    // per expert e (thread e): the waves' counts become offsets within the expert; then exclusive scans over the
    // experts of the pair totals and of the active flags (ne <= 1024 = one entry per thread)
    {
        const int e = tid;
        int a = 0;
        if (e < ne)
            for (int ww = 0; ww < ORD_WAVES; ++ww) { const int v = c[ww * ne + e]; c[ww * ne + e] = a; a += v; }
        const int b = a > 0;
        int sa = a, sb = b;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int ta = __shfl_up(sa, o), tb = __shfl_up(sb, o);
            if (lane >= o) { sa += ta; sb += tb; }
        }
        if (lane == 63) { wsum[0][w] = sa; wsum[1][w] = sb; }
        __syncthreads();
        int oa = 0, ob = 0;
        for (int ww = 0; ww < w; ++ww) { oa += wsum[0][ww]; ob += wsum[1][ww]; }
        const int ea = oa + sa - a, eb = ob + sb - b;   // exclusive prefixes before e
        if (e < ne) {
            tot[e] = ea;
            if (b && egrp) { egrp[3 * eb] = e; egrp[3 * eb + 1] = ea; egrp[3 * eb + 2] = a; }
        }
        if (tid == blockDim.x - 1) {
            int ta = 0, tb = 0;
            for (int ww = 0; ww < ORD_WAVES; ++ww) { ta += wsum[0][ww]; tb += wsum[1][ww]; }
            order_n[0] = ta; order_n[1] = tb;
        }
    }
    __syncthreads();
    for (int i = tid; i < ORD_WAVES * ne; i += blockDim.x) c[i] += tot[i % ne];
    __syncthreads();
    int *cw = c + w * ne;
    const unsigned long long below = (1ull << lane) - 1;
    for (int q0 = p0; q0 < p1; q0 += 64) {
        const int p = q0 + lane;
        const int e = p < p1 ? ids[p] : -1;
        const bool valid = e >= 0 && e < ne && slot[e] >= 0;
        unsigned long long same = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 10; ++bit) {
            const unsigned long long ones = __ballot((e >> bit) & 1);
            same &= ((e >> bit) & 1) ? ones : ~ones;
        }
        if (valid) {
            const int rank = __popcll(same & below);
            const int base = cw[e];
            order[base + rank] = p;
            if (rank == __popcll(same) - 1) cw[e] = base + rank + 1;   // the group's highest lane
        }
        __builtin_amdgcn_wave_barrier();
    }
}

int launch_order(const int *slot, const int *ids, int P, int ne, int *order, int *order_n, int *egrp, hipStream_t s) {
    hipLaunchKernelGGL(k_order, dim3(1), dim3(64 * ORD_WAVES), 0, s, slot, ids, P, ne, order, order_n, egrp);
    return check_launch("hy_moe_order");
}

} // namespace hy
