// Router GEMV, softmax/top-k routing and token->expert bucketing.
#include "hy_internal.h"
#include "hy_routing.cuh"

namespace hy {

// ---------------------------------------------------------------- router logits (A1)
// y[t][r] = W[r] . x[t] (+ bias[t][r]): src/kernels4.cu:163-180 (gemv_f32), and with bf16 weights (WT = uint16_t,
// widened on load) src/kernels4.cu:181-197 (gemv_bf16w): the same products and sums.  Summation order of the contract:
// lane L of a wave accumulates elements 256 i + 4 L + j (j = 0..3) with fmaf in index order, then the
// 64 partial sums meet in an xor butterfly (1, 2, ..., 32).  A wave computes RW rows x TW tokens; its loads for
// step i + 1 are in flight while step i's fmas run (two register sets, a uniform trip count: past the row's end a
// lane re-reads its first element and skips the fmas).
template <int RW, int TW, typename WT>
__device__ __forceinline__ void gemv_tile(const WT *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                          float *__restrict__ y, int ys, int nt, const float *__restrict__ bias, int bs, int r0, int t0) {
    const int lane = threadIdx.x & 63;
    if (r0 >= rows) return;
    float acc[RW][TW];
#pragma unroll
    for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int b = 0; b < TW; ++b) acc[a][b] = 0.0f;
    const WT *wr[RW];
    const float *xr[TW];
#pragma unroll
    for (int a = 0; a < RW; ++a) wr[a] = W + (size_t) (r0 + a < rows ? r0 + a : r0) * kdim;
#pragma unroll
    for (int b = 0; b < TW; ++b) xr[b] = x + (size_t) (t0 + b < nt ? t0 + b : t0) * xs;
    const int niter = (kdim + 255) / 256;
    // the tile's biases, lane a TW + b holding (row r0 + a, token t0 + b): loaded now, added after the butterfly
    static_assert(RW * TW <= 64, "one bias per lane");
    float bv = 0.0f;
    if (bias && lane < RW * TW && r0 + lane / TW < rows && t0 + lane % TW < nt) bv = bias[(size_t) (t0 + lane % TW) * bs + r0 + lane / TW];
    float4 wa[RW], xa[TW], wb[RW], xb[TW];
    auto ld = [&](int i, float4 (&wd)[RW], float4 (&xd)[TW]) {
        const int e = 256 * i + 4 * lane < kdim ? 256 * i + 4 * lane : 4 * lane < kdim ? 4 * lane : 0;
#pragma unroll
        for (int a = 0; a < RW; ++a) wd[a] = ld_w4(wr[a] + e);
#pragma unroll
        for (int b = 0; b < TW; ++b) xd[b] = *(const float4 *) (xr[b] + e);
    };
    auto fma_step = [&](int i, const float4 (&wd)[RW], const float4 (&xd)[TW]) {
        if (i >= niter || 256 * i + 4 * lane >= kdim) return;
#pragma unroll
        for (int a = 0; a < RW; ++a)
#pragma unroll
            for (int b = 0; b < TW; ++b) {
                float s = acc[a][b];
                s = __builtin_fmaf(wd[a].x, xd[b].x, s);
                s = __builtin_fmaf(wd[a].y, xd[b].y, s);
                s = __builtin_fmaf(wd[a].z, xd[b].z, s);
                s = __builtin_fmaf(wd[a].w, xd[b].w, s);
                acc[a][b] = s;
            }
    };
    ld(0, wa, xa);
    for (int i = 0; i < niter; i += 2) {
        ld(i + 1, wb, xb);
        fma_step(i, wa, xa);
        ld(i + 2, wa, xa);
        fma_step(i + 1, wb, xb);
    }
#pragma unroll
    for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int b = 0; b < TW; ++b) {
            float s = wave_sum_xor(acc[a][b]);
            if (bias) s = s + readlane_f(bv, a * TW + b);
            if (lane == 0 && r0 + a < rows && t0 + b < nt) y[(size_t) (t0 + b) * ys + r0 + a] = s;
        }
}

// Block bid of a gx x gy grid of (row group, token group) tiles.  Workgroups go to the 8 XCDs round robin (bid % 8)
// and each XCD has its own L2, so when gy % 8 == 0 every token group's gx row groups run on one XCD: each XCD then
// streams 1/8 of the tokens (and all of W) instead of all of them.
__device__ __forceinline__ void gemv_tile_of(int bid, int gx, int gy, int &bx, int &by) {
    if (gy % 8 == 0) {
        const int slot = bid >> 3;
        bx = slot % gx;
        by = (bid & 7) + 8 * (slot / gx);
    } else {
        bx = bid % gx;
        by = bid / gx;
    }
}

template <int RW, int TW, typename WT>
__global__ __launch_bounds__(256) void k_gemv(const WT *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                              float *__restrict__ y, int ys, int nt, const float *__restrict__ bias, int bs, int gx,
                                              int gy) {
    int bx, by;
    gemv_tile_of(blockIdx.x, gx, gy, bx, by);
    gemv_tile<RW, TW>(W, rows, kdim, x, xs, y, ys, nt, bias, bs, (bx * 4 + (threadIdx.x >> 6)) * RW, by * TW);
}

template <typename WT>
static int gemv_any(const WT *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bs,
                    hipStream_t s, const char *what) {
    if (nt <= 4) {
        const int gx = (rows + 3) / 4, gy = nt;
        hipLaunchKernelGGL((k_gemv<1, 1, WT>), dim3(gx * gy), dim3(256), 0, s, W, rows, kdim, x, xs, y, ys, nt, bias, bs, gx, gy);
    } else {
        const int gx = (rows + 15) / 16, gy = (nt + 7) / 8;
        hipLaunchKernelGGL((k_gemv<4, 8, WT>), dim3(gx * gy), dim3(256), 0, s, W, rows, kdim, x, xs, y, ys, nt, bias, bs, gx, gy);
    }
    return check_launch(what);
}
int launch_gemv_f32(const float *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bs,
                    hipStream_t s) {
    return gemv_any(W, rows, kdim, x, xs, y, ys, nt, bias, bs, s, "hy_gemv_f32");
}
int launch_gemv_f32(const uint16_t *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bs,
                    hipStream_t s) {
    return gemv_any(W, rows, kdim, x, xs, y, ys, nt, bias, bs, s, "hy_gemv_bf16w");
}

// bf16 bit patterns -> fp32 (exact), four a thread: src/kernels4.cu:198-201 (bf16_to_f32)
__global__ __launch_bounds__(256) void k_bf16_to_f32(const uint16_t *__restrict__ W, size_t n, float *__restrict__ out) {
    const size_t i = 4 * ((size_t) blockIdx.x * 256 + threadIdx.x);
    if (i + 4 <= n) {
        *(float4 *) (out + i) = ld_w4(W + i);
    } else {
        for (size_t j = i; j < n; ++j) out[j] = __uint_as_float((uint32_t) W[j] << 16);
    }
}
int launch_bf16_to_f32(const uint16_t *W, size_t n, float *out, hipStream_t s) {
    if (n == 0) return HY_OK;
    const size_t blocks = (n + 1023) / 1024;
    hipLaunchKernelGGL(k_bf16_to_f32, dim3((unsigned) blocks), dim3(256), 0, s, W, n, out);
    return check_launch("hy_bf16_to_f32");
}

// The same contract for a block tile of 16 rows x 16 tokens (kdim a multiple of 256), 8 waves: each 256-value step
// of the 16 W rows and 16 x rows goes through LDS once (32 KB, one global read per block instead of one per wave),
// and wave w computes rows 4 (w % 4) .. + 3 of tokens 8 (w / 4) .. + 7 from it.  Lane L reads the float4 at 4 L of
// each row, so every lane's partial sums see the elements of gemv_tile in the same order.  The next step's 32 KB are
// loaded into registers while this step's fmas run.
constexpr int GL_R = 16, GL_THREADS = 512;
typedef float f4v __attribute__((ext_vector_type(4)));
// GT tokens a block (16, or 8 when 16-token tiles would leave CUs with fewer than two blocks); the waves are 4 row
// groups x 2 token groups whatever GT, and lane l always takes columns 4 l .. 4 l + 3 of each 256-column step
template <int GT, typename WT>
__device__ __forceinline__ void gemv_block_lds(const WT *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                               float *__restrict__ y, int ys, int nt, const float *__restrict__ bias, int bs, int r0,
                                               int t0, f4v *st) {   // st: LDS, (GL_R + GT) rows of 64 float4
    constexpr int RW = 4, TW = GT / 2, NS = (GL_R + GT) * 64 / GL_THREADS;   // float4 staged by each thread per step
    static_assert((GL_R + GT) * 64 % GL_THREADS == 0, "whole float4 per thread");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr0 = r0 + RW * (wave & 3), wt0 = t0 + TW * (wave >> 2);   // this wave's rows and tokens
    // the NS float4 this thread stages per step: tile row (tid + 512 k) / 64 (W rows, then x rows), column tid % 64;
    // the first NW are W rows
    constexpr int NW = GL_R * 64 / GL_THREADS;
    static_assert(NW * GL_THREADS == GL_R * 64 && NW < NS, "whole W rows per thread index");
    const WT *wsrc[NW];
    const float *xsrc[NS - NW];
#pragma clang loop unroll(full)
    for (int k = 0; k < NS; ++k) {
        const int row = (tid >> 6) + (GL_THREADS / 64) * k;
        if (k < NW) { const int r = r0 + row; wsrc[k] = W + (size_t) (r < rows ? r : rows - 1) * kdim + 4 * lane; }
        else { const int t = t0 + row - GL_R; xsrc[k - NW] = x + (size_t) (t < nt ? t : nt - 1) * xs + 4 * lane; }
    }
    auto ld = [&](int k, int e) -> f4v {
        if (k < NW) { const float4 v = ld_w4(wsrc[k] + e); return f4v{v.x, v.y, v.z, v.w}; }
        return *(const f4v *) (xsrc[k - NW] + e);
    };
    float acc[RW][TW];
#pragma unroll
    for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int b = 0; b < TW; ++b) acc[a][b] = 0.0f;
    f4v pre[NS];
#pragma clang loop unroll(full)
    for (int k = 0; k < NS; ++k) pre[k] = ld(k, 0);
    const int niter = kdim / 256;
    for (int i = 0; i < niter; ++i) {
        __syncthreads();   // the previous step's reads of st are done
#pragma clang loop unroll(full)
        for (int k = 0; k < NS; ++k) st[tid + GL_THREADS * k] = pre[k];
        __syncthreads();
        if (i + 1 < niter) {
#pragma clang loop unroll(full)
            for (int k = 0; k < NS; ++k) pre[k] = ld(k, 256 * (i + 1));
        }
        f4v xv[TW];
#pragma unroll
        for (int b = 0; b < TW; ++b) xv[b] = st[(GL_R + TW * (wave >> 2) + b) * 64 + lane];
#pragma unroll
        for (int a = 0; a < RW; ++a) {
            const f4v wv = st[(RW * (wave & 3) + a) * 64 + lane];
#pragma unroll
            for (int b = 0; b < TW; ++b) {
                float s = acc[a][b];
                s = __builtin_fmaf(wv.x, xv[b].x, s);
                s = __builtin_fmaf(wv.y, xv[b].y, s);
                s = __builtin_fmaf(wv.z, xv[b].z, s);
                s = __builtin_fmaf(wv.w, xv[b].w, s);
                acc[a][b] = s;
            }
        }
    }
    // The butterfly sums through LDS (the stage is free once every wave is past the last step's reads).  A pass
    // takes P outputs of the wave: each lane writes its P partial sums, then LPO = 64 / P lanes sum one output's 64
    // partials -- lane q of them the pairwise tree over partials q (64 / LPO) .. , the butterfly's subtree over those
    // lanes -- and combine their subtrees with DPP in the butterfly's order: the same tree, far fewer instructions
    // than a butterfly per output.
    constexpr int NOUT = RW * TW, P = GT == 16 ? 16 : 8, LPO = 64 / P, SUB = 64 / LPO;
    static_assert(NOUT % P == 0 && 8 * 64 * P * 4 <= (GL_R + GT) * 64 * 16, "the passes fit the stage");
    float *red = (float *) st + wave * 64 * P;
    __syncthreads();
    const int o = lane / LPO, q = lane % LPO;
#pragma unroll
    for (int p0 = 0; p0 < NOUT; p0 += P) {
#pragma unroll
        for (int u = 0; u < P; ++u) red[u * 64 + lane] = acc[(p0 + u) / TW][(p0 + u) % TW];
        wave_lds_sync();
        float v[SUB];
#pragma unroll
        for (int u = 0; u < SUB; u += 4) {
            const f4v w4 = *(const f4v *) (red + o * 64 + q * SUB + u);
            v[u] = w4.x; v[u + 1] = w4.y; v[u + 2] = w4.z; v[u + 3] = w4.w;
        }
#pragma unroll
        for (int h = 1; h < SUB; h <<= 1)   // pairwise tree, natural order
#pragma unroll
            for (int u = 0; u < SUB; u += 2 * h) v[u] = v[u] + v[u + h];
        float sum = v[0];
        sum = sum + dpp_f<DPP_XOR1>(sum);                         // lanes q, q ^ 1 (the next two levels up)
        sum = sum + dpp_f<DPP_XOR2>(sum);
        if constexpr (LPO == 8) sum = sum + dpp_f<DPP_HALF_MIRROR>(sum);   // quads 0-3 with 4-7
        const int idx = p0 + o, a = idx / TW, b = idx % TW;
        if (q == 0 && wr0 + a < rows && wt0 + b < nt) {
            if (bias) sum = sum + bias[(size_t) (wt0 + b) * bs + wr0 + a];
            y[(size_t) (wt0 + b) * ys + wr0 + a] = sum;
        }
        wave_lds_sync();   // this pass's reads are done before the next pass writes
    }
}

// Router logits of many tokens and the Q8 rows of x in one launch: blocks [0, gemv_blocks) compute the logits (gx
// blocks of 16 rows per GT tokens through gemv_block_lds when kdim % 256 == 0 (GT 8 or 16), else per 8 tokens
// through gemv_tile (GT 0)), the rest quantize x -- Q8_K: 32 blocks of 256 values per block, 16 lanes each; Q8_0: 8
// pairs of 32-value blocks per block, a wave each.  The LDS variants fit two blocks a CU.
template <int VT, int GT, typename WT>
__global__ __launch_bounds__(GL_THREADS, GT ? 4 : 2) void k_router_pre(const WT *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                                    const float *__restrict__ bias, int bs, float *__restrict__ y, int ys, int nt,
                                                    uint8_t *__restrict__ xq, int gx, int gemv_blocks) {
    __shared__ f4v st[GT ? (GL_R + GT) * 64 : 1];
    const int bid = blockIdx.x;
    if (bid < gemv_blocks) {
        int bx, by;
        gemv_tile_of(bid, gx, gemv_blocks / gx, bx, by);
        if constexpr (GT != 0) gemv_block_lds<GT>(W, rows, kdim, x, xs, y, ys, nt, bias, bs, bx * GL_R, by * GT, st);
        else if (threadIdx.x < 256) gemv_tile<4, 8>(W, rows, kdim, x, xs, y, ys, nt, bias, bs, (bx * 4 + (threadIdx.x >> 6)) * 4, by * 8);
        return;
    }
    const int qb = bid - gemv_blocks;
    if constexpr (VT == Q8_K) {
        const int nb = kdim / 256, u = qb * (GL_THREADS / 16) + (threadIdx.x >> 4);
        if (u >= nt * nb) return;   // uniform over the 16-lane row
        const int t = u / nb, b = u - t * nb;
        q8k_block16_load(x + (size_t) t * xs + 256 * b, xq + ((size_t) t * nb + b) * Q8K_BYTES);
    } else {
        const int nb = kdim / 32, npair = (nb + 1) / 2, u = qb * (GL_THREADS / 64) + (threadIdx.x >> 6);
        if (u >= nt * npair) return;   // wave-uniform
        const int t = u / npair, b = 2 * (u - t * npair);
        q8_0_pair_wave(x + (size_t) t * xs + 32 * b, xq + ((size_t) t * nb + b) * Q8_0_BYTES, b + 1 < nb, Q8_0_BYTES, 2);
    }
}

// Router logits of many tokens with the weight rows held in registers (kdim = 256 NI, NI 4 or 8): a block of 8 waves
// owns 32 rows (wave w: rows 4 w .. 4 w + 3, each lane its float4 at 256 i + 4 L of every row, loaded once) and a range
// of tokens, which reach LDS 8 at a time by DMA (two buffers: chunk c + 1 lands while chunk c's fmas run; wave w
// fetches token w of a chunk).  Every x value read from LDS feeds 4 rows x 4 fmas, half the LDS bytes per fma of the
// tile kernel above, and the weights are read from memory once per block.  The lane partial sums of each chunk meet in
// the same tree as gemv_block_lds (the butterfly's bits).  The Q8 rows of x come from the staged chunk too: every
// row-group block of a range stages the same chunks, and block bx quantizes the chunk's units u with u % gx == bx.
constexpr int RR_ROWS = 4, RR_WAVES = 8, RR_THREADS = 64 * RR_WAVES, RR_TC = 8;
template <int VT, int NI, typename WT>
__global__ __launch_bounds__(RR_THREADS, 2) void k_router_rows(const WT *__restrict__ W, int rows, const float *__restrict__ x, int xs,
                                                             const float *__restrict__ bias, int bs, float *__restrict__ y, int ys, int nt,
                                                             uint8_t *__restrict__ xq, int gx, int tpr) {
    static_assert(RR_TC == RR_WAVES, "a wave fetches one token row of a chunk");
    constexpr int kdim = 256 * NI, ROWF4 = 64 * NI;   // float4 per token row
    __shared__ f4v st[2][RR_TC * ROWF4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // block b runs on XCD b % 8 (each XCD with its own L2): with whole token ranges on one XCD (the grid a multiple of
    // 8 blocks), a range's x rows come into one L2 and serve its gx row-group blocks there
    const int nb = (int) gridDim.x, l = nb % 8 == 0 ? (int) (blockIdx.x % 8) * (nb / 8) + (int) (blockIdx.x / 8) : (int) blockIdx.x;
    const int bx = l % gx, by = l / gx;
    const int t_beg = by * tpr, t_end = min(nt, t_beg + tpr);
    const int r0 = bx * RR_ROWS * RR_WAVES + RR_ROWS * wave;
    const bool wave_on = r0 < rows;   // wave-uniform: waves past the last row stage, quantize and synchronize only
    const int nchunk = t_end > t_beg ? (t_end - t_beg + RR_TC - 1) / RR_TC : 0;
    if (nchunk == 0) return;   // uniform over the block
    // chunk c into buffer buf: wave w's NI DMAs of 1 KB bring token c0 + w (past the range's end: its last token again,
    // whose outputs are never stored), so that every wave issues NI per chunk
    auto dma_chunk = [&](int c, int buf) {
        const int t = min(t_beg + RR_TC * c + wave, t_end - 1);
        const float *src = x + (size_t) t * xs;
#pragma unroll
        for (int i = 0; i < NI; ++i) dma_s128(src + 256 * i, 16u * (uint32_t) lane, lds_addr(&st[buf][wave * ROWF4 + 64 * i]));
    };
    dma_chunk(0, 0);
    // the weights in K order (the first half of every row, then the second): chunk 0's fmas over the first half run
    // while the second half is still on its way
    f4v w[RR_ROWS][NI];
    const WT *wr[RR_ROWS];
#pragma unroll
    for (int a = 0; a < RR_ROWS; ++a) wr[a] = W + (size_t) min(r0 + a, rows - 1) * kdim + 4 * lane;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int a = 0; a < RR_ROWS; ++a) { const float4 v = ld_w4(wr[a] + 256 * i); w[a][i] = f4v{v.x, v.y, v.z, v.w}; }
    float acc[RR_ROWS][RR_TC];
    // the fmas of K half h (i in [h NI / 2, (h + 1) NI / 2)) of a chunk staged in buffer buf: each (row, token) chain
    // runs over i in order, so the halves in turn give the same bits as one pass
    auto fma_half = [&](int buf, int h) {
        if (!wave_on) return;
#pragma unroll
        for (int ii = 0; ii < NI / 2; ++ii) {
            const int i = h * (NI / 2) + ii;
#pragma unroll
            for (int u = 0; u < RR_TC; ++u) {
                const f4v xv = st[buf][u * ROWF4 + 64 * i + lane];
#pragma unroll
                for (int a = 0; a < RR_ROWS; ++a) {
                    float s = acc[a][u];
                    s = __builtin_fmaf(w[a][i].x, xv.x, s);
                    s = __builtin_fmaf(w[a][i].y, xv.y, s);
                    s = __builtin_fmaf(w[a][i].z, xv.z, s);
                    s = __builtin_fmaf(w[a][i].w, xv.w, s);
                    acc[a][u] = s;
                }
            }
        }
    };
    // chunk 0 and the first half of the weights landed (a wave's loads complete in issue order), by waits the compiler
    // sees: it places no wait for the weight registers itself (inside the chunk loop one would also wait for the next
    // chunk's DMAs)
    constexpr int VM_HALF = RR_ROWS * NI / 2;
    __builtin_amdgcn_s_waitcnt((VM_HALF & 15) | ((VM_HALF >> 4) << 14) | 0x0F70);   // vmcnt(VM_HALF), expcnt and lgkmcnt at their maxima
    lds_barrier();   // every wave's DMAs of chunk 0
#pragma unroll
    for (int a = 0; a < RR_ROWS; ++a)
#pragma unroll
        for (int u = 0; u < RR_TC; ++u) acc[a][u] = 0.0f;
    fma_half(0, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the second half
    if (nchunk > 1) dma_chunk(1, 1);
    constexpr int NOUT = RR_ROWS * RR_TC, P = 16, LPO = 64 / P, SUB = 64 / LPO;   // the tree of gemv_block_lds, 16 outputs a pass
    static_assert(NOUT % P == 0 && RR_WAVES * 64 * P <= RR_TC * ROWF4 * 4, "the passes fit a chunk buffer");
    static_assert(NI % 2 == 0 && VM_HALF < 64, "two halves; vmcnt holds 6 bits");
    for (int c = 0; c < nchunk; ++c) {
        const int buf = c & 1, c0 = t_beg + RR_TC * c, ntok = min(RR_TC, t_end - c0);
        if (c > 0) {
            if (c + 1 < nchunk) wait_vm<NI>(); else wait_vm<0>();   // this wave's DMAs of chunk c have landed
            lds_barrier();                                           // and every wave's
        }
        // the chunk's Q8 rows (from LDS): Q8_K a 256-value block per 16-lane row, Q8_0 a pair of 32-value blocks a wave
        if constexpr (VT == Q8_K) {
            const int units = ntok * NI;
            for (int u = bx + gx * (tid >> 4); u < units; u += gx * (RR_THREADS / 16)) {   // uniform over the 16-lane row
                const int tk = u / NI, b = u - tk * NI;
                const f4v *src = &st[buf][tk * ROWF4 + 64 * b + 4 * (lane & 15)];
                float xv[16];
#pragma unroll
                for (int j = 0; j < 4; ++j) { const f4v v = src[j]; xv[4 * j] = v.x; xv[4 * j + 1] = v.y; xv[4 * j + 2] = v.z; xv[4 * j + 3] = v.w; }
                q8k_block16(xv, xq + ((size_t) (c0 + tk) * NI + b) * Q8K_BYTES);
            }
        } else {
            constexpr int NP = 4 * NI;   // pairs of Q8_0 blocks a token row
            const int units = ntok * NP;
            for (int u = bx + gx * wave; u < units; u += gx * RR_WAVES) {   // wave-uniform
                const int tk = u / NP, pb = u - tk * NP;
                const float v = ((const float *) &st[buf][tk * ROWF4])[64 * pb + lane];
                q8_0_pair_vals(v, xq + ((size_t) (c0 + tk) * (8 * NI) + 2 * pb) * Q8_0_BYTES, true, Q8_0_BYTES, 2);
            }
        }
        if (c > 0) {
#pragma unroll
            for (int a = 0; a < RR_ROWS; ++a)
#pragma unroll
                for (int u = 0; u < RR_TC; ++u) acc[a][u] = 0.0f;
            fma_half(buf, 0);
        }
        fma_half(buf, 1);
        lds_barrier();   // every wave is past its reads of this chunk: its buffer is the reduction's scratch now
        if (wave_on) {
            float *red = (float *) st[buf] + wave * 64 * P;
            const int o = lane / LPO, q = lane % LPO;
#pragma unroll
            for (int p0 = 0; p0 < NOUT; p0 += P) {
#pragma unroll
                for (int u = 0; u < P; ++u) red[u * 64 + lane] = acc[(p0 + u) / RR_TC][(p0 + u) % RR_TC];
                wave_lds_sync();
                float v[SUB];
#pragma unroll
                for (int u = 0; u < SUB; u += 4) {
                    const f4v w4 = *(const f4v *) (red + o * 64 + q * SUB + u);
                    v[u] = w4.x; v[u + 1] = w4.y; v[u + 2] = w4.z; v[u + 3] = w4.w;
                }
#pragma unroll
                for (int h = 1; h < SUB; h <<= 1)   // pairwise tree, natural order
#pragma unroll
                    for (int u = 0; u < SUB; u += 2 * h) v[u] = v[u] + v[u + h];
                float sum = v[0];
                sum = sum + dpp_f<DPP_XOR1>(sum);
                sum = sum + dpp_f<DPP_XOR2>(sum);
                const int idx = p0 + o, a = idx / RR_TC, u = idx % RR_TC, r = r0 + a, t = c0 + u;
                if (q == 0 && r < rows && u < ntok) {
                    if (bias) sum = sum + bias[(size_t) t * bs + r];
                    y[(size_t) t * ys + r] = sum;
                }
                wave_lds_sync();   // this pass's reads are done before the next pass writes
            }
        }
        if (c + 2 < nchunk) {
            lds_barrier();        // every wave's scratch reads are done: the buffer takes chunk c + 2
            dma_chunk(c + 2, buf);
        }
    }
}

// Router logits of many tokens on the fp32 matrix cores (v_mfma_f32_16x16x4_f32), and the Q8 rows of x, in one
// launch.  Blocks [0, gemm_blocks) take a 64-row x 64-token tile of the first 64 gm rows: K in chunks of RT_KC, staged
// through LDS in two buffers (rows padded to RT_LD floats, which spreads the operand reads over the banks) with the
// global loads of the next four chunks in registers; each wave multiplies a 32-row x 16 TJ-token part of the tile
// (2 x TJ MFMA tiles, each 16-value step {4 q + s} of lane quarter q, component s).  Blocks [gemm_blocks, +
// tail_blocks) take the rows past the full tiles, a wave per (row, token) logit; the rest quantize x as k_router_pre.
// The sums run in the matrix cores' order, not gemv_f32's fmaf chain: the logits agree with it to fp32 rounding, and
// the routing is defined on the logits it is given.
constexpr int RT_M = 64, RT_N = 64, RT_KC = 64, RT_LD = RT_KC + 8, RT_NW = 8;
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The parts of a matrix-core router launch (NW waves a block) beside its logit tiles.  Q8 block qb of x: Q8_K a
// 256-value block per 16-lane row, Q8_0 a pair of blocks per wave (as k_router_pre).
template <int VT, int NW>
__device__ __forceinline__ void router_q8_part(const float *__restrict__ x, int xs, int kdim, int nt, uint8_t *__restrict__ xq, int qb) {
    const int tid = threadIdx.x, wave = tid >> 6;
    if constexpr (VT == Q8_K) {
        const int nb = kdim / 256, u = qb * (64 * NW / 16) + (tid >> 4);
        if (u >= nt * nb) return;   // uniform over the 16-lane row
        const int t = u / nb, b = u - t * nb;
        q8k_block16_load(x + (size_t) t * xs + 256 * b, xq + ((size_t) t * nb + b) * Q8K_BYTES);
    } else {
        const int nb = kdim / 32, npair = (nb + 1) / 2, u = qb * NW + wave;
        if (u >= nt * npair) return;   // wave-uniform
        const int t = u / npair, b = 2 * (u - t * npair);
        q8_0_pair_wave(x + (size_t) t * xs + 32 * b, xq + ((size_t) t * nb + b) * Q8_0_BYTES, b + 1 < nb, Q8_0_BYTES, 2);
    }
}
// Rows r_first .. rows - 1 (past the full tiles): a wave per (row, token) logit u, lane L summing values 4 L + 256 i ..
template <typename WT>
__device__ __forceinline__ void router_tail_part(const WT *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                                 const float *__restrict__ bias, int bs, float *__restrict__ y, int ys, int nt, int r_first, int u) {
    const int lane = threadIdx.x & 63, rt = rows - r_first;
    if (u >= rt * nt) return;   // wave-uniform
    const int r = r_first + u % rt, t = u / rt;
    const WT *wr = W + (size_t) r * kdim;
    const float *xt = x + (size_t) t * xs;
    float acc = 0.0f;
    for (int e = 4 * lane; e < kdim; e += 256) {
        const float4 w = ld_w4(wr + e), v = *(const float4 *) (xt + e);
        acc = __builtin_fmaf(w.x, v.x, acc); acc = __builtin_fmaf(w.y, v.y, acc);
        acc = __builtin_fmaf(w.z, v.z, acc); acc = __builtin_fmaf(w.w, v.w, acc);
    }
    float sum = wave_sum_xor(acc);
    if (bias) sum = sum + bias[(size_t) t * bs + r];
    if (lane == 0) y[(size_t) t * ys + r] = sum;
}

template <int VT, typename WT, int NW>
__global__ __launch_bounds__(64 * NW) void k_router_tile(const WT *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                                      const float *__restrict__ bias, int bs, float *__restrict__ y, int ys, int nt,
                                                      uint8_t *__restrict__ xq, int gm, int gemm_blocks, int tail_blocks) {
    constexpr int TH = 64 * NW, NL = RT_M * RT_KC / 4 / TH;   // threads; float4 of A (and of B) each thread moves a chunk
    constexpr int TJ = NW == 4 ? 2 : 1;                         // 16-token MFMA tiles a wave (2 x TJ tiles)
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr int CPR = RT_KC / 4, RS = TH / CPR;   // float4 a row and chunk; rows apart of a thread's float4
    static_assert(RT_KC % 16 == 0 && TH % CPR == 0 && RS * NL == RT_M, "whole rows a pass");
    __shared__ __align__(16) float As[2][RT_M * RT_LD], Bs[2][RT_N * RT_LD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int bid = blockIdx.x;
    if (bid >= gemm_blocks + tail_blocks) {   // the Q8 rows of x
        router_q8_part<VT, NW>(x, xs, kdim, nt, xq, bid - gemm_blocks - tail_blocks);
        return;
    }
    if (bid >= gemm_blocks) {   // rows past the full tiles
        router_tail_part<WT>(W, rows, kdim, x, xs, bias, bs, y, ys, nt, RT_M * gm, (bid - gemm_blocks) * NW + wave);
        return;
    }
    // consecutive blocks take consecutive token tiles (blocks go to the 8 XCDs in turn, each with its own L2): an XCD
    // keeps a few token tiles of x for every row tile, fetching x once, where the other order fetched it once per XCD
    const int gn = gemm_blocks / gm, r0 = (bid / gn) * RT_M, t0 = (bid % gn) * RT_N;
    const int wm = wave & 1, wn = wave >> 1, li = lane & 15, lq = lane >> 4;   // wave: rows 32 wm .., tokens 16 TJ wn ..
    // global -> LDS: thread tid moves float4 tid % CPR of rows tid / CPR + RS h, h < NL, of the A and B chunks
    const int lr = tid / CPR, lc = 4 * (tid % CPR);
    const WT *ga[NL];
    const float *gb[NL];
#pragma unroll
    for (int h = 0; h < NL; ++h) {
        ga[h] = W + (size_t) (r0 + lr + RS * h) * kdim + lc;
        gb[h] = x + (size_t) min(t0 + lr + RS * h, nt - 1) * xs + lc;
    }
    const int nst = kdim / RT_KC;
    // the ring of four chunks on their way, in named slots of up to two float4 of A and of B (named variables: they
    // stay in registers)
    static_assert(NL == 1 || NL == 2, "one or two float4 of each operand a thread");
    float4 sa0, sb0, ta0, tb0, sa1, sb1, ta1, tb1, sa2, sb2, ta2, tb2, sa3, sb3, ta3, tb3;
#define HY_RT_LOAD(c, SA, SB, TA, TB)                                                              \
    {                                                                                            \
        SA = ld_w4(ga[0] + RT_KC * (c)); SB = *(const float4 *) (gb[0] + RT_KC * (c));           \
        if constexpr (NL == 2) { TA = ld_w4(ga[NL - 1] + RT_KC * (c)); TB = *(const float4 *) (gb[NL - 1] + RT_KC * (c)); } \
    }
#define HY_RT_STORE(buf, SA, SB, TA, TB)                                                           \
    {                                                                                            \
        *(float4 *) &As[buf][lr * RT_LD + lc] = SA; *(float4 *) &Bs[buf][lr * RT_LD + lc] = SB;  \
        if constexpr (NL == 2) {                                                                 \
            *(float4 *) &As[buf][(lr + RS) * RT_LD + lc] = TA; *(float4 *) &Bs[buf][(lr + RS) * RT_LD + lc] = TB; \
        }                                                                                        \
    }
    f32x4 acc[2][TJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf) {
        const float *as = As[buf] + (32 * wm + li) * RT_LD + 4 * lq, *bsm = Bs[buf] + (16 * TJ * wn + li) * RT_LD + 4 * lq;
#pragma unroll
        for (int kk = 0; kk < RT_KC / 16; ++kk) {
            f32x4 a[2], b[TJ];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = *(const f32x4 *) (as + 16 * i * RT_LD + 16 * kk);
#pragma unroll
            for (int j = 0; j < TJ; ++j) b[j] = *(const f32x4 *) (bsm + 16 * j * RT_LD + 16 * kk);
#pragma unroll
            for (int sc = 0; sc < 4; ++sc)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][sc], b[j][sc], acc[i][j], 0, 0, 0);
        }
    };
    // chunk c sits in slot c % 4; step c computes it from buffer c & 1, stores chunk c + 1 (slot (c + 1) % 4) into the
    // other buffer (last read in step c - 1), then loads chunk c + 5 into that slot.  Steps -4 .. -1 only load (chunks
    // 1 .. 4) and store chunk 0, so every load of the ring is issued by the loop, in one order; the loop runs whole
    // rounds of four steps and leaves only at its end; and every step issues its loads (past the last chunk, the last
    // chunk again, never stored).  So the compiler counts 16 loads in flight at every store and waits for the oldest
    // chunk only: loads under a condition, a loop left from the middle of a round, or the first chunks' loads issued
    // before the loop (in an order of the compiler's choosing) made it wait for all of them.  (Three chunks ahead:
    // 53.7 us on the 2048-token, 513-row router; four: 50.9; five and six lose occupancy and take 53-55.)
    const int last = nst - 1;
    HY_RT_LOAD(0, sa0, sb0, ta0, tb0);
#define HY_RT_STEP(C, SA, SB, TA, TB)                                                              \
    {                                                                                            \
        if ((C) >= 0 && (C) < nst) compute((C) & 1);                                             \
        if ((C) + 1 >= 0 && (C) + 1 < nst) HY_RT_STORE(((C) + 1) & 1, SA, SB, TA, TB);           \
        HY_RT_LOAD(min((C) + 5, last), SA, SB, TA, TB);                                          \
        __syncthreads();                                                                         \
    }
    for (int c = -4; c < nst; c += 4) {   // uniform trip count; chunk c + 1 lies in slot (c + 1) % 4
        HY_RT_STEP(c + 0, sa1, sb1, ta1, tb1)
        HY_RT_STEP(c + 1, sa2, sb2, ta2, tb2)
        HY_RT_STEP(c + 2, sa3, sb3, ta3, tb3)
        HY_RT_STEP(c + 3, sa0, sb0, ta0, tb0)
    }
#undef HY_RT_STEP
#undef HY_RT_LOAD
#undef HY_RT_STORE
    // lane holds D[4 lq + v][li] of each 16 x 16 tile: weight row r0 + 32 wm + 16 i + 4 lq + v, token t0 + 16 (TJ wn + j) + li
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int t = t0 + 16 * (TJ * wn + j) + li;
        if (t >= nt) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = r0 + 32 * wm + 16 * i + 4 * lq + v;
                float sum = acc[i][j][v];
                if (bias) sum = sum + bias[(size_t) t * bs + r];
                y[(size_t) t * ys + r] = sum;
            }
    }
}

template <typename WT>
static int router_tile_any(const WT *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                           int vtype, void *xq, int nt, hipStream_t s) {
    constexpr int NW = RT_NW;
    const int gm = rows / RT_M, gn = (nt + RT_N - 1) / RT_N, gemm_blocks = gm * gn;
    const int tail_blocks = ((rows - RT_M * gm) * nt + NW - 1) / NW;
    const int qblocks = vtype == Q8_K ? (nt * (kdim / 256) + 4 * NW - 1) / (4 * NW) : (nt * ((kdim / 32 + 1) / 2) + NW - 1) / NW;
#define HY_RT(VV) hipLaunchKernelGGL((k_router_tile<VV, WT, NW>), dim3(gemm_blocks + tail_blocks + qblocks), dim3(64 * NW), 0, s, W, rows, kdim, \
                                     x, xs, bias, bs, logits, ls, nt, (uint8_t *) xq, gm, gemm_blocks, tail_blocks)
    if (vtype == Q8_K) HY_RT(Q8_K); else HY_RT(Q8_0);
#undef HY_RT
    return check_launch("hy_moe_router_q8");
}

template <typename WT>
static int router_pre_any(const WT *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                          int vtype, void *xq, int nt, hipStream_t s) {
    if (nt == 0) return HY_OK;
    // the matrix cores when the full 64 x 64 tiles alone fill every CU (their grid: at least 256 blocks)
    if (kdim % RT_KC == 0 && (xs & 3) == 0 && ((uintptr_t) x & 15) == 0 && (long) (rows / RT_M) * ((nt + RT_N - 1) / RT_N) >= 256)
        return router_tile_any(W, rows, kdim, x, xs, bias, bs, logits, ls, vtype, xq, nt, s);
    {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        const int gx = (rows + RR_ROWS * RR_WAVES - 1) / (RR_ROWS * RR_WAVES);
        if ((kdim == 1024 || kdim == 2048) && gx * ((nt + RR_TC - 1) / RR_TC) >= cus && (xs & 3) == 0 && ((uintptr_t) x & 15) == 0) {
            // one block a CU: the token ranges (whole chunks) that give gx x gy <= cus blocks
            const int gy0 = std::max(1, cus / gx);
            const int tpr = (nt + gy0 * RR_TC - 1) / (gy0 * RR_TC) * RR_TC, gy = (nt + tpr - 1) / tpr;
#define HY_RR(VV, NN) hipLaunchKernelGGL((k_router_rows<VV, NN, WT>), dim3(gx * gy), dim3(RR_THREADS), 0, s, W, rows, x, xs, bias, bs, logits, ls, nt, \
                                         (uint8_t *) xq, gx, tpr)
            if (vtype == Q8_K) { if (kdim == 2048) HY_RR(Q8_K, 8); else HY_RR(Q8_K, 4); }
            else { if (kdim == 2048) HY_RR(Q8_0, 8); else HY_RR(Q8_0, 4); }
#undef HY_RR
            return check_launch("hy_moe_router_q8");
        }
    }
    // kdim % 256 == 0: 16 x GT tiles through LDS (gemv_block_lds), GT = 16, or 8 when 16-token tiles number fewer
    // than two per CU (more blocks to hide the steps' barriers); else 16 rows x 8 tokens a block (gemv_tile, GT 0)
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    const int gx = (rows + 15) / 16;
    const int gt = kdim % 256 != 0 ? 0 : gx * ((nt + 15) / 16) < 2 * cus ? 8 : 16;
    const int gemv_blocks = gx * ((nt + (gt ? gt : 8) - 1) / (gt ? gt : 8));
#define HY_RP(VV, GG) hipLaunchKernelGGL((k_router_pre<VV, GG, WT>), dim3(gemv_blocks + qblocks), dim3(GL_THREADS), 0, s, W, rows, kdim, x, xs, bias, bs, \
                                         logits, ls, nt, (uint8_t *) xq, gx, gemv_blocks)
    if (vtype == Q8_K) {
        const int qblocks = (nt * (kdim / 256) + GL_THREADS / 16 - 1) / (GL_THREADS / 16);
        if (gt == 8) HY_RP(Q8_K, 8); else if (gt == 16) HY_RP(Q8_K, 16); else HY_RP(Q8_K, 0);
    } else {
        const int qblocks = (nt * ((kdim / 32 + 1) / 2) + GL_THREADS / 64 - 1) / (GL_THREADS / 64);
        if (gt == 8) HY_RP(Q8_0, 8); else if (gt == 16) HY_RP(Q8_0, 16); else HY_RP(Q8_0, 0);
    }
#undef HY_RP
    return check_launch("hy_moe_router_q8");
}
int launch_router_pre(const float *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                      int vtype, void *xq, int nt, hipStream_t s) {
    return router_pre_any(W, rows, kdim, x, xs, bias, bs, logits, ls, vtype, xq, nt, s);
}
int launch_router_pre(const uint16_t *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                      int vtype, void *xq, int nt, hipStream_t s) {
    return router_pre_any(W, rows, kdim, x, xs, bias, bs, logits, ls, vtype, xq, nt, s);
}

// ---------------------------------------------------------------- routing (A2)
// A token per block: up to 128 experts by eight waves (route_rank8), more by one wave (route_wave: wave_topk);
// both give the bits of src/kernels4.cu:297-344's contract (hy_routing.cuh).
template <int V>
__global__ __launch_bounds__(512) void k_route8(const float *__restrict__ logits, int ls, int ne, int k, int *__restrict__ ids,
                                                float *__restrict__ wts, float *__restrict__ sg) {
    const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int er;
    float pr, tot, lsg;
    route_rank8<V>(logits + (size_t) t * ls, ne, k, sg != nullptr, er, pr, tot, lsg, [] {});
    if (wave == 0) {
        if (lane < k) { ids[(size_t) t * k + lane] = er; wts[(size_t) t * k + lane] = pr / tot; }
        if (lane == 0 && sg) sg[t] = 1.0f / (1.0f + hy_expf(-lsg));
    }
}
template <int V>
__global__ __launch_bounds__(64) void k_route(const float *__restrict__ logits, int ls, int ne, int k, int *__restrict__ ids,
                                              float *__restrict__ wts, float *__restrict__ sg) {
    const int t = blockIdx.x;
    route_wave<V>(logits + (size_t) t * ls, ne, k, ids + (size_t) t * k, wts + (size_t) t * k, sg ? sg + t : nullptr);
}

int launch_route(const float *logits, int ls, int ne, int k, int *ids, float *wts, float *sg, int nt, hipStream_t s) {
    if (nt == 0) return HY_OK;
    const int V = (ne + 63) / 64;
    dim3 g(nt);
    if (V <= 1) hipLaunchKernelGGL((k_route8<1>), g, dim3(512), 0, s, logits, ls, ne, k, ids, wts, sg);
    else if (V <= 2) hipLaunchKernelGGL((k_route8<2>), g, dim3(512), 0, s, logits, ls, ne, k, ids, wts, sg);
    else if (V <= 4) hipLaunchKernelGGL((k_route<4>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    else if (V <= 8) hipLaunchKernelGGL((k_route<8>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    else hipLaunchKernelGGL((k_route<16>), g, dim3(64), 0, s, logits, ls, ne, k, ids, wts, sg);
    return check_launch("hy_moe_route");
}

// Routers with a selection bias (one wave per token): score s_e from the logit -- MODE 0: sigmoid, the contract of
// k_moe_route_sig (src/kernels5.cu:1090-1122); MODE 1: sqrt(softplus), the contract of k_route7 (src/kernels7.cu:
// 816-865) -- then the top k of s_e + bias[e] (ties to the lower index) by wave_topk, the scores riding along; the
// weights use the scores alone, summed in selection order: MODE 0: s scale / max(sum, 2^-14) (and sg = 1);
// MODE 1: s / (sum + 1e-20) scale.
template <int V, int MODE>
__global__ __launch_bounds__(64) void k_route_bias(const float *__restrict__ logits, int ls, const float *__restrict__ bias, int ne, int k,
                                                   float scale, int *__restrict__ ids, float *__restrict__ wts, float *__restrict__ sg) {
    const int t = blockIdx.x, lane = threadIdx.x;
    const float *l = logits + (size_t) t * ls;
    float key[V], score[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int e = lane + 64 * i;
        score[i] = 0.0f;
        key[i] = 0.0f;
        if (e < ne) {
            const float x = l[e];
            score[i] = MODE == 0 ? hy_sigmoid(x) : hy_sqrt_softplus(x);
            key[i] = score[i] + bias[e];
        }
    }
    int e_r;
    float s_r;
    wave_topk<V>(key, score, ne, k, e_r, s_r);
    float tot = 0.0f;
    for (int r = 0; r < k; ++r) tot = tot + readlane_f(s_r, r);
    if (lane < k) {
        ids[(size_t) t * k + lane] = e_r;
        wts[(size_t) t * k + lane] = MODE == 0 ? s_r * (scale / fmaxf(tot, 6.103515625e-5f)) : s_r / (tot + 1e-20f) * scale;
    }
    if (MODE == 0 && sg && lane == 0) sg[t] = 1.0f;
}

int launch_route_bias(int mode, const float *logits, int ls, const float *bias, int ne, int k, float scale, int *ids, float *wts,
                      float *sg, int nt, hipStream_t s) {
    if (nt == 0) return HY_OK;
    const int V = (ne + 63) / 64;
#define HY_RB(VV) { if (mode == 0) hipLaunchKernelGGL((k_route_bias<VV, 0>), dim3(nt), dim3(64), 0, s, logits, ls, bias, ne, k, scale, ids, wts, sg); \
                    else hipLaunchKernelGGL((k_route_bias<VV, 1>), dim3(nt), dim3(64), 0, s, logits, ls, bias, ne, k, scale, ids, wts, sg); }
    if (V <= 1) HY_RB(1) else if (V <= 2) HY_RB(2) else if (V <= 4) HY_RB(4) else if (V <= 8) HY_RB(8) else HY_RB(16)
#undef HY_RB
    return check_launch(mode == 0 ? "hy_moe_route_sig" : "hy_moe_route_sqrtsp");
}

// ---------------------------------------------------------------- bucketing (A3)
// Pairs p with slot[ids[p]] >= 0, grouped by expert, stable by pair index (src/cpu_moe.cpp:672-687 order; the GPU
// reference src/kernels4.cu:1275-1295 is unordered within an expert).  Block i places pairs [1024 i, 1024 i + 1024),
// a 64-pair row a wave, with no word from the other blocks: (1) every block counts all pairs per expert (tot, the
// experts' starts) and those before its range (pre) -- the ids are re-read from L2 by each block, 4 P bytes --, and
// its rows per expert; (2) per expert e (thread e): the exclusive scan of the totals over the experts gives e's start,
// and start + pre[e] + the block's earlier rows the offset of each row's first e; block 0 writes egrp and order_n;
// (3) a lane's rank among its row's lanes of the same expert comes from log2(ne) ballots (one per bit of the id).
constexpr int ORD_T = 1024, ORD_W = ORD_T / 64;   // pairs (threads) a block; rows (waves) a block
constexpr int ORD_B = 8;                          // ids a thread loads together in the counting pass
__global__ __launch_bounds__(ORD_T) void k_order(const int *__restrict__ slot, int n_local, const int *__restrict__ ids, int P, int ne, int nbits,
                                                 int *__restrict__ order, int *__restrict__ order_n, int *__restrict__ egrp) {
    __shared__ int c[ORD_W * 1024];   // the rows' counts per expert, then the offset of each row's first pair of e
    __shared__ int tot[1024], pre[1024], s_slot[1024];
    __shared__ int wsum[2][ORD_W];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int b0 = blockIdx.x * ORD_T, p = b0 + tid;
    const int my_e = p < P ? ids[p] : -1;
    const int sl = tid < ne ? bound_slot(slot[tid], n_local) : -1;
    for (int i = tid; i < ORD_W * ne; i += ORD_T) c[i] = 0;
    if (tid < ne) { s_slot[tid] = sl; tot[tid] = 0; pre[tid] = 0; }
    __syncthreads();
    auto valid_e = [&](int e) { return e >= 0 && e < ne && s_slot[e] >= 0; };
    for (int q0 = 0; q0 < P; q0 += ORD_T * ORD_B) {
        int idv[ORD_B];
#pragma unroll
        for (int r = 0; r < ORD_B; ++r) {
            const int q = q0 + ORD_T * r + tid;
            idv[r] = q < P ? ids[q] : -1;
        }
#pragma unroll
        for (int r = 0; r < ORD_B; ++r) {
            if (valid_e(idv[r])) {
                atomicAdd(&tot[idv[r]], 1);
                if (q0 + ORD_T * r + tid < b0) atomicAdd(&pre[idv[r]], 1);
            }
        }
    }
    const bool valid = valid_e(my_e);
    if (valid) atomicAdd(&c[w * ne + my_e], 1);
    __syncthreads();
    {
        // thread e: exclusive scans over the experts of the pair totals and of the active flags (ne <= 1024)
        const int e = tid;
        int cnt[ORD_W];
#pragma unroll
        for (int ww = 0; ww < ORD_W; ++ww) cnt[ww] = e < ne ? c[ww * ne + e] : 0;
        const int a = e < ne ? tot[e] : 0, b = a > 0;
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
            int base = ea + pre[e];
#pragma unroll
            for (int ww = 0; ww < ORD_W; ++ww) { c[ww * ne + e] = base; base += cnt[ww]; }
            if (blockIdx.x == 0 && b && egrp) { egrp[3 * eb] = e; egrp[3 * eb + 1] = ea; egrp[3 * eb + 2] = a; }
        }
        if (blockIdx.x == 0 && tid == ORD_T - 1) {
            int ta = 0, tb = 0;
            for (int ww = 0; ww < ORD_W; ++ww) { ta += wsum[0][ww]; tb += wsum[1][ww]; }
            order_n[0] = ta; order_n[1] = tb;
        }
    }
    __syncthreads();
    // the row: lanes of the same expert from the ballots of the id's bits (ids < ne < 2^nbits for valid lanes)
    unsigned long long same = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
        const unsigned long long ones = __ballot((my_e >> bit) & 1);
        same &= ((my_e >> bit) & 1) ? ones : ~ones;
    }
    if (valid) order[c[w * ne + my_e] + __popcll(same & ((1ull << lane) - 1))] = p;
}

int launch_order(const int *slot, int n_local, const int *ids, int P, int ne, int *order, int *order_n, int *egrp, hipStream_t s) {
    const int blocks = std::max(1, (P + ORD_T - 1) / ORD_T), nbits = ne > 1 ? 32 - __builtin_clz((unsigned) (ne - 1)) : 0;
    hipLaunchKernelGGL(k_order, dim3(blocks), dim3(ORD_T), 0, s, slot, n_local, ids, P, ne, nbits, order, order_n, egrp);
    return check_launch("hy_moe_order");
}

} // namespace hy
