// Decode / short-verify path in three launches per MoE layer, with no hand-off between blocks of a launch
// (device-scope fences and contended atomics cost more than a launch boundary on MI355X):
//   k_router_q8      router GEMV, a wave per (row, token) logit with its loads in flight together, and separate
//                    waves for the Q8 blocks of x (gemv_f32, src/kernels4.cu:163-180);
//   k_route_gate_up  every block routes its own token from the logits (softmax / top-k / renormalise / shared gate,
//                    src/kernels4.cu:297-344: up to 128 experts ranked by all eight waves at once, more by one wave),
//                    then each wave takes rw ff rows of its pair, gate and up against the Q8 x, and one wave folds
//                    and applies SwiGLU for the block's rows (moe_gate_up, src/kernels4.cu:1973-2006);
//   k_dec_down       each block brings in its token's pairs, the slot table and the k hidden rows at once, quantizes
//                    the rows into LDS (16 lanes per Q8_K block) while the down weights travel, then a wave per
//                    output row computes the down dots of all k pairs and the combine in ascending expert id
//                    (moe_down + moe_reduce, src/kernels4.cu:2007-2022, :1182-1206).
// Inside a wave the 8-lane groups take 256-value items (Item<T>, exact integers), the group's integers are summed
// with DPP, and each row's blocks are folded in block order: the same contract as the oracle.  Block barriers are
// LDS-only (lds_barrier), so global loads stay in flight across them.
#include "hy_internal.h"
#include "hy_blocks.cuh"
#include "hy_routing.cuh"
#include "hy_stamps.cuh"

#include <algorithm>

namespace hy {

#ifdef HY_STAMPS
__device__ unsigned long long g_stamps[STAMP_CAP];
extern "C" int hy_stamps_read(void *dst, size_t bytes) {
    return (int) hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps), bytes < sizeof(g_stamps) ? bytes : sizeof(g_stamps), 0, hipMemcpyDeviceToHost);
}
extern "C" int hy_stamps_clear() {
    static unsigned long long zero[STAMP_CAP];
    return (int) hipMemcpyToSymbol(HIP_SYMBOL(g_stamps), zero, sizeof(zero), 0, hipMemcpyHostToDevice);
}
#endif

constexpr int DEC_MAXP = 8;        // passes of 8 items per wave: up to 64 items (256-value spans) per wave
constexpr int DEC_ROUTE_NT = 8;    // tokens the fused router takes (more: the separate kernels)
constexpr int DEC_Y_BYTES = 9344;  // LDS for one Q8 activation row: 32 Q8_K blocks (n <= 8192), or 256 Q8_0 blocks (8704 B)

// Position of the items g, g + 8, g + 16, ... of a wave's flat item list, a list of units of `per` items each (gate/up:
// a 256-value span of each of the wave's rows; down: a pair's row of spans), without a division per item: advancing by
// 8 items moves q8 = 8 / per units and r8 = 8 % per items (both from the host), plus one unit when the item index wraps.
struct Cursor {
    int u, s;   // unit, span in the unit
    __device__ __forceinline__ void start(int g, int per) {   // per: uniform over the wave
        if ((per & (per - 1)) == 0) {   // a power of two (rows per wave 1, 2, 4, 8): no loop
            const int sh = __builtin_ctz((unsigned) per);
            u = g >> sh; s = g & (per - 1);
            return;
        }
        u = 0; s = g;
        while (s >= per) { s -= per; ++u; }
    }
    __device__ __forceinline__ void next(int per, int q8, int r8) {
        s += r8;
        const int c = s >= per ? 1 : 0;
        s -= c * per;
        u += q8 + c;
    }
};

// ---------------------------------------------------------------- k_router

template <int VT, typename WT, int RB>
__global__ __launch_bounds__(256) void k_router_q8(const WT *__restrict__ W, int rows, int kdim, const float *__restrict__ x, int xs,
                                                   const float *__restrict__ bias, int bs, float *__restrict__ logits, int ls,
                                                   uint8_t *__restrict__ xq, int nt) {
    HY_STAMP_VARS(3);
    HY_STAMP(0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + wave, lw = rows * nt;   // waves [0, lw): one (row, token) logit each
    // waves [lw, lw + units): the Q8 of x, a Q8_K block (token q / nb) or a Q8_0 pair of blocks each -- no wave does
    // both, so neither waits for the other
    if (gw >= lw) {
        const int q = gw - lw;
        if (VT == Q8_K) {
            const int nb = kdim / 256;
            if (q < nt * nb) {
                const int t = q / nb, b = q % nb;
                q8k_block_wave(x + (size_t) t * xs + 256 * b, xq + ((size_t) t * nb + b) * Q8K_BYTES);
            }
        } else {
            const int nb = kdim / 32, npair = (nb + 1) / 2;
            if (q < nt * npair) {
                const int t = q / npair, b = 2 * (q % npair);
                q8_0_pair_wave(x + (size_t) t * xs + 32 * b, xq + ((size_t) t * nb + b) * Q8_0_BYTES, b + 1 < nb, Q8_0_BYTES, 2);
            }
        }
        HY_STAMP(1);
        HY_STAMP_SET(2, 2);
        HY_STAMP_SAVE(4 * gw, 3, lane == 0 && gw < 4094, false);
        return;
    }
    // logit (row r, token t), the token waves of a row next to each other (they share its weight loads in L2): lane L
    // sums elements 256 i + 4 L + j with fmaf, then the butterfly.  The loads go out RB float4 pairs at a time (one
    // memory round trip per 256 RB values), then the fma chain.  RB 16 for one token and d > 2048 (d 4096 in one round
    // trip, 7168 in two), else 8 (more tokens' waves need the occupancy of fewer registers).
    const int r = gw / nt, t = gw - r * nt;
    const WT *wr = W + (size_t) r * kdim;
    const float *xt = x + (size_t) t * xs;
    float acc = 0.0f;
    for (int e0 = 0; e0 < kdim; e0 += 256 * RB) {
        float4 w[RB], xv[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int e = e0 + 256 * i + 4 * lane;
            w[i] = e < kdim ? ld_w4(wr + e) : make_float4(0, 0, 0, 0);
            xv[i] = e < kdim ? *(const float4 *) (xt + e) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            if (e0 + 256 * i + 4 * lane < kdim) {
                acc = __builtin_fmaf(w[i].x, xv[i].x, acc);
                acc = __builtin_fmaf(w[i].y, xv[i].y, acc);
                acc = __builtin_fmaf(w[i].z, xv[i].z, acc);
                acc = __builtin_fmaf(w[i].w, xv[i].w, acc);
            }
        }
    }
    float v = wave_sum_xor(acc);
    if (bias) v = v + bias[(size_t) t * bs + r];   // the token's bias, added after the butterfly
    if (lane == 0) logits[(size_t) t * ls + r] = v;
    HY_STAMP(1);
    HY_STAMP_SET(2, 1);
    HY_STAMP_SAVE(4 * gw, 3, lane == 0 && gw < 4094, false);
}

// ---------------------------------------------------------------- item dots against Q8 rows in LDS

// the integers of item `it` (256 values, span gi of a row) against the Q8 row `y` (LDS); K-quants: summed over the
// 8 lanes (every lane of the group gets them).  Q8_0 rows in LDS are split: the blocks' qs, 32 bytes each (16-byte
// aligned), with the scales kept apart.
template <int T>
__device__ __forceinline__ float item_t(const Item<T> &it, const uint8_t *y, int gi, int L, bool valid, float *tv_out, int tv_idx) {
    if constexpr (block_elems(T) == 32) {
        // lane L takes block 8 gi + L whole
        const uint8_t *yb = y + (size_t) (8 * gi + L) * 32;
        if (valid) {
            const uint4 y0 = *(const uint4 *) yb, y1 = *(const uint4 *) (yb + 16);
            const uint32_t ya[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
            tv_out[tv_idx + L] = it.tval(it.dot32(ya), ysum_type(T) ? ysum32(ya) : 0);
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
// item_t without the branch on `valid`: every lane computes (an invalid lane against span 0 of the row, its result
// unused) and only valid lanes store.  Straight-line code lets the compiler compute an item's weight side (scales,
// unpacked quants) once for several rows y taken in turn; the arithmetic, and so the bits stored, are item_t's.
template <int T>
__device__ __forceinline__ void item_t_all(const Item<T> &it, const uint8_t *y, int gi, int L, bool valid, float *tv_out, int tv_idx) {
    const int gs = valid ? gi : 0;
    if constexpr (block_elems(T) == 32) {
        const uint8_t *yb = y + (size_t) (8 * gs + L) * 32;
        const uint4 y0 = *(const uint4 *) yb, y1 = *(const uint4 *) (yb + 16);
        const uint32_t ya[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
        const float v = it.tval(it.dot32(ya), ysum_type(T) ? ysum32(ya) : 0);
        if (valid) tv_out[tv_idx + L] = v;
    } else {
        int si = 0, sm = 0;
        it.ints(y + (size_t) gs * Q8K_BYTES, L, si, sm);
        si = group8_isum(si);
        sm = group8_isum(sm);
        if (valid && L == 0) tv_out[tv_idx] = it.tval(si, sm);
    }
}
// activation scale of block b of a Q8 row
template <int VT> __device__ __forceinline__ float q8_scale(const uint8_t *y, int b) {
    if constexpr (VT == Q8_K) return *(const float *) (y + (size_t) b * Q8K_BYTES);
    else return h2f(ld_u16(y + (size_t) b * Q8_0_BYTES));
}

// One lane's block-order fold: acc[c] = fmaf(xs(b), tv(c, b), acc[c]) for b = 0 .. nb - 1, NC chains sharing the
// activation scales.  The LDS operands come in batches of 8 blocks held in two register sets that alternate, so a
// batch's reads are in flight while the previous batch's fma chain runs; full batches carry no guards and the last
// nb % 8 blocks go one by one.  The fmas are those of the plain loop, in its order.
template <int NC, typename XS, typename TV>
__device__ __forceinline__ void fold_blocks(int nb, XS xs, TV tv, float (&acc)[NC]) {
    constexpr int B = 8;
    const int nf = nb - nb % B;
    float x0[B], x1[B], t0[NC][B], t1[NC][B];
    auto ld = [&](float (&x)[B], float (&t)[NC][B], int b0) {
#pragma unroll
        for (int u = 0; u < B; ++u) {
            x[u] = xs(b0 + u);
#pragma unroll
            for (int c = 0; c < NC; ++c) t[c][u] = tv(c, b0 + u);
        }
    };
    auto fm = [&](const float (&x)[B], const float (&t)[NC][B]) {
#pragma unroll
        for (int u = 0; u < B; ++u)
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[c] = __builtin_fmaf(x[u], t[c][u], acc[c]);
    };
    if (nf) {
        ld(x0, t0, 0);
        for (int b0 = 0;; b0 += 2 * B) {   // uniform over the lanes that fold
            if (b0 + B < nf) ld(x1, t1, b0 + B);
            fm(x0, t0);
            if (b0 + B >= nf) break;
            if (b0 + 2 * B < nf) ld(x0, t0, b0 + 2 * B);
            fm(x1, t1);
            if (b0 + 2 * B >= nf) break;
        }
    }
    for (int b = nf; b < nb; ++b) {
        const float x = xs(b);
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[c] = __builtin_fmaf(x, tv(c, b), acc[c]);
    }
}

// ---------------------------------------------------------------- k_dec_gate_up

constexpr int DEC_GU_TV = 2 * 256;   // fold inputs per wave: 2 matrices x up to 256 blocks (IQ4_NL, n <= 8192)
constexpr int DEC_GU_WAVES = 8;      // waves per block, rw ff rows each
#ifndef HY_DEC_GU_BLOCKS
#define HY_DEC_GU_BLOCKS 768
#endif
constexpr int DEC_GU_BLOCKS = HY_DEC_GU_BLOCKS;   // grid size the rows per wave aim below
#ifndef HY_DEC_PIPE_NP
#define HY_DEC_PIPE_NP 2
#endif
constexpr int DEC_PIPE_NP = HY_DEC_PIPE_NP;        // passes per round when a wave's positions take several rounds

// V = 0: no routing, the pairs are the tokens and their expert the descriptor's local expert 0 (a shared expert).
// HQ: the block's 8 rw = 32 rows form one Q8_0 block of every pair's hidden row, and the fold also writes it to hq
// (the down kernel then reads the hidden quantized instead of quantizing it in every block).  PIPE: for waves with
// several rounds of items, each round's loads go out before the previous round's dots.
template <int T, int V, int NP, bool HQ = false, bool PIPE = false>
__global__ __launch_bounds__(64 * DEC_GU_WAVES) void k_route_gate_up(hy_moe_dev m, const float *__restrict__ logits, int ls, int ne, int k,
                                                                   const uint8_t *__restrict__ xq, int *__restrict__ ids,
                                                                   float *__restrict__ wts, float *__restrict__ sg, float *__restrict__ h,
                                                                   int rw, int q8, int r8, uint8_t *__restrict__ hq) {
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    constexpr int SPAN_W = 256 / BE * block_bytes(T);
    constexpr int SPAN_Y = VT == Q8_K ? Q8K_BYTES : 8 * Q8_0_BYTES;
    constexpr int TVN = HQ ? 2 * DEC_GU_TV : DEC_GU_TV;   // fold inputs per wave (HQ: 4 rows)
    // fold inputs of the block's rows, row l at l (2 nb + 1): an odd stride puts the rows' entries in distinct LDS
    // banks when the fold lanes (one row each) read entry b together
    __shared__ float tv[DEC_GU_WAVES * TVN + 64];
    __shared__ int s_ids[64];
    __shared__ float s_wts[64], s_sg;
    constexpr int VA = V < 0 ? -V : V;   // V < 0: the pairs were routed beforehand (ids given), the slot table as for -V
    __shared__ int s_slot[VA ? 64 * VA : 1];
    __shared__ uint2 grid[iq2_lds(T)];
    __shared__ float s_xd[DEC_GU_TV / 2];   // activation scales of the token's Q8 row, one per weight block
    __shared__ __align__(16) uint8_t s_y[DEC_Y_BYTES];   // the token's Q8 row (every item reads its 256-value span here)
    HY_STAMP_VARS(5);
    HY_STAMP(0);
    const int p = blockIdx.y, t = p / k, j = p - t * k;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 3, L = lane & 7;
    const int ff = m.ff, ng = m.n / 256, nb = m.n / BE;
    const uint8_t *y = xq + (size_t) t * ng * SPAN_Y;
    // Everything the block stages goes out at once, into registers: the token's Q8 row (Q8_K rows as they are, 292
    // bytes a block; Q8_0 rows as the qs of their blocks, 32 bytes each), the slot table and the activation scales;
    // `stage` stores them to LDS ahead of the routing barrier.
    constexpr int SY = (DEC_Y_BYTES / 4 + 64 * DEC_GU_WAVES - 1) / (64 * DEC_GU_WAVES);
    const int tid = (int) threadIdx.x, ny = VT == Q8_K ? ng * (Q8K_BYTES / 4) : nb * 8;
    uint32_t yv[SY];
#pragma unroll
    for (int u = 0; u < SY; ++u) {
        const int i = tid + u * 64 * DEC_GU_WAVES;
        yv[u] = 0;
        if (i < ny) {
            if constexpr (VT == Q8_K) {
                yv[u] = ((const uint32_t *) y)[i];
            } else {   // qs dword i & 7 of block i >> 3: 2-byte aligned in the row
                const uint8_t *q = y + (size_t) (i >> 3) * Q8_0_BYTES + 2 + 4 * (i & 7);
                yv[u] = (uint32_t) ld_u16(q) | ((uint32_t) ld_u16(q + 2) << 16);
            }
        }
    }
    constexpr int NS = 64 * VA;   // slot-table entries held (n_expert <= NS)
    const int e_given = V < 0 ? ids[(size_t) t * k + j] : 0;   // (loaded with the rest, used after the barrier)
    // the slot table as loaded; bounded where it is stored, so that no compare waits on it before the loads after
    // it (the logits) have gone out
    const int sl0 = tid < ne ? m.slot[tid] : -1;
    const int sl1 = NS > 64 * DEC_GU_WAVES && tid + 64 * DEC_GU_WAVES < ne ? m.slot[tid + 64 * DEC_GU_WAVES] : -1;
    const float xd = tid < nb ? q8_scale<VT>(y, tid) : 0.0f;
    auto stage = [&] {
#pragma unroll
        for (int u = 0; u < SY; ++u) {
            const int i = tid + u * 64 * DEC_GU_WAVES;
            if (i < ny) ((uint32_t *) s_y)[i] = yv[u];
        }
        if (tid < ne) s_slot[tid] = bound_slot(sl0, m.n_local);
        if constexpr (NS > 64 * DEC_GU_WAVES) {
            if (tid + 64 * DEC_GU_WAVES < ne) s_slot[tid + 64 * DEC_GU_WAVES] = bound_slot(sl1, m.n_local);
        }
        if (tid < nb) s_xd[tid] = xd;
        if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
    };
    const float *lg = logits + (size_t) t * ls;
    // the token's routing: every block of the token computes the same bits
    int e_sel;   // the expert of pair j
    if constexpr (V == 0) {   // no routing: every pair is local expert 0 (the always-on shared expert, k = 1)
        stage();
        lds_barrier();
        e_sel = 0;
    } else if constexpr (V < 0) {   // routed beforehand (hy_moe_route's bits): pair j's expert from ids
        stage();
        lds_barrier();
        e_sel = e_given;
    } else if constexpr (V <= 2) {
        static_assert(DEC_GU_WAVES == 8, "route_rank8 takes eight waves");
        int er;
        float pr, tot, lsg;
        route_rank8<V>(lg, ne, k, sg != nullptr, er, pr, tot, lsg, stage);   // the staged data shares its barrier
        e_sel = __builtin_amdgcn_readlane(er, j);
        if (blockIdx.x == 0 && j == 0 && wave == 0) {   // the first block of each token publishes the routing
            if (lane < k) { ids[(size_t) t * k + lane] = er; wts[(size_t) t * k + lane] = pr / tot; }
            if (lane == 0 && sg) sg[t] = 1.0f / (1.0f + hy_expf(-lsg));
        }
    } else {
        // wave 0 routes the token (one wave for more than 128 experts); every wave then stores its staged share
        if (wave == 0) route_wave<V>(lg, ne, k, s_ids, s_wts, sg ? &s_sg : nullptr);
        stage();
        lds_barrier();
        if (blockIdx.x == 0 && j == 0 && wave == 0) {   // the first block of each token publishes the routing
            if (lane < k) { ids[(size_t) t * k + lane] = s_ids[lane]; wts[(size_t) t * k + lane] = s_wts[lane]; }
            if (lane == 0 && sg) sg[t] = s_sg;
        }
        e_sel = s_ids[j];
    }
    const int e = e_sel;
    const int slot = __builtin_amdgcn_readfirstlane((e >= 0 && e < ne) ? s_slot[e] : -1);   // block-uniform
    HY_STAMP(1);
    if (slot < 0) return;   // uniform over the block: the pair's h rows are not written
    // the wave's rows row0 .. row0 + rw - 1: position p = (span p / rw, row p % rw), one gate item and one up item at
    // the same offset -- span-major, so that the rw neighbouring items of one span (adjacent bytes of a 16-row tile)
    // are fetched in one round rather than rw rounds apart, when the cache may have let their shared lines go; lane
    // group g takes positions g, g + 8, ... (a cursor over spans and rows); rows past ff sit out
    const int npos = rw * ng, row0 = (blockIdx.x * DEC_GU_WAVES + wave) * rw;
    const uint8_t *Wg = m.gate + (size_t) slot * m.gate_bytes, *Wu = m.up + (size_t) slot * m.gate_bytes;
    const int rs = 2 * nb + 1;
    float *tw = tv + wave * rw * rs;
    Cursor lc, cc;
    lc.start(g, rw);
    cc.start(g, rw);
    // a round: up to 8 NP positions loaded into (bg, bu) (the load cursor moves on), then their dots (the dot cursor)
    auto load_r = [&](Item<T> (&bg)[NP], Item<T> (&bu)[NP]) {
#pragma unroll
        for (int ps = 0; ps < NP; ++ps) {
            if (lc.u < ng && row0 + lc.s < ff) {
                const uint32_t off = tiled_off32(row0 + lc.s, lc.u, ng, SPAN_W);
                bg[ps].load(Wg + off, L);
                bu[ps].load(Wu + off, L);
            }
            lc.next(rw, q8, r8);
        }
    };
    auto dots_r = [&](Item<T> (&bg)[NP], Item<T> (&bu)[NP], int base) {
#pragma unroll
        for (int ps = 0; ps < NP; ++ps) {
            if (base + 8 * ps >= npos) break;   // wave-uniform
            const int r = cc.s, gi = cc.u, blk = block_elems(T) == 32 ? 8 * gi : gi;
            const bool valid = gi < ng && row0 + r < ff;
            if constexpr (iq2_type(T)) { bg[ps].grid = grid; bu[ps].grid = grid; }
            item_t<T>(bg[ps], s_y, gi, L, valid, tw, r * rs + blk);
            item_t<T>(bu[ps], s_y, gi, L, valid, tw, r * rs + nb + blk);
            cc.next(rw, q8, r8);
        }
    };
    Item<T> ig[NP], iu[NP];
    if constexpr (!PIPE) {
        for (int base = 0; base < npos; base += 8 * NP) {   // wave-uniform rounds
            load_r(ig, iu);
            if (base == 0) HY_STAMP_WAIT(2);
            dots_r(ig, iu, base);
        }
    } else {   // two sets of item registers: the next round's bytes travel while this round's dots run
        Item<T> ig2[NP], iu2[NP];
        load_r(ig, iu);
        HY_STAMP_WAIT(2);
        for (int base = 0; base < npos; base += 16 * NP) {
            if (base + 8 * NP < npos) load_r(ig2, iu2);
            dots_r(ig, iu, base);
            if (base + 16 * NP < npos) load_r(ig, iu);
            if (base + 8 * NP < npos) dots_r(ig2, iu2, base + 8 * NP);
        }
    }
    lds_barrier();
    HY_STAMP(3);
    // the folds, in block order, by wave 0: lane l takes the block's row l (wave l / rw, its row l % rw), gate and
    // up chains side by side (fold_blocks)
    if (wave != 0 || (!HQ && lane >= DEC_GU_WAVES * rw)) return;
    const int row = blockIdx.x * DEC_GU_WAVES * rw + lane;
    if (!HQ && row >= ff) return;
    float hv = 0.0f;
    if (lane < DEC_GU_WAVES * rw) {   // (HQ: lanes 32-63 stay for the quantizer's cross-lane max)
        const float *tg = tv + lane * rs;
        float a[2] = {0.0f, 0.0f};
        fold_blocks(nb, [&](int b) { return s_xd[b]; }, [&](int c, int b) { return tg[c * nb + b]; }, a);
        hv = hy_swiglu(a[0], a[1], m.clamp);
        h[(size_t) p * ff + row] = hv;
    }
    HY_STAMP(4);
    HY_STAMP_SAVE(16384 + 8 * (int) (blockIdx.y * gridDim.x + blockIdx.x), 5, lane == 0 && blockIdx.y * gridDim.x + blockIdx.x < 2047, true);
    if constexpr (HQ) {   // lanes 0-31: the 32 values of Q8_0 block blockIdx.x of pair p's hidden row (split layout)
        const int nbh = ff / 32;
        uint8_t *tok = hq + (size_t) t * k * nbh * Q8_0_BYTES;
        q8_0_pair_split(hv, tok + ((size_t) j * nbh + blockIdx.x) * 32, (uint16_t *) (tok + (size_t) k * nbh * 32) + j * nbh + blockIdx.x, false);
    }
}

// ---------------------------------------------------------------- k_dec_down

constexpr int DEC_DN_WAVES = 8;       // output rows per block (a wave each)
constexpr int DEC_DN_TV = 512;        // fold inputs per wave: k pairs x blocks of ff (k * nb <= 512)
constexpr int DEC_DN_HQ = 32768;      // LDS bytes for the token's k quantized hidden rows
#ifndef HY_DEC_DN_BLOCKS
#define HY_DEC_DN_BLOCKS 512
#endif
constexpr int DEC_DN_BLOCKS = HY_DEC_DN_BLOCKS;   // grid size the rows per wave aim below

// SEP: one expert's rows for several tokens (the shared expert; pair j = token j, ids 0, weights 1): each pair's value
// is written as its own output row, with no combine.
template <int T, int NP, bool SEP = false>
__global__ __launch_bounds__(64 * DEC_DN_WAVES) void k_dec_down(hy_moe_dev m, const float *__restrict__ h, const int *__restrict__ ids,
                                                               const float *__restrict__ wts, int k, const float *__restrict__ shexp,
                                                               const float *__restrict__ sg, float *__restrict__ out, int res, int q8, int r8,
                                                               const uint8_t *__restrict__ hqg, int rpw) {
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    constexpr int SPAN_W = 256 / BE * block_bytes(T);
    // the token's k hidden rows in LDS: Q8_K blocks as they are (SPAN_L = 292 bytes a span); Q8_0 split into the
    // blocks' qs (32 bytes each, SPAN_L = 256 a span) followed by their fp16 scales (hdq, k nb of them)
    constexpr int SPAN_L = VT == Q8_K ? Q8K_BYTES : 256;
    __shared__ __align__(16) uint8_t hq[DEC_DN_HQ];
    __shared__ float tv[DEC_DN_WAVES][DEC_DN_TV + 64];   // pair j's inputs at j (nb | 1): an odd stride, distinct banks
    __shared__ int s_slot[2 * 64 * DEC_DN_WAVES];   // n_expert <= 1024
    __shared__ int s_ord[DEC_DN_WAVES][64];
    __shared__ uint2 grid[iq2_lds(T)];
    HY_STAMP_VARS(6);
    HY_STAMP(0);
    const int t = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 3, L = lane & 7;
    // items: (pair, span) positions; SEP (one expert, the k pairs its tokens): the spans of the row, each item taken
    // against every token's hidden row in turn
    const int n = m.n, ff = m.ff, ng = ff / 256, nb = ff / BE, items = SEP ? ng : k * ng;
    uint16_t *hdq = (uint16_t *) (hq + (VT == Q8_K ? 0 : k * nb * 32));
    // the wave's output rows, one after the other (the block's hidden rows serve them all): row w of each of the
    // block's rpw groups of 8 consecutive rows, so that at every step the block's waves read 8 neighbouring rows
    // (adjacent bytes of a 16-row tile, fetched together) rather than rows rpw apart
    int row = blockIdx.x * DEC_DN_WAVES * rpw + wave;
    bool row_ok = row < n;
    const float *hp = h + (size_t) t * k * ff;
    // Everything the block reads first goes out together: lane j < k's pair (expert, weight), the slot table and
    // the first batch of hidden rows (all k pairs' rows; those of skipped pairs are read but never used).
    const int my_e = lane < k ? ids[t * k + lane] : -1;
    const float my_w = lane < k ? wts[t * k + lane] : 0.0f;
    const int tid = (int) threadIdx.x;
    const int sl0 = tid < m.n_expert ? m.slot[tid] : -1;   // bounded where stored: the loads below go out first
    const int sl1 = tid + 64 * DEC_DN_WAVES < m.n_expert ? m.slot[tid + 64 * DEC_DN_WAVES] : -1;
    float sh_x = 0.0f, sh_g = 1.0f;   // the shared expert's value and gate of this output, used at the end
    if (shexp && row_ok) {
        sh_x = shexp[(size_t) t * n + row];
        if (sg) sh_g = sg[t];
    }
    // Hidden-row units: Q8_K a 256-value block per 16-lane row (4 per wave), Q8_0 a pair of 32-value blocks per
    // wave (QU per wave); a batch is UB units.
    constexpr int QU = 4;
    constexpr int UB = (VT == Q8_K ? 4 : QU) * DEC_DN_WAVES;
    const int npair = (nb + 1) / 2, units = VT == Q8_K ? k * ng : k * npair;
    float xv[16];
    auto hload = [&](int ub) {
        if constexpr (VT == Q8_K) {
            const int u = ub + 4 * wave + (lane >> 4);
            if (u < units) {
                const float4 *src = (const float4 *) (hp + (size_t) u * 256 + 16 * (lane & 15));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 v = src[i];
                    xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < QU; ++q) {
                const int u = ub + wave + q * DEC_DN_WAVES;
                xv[q] = 0.0f;
                if (u < units) {
                    const int j = u / npair, b = 2 * (u - j * npair);
                    if (lane < 32 || b + 1 < nb) xv[q] = hp[(size_t) j * ff + 32 * b + lane];
                }
            }
        }
    };
    // hqg (Q8_0 partner types): the token's k hidden rows already quantized, in the split layout of LDS (the k nb
    // blocks' qs, then their scales: k nb 34 bytes, a multiple of 16): copied as 16-byte pieces ahead of the first
    // barrier, instead of loaded and quantized
    const bool hcopy = VT == Q8_0 && hqg;
    if (hcopy) {
        constexpr int HQV = DEC_DN_HQ / (16 * 64 * DEC_DN_WAVES);
        const int n16 = k * nb * Q8_0_BYTES / 16;
        const uint4 *src = (const uint4 *) (hqg + (size_t) t * k * nb * Q8_0_BYTES);
#pragma unroll
        for (int i = 0; i < HQV; ++i) {
            const int o = tid + i * 64 * DEC_DN_WAVES;
            if (o < n16) ((uint4 *) hq)[o] = src[o];
        }
    } else {
        hload(0);
    }
    s_slot[tid] = bound_slot(sl0, m.n_local);
    s_slot[tid + 64 * DEC_DN_WAVES] = bound_slot(sl1, m.n_local);
    lds_barrier();
    HY_STAMP(1);
    // lane j < k: pair j's slot (-1: skipped); `okm`: the valid pairs as a wave-uniform bit mask
    const int my_slot = (my_e >= 0 && my_e < m.n_expert) ? s_slot[my_e] : -1;
    const uint64_t okm = __ballot(my_slot >= 0);
    auto pair_ok = [&](int j) { return (okm >> j) & 1; };
    Item<T> it[NP];
    // item i = pair j's span gi; lane group g takes items g, g + 8, ... (cursors over pairs and spans: one for the loads,
    // one for the dots, each moving 8 items a pass)
    Cursor lc, cc;
    lc.start(g, ng);
    cc.start(g, ng);
    auto load_round = [&](int base) {
#pragma unroll
        for (int ps = 0; ps < NP; ++ps) {
            const int i = base + g + 8 * ps;
            if constexpr (SEP) {   // span i of the row, the expert of pair 0 (every pair's)
                const int sl = __builtin_amdgcn_readfirstlane(my_slot);
                if (i < items && row_ok && sl >= 0) it[ps].load(m.down + (size_t) sl * m.down_bytes + tiled_off(row, i, ng, SPAN_W), L);
            } else {
                const int j = lc.u, gi = lc.s;
                const int sl = __shfl(my_slot, j < 64 ? j : 0);
                if (i < items && row_ok && sl >= 0) it[ps].load(m.down + (size_t) sl * m.down_bytes + tiled_off(row, gi, ng, SPAN_W), L);
                lc.next(ng, q8, r8);
            }
        }
    };
    // the first round of weight bytes goes out before the hidden rows are quantized (wave-uniform branches below)
    load_round(0);
    // while they travel: each valid pair's rank by (expert id, j) is its place in the combine; `ordl` (lane r) is
    // the lane of rank r
    int rank = 0;
    for (int i = 0; i < k; ++i) {   // uniform trip count; the other lanes' experts by lane read
        const int ei = __builtin_amdgcn_readlane(my_e, i);
        if (pair_ok(i) && (ei < my_e || (ei == my_e && i < lane))) ++rank;
    }
    const bool mine = lane < k && pair_ok(lane);
    if (mine) s_ord[wave][rank] = lane;
    wave_lds_sync();
    const int ordl = s_ord[wave][lane];
    auto hquant = [&](int ub) {
        if constexpr (VT == Q8_K) {
            const int u = ub + 4 * wave + (lane >> 4);
            if (u < units && pair_ok(u / ng)) q8k_block16(xv, hq + (size_t) u * Q8K_BYTES);   // uniform over the row
        } else {
#pragma unroll
            for (int q = 0; q < QU; ++q) {
                const int u = ub + wave + q * DEC_DN_WAVES;
                if (u < units) {
                    const int j = u / npair, b = 2 * (u - j * npair);
                    if (pair_ok(j)) q8_0_pair_split(xv[q], hq + ((size_t) j * nb + b) * 32, hdq + j * nb + b, b + 1 < nb);
                }
            }
        }
    };
    if (!hcopy) {
        hquant(0);
        for (int ub = UB; ub < units; ub += UB) { hload(ub); hquant(ub); }
    }
    if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
    lds_barrier();
    HY_STAMP(2);
    HY_STAMP_WAIT(3);
    if (!row_ok) return;   // wave-uniform; no block barrier follows
    float *tw = tv[wave];
    for (int rr = 0;;) {
        for (int base = 0; base < items; base += 8 * NP) {   // wave-uniform rounds of up to 8 NP items
            if (base) load_round(base);
#pragma unroll
            for (int ps = 0; ps < NP; ++ps) {
                const int i = base + g + 8 * ps;
                if (base + 8 * ps >= items) break;   // wave-uniform
                if constexpr (iq2_type(T)) it[ps].grid = grid;
                if constexpr (SEP) {   // span i against each token's row: the item's weight side unpacked once
                    const int blk = block_elems(T) == 32 ? 8 * i : i;
#pragma unroll 8
                    for (int j = 0; j < k; ++j)
                        item_t_all<T>(it[ps], hq + (size_t) j * ng * SPAN_L, i, L, i < items && pair_ok(j), tw, j * (nb | 1) + blk);
                } else {
                    const int j = cc.u, gi = cc.s;
                    const bool valid = i < items && pair_ok(j);
                    item_t<T>(it[ps], hq + (size_t) j * ng * SPAN_L, gi, L, valid, tw, j * (nb | 1) + (block_elems(T) == 32 ? 8 * gi : gi));
                    cc.next(ng, q8, r8);
                }
            }
        }
        wave_lds_sync();
        HY_STAMP(4);
        // lane j folds pair j in block order
        float fo = 0.0f;
        if (mine) {
            const uint8_t *yj = hq + (size_t) lane * ng * SPAN_L;
            const float *tj = tw + lane * (nb | 1);
            float acc = 0.0f;
            if constexpr (block_elems(T) == 32) {   // ff / 32 blocks: batches in flight ahead of the chain
                float a1[1] = {0.0f};
                fold_blocks(nb, [&](int b) { return VT == Q8_K ? q8_scale<VT>(yj, b) : h2f(hdq[lane * nb + b]); },
                            [&](int, int b) { return tj[b]; }, a1);
                acc = a1[0];
            } else {   // ff / 256 blocks (a few): four blocks' inputs per LDS round trip, then the fma chain
                for (int b0 = 0; b0 < nb; b0 += 4) {
                    float sc[4], tq[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (b0 + u < nb) { sc[u] = q8_scale<VT>(yj, b0 + u); tq[u] = tj[b0 + u]; }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (b0 + u < nb) acc = __builtin_fmaf(sc[u], tq[u], acc);
                }
            }
            fo = my_w * acc;
        }
        if constexpr (SEP) {   // pair j's value is output row j
            if (mine) out[(size_t) lane * n + row] = fo;
            if (++rr == rpw || (row += DEC_DN_WAVES) >= n) break;   // wave-uniform
            lc.start(g, ng);
            cc.start(g, ng);
            wave_lds_sync();
            load_round(0);
            continue;
        }
        // the combine in rank order, each value read from the lane that holds it
        const int nv = __builtin_popcountll(okm);
        float acc = 0.0f;
        bool first = true;
        if (shexp) { acc = sh_g * sh_x; first = false; }
        for (int r = 0; r < nv; ++r) {
            const float v = readlane_f(fo, __builtin_amdgcn_readlane(ordl, r));
            if (first) { acc = v; first = false; } else acc = acc + v;
        }
        if (lane == 0) out[(size_t) t * n + row] = res ? out[(size_t) t * n + row] + acc : acc;   // res: the residual add
        if (++rr == rpw || (row += DEC_DN_WAVES) >= n) break;   // wave-uniform
        // the next row: its shared-expert value, fresh cursors, the first round of its weight bytes
        if (shexp) sh_x = shexp[(size_t) t * n + row];
        lc.start(g, ng);
        cc.start(g, ng);
        wave_lds_sync();   // this row's fold inputs are read before the next row's dots write them
        load_round(0);
    }
    HY_STAMP(5);
    HY_STAMP_SAVE(32768 + 8 * (int) (blockIdx.y * gridDim.x + blockIdx.x), 6, wave == 0 && lane == 0 && blockIdx.y * gridDim.x + blockIdx.x < 4095, true);
}

// ---------------------------------------------------------------- shared expert, several tokens

// The always-on expert (the descriptor's local expert 0) for 2..SH_MAX tokens: a block takes up to SH_NT of them,
// stages their Q8 rows in LDS, and each wave loads its rows' gate and up items once and takes their integers against
// every staged row; one lane a (row, token) folds the blocks in order -- the expressions of k_route_gate_up with
// V = 0 (the one-token form), so the bits are those.  SH_NT rows keep the block's LDS small enough for two blocks a
// CU next to the routed experts' kernels (the shared expert runs beside them on a second stream).
constexpr int SH_NT = 4;          // tokens a block takes (grid.y: token groups)
constexpr int SH_MAX = 8;         // tokens a launch takes
constexpr int SH_TV = 4096;       // fold inputs a block holds: tokens x rows x (2 nb + 1)
constexpr int SH_LD = 16;         // staging loads in flight a thread

template <int T, int NP>
__global__ __launch_bounds__(64 * DEC_GU_WAVES) void k_shared_gate_up(hy_moe_dev m, const uint8_t *__restrict__ xq, float *__restrict__ h,
                                                                    int nt, int rw, int q8, int r8) {
    constexpr int VT = vec_dot_type(T), BE = block_elems(T);
    constexpr int SPAN_W = 256 / BE * block_bytes(T);
    constexpr int SPAN_Y = VT == Q8_K ? Q8K_BYTES : 8 * Q8_0_BYTES;
    __shared__ __align__(16) uint8_t s_y[SH_NT * DEC_Y_BYTES];   // token t's row at t * ybytes, laid out as k_route_gate_up's
    __shared__ float s_xd[SH_NT * (DEC_GU_TV / 2)];             // token t's activation scales at t * nb
    __shared__ float tv[SH_TV];
    __shared__ uint2 grid[iq2_lds(T)];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 3, L = lane & 7, tid = threadIdx.x;
    const int ff = m.ff, ng = m.n / 256, nb = m.n / BE, RB = DEC_GU_WAVES * rw, rs = 2 * nb + 1;
    const int ny = VT == Q8_K ? ng * (Q8K_BYTES / 4) : nb * 8, ybytes = 4 * ny;
    const int t0 = blockIdx.y * SH_NT, ntb = min(SH_NT, nt - t0);   // this block's tokens
    xq += (size_t) t0 * ng * SPAN_Y;
    h += (size_t) t0 * ff;
    // the tokens' rows into LDS, SH_LD dwords a thread in flight at once
    for (int i0 = tid; i0 < ntb * ny; i0 += SH_LD * 64 * DEC_GU_WAVES) {
        uint32_t v[SH_LD];
#pragma unroll
        for (int u = 0; u < SH_LD; ++u) {
            const int i = i0 + u * 64 * DEC_GU_WAVES, t = i / ny, w = i - t * ny;
            v[u] = 0;
            if (i < ntb * ny) {
                const uint8_t *y = xq + (size_t) t * ng * SPAN_Y;
                if constexpr (VT == Q8_K) v[u] = ((const uint32_t *) y)[w];
                else {   // qs dword w & 7 of block w >> 3: 2-byte aligned in the row
                    const uint8_t *q = y + (size_t) (w >> 3) * Q8_0_BYTES + 2 + 4 * (w & 7);
                    v[u] = (uint32_t) ld_u16(q) | ((uint32_t) ld_u16(q + 2) << 16);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < SH_LD; ++u) {
            const int i = i0 + u * 64 * DEC_GU_WAVES, t = i / ny;
            if (i < ntb * ny) ((uint32_t *) (s_y + (size_t) t * ybytes))[i - t * ny] = v[u];
        }
    }
    for (int i = tid; i < ntb * nb; i += 64 * DEC_GU_WAVES) {
        const int t = i / nb;
        s_xd[t * nb + (i - t * nb)] = q8_scale<VT>(xq + (size_t) t * ng * SPAN_Y, i - t * nb);
    }
    if constexpr (iq2_type(T)) expand_iq2_grid<T>(grid);
    const int slot = bound_slot(m.slot[0], m.n_local);
    lds_barrier();
    if (slot < 0) return;   // uniform: the expert is not local, h is not written
    const int npos = rw * ng, row0 = (blockIdx.x * DEC_GU_WAVES + wave) * rw;
    const uint8_t *Wg = m.gate + (size_t) slot * m.gate_bytes, *Wu = m.up + (size_t) slot * m.gate_bytes;
    Cursor lc, cc;   // positions span-major, as in k_route_gate_up
    lc.start(g, rw);
    cc.start(g, rw);
    Item<T> ig[NP], iu[NP];
    for (int base = 0; base < npos; base += 8 * NP) {   // wave-uniform rounds of up to 8 NP positions
#pragma unroll
        for (int ps = 0; ps < NP; ++ps) {
            if (lc.u < ng && row0 + lc.s < ff) {
                const uint32_t off = tiled_off32(row0 + lc.s, lc.u, ng, SPAN_W);
                ig[ps].load(Wg + off, L);
                iu[ps].load(Wu + off, L);
            }
            lc.next(rw, q8, r8);
        }
#pragma unroll
        for (int ps = 0; ps < NP; ++ps) {
            if (base + 8 * ps >= npos) break;   // wave-uniform
            const int r = cc.s, gi = cc.u, blk = BE == 32 ? 8 * gi : gi;
            const bool valid = gi < ng && row0 + r < ff;
            if constexpr (iq2_type(T)) { ig[ps].grid = grid; iu[ps].grid = grid; }
            const int rr = wave * rw + r;
#pragma unroll
            for (int t = 0; t < SH_NT; ++t) {
                if (t >= ntb) break;   // uniform (token 0 always runs: its weight-side work serves the others)
                const uint8_t *yt = s_y + (size_t) t * ybytes;
                item_t_all<T>(ig[ps], yt, gi, L, valid, tv, (t * RB + rr) * rs + blk);
                item_t_all<T>(iu[ps], yt, gi, L, valid, tv, (t * RB + rr) * rs + nb + blk);
            }
            cc.next(rw, q8, r8);
        }
    }
    lds_barrier();
    // lane (t, rr) folds row rr of the block for token t: gate and up chains side by side
    const int t = tid / RB, rr = tid - t * RB, row = blockIdx.x * RB + rr;
    if (t >= ntb || row >= ff) return;
    const float *tg = tv + (t * RB + rr) * rs;
    const float *xd = s_xd + t * nb;
    float a[2] = {0.0f, 0.0f};
    fold_blocks(nb, [&](int b) { return xd[b]; }, [&](int c, int b) { return tg[c * nb + b]; }, a);
    h[(size_t) t * ff + row] = hy_swiglu(a[0], a[1], m.clamp);
}

// ---------------------------------------------------------------- launchers

#define HY_DEC_SWITCH(T, CALL)                                                                   \
    switch (T) {                                                                                 \
    case Q4_K: { constexpr int TT = Q4_K; CALL; }                                               \
    case Q5_K: { constexpr int TT = Q5_K; CALL; }                                               \
    case Q6_K: { constexpr int TT = Q6_K; CALL; }                                               \
    case IQ4_XS: { constexpr int TT = IQ4_XS; CALL; }                                           \
    case IQ2_XS: { constexpr int TT = IQ2_XS; CALL; }                                           \
    case IQ2_XXS: { constexpr int TT = IQ2_XXS; CALL; }                                         \
    case IQ4_NL: { constexpr int TT = IQ4_NL; CALL; }                                           \
    case Q8_0: { constexpr int TT = Q8_0; CALL; }                                               \
    case MXFP4: { constexpr int TT = MXFP4; CALL; }                                             \
    case Q5_0: { constexpr int TT = Q5_0; CALL; }                                               \
    case Q5_1: { constexpr int TT = Q5_1; CALL; }                                               \
    case Q2_K: { constexpr int TT = Q2_K; CALL; }                                               \
    case Q3_K: { constexpr int TT = Q3_K; CALL; }                                               \
    case IQ3_XXS: { constexpr int TT = IQ3_XXS; CALL; }                                         \
    case IQ3_S: { constexpr int TT = IQ3_S; CALL; }                                             \
    case IQ2_S: { constexpr int TT = IQ2_S; CALL; }                                             \
    case IQ1_S: { constexpr int TT = IQ1_S; CALL; }                                             \
    default: set_error("unsupported expert type %d", (int) (T)); return HY_EUNSUPPORTED_TYPE;   \
    }

template <typename WT>
static int router_q8_any(const WT *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                         int vtype, void *xq, int nt, hipStream_t s) {
    if (nt == 0) return HY_OK;
    if (nt > DEC_ROUTE_NT) return launch_router_pre(W, rows, kdim, x, xs, bias, bs, logits, ls, vtype, xq, nt, s);   // batched rows
    const int qwaves = vtype == Q8_K ? nt * (kdim / 256) : nt * ((kdim / 32 + 1) / 2);
    const int blocks = (rows * nt + qwaves + 3) / 4;   // a wave per (row, token) logit, then the Q8 waves
#define HY_RQ(VV, RR) hipLaunchKernelGGL((k_router_q8<VV, WT, RR>), dim3(blocks), dim3(256), 0, s, W, rows, kdim, x, xs, bias, bs, logits, ls, \
                                         (uint8_t *) xq, nt)
    const bool wide = nt == 1 && kdim > 2048;   // RB 8 already takes d <= 2048 in one round trip
    if (vtype == Q8_K) { if (wide) HY_RQ(Q8_K, 16); else HY_RQ(Q8_K, 8); }
    else { if (wide) HY_RQ(Q8_0, 16); else HY_RQ(Q8_0, 8); }
#undef HY_RQ
    return check_launch("hy_moe_router_q8");
}
int launch_router_q8(const float *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                     int vtype, void *xq, int nt, hipStream_t s) {
    return router_q8_any(W, rows, kdim, x, xs, bias, bs, logits, ls, vtype, xq, nt, s);
}
int launch_router_q8(const uint16_t *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                     int vtype, void *xq, int nt, hipStream_t s) {
    return router_q8_any(W, rows, kdim, x, xs, bias, bs, logits, ls, vtype, xq, nt, s);
}

int launch_route_gate_up(const hy_moe_dev &m, const float *logits, int ls, int ne, int k, const void *xq, int *ids, float *wts, float *sg,
                         float *h, int nt, hipStream_t s, uint8_t *hq) {
    const int ng = m.n / 256, nb = m.n / block_elems(m.tg);
    if (2 * ng > 8 * DEC_MAXP || 2 * nb > DEC_GU_TV) { set_error("hy_moe_route_gate_up: n = %d exceeds %d", m.n, 256 * 4 * DEC_MAXP); return HY_EBAD_SHAPE; }
    if (m.gate_bytes >= ((size_t) 1 << 32)) { set_error("hy_moe_route_gate_up: an expert matrix of %zu bytes (4 GiB or more)", m.gate_bytes); return HY_EBAD_SHAPE; }
    if (hq) {   // the Q8_0 hidden as well: 32-row blocks (rw 4), items and fold inputs within the HQ instantiation's limits
        if (vec_dot_type(m.tg) != Q8_0 || vec_dot_type(m.td) != Q8_0 || 4 * 2 * nb > 2 * DEC_GU_TV) {
            set_error("hy_moe_route_gate_up_q8: needs IQ4_NL, Q8_0, MXFP4, Q5_0 or Q5_1 gate/up and down weights and n <= 4096 (types %d/%d, n %d)", m.tg, m.td, m.n);
            return HY_EUNSUPPORTED_TYPE;
        }
        if (nt == 0) return HY_OK;
        const int V = (ne + 63) / 64, q8 = 8 / 4, r8 = 8 % 4;   // the position cursor's step (rw 4)
        dim3 grid(m.ff / 32, nt * k);
        if ((long) grid.x * grid.y > DEC_GU_BLOCKS && ne <= 1024) {   // more than one round of blocks: route once first
            int rc = launch_route(logits, ls, ne, k, ids, wts, sg, nt, s);
            if (rc) return rc;
#define HY_RGUQI(TQ) hipLaunchKernelGGL((k_route_gate_up<TQ, -16, DEC_PIPE_NP, true, true>), grid, dim3(64 * DEC_GU_WAVES), 0, s, m, logits, ls, ne, k, (const uint8_t *) xq, ids, wts, sg, h, 4, q8, r8, hq)
            if (m.tg == IQ4_NL) { HY_RGUQI(IQ4_NL); } else if (m.tg == MXFP4) { HY_RGUQI(MXFP4); } else if (m.tg == Q5_0) { HY_RGUQI(Q5_0); }
            else if (m.tg == Q5_1) { HY_RGUQI(Q5_1); }
            else { HY_RGUQI(Q8_0); }
#undef HY_RGUQI
            return check_launch("hy_moe_route_gate_up_q8");
        }
#define HY_RGUQ(TQ, VV) hipLaunchKernelGGL((k_route_gate_up<TQ, VV, DEC_PIPE_NP, true, true>), grid, dim3(64 * DEC_GU_WAVES), 0, s, m, logits, ls, ne, k, (const uint8_t *) xq, ids, wts, sg, h, 4, q8, r8, hq)
#define HY_RGUQ_V(TQ) if (V <= 1) HY_RGUQ(TQ, 1); else if (V <= 2) HY_RGUQ(TQ, 2); else if (V <= 4) HY_RGUQ(TQ, 4); else if (V <= 8) HY_RGUQ(TQ, 8); else HY_RGUQ(TQ, 16);
        if (m.tg == IQ4_NL) { HY_RGUQ_V(IQ4_NL) } else if (m.tg == MXFP4) { HY_RGUQ_V(MXFP4) } else if (m.tg == Q5_0) { HY_RGUQ_V(Q5_0) }
        else if (m.tg == Q5_1) { HY_RGUQ_V(Q5_1) }
        else { HY_RGUQ_V(Q8_0) }
#undef HY_RGUQ_V
#undef HY_RGUQ
        return check_launch("hy_moe_route_gate_up_q8");
    }
    if (nt == 0) return HY_OK;
    // rows per wave: every block routes its token again, so the grid is kept near DEC_GU_BLOCKS blocks, within the
    // fold inputs (rw 2 nb <= DEC_GU_TV); a wave's rw ng positions run in rounds of up to 8 NP
    int rw = 1;
    auto nblocks = [&](int r) { return (long) ((m.ff + DEC_GU_WAVES * r - 1) / (DEC_GU_WAVES * r)) * nt * k; };
    while (rw < 8 && nblocks(rw) > DEC_GU_BLOCKS && (rw + 1) * 2 * nb <= DEC_GU_TV) ++rw;
    dim3 grid((m.ff + DEC_GU_WAVES * rw - 1) / (DEC_GU_WAVES * rw), nt * k);
    const int V = (ne + 63) / 64;
    const int np = (rw * ng + 7) / 8;   // passes of 8 positions (a gate and an up item each)
    const int q8 = 8 / rw, r8 = 8 % rw;   // the position cursor's step (span-major positions)
#define HY_RGU(VV, NN, PP) hipLaunchKernelGGL((k_route_gate_up<TT, VV, NN, false, PP>), grid, dim3(64 * DEC_GU_WAVES), 0, s, m, logits, ls, ne, k, (const uint8_t *) xq, ids, wts, sg, h, rw, q8, r8, nullptr)
#define HY_RGU_V(NN, PP) if (V <= 1) HY_RGU(1, NN, PP); else if (V <= 2) HY_RGU(2, NN, PP); else if (V <= 4) HY_RGU(4, NN, PP); else if (V <= 8) HY_RGU(8, NN, PP); else HY_RGU(16, NN, PP);
    // more than one round of blocks (every block would route its token again, the later blocks after the earlier
    // ones): route once first (hy_moe_route's kernel, the same bits), the blocks then read their pair's expert
    const bool pre = (long) grid.x * grid.y > DEC_GU_BLOCKS && ne <= 1024;
    if (pre) {
        int rc = launch_route(logits, ls, ne, k, ids, wts, sg, nt, s);
        if (rc) return rc;
    }
    HY_DEC_SWITCH(m.tg, {
        if (pre) {
            if (np <= 1) { HY_RGU(-16, 1, false); } else if (np <= 2) { HY_RGU(-16, 2, false); } else if (np <= 4) { HY_RGU(-16, 4, false); } else { HY_RGU(-16, DEC_PIPE_NP, true); }
        } else if (np <= 1) { HY_RGU_V(1, false) } else if (np <= 2) { HY_RGU_V(2, false) } else if (np <= 4) { HY_RGU_V(4, false) } else { HY_RGU_V(DEC_PIPE_NP, true) }
        return check_launch("hy_moe_route_gate_up");
    });
#undef HY_RGU_V
#undef HY_RGU
}

// the gate/up of local expert 0 for every token (a shared expert) from the Q8 rows: k_route_gate_up without routing
int launch_fixed_gate_up(const hy_moe_dev &m, const void *xq, float *h, int nt, hipStream_t s) {
    const int ng = m.n / 256, nb = m.n / block_elems(m.tg);
    if (2 * ng > 8 * DEC_MAXP || 2 * nb > DEC_GU_TV) { set_error("hy_moe_shared_gate_up: n = %d exceeds %d", m.n, 256 * 4 * DEC_MAXP); return HY_EBAD_SHAPE; }
    if (m.gate_bytes >= ((size_t) 1 << 32)) { set_error("hy_moe_shared_gate_up: an expert matrix of %zu bytes (4 GiB or more)", m.gate_bytes); return HY_EBAD_SHAPE; }
    if (nt == 0) return HY_OK;
    int rw = 1;   // rows per wave, as in launch_route_gate_up
    auto nblocks = [&](int r) { return (long) ((m.ff + DEC_GU_WAVES * r - 1) / (DEC_GU_WAVES * r)) * nt; };
    while (rw < 8 && nblocks(rw) > DEC_GU_BLOCKS && (rw + 1) * 2 * nb <= DEC_GU_TV) ++rw;
    dim3 grid((m.ff + DEC_GU_WAVES * rw - 1) / (DEC_GU_WAVES * rw), nt);
    const int np = (rw * ng + 7) / 8, q8 = 8 / rw, r8 = 8 % rw;
#define HY_FGU(NN, PP) hipLaunchKernelGGL((k_route_gate_up<TT, 0, NN, false, PP>), grid, dim3(64 * DEC_GU_WAVES), 0, s, m, nullptr, 0, 1, 1, (const uint8_t *) xq, nullptr, nullptr, nullptr, h, rw, q8, r8, nullptr)
    HY_DEC_SWITCH(m.tg, {
        if (np <= 1) { HY_FGU(1, false); } else if (np <= 2) { HY_FGU(2, false); } else if (np <= 4) { HY_FGU(4, false); } else { HY_FGU(DEC_PIPE_NP, true); }
        return check_launch("hy_moe_shared_gate_up");
    });
#undef HY_FGU
}

// the shared expert's gate/up for 2..SH_MAX tokens, one pass over its weights for every SH_NT (k_shared_gate_up); HY_EUNSUPPORTED_TYPE
// when the tokens' rows or fold inputs exceed its LDS (the caller then takes launch_fixed_gate_up)
int launch_shared_gate_up(const hy_moe_dev &m, const void *xq, float *h, int nt, hipStream_t s) {
    const int ng = m.n / 256, nb = m.n / block_elems(m.tg);
    const int ybytes = vec_dot_type(m.tg) == Q8_K ? ng * Q8K_BYTES : nb * 32;
    const int ntb = std::min(nt, SH_NT);   // tokens a block holds
    if (nt < 2 || nt > SH_MAX || ybytes > DEC_Y_BYTES || 2 * nb > DEC_GU_TV || 2 * ng > 8 * DEC_MAXP ||
        (long) ntb * DEC_GU_WAVES * (2 * nb + 1) > SH_TV || m.gate_bytes >= ((size_t) 1 << 32))
        return HY_EUNSUPPORTED_TYPE;
    // rows per wave: blocks enough for every CU (one row a wave when ff allows), within the fold inputs
    const int groups = (nt + SH_NT - 1) / SH_NT;
    int rw = 1;
    while (rw < 4 && (long) ((m.ff + DEC_GU_WAVES * (rw + 1) - 1) / (DEC_GU_WAVES * (rw + 1))) * groups >= 256 &&
           (long) ntb * DEC_GU_WAVES * (rw + 1) * (2 * nb + 1) <= SH_TV)
        ++rw;
    dim3 grid((m.ff + DEC_GU_WAVES * rw - 1) / (DEC_GU_WAVES * rw), groups);
    const int np = (rw * ng + 7) / 8, q8 = 8 / rw, r8 = 8 % rw;
#define HY_SGU(NN) hipLaunchKernelGGL((k_shared_gate_up<TT, NN>), grid, dim3(64 * DEC_GU_WAVES), 0, s, m, (const uint8_t *) xq, h, nt, rw, q8, r8)
    HY_DEC_SWITCH(m.tg, {
        if (np <= 1) HY_SGU(1); else if (np <= 2) HY_SGU(2); else HY_SGU(4);
        return check_launch("hy_moe_shared_gate_up");
    });
#undef HY_SGU
}

static bool dec_down_fits(const hy_moe_dev &m, int k) {
    const int vt = vec_dot_type(m.td), ng = m.ff / 256, nb = m.ff / block_elems(m.td);
    const int span_y = vt == Q8_K ? Q8K_BYTES : 8 * Q8_0_BYTES;
    return k <= 64 && k * nb <= DEC_DN_TV && (size_t) k * ng * span_y <= (size_t) DEC_DN_HQ && m.n_expert <= 2 * 64 * DEC_DN_WAVES;
}
bool dec_down_takes_q8(const hy_moe_dev &m, int k) { return vec_dot_type(m.td) == Q8_0 && dec_down_fits(m, k); }

// the fused decode down + combine; shapes beyond its LDS budget return HY_EUNSUPPORTED_TYPE (caller falls back)
int launch_dec_down(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp, const float *sg,
                    float *out, int nt, hipStream_t s, int res, const uint8_t *hq) {
    const int vt = vec_dot_type(m.td), ng = m.ff / 256;
    if (hq && vt != Q8_0) { set_error("hy_moe_down_reduce_q8: down type %d does not take Q8_0 rows", m.td); return HY_EUNSUPPORTED_TYPE; }
    if (!dec_down_fits(m, k)) {
        if (hq) set_error("hy_moe_down_reduce_q8: k * ff = %d * %d exceeds the kernel's hidden-row budget", k, m.ff);
        return HY_EUNSUPPORTED_TYPE;
    }
    if (nt == 0) return HY_OK;
    // rows per wave: more than one when one row a wave would take more blocks than the CUs hold at once (about two
    // blocks a CU), so that the blocks run in one round and each block quantizes its hidden rows once for them all
    int rpw = 1;
    while (rpw < 16 && (long) ((m.n + DEC_DN_WAVES * rpw - 1) / (DEC_DN_WAVES * rpw)) * nt > DEC_DN_BLOCKS) ++rpw;
    dim3 grid((m.n + DEC_DN_WAVES * rpw - 1) / (DEC_DN_WAVES * rpw), nt);
    const int np = (k * ng + 7) / 8;   // passes of 8 items (more than 8: rounds)
    const int q8 = 8 / ng, r8 = 8 % ng;   // the item cursors' step
#define HY_DN(NN) hipLaunchKernelGGL((k_dec_down<TT, NN>), grid, dim3(64 * DEC_DN_WAVES), 0, s, m, h, ids, wts, k, shexp, sg, out, res, q8, r8, hq, rpw)
    HY_DEC_SWITCH(m.td, {
        // 8 passes a round only for IQ2_XS (same occupancy as 4); the others take more rounds at a higher occupancy
        if (np <= 2) HY_DN(2);
        else if constexpr (TT != IQ2_XS) HY_DN(4);
        else if (np <= 4) HY_DN(4); else HY_DN(8);
        return check_launch("hy_moe_down_reduce");
    });
#undef HY_DN
}

// the shared expert's down for nt tokens in one pass over its weights: k_dec_down with the tokens as its k pairs
// (ids all 0, weights all 1) and one output row per pair; HY_EUNSUPPORTED_TYPE beyond its LDS budget
int launch_shared_down(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, float *out, int nt, hipStream_t s) {
    if (nt < 2 || !dec_down_fits(m, nt)) return HY_EUNSUPPORTED_TYPE;
    const int ng = m.ff / 256;
    int rpw = 1;
    while (rpw < 4 && (m.n + DEC_DN_WAVES * rpw - 1) / (DEC_DN_WAVES * rpw) > DEC_DN_BLOCKS) ++rpw;
    dim3 grid((m.n + DEC_DN_WAVES * rpw - 1) / (DEC_DN_WAVES * rpw), 1);
    const int np = (ng + 7) / 8, q8 = 8 / ng, r8 = 8 % ng;   // passes of 8 spans (each against every token)
#define HY_SDN(NN) hipLaunchKernelGGL((k_dec_down<TT, NN, true>), grid, dim3(64 * DEC_DN_WAVES), 0, s, m, h, ids, wts, nt, nullptr, nullptr, out, 0, q8, r8, nullptr, rpw)
    HY_DEC_SWITCH(m.td, {
        if (np <= 2) HY_SDN(2);
        else if constexpr (TT != IQ2_XS) HY_SDN(4);
        else if (np <= 4) HY_SDN(4); else HY_SDN(8);
        return check_launch("hy_moe_shared_down");
    });
#undef HY_SDN
}

} // namespace hy
