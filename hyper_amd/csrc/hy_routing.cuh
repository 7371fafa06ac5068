// Routing of one token (the contract of k_route, src/kernels4.cu:297-344): softmax over the first ne logits, top-k
// by probability with ties to the lower expert id, weights renormalised over the selected in selection order, the
// shared-expert gate sigmoid(logit ne).  Two implementations with identical bits: one wave (a threshold that keeps
// at most 64 candidates, then ranks by counting among them), and eight waves for up to 128 experts (ranks).
#pragma once
#include "hy_common.cuh"

namespace hy {

__device__ __forceinline__ void wave_lds_sync() {   // a wave's own LDS writes, visible to its other lanes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bool rt_better2(float a, int ia, float b, int ib) { return (a > b) | ((a == b) & (ia < ib)); }   // no short circuit: no branches

// lanes below this one whose bit is set in m
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return (int) __builtin_amdgcn_mbcnt_hi((uint32_t) (m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t) m, 0u));
}

// A float as an unsigned key with the same order (-0 as +0; NaN below every number, so it is never preferred).
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
    return f != f ? 0u : ((u >> 31) ? ~u : (u | 0x80000000u));
}

// The k-th largest of the keys held by the lanes with on = true (k <= their number): the largest t with at least k
// keys >= t, built bit by bit from the top (one ballot a bit and key slot).
template <int V>
__device__ __forceinline__ uint32_t wave_kth_key(const uint32_t (&u)[V], const bool (&on)[V], int k) {
    uint32_t t = 0;
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = t | (1u << b);
        int n = 0;
#pragma unroll
        for (int i = 0; i < V; ++i) n += __popcll(__ballot(on[i] && u[i] >= c));
        if (n >= k) t = c;   // wave-uniform
    }
    return t;
}

// Top k (1 <= k <= 64, k <= ne) of a wave's keys, best first by (key descending, index ascending); element
// e = lane + 64 i sits in slot i and exists below ne.  Lane r < k gets the index of rank r and its `val`.
//  1. A lower bound of the k-th largest key: the k-th largest of the lanes' maxima (those are k of the keys).
//     Every element of the top k lies at or above it; when at most 64 elements do (the usual case), they are the
//     candidates.  Otherwise the bound is the k-th largest key itself (ballots over all slots), and the candidates
//     are the elements above it and, at it, the lowest indices up to k in all.
//  2. The candidates are gathered into LDS in index order and each one's rank is the number of candidates before
//     it in the order: a larger key, or the same key earlier in the gather (a lower index).
template <int V>
__device__ void wave_topk(const float (&key)[V], const float (&val)[V], int ne, int k, int &e_out, float &v_out) {
    __shared__ uint32_t c_key[64];
    __shared__ int c_idx[64];
    __shared__ float c_val[64];
    __shared__ int r_idx[64];
    __shared__ float r_val[64];
    const int lane = threadIdx.x & 63;
    uint32_t u[V], lmax = 0;
    bool ok[V], lane_on = false;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        ok[i] = lane + 64 * i < ne;
        u[i] = ok[i] ? order_key(key[i]) : 0u;
        if (ok[i]) { lmax = u[i] > lmax ? u[i] : lmax; lane_on = true; }
    }
    const uint32_t lmaxv[1] = {lmax};
    const bool lonv[1] = {lane_on};
    uint32_t th = wave_kth_key<1>(lmaxv, lonv, k);
    int n_at = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) n_at += __popcll(__ballot(ok[i] && u[i] >= th));
    int quota = 64;   // elements equal to the bound that may be taken (all of them on the first path)
    if (n_at > 64) {
        th = wave_kth_key<V>(u, ok, k);
        int n_gt = 0;
#pragma unroll
        for (int i = 0; i < V; ++i) n_gt += __popcll(__ballot(ok[i] && u[i] > th));
        quota = k - n_gt;
    }
    int n_c = 0, eq_seen = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const bool gt = ok[i] && u[i] > th, eq = ok[i] && u[i] == th;
        const uint64_t meq = __ballot(eq);
        const bool take = gt || (eq && eq_seen + lanes_below(meq) < quota);
        eq_seen += __popcll(meq);
        const uint64_t mt = __ballot(take);
        if (take) {
            const int at = n_c + lanes_below(mt);
            c_key[at] = u[i]; c_idx[at] = lane + 64 * i; c_val[at] = val[i];
        }
        n_c += __popcll(mt);
    }
    wave_lds_sync();
    const uint32_t my_k = lane < n_c ? c_key[lane] : 0u;
    int rank = 0;
    for (int m = 0; m < n_c; ++m) {
        const uint32_t km = (uint32_t) __builtin_amdgcn_readlane((int) my_k, m);
        rank += (km > my_k) | ((km == my_k) & (m < lane));
    }
    if (lane < n_c && rank < k) { r_idx[rank] = c_idx[lane]; r_val[rank] = c_val[lane]; }
    wave_lds_sync();
    e_out = lane < k ? r_idx[lane] : 0;
    v_out = lane < k ? r_val[lane] : 0.0f;
}

// One token's logits into a wave: expert lane + 64 i in slot i, -inf past ne.
template <int V>
__device__ __forceinline__ void load_logits(const float *l, int ne, float (&x)[V]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < V; ++i) x[i] = lane + 64 * i < ne ? l[lane + 64 * i] : -__builtin_huge_valf();
}
// Probabilities in place of the logits of load_logits: m = their max; v = expf(l - m); the sum over each lane's
// slots in slot order, then across the wave by the xor butterfly (the contract's order); p = v / sum.  Slots past
// ne get 0 (wave_topk leaves them out by index).
template <int V>
__device__ __forceinline__ void softmax_wave(float (&p)[V], int ne) {
    const int lane = threadIdx.x & 63;
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < V; ++i) m = fmaxf(m, p[i]);
    m = wave_max(m);
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const float v = lane + 64 * i < ne ? hy_expf(p[i] - m) : 0.0f;
        if (lane + 64 * i < ne) part = part + v;
        p[i] = v;
    }
    const float sum = wave_sum_xor(part);
#pragma unroll
    for (int i = 0; i < V; ++i) p[i] = lane + 64 * i < ne ? p[i] / sum : 0.0f;
}

// softmax / top-k of one token by one wave (the contract of k_route); the weights are the selected probabilities
// over their sum taken in selection order
template <int V>
__device__ void route_wave(const float *l, int ne, int k, int *ids, float *wts, float *sg) {
    const int lane = threadIdx.x & 63;
    float p[V];
    load_logits<V>(l, ne, p);
    softmax_wave<V>(p, ne);
    int e_r;
    float p_r;
    wave_topk<V>(p, p, ne, k, e_r, p_r);
    float tot = 0.0f;
    for (int r = 0; r < k; ++r) tot = tot + readlane_f(p_r, r);
    if (lane < k) { ids[lane] = e_r; wts[lane] = p_r / tot; }
    if (lane == 0 && sg) sg[0] = 1.0f / (1.0f + hy_expf(-l[ne]));
}


// Eight waves route one token of up to 128 experts (V <= 2).  p = softmax(l) is monotone in l, so the order of
// k_route (p descending, then the lower index) is the order of the logits unless two probabilities round to the
// same value.  Every wave ranks 8 V experts by logit (4 / V lanes per expert, each against 16 V^2 experts, the
// counts summed with DPP) while wave 0 computes the probabilities; after one block barrier every wave reads the
// k + 1 best by logit and, if their probabilities fall strictly (the usual case), the logit order is the
// contract's; else the ranking is redone on the probabilities (a block-uniform branch with a second barrier).
// Out, in every wave: lane r < k holds selection r (er, its probability pr), tot = the selected probabilities
// summed in selection order (weight r = pr / tot), lsg = logit ne (if want_sg).  `pre` runs in every thread just
// before the first barrier (the caller's LDS writes that share it).  Needs a block of exactly 8 waves.
template <int V, class Pre>
__device__ __forceinline__ void route_rank8(const float *lg, int ne, int k, bool want_sg, int &er, float &pr, float &tot, float &lsg, Pre pre) {
    static_assert(V <= 2, "up to 128 experts");
    constexpr int CH = 8 * V, LPE = 64 / CH, VPL = 64 * V / LPE;   // experts per wave, lanes per expert, values per lane
    __shared__ __align__(16) float s_l[8][64 * V];   // each wave's copy of the logits
    __shared__ __align__(16) float s_p[64 * V];
    __shared__ int s_sel[2][65];                     // experts by logit rank (0..k), by probability rank
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float lv[V];
    load_logits<V>(lg, ne, lv);
    lsg = (wave == 0 && want_sg) ? lg[ne] : 0.0f;
    float *my_l = s_l[wave];
#pragma unroll
    for (int i = 0; i < V; ++i) my_l[lane + 64 * i] = lv[i];
    wave_lds_sync();
    const int c = lane / LPE, q = lane % LPE, e = wave * CH + c;
    // rank of expert e under `vals` (experts past ne rank as index 0x7fffffff)
    auto rank_of = [&](const float *vals) {
        const float ve = vals[e];
        const int ie = e < ne ? e : 0x7fffffff;
        float w[VPL];
#pragma unroll
        for (int u = 0; u < VPL; u += 4) {
            const float4 f4 = *(const float4 *) (vals + q * VPL + u);
            w[u] = f4.x; w[u + 1] = f4.y; w[u + 2] = f4.z; w[u + 3] = f4.w;
        }
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < VPL; ++u) {
            const int iu = q * VPL + u < ne ? q * VPL + u : 0x7fffffff;
            cnt += rt_better2(w[u], iu, ve, ie) ? 1 : 0;
        }
        cnt += dpp_i<DPP_XOR1>(cnt);
        cnt += dpp_i<DPP_XOR2>(cnt);
        if constexpr (LPE == 8) cnt += dpp_i<DPP_HALF_MIRROR>(cnt);
        return cnt;
    };
    const int rl = rank_of(my_l);
    if (q == 0 && e < ne && rl <= k) s_sel[0][rl] = e;
    if (wave == 0) {
        float v[V];
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = lv[i];
        softmax_wave<V>(v, ne);
#pragma unroll
        for (int i = 0; i < V; ++i) s_p[lane + 64 * i] = lane + 64 * i < ne ? v[i] : -1.0f;
    }
    pre();
    lds_barrier();
    // lane r <= k: the expert of logit rank r (ranks stop at ne - 1; a stale entry, possible only with NaN logits, is
    // clamped to a valid index)
    er = lane <= k && lane < ne ? s_sel[0][lane] : 0;
    er = (unsigned) er < (unsigned) ne ? er : 0;
    pr = lane <= k && lane < ne ? s_p[er] : 0.0f;
    const float pn = __shfl_down(pr, 1);
    const bool tie = k < 64 ? (lane < k && lane + 1 < ne && !(pr > pn)) : true;
    if (__ballot(tie)) {   // block-uniform: every wave read the same LDS
        const int rp = rank_of(s_p);
        if (q == 0 && e < ne && rp < k) s_sel[1][rp] = e;
        lds_barrier();
        er = lane < k ? s_sel[1][lane] : 0;
        er = (unsigned) er < (unsigned) ne ? er : 0;
        pr = lane < k ? s_p[er] : 0.0f;
    }
    tot = 0.0f;
    for (int r = 0; r < k; ++r) tot = tot + readlane_f(pr, r);   // selection order
}

} // namespace hy
