// Routing of one token (the contract of k_route, src/kernels4.cu:297-344): softmax over the first ne logits, top-k
// by probability with ties to the lower expert id, weights renormalised over the selected in selection order, the
// shared-expert gate sigmoid(logit ne).  Two implementations with identical bits: one wave (k rounds of wave
// argmax over each lane's sorted candidates), and eight waves for up to 128 experts (ranks).
#pragma once
#include "hy_common.cuh"

namespace hy {

__device__ __forceinline__ void wave_lds_sync() {   // a wave's own LDS writes, visible to its other lanes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bool rt_better2(float a, int ia, float b, int ib) { return (a > b) | ((a == b) & (ia < ib)); }   // no short circuit: no branches

// one token's logits in a wave: expert e in lane e % 64, slot e / 64; -inf / index 0x7fffffff past ne
template <int V>
__device__ __forceinline__ void route_load(const float *l, int ne, float (&v)[V], int (&vi)[V]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int e = lane + 64 * i;
        v[i] = e < ne ? l[e] : -__builtin_huge_valf();
        vi[i] = e < ne ? e : 0x7fffffff;
    }
}
// the logits -> probabilities of k_route: max, exp, the contract's sum (slot order, then the xor butterfly),
// p = v / s; -1 for the empty slots
template <int V>
__device__ __forceinline__ void route_probs(float (&v)[V], const int (&vi)[V], int ne) {
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < V; ++i) mx = fmaxf(mx, v[i]);
    mx = wave_max(mx);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i)
        if (vi[i] < ne) { v[i] = hy_expf(v[i] - mx); acc = acc + v[i]; }
    const float s = wave_sum_xor(acc);
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = vi[i] < ne ? v[i] / s : -1.0f;
}

// sort each lane's V candidates best first (rt_better2), then k rounds of wave argmax over the lanes' first candidates:
// lane j < k gets the j-th best (value selw, index seli), every lane tot = the selected values summed in selection
// order; a lane whose candidate is taken moves its next one up (the emptied slot gets `empty`)
template <int V>
__device__ __forceinline__ void select_sorted(float (&v)[V], int (&vi)[V], int k, float empty, float &selw, int &seli, float &tot) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 1; i < V; ++i)
#pragma unroll
        for (int j = i; j > 0; --j)
            if (rt_better2(v[j], vi[j], v[j - 1], vi[j - 1])) {
                const float tv = v[j]; v[j] = v[j - 1]; v[j - 1] = tv;
                const int ti = vi[j]; vi[j] = vi[j - 1]; vi[j - 1] = ti;
            }
    selw = 0.0f; tot = 0.0f; seli = 0;
    for (int j = 0; j < k; ++j) {
        float bv = v[0];
        int bi = vi[0];
        wave_best(bv, bi, rt_better2);
        if (lane == j) { selw = bv; seli = bi; }
        tot = tot + bv;
        if (vi[0] == bi) {
#pragma unroll
            for (int i = 0; i < V - 1; ++i) { v[i] = v[i + 1]; vi[i] = vi[i + 1]; }
            v[V - 1] = empty; vi[V - 1] = 0x7fffffff;
        }
    }
}

// softmax / top-k of one token by one wave, the contract of k_route: k rounds of wave argmax over the lanes'
// sorted candidates
template <int V>
__device__ void route_wave(const float *l, int ne, int k, int *ids, float *wts, float *sg) {
    const int lane = threadIdx.x & 63;
    float v[V];
    int vi[V];
    route_load<V>(l, ne, v, vi);
    route_probs<V>(v, vi, ne);
    float selw, tot;
    int seli;
    select_sorted<V>(v, vi, k, -1.0f, selw, seli, tot);
    if (lane < k) { ids[lane] = seli; wts[lane] = selw / tot; }
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
    int li[V];
    route_load<V>(lg, ne, lv, li);
    lsg = (wave == 0 && want_sg) ? lg[ne] : 0.0f;
    float *my_l = s_l[wave];
#pragma unroll
    for (int i = 0; i < V; ++i) my_l[lane + 64 * i] = lv[i];
    wave_lds_sync();
    const int c = lane / LPE, q = lane % LPE, e = wave * CH + c;
    // rank of expert e under `vals` (index convention of route_load: past ne -> 0x7fffffff)
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
        route_probs<V>(v, li, ne);
#pragma unroll
        for (int i = 0; i < V; ++i) s_p[lane + 64 * i] = v[i];
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
