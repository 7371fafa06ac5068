// A C++ caller of libhymoe through include/hymoe.hpp, as the reference's engine would call it: experts uploaded from
// GGUF-layout bytes, one decode step (moe_decode on a workspace, then moe_decode_noalloc), and one prefill step through
// the reference-signature sequence (gemv_f32, moe_route, moe_order, q8_quantize, moe_gemm_gate_up, q8_quantize,
// moe_gemm_down, moe_reduce); and the CPU path's host quantizer q8k_test_quantize on std::vector data (src/cpu_moe.h:46,
// called as tools/cpumoebench.cu:68 calls it).  Reads its inputs from argv[1], writes the outputs to argv[2]; the test
// compares them with the CPU oracle.
//
// input:  int32 E, d, ff, k, nt_dec, nt_pre, tg, td; uint64 gb, db; gate[E gb], up[E gb], down[E db] (GGUF rows);
//         float W_r[E][d], x_dec[nt_dec][d], x_pre[nt_pre][d]
// output: float out_dec[nt_dec][d], out_dec_noalloc[nt_dec][d], out_pre[nt_pre][d]; int32 ids_pre[nt_pre][k];
//         Q8_K blocks of x_pre (nt_pre d / 256 x 292 bytes, from the host quantizer)
#include "hymoe.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define HIP_OK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_)); std::exit(3); } } while (0)

template <class T> static T *dev_alloc(size_t n) { T *p = nullptr; HIP_OK(hipMalloc(&p, n * sizeof(T) + 256)); return p; }
template <class T> static T *dev_copy(const std::vector<T> &v) { T *p = dev_alloc<T>(v.size()); HIP_OK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice)); return p; }
template <class T> static std::vector<T> host_copy(const T *p, size_t n) { std::vector<T> v(n); HIP_OK(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost)); return v; }

int main(int argc, char **argv) {
    if (argc != 3) { std::fprintf(stderr, "usage: moe_step in.bin out.bin\n"); return 2; }
    FILE *f = std::fopen(argv[1], "rb");
    if (!f) { std::perror(argv[1]); return 2; }
    int32_t hdr[8];
    uint64_t gbdb[2];
    if (std::fread(hdr, 4, 8, f) != 8 || std::fread(gbdb, 8, 2, f) != 2) { std::fprintf(stderr, "short header\n"); return 2; }
    const int E = hdr[0], d = hdr[1], ff = hdr[2], k = hdr[3], ntd = hdr[4], ntp = hdr[5], tg = hdr[6], td = hdr[7];
    const size_t gb = gbdb[0], db = gbdb[1];
    std::vector<uint8_t> gate(E * gb), up(E * gb), down(E * db);
    std::vector<float> W((size_t) E * d), xd((size_t) ntd * d), xp((size_t) ntp * d);
    bool ok = std::fread(gate.data(), 1, gate.size(), f) == gate.size() && std::fread(up.data(), 1, up.size(), f) == up.size() &&
              std::fread(down.data(), 1, down.size(), f) == down.size() && std::fread(W.data(), 4, W.size(), f) == W.size() &&
              std::fread(xd.data(), 4, xd.size(), f) == xd.size() && std::fread(xp.data(), 4, xp.size(), f) == xp.size();
    std::fclose(f);
    if (!ok) { std::fprintf(stderr, "short input\n"); return 2; }

    try {
        hymoe::ExpertTensors t{gate.data(), up.data(), down.data(), gb, db, E, tg, td};
        std::vector<int> slot(E);
        for (int e = 0; e < E; ++e) slot[e] = e;
        hymoe::MoeDev m = hymoe::upload_experts(t, slot, ff, d, 0.0f);
        hipStream_t s;
        HIP_OK(hipStreamCreate(&s));
        float *Wd = dev_copy(W), *xdd = dev_copy(xd), *xpd = dev_copy(xp);

        // decode: one call on a workspace, then the no-allocation variant
        const size_t wsb = hymoe::moe_decode_ws_bytes(m, E, k, nullptr, ntd);
        uint8_t *ws = nullptr;
        HIP_OK(hipMalloc(&ws, wsb));
        float *od = dev_alloc<float>((size_t) ntd * d), *on = dev_alloc<float>((size_t) ntd * d);
        hymoe::moe_decode(m, Wd, E, xdd, d, nullptr, 0, k, nullptr, od, false, ntd, ws, wsb, s);
        hymoe::moe_decode_noalloc(m, Wd, E, xdd, d, nullptr, 0, k, nullptr, on, false, ntd, s);

        // prefill through the reference-signature calls
        const int P = ntp * k, vg = hy_vec_dot_type(tg), vd = hy_vec_dot_type(td);
        float *logits = dev_alloc<float>((size_t) ntp * E), *wts = dev_alloc<float>(P), *h = dev_alloc<float>((size_t) P * ff);
        float *y = dev_alloc<float>((size_t) P * d), *op = dev_alloc<float>((size_t) ntp * d);
        int *ids = dev_alloc<int>(P), *order = dev_alloc<int>(P), *order_n = dev_alloc<int>(2), *egrp = dev_alloc<int>(3 * E);
        uint8_t *xq = dev_alloc<uint8_t>((size_t) ntp * hy_q8_row_bytes(vg, d)), *hq = dev_alloc<uint8_t>((size_t) P * hy_q8_row_bytes(vd, ff));
        hymoe::gemv_f32(Wd, E, d, xpd, d, logits, E, ntp, s);
        hymoe::moe_route(logits, E, E, k, ids, wts, nullptr, ntp, s);
        hymoe::moe_order(m, ids, P, E, order, order_n, s, egrp);
        hymoe::q8_quantize(vg, xpd, d, d, ntp, xq, s);
        const int max_active = E < P ? E : P;
        hymoe::moe_gemm_gate_up(m, xq, k, P, order, order_n, egrp, max_active, h, s);
        hymoe::q8_quantize(vd, h, ff, ff, P, hq, s);
        hymoe::moe_gemm_down(m, hq, P, order, order_n, egrp, max_active, wts, y, s);
        hymoe::moe_reduce(nullptr, nullptr, y, k, op, d, ntp, ids, s);
        HIP_OK(hipStreamSynchronize(s));
        // the host quantizer on host vectors, as the reference's quantizer test calls it
        std::vector<uint8_t> xq_host((size_t) ntp * d / 256 * 292);
        hymoe::q8k_test_quantize(xp.data(), xq_host.data(), (int64_t) xp.size());

        FILE *o = std::fopen(argv[2], "wb");
        if (!o) { std::perror(argv[2]); return 2; }
        const auto a = host_copy(od, (size_t) ntd * d), b = host_copy(on, (size_t) ntd * d), c = host_copy(op, (size_t) ntp * d);
        const auto i = host_copy(ids, (size_t) P);
        std::fwrite(a.data(), 4, a.size(), o); std::fwrite(b.data(), 4, b.size(), o);
        std::fwrite(c.data(), 4, c.size(), o); std::fwrite(i.data(), 4, i.size(), o);
        std::fwrite(xq_host.data(), 1, xq_host.size(), o);
        std::fclose(o);
        hymoe::free_experts(m);
        HIP_OK(hipStreamDestroy(s));
    } catch (const std::exception &e) {
        std::fprintf(stderr, "moe_step: %s\n", e.what());
        return 1;
    }
    std::printf("moe_step: done\n");
    return 0;
}
