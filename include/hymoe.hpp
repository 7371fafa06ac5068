// C++ face of libhymoe with the reference's expert-compute signatures (hyper src/kernels4.cuh:45-91,
// src/experts.h:20-50): the same function names, argument order and meaning, std::runtime_error on failure
// (the reference throws at the same places, src/kernels4.cu:1926-1927, :1970, :2027-2030, :2066, :2081).
// Header-only over include/hymoe.h; device pointers and the stream are the caller's.
#pragma once
#include "hymoe.h"

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace hymoe {

using MoeDev = hy_moe_dev;                 // src/kernels4.cuh:56-63 (+ n_expert)

inline void check(int rc) {
    if (rc != HY_OK) throw std::runtime_error(std::string("hymoe: ") + hy_last_error());
}

// src/experts.h:20-26 -- one layer's GGUF expert tensors on the host
struct ExpertTensors {
    const uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
    size_t gb = 0, db = 0;
    int E = 0;
    int tg = 0, td = 0;
};
// src/experts.h:50 -- the experts with slot[e] >= 0 copied to their device slots
inline MoeDev upload_experts(const ExpertTensors &t, const std::vector<int> &slot, int ff, int n, float clamp) {
    if ((int) slot.size() != t.E) throw std::runtime_error("upload_experts: slot table size != E");
    hy_expert_tensors c{t.gate, t.up, t.down, t.gb, t.db, t.E, t.tg, t.td};
    MoeDev m{};
    check(hy_upload_experts(&c, slot.data(), ff, n, clamp, &m));
    return m;
}
inline void free_experts(MoeDev &m) { check(hy_free_experts(&m)); }

// src/gguf.h:22-32 -- a tensor of a GGUF file (host data inside the mapping)
struct GTensor {
    std::string name;
    int type = 0;
    std::vector<int64_t> ne;
    const uint8_t *data = nullptr;
    size_t nbytes = 0;
};
// src/gguf.h:38-70 -- a read-only GGUF file (or the shards of a split model), memory-mapped while the object lives
class GGUF {
public:
    explicit GGUF(const std::string &path) { check(hy_gguf_open(path.c_str(), &g_)); }
    ~GGUF() { hy_gguf_close(g_); }
    GGUF(const GGUF &) = delete;
    GGUF &operator=(const GGUF &) = delete;
    bool has(const std::string &key) const { return hy_gguf_has(g_, key.c_str()) != 0; }
    int64_t get_int(const std::string &key) const { int64_t v = 0; check(hy_gguf_get_int(g_, key.c_str(), &v)); return v; }
    int64_t get_int(const std::string &key, int64_t def) const { return has(key) ? get_int(key) : def; }
    double get_float(const std::string &key) const { double v = 0; check(hy_gguf_get_float(g_, key.c_str(), &v)); return v; }
    double get_float(const std::string &key, double def) const { return has(key) ? get_float(key) : def; }
    std::string get_str(const std::string &key) const { const char *v = nullptr; check(hy_gguf_get_str(g_, key.c_str(), &v)); return v; }
    std::vector<int64_t> get_int_arr(const std::string &key) const {
        size_t n = 0;
        check(hy_gguf_get_int_arr(g_, key.c_str(), nullptr, 0, &n));
        std::vector<int64_t> v(n);
        check(hy_gguf_get_int_arr(g_, key.c_str(), v.data(), n, &n));
        return v;
    }
    std::vector<double> get_float_arr(const std::string &key) const {
        size_t n = 0;
        check(hy_gguf_get_float_arr(g_, key.c_str(), nullptr, 0, &n));
        std::vector<double> v(n);
        check(hy_gguf_get_float_arr(g_, key.c_str(), v.data(), n, &n));
        return v;
    }
    std::string arch() const { return hy_gguf_arch(g_); }
    bool tensor(const std::string &name, GTensor &out) const {   // false if missing (GGUF::tensor returns nullptr)
        hy_gguf_tensor_info t;
        if (hy_gguf_tensor(g_, name.c_str(), &t) != HY_OK) return false;
        out = {t.name, t.type, std::vector<int64_t>(t.ne, t.ne + t.n_dims), t.data, t.nbytes};
        return true;
    }
    GTensor need(const std::string &name) const {
        GTensor t;
        if (!tensor(name, t)) throw std::runtime_error("gguf: missing tensor " + name);
        return t;
    }
    const hy_gguf *handle() const { return g_; }

private:
    hy_gguf *g_ = nullptr;
};
// src/experts.h:26 / src/experts.cu:12-22 -- blk.<il>.ffn_{gate,up,down}_exps.weight of E experts
inline ExpertTensors expert_tensors(const GGUF &g, int il, int E) {
    hy_expert_tensors c{};
    check(hy_gguf_expert_tensors(g.handle(), il, E, &c));
    return {c.gate, c.up, c.down, c.gb, c.db, c.E, c.tg, c.td};
}

// src/kernels4.cuh:35
inline void gemv_f32(const float *W, int rows, int k, const float *x, int xs, float *y, int ys, int nt, hipStream_t s,
                     const float *bias = nullptr, int bias_stride = 0) {
    check(hy_gemv_f32(W, rows, k, x, xs, y, ys, nt, bias, bias_stride, s));
}
// src/kernels4.cuh:38 (bf16 router weights; the reference's ys is the output stride here too)
inline void gemv_bf16w(const uint16_t *W, int rows, int k, const float *x, int xs, float *y, int ys, int nt, hipStream_t s,
                       const float *bias = nullptr, int bias_stride = 0) {
    check(hy_gemv_bf16w(W, rows, k, x, xs, y, ys, nt, bias, bias_stride, s));
}
// src/kernels4.cuh:39
inline void bf16_to_f32(const uint16_t *W, size_t n, float *out, hipStream_t s) { check(hy_bf16_to_f32(W, n, out, s)); }
// src/kernels4.cuh:48
inline void moe_route(const float *logits, int ls, int n_expert, int k, int *ids, float *wts, float *sg, int nt, hipStream_t s) {
    check(hy_moe_route(logits, ls, n_expert, k, ids, wts, sg, nt, s));
}
// src/kernels5.cuh:74 -- sigmoid router with a selection bias
inline void moe_route_sig(const float *logits, int ls, const float *bias, int n_expert, int k, float scale, int *ids, float *wts,
                          float *sg, int nt, hipStream_t s) {
    check(hy_moe_route_sig(logits, ls, bias, n_expert, k, scale, ids, wts, sg, nt, s));
}
// src/kernels7.cuh:75 -- sqrt-softplus router with a selection bias
inline void route7(const float *logits, int ls, const float *bias, int n, int k, float scale, int *ids, float *wts, int nt, hipStream_t s) {
    check(hy_moe_route_sqrtsp(logits, ls, bias, n, k, scale, ids, wts, nt, s));
}
// src/kernels4.cuh:67-68
inline void moe_gate_up(const MoeDev &m, const float *x, int xs, const int *ids, int k, float *h, int nt, hipStream_t s,
                        const int *order = nullptr, const int *order_n = nullptr) {
    check(hy_moe_gate_up(&m, x, xs, ids, k, h, nt, s, order, order_n));
}
// src/kernels4.cuh:70-71
inline void moe_down(const MoeDev &m, const float *h, const int *ids, const float *wts, int k, float *y, int nt, hipStream_t s,
                     const int *order = nullptr, const int *order_n = nullptr) {
    check(hy_moe_down(&m, h, ids, wts, k, y, nt, s, order, order_n));
}
// src/kernels4.cuh:74-75
inline void moe_order(const MoeDev &m, const int *ids, int n_pairs, int n_expert, int *order, int *order_n, hipStream_t s,
                      int *egrp = nullptr) {
    check(hy_moe_order(&m, ids, n_pairs, n_expert, order, order_n, s, egrp));
}
// activation quantizer: replaces to_half (src/kernels.cu:2235-2237) ahead of the grouped GEMMs
inline void q8_quantize(int vtype, const float *x, int xs, int n, int nt, void *q, hipStream_t s) {
    check(hy_q8_quantize(vtype, x, xs, n, nt, q, s));
}
// src/kernels4.cuh:77-80 (Q8 activations instead of fp16, fp32 hidden; n_pairs bounds the work items)
inline void moe_gemm_gate_up(const MoeDev &m, const void *xq, int k, int n_pairs, const int *order, const int *order_n, const int *egrp,
                             int max_active, float *h, hipStream_t s) {
    check(hy_moe_gemm_gate_up(&m, xq, k, n_pairs, order, order_n, egrp, max_active, h, s));
}
inline void moe_gemm_down(const MoeDev &m, const void *hq, int n_pairs, const int *order, const int *order_n, const int *egrp,
                          int max_active, const float *wts, float *y, hipStream_t s) {
    check(hy_moe_gemm_down(&m, hq, n_pairs, order, order_n, egrp, max_active, wts, y, s));
}
// src/kernels4.cuh:88-91 (single device: no owner tables, no CPU hand-off)
inline void moe_reduce(const float *shexp, const float *sg, const float *y, int k, float *out, int n, int nt, const int *ids,
                       hipStream_t s) {
    check(hy_moe_reduce(shexp, sg, y, k, out, n, nt, ids, s));
}
// the combine added into the residual in place (moe_reduce, then the engine's residual add, src/engine4.cu:887-895)
inline void moe_reduce_residual(const float *shexp, const float *sg, const float *y, int k, float *resid, int n, int nt, const int *ids,
                                hipStream_t s) {
    check(hy_moe_reduce_residual(shexp, sg, y, k, resid, n, nt, ids, s));
}
inline void moe_down_reduce_residual(const MoeDev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp,
                                     const float *sg, float *resid, int nt, hipStream_t s) {
    check(hy_moe_down_reduce_residual(&m, h, ids, wts, k, shexp, sg, resid, nt, s));
}
inline void moe_down_reduce(const MoeDev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp,
                            const float *sg, float *out, int nt, hipStream_t s) {
    check(hy_moe_down_reduce(&m, h, ids, wts, k, shexp, sg, out, nt, s));
}
// decode: gemv_f32 and the experts' Q8 rows of x in one launch (src/kernels4.cu:1910-1913 + the activation quantizer)
inline void moe_router_q8(const float *W_r, int rows, int kdim, const float *x, int xs, const float *bias, int bias_stride, float *logits,
                          int ls, int vtype, void *xq, int nt, hipStream_t s) {
    check(hy_moe_router_q8(W_r, rows, kdim, x, xs, bias, bias_stride, logits, ls, vtype, xq, nt, s));
}
// the same with bf16 router weights (gemv_bf16w, src/kernels4.cuh:38, + the activation quantizer)
inline void moe_router_q8(const uint16_t *W_r, int rows, int kdim, const float *x, int xs, const float *bias, int bias_stride, float *logits,
                          int ls, int vtype, void *xq, int nt, hipStream_t s) {
    check(hy_moe_router_q8_bf16w(W_r, rows, kdim, x, xs, bias, bias_stride, logits, ls, vtype, xq, nt, s));
}
// decode: moe_route and moe_gate_up (on the Q8 rows) in one launch
inline void moe_route_gate_up(const MoeDev &m, const float *logits, int ls, int n_expert, int k, const void *xq, int *ids, float *wts,
                              float *sg, float *h, int nt, hipStream_t s) {
    check(hy_moe_route_gate_up(&m, logits, ls, n_expert, k, xq, ids, wts, sg, h, nt, s));
}
// the shared expert's decode gate/up from the Q8 rows of x (moe_gate_up with every id 0, k = 1)
inline void moe_shared_gate_up(const MoeDev &m, const void *xq, float *h, int nt, hipStream_t s) {
    check(hy_moe_shared_gate_up(&m, xq, h, nt, s));
}
// moe_route_gate_up that also writes the hidden rows as Q8_0 blocks, and the down + combine that reads them (down types
// whose partner is Q8_0)
inline void moe_route_gate_up_q8(const MoeDev &m, const float *logits, int ls, int n_expert, int k, const void *xq, int *ids, float *wts,
                                 float *sg, float *h, void *hq, int nt, hipStream_t s) {
    check(hy_moe_route_gate_up_q8(&m, logits, ls, n_expert, k, xq, ids, wts, sg, h, hq, nt, s));
}
inline void moe_down_reduce_q8(const MoeDev &m, const void *hq, const int *ids, const float *wts, int k, const float *shexp,
                               const float *sg, float *out, int residual, int nt, hipStream_t s) {
    check(hy_moe_down_reduce_q8(&m, hq, ids, wts, k, shexp, sg, out, residual, nt, s));
}
// one layer's decode step (src/engine4.cu:795-890) on a caller workspace of moe_decode_ws_bytes(...) bytes
inline size_t moe_decode_ws_bytes(const MoeDev &m, int rows, int k, const MoeDev *shared, int nt) {
    return hy_moe_decode_ws_bytes(&m, rows, k, shared, nt);
}
inline void moe_decode(const MoeDev &m, const float *W_r, int rows, const float *x, int xs, const float *bias, int bias_stride, int k,
                       const MoeDev *shared, float *out, bool residual, int nt, void *ws, size_t ws_bytes, hipStream_t s) {
    check(hy_moe_decode(&m, W_r, rows, x, xs, bias, bias_stride, k, shared, out, residual ? 1 : 0, nt, ws, ws_bytes, s));
}
// the same step with no workspace and no allocation (the library's per-GPU scratch array; overlapping calls race)
inline void moe_decode_noalloc(const MoeDev &m, const float *W_r, int rows, const float *x, int xs, const float *bias, int bias_stride,
                               int k, const MoeDev *shared, float *out, bool residual, int nt, hipStream_t s) {
    check(hy_moe_decode_noalloc(&m, W_r, rows, x, xs, bias, bias_stride, k, shared, out, residual ? 1 : 0, nt, s));
}
// src/cpu_moe.h:46 q8k_test_quantize(x, y, k): the CPU expert path's Q8_K quantizer, host buffers in and out,
// synchronous (src/cpu_moe.cpp:35-78; the blocks equal the device quantizer's bit for bit)
inline void q8k_test_quantize(const float *x, void *y, int64_t k) {
    check(hy_q8k_quantize_host(x, y, k));
}
// the same quantizer on device memory, stream-ordered: one row of k values (the kernels' own quantizer)
inline void q8k_quantize_device(const float *x, void *y, int64_t k, hipStream_t s) {
    if (k < 0 || k % 256 || k > 0x7fffff00) throw std::runtime_error("q8k_quantize_device: k must be a multiple of 256 below 2^31");
    check(hy_q8_quantize(HY_Q8_K, x, (int) k, (int) k, 1, y, s));
}
// src/kernels4.cuh:181 test hook
inline void deq_row_test(int type, const uint8_t *row, int n, float *out, hipStream_t s = nullptr) {
    check(hy_dequant_row(type, row, n, out, s));
}

} // namespace hymoe
