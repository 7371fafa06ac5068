// One MoE layer's decode step behind a single C entry point: the per-layer sequence of the reference engine
// (src/engine4.cu:807-890: router GEMV, moe_route, moe_gate_up, moe_down, moe_reduce, with the shared expert of
// src/engine4.cu:795-804) on this library's three decode launches, its intermediates in a caller workspace.
#include "hy_internal.h"

#include <hip/hip_runtime.h>

#include <mutex>

namespace hy {

constexpr int DECODE_MAX_ROWS = 64;   // decode / verify rows per call (prefill takes the grouped GEMMs)

// the shared expert's pair tables: expert 0 with weight 1 for every row (the "ids" and "wts" of a k = 1 layer)
__device__ int32_t g_shared_ids[DECODE_MAX_ROWS];   // zero-initialised
__device__ float g_shared_wts[DECODE_MAX_ROWS] = {
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};

constexpr int MAX_DEVICES = 64;
struct SharedTables { const int32_t *ids; const float *wts; };
static SharedTables g_tables[MAX_DEVICES];
static std::once_flag g_tables_once[MAX_DEVICES];
static int g_tables_rc[MAX_DEVICES];

// the device addresses of the shared-expert tables on the current device (each device holds its own copy)
static int shared_tables(SharedTables &out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) { set_error("hy_moe_decode: no current device"); return HY_EHIP; }
    std::call_once(g_tables_once[dev], [dev] {
        void *a = nullptr, *b = nullptr;
        hipError_t e = hipGetSymbolAddress(&a, HIP_SYMBOL(g_shared_ids));
        if (e == hipSuccess) e = hipGetSymbolAddress(&b, HIP_SYMBOL(g_shared_wts));
        g_tables_rc[dev] = e == hipSuccess ? HY_OK : HY_EHIP;
        if (e == hipSuccess) g_tables[dev] = {(const int32_t *) a, (const float *) b};
    });
    if (g_tables_rc[dev] != HY_OK) { set_error("hy_moe_decode: hipGetSymbolAddress of the shared-expert tables failed"); return HY_EHIP; }
    out = g_tables[dev];
    return HY_OK;
}

// the shared expert's down for nt tokens: one pass over its weights for 2 or more tokens, else (or beyond that
// kernel's limits) the fused down with k = 1, else the R-row kernel
static int shared_down(const hy_moe_dev &S, const float *sh_h, const SharedTables &T, float *shexp, int nt, hipStream_t s) {
    int rc = launch_shared_down(S, sh_h, T.ids, T.wts, shexp, nt, s);
    if (rc == HY_EUNSUPPORTED_TYPE) rc = launch_dec_down(S, sh_h, T.ids, T.wts, 1, nullptr, nullptr, shexp, nt, s);
    if (rc == HY_EUNSUPPORTED_TYPE) rc = launch_down_reduce(S, sh_h, T.ids, T.wts, 1, nullptr, nullptr, shexp, nt, s);
    return rc;
}

// workspace layout: each piece 256-byte aligned
struct DecodeLayout {
    size_t logits, ids, wts, sg, xq, h, hq, sh_h, sh_y, total;
};
static size_t up256(size_t v) { return (v + 255) & ~(size_t) 255; }
static DecodeLayout decode_layout(const hy_moe_dev &m, int rows, int k, const hy_moe_dev *S, int nt) {
    DecodeLayout L{};
    size_t o = 0;
    auto take = [&](size_t bytes) { const size_t at = o; o += up256(bytes); return at; };
    const int vg = vec_dot_type(m.tg);
    const size_t xq_row = vg == Q8_K ? (size_t) (m.n / 256) * Q8K_BYTES : (size_t) (m.n / 32) * Q8_0_BYTES;
    L.logits = take((size_t) nt * rows * 4);
    L.ids = take((size_t) nt * k * 4);
    L.wts = take((size_t) nt * k * 4);
    L.sg = take((size_t) nt * 4);
    L.xq = take((size_t) nt * xq_row);
    L.h = take((size_t) nt * k * m.ff * 4);
    L.hq = vec_dot_type(m.td) == Q8_0 ? take((size_t) nt * k * (m.ff / 32) * Q8_0_BYTES) : 0;   // the hidden as Q8_0 rows
    L.sh_h = S ? take((size_t) nt * S->ff * 4) : 0;
    L.sh_y = S ? take((size_t) nt * m.n * 4) : 0;
    L.total = o;
    return L;
}

// argument checks shared by the workspace and the no-workspace entry points
int decode_args(const char *what, const hy_moe_dev *m, const float *W_r, int rows, const float *x, int xs, int k, const hy_moe_dev *S,
                const float *out, int nt) {
    if (!m || !W_r || !x || !out || nt < 0) { set_error("%s: bad argument", what); return HY_EINVAL; }
    const int E = m->n_expert;
    if (E <= 0 || E > 1024) { set_error("%s: n_expert %d out of range (1..1024)", what, E); return HY_EBAD_SHAPE; }
    if (rows != E && rows != E + 1) { set_error("%s: router rows %d must be n_expert (%d) or n_expert + 1 (shared-expert gate)", what, rows, E); return HY_EBAD_SHAPE; }
    if (k <= 0 || k > 64 || k > E) { set_error("%s: k = %d out of range", what, k); return HY_EBAD_SHAPE; }
    if (nt > DECODE_MAX_ROWS) { set_error("%s: %d rows exceed %d (prefill rows take the grouped GEMMs)", what, nt, DECODE_MAX_ROWS); return HY_EBAD_SHAPE; }
    if (xs % 4 || ((uintptr_t) x & 15) || ((uintptr_t) W_r & 15)) { set_error("%s: W_r and x rows must be 16-byte aligned", what); return HY_EBAD_SHAPE; }
    if (S && (S->n != m->n || S->n_expert < 1)) { set_error("%s: the shared expert's n (%d) differs from the layer's (%d)", what, S->n, m->n); return HY_EBAD_SHAPE; }
    return HY_OK;
}

// the step itself on a workspace of at least decode_layout(...).total bytes (256-byte aligned)
int run_decode(const hy_moe_dev &m, const float *W_r, int rows, const float *x, int xs, const float *bias, int bias_stride, int k,
               const hy_moe_dev *S, float *out, int residual, int nt, uint8_t *ws, hipStream_t s) {
    if (nt == 0) return HY_OK;
    const DecodeLayout L = decode_layout(m, rows, k, S, nt);
    float *logits = (float *) (ws + L.logits), *wts = (float *) (ws + L.wts), *sg = (float *) (ws + L.sg), *h = (float *) (ws + L.h);
    int32_t *ids = (int32_t *) (ws + L.ids);
    uint8_t *xq = ws + L.xq;
    const int E = m.n_expert;
    const bool gate_logit = rows > E;
    int rc = launch_router_q8(W_r, rows, m.n, x, xs, bias, bias_stride, logits, rows, vec_dot_type(m.tg), xq, nt, s);
    if (rc) return rc;
    float *shexp = nullptr;
    if (S) {   // the always-on expert: a k = 1 layer whose only pair is expert 0 with weight 1
        SharedTables T;
        if ((rc = shared_tables(T))) return rc;
        float *sh_h = (float *) (ws + L.sh_h);
        shexp = (float *) (ws + L.sh_y);
        // from the Q8 rows of x when the shared expert's gate type takes the same activation type, else from x
        if (vec_dot_type(S->tg) == vec_dot_type(m.tg)) {
            rc = launch_shared_gate_up(*S, xq, sh_h, nt, s);   // several tokens: one pass over the weights
            if (rc == HY_EUNSUPPORTED_TYPE) rc = launch_fixed_gate_up(*S, xq, sh_h, nt, s);
        } else {
            rc = launch_gate_up(*S, x, xs, T.ids, 1, sh_h, nt, s, nullptr, nullptr);
        }
        if (rc) return rc;
        rc = shared_down(*S, sh_h, T, shexp, nt, s);
        if (rc) return rc;
    }
    // down types with a Q8_0 partner: gate/up also writes the hidden as Q8_0 rows, which the down kernel reads (shapes
    // beyond either kernel's limits take the fp32 hidden)
    uint8_t *hq = vec_dot_type(m.tg) == Q8_0 && dec_down_takes_q8(m, k) ? ws + L.hq : nullptr;
    rc = launch_route_gate_up(m, logits, rows, E, k, xq, ids, wts, gate_logit ? sg : nullptr, h, nt, s, hq);
    if (rc == HY_EUNSUPPORTED_TYPE && hq) {
        hq = nullptr;
        rc = launch_route_gate_up(m, logits, rows, E, k, xq, ids, wts, gate_logit ? sg : nullptr, h, nt, s);
    }
    if (rc) return rc;
    const float *g = gate_logit ? sg : nullptr;
    rc = launch_dec_down(m, h, ids, wts, k, shexp, g, out, nt, s, residual ? 1 : 0, hq);
    if (rc == HY_EUNSUPPORTED_TYPE) rc = launch_down_reduce(m, h, ids, wts, k, shexp, g, out, nt, s, residual ? 1 : 0);
    return rc;
}

size_t decode_ws_bytes(const hy_moe_dev &m, int rows, int k, const hy_moe_dev *S, int nt) { return decode_layout(m, rows, k, S, nt).total; }

// ---- the decode step without a workspace argument: its intermediates in `scratch`, a file-scope device array that
// every device running the library holds until the process ends (1 MiB: e.g. 8 rows of a d_model 7168, top-6, ff 2048
// layer with a shared expert need 0.75 MiB).  In host code `scratch` names a host-side stand-in, not device memory:
// kernels get the per-device address that hipGetSymbolAddress returns, taken once per device with that device current.
constexpr size_t DECODE_SCRATCH_BYTES = 1u << 20;
__device__ __align__(256) uint8_t scratch[DECODE_SCRATCH_BYTES];

static uint8_t *g_scratch[MAX_DEVICES];
static std::once_flag g_scratch_once[MAX_DEVICES];
static int g_scratch_rc[MAX_DEVICES];

static int scratch_ptr(uint8_t *&out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) { set_error("hy_moe_decode_noalloc: no current device"); return HY_EHIP; }
    std::call_once(g_scratch_once[dev], [dev] {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_rc[dev] = e == hipSuccess && p ? HY_OK : HY_EHIP;
        if (g_scratch_rc[dev] == HY_OK) g_scratch[dev] = (uint8_t *) p;
    });
    if (g_scratch_rc[dev] != HY_OK) { set_error("hy_moe_decode_noalloc: hipGetSymbolAddress of the scratch array failed on device %d", dev); return HY_EHIP; }
    out = g_scratch[dev];
    return HY_OK;
}

} // namespace hy

using namespace hy;

extern "C" {

int hy_moe_shared_down(const hy_moe_dev *m, const float *h, float *out, int nt, hipStream_t s) {
    int rc = check_dev_decode(m, nullptr, "hy_moe_shared_down");
    if (rc) return rc;
    if (!h || !out || nt < 0 || nt > DECODE_MAX_ROWS) { set_error("hy_moe_shared_down: bad argument (nt %d, at most %d)", nt, DECODE_MAX_ROWS); return HY_EINVAL; }
    if (nt == 0) return HY_OK;
    SharedTables T;
    if ((rc = shared_tables(T))) return rc;
    return shared_down(*m, h, T, out, nt, s);
}

size_t hy_moe_decode_ws_bytes(const hy_moe_dev *m, int rows, int k, const hy_moe_dev *shared, int nt) {
    if (!m || nt < 0 || k <= 0 || rows <= 0) return 0;
    return decode_ws_bytes(*m, rows, k, shared, nt);
}

int hy_moe_decode(const hy_moe_dev *m, const float *W_r, int rows, const float *x, int xs, const float *bias, int bias_stride, int k,
                  const hy_moe_dev *shared, float *out, int residual, int nt, void *ws, size_t ws_bytes, hipStream_t s) {
    int rc = decode_args("hy_moe_decode", m, W_r, rows, x, xs, k, shared, out, nt);
    if (rc) return rc;
    if ((rc = check_dev_decode(m, shared, "hy_moe_decode"))) return rc;
    const size_t need = decode_ws_bytes(*m, rows, k, shared, nt);
    if (!ws || ((uintptr_t) ws & 255) || ws_bytes < need) {
        set_error("hy_moe_decode: workspace of %zu bytes at %p; %zu bytes, 256-byte aligned, needed", ws_bytes, ws, need);
        return HY_EINVAL;
    }
    return run_decode(*m, W_r, rows, x, xs, bias, bias_stride, k, shared, out, residual, nt, (uint8_t *) ws, s);
}

int hy_moe_decode_noalloc(const hy_moe_dev *m, const float *W_r, int rows, const float *x, int xs, const float *bias, int bias_stride, int k,
                          const hy_moe_dev *shared, float *out, int residual, int nt, hipStream_t s) {
    int rc = decode_args("hy_moe_decode_noalloc", m, W_r, rows, x, xs, k, shared, out, nt);
    if (rc) return rc;
    if ((rc = check_dev_decode(m, shared, "hy_moe_decode_noalloc"))) return rc;
    const size_t need = decode_ws_bytes(*m, rows, k, shared, nt);
    if (need > DECODE_SCRATCH_BYTES) {
        set_error("hy_moe_decode_noalloc: %d rows of this layer need %zu bytes of scratch, more than its %zu", nt, need, DECODE_SCRATCH_BYTES);
        return HY_EBAD_SHAPE;
    }
    uint8_t *ws = nullptr;
    if ((rc = scratch_ptr(ws))) return rc;
    return run_decode(*m, W_r, rows, x, xs, bias, bias_stride, k, shared, out, residual, nt, ws, s);
}

} // extern "C"
