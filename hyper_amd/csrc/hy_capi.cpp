// The C ABI (include/hymoe.h): argument validation, error state, and the host-side expert upload.
#include "hy_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace hy {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) { set_error("%s: %s", what, hipGetErrorString(e)); return HY_EHIP; }
    return HY_OK;
}

static bool dot_type(int t) { return t == Q4_K || t == Q5_K || t == Q6_K || t == IQ4_XS || t == IQ2_XS || t == IQ2_XXS || t == IQ4_NL || t == Q8_0 || t == MXFP4 || t == Q5_0 || t == Q5_1 || t == Q2_K || t == Q3_K || t == IQ3_XXS || t == IQ3_S || t == IQ2_S || t == IQ1_S; }
static bool gemm_type(int t) { return dot_type(t); }

// the expert layer descriptor is usable: types, sizes, pointers, row sizes that the kernels assume
static int check_dev(const hy_moe_dev *m, const char *what, bool need_gate, bool need_down) {
    if (!m) { set_error("%s: null hy_moe_dev", what); return HY_EINVAL; }
    if (!m->slot || m->n_expert <= 0) { set_error("%s: slot table missing", what); return HY_EINVAL; }
    if (m->n_local <= 0) { set_error("%s: n_local %d (the expert matrices behind gate/up/down) must be >= 1", what, m->n_local); return HY_EINVAL; }
    if (m->ff <= 0 || m->n <= 0) { set_error("%s: ff %d, n %d", what, m->ff, m->n); return HY_EBAD_SHAPE; }
    // every kernel's grid covers ff and n in whole 256-row / 256-value units (the tiled layout's 16-row tiles, the
    // GEMMs' 64- and 128-row blocks): both are checked whichever matrices the entry point reads
    if (m->n % 256 || m->ff % 256) { set_error("%s: n = %d and ff = %d must be multiples of 256", what, m->n, m->ff); return HY_EBAD_SHAPE; }
    // the kernels read weight bytes in 16-byte pieces and rely on the tiles (16 rows of a span: a multiple of 16
    // bytes, as every expert matrix is) starting 16-byte aligned, so the matrices themselves must
    if (((uintptr_t) m->gate | (uintptr_t) m->up | (uintptr_t) m->down) & 15) { set_error("%s: weight matrices must be 16-byte aligned", what); return HY_EBAD_SHAPE; }
    if (need_gate) {
        if (!dot_type(m->tg)) { set_error("%s: unsupported gate/up type %d", what, m->tg); return HY_EUNSUPPORTED_TYPE; }
        if (!m->gate || !m->up) { set_error("%s: null gate/up", what); return HY_EINVAL; }
        const size_t rb = (size_t) (m->n / block_elems(m->tg)) * block_bytes(m->tg);
        if (m->gate_bytes != rb * (size_t) m->ff) { set_error("%s: gate_bytes %zu != ff * row bytes %zu", what, m->gate_bytes, rb * m->ff); return HY_EBAD_SHAPE; }
    }
    if (need_down) {
        if (!dot_type(m->td)) { set_error("%s: unsupported down type %d", what, m->td); return HY_EUNSUPPORTED_TYPE; }
        if (!m->down) { set_error("%s: null down", what); return HY_EINVAL; }
        const size_t rb = (size_t) (m->ff / block_elems(m->td)) * block_bytes(m->td);
        if (m->down_bytes != rb * (size_t) m->n) { set_error("%s: down_bytes %zu != n * row bytes %zu", what, m->down_bytes, rb * m->n); return HY_EBAD_SHAPE; }
    }
    return HY_OK;
}
static bool aligned16(const void *p) { return ((uintptr_t) p & 15) == 0; }
// the layer (and the shared expert's) descriptors for a whole decode step: gate/up and down read
int check_dev_decode(const hy_moe_dev *m, const hy_moe_dev *shared, const char *what) {
    int rc = check_dev(m, what, true, true);
    if (rc == HY_OK && shared) rc = check_dev(shared, what, true, true);
    return rc;
}

// the router GEMV entries' checks, for fp32 and bf16 weights
template <typename WT>
static int gemv_checked(const WT *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bias_stride,
                        hipStream_t s, const char *what) {
    if (!W || !x || !y || rows < 0 || nt < 0) { set_error("%s: bad argument", what); return HY_EINVAL; }
    if (kdim <= 0 || kdim % 4 || xs % 4 || !aligned16(W) || !aligned16(x)) { set_error("%s: kdim/xs must be multiples of 4, W/x 16-byte aligned", what); return HY_EBAD_SHAPE; }
    if (rows == 0 || nt == 0) return HY_OK;
    return launch_gemv_f32(W, rows, kdim, x, xs, y, ys, nt, bias, bias_stride, s);
}
template <typename WT>
static int router_q8_checked(const WT *W_r, int rows, int kdim, const float *x, int xs, const float *bias, int bias_stride, float *logits,
                             int ls, int vtype, void *xq, int nt, hipStream_t s, const char *what) {
    if (!W_r || !x || !logits || !xq || rows <= 0 || nt < 0) { set_error("%s: bad argument", what); return HY_EINVAL; }
    if (kdim <= 0 || xs % 4 || !aligned16(W_r) || !aligned16(x)) { set_error("%s: W_r / x rows must be 16-byte aligned", what); return HY_EBAD_SHAPE; }
    if (vtype == Q8_K) {
        if (kdim % 256 || ((uintptr_t) xq & 3)) { set_error("%s: Q8_K needs kdim %% 256 == 0", what); return HY_EBAD_SHAPE; }
    } else if (vtype == Q8_0) {
        if (kdim % 32 || ((uintptr_t) xq & 1)) { set_error("%s: Q8_0 needs kdim %% 32 == 0", what); return HY_EBAD_SHAPE; }
    } else { set_error("%s: vtype %d", what, vtype); return HY_EUNSUPPORTED_TYPE; }
    if (rows > ls) { set_error("%s: %d rows do not fit the logit stride %d", what, rows, ls); return HY_EBAD_SHAPE; }
    return launch_router_q8(W_r, rows, kdim, x, xs, bias, bias_stride, logits, ls, vtype, xq, nt, s);
}
} // namespace hy

using namespace hy;

extern "C" {

const char *hy_last_error(void) { return g_err; }
int hy_abi_version(void) { return 2; }   // 2: hy_moe_dev.n_local

size_t hy_block_bytes(int type) { return (size_t) block_bytes(type); }
int hy_block_elems(int type) { return block_elems(type); }
int hy_vec_dot_type(int type) { return dot_type(type) ? vec_dot_type(type) : -1; }
size_t hy_q8_row_bytes(int vtype, int n) {
    if (vtype == Q8_K && n % 256 == 0) return (size_t) (n / 256) * Q8K_BYTES;
    if (vtype == Q8_0 && n % 32 == 0) return (size_t) (n / 32) * Q8_0_BYTES;
    return 0;
}

int hy_upload_experts(const hy_expert_tensors *t, const int32_t *slot_host, int32_t ff, int32_t n, float clamp, hy_moe_dev *out) {
    if (!t || !slot_host || !out || !t->gate || !t->up || !t->down || t->E <= 0) { set_error("hy_upload_experts: null argument"); return HY_EINVAL; }
    if (!dot_type(t->tg) || !dot_type(t->td)) { set_error("hy_upload_experts: unsupported expert type"); return HY_EUNSUPPORTED_TYPE; }
    if (ff <= 0 || n <= 0 || ff % 256 || n % 256 || t->gb != (size_t) ff * (n / 256) * span_bytes(t->tg) ||
        t->db != (size_t) n * (ff / 256) * span_bytes(t->td)) {
        set_error("hy_upload_experts: ff and n must be multiples of 256 and gb/db the matrices' GGUF sizes");
        return HY_EBAD_SHAPE;
    }
    // slots: -1 (absent) or a local index below E, each used once -- two experts on one slot would overwrite each
    // other, and one stray large value would size the allocation
    int nl = 0;
    std::vector<uint8_t> used(t->E, 0);
    for (int e = 0; e < t->E; ++e) {
        const int sl = slot_host[e];
        if (sl < -1 || sl >= t->E) { set_error("hy_upload_experts: slot[%d] = %d outside [-1, %d)", e, sl, t->E); return HY_EINVAL; }
        if (sl < 0) continue;
        if (used[sl]) { set_error("hy_upload_experts: slot %d given to two experts (second: %d)", sl, e); return HY_EINVAL; }
        used[sl] = 1;
        nl = std::max(nl, sl + 1);
    }
    const size_t n_alloc = std::max(nl, 1);
    uint8_t *dg = nullptr, *du = nullptr, *dd = nullptr;
    int32_t *ds = nullptr;
    hipError_t err = hipMalloc(&dg, t->gb * n_alloc);
    if (err == hipSuccess) err = hipMalloc(&du, t->gb * n_alloc);
    if (err == hipSuccess) err = hipMalloc(&dd, t->db * n_alloc);
    if (err == hipSuccess) err = hipMalloc(&ds, sizeof(int32_t) * t->E);
    // GGUF rows -> 16-row tiles (tiled_off), one expert matrix at a time through a host staging buffer
    std::vector<uint8_t> stage(std::max(t->gb, t->db));
    auto put = [&](uint8_t *dst, const uint8_t *src, int rows, int in_dim, int type) {
        const int nspan = in_dim / 256, sb = span_bytes(type);
        for (int r = 0; r < rows; ++r)
            for (int sp = 0; sp < nspan; ++sp)
                std::memcpy(stage.data() + tiled_off(r, sp, nspan, sb), src + ((size_t) r * nspan + sp) * sb, sb);
        return hipMemcpy(dst, stage.data(), (size_t) rows * nspan * sb, hipMemcpyHostToDevice);
    };
    for (int e = 0; err == hipSuccess && e < t->E; ++e) {
        if (slot_host[e] < 0) continue;
        const size_t sl = (size_t) slot_host[e];
        err = put(dg + sl * t->gb, t->gate + (size_t) e * t->gb, ff, n, t->tg);
        if (err == hipSuccess) err = put(du + sl * t->gb, t->up + (size_t) e * t->gb, ff, n, t->tg);
        if (err == hipSuccess) err = put(dd + sl * t->db, t->down + (size_t) e * t->db, n, ff, t->td);
    }
    if (err == hipSuccess) err = hipMemcpy(ds, slot_host, sizeof(int32_t) * t->E, hipMemcpyHostToDevice);
    if (err != hipSuccess) {
        (void) hipFree(dg); (void) hipFree(du); (void) hipFree(dd); (void) hipFree(ds);
        set_error("hy_upload_experts: %s", hipGetErrorString(err));
        return HY_EHIP;
    }
    hy_moe_dev m;
    m.gate = dg; m.up = du; m.down = dd;
    m.tg = t->tg; m.td = t->td;
    m.gate_bytes = t->gb; m.down_bytes = t->db;
    m.slot = ds;
    m.ff = ff; m.n = n; m.clamp = clamp; m.n_expert = t->E; m.n_local = (int32_t) n_alloc;
    *out = m;
    return HY_OK;
}
int hy_free_experts(hy_moe_dev *m) {
    if (!m) return HY_EINVAL;
    (void) hipFree((void *) m->gate); (void) hipFree((void *) m->up); (void) hipFree((void *) m->down); (void) hipFree((void *) m->slot);
    m->gate = m->up = m->down = nullptr;
    m->slot = nullptr;
    return HY_OK;
}

int hy_gemv_f32(const float *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bias_stride,
                hipStream_t s) {
    return gemv_checked(W, rows, kdim, x, xs, y, ys, nt, bias, bias_stride, s, "hy_gemv_f32");
}
int hy_gemv_bf16w(const uint16_t *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bias_stride,
                  hipStream_t s) {
    return gemv_checked(W, rows, kdim, x, xs, y, ys, nt, bias, bias_stride, s, "hy_gemv_bf16w");
}
int hy_bf16_to_f32(const uint16_t *W, size_t n, float *out, hipStream_t s) {
    if ((!W || !out) && n) { set_error("hy_bf16_to_f32: bad argument"); return HY_EINVAL; }
    if (((uintptr_t) W & 7) || !aligned16(out)) { set_error("hy_bf16_to_f32: W must be 8-byte and out 16-byte aligned"); return HY_EBAD_SHAPE; }
    return launch_bf16_to_f32(W, n, out, s);
}

int hy_moe_route(const float *logits, int ls, int n_expert, int k, int32_t *ids, float *wts, float *sg, int nt, hipStream_t s) {
    if (!logits || !ids || !wts || nt < 0) { set_error("hy_moe_route: bad argument"); return HY_EINVAL; }
    if (n_expert <= 0 || n_expert > 1024) { set_error("hy_moe_route: too many experts (%d > 1024)", n_expert); return HY_EBAD_SHAPE; }
    if (k <= 0 || k > 64 || k > n_expert) { set_error("hy_moe_route: k = %d out of range", k); return HY_EBAD_SHAPE; }
    if (ls < n_expert || (sg && ls <= n_expert)) { set_error("hy_moe_route: logit stride %d too small", ls); return HY_EBAD_SHAPE; }
    return launch_route(logits, ls, n_expert, k, ids, wts, sg, nt, s);
}

static int route_bias_args(const char *what, const float *logits, int ls, const float *bias, int n_expert, int k, const int32_t *ids,
                           const float *wts, int nt) {
    if (!logits || !bias || !ids || !wts || nt < 0) { set_error("%s: bad argument", what); return HY_EINVAL; }
    if (n_expert <= 0 || n_expert > 1024) { set_error("%s: n_expert %d out of range (1..1024)", what, n_expert); return HY_EBAD_SHAPE; }
    if (k <= 0 || k > 16 || k > n_expert) { set_error("%s: k = %d out of range (1..16)", what, k); return HY_EBAD_SHAPE; }
    if (ls < n_expert) { set_error("%s: logit stride %d too small", what, ls); return HY_EBAD_SHAPE; }
    return HY_OK;
}
int hy_moe_route_sig(const float *logits, int ls, const float *bias, int n_expert, int k, float scale, int32_t *ids, float *wts, float *sg,
                     int nt, hipStream_t s) {
    const int rc = route_bias_args("hy_moe_route_sig", logits, ls, bias, n_expert, k, ids, wts, nt);
    return rc != HY_OK ? rc : launch_route_bias(0, logits, ls, bias, n_expert, k, scale, ids, wts, sg, nt, s);
}
int hy_moe_route_sqrtsp(const float *logits, int ls, const float *bias, int n_expert, int k, float scale, int32_t *ids, float *wts, int nt,
                        hipStream_t s) {
    const int rc = route_bias_args("hy_moe_route_sqrtsp", logits, ls, bias, n_expert, k, ids, wts, nt);
    return rc != HY_OK ? rc : launch_route_bias(1, logits, ls, bias, n_expert, k, scale, ids, wts, nullptr, nt, s);
}

int hy_moe_order(const hy_moe_dev *m, const int32_t *ids, int n_pairs, int n_expert, int32_t *order, int32_t *order_n, hipStream_t s,
                 int32_t *egrp) {
    if (!m || !m->slot || !ids || !order || !order_n || n_pairs < 0) { set_error("hy_moe_order: bad argument"); return HY_EINVAL; }
    if (m->n_local <= 0) { set_error("hy_moe_order: n_local %d must be >= 1", m->n_local); return HY_EINVAL; }
    if (n_expert <= 0 || n_expert > 1024 || n_expert > m->n_expert) { set_error("hy_moe_order: n_expert %d out of range", n_expert); return HY_EBAD_SHAPE; }
    return launch_order(m->slot, m->n_local, ids, n_pairs, n_expert, order, order_n, egrp, s);
}

int hy_q8_quantize(int vtype, const float *x, int xs, int n, int nt, void *q, hipStream_t s) {
    if (!x || !q || nt < 0) { set_error("hy_q8_quantize: bad argument"); return HY_EINVAL; }
    if (vtype == Q8_K) {
        if (n <= 0 || n % 256 || xs % 4 || !aligned16(x) || ((uintptr_t) q & 3)) { set_error("hy_q8_quantize: Q8_K needs n %% 256 == 0, xs %% 4 == 0, aligned rows"); return HY_EBAD_SHAPE; }
    } else if (vtype == Q8_0) {
        if (n <= 0 || n % 32 || ((uintptr_t) q & 1)) { set_error("hy_q8_quantize: Q8_0 needs n %% 32 == 0"); return HY_EBAD_SHAPE; }
    } else { set_error("hy_q8_quantize: vtype %d", vtype); return HY_EUNSUPPORTED_TYPE; }
    return launch_q8(vtype, x, xs, n, nt, q, s);
}

// src/cpu_moe.h:46 q8k_test_quantize on host memory: the block steps of src/cpu_moe.cpp:35-78 (the same ones the
// device quantizer runs, hy_common.cuh q8k_block16), one 16-value group at a time.  Rounding: the product is
// rounded to fp32 first (the build compiles with -ffp-contract=off), then 1.5 * 2^23 is added, which rounds it
// half-to-even to an integer held in the low mantissa bits.
int hy_q8k_quantize_host(const float *x, void *y, int64_t k) {
    if (!x || !y || k < 0) { set_error("hy_q8k_quantize_host: bad argument"); return HY_EINVAL; }
    if (k % 256) { set_error("hy_q8k_quantize_host: k = %lld is not a multiple of 256", (long long) k); return HY_EBAD_SHAPE; }
    uint8_t *out = (uint8_t *) y;
    for (int64_t b = 0; b < k / 256; ++b, x += 256, out += Q8K_BYTES) {
        int at = -1;            // first position of the largest magnitude (NaNs never compare greater)
        float best = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float a = std::fabs(x[j]);
            if (a > best) { best = a; at = j; }
        }
        float d = 0.0f;
        int8_t q[256];
        int16_t sums[16];
        if (at < 0) {
            std::memset(q, 0, sizeof q);
            std::memset(sums, 0, sizeof sums);
        } else {
            const float iscale = -127.0f / x[at];
            for (int g = 0; g < 16; ++g) {
                int s16 = 0;
                for (int l = 0; l < 16; ++l) {
                    const float prod = iscale * x[16 * g + l];
                    const float biased = prod + 12582912.0f;
                    uint32_t bits;
                    std::memcpy(&bits, &biased, 4);
                    int v = (int) (bits & 0x007fffffu) - 0x00400000;
                    v = std::min(v, 127);
                    q[16 * g + l] = (int8_t) v;
                    s16 += v;
                }
                sums[g] = (int16_t) s16;
            }
            d = 1.0f / iscale;
        }
        std::memcpy(out, &d, 4);
        std::memcpy(out + 4, q, 256);
        std::memcpy(out + 260, sums, 32);
    }
    return HY_OK;
}

int hy_moe_gate_up(const hy_moe_dev *m, const float *x, int xs, const int32_t *ids, int k, float *h, int nt, hipStream_t s,
                   const int32_t *order, const int32_t *order_n) {
    int rc = check_dev(m, "hy_moe_gate_up", true, false);
    if (rc) return rc;
    if (!x || !ids || !h || k <= 0 || nt < 0 || (order && !order_n)) { set_error("hy_moe_gate_up: bad argument"); return HY_EINVAL; }
    if (xs % 4 || !aligned16(x)) { set_error("hy_moe_gate_up: x rows must be 16-byte aligned"); return HY_EBAD_SHAPE; }
    return launch_gate_up(*m, x, xs, ids, k, h, nt, s, order, order_n);
}

int hy_moe_down(const hy_moe_dev *m, const float *h, const int32_t *ids, const float *wts, int k, float *y, int nt, hipStream_t s,
                const int32_t *order, const int32_t *order_n) {
    int rc = check_dev(m, "hy_moe_down", false, true);
    if (rc) return rc;
    if (!h || !ids || !wts || !y || k <= 0 || nt < 0 || (order && !order_n)) { set_error("hy_moe_down: bad argument"); return HY_EINVAL; }
    if (m->ff % 4 || !aligned16(h)) { set_error("hy_moe_down: h rows must be 16-byte aligned"); return HY_EBAD_SHAPE; }
    return launch_down(*m, h, ids, wts, k, y, nt, s, order, order_n);
}

int hy_moe_gemm_gate_up(const hy_moe_dev *m, const void *xq, int k, int n_pairs, const int32_t *order, const int32_t *order_n,
                        const int32_t *egrp, int max_active, float *h, hipStream_t s) {
    int rc = check_dev(m, "hy_moe_gemm_gate_up", true, false);
    if (rc) return rc;
    if (!gemm_type(m->tg)) { set_error("hy_moe_gemm_gate_up: no grouped GEMM for type %d", m->tg); return HY_EUNSUPPORTED_TYPE; }
    if (!xq || !order || !order_n || !egrp || !h || k <= 0 || max_active < 0 || n_pairs < 0) { set_error("hy_moe_gemm_gate_up: bad argument"); return HY_EINVAL; }
    if ((uintptr_t) xq & 3) { set_error("hy_moe_gemm_gate_up: xq must be 4-byte aligned"); return HY_EBAD_SHAPE; }
    if (max_active > 1024 || max_active > m->n_expert) { set_error("hy_moe_gemm_gate_up: max_active %d > experts", max_active); return HY_EBAD_SHAPE; }
    return launch_gemm_gate_up(*m, xq, k, n_pairs, order, order_n, egrp, max_active, h, s);
}

int hy_moe_gemm_down(const hy_moe_dev *m, const void *hq, int n_pairs, const int32_t *order, const int32_t *order_n, const int32_t *egrp,
                     int max_active, const float *wts, float *y, hipStream_t s) {
    int rc = check_dev(m, "hy_moe_gemm_down", false, true);
    if (rc) return rc;
    if (!gemm_type(m->td)) { set_error("hy_moe_gemm_down: no grouped GEMM for type %d", m->td); return HY_EUNSUPPORTED_TYPE; }
    if (!hq || !order || !order_n || !egrp || !wts || !y || max_active < 0 || n_pairs < 0) { set_error("hy_moe_gemm_down: bad argument"); return HY_EINVAL; }
    if ((uintptr_t) hq & 3) { set_error("hy_moe_gemm_down: hq must be 4-byte aligned"); return HY_EBAD_SHAPE; }
    if (max_active > 1024 || max_active > m->n_expert) { set_error("hy_moe_gemm_down: max_active %d > experts", max_active); return HY_EBAD_SHAPE; }
    return launch_gemm_down(*m, hq, n_pairs, order, order_n, egrp, max_active, wts, y, s);
}

int hy_moe_reduce(const float *shexp, const float *sg, const float *y, int k, float *out, int n, int nt, const int32_t *ids, hipStream_t s) {
    if (!y || !out || !ids || k <= 0 || k > 64 || n <= 0 || nt < 0) { set_error("hy_moe_reduce: bad argument"); return HY_EINVAL; }
    return launch_reduce(shexp, sg, y, k, out, n, nt, ids, s);
}
int hy_moe_reduce_residual(const float *shexp, const float *sg, const float *y, int k, float *resid, int n, int nt, const int32_t *ids,
                           hipStream_t s) {
    if (!y || !resid || !ids || k <= 0 || k > 64 || n <= 0 || nt < 0) { set_error("hy_moe_reduce_residual: bad argument"); return HY_EINVAL; }
    return launch_reduce(shexp, sg, y, k, resid, n, nt, ids, s, 1);
}

int hy_moe_down_reduce(const hy_moe_dev *m, const float *h, const int32_t *ids, const float *wts, int k, const float *shexp, const float *sg,
                       float *out, int nt, hipStream_t s) {
    int rc = check_dev(m, "hy_moe_down_reduce", false, true);
    if (rc) return rc;
    if (!h || !ids || !wts || !out || k <= 0 || k > 64 || nt < 0) { set_error("hy_moe_down_reduce: bad argument"); return HY_EINVAL; }
    if (!aligned16(h)) { set_error("hy_moe_down_reduce: h must be 16-byte aligned"); return HY_EBAD_SHAPE; }
    rc = launch_dec_down(*m, h, ids, wts, k, shexp, sg, out, nt, s);
    if (rc != HY_EUNSUPPORTED_TYPE) return rc;
    return launch_down_reduce(*m, h, ids, wts, k, shexp, sg, out, nt, s);   // shapes beyond the fused kernel's LDS budget
}
int hy_moe_down_reduce_residual(const hy_moe_dev *m, const float *h, const int32_t *ids, const float *wts, int k, const float *shexp,
                                const float *sg, float *resid, int nt, hipStream_t s) {
    int rc = check_dev(m, "hy_moe_down_reduce_residual", false, true);
    if (rc) return rc;
    if (!h || !ids || !wts || !resid || k <= 0 || k > 64 || nt < 0) { set_error("hy_moe_down_reduce_residual: bad argument"); return HY_EINVAL; }
    if (!aligned16(h)) { set_error("hy_moe_down_reduce_residual: h must be 16-byte aligned"); return HY_EBAD_SHAPE; }
    rc = launch_dec_down(*m, h, ids, wts, k, shexp, sg, resid, nt, s, 1);
    if (rc != HY_EUNSUPPORTED_TYPE) return rc;
    return launch_down_reduce(*m, h, ids, wts, k, shexp, sg, resid, nt, s, 1);
}

int hy_moe_router_q8(const float *W_r, int rows, int kdim, const float *x, int xs, const float *bias, int bias_stride, float *logits,
                     int ls, int vtype, void *xq, int nt, hipStream_t s) {
    return router_q8_checked(W_r, rows, kdim, x, xs, bias, bias_stride, logits, ls, vtype, xq, nt, s, "hy_moe_router_q8");
}
int hy_moe_router_q8_bf16w(const uint16_t *W_r, int rows, int kdim, const float *x, int xs, const float *bias, int bias_stride, float *logits,
                           int ls, int vtype, void *xq, int nt, hipStream_t s) {
    return router_q8_checked(W_r, rows, kdim, x, xs, bias, bias_stride, logits, ls, vtype, xq, nt, s, "hy_moe_router_q8_bf16w");
}

int hy_moe_route_gate_up(const hy_moe_dev *m, const float *logits, int ls, int n_expert, int k, const void *xq, int32_t *ids, float *wts,
                         float *sg, float *h, int nt, hipStream_t s) {
    int rc = check_dev(m, "hy_moe_route_gate_up", true, false);
    if (rc) return rc;
    if (!logits || !xq || !ids || !wts || !h || nt < 0) { set_error("hy_moe_route_gate_up: bad argument"); return HY_EINVAL; }
    if (n_expert <= 0 || n_expert > 1024 || n_expert > m->n_expert) { set_error("hy_moe_route_gate_up: n_expert %d out of range", n_expert); return HY_EBAD_SHAPE; }
    if (k <= 0 || k > 64 || k > n_expert) { set_error("hy_moe_route_gate_up: k = %d out of range", k); return HY_EBAD_SHAPE; }
    if (ls < n_expert || (sg && ls <= n_expert)) { set_error("hy_moe_route_gate_up: logit stride %d too small", ls); return HY_EBAD_SHAPE; }
    if ((uintptr_t) xq & 3) { set_error("hy_moe_route_gate_up: xq must be 4-byte aligned"); return HY_EBAD_SHAPE; }
    return launch_route_gate_up(*m, logits, ls, n_expert, k, xq, ids, wts, sg, h, nt, s);
}

int hy_moe_shared_gate_up(const hy_moe_dev *m, const void *xq, float *h, int nt, hipStream_t s) {
    int rc = check_dev(m, "hy_moe_shared_gate_up", true, false);
    if (rc) return rc;
    if (!xq || !h || nt < 0) { set_error("hy_moe_shared_gate_up: bad argument"); return HY_EINVAL; }
    if ((uintptr_t) xq & 3) { set_error("hy_moe_shared_gate_up: xq must be 4-byte aligned"); return HY_EBAD_SHAPE; }
    rc = launch_shared_gate_up(*m, xq, h, nt, s);   // 2..8 tokens: a pass over the weights for every 4
    return rc == HY_EUNSUPPORTED_TYPE ? launch_fixed_gate_up(*m, xq, h, nt, s) : rc;
}

int hy_moe_route_gate_up_q8(const hy_moe_dev *m, const float *logits, int ls, int n_expert, int k, const void *xq, int32_t *ids,
                            float *wts, float *sg, float *h, void *hq, int nt, hipStream_t s) {
    if (!hq) { set_error("hy_moe_route_gate_up_q8: bad argument"); return HY_EINVAL; }
    int rc = check_dev(m, "hy_moe_route_gate_up_q8", true, false);
    if (rc) return rc;
    if (!logits || !xq || !ids || !wts || !h || nt < 0) { set_error("hy_moe_route_gate_up_q8: bad argument"); return HY_EINVAL; }
    if (n_expert <= 0 || n_expert > 1024 || n_expert > m->n_expert) { set_error("hy_moe_route_gate_up_q8: n_expert %d out of range", n_expert); return HY_EBAD_SHAPE; }
    if (k <= 0 || k > 64 || k > n_expert) { set_error("hy_moe_route_gate_up_q8: k = %d out of range", k); return HY_EBAD_SHAPE; }
    if (ls < n_expert || (sg && ls <= n_expert)) { set_error("hy_moe_route_gate_up_q8: logit stride %d too small", ls); return HY_EBAD_SHAPE; }
    if ((uintptr_t) xq & 3) { set_error("hy_moe_route_gate_up_q8: xq must be 4-byte aligned"); return HY_EBAD_SHAPE; }
    return launch_route_gate_up(*m, logits, ls, n_expert, k, xq, ids, wts, sg, h, nt, s, (uint8_t *) hq);
}

int hy_moe_down_reduce_q8(const hy_moe_dev *m, const void *hq, const int32_t *ids, const float *wts, int k, const float *shexp,
                          const float *sg, float *out, int residual, int nt, hipStream_t s) {
    int rc = check_dev(m, "hy_moe_down_reduce_q8", false, true);
    if (rc) return rc;
    if (!hq || !ids || !wts || !out || k <= 0 || k > 64 || nt < 0) { set_error("hy_moe_down_reduce_q8: bad argument"); return HY_EINVAL; }
    if (!aligned16(hq)) { set_error("hy_moe_down_reduce_q8: hq must be 16-byte aligned"); return HY_EBAD_SHAPE; }
    return launch_dec_down(*m, nullptr, ids, wts, k, shexp, sg, out, nt, s, residual ? 1 : 0, (const uint8_t *) hq);
}

int hy_dequant_row(int type, const uint8_t *row, int n, float *out, hipStream_t s) {
    if (!row || !out || n < 0) { set_error("hy_dequant_row: bad argument"); return HY_EINVAL; }
    if (!(dot_type(type) || type == Q8_0 || type == Q8_K)) { set_error("hy_dequant_row: type %d", type); return HY_EUNSUPPORTED_TYPE; }
    if (n % block_elems(type) || ((uintptr_t) row & 3)) { set_error("hy_dequant_row: n %% block != 0 or row unaligned"); return HY_EBAD_SHAPE; }
    return launch_dequant_row(type, row, n, out, s);
}

int hy_block_ints(int type, const uint8_t *rows, size_t row_bytes, int nrows, const void *xq, int n, int32_t *sumi, int32_t *summ,
                  hipStream_t s) {
    if (!rows || !xq || !sumi || !summ || nrows < 0) { set_error("hy_block_ints: bad argument"); return HY_EINVAL; }
    if (!dot_type(type)) { set_error("hy_block_ints: type %d", type); return HY_EUNSUPPORTED_TYPE; }
    // rows keep the alignment their 256-value spans have in the uploaded layout (the largest power of two dividing
    // the span, at most 16): the item loads of the 17- and 18-byte block types count on it to end within the span
    const int sb = span_bytes(type), ra = std::min(16, sb & -sb);
    if (n <= 0 || n % 256 || row_bytes % ra || ((uintptr_t) rows & 15) || ((uintptr_t) xq & 3)) {
        set_error("hy_block_ints: n %% 256 != 0, rows unaligned or row_bytes not a multiple of %d", ra);
        return HY_EBAD_SHAPE;
    }
    return launch_block_ints(type, rows, row_bytes, nrows, xq, n, sumi, summ, s);
}

} // extern "C"
