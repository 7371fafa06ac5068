/*
 * hymoe -- C ABI of the MI355X (gfx950) quantized MoE expert-FFN path.
 *
 * Every entry point replaces one function of the reference's expert-compute API (hyper, src/kernels4.cuh:45-91,
 * src/experts.h:26-50, src/cpu_moe.h:31-90); the citation above each declaration names it.  Differences that
 * apply to all of them:
 *   - plain C: pointers and sizes, a hipStream_t, an int status instead of a C++ exception
 *     (HY_OK, or an HY_E* code with a message from hy_last_error(), thread-local);
 *   - every device pointer is caller-owned (the reference's callers own theirs as well); no entry point
 *     except hy_upload_experts allocates, and all are stream-ordered and free of host synchronisation;
 *   - activations reach the expert matrices as Q8 blocks (block_q8_K, 292 B per 256 values, or block_q8_0,
 *     34 B per 32 values for IQ4_NL, Q8_0, MXFP4, Q5_0 and Q5_1 weights), the partner types of the reference's CPU path
 *     (src/cpu_moe.cpp:711-715), and every block dot product is an exact integer.
 *
 * Results are bit-identical to the CPU oracle of this repository (oracle/), which restates the reference's
 * CPU expert path src/cpu_moe.cpp:668-1008.
 */
#ifndef HYMOE_H
#define HYMOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    HY_OK = 0,
    HY_EUNSUPPORTED_TYPE = 1,   /* weight type without kernels (reference: runtime_error, src/kernels4.cu:1970) */
    HY_EBAD_SHAPE = 2,          /* sizes / strides the kernels do not take (src/kernels4.cu:1926-1927, :2027-2030) */
    HY_EHIP = 3,                /* a HIP runtime error (reference: CUDA_CHECK, src/cuda_check.h:7-8) */
    HY_EINVAL = 4               /* null pointer or out-of-range argument */
};

/* GGUF type ids used by the path (src/gguf.h:13-18); expert weights: Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ1_S, IQ2_XXS, IQ2_XS,
   IQ2_S, IQ3_XXS, IQ3_S, IQ4_NL, IQ4_XS, Q8_0, MXFP4, Q5_0 and Q5_1 (every type of src/kernels4.cu:1951-1971's list); Q8_K and Q8_0 as activation rows */
enum {
    HY_Q5_0 = 6, HY_Q5_1 = 7, HY_Q8_0 = 8, HY_Q2_K = 10, HY_Q3_K = 11, HY_Q4_K = 12, HY_Q5_K = 13, HY_Q6_K = 14, HY_Q8_K = 15,
    HY_IQ2_XXS = 16, HY_IQ2_XS = 17, HY_IQ3_XXS = 18, HY_IQ1_S = 19, HY_IQ4_NL = 20, HY_IQ3_S = 21, HY_IQ2_S = 22, HY_IQ4_XS = 23, HY_MXFP4 = 39
};

/* Expert weights of one layer on the device (replaces MoeDev, src/kernels4.cuh:56-63): n_local experts,
   gate/up [n_local][ff rows of n values] and down [n_local][n rows of ff values] in their GGUF types, each expert
   matrix in the tiled order the kernels read: 16-row tiles whose 256-value spans lie together -- span s (sb bytes,
   the GGUF blocks of 256 values) of row r at byte ((r / 16) * nspan + s) * 16 * sb + (r % 16) * sb, nspan = values
   per row / 256.  The block bytes themselves are GGUF's; hy_upload_experts writes this order from GGUF rows.
   gate, up and down start 16-byte aligned (checked: HY_EBAD_SHAPE).
   slot[e] (device, n_expert entries) = local index of expert e in [0, n_local), or -1; an entry outside
   [0, n_local) is treated as -1 (absent) by every kernel, so a stale or corrupt table cannot index past the
   allocation.  n_local: expert matrices allocated (hy_upload_experts sets it; must be >= 1). */
typedef struct hy_moe_dev {
    const uint8_t *gate, *up, *down;
    int32_t tg, td;                 /* gate/up type, down type */
    size_t gate_bytes, down_bytes;  /* bytes per expert matrix */
    const int32_t *slot;
    int32_t ff, n;                  /* expert intermediate size, d_model */
    float clamp;                    /* SwiGLU limit (0: none) */
    int32_t n_expert;               /* entries of slot (not in MoeDev: ids outside [0, n_expert) are skipped, as on the CPU,
                                       src/cpu_moe.cpp:679, instead of indexing slot out of bounds) */
    int32_t n_local;                /* expert matrices behind gate/up/down (not in MoeDev: bounds every slot entry) */
} hy_moe_dev;

/* Host view of one layer's GGUF expert tensors (replaces ExpertTensors, src/experts.h:20-26). */
typedef struct hy_expert_tensors {
    const uint8_t *gate, *up, *down;   /* host, [E] expert matrices back to back */
    size_t gb, db;                     /* bytes of one expert's gate (= up) / down matrix */
    int32_t E;
    int32_t tg, td;
} hy_expert_tensors;

const char *hy_last_error(void);
int hy_abi_version(void);

/* ---- GGUF expert loading (replaces class GGUF, src/gguf.h:38-70 / src/gguf.cpp:84-285, and expert_tensors,
   src/experts.h:26 / src/experts.cu:12-22).  A read-only view of a GGUF v2/v3 file, memory-mapped; path may name the
   first shard of a split model (<name>-00001-of-0000N.gguf): every shard is mapped and the metadata comes from the
   first.  Opening fails (HY_EINVAL with a message) on a bad magic, a truncated header, a tensor outside its file or
   named twice, or a missing general.architecture; HY_EUNSUPPORTED_TYPE on a tensor type outside the reader's table
   (src/gguf.cpp:43-82).  Tensor data pointers stay valid until hy_gguf_close. */
typedef struct hy_gguf hy_gguf;
typedef struct hy_gguf_tensor_info {    /* GTensor, src/gguf.h:22-32 */
    const char *name;
    const uint8_t *data;           /* host, inside the mapping */
    size_t nbytes;
    int32_t type;                  /* GGUF type id */
    int32_t n_dims;
    int64_t ne[4];                 /* ggml order: ne[0] is the row length; unused dimensions are 1 */
} hy_gguf_tensor_info;
int hy_gguf_open(const char *path, hy_gguf **out);
int hy_gguf_close(hy_gguf *g);
const char *hy_gguf_arch(const hy_gguf *g);                   /* general.architecture (GGUF::arch) */
int hy_gguf_has(const hy_gguf *g, const char *key);           /* 1 if the key is present (GGUF::has) */
/* metadata (GGUF::get_int / get_float / get_str / get_int_arr / get_float_arr): HY_EINVAL if the key is missing or of
   another kind; an int reads as a float, a scalar as a one-element array; arrays copy min(cap, length) elements and
   set *n to the length; strings stay valid until hy_gguf_close */
int hy_gguf_get_int(const hy_gguf *g, const char *key, int64_t *out);
int hy_gguf_get_float(const hy_gguf *g, const char *key, double *out);
int hy_gguf_get_str(const hy_gguf *g, const char *key, const char **out);
int hy_gguf_get_int_arr(const hy_gguf *g, const char *key, int64_t *out, size_t cap, size_t *n);
int hy_gguf_get_float_arr(const hy_gguf *g, const char *key, double *out, size_t cap, size_t *n);
/* the tensor table (GGUF::tensors / tensor / need): by position in file order, or by name (HY_EINVAL if missing) */
int hy_gguf_n_tensors(const hy_gguf *g);
int hy_gguf_tensor_at(const hy_gguf *g, int i, hy_gguf_tensor_info *out);
int hy_gguf_tensor(const hy_gguf *g, const char *name, hy_gguf_tensor_info *out);
/* blk.<il>.ffn_{gate,up,down}_exps.weight of E experts: host pointers, bytes per expert matrix, types (gate and up
   alike, else HY_EBAD_SHAPE) -- ready for hy_upload_experts */
int hy_gguf_expert_tensors(const hy_gguf *g, int il, int E, hy_expert_tensors *out);

/* bytes per block / values per block / activation partner type of a GGUF type (src/gguf.cpp:43-82;
   vec_dot_type: src/cpu_moe.cpp:711-715); 0 or -1 for types the path does not take */
size_t hy_block_bytes(int type);
int hy_block_elems(int type);
int hy_vec_dot_type(int type);
/* bytes of one quantized activation row of n values in partner type vtype */
size_t hy_q8_row_bytes(int vtype, int n);

/* Upload the experts with slot_host[e] >= 0 to their slots (replaces upload_experts, src/experts.h:50 /
   src/experts.cu:56-74), re-laid from GGUF rows into the tiled order above (ff and n multiples of 256, gb / db the
   matrices' GGUF sizes).  Allocates gate/up/down and the slot table with hipMalloc; hy_free_experts releases. */
int hy_upload_experts(const hy_expert_tensors *t, const int32_t *slot_host, int32_t ff, int32_t n, float clamp, hy_moe_dev *out);
int hy_free_experts(hy_moe_dev *m);

/* Router logits y[t][r] = W[r] . x[t] (+ bias[t * bias_stride + r] if bias) for fp32 W [rows][kdim]
   (replaces gemv_f32, src/kernels4.cuh:35 / src/kernels4.cu:1910-1913).  kdim % 4 == 0, xs % 4 == 0. */
int hy_gemv_f32(const float *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt,
                const float *bias, int bias_stride, hipStream_t s);
/* The same with bf16 router weights (uint16 bit patterns holding the fp32 values' high halves), widened on load:
   identical products and sums to hy_gemv_f32 on the widened matrix, half the bytes (replaces gemv_bf16w,
   src/kernels4.cuh:38 / src/kernels4.cu:1914-1917).  W 16-byte aligned, kdim % 4 == 0, xs % 4 == 0. */
int hy_gemv_bf16w(const uint16_t *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt,
                  const float *bias, int bias_stride, hipStream_t s);
/* out[i] = the fp32 value of bf16 W[i], i < n (exact; replaces bf16_to_f32, src/kernels4.cuh:39 /
   src/kernels4.cu:1918-1920).  W 8-byte and out 16-byte aligned. */
int hy_bf16_to_f32(const uint16_t *W, size_t n, float *out, hipStream_t s);

/* Softmax over logits[t][0..n_expert), top-k (ties to the lower index), weights renormalised over the selected;
   sg[t] = sigmoid(logits[t][n_expert]) when sg is not NULL (needs ls > n_expert)
   (replaces moe_route, src/kernels4.cuh:48 / src/kernels4.cu:1925-1935).  n_expert <= 1024, k <= 64. */
int hy_moe_route(const float *logits, int ls, int n_expert, int k, int32_t *ids, float *wts, float *sg, int nt, hipStream_t s);

/* Sigmoid router with a selection bias (replaces moe_route_sig, src/kernels5.cuh:74 / src/kernels5.cu:1090-1122,
   :1291-1295): p = 1 / (1 + exp(-logits[t][e])), the k experts with the largest p + bias[e] (ties to the lower index),
   weights p scale / max(the selected p summed in selection order, 2^-14); sg[t] = 1 when sg is not NULL.
   bias: n_expert floats on the device.  n_expert <= 1024, k <= 16. */
int hy_moe_route_sig(const float *logits, int ls, const float *bias, int n_expert, int k, float scale, int32_t *ids, float *wts, float *sg,
                     int nt, hipStream_t s);
/* sqrt-softplus router (replaces route7, src/kernels7.cuh:75 / src/kernels7.cu:816-865, :987-990):
   s = sqrt(softplus(logits[t][e])) with softplus(l) = l above 20, else log1p(exp(l)); the top k of s + bias[e] (ties
   to the lower index); weights s / (the selected s summed in selection order + 1e-20) scale.  Limits as above. */
int hy_moe_route_sqrtsp(const float *logits, int ls, const float *bias, int n_expert, int k, float scale, int32_t *ids, float *wts, int nt,
                        hipStream_t s);

/* Pairs p < n_pairs whose expert has slot >= 0, grouped by expert in ascending id, stable by pair index:
   order[], order_n[0] = their count, order_n[1] = active experts, egrp[3 i ..] = (expert, start, count)
   (replaces moe_order, src/kernels4.cuh:74-75 / src/kernels4.cu:2059-2062).  n_expert <= 1024. */
int hy_moe_order(const hy_moe_dev *m, const int32_t *ids, int n_pairs, int n_expert, int32_t *order, int32_t *order_n,
                 hipStream_t s, int32_t *egrp);

/* Activations to Q8 blocks: rows x[t * xs ..][0..n) -> q (nt rows of hy_q8_row_bytes(vtype, n) bytes)
   (replaces to_half before the grouped GEMMs, src/kernels.cu:2235-2237, and the CPU path's quantizer,
   src/cpu_moe.cpp:35-78 for Q8_K).  vtype HY_Q8_K (n % 256 == 0) or HY_Q8_0 (n % 32 == 0). */
int hy_q8_quantize(int vtype, const float *x, int xs, int n, int nt, void *q, hipStream_t s);

/* The CPU expert path's Q8_K quantizer on host memory (replaces q8k_test_quantize, src/cpu_moe.h:46 /
   src/cpu_moe.cpp:35-78): k values of x (host) -> k / 256 blocks of 292 bytes at y (host), synchronous, no HIP
   call.  Per block: the first value of largest magnitude mx, iscale = -127 / mx, q = min(127, round-half-even of the
   rounded product iscale * x), int16 sums of 16, d = 1 / iscale; an all-zero block gets d = 0, q = 0 and zero sums.
   The blocks are bit-identical to hy_q8_quantize's.  k must be a multiple of 256 (HY_EBAD_SHAPE). */
int hy_q8k_quantize_host(const float *x, void *y, int64_t k);

/* Decode gate/up: h[p][f] = silu(gate_e[f] . x[t]) * (up_e[f] . x[t]) for pairs p = t*k + j (or the order_n[0]
   pairs in order) whose expert is local; x is quantized inside (replaces moe_gate_up, src/kernels4.cuh:67-68 /
   src/kernels4.cu:1973-2006). */
int hy_moe_gate_up(const hy_moe_dev *m, const float *x, int xs, const int32_t *ids, int k, float *h, int nt, hipStream_t s,
                   const int32_t *order, const int32_t *order_n);

/* Decode down: y[p][r] = wts[p] * (down_e[r] . q8(h[p])); without order non-local pairs get 0
   (replaces moe_down, src/kernels4.cuh:70-71 / src/kernels4.cu:2007-2022). */
int hy_moe_down(const hy_moe_dev *m, const float *h, const int32_t *ids, const float *wts, int k, float *y, int nt, hipStream_t s,
                const int32_t *order, const int32_t *order_n);

/* Prefill / verify grouped GEMMs over bucketed pairs (replace moe_gemm_gate_up / moe_gemm_down,
   src/kernels4.cuh:77-80 / src/kernels4.cu:2063-2093).  xq: Q8 rows of the tokens (pair p reads row p / k);
   h [n_pairs][ff] fp32; hq: Q8 rows of h per pair; y[p][r] = wts[p] * (down_e[r] . hq[p]).
   n_pairs (not in the reference: its grid was one block per active expert) bounds the work items, chunks of
   up to 64 tokens of one expert; max_active >= order_n[1] (<= 1024). */
int hy_moe_gemm_gate_up(const hy_moe_dev *m, const void *xq, int k, int n_pairs, const int32_t *order, const int32_t *order_n,
                        const int32_t *egrp, int max_active, float *h, hipStream_t s);
int hy_moe_gemm_down(const hy_moe_dev *m, const void *hq, int n_pairs, const int32_t *order, const int32_t *order_n, const int32_t *egrp,
                     int max_active, const float *wts, float *y, hipStream_t s);

/* Combine: out[t][r] = sg[t] * shexp[t][r] (when shexp; sg NULL: 1) + the pairs' y[t*k + j][r] added in ascending
   expert-id order (without shexp the first pair is the start value); ids with a negative expert are skipped
   (replaces moe_reduce, src/kernels4.cuh:88-91 / src/kernels4.cu:1182-1206, single device, no CPU owner). */
int hy_moe_reduce(const float *shexp, const float *sg, const float *y, int k, float *out, int n, int nt, const int32_t *ids,
                  hipStream_t s);
/* The combine written straight into the residual (the next row after moe_reduce, src/kernels4.cu:1182-1206: on one GPU
   the engine adds the reduced part to the residual, src/engine4.cu:887-895): resid[t][r] = resid[t][r] + part, part
   formed exactly as hy_moe_reduce forms out, then one fp32 addition. */
int hy_moe_reduce_residual(const float *shexp, const float *sg, const float *y, int k, float *resid, int n, int nt, const int32_t *ids,
                           hipStream_t s);

/* Decode down + combine in one launch: out[t][r] as hy_moe_reduce of hy_moe_down's y, without materialising y;
   pairs whose expert is not local (or whose id is out of range) are left out of the sum
   (fuses src/kernels4.cu:2007-2022 with :1182-1206). */
int hy_moe_down_reduce(const hy_moe_dev *m, const float *h, const int32_t *ids, const float *wts, int k, const float *shexp,
                       const float *sg, float *out, int nt, hipStream_t s);
/* Decode: hy_moe_down_reduce with the result added into the residual (resid[t][r] = resid[t][r] + out[t][r]), one launch. */
int hy_moe_down_reduce_residual(const hy_moe_dev *m, const float *h, const int32_t *ids, const float *wts, int k, const float *shexp,
                                const float *sg, float *resid, int nt, hipStream_t s);

/* Router logits and the Q8 rows of x in one launch: logits as hy_gemv_f32 (rows of W_r, stride ls >= rows) and xq as
   hy_q8_quantize(vtype, x, xs, kdim, nt) -- fuses gemv_f32 (src/kernels4.cu:1910-1913) with the activation
   quantization of the expert kernels.  Up to 8 tokens a wave per (row, token) logit; more, the batched routers, still
   one launch with the quantization.  The logits are hy_gemv_f32's bits except for large batches whose full 64 x 64
   logit tiles number at least 256 (kdim a multiple of 64, x 16-byte aligned, xs a multiple of 4: e.g. 2048 tokens x
   512 experts), which run on the fp32 matrix cores in their own summation order: there the logits agree with
   hy_gemv_f32 to fp32 rounding (within 2 kdim 2^-24 sum |w x|), and the routing is defined on the logits given. */
int hy_moe_router_q8(const float *W_r, int rows, int kdim, const float *x, int xs, const float *bias, int bias_stride, float *logits,
                     int ls, int vtype, void *xq, int nt, hipStream_t s);
/* The same with bf16 router weights, widened on load as in hy_gemv_bf16w (the router16 path of src/engine4.cu:808:
   gemv_bf16w, then the expert kernels' quantization of x): logits identical to hy_moe_router_q8 on the widened W_r. */
int hy_moe_router_q8_bf16w(const uint16_t *W_r, int rows, int kdim, const float *x, int xs, const float *bias, int bias_stride,
                           float *logits, int ls, int vtype, void *xq, int nt, hipStream_t s);

/* Routing + decode gate/up in one launch: each token's softmax / top-k / weights / sg exactly as hy_moe_route
   (written to ids, wts, sg), then h[t*k + j] as hy_moe_gate_up, from the Q8 rows xq (partner type of the gate
   type, e.g. from hy_moe_router_q8).  Pairs whose expert is not local leave their h rows unwritten
   (fuses moe_route and moe_gate_up, src/kernels4.cu:1925-1935 and :1973-2006). */
int hy_moe_route_gate_up(const hy_moe_dev *m, const float *logits, int ls, int n_expert, int k, const void *xq, int32_t *ids, float *wts,
                         float *sg, float *h, int nt, hipStream_t s);

/* Decode gate/up of the always-on (shared) expert: h[t] = SwiGLU(gate . x_t, up . x_t) of the descriptor's local
   expert 0 for nt tokens, from their Q8 rows xq (partner type of the gate type), as hy_moe_gate_up with every id 0
   and k = 1 computes it from x (the reference's shared-expert call of moe_gate_up, src/engine4.cu:795-804).  From 2 to 8
   tokens, one pass over the weights serves up to 4 tokens. */
int hy_moe_shared_gate_up(const hy_moe_dev *m, const void *xq, float *h, int nt, hipStream_t s);

/* hy_moe_route_gate_up that also writes hq: the pairs' hidden rows as Q8_0 blocks (the values and scales
   hy_q8_quantize(Q8_0, h row) gives), so the down step reads them instead of quantizing h in every block -- the down
   kernels' activation quantization (src/kernels4.cu:2007-2022 quantizes h per launch) moved into the producer.
   Layout, per token t at t * k * nbh * 34 bytes (nbh = ff / 32): the 32 int8 values of block b of pair j at
   (j * nbh + b) * 32, then the fp16 scales, block b of pair j at k * nbh * 32 + 2 * (j * nbh + b).  For IQ4_NL
   gate/up and down weights and n <= 4096, else HY_EUNSUPPORTED_TYPE. */
int hy_moe_route_gate_up_q8(const hy_moe_dev *m, const float *logits, int ls, int n_expert, int k, const void *xq, int32_t *ids,
                            float *wts, float *sg, float *h, void *hq, int nt, hipStream_t s);
/* hy_moe_down_reduce (residual == 0) or hy_moe_down_reduce_residual (residual != 0) from those Q8_0 blocks (hq
   16-byte aligned); bit-identical to them on the h the blocks came from.  HY_EUNSUPPORTED_TYPE for other down types. */
int hy_moe_down_reduce_q8(const hy_moe_dev *m, const void *hq, const int32_t *ids, const float *wts, int k, const float *shexp,
                          const float *sg, float *out, int residual, int nt, hipStream_t s);

/* The shared (always-on) expert's decode down for nt <= 64 rows: out[t][r] = down_0[r] . q8(h[t]) -- moe_down of a
   k = 1 layer whose pairs are all its local expert 0 with weight 1 (src/engine4.cu:795-804's mm(L.sh_down)), each
   row's value alone (no combine).  From 2 rows on one pass over the weights serves every row.  Bit-identical to
   hy_moe_down_reduce(m, h, ids = 0, wts = 1, k = 1, NULL, NULL, out, nt). */
int hy_moe_shared_down(const hy_moe_dev *m, const float *h, float *out, int nt, hipStream_t s);

/* One MoE layer's decode step (nt <= 64 rows) in one call: the reference engine's per-layer sequence
   (src/engine4.cu:807-890 -- gemv_f32, moe_route, moe_gate_up, moe_down, moe_reduce -- and the shared expert of
   src/engine4.cu:795-804) on the decode launches above: hy_moe_router_q8, hy_moe_route_gate_up (softmax routing),
   hy_moe_down_reduce.  W_r: fp32 [rows][n] with rows = n_expert, or n_expert + 1 whose last row is the shared-expert
   gate logit (sg = sigmoid of it; without that row the shared expert's gate is 1); bias as in hy_gemv_f32 (NULL:
   none).  shared: the always-on expert (NULL: none; its slot 0 holds it).  out [nt][n] fp32, or with residual != 0
   the step is added into it.  The intermediates (logits, ids, wts, sg, Q8 rows of x, h, the shared expert's h and
   output) live in the caller's workspace `ws` of at least hy_moe_decode_ws_bytes(...) bytes, 256-byte aligned; the
   routing (ids, wts) is left there.  Results are bit-identical to the separate entry points. */
size_t hy_moe_decode_ws_bytes(const hy_moe_dev *m, int rows, int k, const hy_moe_dev *shared, int nt);
int hy_moe_decode(const hy_moe_dev *m, const float *W_r, int rows, const float *x, int xs, const float *bias, int bias_stride, int k,
                  const hy_moe_dev *shared, float *out, int residual, int nt, void *ws, size_t ws_bytes, hipStream_t s);
/* hy_moe_decode without a workspace argument.  No counterpart in the reference: it is for callers that cannot
   allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
   allocates nothing: the intermediates live in a file-scope device array of 1 MiB that each GPU running the library
   holds until the process ends (hy_moe_decode_ws_bytes must not exceed it, else HY_EBAD_SHAPE).  Every call on one
   GPU shares that GPU's array and nothing in it needs to start at zero; calls that overlap on one GPU (other streams,
   other threads) race on it and must be ordered by the caller. */
int hy_moe_decode_noalloc(const hy_moe_dev *m, const float *W_r, int rows, const float *x, int xs, const float *bias, int bias_stride,
                          int k, const hy_moe_dev *shared, float *out, int residual, int nt, hipStream_t s);

/* Test hooks.  One row of n weights dequantized by the kernels' block decoders (replaces deq_row_test,
   src/kernels4.cuh:181 / src/kernels4.cu:2036-2044); and the exact integers of every block of nrows weight rows
   (row stride row_bytes) against one Q8 activation row: sumi/summ [nrows][n / block_elems] (summ 0 for types
   without mins) -- the per-block int32 dot products of the contract.  rows is 16-byte aligned and row_bytes a
   multiple of the alignment of the type's 256-value span (its largest power-of-two factor, at most 16: 8 for
   MXFP4's 136 bytes, 2 for Q6_K's 210). */
int hy_dequant_row(int type, const uint8_t *row, int n, float *out, hipStream_t s);
int hy_block_ints(int type, const uint8_t *rows, size_t row_bytes, int nrows, const void *xq, int n, int32_t *sumi, int32_t *summ,
                  hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif
