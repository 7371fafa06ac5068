/*
 * CPU oracle for the quantized MoE expert-FFN path -- TEST INFRASTRUCTURE ONLY.
 *
 * It checks the GPU results and is never what is measured: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it.  The product (hyper_amd/) never
 * links or calls it.
 *
 * It restates, in plain C, the semantics of hyper's CPU expert path
 * (src/cpu_moe.cpp:668-1008, CpuMoe::run_layer) and of the block formats the
 * GPU kernels decode (src/kernels4.cu:421-714, deq8<T>), under one numeric
 * contract shared with the HIP kernels:
 *
 *  - activations are quantized to the weight type's ggml vec_dot partner:
 *    Q8_K for the K-quants / IQ4_XS / IQ2_XS (src/cpu_moe.cpp:35-78),
 *    Q8_0 for IQ4_NL, Q8_0, MXFP4, Q5_0 and Q5_1 (ggml's x86 quantize_row_q8_0, see or_quantize_q8_0);
 *  - every weight block against its activation block gives exact integers
 *    (sumi, and summ for the types with mins);
 *  - a row dot product folds block b's integers with one fixed fp32 formula
 *    and accumulates blocks in order b = 0, 1, ...:
 *        with mins:    t = fmaf(d, (float) sumi, -(dmin * (float) summ))
 *        without:      t = dw * (float) sumi
 *                      acc = fmaf(xd, t, acc)          (acc starts at 0.0f)
 *  - SwiGLU h = (g / (1 + exp(-g))) * u with this file's own exp
 *    (or_expf: Cephes-style Cody-Waite reduction + degree-5 polynomial);
 *  - weighted sum per token in expert-id order: the first pair assigns w*y,
 *    later pairs add w*y (src/cpu_moe.cpp:863-874, :994-1006).
 *
 * Parity status per function: each function's pinning tests are named in the test files.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 */
#ifndef HY_MOE_ORACLE_H
#define HY_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids (src/gguf.h:13-18) */
enum {
    OR_Q5_0 = 6, OR_Q5_1 = 7, OR_Q8_0 = 8, OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_Q8_K = 15,
    OR_IQ2_XXS = 16, OR_IQ2_XS = 17, OR_IQ3_XXS = 18, OR_IQ1_S = 19, OR_IQ4_NL = 20, OR_IQ3_S = 21, OR_IQ2_S = 22, OR_IQ4_XS = 23, OR_MXFP4 = 39
};

size_t or_block_bytes(int type);      /* bytes per block (src/gguf.cpp:43-82) */
int or_block_elems(int type);         /* values per block */
int or_vec_dot_type(int type);        /* activation partner type: OR_Q8_K or OR_Q8_0 */

float or_expf(float x);
float or_silu(float x);
float or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);

/* activations -> Q8_K (n % 256 == 0) / Q8_0 (n % 32 == 0) / the partner of a weight type */
void or_quantize_q8_K(const float *x, void *y, int n);
void or_quantize_q8_0(const float *x, void *y, int n);
int or_quantize_row(int vtype, const float *x, void *y, int n);

/* one row of n weights dequantized (deq8 formulas) */
int or_dequant_row(int type, const uint8_t *row, int n, float *out);

/* exact integers of every block of one weight row against a quantized activation row:
   sumi[b], summ[b] (summ is 0 for types without mins) */
int or_block_ints(int type, const uint8_t *row, const void *xq, int n, int32_t *sumi, int32_t *summ);
/* the same integers by the element-by-element restatement only (the K-quants' AVX2 path is checked against it) */
int or_block_ints_scalar(int type, const uint8_t *row, const void *xq, int n, int32_t *sumi, int32_t *summ);
/* the contract's row dot product */
float or_row_dot(int type, const uint8_t *row, const void *xq, int n);

/* fp32 router GEMV logits[t][r] = W[r] . x[t] in the contract's order (64 partial sums, lane L takes
   elements 256 i + 4 L + j, fma in index order, xor butterfly 32..1) */
void or_gemv_f32(const float *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt);
/* softmax top-k routing (src/kernels4.cu:297-344): ids/wts [nt][k]; sg[t] = sigmoid(logits[t][ne]) if sg */
int or_route(const float *logits, int ls, int ne, int k, int nt, int32_t *ids, float *wts, float *sg);
/* log and log1p (Cephes logf polynomial; Goldberg's log1p correction), the routers' scores */
float or_logf(float x);
float or_log1pf(float x);
float or_sigmoid(float l);
float or_sqrt_softplus(float l);
/* sigmoid router with selection bias (src/kernels5.cu:1090-1122) and sqrt-softplus router (src/kernels7.cu:816-865):
   top k of score + bias[e] (ties to the lower index); weights from the scores alone */
int or_route_sig(const float *logits, int ls, const float *bias, int ne, int k, float scale, int nt, int32_t *ids, float *wts, float *sg);
int or_route_sqrtsp(const float *logits, int ls, const float *bias, int ne, int k, float scale, int nt, int32_t *ids, float *wts);
/* bucketing: pairs with slot[ids[p]] >= 0 grouped by expert, stable by pair index
   (src/kernels4.cu:1275-1295, src/cpu_moe.cpp:672-687); egrp may be NULL */
int or_order(const int32_t *slot, const int32_t *ids, int n_pairs, int ne, int32_t *order, int32_t *order_n, int32_t *egrp);

/* one MoE layer's experts (src/cpu_moe.h:31-44 CpuExpertLayer, every expert owned) */
typedef struct {
    int tg, td;                            /* gate/up and down GGUF types */
    const uint8_t *gate, *up, *down;       /* [E][rows][row bytes] */
    size_t gate_bytes, down_bytes;         /* bytes per expert matrix */
    int ff, n, E;                          /* expert intermediate, d_model, experts */
    float clamp;                           /* SwiGLU limit, 0 = none */
} or_layer;

/* CpuMoe::run_layer semantics for nt tokens (x rows of stride xs, ids/wts [nt][k]), out [nt][os].
   Optional: a shared expert (weights `sh`, one expert of sh->ff rows, gate sg[t] or 1 when sg is
   NULL), scratch outputs h [P][ff] and y [P][n] in pair order t*k+j (NULL: internal).
   Tokens without a valid pair get zeros (or the shared term only). */
int or_moe_layer(const or_layer *L, int nt, const float *x, int xs, const int32_t *ids, const float *wts, int k,
                 float *out, int os, const or_layer *sh, const float *sg, float *h_out, float *y_out, int n_threads);

/* shared-expert style FFN of one expert e of L for nt rows: y[t][r] = down_e . q(h), h = swiglu(gate/up) */
int or_expert_ffn(const or_layer *L, int e, int nt, const float *x, int xs, float *h, float *y, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
