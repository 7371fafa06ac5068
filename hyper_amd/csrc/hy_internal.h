// Internal declarations shared by the HIP translation units of libhymoe.so.
#pragma once
#include "../../include/hymoe.h"
#include "hy_common.cuh"
#include "hy_error.h"

namespace hy {

// after a launch: HY_OK, or HY_EHIP with the launch error recorded under `what`
int check_launch(const char *what);
// checks of the layer descriptors a whole decode step reads (gate/up and down of the layer and of the shared expert)
int check_dev_decode(const hy_moe_dev *m, const hy_moe_dev *shared, const char *what);

// router GEMVs: W fp32, or bf16 bit patterns (uint16) widened on load -- the same products and sums
int launch_gemv_f32(const float *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bs,
                    hipStream_t s);
int launch_gemv_f32(const uint16_t *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt, const float *bias, int bs,
                    hipStream_t s);
int launch_bf16_to_f32(const uint16_t *W, size_t n, float *out, hipStream_t s);
int launch_route(const float *logits, int ls, int ne, int k, int *ids, float *wts, float *sg, int nt, hipStream_t s);
int launch_route_bias(int mode, const float *logits, int ls, const float *bias, int ne, int k, float scale, int *ids, float *wts,
                      float *sg, int nt, hipStream_t s);
int launch_order(const int *slot, int n_local, const int *ids, int P, int ne, int *order, int *order_n, int *egrp, hipStream_t s);
int launch_q8(int vtype, const float *x, int xs, int n, int nt, void *q, hipStream_t s);
int launch_router_pre(const float *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                      int vtype, void *xq, int nt, hipStream_t s);
int launch_router_pre(const uint16_t *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                      int vtype, void *xq, int nt, hipStream_t s);
int launch_gate_up(const hy_moe_dev &m, const float *x, int xs, const int *ids, int k, float *h, int nt, hipStream_t s, const int *order,
                   const int *order_n);
int launch_down(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, float *y, int nt, hipStream_t s,
                const int *order, const int *order_n);
int launch_down_reduce(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp, const float *sg,
                       float *out, int nt, hipStream_t s, int res = 0);
int launch_reduce(const float *shexp, const float *sg, const float *y, int k, float *out, int n, int nt, const int *ids, hipStream_t s,
                  int res = 0);
int launch_gemm_gate_up(const hy_moe_dev &m, const void *xq, int k, int n_pairs, const int *order, const int *order_n, const int *egrp,
                        int max_active, float *h, hipStream_t s);
int launch_gemm_down(const hy_moe_dev &m, const void *hq, int n_pairs, const int *order, const int *order_n, const int *egrp, int max_active,
                     const float *wts, float *y, hipStream_t s);
int launch_router_q8(const float *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                     int vtype, void *xq, int nt, hipStream_t s);
int launch_router_q8(const uint16_t *W, int rows, int kdim, const float *x, int xs, const float *bias, int bs, float *logits, int ls,
                     int vtype, void *xq, int nt, hipStream_t s);
// hq: also write the Q8_0 rows of h (down types whose partner is Q8_0); HY_EUNSUPPORTED_TYPE where that does not apply
int launch_route_gate_up(const hy_moe_dev &m, const float *logits, int ls, int ne, int k, const void *xq, int *ids, float *wts, float *sg,
                         float *h, int nt, hipStream_t s, uint8_t *hq = nullptr);
// SwiGLU(gate, up) of the descriptor's local expert 0 for nt Q8 rows (a shared expert's decode gate/up, no routing)
int launch_fixed_gate_up(const hy_moe_dev &m, const void *xq, float *h, int nt, hipStream_t s);
// the same for 2..8 tokens in one pass over the weights; HY_EUNSUPPORTED_TYPE outside its limits (use the one above)
int launch_shared_gate_up(const hy_moe_dev &m, const void *xq, float *h, int nt, hipStream_t s);
// the shared expert's down for 2 or more tokens in one pass over the weights: out[t] = down . q8(h[t]) (ids all 0 and
// wts all 1, nt entries each); HY_EUNSUPPORTED_TYPE outside its limits (use launch_dec_down with k = 1)
int launch_shared_down(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, float *out, int nt, hipStream_t s);
// whether launch_dec_down runs its fused kernel (not HY_EUNSUPPORTED_TYPE) for this layer and k
bool dec_down_takes_q8(const hy_moe_dev &m, int k);
// hq: the hidden as Q8_0 rows (from launch_route_gate_up) instead of h
int launch_dec_down(const hy_moe_dev &m, const float *h, const int *ids, const float *wts, int k, const float *shexp, const float *sg,
                    float *out, int nt, hipStream_t s, int res = 0, const uint8_t *hq = nullptr);
int launch_dequant_row(int type, const uint8_t *row, int n, float *out, hipStream_t s);
int launch_block_ints(int type, const uint8_t *rows, size_t row_bytes, int nrows, const void *xq, int n, int *sumi, int *summ,
                      hipStream_t s);

} // namespace hy
