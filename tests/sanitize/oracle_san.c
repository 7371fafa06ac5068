/* The CPU oracle (oracle/moe_oracle.c) under AddressSanitizer and UBSan: every entry point on seeded random inputs,
   every weight type, shapes with tails (d % 256 != 0 for the GEMV, expert counts that are not powers of two), garbage
   and absent expert ids, a shared expert.  Exit 0 unless a sanitizer reports (they abort).  Built by
   tests/sanitize/Makefile; run by tests/test_sanitize.py.  The random bytes make valid blocks except for fp16 scale
   fields, which are set to small finite values. */
#include "../../oracle/moe_oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static unsigned long long rs = 88172645463325252ull;
static unsigned rnd(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return (unsigned) rs; }
static float rndf(void) { return ((int) (rnd() % 2001) - 1000) / 250.0f; }

/* random blocks of a type whose fp16 d (and dmin) fields hold small finite values */
static void fill_blocks(int type, uint8_t *p, size_t nblocks) {
    const size_t bb = or_block_bytes(type);
    for (size_t i = 0; i < nblocks * bb; ++i) p[i] = (uint8_t) rnd();
    for (size_t b = 0; b < nblocks; ++b) {
        uint8_t *blk = p + b * bb;
        const uint16_t d = or_fp32_to_fp16(1e-3f * (float) (1 + rnd() % 9));
        if (type == OR_Q6_K) memcpy(blk + 208, &d, 2);
        else memcpy(blk, &d, 2);
        if (type == OR_Q4_K || type == OR_Q5_K) memcpy(blk + 2, &d, 2);
    }
}

int main(void) {
    const int types[6] = {OR_Q4_K, OR_Q5_K, OR_Q6_K, OR_IQ4_XS, OR_IQ2_XS, OR_IQ4_NL};
    float x[2048], out[2048];
    for (int i = 0; i < 2048; ++i) x[i] = rndf();
    uint8_t q[2048 / 32 * 34 + 2048 / 256 * 292];
    or_quantize_q8_K(x, q, 2048);
    or_quantize_q8_0(x, q, 2048);
    for (int ti = 0; ti < 6; ++ti) {
        const int t = types[ti], n = 1024, be = or_block_elems(t);
        uint8_t *row = (uint8_t *) malloc((size_t) (n / be) * or_block_bytes(t));
        fill_blocks(t, row, n / be);
        uint8_t xq[1024 / 32 * 34 + 1024 / 256 * 292];
        if (or_quantize_row(or_vec_dot_type(t), x, xq, n)) return 3;
        if (or_dequant_row(t, row, n, out)) return 3;
        int32_t si[1024 / 32], sm[1024 / 32];
        if (or_block_ints(t, row, xq, n, si, sm)) return 3;
        volatile float r = or_row_dot(t, row, xq, n);
        (void) r;
        free(row);
    }
    /* router GEMV with a tail, the routers, bucketing */
    {
        const int rows = 37, kd = 300, nt = 3;
        float *W = malloc(sizeof(float) * rows * kd), *xs = malloc(sizeof(float) * nt * kd), y[3 * 40];
        for (int i = 0; i < rows * kd; ++i) W[i] = rndf();
        for (int i = 0; i < nt * kd; ++i) xs[i] = rndf();
        or_gemv_f32(W, rows, kd, xs, kd, y, 40, nt);
        int32_t ids[3 * 8];
        float wts[3 * 8], sg[3], bias[36];
        for (int i = 0; i < 36; ++i) bias[i] = rndf();
        if (or_route(y, 40, 36, 8, nt, ids, wts, sg)) return 3;
        if (or_route_sig(y, 40, bias, 36, 8, 2.5f, nt, ids, wts, sg)) return 3;
        if (or_route_sqrtsp(y, 40, bias, 36, 8, 1.0f, nt, ids, wts)) return 3;
        int32_t slot[36], order[24], order_n[2], egrp[3 * 36];
        for (int e = 0; e < 36; ++e) slot[e] = e % 5 == 3 ? -1 : e;
        ids[4] = -1; ids[9] = 1000;
        if (or_order(slot, ids, 24, 36, order, order_n, egrp)) return 3;
        free(W); free(xs);
    }
    /* whole layers, every gate/up x down type pair, with a shared expert and garbage ids */
    for (int gi = 0; gi < 6; ++gi) {
        for (int di = 0; di < 6; ++di) {
            const int tg = types[gi], td = types[di], E = 5, ff = 256, n = 512, nt = 3, k = 3;
            const size_t gb = (size_t) ff * (n / or_block_elems(tg)) * or_block_bytes(tg), db = (size_t) n * (ff / or_block_elems(td)) * or_block_bytes(td);
            uint8_t *g = malloc(E * gb), *u = malloc(E * gb), *dn = malloc(E * db);
            fill_blocks(tg, g, E * gb / or_block_bytes(tg));
            fill_blocks(tg, u, E * gb / or_block_bytes(tg));
            fill_blocks(td, dn, E * db / or_block_bytes(td));
            or_layer L = {tg, td, g, u, dn, gb, db, ff, n, E, gi == di ? 4.0f : 0.0f};
            or_layer S = {tg, td, g + gb, u + gb, dn + db, gb, db, ff, n, 1, 0.0f};
            float xs[3 * 512], o[3 * 512], sg[3] = {0.5f, 1.0f, 0.25f}, w[9];
            int32_t ids[9];
            for (int i = 0; i < nt * n; ++i) xs[i] = rndf();
            for (int i = 0; i < nt * k; ++i) { ids[i] = (int) (rnd() % 7) - 1; w[i] = 0.3f; }   /* -1 and 5: skipped */
            if (or_moe_layer(&L, nt, xs, n, ids, w, k, o, n, &S, sg, NULL, NULL, 2)) return 3;
            float h[3 * 256], yy[3 * 512];
            if (or_expert_ffn(&L, 2, nt, xs, n, h, yy, 2)) return 3;
            free(g); free(u); free(dn);
        }
    }
    printf("oracle_san: done\n");
    return 0;
}
