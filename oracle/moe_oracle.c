/*
 * CPU oracle for the quantized MoE expert-FFN path -- TEST INFRASTRUCTURE ONLY (see moe_oracle.h).
 *
 * Every function names the reference lines it restates.  The reference's CPU path takes its block dot
 * products and the Q8_0 quantizer from ggml, which is not vendored (Makefile:4, :15, :33-34); those are
 * restated here from the block layouts the reference itself decodes (src/kernels4.cu:421-714) and the
 * integer structure of its own IQ4_XS x Q8_K dot (src/iq3s_dot.h:136-166).
 */
#define _GNU_SOURCE
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ formats / tables */

size_t or_block_bytes(int type) {
    switch (type) {                      /* src/gguf.cpp:43-82 */
    case OR_Q8_0: return 34;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    case OR_Q8_K: return 292;
    case OR_IQ2_XS: return 74;
    case OR_IQ2_XXS: return 66;
    case OR_IQ4_NL: return 18;
    case OR_IQ4_XS: return 136;
    case OR_MXFP4: return 17;
    case OR_Q5_0: return 22;
    case OR_Q2_K: return 84;
    case OR_Q3_K: return 110;
    case OR_IQ3_XXS: return 98;
    case OR_IQ3_S: return 110;
    case OR_IQ2_S: return 82;
    case OR_IQ1_S: return 50;
    case OR_Q5_1: return 24;
    default: return 0;
    }
}
int or_block_elems(int type) {
    switch (type) {
    case OR_Q8_0: case OR_IQ4_NL: case OR_MXFP4: case OR_Q5_0: case OR_Q5_1: return 32;
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_Q8_K: case OR_IQ2_XS: case OR_IQ2_XXS: case OR_IQ4_XS: case OR_Q2_K:
    case OR_Q3_K: case OR_IQ3_XXS: case OR_IQ3_S: case OR_IQ2_S: case OR_IQ1_S: return 256;
    default: return 0;
    }
}
/* ggml's vec_dot_type: Q8_0 for IQ4_NL, Q8_0, MXFP4 and Q5_0 weights, Q8_K for the K-quants and the 256-block IQ types
   (the activation quantizer is chosen per weight type: src/cpu_moe.cpp:711-715).  Q5_1's partner there is Q8_1, whose d
   and q are Q8_0's and whose s is fp16(d sum q); here Q5_1 takes the Q8_0 row and the exact integer sum q instead of s */
int or_vec_dot_type(int type) {
    switch (type) {
    case OR_IQ4_NL: case OR_Q8_0: case OR_MXFP4: case OR_Q5_0: case OR_Q5_1: return OR_Q8_0;
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_IQ2_XS: case OR_IQ2_XXS: case OR_IQ4_XS: case OR_Q2_K: case OR_Q3_K: case OR_IQ3_XXS:
    case OR_IQ3_S: case OR_IQ2_S: case OR_IQ1_S: return OR_Q8_K;
    default: return -1;
    }
}

/* IQ4_NL / IQ4_XS codebook (src/kernels4.cu:546) */
static const int8_t kv_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* MXFP4 codebook: the E2M1 values doubled (src/kernels4.cu:550-551) */
static const int8_t kv_mxfp4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
/* the MXFP4 block scale 2^(e - 128), ggml_e8m0_to_fp32_half (src/kernels4.cu:567-568): the fp32 bit pattern
   (e - 1) << 23 for e >= 2, the subnormals 0x00200000 << e for e = 0, 1 */
static float e8m0_half(unsigned e) {
    const uint32_t bits = e < 2 ? 0x00200000u << e : (e - 1) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IQ2_XS codebook: 512 rows, base-3 coded; expanded once (values of src/iq_grids.h:80-209) */
static const uint16_t iq2xs_code[512] = {
#include "../hyper_amd/csrc/iq2xs_grid.inc"
};
/* IQ2_XXS codebook: 256 rows, the same coding (values of src/iq_grids.h:14-79) */
static const uint16_t iq2xxs_code[256] = {
#include "../hyper_amd/csrc/iq2xxs_grid.inc"
};
/* IQ3_XXS codebook: 256 rows of 4 bytes, base-8 coded, digit i = byte i's level 4 + 8 d (62 for d = 7) (values of
   src/iq_grids.h:468-503) */
static const uint16_t iq3xxs_code[256] = {
#include "../hyper_amd/csrc/iq3xxs_grid.inc"
};
/* IQ3_S codebook: 512 rows of 4 bytes, base-8 coded, digit i = byte i's level 2 d + 1 (values of
   src/kernels4.cu:480-545) */
static const uint16_t iq3s_code[512] = {
#include "../hyper_amd/csrc/iq3s_grid.inc"
};
/* IQ2_S codebook: 1024 rows of 8 bytes, base-3 coded as IQ2_XS's (values of src/iq_grids.h:210-467) */
static const uint16_t iq2s_code[1024] = {
#include "../hyper_amd/csrc/iq2s_grid.inc"
};
/* IQ1_S codebook: 2048 rows of 8 int8 values in {-1, 0, 1}, base-3 coded with digit = value + 1 (values of
   src/iq_grids.h:504-1017) */
static const uint16_t iq1s_code[2048] = {
#include "../hyper_amd/csrc/iq1s_grid.inc"
};
static uint8_t iq2xs_rows[512][8], iq2xxs_rows[256][8], iq2s_rows[1024][8], iq3xxs_rows[256][4], iq3s_rows[512][4];
static int8_t iq1s_rows[2048][8];
static int iq2xs_ready = 0;
static void iq2xs_init(void) {   /* the grid codebooks */
    if (__atomic_load_n(&iq2xs_ready, __ATOMIC_ACQUIRE)) return;
    static const uint8_t lv[3] = {8, 25, 43};
    for (int i = 0; i < 512; ++i) {
        unsigned c = iq2xs_code[i];
        for (int j = 0; j < 8; ++j) { iq2xs_rows[i][j] = lv[c % 3]; c /= 3; }
    }
    for (int i = 0; i < 256; ++i) {
        unsigned c = iq2xxs_code[i];
        for (int j = 0; j < 8; ++j) { iq2xxs_rows[i][j] = lv[c % 3]; c /= 3; }
    }
    for (int i = 0; i < 256; ++i) {
        unsigned c = iq3xxs_code[i];
        for (int j = 0; j < 4; ++j) { iq3xxs_rows[i][j] = (uint8_t) ((c & 7) == 7 ? 62 : 4 + 8 * (c & 7)); c >>= 3; }
    }
    for (int i = 0; i < 2048; ++i) {
        unsigned c = iq1s_code[i];
        for (int j = 0; j < 8; ++j) { iq1s_rows[i][j] = (int8_t) ((int) (c % 3) - 1); c /= 3; }
    }
    for (int i = 0; i < 1024; ++i) {
        unsigned c = iq2s_code[i];
        for (int j = 0; j < 8; ++j) { iq2s_rows[i][j] = lv[c % 3]; c /= 3; }
    }
    for (int i = 0; i < 512; ++i) {
        unsigned c = iq3s_code[i];
        for (int j = 0; j < 4; ++j) { iq3s_rows[i][j] = (uint8_t) (2 * (c & 7) + 1); c >>= 3; }
    }
    __atomic_store_n(&iq2xs_ready, 1, __ATOMIC_RELEASE);
}
/* the IQ2 sign table (src/iq_grids.h:4-13): 7 sign bits plus an 8th that makes the count even */
static inline uint8_t ksign(unsigned i) { return (uint8_t) (i | ((unsigned) __builtin_parity(i) << 7)); }

/* ------------------------------------------------------------------ scalar helpers */

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t s = (uint32_t) (h & 0x8000) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = s;
        else { float f = (float) m * (1.0f / 16777216.0f); memcpy(&x, &f, 4); x |= s; }
    } else if (e == 31) x = s | 0x7f800000 | (m << 13);
    else x = s | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &x, 4);
    return f;
}
uint16_t or_fp32_to_fp16(float f) {          /* round to nearest even */
    uint32_t x; memcpy(&x, &f, 4);
    const uint16_t s = (uint16_t) ((x >> 16) & 0x8000);
    const uint32_t a = x & 0x7fffffff;
    if (a >= 0x7f800000) return s | (a > 0x7f800000 ? 0x7e00 : 0x7c00);
    if (a >= 0x477ff000) return s | 0x7c00;                       /* >= 65520: inf */
    if (a < 0x38800000) {                                         /* below 2^-14: subnormal half */
        float v; memcpy(&v, &a, 4);
        return s | (uint16_t) lrintf(v * 16777216.0f);           /* exact scaling, RNE */
    }
    const uint32_t mant = a & 0x7fffff, rem = mant & 0x1fff;
    uint32_t h = ((((a >> 23) - 112) << 10) | (mant >> 13));
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h;
    return s | (uint16_t) h;
}

/* exp(x): Cody-Waite reduction x = n ln2 + r with ln2 = C1 + C2 (C1 exact in 9 bits), exp(r) by the Cephes
   degree-5 polynomial (S. L. Moshier, Cephes Math Library, expf.c), 2^n applied as two exact power-of-two
   scalings.  Results below exp(-87) (about 1.6e-38) are flushed to 0, so no subnormal is ever produced. */
float or_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    const float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693359375f, x);
    r = fmaf(n, 2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    const float z = r * r;
    float y = fmaf(p, z, r);
    y = y + 1.0f;
    const int ni = (int) n, n1 = ni / 2, n2 = ni - n1;
    uint32_t b1 = (uint32_t) (n1 + 127) << 23, b2 = (uint32_t) (n2 + 127) << 23;
    float s1, s2; memcpy(&s1, &b1, 4); memcpy(&s2, &b2, 4);
    return (y * s1) * s2;
}
/* src/cpu_moe.cpp:29 */
float or_silu(float x) { return x / (1.0f + or_expf(-x)); }

/* ------------------------------------------------------------------ activation quantizers */

/* Q8_K (src/cpu_moe.cpp:35-78, ggml's quantize_row_q8_K): first-occurrence signed max, iscale = -127/max,
   products rounded by the 1.5 * 2^23 trick, min(127, v), int16 sums of 16, d = 1/iscale.  An all-zero
   block gets d = 0, qs = 0 and (unlike the reference, which leaves them) bsums = 0. */
static inline int nearest_int(float f) {
    float v = f + 12582912.f;
    int i; memcpy(&i, &v, 4);
    return (i & 0x007fffff) - 0x00400000;
}
void or_quantize_q8_K(const float *x, void *vy, int n) {
    uint8_t *y = (uint8_t *) vy;
    for (int i = 0; i < n / 256; ++i, x += 256, y += 292) {
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 256; ++j) { const float ax = fabsf(x[j]); if (ax > amax) { amax = ax; mx = x[j]; } }
        int8_t qs[256];
        int16_t bs[16];
        float d;
        if (amax == 0.0f) {
            d = 0.0f; memset(qs, 0, sizeof qs); memset(bs, 0, sizeof bs);
        } else {
            const float iscale = -127.f / mx;
            for (int j = 0; j < 256; ++j) {
                const float pr = iscale * x[j];
                const int v = nearest_int(pr);
                qs[j] = (int8_t) (v < 127 ? v : 127);
            }
            for (int j = 0; j < 16; ++j) { int s = 0; for (int l = 0; l < 16; ++l) s += qs[16 * j + l]; bs[j] = (int16_t) s; }
            d = 1.0f / iscale;
        }
        memcpy(y, &d, 4); memcpy(y + 4, qs, 256); memcpy(y + 260, bs, 32);
    }
}
/* Q8_0 as ggml's x86 (AVX2) quantize_row_q8_0 computes it (the path the reference reaches through
   from_float for IQ4_NL activations, src/cpu_moe.cpp:711-715): amax over 32, d = amax / 127 stored as fp16,
   id = 127 / amax (0 for an all-zero block), q = round-to-nearest-even(x * id). */
void or_quantize_q8_0(const float *x, void *vy, int n) {
    uint8_t *y = (uint8_t *) vy;
    for (int i = 0; i < n / 32; ++i, x += 32, y += 34) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.f;
        const uint16_t dh = or_fp32_to_fp16(d);
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        memcpy(y, &dh, 2);
        for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t) (int8_t) (int) rintf(x[j] * id);
    }
}
int or_quantize_row(int vtype, const float *x, void *y, int n) {
    if (vtype == OR_Q8_K) { if (n % 256) return -1; or_quantize_q8_K(x, y, n); return 0; }
    if (vtype == OR_Q8_0) { if (n % 32) return -1; or_quantize_q8_0(x, y, n); return 0; }
    return -1;
}

/* ------------------------------------------------------------------ block decoding */

static inline float h2f(const uint8_t *p) { uint16_t h; memcpy(&h, p, 2); return or_fp16_to_fp32(h); }

/* src/kernels4.cu:423-426 */
static inline void scale_min_k4(int j, const uint8_t *q, int *d, int *m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else { *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}
/* quant value of element e (0..255) of a Q4_K super-block: nibble e % 32 of sub-block e / 32 sits at
   byte 16 + 32 (j / 2) + l, low nibble for even j (src/kernels4.cu:427-436) */
static inline int q4k_q(const uint8_t *b, int e) {
    const int j = e >> 5, l = e & 31;
    return (b[16 + 32 * (j >> 1) + l] >> (4 * (j & 1))) & 0xF;
}
/* Q5_K: as Q4_K with qs at 48 and bit j of qh[l] as bit 4 (src/kernels4.cu:437-448) */
static inline int q5k_q(const uint8_t *b, int e) {
    const int j = e >> 5, l = e & 31;
    return ((b[48 + 32 * (j >> 1) + l] >> (4 * (j & 1))) & 0xF) | (((b[16 + l] >> j) & 1) << 4);
}
/* Q6_K: q6 - 32 of element e (src/kernels4.cu:671-681) */
static inline int q6k_q(const uint8_t *b, int e) {
    const int hf = e >> 7, qt = (e >> 5) & 3, l = e & 31;
    const int lo = (b[hf * 64 + (qt & 1) * 32 + l] >> (qt >= 2 ? 4 : 0)) & 0xF;
    const int hi = (b[128 + hf * 32 + l] >> (2 * qt)) & 3;
    return (lo | (hi << 4)) - 32;
}
/* IQ4_XS 6-bit group scale ls of 32-group ib (src/kernels4.cu:660-670) */
static inline int iq4xs_ls(const uint8_t *b, int ib) {
    const unsigned sh = (unsigned) b[2] | ((unsigned) b[3] << 8);
    return ((b[4 + (ib >> 1)] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
}
static inline int iq4xs_q(const uint8_t *b, int e) {    /* codebook value of element e */
    const int ib = e >> 5, l = e & 31;
    return kv_iq4nl[(b[8 + 16 * ib + (l & 15)] >> (l >= 16 ? 4 : 0)) & 0xF];
}
static inline int iq4nl_q(const uint8_t *b, int e) {    /* element e (0..31) of an 18-byte block */
    return kv_iq4nl[(b[2 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF];
}
/* element e (0..31) of a 17-byte MXFP4 block (e, qs[16]): value j < 16 from the low nibble of qs[j], 16 + j from
   its high nibble (src/kernels4.cu:569-577) */
static inline int mxfp4_q(const uint8_t *b, int e) {
    return kv_mxfp4[(b[1 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF];
}
/* element e (0..255) of an 84-byte Q2_K block: 2-bit field 2 ((e >> 5) & 3) of qs byte 32 (e >> 7) + (e & 31) (qs at
   16); its 16-group e >> 4 has scale byte e >> 4: low nibble the scale, high nibble the min (src/kernels4.cu:639-647) */
static inline int q2k_q(const uint8_t *b, int e) { return (b[16 + 32 * (e >> 7) + (e & 31)] >> (2 * ((e >> 5) & 3))) & 3; }
/* element e = 128 hf + 32 j + l of a 110-byte Q3_K block (hmask[32], qs[64] @32, scales[12] @96, d @108): the 2-bit
   field 2 j of qs byte 32 hf + l, less 4 where bit 4 hf + j of hmask[l] is clear; the signed 6-bit scale of 16-group is
   from bytes 96 + 4 ((is >> 2) & 1) + (is & 3) (a nibble, by is >> 3) and 104 + (is & 3) (two bits, by is >> 2)
   (src/kernels4.cu:698-707) */
static inline int q3k_q(const uint8_t *b, int e) {
    const int hf = e >> 7, j = (e >> 5) & 3, l = e & 31;
    return ((b[32 + 32 * hf + l] >> (2 * j)) & 3) - ((b[l] & (1 << (4 * hf + j))) ? 0 : 4);
}
static inline int q3k_sc(const uint8_t *b, int is) {
    const int grp = is >> 2, k = is & 3;
    return (((b[96 + (grp & 1) * 4 + k] >> (4 * (grp >> 1))) & 0xF) | (((b[104 + k] >> (2 * grp)) & 3) << 4)) - 32;
}
/* element e (0..31) of a 24-byte Q5_1 block (d, m, qh u32 @4, qs[16] @8): nibble | qh bit e << 4, 0..31, the nibble
   the low one of qs[e] for e < 16, else the high one of qs[e - 16] (src/kernels4.cu:449-462); value x d + m */
static inline int q5_1_q(const uint8_t *b, int e) {
    const uint32_t qh = (uint32_t) b[4] | ((uint32_t) b[5] << 8) | ((uint32_t) b[6] << 16) | ((uint32_t) b[7] << 24);
    return ((b[8 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF) | (((qh >> e) & 1) << 4);
}
/* element e (0..31) of a 22-byte Q5_0 block (d, qh u32, qs[16]): (nibble | qh bit e << 4) - 16, the nibble the low
   one of qs[e] for e < 16, else the high one of qs[e - 16] (src/kernels4.cu:464-478) */
static inline int q5_0_q(const uint8_t *b, int e) {
    const uint32_t qh = (uint32_t) b[2] | ((uint32_t) b[3] << 8) | ((uint32_t) b[4] << 16) | ((uint32_t) b[5] << 24);
    return (((b[6 + (e & 15)] >> (e >= 16 ? 4 : 0)) & 0xF) | (((qh >> e) & 1) << 4)) - 16;
}
/* IQ2_XS signed grid value of element e and the 4-bit scale of its 8-group (src/kernels4.cu:592-601) */
static inline int iq2xs_q(const uint8_t *b, int e) {
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const unsigned q = (unsigned) b[2 + 2 * (4 * ib + l)] | ((unsigned) b[3 + 2 * (4 * ib + l)] << 8);
    const int g = iq2xs_rows[q & 511][j];
    return (ksign(q >> 9) >> j) & 1 ? -g : g;
}
/* IQ2_XXS (src/kernels4.cu:578-589): 32-group ib is two words at 2 + 8 ib -- grid rows (byte l of the first) and
   4 x 7 sign bits with the 4-bit scale in bits 28..31 (the second) */
static inline unsigned iq2xxs_a1(const uint8_t *b, int ib) {
    return (unsigned) b[6 + 8 * ib] | ((unsigned) b[7 + 8 * ib] << 8) | ((unsigned) b[8 + 8 * ib] << 16) | ((unsigned) b[9 + 8 * ib] << 24);
}
static inline int iq2xxs_q(const uint8_t *b, int e) {   /* signed grid value of element e */
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const int g = iq2xxs_rows[b[2 + 8 * ib + l]][j];
    return (ksign((iq2xxs_a1(b, ib) >> (7 * l)) & 127) >> j) & 1 ? -g : g;
}
/* IQ3_XXS (src/kernels4.cu:613-627): 32-group ib has the grid indices qs[8 ib .. 8 ib + 7] at 2 (two 4-byte rows per
   8-group l) and the word at 66 + 4 ib: 4 x 7 sign indices and the 4-bit scale in bits 28..31 */
static inline unsigned iq3xxs_a(const uint8_t *b, int ib) {
    return (unsigned) b[66 + 4 * ib] | ((unsigned) b[67 + 4 * ib] << 8) | ((unsigned) b[68 + 4 * ib] << 16) | ((unsigned) b[69 + 4 * ib] << 24);
}
static inline int iq3xxs_q(const uint8_t *b, int e) {   /* signed grid value of element e */
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const int g = iq3xxs_rows[b[2 + 8 * ib + 2 * l + (j >> 2)]][j & 3];
    return (ksign((iq3xxs_a(b, ib) >> (7 * l)) & 127) >> j) & 1 ? -g : g;
}
/* IQ3_S (src/kernels4.cu:682-695): element e of 32-group ib, 8-group l, position j: grid row qs[8 ib + 2 l + j / 4]
   (qs at 2) with bit 2 l + j / 4 of qh[ib] (at 66) as its 9th bit, byte j % 4; negated where bit j of signs[4 ib + l]
   (at 74) is set; the group's scale is nibble ib & 1 of scales[ib / 2] (at 106) */
static inline int iq3s_q(const uint8_t *b, int e) {
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7, hb = 2 * l + (j >> 2);
    const int g = iq3s_rows[b[2 + 8 * ib + hb] | (((b[66 + ib] >> hb) & 1) << 8)][j & 3];
    return (b[74 + 4 * ib + l] >> j) & 1 ? -g : g;
}
/* IQ2_S (src/kernels4.cu:602-613): element e of 32-group ib, 8-group l, position j: grid row qs[4 ib + l] (qs at 2)
   with bits 2 l, 2 l + 1 of qh[ib] (at 66) as index bits 8-9, byte j; negated where bit j of signs[4 ib + l] (at 34)
   is set; its 16-group's scale is nibble l / 2 of scales[ib] (at 74) */
static inline int iq2s_q(const uint8_t *b, int e) {
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const int g = iq2s_rows[b[2 + 4 * ib + l] | (((b[66 + ib] >> (2 * l)) & 3) << 8)][j];
    return (b[34 + 4 * ib + l] >> j) & 1 ? -g : g;
}
/* IQ1_S (src/kernels4.cu:650-659): element e of 32-group ib, 8-group l, position j: grid row qs[4 ib + l] (qs at 2)
   with 3 bits (3 l) of qh[ib] (u16 at 34) as index bits 8-10, value j (-1, 0 or 1); the group's scale 2 ((qh >> 12) & 7)
   + 1, its delta -1/8 if qh's top bit is set, else +1/8 */
static inline unsigned iq1s_qh(const uint8_t *b, int ib) { return (unsigned) b[34 + 2 * ib] | ((unsigned) b[35 + 2 * ib] << 8); }
static inline int iq1s_q(const uint8_t *b, int e) {
    const int ib = e >> 5, l = (e >> 3) & 3;
    return iq1s_rows[b[2 + 4 * ib + l] | (((iq1s_qh(b, ib) >> (3 * l)) & 7) << 8)][e & 7];
}
static inline int iq1s_ls(const uint8_t *b, int ib) { return 2 * (int) ((iq1s_qh(b, ib) >> 12) & 7) + 1; }
static inline int iq2s_sc(const uint8_t *b, int e) { return (b[74 + (e >> 5)] >> (4 * ((e >> 4) & 1))) & 15; }
static inline int iq3s_sc(const uint8_t *b, int ib) { return (b[106 + (ib >> 1)] >> (4 * (ib & 1))) & 15; }
static inline int iq2xs_sc(const uint8_t *b, int e) {
    const int ib = e >> 5, l = (e >> 3) & 3;
    return (b[66 + ib] >> (4 * (l >> 1))) & 0xF;
}

/* dequantized values: the deq8<T> expressions (src/kernels4.cu:427-714), each product rounded */
int or_dequant_row(int type, const uint8_t *row, int n, float *out) {
    const int be = or_block_elems(type);
    const size_t bb = or_block_bytes(type);
    if (!be || n % be) return -1;
    iq2xs_init();
    for (int ib = 0; ib < n / be; ++ib) {
        const uint8_t *b = row + ib * bb;
        float *o = out + (size_t) ib * be;
        switch (type) {
        case OR_Q4_K: case OR_Q5_K:
            for (int e = 0; e < 256; ++e) {
                int sc, m; scale_min_k4(e >> 5, b + 4, &sc, &m);
                const float d = h2f(b) * (float) sc, mn = h2f(b + 2) * (float) m;
                const int q = type == OR_Q4_K ? q4k_q(b, e) : q5k_q(b, e);
                o[e] = d * (float) q - mn;
            }
            break;
        case OR_Q6_K:
            for (int e = 0; e < 256; ++e) {
                const int hf = e >> 7, qt = (e >> 5) & 3, l = e & 31;
                const float d = h2f(b + 208) * (float) (int8_t) b[192 + hf * 8 + (l >> 4) + 2 * qt];
                o[e] = d * (float) q6k_q(b, e);
            }
            break;
        case OR_IQ4_XS:
            for (int e = 0; e < 256; ++e) o[e] = (h2f(b) * (float) (iq4xs_ls(b, e >> 5) - 32)) * (float) iq4xs_q(b, e);
            break;
        case OR_IQ4_NL:
            for (int e = 0; e < 32; ++e) o[e] = (float) iq4nl_q(b, e) * h2f(b);
            break;
        case OR_IQ2_XS:
            for (int e = 0; e < 256; ++e) {
                const float db = h2f(b) * (0.5f + (float) iq2xs_sc(b, e)) * 0.25f;
                const int q = iq2xs_q(b, e);
                o[e] = (db * (float) (q < 0 ? -q : q)) * (q < 0 ? -1.0f : 1.0f);
            }
            break;
        case OR_IQ2_XXS:
            for (int e = 0; e < 256; ++e) {
                const float db = h2f(b) * (0.5f + (float) (iq2xxs_a1(b, e >> 5) >> 28)) * 0.25f;
                const int q = iq2xxs_q(b, e);
                o[e] = (db * (float) (q < 0 ? -q : q)) * (q < 0 ? -1.0f : 1.0f);
            }
            break;
        case OR_Q8_0:
            for (int e = 0; e < 32; ++e) o[e] = h2f(b) * (float) (int8_t) b[2 + e];
            break;
        case OR_IQ1_S:
            for (int e = 0; e < 256; ++e) {
                const float dl = h2f(b) * (float) iq1s_ls(b, e >> 5);
                const float delta = iq1s_qh(b, e >> 5) & 0x8000 ? -0.125f : 0.125f;
                o[e] = dl * ((float) iq1s_q(b, e) + delta);
            }
            break;
        case OR_IQ2_S:
            for (int e = 0; e < 256; ++e) {
                const float db = h2f(b) * (0.5f + (float) iq2s_sc(b, e)) * 0.25f;
                const int q = iq2s_q(b, e);
                o[e] = (db * (float) (q < 0 ? -q : q)) * (q < 0 ? -1.0f : 1.0f);
            }
            break;
        case OR_IQ3_S:
            for (int e = 0; e < 256; ++e) {
                const float db = h2f(b) * (float) (1 + 2 * iq3s_sc(b, e >> 5));
                const int q = iq3s_q(b, e);
                o[e] = (db * (float) (q < 0 ? -q : q)) * (q < 0 ? -1.0f : 1.0f);
            }
            break;
        case OR_IQ3_XXS:
            for (int e = 0; e < 256; ++e) {
                const float db = h2f(b) * (0.5f + (float) (iq3xxs_a(b, e >> 5) >> 28)) * 0.5f;
                const int q = iq3xxs_q(b, e);
                o[e] = (db * (float) (q < 0 ? -q : q)) * (q < 0 ? -1.0f : 1.0f);
            }
            break;
        case OR_MXFP4:
            for (int e = 0; e < 32; ++e) o[e] = (float) mxfp4_q(b, e) * e8m0_half(b[0]);
            break;
        case OR_Q5_0:
            for (int e = 0; e < 32; ++e) o[e] = (float) q5_0_q(b, e) * h2f(b);
            break;
        case OR_Q5_1:
            for (int e = 0; e < 32; ++e) o[e] = (float) q5_1_q(b, e) * h2f(b) + h2f(b + 2);
            break;
        case OR_Q3_K:
            for (int e = 0; e < 256; ++e) o[e] = (h2f(b + 108) * (float) q3k_sc(b, e >> 4)) * (float) q3k_q(b, e);
            break;
        case OR_Q2_K:
            for (int e = 0; e < 256; ++e) {
                const int sc = b[e >> 4];
                const float dl = h2f(b + 80) * (float) (sc & 15), ml = h2f(b + 82) * (float) (sc >> 4);
                o[e] = dl * (float) q2k_q(b, e) - ml;
            }
            break;
        case OR_Q8_K: {
            float d; memcpy(&d, b, 4);
            for (int e = 0; e < 256; ++e) o[e] = d * (float) (int8_t) b[4 + e];
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ integer block dots */

/* exact integers of one weight block (type, bytes b) against activation block y (Q8_K: 292 B, Q8_0: 34 B).
   K-quants: sumi = sum_j sc_j S_j, summ = sum_j m_j (bsums[2j] + bsums[2j+1]) (ggml q4_K/q5_K x q8_K);
   Q6_K: sumi = sum_g sc_g sum_16 (q6 - 32) y; IQ4_XS: sumi = sum_ib (ls - 32) sum_32 kv y (src/iq3s_dot.h:
   136-166); IQ2_XS: sumi = sum (2 sc + 1) sum_16 grid sign y; IQ4_NL x Q8_0: sumi = sum_32 kv q8; Q8_0 x Q8_0:
   sumi = sum_32 q q8 (ggml's vec_dot_q8_0_q8_0 integer part); MXFP4 x Q8_0: sumi = sum_32 kv q8; Q5_0 x Q8_0: sumi = sum_32 (x - 16) q8. */
static void block_ints_scalar(int type, const uint8_t *b, const uint8_t *y, int32_t *sumi, int32_t *summ) {
    int32_t si = 0, sm = 0;
    const int8_t *q8 = (const int8_t *) (y + (or_vec_dot_type(type) == OR_Q8_0 ? 2 : 4));
    switch (type) {
    case OR_Q4_K: case OR_Q5_K: {
        int16_t bs[16]; memcpy(bs, y + 260, 32);
        for (int j = 0; j < 8; ++j) {
            int sc, m; scale_min_k4(j, b + 4, &sc, &m);
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += (type == OR_Q4_K ? q4k_q(b, 32 * j + l) : q5k_q(b, 32 * j + l)) * q8[32 * j + l];
            si += sc * s;
            sm += m * (bs[2 * j] + bs[2 * j + 1]);
        }
        break;
    }
    case OR_Q6_K:
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += q6k_q(b, 16 * g + l) * q8[16 * g + l];
            si += (int8_t) b[192 + g] * s;
        }
        break;
    case OR_IQ4_XS:
        for (int ib = 0; ib < 8; ++ib) {
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += iq4xs_q(b, 32 * ib + l) * q8[32 * ib + l];
            si += (iq4xs_ls(b, ib) - 32) * s;
        }
        break;
    case OR_IQ2_XS:
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += iq2xs_q(b, 16 * g + l) * q8[16 * g + l];
            si += (2 * iq2xs_sc(b, 16 * g) + 1) * s;
        }
        break;
    case OR_IQ4_NL:
        for (int l = 0; l < 32; ++l) si += iq4nl_q(b, l) * q8[l];
        break;
    case OR_Q8_0:
        for (int l = 0; l < 32; ++l) si += (int8_t) b[2 + l] * q8[l];
        break;
    case OR_MXFP4:     /* ggml's vec_dot_mxfp4_q8_0 integer part: sum_32 kv q8 */
        for (int l = 0; l < 32; ++l) si += mxfp4_q(b, l) * q8[l];
        break;
    case OR_Q5_0:      /* ggml's vec_dot_q5_0_q8_0 integer part: sum_32 (x - 16) q8 */
        for (int l = 0; l < 32; ++l) si += q5_0_q(b, l) * q8[l];
        break;
    case OR_Q5_1:      /* ggml's vec_dot_q5_1_q8_1 integer part sum_32 x q8, and the activation sum sum_32 q8 */
        for (int l = 0; l < 32; ++l) { si += q5_1_q(b, l) * q8[l]; sm += q8[l]; }
        break;
    case OR_IQ1_S: {   /* the reference's IQ1_S x Q8_K dot (src/iq1s_dot.h:26-64): sumi = sum_ib ls sum_32 grid y,
                          summ = sum_ib ls (-1 if qh's top bit) (sum_32 y, the bsum pair) */
        int16_t bs[16]; memcpy(bs, y + 260, 32);
        for (int ib = 0; ib < 8; ++ib) {
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += iq1s_q(b, 32 * ib + l) * q8[32 * ib + l];
            const int ls = iq1s_ls(b, ib);
            si += ls * s;
            sm += (iq1s_qh(b, ib) & 0x8000 ? -ls : ls) * (bs[2 * ib] + bs[2 * ib + 1]);
        }
        break;
    }
    case OR_IQ2_S:     /* ggml's vec_dot_iq2_s_q8_K: sum over 16-groups (2 sc + 1) sum_16 grid sign y */
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += iq2s_q(b, 16 * g + l) * q8[16 * g + l];
            si += (2 * iq2s_sc(b, 16 * g) + 1) * s;
        }
        break;
    case OR_IQ3_S:     /* the reference's IQ3_S x Q8_K dot (src/iq3s_dot.h:48-76): sum_ib (2 sc + 1) sum_32 grid sign y */
        for (int ib = 0; ib < 8; ++ib) {
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += iq3s_q(b, 32 * ib + l) * q8[32 * ib + l];
            si += (2 * iq3s_sc(b, ib) + 1) * s;
        }
        break;
    case OR_IQ3_XXS:   /* ggml's vec_dot_iq3_xxs_q8_K: sum_ib (2 sc + 1) sum_32 grid sign y */
        for (int ib = 0; ib < 8; ++ib) {
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += iq3xxs_q(b, 32 * ib + l) * q8[32 * ib + l];
            si += (2 * (int) (iq3xxs_a(b, ib) >> 28) + 1) * s;
        }
        break;
    case OR_Q3_K:      /* ggml's vec_dot_q3_K_q8_K: sum_g sc_g sum_16 q y */
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += q3k_q(b, 16 * g + l) * q8[16 * g + l];
            si += q3k_sc(b, g) * s;
        }
        break;
    case OR_Q2_K: {    /* ggml's vec_dot_q2_K_q8_K: sumi = sum_g sc_g sum_16 q q8, summ = sum_g m_g bsum_g */
        int16_t bs[16]; memcpy(bs, y + 260, 32);
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += q2k_q(b, 16 * g + l) * q8[16 * g + l];
            si += (b[g] & 15) * s;
            sm += (b[g] >> 4) * bs[g];
        }
        break;
    }
    case OR_IQ2_XXS:   /* ggml's vec_dot_iq2_xxs_q8_K: sum_ib (2 sc + 1) sum_32 grid sign y */
        for (int ib = 0; ib < 8; ++ib) {
            int32_t s = 0;
            for (int l = 0; l < 32; ++l) s += iq2xxs_q(b, 32 * ib + l) * q8[32 * ib + l];
            si += (2 * (int) (iq2xxs_a1(b, ib) >> 28) + 1) * s;
        }
        break;
    default: break;
    }
    *sumi = si; *summ = sm;
}
#if defined(__AVX2__)
#include <immintrin.h>
/* The same integers with AVX2 for the K-quants (the CPU baseline's speed; the scalar restatement above stays the
   definition, and tests/test_oracle.py checks the two against each other).  Integer sums do not depend on their
   order: maddubs forms exact int16 pair sums (|q y + q y| <= 63 * 127 * 2 < 2^15), madd with the broadcast scale
   exact int32 products, and everything stays far below 2^31. */
static inline int32_t hsum8_epi32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}
/* Q4_K / Q5_K: sub-block j's 32 values are the low (even j) or high (odd j) nibbles of qs[32 (j / 2) ..], plus bit j
   of qh[l] as bit 4 for Q5_K; sumi = sum_j sc_j S_j, summ = sum_j m_j (bsums[2j] + bsums[2j+1]) */
static void block_ints_q45k_avx2(int type, const uint8_t *b, const uint8_t *y, int32_t *sumi, int32_t *summ) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), one = _mm256_set1_epi8(1);
    const int8_t *q8 = (const int8_t *) (y + 4);
    int16_t bs[16]; memcpy(bs, y + 260, 32);
    const uint8_t *qs = b + (type == OR_Q4_K ? 16 : 48);
    const __m256i qh = type == OR_Q5_K ? _mm256_loadu_si256((const __m256i *) (b + 16)) : _mm256_setzero_si256();
    __m256i acc = _mm256_setzero_si256();
    int32_t sm = 0;
    for (int j2 = 0; j2 < 4; ++j2) {
        const __m256i raw = _mm256_loadu_si256((const __m256i *) (qs + 32 * j2));
        __m256i v[2] = {_mm256_and_si256(raw, m4), _mm256_and_si256(_mm256_srli_epi16(raw, 4), m4)};
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * j2 + h;
            if (type == OR_Q5_K) v[h] = _mm256_or_si256(v[h], _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, j), one), 4));
            int sc, m; scale_min_k4(j, b + 4, &sc, &m);
            const __m256i p16 = _mm256_maddubs_epi16(v[h], _mm256_loadu_si256((const __m256i *) (q8 + 32 * j)));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p16, _mm256_set1_epi16((short) sc)));
            sm += m * (bs[2 * j] + bs[2 * j + 1]);
        }
    }
    *sumi = hsum8_epi32(acc); *summ = sm;
}
/* Q6_K: value e = 128 hf + 32 qt + l is nibble (qt >= 2) of ql[64 hf + 32 (qt & 1) + l] | bits 2 qt of qh[32 hf + l] << 4;
   sum_g sc_g sum_16 (q6 - 32) y = sum_g sc_g sum_16 q6 y - 32 sum_g sc_g bsums[g] */
static void block_ints_q6k_avx2(const uint8_t *b, const uint8_t *y, int32_t *sumi) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(0x03);
    const int8_t *q8 = (const int8_t *) (y + 4), *sc = (const int8_t *) (b + 192);
    int16_t bs[16]; memcpy(bs, y + 260, 32);
    __m256i acc = _mm256_setzero_si256();
    for (int hf = 0; hf < 2; ++hf) {
        const __m256i l0 = _mm256_loadu_si256((const __m256i *) (b + 64 * hf)), l1 = _mm256_loadu_si256((const __m256i *) (b + 64 * hf + 32));
        const __m256i h = _mm256_loadu_si256((const __m256i *) (b + 128 + 32 * hf));
        for (int qt = 0; qt < 4; ++qt) {
            const __m256i src = (qt & 1) ? l1 : l0;
            const __m256i nib = qt >= 2 ? _mm256_and_si256(_mm256_srli_epi16(src, 4), m4) : _mm256_and_si256(src, m4);
            const __m256i hb = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2 * qt), m2), 4);
            const __m256i q = _mm256_or_si256(nib, hb);
            const __m256i p16 = _mm256_maddubs_epi16(q, _mm256_loadu_si256((const __m256i *) (q8 + 128 * hf + 32 * qt)));
            const int g = 8 * hf + 2 * qt;
            const __m256i s16 = _mm256_set_m128i(_mm_set1_epi16(sc[g + 1]), _mm_set1_epi16(sc[g]));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p16, s16));
        }
    }
    int32_t off = 0;
    for (int g = 0; g < 16; ++g) off += sc[g] * bs[g];
    *sumi = hsum8_epi32(acc) - 32 * off;
}
#endif

static void block_ints(int type, const uint8_t *b, const uint8_t *y, int32_t *sumi, int32_t *summ) {
#if defined(__AVX2__)
    if (type == OR_Q4_K || type == OR_Q5_K) { block_ints_q45k_avx2(type, b, y, sumi, summ); return; }
    if (type == OR_Q6_K) { block_ints_q6k_avx2(b, y, sumi); *summ = 0; return; }
#endif
    block_ints_scalar(type, b, y, sumi, summ);
}

static int dot_ok(int type) {
    return type == OR_Q4_K || type == OR_Q5_K || type == OR_Q6_K || type == OR_IQ4_XS || type == OR_IQ2_XS || type == OR_IQ4_NL ||
           type == OR_Q8_0 || type == OR_IQ2_XXS || type == OR_MXFP4 || type == OR_Q5_0 || type == OR_Q2_K || type == OR_Q3_K ||
           type == OR_IQ3_XXS || type == OR_IQ3_S || type == OR_IQ2_S || type == OR_IQ1_S ||
           type == OR_Q5_1;
}
int or_block_ints(int type, const uint8_t *row, const void *xq, int n, int32_t *sumi, int32_t *summ) {
    if (!dot_ok(type) || n % or_block_elems(type)) return -1;
    iq2xs_init();
    const size_t bb = or_block_bytes(type), yb = or_block_bytes(or_vec_dot_type(type));
    for (int ib = 0; ib < n / or_block_elems(type); ++ib)
        block_ints(type, row + ib * bb, (const uint8_t *) xq + ib * yb, sumi + ib, summ + ib);
    return 0;
}
int or_block_ints_scalar(int type, const uint8_t *row, const void *xq, int n, int32_t *sumi, int32_t *summ) {
    if (!dot_ok(type) || n % or_block_elems(type)) return -1;
    iq2xs_init();
    const size_t bb = or_block_bytes(type), yb = or_block_bytes(or_vec_dot_type(type));
    for (int ib = 0; ib < n / or_block_elems(type); ++ib)
        block_ints_scalar(type, row + ib * bb, (const uint8_t *) xq + ib * yb, sumi + ib, summ + ib);
    return 0;
}
/* the contract's per-block fp32 fold, blocks accumulated in order */
static float row_dot(int type, const uint8_t *row, const uint8_t *xq, int n) {
    const size_t bb = or_block_bytes(type), yb = or_block_bytes(or_vec_dot_type(type));
    float acc = 0.0f;
    for (int ib = 0; ib < n / or_block_elems(type); ++ib) {
        const uint8_t *b = row + ib * bb, *y = xq + ib * yb;
        int32_t si, sm;
        block_ints(type, b, y, &si, &sm);
        float xd, t;
        if (or_vec_dot_type(type) == OR_Q8_0) xd = h2f(y); else memcpy(&xd, y, 4);
        switch (type) {
        case OR_Q4_K: case OR_Q5_K: t = fmaf(h2f(b), (float) si, -(h2f(b + 2) * (float) sm)); break;
        case OR_Q6_K: t = h2f(b + 208) * (float) si; break;
        case OR_Q3_K: t = h2f(b + 108) * (float) si; break;
        case OR_IQ3_XXS: t = (h2f(b) * 0.25f) * (float) si; break;
        case OR_IQ3_S: t = h2f(b) * (float) si; break;
        case OR_IQ1_S: t = (h2f(b) * 0.125f) * (float) (8 * si + sm); break;   /* exact: |8 si + sm| < 2^24 */
        case OR_Q5_1: t = fmaf(h2f(b), (float) si, h2f(b + 2) * (float) sm); break;
        case OR_Q2_K: t = fmaf(h2f(b + 80), (float) si, -(h2f(b + 82) * (float) sm)); break;
        case OR_IQ2_XS: case OR_IQ2_XXS: case OR_IQ2_S: t = (h2f(b) * 0.125f) * (float) si; break;
        case OR_MXFP4: t = e8m0_half(b[0]) * (float) si; break;
        default: t = h2f(b) * (float) si; break;        /* IQ4_XS, IQ4_NL, Q8_0, Q5_0 */
        }
        acc = fmaf(xd, t, acc);
    }
    return acc;
}
float or_row_dot(int type, const uint8_t *row, const void *xq, int n) {
    if (!dot_ok(type) || n % or_block_elems(type)) return NAN;
    iq2xs_init();
    return row_dot(type, row, (const uint8_t *) xq, n);
}

/* ------------------------------------------------------------------ router */

/* y[t][r] = W[r] . x[t] (the fp32 router GEMV, src/kernels4.cu:163-180) in the contract's order */
void or_gemv_f32(const float *W, int rows, int kdim, const float *x, int xs, float *y, int ys, int nt) {
    for (int t = 0; t < nt; ++t)
        for (int r = 0; r < rows; ++r) {
            const float *w = W + (size_t) r * kdim, *xv = x + (size_t) t * xs;
            float acc[64];
            for (int L = 0; L < 64; ++L) {
                float a = 0.0f;
                for (int i = 0; 256 * i + 4 * L < kdim; ++i)
                    for (int j = 0; j < 4; ++j) {
                        const int e = 256 * i + 4 * L + j;
                        if (e < kdim) a = fmaf(w[e], xv[e], a);
                    }
                acc[L] = a;
            }
            for (int off = 1; off < 64; off <<= 1) {
                float nx[64];
                for (int L = 0; L < 64; ++L) nx[L] = acc[L] + acc[L ^ off];
                memcpy(acc, nx, sizeof acc);
            }
            y[(size_t) t * ys + r] = acc[0];
        }
}
/* 64 partial sums (lane L: e = L + 64 i in order), then the xor butterfly 1, 2, ..., 32 */
static float tree_sum64(const float *v, int n) {
    float acc[64];
    for (int L = 0; L < 64; ++L) { float a = 0.0f; for (int e = L; e < n; e += 64) a = a + v[e]; acc[L] = a; }
    for (int off = 1; off < 64; off <<= 1) {
        float nx[64];
        for (int L = 0; L < 64; ++L) nx[L] = acc[L] + acc[L ^ off];
        memcpy(acc, nx, sizeof acc);
    }
    return acc[0];
}
/* softmax, top-k by (p descending, index ascending), weights renormalized over the selected in selection
   order, sg = sigmoid(logit ne) (src/kernels4.cu:297-344; ties: rt_better :295) */
int or_route(const float *logits, int ls, int ne, int k, int nt, int32_t *ids, float *wts, float *sg) {
    if (ne <= 0 || k <= 0 || k > ne || (sg && ls <= ne)) return -1;
    float *v = (float *) malloc(sizeof(float) * ne);
    unsigned char *used = (unsigned char *) malloc(ne);
    if (!v || !used) { free(v); free(used); return -1; }
    for (int t = 0; t < nt; ++t) {
        const float *l = logits + (size_t) t * ls;
        float mx = -INFINITY;
        for (int e = 0; e < ne; ++e) mx = fmaxf(mx, l[e]);
        for (int e = 0; e < ne; ++e) v[e] = or_expf(l[e] - mx);
        const float s = tree_sum64(v, ne);
        for (int e = 0; e < ne; ++e) v[e] = v[e] / s;
        memset(used, 0, ne);
        float sel[64];
        float tot = 0.0f;
        for (int j = 0; j < k; ++j) {
            int bi = -1;
            for (int e = 0; e < ne; ++e)
                if (!used[e] && (bi < 0 || v[e] > v[bi])) bi = e;   /* strict >: ties keep the lower index */
            used[bi] = 1;
            ids[(size_t) t * k + j] = bi;
            sel[j < 64 ? j : 63] = v[bi];
            tot = tot + v[bi];
        }
        for (int j = 0; j < k; ++j) wts[(size_t) t * k + j] = v[ids[(size_t) t * k + j]] / tot;
        if (sg) sg[t] = 1.0f / (1.0f + or_expf(-l[ne]));
        (void) sel;
    }
    free(v); free(used);
    return 0;
}

/* log(x) for x > 0: x = 2^e m with m in [sqrt(1/2), sqrt(2)), log(m) by the Cephes single-precision polynomial in
   f = m - 1 (S. L. Moshier, Cephes Math Library, logf.c) evaluated with fmaf, e ln2 added as e C2 + e C1 with
   C1 = 0.693359375 exact in 9 bits (the same split as or_expf).  Subnormal x is scaled by 2^23 first. */
float or_logf(float x) {
    if (x != x || x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (isinf(x)) return x;
    int e = 0;
    if (x < 1.17549435e-38f) { x = x * 8388608.0f; e = -23; }
    uint32_t b;
    memcpy(&b, &x, 4);
    e += (int) ((b >> 23) & 0xffu) - 126;   /* x = 2^e m, m in [0.5, 1) */
    const uint32_t mb = (b & 0x007fffffu) | 0x3f000000u;
    float m;
    memcpy(&m, &mb, 4);
    float f;
    if (m < 0.70710678118654752f) { e -= 1; f = m + m - 1.0f; } else { f = m - 1.0f; }
    const float z = f * f;
    float y = 7.0376836292e-2f;
    y = fmaf(y, f, -1.1514610310e-1f);
    y = fmaf(y, f, 1.1676998740e-1f);
    y = fmaf(y, f, -1.2420140846e-1f);
    y = fmaf(y, f, 1.4249322787e-1f);
    y = fmaf(y, f, -1.6668057665e-1f);
    y = fmaf(y, f, 2.0000714765e-1f);
    y = fmaf(y, f, -2.4999993993e-1f);
    y = fmaf(y, f, 3.3333331174e-1f);
    y = (y * f) * z;
    const float fe = (float) e;
    y = fmaf(fe, -2.12194440e-4f, y);
    y = fmaf(-0.5f, z, y);
    return fmaf(fe, 0.693359375f, f + y);
}
/* log(1 + x), x >= -1: u = 1 + x rounded, then log(u) x / (u - 1) (D. Goldberg, "What every computer scientist should
   know about floating-point arithmetic", 1991, theorem 4), which cancels the rounding of u; x itself when u == 1 */
float or_log1pf(float x) {
    if (x != x) return x;
    const float u = 1.0f + x;
    if (u == 1.0f) return x;
    if (isinf(u)) return u;
    return or_logf(u) * (x / (u - 1.0f));
}
/* the routers' scores: sigmoid 1 / (1 + exp(-l)) (src/kernels5.cu:35) and sqrt(softplus(l)) with softplus(l) = l
   above 20, else log1p(exp(l)) (src/kernels7.cu:823-826) */
float or_sigmoid(float l) { return 1.0f / (1.0f + or_expf(-l)); }
float or_sqrt_softplus(float l) { return sqrtf(l > 20.0f ? l : or_log1pf(or_expf(l))); }

/* top k of key (descending, ties to the lower index) -> ids; val of the selected summed in selection order */
static float topk_by_key(const float *key, const float *val, int ne, int k, unsigned char *used, int32_t *ids) {
    memset(used, 0, (size_t) ne);
    float tot = 0.0f;
    for (int j = 0; j < k; ++j) {
        int bi = -1;
        for (int e = 0; e < ne; ++e)
            if (!used[e] && (bi < 0 || key[e] > key[bi])) bi = e;   /* strict >: ties keep the lower index */
        used[bi] = 1;
        ids[j] = bi;
        tot = tot + val[bi];
    }
    return tot;
}
/* the sigmoid router with a selection bias (src/kernels5.cu:1090-1122): p = sigmoid(l), the top k of p + bias[e],
   weights p scale / max(sum of the selected p, 2^-14), sg = 1 */
int or_route_sig(const float *logits, int ls, const float *bias, int ne, int k, float scale, int nt, int32_t *ids, float *wts, float *sg) {
    if (ne <= 0 || k <= 0 || k > ne || ls < ne) return -1;
    float *p = (float *) malloc(sizeof(float) * ne), *key = (float *) malloc(sizeof(float) * ne);
    unsigned char *used = (unsigned char *) malloc((size_t) ne);
    if (!p || !key || !used) { free(p); free(key); free(used); return -1; }
    for (int t = 0; t < nt; ++t) {
        const float *l = logits + (size_t) t * ls;
        for (int e = 0; e < ne; ++e) { p[e] = or_sigmoid(l[e]); key[e] = p[e] + bias[e]; }
        int32_t *id = ids + (size_t) t * k;
        const float tot = topk_by_key(key, p, ne, k, used, id);
        const float inv = scale / fmaxf(tot, 6.103515625e-5f);
        for (int j = 0; j < k; ++j) wts[(size_t) t * k + j] = p[id[j]] * inv;
        if (sg) sg[t] = 1.0f;
    }
    free(p); free(key); free(used);
    return 0;
}
/* the sqrt-softplus router (src/kernels7.cu:816-865): s = sqrt(softplus(l)), the top k of s + bias[e], weights
   s / (sum of the selected s + 1e-20) scale */
int or_route_sqrtsp(const float *logits, int ls, const float *bias, int ne, int k, float scale, int nt, int32_t *ids, float *wts) {
    if (ne <= 0 || k <= 0 || k > ne || ls < ne) return -1;
    float *sc = (float *) malloc(sizeof(float) * ne), *key = (float *) malloc(sizeof(float) * ne);
    unsigned char *used = (unsigned char *) malloc((size_t) ne);
    if (!sc || !key || !used) { free(sc); free(key); free(used); return -1; }
    for (int t = 0; t < nt; ++t) {
        const float *l = logits + (size_t) t * ls;
        for (int e = 0; e < ne; ++e) { sc[e] = or_sqrt_softplus(l[e]); key[e] = sc[e] + bias[e]; }
        int32_t *id = ids + (size_t) t * k;
        const float tot = topk_by_key(key, sc, ne, k, used, id);
        for (int j = 0; j < k; ++j) wts[(size_t) t * k + j] = sc[id[j]] / (tot + 1e-20f) * scale;
    }
    free(sc); free(key); free(used);
    return 0;
}

/* ------------------------------------------------------------------ bucketing */

int or_order(const int32_t *slot, const int32_t *ids, int n_pairs, int ne, int32_t *order, int32_t *order_n, int32_t *egrp) {
    int32_t *cnt = (int32_t *) calloc(ne, sizeof(int32_t));
    if (!cnt) return -1;
    for (int p = 0; p < n_pairs; ++p) {
        const int e = ids[p];
        if (e >= 0 && e < ne && slot[e] >= 0) ++cnt[e];
    }
    int s = 0, na = 0;
    for (int e = 0; e < ne; ++e) {
        const int c = cnt[e];
        if (c) { if (egrp) { egrp[3 * na] = e; egrp[3 * na + 1] = s; egrp[3 * na + 2] = c; } ++na; }
        cnt[e] = s;
        s += c;
    }
    for (int p = 0; p < n_pairs; ++p) {
        const int e = ids[p];
        if (e >= 0 && e < ne && slot[e] >= 0) order[cnt[e]++] = p;
    }
    order_n[0] = s; order_n[1] = na;
    free(cnt);
    return 0;
}

/* ------------------------------------------------------------------ the layer job */

static float swiglu(float g, float u, float L) {        /* src/cpu_moe.cpp:891-892, :29 */
    if (L > 0.0f) { g = fminf(g, L); u = fminf(fmaxf(u, -L), L); }
    return or_silu(g) * u;
}

typedef struct { int t, e, p; float w; } pair_t;
static int pair_cmp(const void *a, const void *b) {     /* stable: ties by pair index */
    const pair_t *x = (const pair_t *) a, *y = (const pair_t *) b;
    if (x->e != y->e) return x->e < y->e ? -1 : 1;
    return x->p < y->p ? -1 : x->p > y->p;
}

/* gate/up + SwiGLU for a list of (token, expert) rows, then h quantized, then down: y_out[i][n] */
static int ffn_rows(const or_layer *L, int np, const int *tok, const int *exp_, const uint8_t *qx, size_t qx_row,
                    float *h, float *y, int n_threads) {
    const int ff = L->ff, n = L->n;
    const int vg = or_vec_dot_type(L->tg), vd = or_vec_dot_type(L->td);
    if (vg < 0 || vd < 0 || n % or_block_elems(L->tg) || ff % or_block_elems(L->td)) return -1;
    const size_t g_row = L->gate_bytes / ff, d_row = L->down_bytes / n;
    const size_t qh_row = (size_t) (ff / or_block_elems(vd)) * or_block_bytes(vd);
    uint8_t *qh = (uint8_t *) malloc((size_t) np * qh_row + 1);
    if (!qh) return -1;
    const int RC = 16, gchunks = (ff + RC - 1) / RC;
#pragma omp parallel for schedule(dynamic) num_threads(n_threads)
    for (int task = 0; task < np * gchunks; ++task) {
        const int i = task / gchunks, r0 = (task % gchunks) * RC, r1 = r0 + RC < ff ? r0 + RC : ff;
        const uint8_t *gb = L->gate + (size_t) exp_[i] * L->gate_bytes, *ub = L->up + (size_t) exp_[i] * L->gate_bytes;
        const uint8_t *xq = qx + (size_t) tok[i] * qx_row;
        for (int r = r0; r < r1; ++r) {
            const float g = row_dot(L->tg, gb + r * g_row, xq, n);
            const float u = row_dot(L->tg, ub + r * g_row, xq, n);
            h[(size_t) i * ff + r] = swiglu(g, u, L->clamp);
        }
    }
#pragma omp parallel for num_threads(n_threads)
    for (int i = 0; i < np; ++i) or_quantize_row(vd, h + (size_t) i * ff, qh + i * qh_row, ff);
    const int RD = 32, dchunks = (n + RD - 1) / RD;
#pragma omp parallel for schedule(dynamic) num_threads(n_threads)
    for (int task = 0; task < np * dchunks; ++task) {
        const int i = task / dchunks, r0 = (task % dchunks) * RD, r1 = r0 + RD < n ? r0 + RD : n;
        const uint8_t *db = L->down + (size_t) exp_[i] * L->down_bytes;
        for (int r = r0; r < r1; ++r) y[(size_t) i * n + r] = row_dot(L->td, db + r * d_row, qh + i * qh_row, ff);
    }
    free(qh);
    return 0;
}

static int quantize_tokens(int vtype, int nt, const float *x, int xs, int n, uint8_t **qx, size_t *qx_row, int n_threads) {
    *qx_row = (size_t) (n / or_block_elems(vtype)) * or_block_bytes(vtype);
    *qx = (uint8_t *) malloc((size_t) nt * *qx_row + 1);
    if (!*qx) return -1;
#pragma omp parallel for num_threads(n_threads)
    for (int t = 0; t < nt; ++t) or_quantize_row(vtype, x + (size_t) t * xs, *qx + t * *qx_row, n);
    return 0;
}

int or_expert_ffn(const or_layer *L, int e, int nt, const float *x, int xs, float *h, float *y, int n_threads) {
    iq2xs_init();
    if (n_threads <= 0) n_threads = 1;
    uint8_t *qx; size_t qx_row;
    if (or_vec_dot_type(L->tg) < 0 || L->n % or_block_elems(L->tg)) return -1;
    if (quantize_tokens(or_vec_dot_type(L->tg), nt, x, xs, L->n, &qx, &qx_row, n_threads)) return -1;
    int *tok = (int *) malloc(sizeof(int) * (nt + 1)), *ex = (int *) malloc(sizeof(int) * (nt + 1));
    float *hh = h ? h : (float *) malloc(sizeof(float) * (size_t) nt * L->ff + 1);
    int rc = -1;
    if (tok && ex && hh) {
        for (int t = 0; t < nt; ++t) { tok[t] = t; ex[t] = e; }
        rc = ffn_rows(L, nt, tok, ex, qx, qx_row, hh, y, n_threads);
    }
    if (!h) free(hh);
    free(tok); free(ex); free(qx);
    return rc;
}

/* src/cpu_moe.cpp:668-1008 (CpuMoe::run_layer, every expert owned, any nt): pairs grouped by expert
   (stable), activations quantized, gate/up dots + SwiGLU, hidden re-quantized, down dots, weighted sum
   per token in expert-id order.  With a shared expert its term sg * y_sh comes first (src/kernels4.cu:
   1182-1206 starts moe_reduce's sum from it). */
int or_moe_layer(const or_layer *L, int nt, const float *x, int xs, const int32_t *ids, const float *wts, int k,
                 float *out, int os, const or_layer *sh, const float *sg, float *h_out, float *y_out, int n_threads) {
    iq2xs_init();
    if (n_threads <= 0) n_threads = 1;
    const int n = L->n, ff = L->ff, P = nt * k;
    if (or_vec_dot_type(L->tg) < 0 || or_vec_dot_type(L->td) < 0 || n % or_block_elems(L->tg) || ff % or_block_elems(L->td)) return -1;
    pair_t *pairs = (pair_t *) malloc(sizeof(pair_t) * (P + 1));
    int np = 0;
    for (int t = 0; t < nt; ++t)
        for (int j = 0; j < k; ++j) {
            const int e = ids[t * k + j];
            if (e < 0 || e >= L->E) continue;             /* garbage routing is skipped (src/cpu_moe.cpp:679) */
            pairs[np].t = t; pairs[np].e = e; pairs[np].p = t * k + j; pairs[np].w = wts[t * k + j];
            ++np;
        }
    qsort(pairs, np, sizeof(pair_t), pair_cmp);
    uint8_t *qx; size_t qx_row;
    if (quantize_tokens(or_vec_dot_type(L->tg), nt, x, xs, n, &qx, &qx_row, n_threads)) { free(pairs); return -1; }
    int *tok = (int *) malloc(sizeof(int) * (np + 1)), *ex = (int *) malloc(sizeof(int) * (np + 1));
    float *h = (float *) malloc(sizeof(float) * ((size_t) np * ff + 1)), *y = (float *) malloc(sizeof(float) * ((size_t) np * n + 1));
    float *ysh = sh ? (float *) malloc(sizeof(float) * ((size_t) nt * sh->n + 1)) : NULL;
    int rc = -1;
    if (!tok || !ex || !h || !y || (sh && !ysh)) goto done;
    for (int i = 0; i < np; ++i) { tok[i] = pairs[i].t; ex[i] = pairs[i].e; }
    if (ffn_rows(L, np, tok, ex, qx, qx_row, h, y, n_threads)) goto done;
    if (sh && or_expert_ffn(sh, 0, nt, x, xs, NULL, ysh, n_threads)) goto done;
#pragma omp parallel for num_threads(n_threads)
    for (int t = 0; t < nt; ++t) {
        float *o = out + (size_t) t * os;
        int first = 1;
        if (sh) {
            const float g = sg ? sg[t] : 1.0f;
            for (int r = 0; r < n; ++r) o[r] = g * ysh[(size_t) t * sh->n + r];
            first = 0;
        }
        for (int i = 0; i < np; ++i) {
            if (pairs[i].t != t) continue;
            const float w = pairs[i].w, *yy = y + (size_t) i * n;
            if (first) { for (int r = 0; r < n; ++r) o[r] = w * yy[r]; first = 0; }
            else for (int r = 0; r < n; ++r) o[r] = o[r] + w * yy[r];
        }
        if (first) for (int r = 0; r < n; ++r) o[r] = 0.0f;
    }
    if (h_out) for (int i = 0; i < np; ++i) memcpy(h_out + (size_t) pairs[i].p * ff, h + (size_t) i * ff, sizeof(float) * ff);
    if (y_out) for (int i = 0; i < np; ++i) memcpy(y_out + (size_t) pairs[i].p * n, y + (size_t) i * n, sizeof(float) * n);
    rc = 0;
done:
    free(pairs); free(qx); free(tok); free(ex); free(h); free(y); free(ysh);
    return rc;
}
