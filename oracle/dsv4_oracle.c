/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_oracle.c - CPU oracle for the quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY (tests/, the smoke check, bench.py's CPU-baseline
 * leg). The product library never links this file.
 *
 * A scalar restatement of the reference's CPU kernels. The reference computes
 * with AVX2 vectors; here every vector lane is written out as its own scalar
 * operation in the same order, so each IEEE-754 single-precision rounding
 * happens on the same operands and the results are bit-identical. Build with
 * -ffp-contract=off (oracle/Makefile) so no multiply/add pair is fused that the
 * reference keeps separate; every fused multiply-add below is an explicit
 * fmaf() standing for one _mm*_fmadd_ps lane.
 *
 * Reduction trees restated (reference lane semantics written out):
 *   fp8 block lanes  s[l] = (a0[l]+a1[l]) + (a2[l]+a3[l]),
 *                    aj[l] = fma-chain over i = 0,32,64,96 of w[i+8j+l]*x[..]
 *                    (src/10_compute/dsv4_dec_fp8.h:70-85)
 *   fp4 block lanes  s[l] = (p[l]+p[8+l]) + (p[16+l]+p[24+l]), p = 2w*x
 *                    (src/10_compute/dsv4_dec_fp4.h:297-310)
 *   fold4            b = ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7))
 *                    (_mm256_hadd_ps x3 + lane add, dsv4_dec_fp8.h:105-113)
 *   hsum256          ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7))  (dsv4_dec_common.h:135-143)
 *   hsum128          (t0+t1) + (t2+t3)                      (dsv4_dec_fp8.h:115-120)
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "dsv4_oracle.h"

static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ------------------------------------------------------------ decoders --- */

/* src/10_compute/dsv4_dec_common.h:24-29 (bf16d): the halfword is the top
 * of the float, widened to double (exact). */
static inline double orc_bf16_to_f64(uint16_t h)
{
    return (double)bits_f((uint32_t)h << 16);
}

/* src/10_compute/dsv4_quant.h:72-86: 2^(b-127); 0 -> 2^-127 (subnormal),
 * 255 -> NaN. */
float orc_e8m0(uint8_t b)
{
    if (b == 0xFFu) return bits_f(0x7FC00000u);
    if (b == 0x00u) return bits_f(0x00400000u);
    return bits_f((uint32_t)b << 23);
}

/* src/10_compute/dsv4_quant.h:99-128 (OCP e4m3fn: bias 7, no inf, 0x7F/0xFF
 * NaN, max 448). The reference's closed-form fast path and its table give
 * the same value per code, so one exact decode stands for both. */
float orc_e4m3(uint8_t b)
{
    const uint32_t sign = (uint32_t)(b & 0x80u) << 24;
    const uint32_t e = (b >> 3) & 0x0Fu, m = b & 0x07u;
    if (e == 0) {
        if (m == 0) return bits_f(sign);
        /* m * 2^-9 is exact in fp32 */
        return bits_f(f_bits((float)m * 0x1p-9f) | sign);
    }
    if (e == 0x0Fu && m == 0x07u) return bits_f(sign | 0x7FC00000u);
    return bits_f(sign | ((e + 120u) << 23) | (m << 20));
}

/* src/10_compute/dsv4_quant.h:139-147 */
float orc_e2m1(uint8_t nib)
{
    static const float mag[8] = { 0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f };
    const float v = mag[nib & 7u];
    return (nib & 8u) ? -v : v;
}

/* src/10_compute/dsv4_quant.h:153-158: element i of a packed row; the even
 * element is the LOW nibble. */
float orc_fp4_at(const uint8_t *row, int64_t i)
{
    const uint8_t byte = row[i >> 1];
    return orc_e2m1((i & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0Fu));
}

/* Twice the e2m1 magnitude as the reference's integer byte LUT produces it
 * (src/10_compute/dsv4_dec_fp4.h:236-255). Code 8 gives +0, not -0. */
static inline float e2m1_x2(uint8_t nib)
{
    static const float tab[16] = { 0, 1, 2, 3, 4, 6, 8, 12,
                                   0, -1, -2, -3, -4, -6, -8, -12 };
    return tab[nib & 15u];
}

/* --------------------------------------------------------- lane trees --- */

static inline float fold8(const float s[8])
{
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

static inline float hsum256(const float s[8])
{
    return ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7]));
}

static inline float hsum128(const float t[4])
{
    return (t[0] + t[1]) + (t[2] + t[3]);
}

/* One 128-wide FP8 block as eight lane sums (dsv4_dec_fp8.h:70-85). */
static inline void fp8_lanes128(float s[8], const uint8_t *wb, const float *xb)
{
    float a[4][8];
    memset(a, 0, sizeof a);
    for (int i = 0; i < 128; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++) {
                const int c = i + 8 * j + l;
                a[j][l] = fmaf(orc_e4m3(wb[c]), xb[c], a[j][l]);
            }
    for (int l = 0; l < 8; l++)
        s[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
}

/* One 32-wide FP4 block as eight lane sums of 2w*x (dsv4_dec_fp4.h:297-310). */
static inline void fp4_lanes32(float s[8], const uint8_t *row, int64_t base,
                               const float *xb)
{
    const uint8_t *b = row + (base >> 1);
    float w[32];
    for (int e = 0; e < 32; e++)
        w[e] = e2m1_x2((e & 1) ? (uint8_t)(b[e >> 1] >> 4)
                               : (uint8_t)(b[e >> 1] & 0x0Fu));
    for (int l = 0; l < 8; l++)
        s[l] = (fmaf(w[l], xb[l], 0.0f) + fmaf(w[8 + l], xb[8 + l], 0.0f)) +
               (fmaf(w[16 + l], xb[16 + l], 0.0f) +
                fmaf(w[24 + l], xb[24 + l], 0.0f));
}

/* Generic-width FP8 block dot (src/10_compute/dsv4_matmul_fp8_int.h:275-304). */
static double fp8_block_dot_generic(const uint8_t *wb, const float *xb, int n)
{
    float a[4][8];
    memset(a, 0, sizeof a);
    int i = 0;
    for (; i + 31 < n; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++) {
                const int c = i + 8 * j + l;
                a[j][l] = fmaf(orc_e4m3(wb[c]), xb[c], a[j][l]);
            }
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    double acc = (double)hsum256(s);
    for (; i < n; i++) acc += (double)orc_e4m3(wb[i]) * (double)xb[i];
    return acc;
}

/* Generic-width FP4 block dot (src/10_compute/dsv4_matmul_fp4.c:10-39). Lane k
 * of each eight-wide load is nibble k of the 32-bit word at row + (pos >> 1)
 * (dsv4_dec_fp4.h:257-271), decoded with its sign (code 8 -> -0). */
static double fp4_block_dot_generic(const uint8_t *row, int64_t base,
                                    const float *xb, int n)
{
    float a[4][8];
    memset(a, 0, sizeof a);
    int i = 0;
    for (; i + 31 < n; i += 32)
        for (int j = 0; j < 4; j++) {
            const uint8_t *p = row + ((base + i + 8 * j) >> 1);
            const uint32_t word = (uint32_t)p[0] | ((uint32_t)p[1] << 8) |
                                  ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
            for (int l = 0; l < 8; l++) {
                const float wv = orc_e2m1((uint8_t)((word >> (4 * l)) & 0x0Fu));
                a[j][l] = fmaf(wv, xb[i + 8 * j + l], a[j][l]);
            }
        }
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    double acc = (double)hsum256(s);
    for (; i < n; i++) acc += (double)orc_fp4_at(row, base + i) * (double)xb[i];
    return acc;
}

/* ------------------------------------------------------------- FP8 n ---- */

/* The 128x128 fast path of fp8_n for one row and one token, given the row's
 * widened scales sf[] (dsv4_matmul_fp8.c:55-97; the nt > 1 form at :102-153
 * runs the same tree on the same decoded values, so one body serves both). */
static float fp8_row_fast(const uint8_t *rw, const float *x, const float *sf,
                          int nblk)
{
    float acc[4][4];
    memset(acc, 0, sizeof acc);
    float tail = 0.0f;
    int bi = 0;
    for (; bi + 3 < nblk; bi += 4) {
        const int slot = (bi >> 2) & 3;
        for (int m = 0; m < 4; m++) {
            float s[8];
            fp8_lanes128(s, rw + (size_t)(bi + m) * 128, x + (size_t)(bi + m) * 128);
            acc[slot][m] = fmaf(fold8(s), sf[bi + m], acc[slot][m]);
        }
    }
    for (; bi < nblk; bi++) {
        float s[8];
        fp8_lanes128(s, rw + (size_t)bi * 128, x + (size_t)bi * 128);
        const float p = hsum256(s) * sf[bi];
        tail = tail + p;
    }
    float t[4];
    for (int m = 0; m < 4; m++)
        t[m] = (acc[0][m] + acc[1][m]) + (acc[2][m] + acc[3][m]);
    return hsum128(t) + tail;
}

/* fp8_n with the widened scale grid supplied by `scale_at(grid, idx)`. */
static void fp8_n_common(float *y, const float *x, const uint8_t *W,
                         const void *S, int f32s, int in, int out, int blk_r,
                         int blk_c, int nt)
{
    const int nblk = in / 128;
    if (blk_c == 128 && (in & 127) == 0 && blk_r == 128 && nblk <= 256) {
        #pragma omp parallel for schedule(static) if (out > 64)
        for (int o = 0; o < out; o++) {
            const int rb = o / 128;
            float sf[256];
            for (int b = 0; b < nblk; b++)
                sf[b] = f32s ? ((const float *)S)[(size_t)rb * nblk + b]
                             : orc_e8m0(((const uint8_t *)S)[(size_t)rb * nblk + b]);
            const uint8_t *rw = W + (size_t)o * in;
            for (int t = 0; t < nt; t++)
                y[(size_t)t * out + o] =
                    fp8_row_fast(rw, x + (size_t)t * in, sf, nblk);
        }
        return;
    }
    /* generic geometry (dsv4_matmul_fp8.c:158-176) */
    const int scg = (in + blk_c - 1) / blk_c;
    #pragma omp parallel for schedule(static) if (out > 64)
    for (int o = 0; o < out; o++) {
        const uint8_t *rw = W + (size_t)o * in;
        const size_t srow = (size_t)(o / blk_r) * scg;
        for (int t = 0; t < nt; t++) {
            float total = 0.0f;
            int bi = 0;
            for (int c0 = 0; c0 < in; c0 += blk_c, bi++) {
                const int n = (in - c0 < blk_c) ? (in - c0) : blk_c;
                const float s = f32s ? ((const float *)S)[srow + bi]
                                     : orc_e8m0(((const uint8_t *)S)[srow + bi]);
                const float d = (float)fp8_block_dot_generic(
                    rw + c0, x + (size_t)t * in + c0, n);
                total = total + d * s;
            }
            y[(size_t)t * out + o] = total;
        }
    }
}

void orc_fp8_n(float *y, const float *x, const uint8_t *W, const uint8_t *S,
               int in, int out, int blk_r, int blk_c, int nt)
{
    fp8_n_common(y, x, W, S, 0, in, out, blk_r, blk_c, nt);
}

void orc_fp8f_n(float *y, const float *x, const uint8_t *W, const float *S,
                int in, int out, int blk_r, int blk_c, int nt)
{
    fp8_n_common(y, x, W, S, 1, in, out, blk_r, blk_c, nt);
}

/* ------------------------------------------------------------- FP4 n ---- */

/* src/10_compute/dsv4_matmul_fp4.c:46-162 */
void orc_fp4_n(float *y, const float *x, const uint8_t *W, const uint8_t *S,
               int in, int out, int blk_r, int blk_c, int nt)
{
    const int sc = (in + blk_c - 1) / blk_c;
    if (blk_r > 0 && blk_c == 32 && (in & 31) == 0 && sc <= 512) {
        #pragma omp parallel for schedule(static) if (out > 64)
        for (int o = 0; o < out; o++) {
            const uint8_t *row = W + (size_t)o * ((size_t)in / 2);
            const uint8_t *srow = S + (size_t)(o / blk_r) * sc;
            for (int t = 0; t < nt; t++) {
                const float *xt = x + (size_t)t * in;
                float acc[4][4];
                memset(acc, 0, sizeof acc);
                float tail = 0.0f;
                int bi = 0, c0 = 0;
                for (; c0 + 127 < in; c0 += 128, bi += 4) {
                    const int slot = (bi >> 2) & 3;
                    for (int m = 0; m < 4; m++) {
                        float s[8];
                        fp4_lanes32(s, row, c0 + 32 * m, xt + c0 + 32 * m);
                        acc[slot][m] = fmaf(fold8(s), orc_e8m0(srow[bi + m]),
                                            acc[slot][m]);
                    }
                }
                for (; c0 < in; c0 += 32, bi++) {
                    float s[8];
                    fp4_lanes32(s, row, c0, xt + c0);
                    const float p = hsum256(s) * orc_e8m0(srow[bi]);
                    tail = tail + p;
                }
                float tt[4];
                for (int m = 0; m < 4; m++)
                    tt[m] = (acc[0][m] + acc[1][m]) + (acc[2][m] + acc[3][m]);
                y[(size_t)t * out + o] = 0.5f * (hsum128(tt) + tail);
            }
        }
        return;
    }
    #pragma omp parallel for schedule(static) if (out > 64)
    for (int o = 0; o < out; o++) {
        const uint8_t *row = W + (size_t)o * ((size_t)in / 2);
        const uint8_t *srow = S + (size_t)(o / blk_r) * sc;
        for (int t = 0; t < nt; t++) {
            float total = 0.0f;
            int bi = 0;
            for (int c0 = 0; c0 < in; c0 += blk_c, bi++) {
                const int n = (in - c0 < blk_c) ? (in - c0) : blk_c;
                const float s = orc_e8m0(srow[bi]);
                const float d = (float)fp4_block_dot_generic(
                    row, (int64_t)c0, x + (size_t)t * in + c0, n);
                total = total + d * s;
            }
            y[(size_t)t * out + o] = total;
        }
    }
}

/* src/10_compute/dsv4_matmul.c:96-127 (token tiling cannot change a row's
 * arithmetic, so the bodies are called on the whole block). */
/* bf16_n (src/10_compute/dsv4_matmul.c:88-113) with its BLOCK_DOT_V tree
 * (src/10_compute/dsv4_dec_common.h:23-61): weights and activations widened
 * to double (both exact); four 4-lane double accumulators v0..v3 take
 * columns i..i+3, i+4..i+7, i+8..i+11, i+12..i+15 of every 16-column step
 * with one fma per lane; lanes are summed v0+v1 and v2+v3 first, then the
 * four lane totals as (l0+l1)+(l2+l3); the tail past the last whole step
 * takes one fma per column; the row total is rounded to float once. */
void orc_bf16_n(float *y, const float *x, const uint16_t *W, int in, int out, int nt)
{
    for (int o = 0; o < out; o++) {
        const uint16_t *row = W + (size_t)o * in;
        for (int t = 0; t < nt; t++) {
            const float *xb = x + (size_t)t * in;
            double v[4][4] = {{0}};
            int i = 0;
            for (; i + 15 < in; i += 16)
                for (int q = 0; q < 4; q++)
                    for (int l = 0; l < 4; l++) {
                        const int c = i + 4 * q + l;
                        v[q][l] = fma(orc_bf16_to_f64(row[c]), (double)xb[c], v[q][l]);
                    }
            double bb[4];
            for (int l = 0; l < 4; l++) bb[l] = (v[0][l] + v[1][l]) + (v[2][l] + v[3][l]);
            double acc = (bb[0] + bb[1]) + (bb[2] + bb[3]);
            for (; i < in; i++) acc = fma(orc_bf16_to_f64(row[i]), (double)xb[i], acc);
            y[(size_t)t * out + o] = (float)acc;
        }
    }
}

int orc_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt)
{
    if (nt <= 0) return 0;
    switch (m->wdt) {
    case DSV4_WBF16:
        orc_bf16_n(y, x, (const uint16_t *)m->w, m->cols, m->rows, nt);
        return 0;
    case DSV4_WFP8:
        orc_fp8_n(y, x, (const uint8_t *)m->w, (const uint8_t *)m->s,
                  m->cols, m->rows, m->blk_r, m->blk_c, nt);
        return 0;
    case DSV4_WFP8_F32S:
        orc_fp8f_n(y, x, (const uint8_t *)m->w, (const float *)m->s,
                   m->cols, m->rows, m->blk_r, m->blk_c, nt);
        return 0;
    case DSV4_WFP4:
        orc_fp4_n(y, x, (const uint8_t *)m->w, (const uint8_t *)m->s,
                  m->cols, m->rows, m->blk_r, m->blk_c, nt);
        return 0;
    default:
        return -1;
    }
}

/* ------------------------------------------------ scalar double oracle --- */

/* tests/unit/test_matmul.c:54-67 (BLOCK_DOT_S) */
static double block_dot_double(const double *w, const float *xb, int n)
{
    double a[16] = { 0 };
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int l = 0; l < 16; l++)
            a[l] = fma(w[i + l], (double)xb[i + l], a[l]);
    const double b0 = (a[0] + a[4]) + (a[8] + a[12]);
    const double b1 = (a[1] + a[5]) + (a[9] + a[13]);
    const double b2 = (a[2] + a[6]) + (a[10] + a[14]);
    const double b3 = (a[3] + a[7]) + (a[11] + a[15]);
    double acc = (b0 + b1) + (b2 + b3);
    for (; i < n; i++) acc = fma(w[i], (double)xb[i], acc);
    return acc;
}

/* tests/unit/test_matmul.c:93-120 */
void orc_fp8_double(float *y, const float *x, const uint8_t *W,
                    const uint8_t *S, int in, int out, int blk_r, int blk_c)
{
    const int sc = (in + blk_c - 1) / blk_c;
    #pragma omp parallel for schedule(static) if (out > 64)
    for (int o = 0; o < out; o++) {
        double wd[1024];
        const uint8_t *rw = W + (size_t)o * in;
        const uint8_t *srow = S + (size_t)(o / blk_r) * sc;
        double total = 0.0;
        int bi = 0;
        for (int c0 = 0; c0 < in; c0 += blk_c) {
            const int n = (in - c0 < blk_c) ? (in - c0) : blk_c;
            double acc = 0.0;
            /* blocks wider than the buffer are summed in buffer-sized runs
             * only if blk_c > 1024, which no geometry here uses */
            for (int i = 0; i < n && i < 1024; i++) wd[i] = (double)orc_e4m3(rw[c0 + i]);
            acc = block_dot_double(wd, x + c0, n < 1024 ? n : 1024);
            total += acc * (double)orc_e8m0(srow[bi++]);
        }
        y[o] = (float)total;
    }
}

/* tests/unit/test_matmul.c:140-166 */
void orc_fp4_double(float *y, const float *x, const uint8_t *W,
                    const uint8_t *S, int in, int out, int blk_r, int blk_c)
{
    const int sc = (in + blk_c - 1) / blk_c;
    #pragma omp parallel for schedule(static) if (out > 64)
    for (int o = 0; o < out; o++) {
        double wd[1024];
        const uint8_t *row = W + (size_t)o * ((size_t)in / 2);
        const uint8_t *srow = S + (size_t)(o / blk_r) * sc;
        double total = 0.0;
        int bi = 0;
        for (int c0 = 0; c0 < in; c0 += blk_c) {
            const int n = (in - c0 < blk_c) ? (in - c0) : blk_c;
            for (int i = 0; i < n && i < 1024; i++)
                wd[i] = (double)orc_fp4_at(row, (int64_t)c0 + i);
            const double acc = block_dot_double(wd, x + c0, n < 1024 ? n : 1024);
            total += acc * (double)orc_e8m0(srow[bi++]);
        }
        y[o] = (float)total;
    }
}

/* ----------------------------------------------------- SwiGLU, expert --- */

/* src/10_compute/dsv4_ops.c:61-79: up clamped both ways, gate from above
 * only, silu = g / (1 + expf(-g)); limit <= 0 disables the clamp. */
void orc_swiglu(float *y, const float *gate, const float *up, int n, float limit)
{
    if (limit > 0.0f) {
        for (int i = 0; i < n; i++) {
            float u = up[i];
            if (u > limit) u = limit;
            if (u < -limit) u = -limit;
            float g = gate[i];
            if (g > limit) g = limit;
            const float s = g / (1.0f + expf(-g));
            y[i] = s * u;
        }
    } else {
        for (int i = 0; i < n; i++) {
            const float g = gate[i];
            y[i] = (g / (1.0f + expf(-g))) * up[i];
        }
    }
}

/* ------------------------------------------------------------- router --- */

/* src/10_compute/dsv4_ops.c:43-46 */
static float orc_softplus(float x)
{
    return (x > 20.0f) ? x : log1pf(expf(x));
}

/* src/10_compute/dsv4_ops.c:117-157: orig = sqrt(softplus(scores)); the
 * selection runs on orig + bias (scores becomes that biased copy), or takes
 * tid2eid's row for hash-routed layers; top-k is descending with ties to the
 * lower index, a candidate replacing the best only when strictly greater;
 * the weights are the UNBIASED orig of the picks, divided by their double
 * sum and scaled by route_scale. */
void orc_route(int *idx, float *wts, float *scores, float *orig, const float *bias,
               const int64_t *tid2eid, int token_id, int n_experts, int topk, float route_scale)
{
    for (int e = 0; e < n_experts; e++) orig[e] = sqrtf(orc_softplus(scores[e]));
    for (int e = 0; e < n_experts; e++) scores[e] = bias ? orig[e] + bias[e] : orig[e];
    if (tid2eid) {
        for (int k = 0; k < topk; k++) idx[k] = (int)tid2eid[(int64_t)token_id * topk + k];
    } else {
        for (int k = 0; k < topk; k++) {
            int best = -1;
            for (int e = 0; e < n_experts; e++) {
                int taken = 0;
                for (int j = 0; j < k; j++)
                    if (idx[j] == e) { taken = 1; break; }
                if (taken) continue;
                if (best < 0 || scores[e] > scores[best]) best = e;
            }
            idx[k] = best;
        }
    }
    double sum = 0.0;
    for (int k = 0; k < topk; k++) {
        wts[k] = orig[idx[k]];
        sum += (double)wts[k];
    }
    const float inv = (sum != 0.0) ? (float)(1.0 / sum) : 0.0f;
    for (int k = 0; k < topk; k++) wts[k] = wts[k] * inv * route_scale;
}

/* src/10_compute/dsv4_ops.c:85-93 */
int orc_expert_forward(float *out, const float *x, const DSV4ExpertW *e,
                       float *gate, float *up, float *mid, int inter,
                       float limit)
{
    if (orc_mmq_n(gate, x, &e->w1, 1)) return -1;
    if (orc_mmq_n(up, x, &e->w3, 1)) return -1;
    orc_swiglu(mid, gate, up, inter, limit);
    return orc_mmq_n(out, mid, &e->w2, 1);
}

/* src/70_decode/dsv4_layer.c:57, 108-116 and
 * src/80_prefill/dsv4_prefill_union_run.c:113-120 */
void orc_moe_combine(float *out, const float *acc, const float *w, int topk,
                     const float *shared, int d)
{
    for (int i = 0; i < d; i++) out[i] = 0.0f;
    for (int k = 0; k < topk; k++) {
        const float wk = w[k];
        const float *a = acc + (size_t)k * d;
        for (int i = 0; i < d; i++) {
            const float p = wk * a[i];
            out[i] = out[i] + p;
        }
    }
    if (shared)
        for (int i = 0; i < d; i++) out[i] = out[i] + shared[i];
}

/* src/80_prefill/dsv4_prefill_union.c:30-66 (without the cache's
 * checkpoint-order sort, which reorders processing only) */
int orc_union_prepare(const int *topk_idx, int n, int topk, int ne,
                      int *ex_count, int *ex_off, int *ex_tok, int *ex_k,
                      int *ex_order)
{
    int *fill = (int *)calloc((size_t)ne, sizeof(int));
    int *seen = (int *)calloc((size_t)ne, sizeof(int));
    if (!fill || !seen) { free(fill); free(seen); return -1; }
    memset(ex_count, 0, (size_t)ne * sizeof(int));
    for (int t = 0; t < n; t++)
        for (int k = 0; k < topk; k++) ex_count[topk_idx[(size_t)t * topk + k]]++;
    ex_off[0] = 0;
    for (int e = 0; e < ne; e++) ex_off[e + 1] = ex_off[e] + ex_count[e];
    for (int t = 0; t < n; t++)
        for (int k = 0; k < topk; k++) {
            const int e = topk_idx[(size_t)t * topk + k];
            const int pos = ex_off[e] + fill[e]++;
            ex_tok[pos] = t;
            ex_k[pos] = k;
        }
    int nord = 0;
    for (int t = 0; t < n; t++)
        for (int k = 0; k < topk; k++) {
            const int e = topk_idx[(size_t)t * topk + k];
            if (!seen[e]) { seen[e] = 1; ex_order[nord++] = e; }
        }
    free(fill);
    free(seen);
    return nord;
}

/* ---------------------------------------------------------- quantizers --- */

uint8_t orc_f32_to_e4m3(float v)
{
    const uint8_t sign = (f_bits(v) >> 24) & 0x80u;
    if (isnan(v)) return (uint8_t)(sign | 0x7Fu);
    const float a = fabsf(v);
    int code;
    if (a < 0x1p-6f) {
        code = (int)rintf(a * 512.0f);             /* subnormal step 2^-9 */
    } else {
        int e2;
        (void)frexpf(a, &e2);                       /* a = f * 2^e2, f in [.5,1) */
        const int E = e2 - 1;                       /* a in [2^E, 2^(E+1)) */
        if (E > 8) return (uint8_t)(sign | 0x7Eu);
        const float frac = ldexpf(a, -E) - 1.0f;    /* exact */
        code = ((E + 7) << 3) + (int)rintf(frac * 8.0f);
    }
    if (code > 0x7E) code = 0x7E;
    return (uint8_t)(sign | (uint8_t)code);
}

uint8_t orc_f32_to_e2m1(float v)
{
    const uint8_t sign = (f_bits(v) >> 28) & 0x08u;
    if (isnan(v)) return (uint8_t)(sign | 0x7u);
    const float a = fabsf(v);
    int code;
    if (a < 1.0f) {
        code = (int)rintf(a * 2.0f);                /* subnormal step 0.5 */
    } else {
        int e2;
        (void)frexpf(a, &e2);
        const int E = e2 - 1;
        if (E > 2) return (uint8_t)(sign | 0x7u);
        const float frac = ldexpf(a, -E) - 1.0f;
        code = ((E + 1) << 1) + (int)rintf(frac * 2.0f);
    }
    if (code > 7) code = 7;
    return (uint8_t)(sign | (uint8_t)code);
}

/* Smallest e with lim * 2^e >= amax, lim = frac_lim * 2^exp_lim written as
 * (frac_lim in [0.5, 1)). Exact: no logarithm is rounded. */
static int pow2_ceil_ratio(float amax, float frac_lim, int exp_lim)
{
    int e2;
    const float f = frexpf(amax, &e2);              /* amax = f * 2^e2 */
    return (f <= frac_lim) ? e2 - exp_lim : e2 - exp_lim + 1;
}

static uint8_t e8m0_clamp(int e)
{
    int b = 127 + e;
    if (b < 0) b = 0;
    if (b > 254) b = 254;
    return (uint8_t)b;
}

void orc_quant_fp8_blk128(uint8_t *W, float *S, const float *w, int rows,
                          int cols)
{
    const int nrb = (rows + 127) / 128, ncb = (cols + 127) / 128;
    for (int rb = 0; rb < nrb; rb++)
        for (int cb = 0; cb < ncb; cb++) {
            const int r1 = (rb + 1) * 128 < rows ? (rb + 1) * 128 : rows;
            const int c1 = (cb + 1) * 128 < cols ? (cb + 1) * 128 : cols;
            float amax = 0.0f;
            for (int r = rb * 128; r < r1; r++)
                for (int c = cb * 128; c < c1; c++) {
                    const float a = fabsf(w[(size_t)r * cols + c]);
                    if (a > amax) amax = a;
                }
            const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            S[(size_t)rb * ncb + cb] = s;
            for (int r = rb * 128; r < r1; r++)
                for (int c = cb * 128; c < c1; c++)
                    W[(size_t)r * cols + c] =
                        orc_f32_to_e4m3(w[(size_t)r * cols + c] / s);
        }
}

void orc_quant_fp4_mx(uint8_t *W, uint8_t *S, const float *w, int rows,
                      int cols)
{
    const int nb = cols / 32;
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const float *src = w + (size_t)r * cols + (size_t)b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++)
                if (fabsf(src[i]) > amax) amax = fabsf(src[i]);
            /* 6 = 0.75 * 2^3 */
            const uint8_t sb = amax > 0.0f ? e8m0_clamp(pow2_ceil_ratio(amax, 0.75f, 3))
                                           : (uint8_t)127;
            const int e = (int)sb - 127;
            S[(size_t)r * nb + b] = sb;
            uint8_t *dst = W + (size_t)r * (cols / 2) + (size_t)b * 16;
            for (int i = 0; i < 16; i++) {
                const uint8_t lo = orc_f32_to_e2m1(ldexpf(src[2 * i], -e));
                const uint8_t hi = orc_f32_to_e2m1(ldexpf(src[2 * i + 1], -e));
                dst[i] = (uint8_t)(lo | (hi << 4));
            }
        }
}

void orc_quant_act_fp8_1x128(uint8_t *Q, float *S, const float *a, int n, int k)
{
    const int ng = k / 128;
    for (int t = 0; t < n; t++)
        for (int g = 0; g < ng; g++) {
            const float *src = a + (size_t)t * k + (size_t)g * 128;
            float amax = 0.0f;
            for (int i = 0; i < 128; i++)
                if (fabsf(src[i]) > amax) amax = fabsf(src[i]);
            const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            S[(size_t)t * ng + g] = s;
            for (int i = 0; i < 128; i++)
                Q[(size_t)t * k + (size_t)g * 128 + i] = orc_f32_to_e4m3(src[i] / s);
        }
}

void orc_quant_act_mxfp8(uint8_t *Q, uint8_t *S, const float *a, int n, int k)
{
    const int ng = k / 32;
    for (int t = 0; t < n; t++)
        for (int g = 0; g < ng; g++) {
            const float *src = a + (size_t)t * k + (size_t)g * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++)
                if (fabsf(src[i]) > amax) amax = fabsf(src[i]);
            /* 448 = 0.875 * 2^9 */
            const uint8_t sb = amax > 0.0f ? e8m0_clamp(pow2_ceil_ratio(amax, 0.875f, 9))
                                           : (uint8_t)127;
            const int e = (int)sb - 127;
            S[(size_t)t * ng + g] = sb;
            for (int i = 0; i < 32; i++)
                Q[(size_t)t * k + (size_t)g * 32 + i] = orc_f32_to_e4m3(ldexpf(src[i], -e));
        }
}

uint16_t orc_f32_to_bf16(float v)
{
    const uint32_t u = f_bits(v);
    if (isnan(v)) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
