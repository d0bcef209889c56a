/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_oracle.h - CPU oracle for the quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a scalar C restatement of the reference's
 * OpenMP/AVX2 CPU path, used by tests/, the smoke check and the CPU-baseline
 * leg of bench.py as the checker. No product code links or calls it.
 *
 * Every function reproduces the reference's arithmetic operation for
 * operation (same roundings, same reduction trees, -ffp-contract=off), so its
 * output is bit-identical to the compiled reference; the citations name the
 * reference code each one restates. Pinning is in tests/test_oracle*.py.
 */
#ifndef DSV4_ORACLE_H
#define DSV4_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#include "../include/dsv4_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- element decoders: src/10_compute/dsv4_quant.h:72-158 ---- */
float orc_e8m0(uint8_t b);
float orc_e4m3(uint8_t b);
float orc_e2m1(uint8_t nib);
float orc_fp4_at(const uint8_t *row, int64_t i);

/* ---- packed matmul bodies: src/10_compute/dsv4_matmul_fp8.c:49-177,
 *      dsv4_matmul_fp4.c:46-162, dsv4_matmul.c:117-127 ---- */
void orc_fp8_n(float *y, const float *x, const uint8_t *W, const uint8_t *S,
               int in, int out, int blk_r, int blk_c, int nt);
/* fp8_n with the fp32 block-scale grid of DSV4_WFP8_F32S (no reference
 * counterpart: the reference only has E8M0 grids). Same trees; only the
 * widened scale row sf[] is filled from floats. */
void orc_fp8f_n(float *y, const float *x, const uint8_t *W, const float *S,
                int in, int out, int blk_r, int blk_c, int nt);
void orc_fp4_n(float *y, const float *x, const uint8_t *W, const uint8_t *S,
               int in, int out, int blk_r, int blk_c, int nt);
/* bf16_n: src/10_compute/dsv4_matmul.c:88-113 (double widening and the
 * BLOCK_DOT_V lane tree of src/10_compute/dsv4_dec_common.h:45-61) */
void orc_bf16_n(float *y, const float *x, const uint16_t *W, int in, int out, int nt);
/* dsv4_mmq_n dispatch over DSV4_WBF16 / DSV4_WFP8 / DSV4_WFP8_F32S /
 * DSV4_WFP4. Returns -1 for other tags (the reference aborts). */
int  orc_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt);

/* ---- scalar double oracle: tests/unit/test_matmul.c:54-176 ---- */
void orc_fp8_double(float *y, const float *x, const uint8_t *W,
                    const uint8_t *S, int in, int out, int blk_r, int blk_c);
void orc_fp4_double(float *y, const float *x, const uint8_t *W,
                    const uint8_t *S, int in, int out, int blk_r, int blk_c);

/* ---- router: src/10_compute/dsv4_ops.c:43-46, 117-157 ---- */
void orc_route(int *idx, float *wts, float *scores, float *orig, const float *bias,
               const int64_t *tid2eid, int token_id, int n_experts, int topk,
               float route_scale);

/* ---- elementwise and expert: src/10_compute/dsv4_ops.c:61-93 ---- */
void orc_swiglu(float *y, const float *gate, const float *up, int n,
                float limit);
int  orc_expert_forward(float *out, const float *x, const DSV4ExpertW *e,
                        float *gate, float *up, float *mid, int inter,
                        float limit);

/* ---- decode MoE combine: src/70_decode/dsv4_layer.c:57-116 ----
 * out = sum_k (in k order) w[k]*acc[k] + shared, separately rounded mul/add.
 * `acc` is topk rows of `d`; `shared` may be NULL. */
void orc_moe_combine(float *out, const float *acc, const float *w, int topk,
                     const float *shared, int d);

/* ---- prefill permutation: src/80_prefill/dsv4_prefill_union.c:30-66 ----
 * Counting sort of the n*topk (token, k) pairs by expert id. ex_count and
 * ex_off ([ne] and [ne+1]), ex_tok / ex_k ([n*topk], stable token-major),
 * ex_order ([ne], first-use order). Returns the number of distinct experts. */
int  orc_union_prepare(const int *topk_idx, int n, int topk, int ne,
                       int *ex_count, int *ex_off, int *ex_tok, int *ex_k,
                       int *ex_order);

/* ---- quantizers: no reference counterpart (the reference ships
 *      pre-quantized weights and never quantizes activations) ---- */
/* fp32 -> e4m3fn byte, round to nearest even, saturating at +-448;
 * NaN -> 0x7F with the sign bit of the input. */
uint8_t orc_f32_to_e4m3(float v);
/* fp32 -> e2m1 nibble, round to nearest even, saturating at +-6. */
uint8_t orc_f32_to_e2m1(float v);
/* rows x cols fp32 -> e4m3 with one fp32 scale per 128x128 block,
 * scale = blockmax / 448 (1.0 for an all-zero block), q = e4m3(w / scale).
 * W is rows*cols bytes; S is [ceil(rows/128)][ceil(cols/128)] floats. */
void orc_quant_fp8_blk128(uint8_t *W, float *S, const float *w, int rows,
                          int cols);
/* rows x cols fp32 (cols % 32 == 0) -> packed e2m1 (low nibble = even
 * element) with one E8M0 scale per 1x32 block. Exponent
 * e = ceil(log2(amax / 6)) computed exactly, byte = 127 + e clamped to
 * [0, 254]; an all-zero block gets byte 127. q = e2m1(w / 2^e). */
void orc_quant_fp4_mx(uint8_t *W, uint8_t *S, const float *w, int rows,
                      int cols);
/* n rows x k (k % 128 == 0) activations -> e4m3 with one fp32 scale per
 * 1x128 group, scale = groupmax / 448 (1.0 for all zero), q = e4m3(a / s).
 * Q is n*k bytes; S is n*(k/128) floats. */
void orc_quant_act_fp8_1x128(uint8_t *Q, float *S, const float *a, int n,
                             int k);
/* n rows x k (k % 32 == 0) activations -> e4m3 with one E8M0 scale per 1x32
 * group: e = ceil(log2(groupmax / 448)) exactly, byte = 127 + e clamped to
 * [0, 254] (127 for all zero), q = e4m3(a / 2^e). */
void orc_quant_act_mxfp8(uint8_t *Q, uint8_t *S, const float *a, int n, int k);

/* fp32 -> bf16 bits, round to nearest even (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float v);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_ORACLE_H */
