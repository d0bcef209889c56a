/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_hip_aux.h - device-pointer helpers around the hot path: the
 * dequantization check, the quantizers that produce the packed formats, and
 * the seeded synthetic-tensor generator. None has a counterpart in the
 * reference, which ships pre-quantized weights and never quantizes
 * activations; they exist so the formats can be produced and checked on the
 * device. All pointers are device addresses; work is enqueued on `stream`.
 * Each returns 0 when enqueued, -1 on an invalid argument or no device. */
#ifndef DSV4_HIP_AUX_H
#define DSV4_HIP_AUX_H

#include "dsv4_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* out[r * cols + c] = decode(W[r, c]) * its block scale (one fp32 multiply),
 * through the same decoders the matmul kernels use. m->w / m->s are device
 * pointers; geometry as accepted by dsv4_hip_mmq_n. */
int dsv4_hip_dequant_dev(float *out, const DSV4QMat *m, void *stream);

/* rows x cols fp32 -> e4m3 bytes W[rows*cols] + fp32 scale per 128x128 block
 * S[ceil(rows/128)][ceil(cols/128)], scale = blockmax/448 (1 if all zero). */
int dsv4_hip_quant_fp8_blk128_dev(uint8_t *W, float *S, const float *w,
                                  int rows, int cols, void *stream);

/* rows x cols fp32 (cols % 32 == 0) -> packed e2m1 W[rows*cols/2] (low nibble
 * = even element) + E8M0 per 1x32 S[rows*cols/32]: 2^e least with
 * 6 * 2^e >= blockmax, byte 127 + e clamped to [0, 254] (127 if all zero). */
int dsv4_hip_quant_fp4_mx_dev(uint8_t *W, uint8_t *S, const float *w,
                              int rows, int cols, void *stream);

/* n x k activations (k % 128 == 0) -> e4m3 Q[n*k] + fp32 scale per 1x128
 * group = groupmax/448 (1 if all zero), stored block-major: the scale of row
 * r, 128-column block b is S[b * n + r] (the layout dsv4_hip_gemm_fp8q_dev
 * reads: one block's scales of consecutive rows are contiguous). Q 8-byte,
 * a 16-byte and S 4-byte aligned. */
int dsv4_hip_quant_act_fp8_1x128_dev(uint8_t *Q, float *S, const float *a,
                                     int n, int k, void *stream);

/* n x k activations (k % 32 == 0) -> e4m3 Q[n*k] + E8M0 per 1x32 S[n][k/32]:
 * 2^e least with 448 * 2^e >= groupmax (127 if all zero). */
int dsv4_hip_quant_act_mxfp8_dev(uint8_t *Q, uint8_t *S, const float *a,
                                 int n, int k, void *stream);

/* The grouped MoE's permutation on its own (the first step of
 * dsv4_hip_moe_grouped_dev): the counting sort of the n * topk routing ids
 * idx[n][topk] by expert, as src/80_prefill/dsv4_prefill_union.c:30-51
 * builds ex_off / ex_tok / ex_k. ex_off [n_experts + 1] is the first row of
 * each expert's bucket (ex_off[e + 1] - ex_off[e] = its count); ex_tok and
 * ex_k [n * topk] the token and k of each row, rows of a bucket in
 * token-major, k-minor order; pos [n * topk] the row of each (token, k)
 * pair. An id outside [0, n_experts) raises status bit 0 and gets pos -1.
 * The reference's ex_order (the order its host processes buckets in) has no
 * counterpart: the device runs every bucket at once. */
int dsv4_hip_moe_route_dev(int *ex_off, int *ex_tok, int *ex_k, int *pos, const int *idx,
                           int n, int topk, int n_experts, void *stream);

/* The first half of dsv4_hip_moe_grouped_mx_dev on its own: the permutation,
 * the tokens' MXFP8 quantization and the routed gate/up GEMMs with SwiGLU,
 * writing the MXFP8 mid that its down GEMMs read: mid [n * topk][inter] e4m3
 * and mid_s [n * topk][inter / 32] E8M0, row r belonging to token row_tok[r]
 * and routing slot row_k[r] (rows bucketed by expert, as
 * dsv4_hip_moe_route_dev orders them). Device arrays; mid and mid_s 4-byte
 * aligned, x 16-byte aligned. */
int dsv4_hip_moe_grouped_mx_mid_dev(uint8_t *mid, uint8_t *mid_s, int *row_tok, int *row_k,
                                    const float *x, int n, const DSV4ExpertW *experts,
                                    int n_experts, const int *idx, int topk, int hidden, int inter,
                                    float limit, void *stream);

/* The FP8 shared expert's mid as dsv4_hip_moe_grouped_mx_dev computes it on
 * its side stream: x [n][hidden] quantized 1x128 to e4m3, the w1 / w3 FP8
 * GEMMs, SwiGLU (clamp `limit`) and mid's own 1x128 quantization: mid
 * [n][inter] e4m3 and mid_s [inter / 128][n] fp32 scales (block-major).
 * Device arrays; x 16-byte and mid 8-byte aligned. */
int dsv4_hip_shared_fp8q_mid_dev(uint8_t *mid, float *mid_s, const float *x, int n,
                                 const DSV4ExpertW *shared, int hidden, float limit, void *stream);

/* out[i] = sigma * N(0,1) sample i of stream `seed` (counter-based splitmix64
 * hash -> Box-Muller in double -> fp32), rounded to bf16 when round_bf16. */
int dsv4_hip_synth_normal_dev(float *out, size_t n, uint64_t seed, float sigma,
                              int round_bf16, void *stream);

/* Number of device allocations (hipMalloc calls) the library has made since
 * it was loaded: workspaces, status words, registered copies, expert arenas.
 * A diagnostic for callers that must not allocate: it stays unchanged
 * across calls of dsv4_hip_moe_decode_routed_noalloc_dev. */
unsigned long long dsv4_hip_alloc_count(void);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_HIP_AUX_H */
