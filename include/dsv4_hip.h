/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_hip.h - C ABI of the MI355X (gfx950) quantized-matmul hot path.
 *
 * Plain C: pointers, sizes and the reference's own matrix descriptor. No HIP,
 * torch or C++ types cross this boundary; a HIP stream is passed as void *.
 *
 * Two families of entry points:
 *   host-pointer   x / y / out are caller-owned host fp32 arrays, exactly as
 *                  the reference's src/10_compute entry points take them.
 *                  Weight pointers (DSV4QMat.w / .s) are host addresses inside
 *                  ranges uploaded once with dsv4_hip_register(); the library
 *                  maps them to their resident HBM copies. These return 0 when
 *                  the GPU produced the whole result and -1 when it did not
 *                  (no device, unregistered weights, unsupported geometry,
 *                  or a kernel of the call raised a status bit: bad routing
 *                  id or descriptor, a value its arithmetic cannot carry) --
 *                  the convention of the reference's GPU backend
 *                  (src/80_prefill/dsv4_prefill_vk.h:31-41): on -1 the caller
 *                  keeps its own CPU path. Nothing in this library computes on
 *                  the CPU.
 *   _dev           every pointer (activations, outputs, weights, scales,
 *                  routing) is a device address and work is enqueued on
 *                  `stream` (NULL = the default stream) without synchronising.
 *
 * Numerics: weights are decoded exactly (e4m3 / e2m1 / e8m0 as the reference
 * defines them); products accumulate in fp32. The reduction order differs from
 * the reference's AVX2 tree, so results agree within relative L2 1e-3 (typically
 * ~1e-7), not bit for bit -- the same contract the reference states for its own
 * Vulkan path (src/10_compute/dsv4_matmul.h:10-17).
 */
#ifndef DSV4_HIP_H
#define DSV4_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- types ---
 * Byte-for-byte the reference's descriptor (src/00_base/dsv4_weights.h:34-40,
 * 103-106) and format tags (src/00_base/dsv4.h:86). When the reference's
 * headers are already included (DSV4_WEIGHTS_H defined) their definitions are
 * used and only the tag this library adds is declared here. */
#ifndef DSV4_WEIGHTS_H
enum { DSV4_WF32 = 0, DSV4_WBF16 = 1, DSV4_WFP8 = 2, DSV4_WFP4 = 3 };

typedef struct {
    const void *w;          /* packed weight bytes                              */
    const void *s;          /* block scales                                     */
    int         wdt;        /* DSV4_W*                                          */
    int         rows, cols; /* logical element dims                             */
    int         blk_r, blk_c;
} DSV4QMat;

typedef struct {
    DSV4QMat w1, w3;        /* FP4 [moe_inter, hidden]                          */
    DSV4QMat w2;            /* FP4 [hidden, moe_inter]                          */
} DSV4ExpertW;
#endif

/* New tag, no counterpart in the reference: e4m3 weights whose block scales
 * are fp32 (one float per blk_r x blk_c block, row-major grid
 * [ceil(rows/blk_r)][ceil(cols/blk_c)]) instead of E8M0 bytes. The value of an
 * element is e4m3(w) * scale, one fp32 multiply. */
#define DSV4_WFP8_F32S 4

/* ---------------------------------------------------------- lifecycle ---- */

/* Select and initialise `device`. 0 ok, -1 when no usable gfx950 GPU exists
 * (the caller keeps its CPU path), mirroring dsv4_prefill_vk_init
 * (src/80_prefill/dsv4_prefill_vk.h:31-35). Idempotent. DSV4_HIP_DISABLE=1
 * in the environment makes it return -1, forcing the CPU path. */
int  dsv4_hip_init(int device);

/* Release every resident copy and staging buffer. */
void dsv4_hip_shutdown(void);

/* Human-readable reason for the last -1 on this thread ("" if none). */
const char *dsv4_hip_last_error(void);

/* Upload [host, host + bytes) to HBM once and remember the mapping. Any
 * DSV4QMat whose w / s lie inside a registered range then runs from the
 * resident copy. Replaces the host-pointer import table of the reference's
 * Vulkan backend (src/80_prefill/dsv4_prefill_vk_region.c:99-148) and the
 * NVMe slot streaming of src/60_cache: the loader (src/50_loader) calls it once
 * per arena. 0 ok, -1 on allocation failure or overlap. */
int  dsv4_hip_register(const void *host, size_t bytes);

/* Drop one registered range (by its start address). 0 ok, -1 unknown. */
int  dsv4_hip_unregister(const void *host);

/* Device address of the resident copy of host byte `p`, or NULL. */
void *dsv4_hip_device_ptr(const void *p);

/* ------------------------------------------------- packed matmul ---------
 * y[t*rows + o] = sum_c x[t*cols + c] * W[o, c] for t in 0..nt-1.
 * Replaces the body of dsv4_mmq_n (src/10_compute/dsv4_matmul.h:40,
 * dsv4_matmul.c:44-73): DSV4_WBF16 (no scales; products and sums in fp64
 * with one final rounding, as bf16_n does, src/10_compute/dsv4_matmul.c:
 * 88-113), DSV4_WFP8 (E8M0 128x128 or any blk_r x 128), DSV4_WFP8_F32S and
 * DSV4_WFP4 (E8M0 1x32) on the fast kernels for rows up to 8192 bytes (FP8
 * 8192 columns, FP4 16384); packed matrices of any other block geometry or
 * wider rows on a generic matvec (the reference's generic bodies,
 * dsv4_matmul_fp8.c:158-176, dsv4_matmul_fp4.c:143-162). BF16 rows up to
 * 8192 columns with cols % 8 == 0; other tags and geometries return -1. */
int  dsv4_hip_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt);

/* One token: dsv4_mmq (src/10_compute/dsv4_matmul.h:43). */
int  dsv4_hip_mmq(float *y, const float *x, const DSV4QMat *m);

int  dsv4_hip_mmq_n_dev(float *y, const float *x, const DSV4QMat *m, int nt,
                        void *stream);

/* One job of the batched-matmul seam: DSV4PMJob's fields
 * (src/80_prefill/dsv4_prefill_int.h:21-28), device pointers. */
typedef struct {
    const DSV4QMat *m;
    const float    *x;
    float          *y;
    int             n;
} DSV4HipJob;

/* dsv4_prefill_pm_multi (src/80_prefill/dsv4_prefill_proj.c:17-27) on the
 * device: y_j = W_j . x_j over n_j tokens for every job (n_j = 0: nothing),
 * the same bits as one dsv4_hip_mmq_n_dev per job. One-token FP8 jobs of one
 * format and width share one launch (the grouped output projection's eight
 * wo_a slices); other jobs run one after another on `stream`. Every job is
 * checked before anything is enqueued: -1 with the reason and nothing
 * enqueued when one is refused. */
int  dsv4_hip_mmq_multi_dev(const DSV4HipJob *jobs, int njobs, void *stream);

/* -------------------------------------------- expert FFN ----------------
 * out = w2 . swiglu(w1 . x, w3 . x) for one token, SwiGLU with the
 * reference's asymmetric clamp (src/10_compute/dsv4_ops.c:61-79; limit <= 0
 * disables it). Replaces dsv4_expert_forward (src/10_compute/dsv4_kernels.h:30-32)
 * minus its caller-owned gate/up/mid rows, which stay on the device. */
int  dsv4_hip_expert_forward(float *out, const float *x, const DSV4ExpertW *e,
                             int inter, float limit);

/* ----------------------------------------- decode MoE ---------------------
 * out = sum_{k in 0..topk-1, in k order} w[k] * expert(ex[k], x)  +  shared(x)
 * for one token; the shared expert (may be NULL) is added unweighted after the
 * routed sum. Replaces the compute of dsv4_layer_moe
 * (src/70_decode/dsv4_layer.c:57-116) once routing is known; all experts run
 * in one pass over their resident weights. topk <= 16. */
int  dsv4_hip_moe_decode(float *out, const float *x,
                         const DSV4ExpertW *const *ex, const float *w, int topk,
                         const DSV4ExpertW *shared, float limit);

/* Device form. `experts` is a DEVICE array of descriptors (with device w / s
 * pointers) indexed by expert id; idx / w are device arrays of topk entries.
 * `shared` is a HOST descriptor holding device pointers (or NULL). Every
 * routed expert must be DSV4_WFP4 [inter x hidden] / [hidden x inter] with
 * 1x32 blocks. With hidden in {512, 1024, 2048, 4096}, inter in {256, 512,
 * 1024, 2048} and topk <= 8 the routed experts run as one launch (gate/up
 * and down workgroups in one grid, mid handed over through a device counter);
 * the environment variable DSV4_HIP_DECODE_LAUNCHES=2 selects the two-launch
 * form, which gives the same bits; DSV4_HIP_DECODE_SPIN bounds the down
 * workgroups' wait in polls (default 2^20, about a second; 0 gives up at
 * once, status bit 3 and NaN output). The launch leaves its hand-off words
 * zero as it found them, so it may be captured in a HIP graph and replayed;
 * calls that overlap on one GPU (two streams at once) race on the library's
 * workspace. */
int  dsv4_hip_moe_decode_dev(float *out, const float *x,
                             const DSV4ExpertW *experts, int n_experts,
                             const int *idx, const float *w, int topk,
                             const DSV4ExpertW *shared, int hidden, int inter,
                             float limit, void *stream);

/* Host-routed device form, for callers whose router runs on the host as the
 * reference's does (src/70_decode/dsv4_layer.c:57-116 picks top-k on the CPU
 * and then calls the experts): `experts` is a HOST array of descriptors
 * holding device pointers, idx / w are HOST arrays of topk <= 8 entries, x /
 * out are device arrays. The topk descriptors and weights travel by value in
 * the kernel arguments, so no device-side lookup precedes the weight stream.
 * Same results as dsv4_hip_moe_decode_dev bit for bit. A routing id out of
 * range, a routed expert that is not FP4 [inter x hidden] or a geometry the
 * FP4 MFMA path does not take (hidden, inter multiples of 128, inter <= 2048)
 * returns -1 before anything is launched. */
int  dsv4_hip_moe_decode_routed_dev(float *out, const float *x,
                                    const DSV4ExpertW *experts, int n_experts,
                                    const int *idx, const float *w, int topk,
                                    const DSV4ExpertW *shared, int hidden, int inter,
                                    float limit, void *stream);

/* Allocation-free form of dsv4_hip_moe_decode_routed_dev. No counterpart in
 * the reference: it exists for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). Same arguments, kernels and results bit for bit; every
 * intermediate (mid rows, mid split tables, the shared expert's output, the
 * one-launch hand-off words) lives in a file-scope device array of 174,592
 * bytes that each GPU holds until the process ends, mapped by
 * dsv4_hip_init. It calls no allocating routine. Limits: topk <= 8, inter
 * <= 2048, hidden <= 4096 (multiples of 128), shared inter <= 2048; larger
 * calls return -1 with the reason. All calls on one GPU share the array:
 * calls that overlap on that GPU (two streams at once) race. */
int  dsv4_hip_moe_decode_routed_noalloc_dev(float *out, const float *x,
                                            const DSV4ExpertW *experts, int n_experts,
                                            const int *idx, const float *w, int topk,
                                            const DSV4ExpertW *shared, int hidden, int inter,
                                            float limit, void *stream);

/* ------------------------------------------- router on the device ---------
 * dsv4_route (src/10_compute/dsv4_ops.c:117-157, declared at
 * src/10_compute/dsv4_kernels.h:23) for n tokens, as the prefill loop calls
 * it (src/80_prefill/dsv4_prefill_moe.c:22-29): scores [n][n_experts] are
 * the gate outputs; orig[e] = sqrt(softplus(scores[e])) (softplus(x) = x
 * for x > 20); the ids are the topk largest orig + bias (bias may be NULL),
 * descending, ties to the lower id, or tid2eid[token_ids[t]] when tid2eid
 * ([n_vocab][topk] int64) is given; w[k] = orig[id_k] / sum (double) *
 * route_scale. The bias steers the selection only. All arrays are device
 * arrays: idx, w [n][topk], orig [n][n_experts] (may be NULL; the
 * reference's scores array is not overwritten). n_experts <= 1024, topk <=
 * 16. Numerics: softplus and sqrt in fp64, rounded once, so orig is the
 * correctly rounded value; glibc's log1pf is not, and the reference's orig
 * differs by one unit in the last place on about 1% of scores in [-104, 20]
 * (ids agree unless two biased scores are that close). A token id outside
 * [0, n_vocab) or a table id outside [0, n_experts) raises status bit 0 and
 * makes the token's weights NaN. */
int  dsv4_hip_route_dev(int *idx, float *w, float *orig, const float *scores, int n,
                        const float *bias, const int64_t *tid2eid, int n_vocab,
                        const int *token_ids, int n_experts, int topk, float route_scale,
                        void *stream);

/* The decode step's MoE block on the device: dsv4_layer_moe
 * (src/70_decode/dsv4_layer.c:49-116) with no host round trip. scores =
 * gate . x (dsv4_mmq at src/70_decode/dsv4_layer.c:52; `gate` is a HOST
 * descriptor with device pointers, [n_experts x hidden], any dsv4_hip_mmq
 * format, BF16 in the released checkpoints), the router as
 * dsv4_hip_route_dev with token id `token_id`, then the routed experts and
 * the shared expert as dsv4_hip_moe_decode_dev (same table, geometry and
 * limits). idx_out / w_out (device, topk entries each, may be NULL) receive
 * the routing. Every launch goes on `stream` and no host value depends on
 * the device, so the call may be captured in a HIP graph once an eager call
 * of the same n_experts has run (that call sizes the router's workspace). */
int  dsv4_hip_moe_layer_dev(float *out, const float *x, const DSV4QMat *gate,
                            const float *bias, const int64_t *tid2eid, int n_vocab,
                            int token_id, float route_scale,
                            const DSV4ExpertW *experts, int n_experts, int topk,
                            const DSV4ExpertW *shared, int hidden, int inter, float limit,
                            int *idx_out, float *w_out, void *stream);

/* ------------------------------------- grouped MoE -------------------------
 * For n tokens (batched decode or a prefill block):
 *   out[t] = sum_{k in 0..topk-1, in k order} w[t][k] * expert_{idx[t][k]}(x[t])
 *            + shared(x[t])            (shared may be NULL; added unweighted)
 * with expert(x) = w2 . swiglu(w1 . x, w3 . x) as in dsv4_expert_forward.
 * Replaces the reference's prefill union path: the permutation of (token, k)
 * pairs by expert (src/80_prefill/dsv4_prefill_union.c:30-66), the per-expert
 * bucket GEMMs (src/80_prefill/dsv4_prefill_experts.c:23-77 and its Vulkan
 * leg src/80_prefill/dsv4_prefill_vk_expert.c:45-172) and the combine
 * (src/80_prefill/dsv4_prefill_union_run.c:109-121); the CPU/GPU bucket
 * scheduler is replaced by one device pass over every bucket.
 * Routed experts: DSV4_WFP4 with 1x32 E8M0 scales, w1/w3 [inter x hidden],
 * w2 [hidden x inter]. Shared: FP4 (1x32) or FP8 (128x128, E8M0 or fp32
 * scales). hidden, inter multiples of 128; n_experts <= 1024; topk <= 16.
 * Numerics: fp16 MFMA with fp32 accumulation; weights decoded exactly (FP4
 * scale bytes 104..140, i.e. |w| in [2^-24, 2^14), else status bit 2); each
 * row of x is scaled by a power of two (undone exactly on the results) and
 * x and the SwiGLU output are rounded to fp16 on the way into the MFMA, a
 * relative error of at most 2^-11 per element; a SwiGLU output beyond the
 * fp16 range raises status bit 4. Tolerance: relative L2 1e-3 against the
 * reference's fp32 path (typically ~1e-4). */
int  dsv4_hip_moe_grouped(float *out, const float *x, int n, const int *topk_idx,
                          const float *topk_w, int topk, const DSV4ExpertW *experts,
                          int n_experts, const DSV4ExpertW *shared, float limit);

/* Device form: x [n][hidden], out [n][hidden] (16-byte aligned), idx and w
 * [n][topk], `experts` a DEVICE table of n_experts descriptors with device
 * pointers; `shared` a HOST descriptor holding device pointers (or NULL).
 * Out-of-range ids raise status bit 0 and make that token's output NaN; a
 * table entry of the wrong format raises bit 1. */
int  dsv4_hip_moe_grouped_dev(float *out, const float *x, int n,
                              const DSV4ExpertW *experts, int n_experts,
                              const int *idx, const float *w, int topk,
                              const DSV4ExpertW *shared, int hidden, int inter,
                              float limit, void *stream);

/* The same prefill MoE layer on CDNA4's block-scaled MFMA (replaces the same
 * reference code as dsv4_hip_moe_grouped_dev; its GPU leg is the Vulkan fused
 * expert, src/80_prefill/dsv4_prefill_vk_expert.c:45-172). The routed
 * experts' FP4 weights enter the MFMA as stored, with their E8M0 scales in
 * the hardware scale operand; the tokens and the SwiGLU output enter as MXFP8
 * (e4m3 with one E8M0 scale per 32 reduction indices, the rule of
 * dsv4_hip_quant_act_mxfp8_dev), fp32 accumulation. The shared expert runs on
 * the exact fp16 path of dsv4_hip_moe_grouped_dev. Numerics: against the
 * reference fed the same MXFP8-rounded tokens and mid, relative L2 1e-3
 * (typically ~1e-5); against the reference on the unrounded fp32 tokens the
 * MXFP8 rounding dominates (a few 1e-2). Same arguments and layout as
 * dsv4_hip_moe_grouped_dev; hidden must be a multiple of 256. */
int  dsv4_hip_moe_grouped_mx_dev(float *out, const float *x, int n,
                                 const DSV4ExpertW *experts, int n_experts,
                                 const int *idx, const float *w, int topk,
                                 const DSV4ExpertW *shared, int hidden, int inter,
                                 float limit, void *stream);

/* The prefill MoE layer (and batched decode) with the router on the device:
 * dsv4_prefill_moe (src/80_prefill/dsv4_prefill_moe.c:12-60) for n tokens
 * x [n][hidden] -- the gate outputs (dsv4_hip_mmq_n_dev with `gate`, a HOST
 * descriptor with device pointers, [n_experts x hidden]), dsv4_route on
 * every token (dsv4_hip_route_dev; token_ids: device int32 [n], the
 * vocabulary ids hash routing looks up), then the routed and shared experts
 * as dsv4_hip_moe_grouped_dev (mx = 0) or dsv4_hip_moe_grouped_mx_dev
 * (mx = 1) -- with no host round trip. idx_out / w_out: device [n][topk]
 * receiving the routing, or NULL. The limits of both entry points apply. */
int  dsv4_hip_moe_layer_n_dev(float *out, const float *x, int n, const DSV4QMat *gate,
                              const float *bias, const int64_t *tid2eid, int n_vocab,
                              const int *token_ids, float route_scale,
                              const DSV4ExpertW *experts, int n_experts, int topk,
                              const DSV4ExpertW *shared, int hidden, int inter, float limit, int mx,
                              int *idx_out, float *w_out, void *stream);

/* ------------------------------------------------ prefill GEMM -------------
 * C[m][n] = sum_k A[m][k] * W[n][k] for m < M on CDNA4 FP8 MFMA, replacing the
 * GPU leg of the prefill projection seam, dsv4_prefill_vk_gemm
 * (src/80_prefill/dsv4_prefill_vk.h:37-41; seam src/80_prefill/dsv4_prefill_proj.c:17-27).
 * W: DSV4_WFP8 (E8M0) or DSV4_WFP8_F32S with 128 x 128 blocks, rows and cols
 * multiples of 128, device pointers. A [M][W->cols] fp32 (a_bf16 = 0) or bf16
 * (a_bf16 = 1), device, quantized on the fly to e4m3 with one fp32 scale per
 * 1 x 128 group (groupmax / 448) into a library-owned workspace. C [M][W->rows]
 * fp32 (out_bf16 = 0) or bf16 (out_bf16 = 1, round to nearest even). All
 * pointers 16-byte aligned. Enqueued on `stream`. 0 enqueued, -1 otherwise. */
int  dsv4_hip_gemm_fp8_dev(void *C, int out_bf16, const void *A, int a_bf16,
                           int M, const DSV4QMat *W, void *stream);

/* The same GEMM on activations the caller already quantized:
 * Aq [M][W->cols] e4m3, Sa [W->cols / 128][M] fp32, block-major (as produced
 * by dsv4_hip_quant_act_fp8_1x128_dev). No workspace. */
int  dsv4_hip_gemm_fp8q_dev(void *C, int out_bf16, const uint8_t *Aq,
                            const float *Sa, int M, const DSV4QMat *W,
                            void *stream);

/* The prefill GEMM for the checkpoint's own FP8 format: W DSV4_WFP8 with
 * E8M0 128 x 128 block scales (src/00_base/dsv4_weights.h:34-40; the scales
 * the reference's packer writes, tools/pack_trunk.py:219-227), replacing the
 * same seam as dsv4_hip_gemm_fp8_dev (src/80_prefill/dsv4_prefill_vk.h:37-41,
 * src/80_prefill/dsv4_prefill_proj.c:17-27). A [M][W->cols] fp32 (a_bf16 = 0)
 * or bf16 (a_bf16 = 1) is quantized on the fly to MXFP8: e4m3 with one E8M0
 * scale per token and 32 columns (the power of two that keeps the group's
 * largest magnitude at or below 448). Both scales ride in the MFMA's
 * hardware scale operands, so the MFMA accumulates across K. C as in
 * dsv4_hip_gemm_fp8_dev. Numerics: against the reference fed the same
 * MXFP8-rounded activations, relative L2 1e-3 (typically ~1e-5). 0 enqueued,
 * -1 otherwise (also for fp32-scaled weights). */
int  dsv4_hip_gemm_mxfp8_dev(void *C, int out_bf16, const void *A, int a_bf16,
                             int M, const DSV4QMat *W, void *stream);

/* The same on activations the caller already quantized: Aq [M][W->cols]
 * e4m3, As [M][W->cols / 32] E8M0 bytes (as dsv4_hip_quant_act_mxfp8_dev
 * writes them). No workspace. */
int  dsv4_hip_gemm_mxfp8q_dev(void *C, int out_bf16, const uint8_t *Aq,
                              const uint8_t *As, int M, const DSV4QMat *W,
                              void *stream);

/* ------------------------------------- checkpoint experts (loader hook) --
 * The loader's upload-once path for the routed experts, which the reference
 * streams from NVMe through its slot cache (src/60_cache/dsv4_cache_load.c)
 * and which here stay resident in HBM. Reads index_dir/experts.idx (magic
 * "DSV4EXP1", int32 n_layers and n_experts, then n_layers x n_experts x 6
 * records {int32 shard, int32 pad, int64 offset, int64 bytes} in the order
 * w1, w1 scales, w2, w2 scales, w3, w3 scales: src/40_io/dsv4_st.h:36-55,
 * src/40_io/dsv4_st.c:60-84, tools/pack_trunk.py:333-346); shard i is the
 * i-th *.safetensors file of model_dir in strcmp order
 * (src/40_io/dsv4_st.c:88-135). Layer `layer`'s experts are uploaded into one
 * device arena, one slot per expert laid out as the reference's cache slot
 * (scales s1 s2 s3, then weights w1 w2 w3: src/60_cache/dsv4_cache_geom.c:
 * 14-50), and table[0..n_experts) receives their descriptors (FP4, 1 x 32
 * E8M0 scales, device pointers) for the _dev MoE entry points. Returns the
 * arena, or NULL with dsv4_hip_last_error() (bad index, a tensor of the wrong
 * size, a short read, no device memory); the index is checked before any
 * device memory is touched. */
void *dsv4_hip_load_experts(const char *model_dir, const char *index_dir, int layer,
                            int hidden, int inter, DSV4ExpertW *table, int max_experts,
                            int *n_experts);

/* Release an arena of dsv4_hip_load_experts (synchronises the device). */
int  dsv4_hip_free_experts(void *arena);

/* Read and clear the device status word that the _dev kernels raise when a
 * routing id is out of range (bit 0) or an expert descriptor in the device
 * table does not match the expected format and geometry (bit 1); the affected
 * outputs are NaN. Bit 2: the grouped MoE met an FP4 scale byte outside
 * 104..140, whose blocks it cannot decode exactly. Bit 3: a one-launch decode
 * MoE gave up waiting for its gate/up half (about a second; only possible
 * when other work keeps its workgroups from running), its output is NaN.
 * Bit 4: an fp16-MFMA path met a SwiGLU output beyond the fp16 range.
 * Host-pointer calls keep a word of their own and turn any bit into -1.
 * Synchronises the device. 0 ok, -1 no device. */
int  dsv4_hip_status(unsigned *bits);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_HIP_H */
