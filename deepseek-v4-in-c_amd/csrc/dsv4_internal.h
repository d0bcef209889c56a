/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_internal.h - kernel launch interfaces shared between the .hip files of
 * the library. Not installed; the public boundary is include/dsv4_hip.h. */
#ifndef DSV4_INTERNAL_H
#define DSV4_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/dsv4_hip.h"
#include "dsv4_dev.h"

namespace dsv4 {

/* Kernel-side weight formats. */
enum {
    FMT_FP8_E8M0 = 0, /* DSV4_WFP8, blk_c == 128      */
    FMT_FP8_F32S = 1, /* DSV4_WFP8_F32S, blk_c == 128 */
    FMT_FP4_E8M0 = 2, /* DSV4_WFP4, blk_c == 32       */
    FMT_BF16 = 3,     /* DSV4_WBF16, no scales, cols % 8 == 0 */
    /* any other block geometry (and rows wider than the fast kernels take),
     * on the generic VALU matvec only */
    FMT_GEN_FP8 = 4,  /* DSV4_WFP8                    */
    FMT_GEN_FP8F = 5, /* DSV4_WFP8_F32S               */
    FMT_GEN_FP4 = 6,  /* DSV4_WFP4, cols even         */
};

/* Status bits a kernel may raise in the device status word. */
enum {
    ST_BAD_EXPERT_ID = 1u << 0,   /* routing index outside [0, n_experts)   */
    ST_BAD_DESCRIPTOR = 1u << 1,  /* expert descriptor of the wrong format  */
    ST_SCALE_RANGE = 1u << 2,     /* FP4 E8M0 scale byte outside 104..140:
                                     the grouped path's fp16 decode is not
                                     exact for that block                   */
    ST_SYNC_TIMEOUT = 1u << 3,    /* a one-launch decode MoE waited past its
                                     spin limit for a slot's mid             */
    ST_F16_RANGE = 1u << 4,       /* an fp16-MFMA path met a SwiGLU output
                                     beyond the fp16 range (|v| >= 65520)    */
};

/* Map a descriptor to the kernel format, or -1 when the GPU path does not
 * support its geometry. */
static inline int qmat_fmt(const DSV4QMat *m)
{
    if (!m || m->rows <= 0 || m->cols <= 0) return -1;
    if (m->wdt == DSV4_WBF16) return (m->cols % 8) == 0 ? FMT_BF16 : -1;
    if (m->blk_r <= 0) return -1;
    if (m->wdt == DSV4_WFP8 && m->blk_c == 128 && (m->cols % 128) == 0)
        return FMT_FP8_E8M0;
    if (m->wdt == DSV4_WFP8_F32S && m->blk_c == 128 && (m->cols % 128) == 0)
        return FMT_FP8_F32S;
    if (m->wdt == DSV4_WFP4 && m->blk_c == 32 && (m->cols % 32) == 0)
        return FMT_FP4_E8M0;
    return -1;
}

/* The generic-geometry format of a packed matrix, or -1 */
static inline int qmat_fmt_generic(const DSV4QMat *m)
{
    if (!m || m->rows <= 0 || m->cols <= 0 || m->blk_r <= 0 || m->blk_c <= 0) return -1;
    if (m->wdt == DSV4_WFP8) return FMT_GEN_FP8;
    if (m->wdt == DSV4_WFP8_F32S) return FMT_GEN_FP8F;
    if (m->wdt == DSV4_WFP4) return (m->cols % 2) == 0 ? FMT_GEN_FP4 : -1;
    return -1;
}

static inline int qmat_row_bytes(const DSV4QMat *m)
{
    return m->wdt == DSV4_WFP4 ? m->cols / 2 : m->wdt == DSV4_WBF16 ? 2 * m->cols : m->cols;
}

/* scale-grid columns (entries per scale row) */
static inline int qmat_sc_cols(const DSV4QMat *m)
{
    return (m->cols + m->blk_c - 1) / m->blk_c;
}

static inline size_t qmat_w_bytes(const DSV4QMat *m)
{
    return (size_t)m->rows * (size_t)qmat_row_bytes(m);
}

static inline size_t qmat_s_bytes(const DSV4QMat *m)
{
    if (m->wdt == DSV4_WBF16) return 0;
    const size_t n = (size_t)((m->rows + m->blk_r - 1) / m->blk_r) *
                     (size_t)qmat_sc_cols(m);
    return m->wdt == DSV4_WFP8_F32S ? n * 4u : n;
}

/* ------------------------------------------------------------- GEMV --- */
struct GemvArgs {
    const uint8_t *W;   /* device, 16-byte aligned */
    const void *S;      /* device scales            */
    const float *x;     /* device, 16-byte aligned  */
    float *y;
    int rows, row_bytes, sc_cols, blk_r;
    int nt;
    int x_ld, y_ld;     /* floats between tokens    */
};
hipError_t gemv_launch(int fmt, const GemvArgs &a, hipStream_t st);

/* y[t * rows + o] for t < nt, any block geometry (FMT_GEN_*): W rows of cols
 * e4m3 bytes or cols / 2 e2m1 bytes, scales [ceil(rows / blk_r)][ceil(cols /
 * blk_c)] (E8M0 bytes, or fp32 for FMT_GEN_FP8F), x [nt][cols]. */
struct GemvGenArgs {
    const uint8_t *W;
    const void *S;
    const float *x;
    float *y;
    int rows, cols, blk_r, blk_c, nt;
};
hipError_t gemv_generic_launch(int fmt, const GemvGenArgs &a, hipStream_t st);

/* y[t*y_ld + o] = (float) sum_c (double) bf16(W[o][c]) * (double) x[t*x_ld + c]
 * for t < nt: BF16 weights (row pitch 2 * cols bytes, 16-byte aligned, cols %
 * 8 == 0), fp32 x and y, products and sums in fp64. */
struct GemvBf16Args {
    const uint16_t *W;
    const float *x;
    float *y;
    int rows, cols;
    int nt, x_ld, y_ld;
};
hipError_t gemv_bf16_launch(const GemvBf16Args &a, hipStream_t st);

/* ---------------------------------------------------- decode MoE ------ */
/* Gate/up + SwiGLU for `nslots` experts: slot s uses table[idx[s]] (or
 * `direct` when use_direct), writing mid[s * mid_ld + j], j < inter. */
struct GateUpArgs {
    const DSV4ExpertW *table; /* device table (ignored when use_direct) */
    const int *idx;           /* device, nslots entries                 */
    int n_experts;
    DSV4ExpertW direct;       /* device pointers                        */
    int use_direct;
    int nslots;
    const float *x;           /* [hidden]                               */
    float *mid;               /* [nslots][mid_ld]                       */
    int mid_ld;
    int inter, hidden;
    float limit;
    unsigned *status;
};
hipError_t gateup_launch(int fmt, const GateUpArgs &a, hipStream_t st);

/* out[i] = sum_k (k order) w[k] * (table[idx[k]].w2 . mid[k])[i] + shared[i]
 * for FP4 routed experts, topk <= 16. */
struct DownArgs {
    const DSV4ExpertW *table;
    const int *idx;
    const float *w;           /* device, topk routing weights           */
    int n_experts;
    int topk;
    const float *mid;         /* [topk][mid_ld], mid_ld % 4 == 0         */
    int mid_ld;
    const float *shared;      /* device [hidden] or NULL                */
    float *out;               /* [hidden]                               */
    int inter, hidden;
    unsigned *status;
};
int down_groups(int hidden);
hipError_t down_launch(const DownArgs &a, hipStream_t st);

/* ------------------------------------------- decode on the MFMA --- */
/* y = W . x for nt tokens (x rows x_ld floats apart, y rows y_ld apart) on
 * the block-scaled MFMA; cols % 128 == 0, FP8 blk_r % 16 == 0, x 16-byte
 * aligned. ncw and tpg are set by the launcher. */
struct GemvMxArgs {
    const uint8_t *W;
    const void *S;
    const float *x;
    float *y;
    int rows, cols, row_bytes, sc_cols, blk_r;
    int nt, x_ld, y_ld;
    int ncw, tpg;
    const uint8_t *tab;       /* x already split (split_x_tab_launch), or NULL */
    int gpw;                  /* token groups per workgroup, with tab */
};
/* chunks of 128 columns per wave, 0 when the MFMA path does not take `cols` */
int gemv_mx_ncw(int fmt, int cols);
/* the same for the gate/up kernels (FP8 hidden at most 4096) */
int gateup_mx_ncw(int fmt, int cols);
hipError_t gemv_mx_launch(int fmt, GemvMxArgs a, hipStream_t st);
/* nt tokens of x (x_ld floats apart, cols a multiple of 128, nt * cols / 8
 * below 2^31) split into the small-batch matvec's e4m3 part tables, token t's
 * chunk c at tab + (t * cols / 128 + c) * gemv_tab_chunk_bytes() */
size_t gemv_tab_chunk_bytes();
hipError_t split_x_tab_launch(uint8_t *tab, const float *x, int x_ld, int nt, int cols, hipStream_t st);
/* whether a one-token FP8 matvec takes the chunk-pair kernel, which can run
 * up to PX8_MAX_JOBS such matvecs of the same format and width in one launch */
constexpr int PX8_MAX_JOBS = 16;
bool gemv_px8_ok(int fmt, const GemvMxArgs &a);
/* the launch shape class of such a matvec: one launch takes one class */
int gemv_px8_class(const GemvMxArgs &a);
hipError_t gemv_px8_multi_launch(int fmt, const GemvMxArgs *jobs, int nj, hipStream_t st);

/* Routed experts whose descriptors travel by value in the kernel arguments
 * (routing known on the host): at most this many slots. */
constexpr int MX_ROUTED_MAX = 8;

/* Gate/up + SwiGLU for `nslots` experts (like GateUpArgs); also writes the
 * split table of each slot's mid (msplit + slot * msplit_ld) when msplit is
 * set. inter % 128 == 0, hidden % 128 == 0. Slot s uses routed[s] when
 * by_value, else direct when use_direct, else table[idx[s]]. */
struct GateUpMxArgs {
    const DSV4ExpertW *table;
    const int *idx;
    int n_experts;
    DSV4ExpertW direct;
    int use_direct;
    int nslots;
    const float *x;
    float *mid;
    int mid_ld;
    uint8_t *msplit;
    size_t msplit_ld;
    int inter, hidden;
    float limit;
    unsigned *status;
    int ncw;
    int by_value;
    DSV4ExpertW routed[MX_ROUTED_MAX];
};
hipError_t gateup_mx_launch(int fmt, GateUpMxArgs a, hipStream_t st);

/* Routed FP4 down projections from the split tables of mid, with the k-order
 * combine (+ shared); topk <= 8. Slot k uses w2v[k] and weight wv[k] when
 * by_value, else table[idx[k]].w2 and w[k]. */
struct DownMxArgs {
    const DSV4ExpertW *table;
    const int *idx;
    const float *w;
    int n_experts;
    int topk;
    const uint8_t *msplit;
    size_t msplit_ld;
    const float *shared;
    float *out;
    int inter, hidden;
    unsigned *status;
    int ncw;
    int by_value;
    DSV4QMat w2v[MX_ROUTED_MAX];
    float wv[MX_ROUTED_MAX];
};
hipError_t down_mx_launch(DownMxArgs a, hipStream_t st);

/* Gate/up and down of the routed FP4 experts in one launch: workgroups
 * [0, gu_blocks) run the gate/up items; each item adds one to *count once its
 * block of mid's split table is out, and the item whose add returns
 * items - 1 writes 1 to *done. The hidden / 16 down workgroups after them
 * load their down weights at once and wait (spin_max polls at most; 0: give
 * up without polling) until *done is 1. Every workgroup, gate/up and down,
 * leaves as its last access to the words: it adds one to the leave counter
 * of its group (workgroup id % ONE_LEAVE_GROUPS, at leave + group *
 * ONE_PUB_LINE_WORDS), the last leaver of a group adds one to the top
 * counter (after the group counters), and the last top add sets every word
 * back to 0, so each launch finds them zero (a HIP graph can replay the
 * launch). Every word is on its own 128-byte line, zero before the first
 * launch: count (ONE_LEAVE_GROUPS group counters and a top counter when every
 * workgroup publishes, as in the balanced form; the first word alone
 * otherwise), done, the leave group counters, the leave top counter. */
struct OnePub {
    unsigned *count, *done, *leave;
    unsigned items, total;
};
constexpr int ONE_PUB_LINE_WORDS = 32;    /* one 128-byte line per word */
constexpr int ONE_LEAVE_GROUPS = 8;
constexpr int ONE_COUNT_LINES = ONE_LEAVE_GROUPS + 1;
struct MoeOneArgs {
    GateUpMxArgs gu;
    DownMxArgs dn;
    OnePub pub;
    int gu_blocks;
    unsigned spin_max;
    /* the balanced form's hand-off of mid: mid_copies replicas of every routed
     * slot's mid table (topk x mx_split_bytes(inter) bytes each), copy_ld bytes
     * apart from midc; every workgroup writes its rows to all of them and reads
     * replica blockIdx % mid_copies, so no few memory channels serve every
     * CU's reads */
    uint8_t *midc;
    int mid_copies;
    size_t copy_ld;
};
/* most replicas of mid the balanced form writes */
constexpr int BAL_MAX_COPIES = 32;
/* whether one launch takes this geometry */
bool moe_one_ok(int hidden, int inter, int topk);
/* balanced: the balanced form (k_moe_bal) when it takes the geometry and the
 * device holds its whole grid at once, else the grid-ordered form (k_moe_one) */
hipError_t moe_one_launch(MoeOneArgs a, hipStream_t st, bool balanced);
/* the publication words of the one-launch forms: the count lines, done, the
 * group leave counters and the top counter, a 128-byte line each */
constexpr size_t ONE_PUB_BYTES = (size_t)(ONE_COUNT_LINES + 1 + ONE_LEAVE_GROUPS + 1) * ONE_PUB_LINE_WORDS * 4;
/* bytes of one slot's split table for a K of `inter` */
size_t mx_split_bytes(int inter);

/* ---------------------------------------------------- prefill GEMM --- */
/* C[m][n] = sum_k A[m][k] W[n][k]: Aq e4m3 [M][K] with one fp32 scale per
 * token and 128-wide K block at Sa[m * sa_tok + kb * sa_kb]; W e4m3 [N][K]
 * with Sw [N/128][K/128] fp32 (w_f32s) or E8M0 bytes; C bf16 or fp32
 * [M][ldc]. K % 128 == 0, N % 128 == 0. */
struct GemmArgs {
    const uint8_t *Aq;
    const float *Sa;
    const uint8_t *W;
    const void *Sw;
    void *C;
    int M, N, K, ldc;
    int sa_tok, sa_kb;
};
hipError_t gemm_fp8_launch(const GemmArgs &a, bool w_f32s, bool out_bf16, hipStream_t st);
/* The same with E8M0 weight bytes and MXFP8 token scales: Sa holds a dword
 * of four E8M0 bytes per token and 128-wide K block, token-major [M][K / 32]
 * bytes (sa_tok = K / 128, sa_kb = 1) or block-major (sa_tok = 1, sa_kb = M:
 * a K block's tokens in one contiguous run, which the workgroup's scale loads
 * read as whole lines). */
hipError_t gemm_mx_launch(const GemmArgs &a, bool out_bf16, hipStream_t st);

/* The seam's dense FP8 form: C fp32 [M][N] = 2^-ex[m] * sum over 128-K blocks
 * of the block scale (fp32 when w_f32s, else E8M0 bytes, [N/128][K/128])
 * times the fp16 MFMA partial of X fp16 [M][K] (rows scaled by 2^ex[m]) and
 * W e4m3 [N][K] decoded exactly. K % 128 == 0, N % 128 == 0. */
struct SeamGemmArgs {
    const uint16_t *X;
    const int *ex;
    const uint8_t *W;
    const void *Sw;
    float *C;
    int M, N, K;
};
bool gemm_seam_ok(int M, int N, int K);
hipError_t gemm_seam_launch(const SeamGemmArgs &s, bool w_f32s, hipStream_t st);

/* ---------------------------------------------- dequant / quantizers --- */
hipError_t dequant_launch(int fmt, const DSV4QMat &m, float *out, hipStream_t st);
hipError_t quant_fp4_mx_launch(uint8_t *W, uint8_t *S, const float *w, int rows,
                               int cols, hipStream_t st);
hipError_t quant_fp8_blk128_launch(uint8_t *W, float *S, const float *w,
                                   int rows, int cols, hipStream_t st);
/* a is fp32, or bf16 bits when bf16_in; S is [n][k/128], or [k/128][n] when
 * s_blk_major */
hipError_t quant_act_fp8_1x128_launch(uint8_t *Q, float *S, const void *a,
                                      int n, int k, bool bf16_in, bool s_blk_major,
                                      hipStream_t st);
/* Q, S (block-major [k/128][n]) = the 1x128 e4m3 quantization of
 * SwiGLU(gate, up) over [n][k] fp32 rows (k % 128 == 0). */
hipError_t swiglu_quant_fp8_launch(uint8_t *Q, float *S, const float *gate, const float *up, int n, int k,
                                   float limit, hipStream_t st);
/* S token-major [n][k / 32], or block-major [k / 128][n] dwords (the four
 * scale bytes of a token's 128-wide K block, k % 128 == 0) when s_blk_major */
hipError_t quant_act_mxfp8_launch(uint8_t *Q, uint8_t *S, const void *a,
                                  int n, int k, hipStream_t st, bool bf16_in = false,
                                  bool s_blk_major = false);
hipError_t synth_normal_launch(float *out, size_t n, uint64_t seed, float sigma,
                               int round_bf16, hipStream_t st);

/* ------------------------------------------------------ grouped MoE --- */

/* One token tile of the grouped GEMMs: its bucket (expert), first bucket
 * row and rows, so a workgroup finds its work in one load. */
struct TileRec {
    int grp, r0, ntok, pad;
};

/* counting sort of the npairs = n * topk routing ids by expert; rows inside
 * a bucket keep pair order (token-major, k-minor) */
struct RouteArgs {
    const int *idx;           /* device [npairs]                          */
    int npairs, topk, n_experts;
    int tile_rows;            /* rows per tile of the grouped GEMM        */
    int *grp_off;             /* [n_experts + 1] first row of each bucket */
    int *tile_pre;            /* [n_experts + 1] prefix of tiles          */
    TileRec *tile_rec;        /* [tiles] bucket, first row, rows per tile */
    int *pos;                 /* [npairs] row of each pair (-1: bad id)   */
    int *row_tok;             /* [npairs] token of each row               */
    int *row_k;               /* [npairs] k of each row, or NULL          */
    int *chist;               /* [chunks of 1024 pairs][n_experts] counts, or
                                 NULL: every placing workgroup counts every pair */
    unsigned *status;
};
/* from this many chunks of 1024 pairs on (and with chist set), a counting
 * launch per chunk precedes the placing launch */
constexpr int ROUTE_PRECOUNT_CHUNKS = 4;
inline size_t route_chist_bytes(long npairs, int n_experts)
{
    return (size_t)((npairs + 1023) / 1024) * (size_t)n_experts * 4;
}
hipError_t moe_route_launch(const RouteArgs &a, hipStream_t st);

/* dsv4_route for n tokens, one wavefront each: scores [n][scores_ld] fp32
 * (the gate matvec's output) -> idx, w [n][topk], orig [n][n_experts] (may
 * be NULL). bias [n_experts] may be NULL. With tid2eid ([n_vocab][topk]
 * int64) the ids are tid2eid[token], token = token_ids[t] (device) or
 * token_id when token_ids is NULL (n == 1).
 * With gate_w set (n == 1) the launch also computes the scores: gate_w is
 * the BF16 gate [n_experts][cols] (cols % 8 == 0, cols <= 4096, 16-byte
 * aligned rows), x the token (fp32, 16-byte aligned); ws_orig / ws_biased
 * hold n_experts floats each and counter GATE_ROUTE_GROUPS + 1 words, each
 * on its own 128-byte line (GATE_ROUTE_COUNTER_BYTES), zero before the
 * launch and zero after it; scores_out (may be NULL) receives the scores. */
constexpr int GATE_ROUTE_GROUPS = 8;
constexpr int GATE_ROUTE_COUNTER_BYTES = (GATE_ROUTE_GROUPS + 1) * 128;
constexpr int GATE_ROUTE_MAX_EXPERTS = 1024;
constexpr int GATE_ROUTE_MAX_TOPK = 16;
struct GateRouteArgs {
    const float *scores;
    int scores_ld;
    int n;
    const float *bias;
    const int64_t *tid2eid;
    int n_vocab;
    const int *token_ids;
    int token_id;
    int n_experts, topk;
    float route_scale;
    int *idx;
    float *w;
    float *orig;
    unsigned *status;
    const uint16_t *gate_w;
    const float *x;
    int cols;
    float *ws_orig, *ws_biased, *scores_out;
    unsigned *counter;
};
hipError_t gate_route_launch(const GateRouteArgs &a, hipStream_t st);

/* Row r of x [rows][cols] (cols % 8 == 0, x 16-byte aligned) ->
 * o[r][c] = fp16(x[r][c] * 2^ex[r]) with ex[r] the power of two that puts the
 * row's largest finite magnitude in [2^14, 2^15) (0 for a row without one),
 * so no finite activation overflows fp16 and every one at or above 2^-28 of
 * the row maximum stays a normal fp16. The GEMMs that read o multiply their
 * fp32 results by 2^-ex[r], which is exact. */
hipError_t to_f16_rows_launch(uint16_t *o, int *ex, const float *x, int rows, int cols,
                              hipStream_t st);

/* out[row][f] for row-groups of one expert each: gate/up with SwiGLU (fp16
 * out, uses w1 and w3) or down (fp32 out). table == NULL: one group, the
 * rows 0..nrows-1, matrices m1 (and m3). */
struct GroupedArgs {
    const DSV4ExpertW *table;
    int n_experts;
    const int *grp_off, *tile_pre;
    const TileRec *tile_rec;
    const int *row_tok;       /* B row of each output row, NULL = itself  */
    DSV4QMat m1, m3;
    int nrows;                /* rows of B                                */
    const uint16_t *B;        /* fp16 [nrows][K]                          */
    const int *bexp;          /* [nrows] power of two B row r carries (its
                                 results are scaled by 2^-bexp[r]), or NULL */
    int K, N;
    void *out;                /* [rows][N]                                */
    float limit;
    unsigned *status;
};
int grouped_rows_per_tile(int tt);
hipError_t grouped_launch(int fmt, bool swiglu, int tt, const GroupedArgs &a, long max_tiles,
                          hipStream_t st);

/* Routed FP4 experts on the block-scaled MFMA with MXFP8 activations, over
 * the buckets of k_moe_route run with grouped_mx_rows_per_tile() rows per
 * tile. Gate/up (swiglu): B = x8 rows gathered through row_tok, out = mid as
 * e4m3 [rows][N] with E8M0 out_s [rows][N / 32]; down: B = mid rows, out =
 * fp32 [rows][N]. K % 128 == 0; N % 128 (gate/up) or % 256 (down) == 0. */
struct GroupedMxArgs {
    const DSV4ExpertW *table;
    int n_experts;
    const int *grp_off, *tile_pre;
    const TileRec *tile_rec;
    const int *row_tok;       /* B row of each bucket row, NULL = itself  */
    const uint8_t *B;         /* e4m3 [nrows][K]                          */
    const uint8_t *BS;        /* E8M0 [nrows][K / 32]                     */
    int nrows;
    int K, N;
    void *out;
    uint8_t *out_s;
    float limit;
    unsigned *status;
};
int grouped_mx_rows_per_tile();
/* fat tiles (more than 64 token rows) on `st`, thin tiles on `st_thin` */
hipError_t grouped_mx_launch(bool swiglu, const GroupedMxArgs &a, long max_tiles, hipStream_t st,
                             hipStream_t st_thin);

/* out[t] = sum_k w[t][k] * Y[pos[t][k]] (k order) + YS[t] */
struct CombineArgs {
    float *out;
    const float *Y, *YS, *w;
    const int *pos;
    int n, topk, hidden;
};
hipError_t moe_combine_launch(const CombineArgs &a, hipStream_t st);

} // namespace dsv4

#endif /* DSV4_INTERNAL_H */
