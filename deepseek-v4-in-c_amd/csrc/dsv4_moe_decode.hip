/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_moe_decode.hip - one token through topk routed experts (+ the shared
 * expert) with the weighted combine, on resident expert weights.
 *
 * Replaces, for one decode token, the six dsv4_expert_forward calls and the
 * k-order sum of dsv4_layer_moe (src/70_decode/dsv4_layer.c:57-116), whose
 * per-expert body is src/10_compute/dsv4_ops.c:85-93.
 *
 * Two launches instead of 3 x topk GEMVs:
 *   k_gateup  every (slot, row-group) of w1 and w3 at once. A wave owns ROWS
 *             rows j of BOTH w1 and w3 of one expert, so the SwiGLU element
 *             mid[j] = swiglu(w1[j].x, w3[j].x) is formed in registers and
 *             only `mid` (inter floats per slot) is written.
 *   k_down    one workgroup per group of 16 output rows with one wave per
 *             routed expert k: wave k forms y_k = w2_k . mid_k for those rows
 *             into LDS; after the barrier the first wave combines them IN k
 *             ORDER exactly as the reference does -- out = 0;
 *             out += w[k] * y_k (product and sum separately rounded) for
 *             k = 0..topk-1; out += shared. No global synchronisation, so the
 *             result is bitwise reproducible.
 * Expert descriptors are read on the device from a table indexed by the
 * routing ids, so routing never has to visit the host.
 *
 * Every wave issues its activation slice, then its scales, then all of its
 * weight chunks (16 x 16 bytes per lane) before any arithmetic, and consumes
 * them in issue order.
 *
 * Bound: HBM (each expert's 13.4 MB read once).
 */
#include "dsv4_internal.h"

namespace dsv4 {

template <int FMT>
__device__ __forceinline__ bool desc_ok(const DSV4QMat &m, int rows, int cols)
{
    const int want = FMT == FMT_FP4_E8M0 ? DSV4_WFP4
                   : FMT == FMT_FP8_F32S ? DSV4_WFP8_F32S : DSV4_WFP8;
    const int blk_c = FMT == FMT_FP4_E8M0 ? 32 : 128;
    return m.wdt == want && m.rows == rows && m.cols == cols &&
           m.blk_c == blk_c && m.blk_r > 0 && m.w != nullptr && m.s != nullptr;
}

__device__ __forceinline__ float qnan() { return __uint_as_float(0x7FC00000u); }

template <int FMT, int KCH, int ROWS, bool FULL>
__global__ __launch_bounds__(256) void k_gateup(GateUpArgs a)
{
    constexpr bool FP4 = FMT == FMT_FP4_E8M0;
    constexpr bool F32S = FMT == FMT_FP8_F32S;
    constexpr int BLK_C = FP4 ? 32 : 128;
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int groups = (a.inter + ROWS - 1) / ROWS;
    const int slot = wave / groups;
    if (slot >= a.nslots) return;
    const int j0 = (wave - slot * groups) * ROWS;
    float *mid = a.mid + (size_t)slot * a.mid_ld;

    DSV4ExpertW e;
    unsigned bad = 0;
    if (a.use_direct) {
        e = a.direct;
    } else {
        const int id = ld_uniform(a.idx, slot);
        if (id < 0 || id >= a.n_experts) bad = ST_BAD_EXPERT_ID;
        else e = ld_uniform(a.table, id);
    }
    if (!bad && (!desc_ok<FMT>(e.w1, a.inter, a.hidden) || !desc_ok<FMT>(e.w3, a.inter, a.hidden)))
        bad = ST_BAD_DESCRIPTOR;
    if (bad) {
        if (lane == 0) atomicOr(a.status, bad);
        if (lane < ROWS && j0 + lane < a.inter) mid[j0 + lane] = qnan();
        return;
    }

    const int row_bytes = FP4 ? a.hidden / 2 : a.hidden;
    const int sc_cols = (a.hidden + BLK_C - 1) / BLK_C;
    const uint8_t *W1 = (const uint8_t *)e.w1.w, *W3 = (const uint8_t *)e.w3.w;

    float xs[KCH][FP4 ? 32 : 16];
    load_x_slice<FP4, KCH, FULL>(xs, a.x, lane, row_bytes);
    DSV4_ORDER();
    uint32_t s1[ROWS][KCH], s3[ROWS][KCH];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = j0 + r < a.inter ? j0 + r : a.inter - 1;
        const size_t sr1 = (size_t)(row / e.w1.blk_r) * sc_cols;
        const size_t sr3 = (size_t)(row / e.w3.blk_r) * sc_cols;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            const int b = chunk_byte(lane, j);
            const bool in = FULL || b < row_bytes;
            const int cb = in ? (FP4 ? 2 * b : b) / BLK_C : 0;
            s1[r][j] = ld_scale_raw<F32S>(e.w1.s, sr1 + cb);
            s3[r][j] = ld_scale_raw<F32S>(e.w3.s, sr3 + cb);
        }
    }
    DSV4_ORDER();
    u32x4 w1[ROWS][KCH], w3[ROWS][KCH];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = j0 + r < a.inter ? j0 + r : a.inter - 1;
        load_w_row<KCH, FULL>(w1[r], W1 + (size_t)row * row_bytes, lane, row_bytes);
        load_w_row<KCH, FULL>(w3[r], W3 + (size_t)row * row_bytes, lane, row_bytes);
    }
    DSV4_ORDER();
    if (!dsv4_opaque_true()) return;
    float keep = 0.0f;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            float c1 = scale_from_raw<F32S>(s1[r][j]), c3 = scale_from_raw<F32S>(s3[r][j]);
            if (!FULL && chunk_byte(lane, j) >= row_bytes) c1 = c3 = 0.0f;
            g = fmaf(dot16<FP4>(w1[r][j], xs[j]), c1, g);
            u = fmaf(dot16<FP4>(w3[r][j], xs[j]), c3, u);
        }
        g = wave_sum(g);
        u = wave_sum(u);
        if (lane == r) keep = dev_swiglu(g, u, a.limit);
    }
    if (lane < ROWS && j0 + lane < a.inter) mid[j0 + lane] = keep;
}

/* Rows of one output group: the combine granule of k_down. */
constexpr int DOWN_ROWS = 16;

/* One workgroup per group of DOWN_ROWS output rows, one wave per routed
 * expert k (blockDim = 64 * topk). Wave k computes y_k = w2_k . mid_k for the
 * group's rows and leaves them in LDS; after the barrier wave 0 combines them
 * in k order. */
template <int KCH, bool FULL>
__global__ __launch_bounds__(1024) void k_down(DownArgs a)
{
    constexpr int ROWS = DOWN_ROWS;
    __shared__ float ylds[16][ROWS];
    const int lane = threadIdx.x & 63;
    const int k = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int i0 = blockIdx.x * ROWS;
    const int row_bytes = a.inter / 2;
    const int sc_cols = a.inter / 32;

    unsigned bad = 0;
    DSV4QMat m;
    const int id = ld_uniform(a.idx, k);
    if (id < 0 || id >= a.n_experts) bad = ST_BAD_EXPERT_ID;
    else {
        m = ld_uniform(a.table, id).w2;
        if (!desc_ok<FMT_FP4_E8M0>(m, a.hidden, a.inter)) bad = ST_BAD_DESCRIPTOR;
    }

    float mine = qnan();
    if (!bad) {
        float xs[KCH][32];
        load_x_slice<true, KCH, FULL>(xs, a.mid + (size_t)k * a.mid_ld, lane, row_bytes);
        DSV4_ORDER();
        uint32_t sraw[ROWS][KCH];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int row = i0 + r < a.hidden ? i0 + r : a.hidden - 1;
            const size_t srow = (size_t)(row / m.blk_r) * sc_cols;
#pragma unroll
            for (int j = 0; j < KCH; j++) {
                const int b = chunk_byte(lane, j);
                const bool in = FULL || b < row_bytes;
                sraw[r][j] = ld_scale_raw<false>(m.s, srow + (in ? (2 * b) / 32 : 0));
            }
        }
        DSV4_ORDER();
        u32x4 w[ROWS][KCH];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int row = i0 + r < a.hidden ? i0 + r : a.hidden - 1;
            load_w_row<KCH, FULL>(w[r], (const uint8_t *)m.w + (size_t)row * row_bytes, lane, row_bytes);
        }
        DSV4_ORDER();
        if (dsv4_opaque_true()) {
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < KCH; j++) {
                    float sc = dev_e8m0(sraw[r][j]);
                    if (!FULL && chunk_byte(lane, j) >= row_bytes) sc = 0.0f;
                    acc = fmaf(dot16<true>(w[r][j], xs[j]), sc, acc);
                }
                acc = wave_sum(acc);
                if (lane == r) mine = acc;
            }
        }
    } else if (lane == 0) {
        atomicOr(a.status, bad);
    }
    if (lane < ROWS) ylds[k][lane] = mine;
    __syncthreads();
    if (k != 0 || lane >= ROWS || i0 + lane >= a.hidden) return;

    /* k-order combine of the group's rows (lane r = row i0 + r) */
    const int row = i0 + lane;
    float o = 0.0f;
    for (int kk = 0; kk < a.topk; kk++)
        o = __fadd_rn(o, __fmul_rn(ld_uniform(a.w, kk), ylds[kk][lane]));
    if (a.shared) o = __fadd_rn(o, a.shared[row]);
    a.out[row] = o;
}

/* Rows per wave chosen so a wave keeps sixteen 16-byte chunks per lane in
 * flight: gate/up reads 2 x ROWS x KCH chunks. */
template <int FMT, int KCH>
static hipError_t launch_gateup_k(const GateUpArgs &a, hipStream_t st)
{
    constexpr int ROWS = KCH >= 8 ? 1 : 8 / KCH, WPB = 4;
    const long waves = (long)a.nslots * ((a.inter + ROWS - 1) / ROWS);
    const long blocks = (waves + WPB - 1) / WPB;
    const int row_bytes = FMT == FMT_FP4_E8M0 ? a.hidden / 2 : a.hidden;
    if (row_bytes == KCH * 1024)
        hipLaunchKernelGGL((k_gateup<FMT, KCH, ROWS, true>), dim3((unsigned)blocks),
                           dim3(64 * WPB), 0, st, a);
    else
        hipLaunchKernelGGL((k_gateup<FMT, KCH, ROWS, false>), dim3((unsigned)blocks),
                           dim3(64 * WPB), 0, st, a);
    return hipGetLastError();
}

template <int FMT>
static hipError_t gateup_fmt(const GateUpArgs &a, hipStream_t st)
{
    const int row_bytes = FMT == FMT_FP4_E8M0 ? a.hidden / 2 : a.hidden;
    switch ((row_bytes + 1023) / 1024) {
    case 1: return launch_gateup_k<FMT, 1>(a, st);
    case 2: return launch_gateup_k<FMT, 2>(a, st);
    case 3: return launch_gateup_k<FMT, 3>(a, st);
    case 4: return launch_gateup_k<FMT, 4>(a, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t gateup_launch(int fmt, const GateUpArgs &a, hipStream_t st)
{
    switch (fmt) {
    case FMT_FP8_E8M0: return gateup_fmt<FMT_FP8_E8M0>(a, st);
    case FMT_FP8_F32S: return gateup_fmt<FMT_FP8_F32S>(a, st);
    case FMT_FP4_E8M0: return gateup_fmt<FMT_FP4_E8M0>(a, st);
    default: return hipErrorInvalidValue;
    }
}

int down_groups(int hidden) { return (hidden + DOWN_ROWS - 1) / DOWN_ROWS; }

hipError_t down_launch(const DownArgs &a, hipStream_t st)
{
    if (a.topk < 1 || a.topk > 16) return hipErrorInvalidValue;
    const int row_bytes = a.inter / 2;
    const dim3 grid((unsigned)down_groups(a.hidden)), block(64 * a.topk);
    switch ((row_bytes + 1023) / 1024) {
    case 1:
        if (row_bytes == 1024) hipLaunchKernelGGL((k_down<1, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((k_down<1, false>), grid, block, 0, st, a);
        break;
    case 2:
        if (row_bytes == 2048) hipLaunchKernelGGL((k_down<2, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((k_down<2, false>), grid, block, 0, st, a);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace dsv4
