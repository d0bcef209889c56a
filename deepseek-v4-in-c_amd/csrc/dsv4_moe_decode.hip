/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_moe_decode.hip - one token through topk routed experts (+ the shared
 * expert) with the weighted combine, on resident expert weights.
 *
 * Replaces, for one decode token, the six dsv4_expert_forward calls and the
 * k-order sum of dsv4_layer_moe (src/70_decode/dsv4_layer.c:57-116), whose
 * per-expert body is src/10_compute/dsv4_ops.c:85-93.
 *
 * Two launches instead of 3 x topk GEMVs:
 *   k_gateup       every (slot, row-group) of w1 and w3 at once. A wave owns
 *                  ROWS rows j of BOTH w1 and w3 of one expert, so the SwiGLU
 *                  element mid[j] = swiglu(w1[j].x, w3[j].x) is formed in
 *                  registers and only `mid` (inter floats per slot) is
 *                  written.
 *   k_down_combine a wave owns ROWS output rows i and runs them through w2 of
 *                  every routed expert, then combines IN k ORDER exactly as
 *                  the reference does: out = 0; out += w[k]*y_k (product and
 *                  sum separately rounded) for k = 0..topk-1; out += shared.
 * Expert descriptors are read on the device from a table indexed by the
 * routing ids, so routing never has to visit the host.
 *
 * Bound: HBM (each expert's 13.4 MB read once).
 */
#include "dsv4_internal.h"

namespace dsv4 {

template <int FMT>
__device__ __forceinline__ float scale_of(const void *S, size_t idx)
{
    if constexpr (FMT == FMT_FP8_F32S) return ((const float *)S)[idx];
    else return dev_e8m0(((const uint8_t *)S)[idx]);
}

template <int FMT>
__device__ __forceinline__ bool desc_ok(const DSV4QMat &m, int rows, int cols)
{
    const int want = FMT == FMT_FP4_E8M0 ? DSV4_WFP4
                   : FMT == FMT_FP8_F32S ? DSV4_WFP8_F32S : DSV4_WFP8;
    const int blk_c = FMT == FMT_FP4_E8M0 ? 32 : 128;
    return m.wdt == want && m.rows == rows && m.cols == cols &&
           m.blk_c == blk_c && m.blk_r > 0;
}

template <int FMT, int KCH, int ROWS>
__global__ __launch_bounds__(256) void k_gateup(GateUpArgs a)
{
    constexpr int CPL = FMT == FMT_FP4_E8M0 ? 32 : 16;
    constexpr int BLK_C = FMT == FMT_FP4_E8M0 ? 32 : 128;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int groups = (a.inter + ROWS - 1) / ROWS;
    const int slot = wave / groups;
    if (slot >= a.nslots) return;
    const int j0 = (wave - slot * groups) * ROWS;

    DSV4ExpertW e;
    if (a.use_direct) {
        e = a.direct;
    } else {
        const int id = a.idx[slot];
        if (id < 0 || id >= a.n_experts) {
            if (lane == 0) atomicOr(a.status, (unsigned)ST_BAD_EXPERT_ID);
            for (int r = 0; r < ROWS; r++)
                if (lane == 0 && j0 + r < a.inter)
                    a.mid[(size_t)slot * a.mid_ld + j0 + r] = __uint_as_float(0x7FC00000u);
            return;
        }
        e = a.table[id];
    }
    if (!desc_ok<FMT>(e.w1, a.inter, a.hidden) || !desc_ok<FMT>(e.w3, a.inter, a.hidden)) {
        if (lane == 0) {
            atomicOr(a.status, (unsigned)ST_BAD_DESCRIPTOR);
            for (int r = 0; r < ROWS; r++)
                if (j0 + r < a.inter)
                    a.mid[(size_t)slot * a.mid_ld + j0 + r] = __uint_as_float(0x7FC00000u);
        }
        return;
    }

    const int row_bytes = FMT == FMT_FP4_E8M0 ? a.hidden / 2 : a.hidden;
    const int sc_cols = (a.hidden + BLK_C - 1) / BLK_C;
    const uint8_t *W1 = (const uint8_t *)e.w1.w, *W3 = (const uint8_t *)e.w3.w;

    u32x4 w1[ROWS][KCH], w3[ROWS][KCH];
    float s1[ROWS][KCH], s3[ROWS][KCH];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = j0 + r < a.inter ? j0 + r : a.inter - 1;
        const size_t sr1 = (size_t)(row / e.w1.blk_r) * sc_cols;
        const size_t sr3 = (size_t)(row / e.w3.blk_r) * sc_cols;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            const int b = 16 * lane + 1024 * j;
            if (b < row_bytes) {
                const int c0 = FMT == FMT_FP4_E8M0 ? 2 * b : b;
                w1[r][j] = ld_stream16(W1 + (size_t)row * row_bytes + b);
                w3[r][j] = ld_stream16(W3 + (size_t)row * row_bytes + b);
                s1[r][j] = scale_of<FMT>(e.w1.s, sr1 + c0 / BLK_C);
                s3[r][j] = scale_of<FMT>(e.w3.s, sr3 + c0 / BLK_C);
            } else {
                w1[r][j] = w3[r][j] = u32x4{0, 0, 0, 0};
                s1[r][j] = s3[r][j] = 0.0f;
            }
        }
    }
    float xs[KCH][CPL];
#pragma unroll
    for (int j = 0; j < KCH; j++) {
        const int b = 16 * lane + 1024 * j;
        const int c0 = FMT == FMT_FP4_E8M0 ? 2 * b : b;
#pragma unroll
        for (int i = 0; i < CPL; i += 4) {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (b < row_bytes) v = ld_f4(a.x + c0 + i);
            xs[j][i] = v.x; xs[j][i + 1] = v.y; xs[j][i + 2] = v.z; xs[j][i + 3] = v.w;
        }
    }
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            g = fmaf(dot16<FMT == FMT_FP4_E8M0>(w1[r][j], xs[j]), s1[r][j], g);
            u = fmaf(dot16<FMT == FMT_FP4_E8M0>(w3[r][j], xs[j]), s3[r][j], u);
        }
        g = wave_sum(g);
        u = wave_sum(u);
        if (lane == 0 && j0 + r < a.inter)
            a.mid[(size_t)slot * a.mid_ld + j0 + r] = dev_swiglu(g, u, a.limit);
    }
}

/* Routed experts are processed in groups of TK so a wave keeps
 * ROWS x TK x KCH loads in flight. */
template <int FMT, int KCH, int ROWS>
__global__ __launch_bounds__(256) void k_down_combine(DownCombineArgs a)
{
    constexpr int CPL = FMT == FMT_FP4_E8M0 ? 32 : 16;
    constexpr int BLK_C = FMT == FMT_FP4_E8M0 ? 32 : 128;
    constexpr int TK = 4;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int i0 = wave * ROWS;
    if (i0 >= a.hidden) return;

    const int row_bytes = FMT == FMT_FP4_E8M0 ? a.inter / 2 : a.inter;
    const int sc_cols = (a.inter + BLK_C - 1) / BLK_C;

    float out[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) out[r] = 0.0f;

    for (int k0 = 0; k0 < a.topk; k0 += TK) {
        u32x4 w[TK][ROWS][KCH];
        float sc[TK][ROWS][KCH];
        bool ok[TK];
#pragma unroll
        for (int q = 0; q < TK; q++) {
            const int k = k0 + q;
            ok[q] = false;
            DSV4QMat m;
            if (k < a.topk) {
                const int id = a.idx[k];
                if (id >= 0 && id < a.n_experts) {
                    m = a.table[id].w2;
                    ok[q] = desc_ok<FMT>(m, a.hidden, a.inter);
                    if (!ok[q] && lane == 0) atomicOr(a.status, (unsigned)ST_BAD_DESCRIPTOR);
                } else if (lane == 0) {
                    atomicOr(a.status, (unsigned)ST_BAD_EXPERT_ID);
                }
            }
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                const int row = i0 + r < a.hidden ? i0 + r : a.hidden - 1;
#pragma unroll
                for (int j = 0; j < KCH; j++) {
                    const int b = 16 * lane + 1024 * j;
                    if (ok[q] && b < row_bytes) {
                        const int c0 = FMT == FMT_FP4_E8M0 ? 2 * b : b;
                        w[q][r][j] = ld_stream16((const uint8_t *)m.w + (size_t)row * row_bytes + b);
                        sc[q][r][j] = scale_of<FMT>(m.s, (size_t)(row / m.blk_r) * sc_cols + c0 / BLK_C);
                    } else {
                        w[q][r][j] = u32x4{0, 0, 0, 0};
                        sc[q][r][j] = 0.0f;
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < TK; q++) {
            const int k = k0 + q;
            if (k >= a.topk) break;
            float xs[KCH][CPL];
#pragma unroll
            for (int j = 0; j < KCH; j++) {
                const int b = 16 * lane + 1024 * j;
                const int c0 = FMT == FMT_FP4_E8M0 ? 2 * b : b;
#pragma unroll
                for (int i = 0; i < CPL; i += 4) {
                    f32x4 v = {0.f, 0.f, 0.f, 0.f};
                    if (b < row_bytes) v = ld_f4(a.mid + (size_t)k * a.mid_ld + c0 + i);
                    xs[j][i] = v.x; xs[j][i + 1] = v.y; xs[j][i + 2] = v.z; xs[j][i + 3] = v.w;
                }
            }
            const float wk = a.w[k];
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < KCH; j++)
                    acc = fmaf(dot16<FMT == FMT_FP4_E8M0>(w[q][r][j], xs[j]), sc[q][r][j], acc);
                float yk = wave_sum(acc);
                if (!ok[q]) yk = __uint_as_float(0x7FC00000u);
                out[r] = __fadd_rn(out[r], __fmul_rn(wk, yk));
            }
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            if (i0 + r >= a.hidden) break;
            float o = out[r];
            if (a.shared) o = __fadd_rn(o, a.shared[i0 + r]);
            a.out[i0 + r] = o;
        }
    }
}

/* Rows per wave chosen so a wave keeps eight 16-byte chunks per lane in
 * flight: gate/up reads 2 x ROWS x KCH chunks, down/combine TK x ROWS x KCH. */
template <int FMT, int KCH>
static hipError_t launch_gateup_k(const GateUpArgs &a, hipStream_t st)
{
    constexpr int ROWS = KCH >= 4 ? 1 : 4 / KCH, WPB = 4;
    const long waves = (long)a.nslots * ((a.inter + ROWS - 1) / ROWS);
    const long blocks = (waves + WPB - 1) / WPB;
    hipLaunchKernelGGL((k_gateup<FMT, KCH, ROWS>), dim3((unsigned)blocks),
                       dim3(64 * WPB), 0, st, a);
    return hipGetLastError();
}

template <int FMT, int KCH>
static hipError_t launch_down_k(const DownCombineArgs &a, hipStream_t st)
{
    constexpr int ROWS = KCH >= 2 ? 1 : 2, WPB = 4;
    const int waves = (a.hidden + ROWS - 1) / ROWS;
    const int blocks = (waves + WPB - 1) / WPB;
    hipLaunchKernelGGL((k_down_combine<FMT, KCH, ROWS>), dim3(blocks),
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

template <int FMT>
static hipError_t down_fmt(const DownCombineArgs &a, hipStream_t st)
{
    const int row_bytes = FMT == FMT_FP4_E8M0 ? a.inter / 2 : a.inter;
    switch ((row_bytes + 1023) / 1024) {
    case 1: return launch_down_k<FMT, 1>(a, st);
    case 2: return launch_down_k<FMT, 2>(a, st);
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

hipError_t down_combine_launch(int fmt, const DownCombineArgs &a, hipStream_t st)
{
    switch (fmt) {
    case FMT_FP8_E8M0: return down_fmt<FMT_FP8_E8M0>(a, st);
    case FMT_FP8_F32S: return down_fmt<FMT_FP8_F32S>(a, st);
    case FMT_FP4_E8M0: return down_fmt<FMT_FP4_E8M0>(a, st);
    default: return hipErrorInvalidValue;
    }
}

} // namespace dsv4
