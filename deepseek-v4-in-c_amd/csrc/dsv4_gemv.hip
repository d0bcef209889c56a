/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_gemv.hip - decode matvec for packed FP8 / FP4 weights on gfx950.
 *
 * Replaces the nt == 1 bodies of fp8_n (src/10_compute/dsv4_matmul_fp8.c:55-100)
 * and fp4_n (src/10_compute/dsv4_matmul_fp4.c:51-86): y[o] = sum_c W[o,c] x[c]
 * with W decoded in registers and its block scale applied once per block.
 *
 * LAYOUT AND SCHEDULE
 *   A wavefront owns ROWS consecutive output rows. Lane L reads the 16 bytes at
 *   row byte offset 16 L + 1024 j (j = 0..KCH-1): one 128-bit load per lane,
 *   1 KiB contiguous per row per wave instruction. 16 bytes are 16 e4m3
 *   columns (inside one 128-wide FP8 scale block) or 32 e2m1 columns (exactly
 *   one 1x32 FP4 scale block), so every lane applies ONE scale per load.
 *   The lane's slice of x (KCH x 16 or KCH x 32 floats) is loaded once into
 *   registers and reused for every row the wave owns. All ROWS x KCH weight
 *   loads are issued before any arithmetic, so a wave keeps ROWS x KCH KiB
 *   in flight. Each row's lane partials are summed with a fixed DPP tree.
 *
 * Bound: HBM. Algorithmic bytes per row = row bytes + its scales; the x
 * vector and y are read/written once per call.
 */
#include "dsv4_internal.h"

namespace dsv4 {

template <int FMT>
struct Fmt;

/* FP8 e4m3, E8M0 scale per blk_r x 128 block. */
template <>
struct Fmt<FMT_FP8_E8M0> {
    static constexpr int COLS_PER_LANE = 16;
    __device__ static float scale(const void *S, size_t idx)
    {
        return dev_e8m0(((const uint8_t *)S)[idx]);
    }
};
/* FP8 e4m3, fp32 scale per blk_r x 128 block. */
template <>
struct Fmt<FMT_FP8_F32S> {
    static constexpr int COLS_PER_LANE = 16;
    __device__ static float scale(const void *S, size_t idx)
    {
        return ((const float *)S)[idx];
    }
};
/* FP4 e2m1, E8M0 scale per blk_r x 32 block. */
template <>
struct Fmt<FMT_FP4_E8M0> {
    static constexpr int COLS_PER_LANE = 32;
    __device__ static float scale(const void *S, size_t idx)
    {
        return dev_e8m0(((const uint8_t *)S)[idx]);
    }
};

/* y[t*y_ld + o] for o in [row0, row0+rows), t in [0, nt).
 * W row pitch = row_bytes; scale grid row pitch = sc_cols entries, scale block
 * height blk_r, width 128 (FP8) or 32 (FP4) columns. */
template <int FMT, int KCH, int ROWS>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a)
{
    constexpr int CPL = Fmt<FMT>::COLS_PER_LANE;
    constexpr int BLK_C = (FMT == FMT_FP4_E8M0) ? 32 : 128;
    const int lane = threadIdx.x & 63;
    const int wave = (blockIdx.x * (blockDim.x >> 6)) + (threadIdx.x >> 6);
    const int r0 = wave * ROWS;
    if (r0 >= a.rows) return;

    /* One pass per token. The weight chunks are (re)loaded inside the pass:
     * for t = 0 they stream from HBM, later tokens find them in cache. Keeping
     * the loads inside the loop also keeps the compiler from decoding every
     * chunk once up front (which would need 8 x 32 live floats). */
    for (int t = 0; t < a.nt; t++) {
        u32x4 w[ROWS][KCH];
        float sc[ROWS][KCH];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int row = r0 + r < a.rows ? r0 + r : a.rows - 1;
            const uint8_t *wr = a.W + (size_t)row * a.row_bytes;
            const size_t srow = (size_t)(row / a.blk_r) * a.sc_cols;
#pragma unroll
            for (int j = 0; j < KCH; j++) {
                const int b = 16 * lane + 1024 * j;
                if (b < a.row_bytes) {
                    w[r][j] = ld_stream16(wr + b);
                    const int c0 = (FMT == FMT_FP4_E8M0) ? 2 * b : b;
                    sc[r][j] = Fmt<FMT>::scale(a.S, srow + c0 / BLK_C);
                } else {
                    w[r][j] = u32x4{0, 0, 0, 0};
                    sc[r][j] = 0.0f;
                }
            }
        }
        const float *xt = a.x + (size_t)t * a.x_ld;
        float xs[KCH][CPL];
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            const int b = 16 * lane + 1024 * j;
            const int c0 = (FMT == FMT_FP4_E8M0) ? 2 * b : b;
            if (b < a.row_bytes) {
#pragma unroll
                for (int i = 0; i < CPL; i += 4) {
                    const f32x4 v = ld_f4(xt + c0 + i);
                    xs[j][i] = v.x; xs[j][i + 1] = v.y;
                    xs[j][i + 2] = v.z; xs[j][i + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < CPL; i++) xs[j][i] = 0.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < KCH; j++)
                acc = fmaf(dot16<FMT == FMT_FP4_E8M0>(w[r][j], xs[j]), sc[r][j], acc);
            const float s = wave_sum(acc);
            if (lane == 0 && r0 + r < a.rows)
                a.y[(size_t)t * a.y_ld + r0 + r] = s;
        }
    }
}

/* Rows per wave so that each wave keeps eight 16-byte chunks per lane (8 KiB)
 * in flight: ROWS x KCH = 8. */
template <int FMT, int KCH>
static hipError_t launch_k(const GemvArgs &a, hipStream_t st)
{
    constexpr int ROWS = 8 / KCH;
    constexpr int WAVES_PER_BLOCK = 4;
    const int waves = (a.rows + ROWS - 1) / ROWS;
    const int blocks = (waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    hipLaunchKernelGGL((k_gemv<FMT, KCH, ROWS>), dim3(blocks),
                       dim3(64 * WAVES_PER_BLOCK), 0, st, a);
    return hipGetLastError();
}

template <int FMT>
static hipError_t launch_fmt(const GemvArgs &a, hipStream_t st)
{
    const int kch = (a.row_bytes + 1023) / 1024;
    switch (kch) {
    case 1: return launch_k<FMT, 1>(a, st);
    case 2: return launch_k<FMT, 2>(a, st);
    case 3: return launch_k<FMT, 3>(a, st);
    case 4: return launch_k<FMT, 4>(a, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t gemv_launch(int fmt, const GemvArgs &a, hipStream_t st)
{
    switch (fmt) {
    case FMT_FP8_E8M0: return launch_fmt<FMT_FP8_E8M0>(a, st);
    case FMT_FP8_F32S: return launch_fmt<FMT_FP8_F32S>(a, st);
    case FMT_FP4_E8M0: return launch_fmt<FMT_FP4_E8M0>(a, st);
    default: return hipErrorInvalidValue;
    }
}

} // namespace dsv4
