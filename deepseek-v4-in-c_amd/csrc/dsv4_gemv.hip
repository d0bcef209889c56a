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
 *   Load order is the schedule: the lane's x slice first (an L2 hit shared by
 *   every wave), then the block scales, then all ROWS x KCH weight chunks of
 *   the wave. Loads complete in issue order, so the first row's arithmetic
 *   starts as soon as its own chunks land while the later rows are still in
 *   flight, and x never waits behind weight traffic.
 *   Each row's lane partials are summed with a fixed DPP tree; lane r keeps
 *   row r's sum so the wave writes its ROWS outputs with one store.
 *
 * Bound: HBM. Algorithmic bytes per row = row bytes + its scales; the x
 * vector and y are read/written once per call.
 */
#include "dsv4_internal.h"
#include "dsv4_bf16.h"

namespace dsv4 {

/* One token's pass over the wave's ROWS rows: y[t*y_ld + o] for o in
 * [r0, r0+ROWS). W row pitch = row_bytes; scale grid row pitch = sc_cols
 * entries, scale block height blk_r, width 128 (FP8) or 32 (FP4) columns.
 * The weight loads sit inside the pass on purpose: for t = 0 they stream from
 * HBM, later tokens of the same call find them in cache, and the compiler
 * never holds a decoded copy of every chunk at once. */
template <int FMT, int KCH, int ROWS, bool FULL>
__device__ __forceinline__ void gemv_pass(const GemvArgs &a, int t, int lane, int r0)
{
    constexpr bool FP4 = FMT == FMT_FP4_E8M0;
    constexpr bool F32S = FMT == FMT_FP8_F32S;
    constexpr int CPL = FP4 ? 32 : 16;
    constexpr int BLK_C = FP4 ? 32 : 128;

    float xs[KCH][CPL];
    load_x_slice<FP4, KCH, FULL>(xs, a.x + (size_t)t * a.x_ld, lane, a.row_bytes);
    DSV4_ORDER();
    uint32_t sraw[ROWS][KCH];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = r0 + r < a.rows ? r0 + r : a.rows - 1;
        const size_t srow = (size_t)(row / a.blk_r) * a.sc_cols;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            const int b = chunk_byte(lane, j);
            const bool in = FULL || b < a.row_bytes;
            sraw[r][j] = ld_scale_raw<F32S>(a.S, srow + (in ? (FP4 ? 2 * b : b) / BLK_C : 0));
        }
    }
    DSV4_ORDER();
    u32x4 w[ROWS][KCH];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = r0 + r < a.rows ? r0 + r : a.rows - 1;
        load_w_row<KCH, FULL>(w[r], a.W + (size_t)row * a.row_bytes, lane, a.row_bytes);
    }
    DSV4_ORDER();
    if (!dsv4_opaque_true()) return;
    float keep = 0.0f;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < KCH; j++) {
            float sc = scale_from_raw<F32S>(sraw[r][j]);
            if (!FULL && chunk_byte(lane, j) >= a.row_bytes) sc = 0.0f;
            acc = fmaf(dot16<FP4>(w[r][j], xs[j]), sc, acc);
        }
        const float s = wave_sum(acc);
        if (lane == r) keep = s;
    }
    if (lane < ROWS && r0 + lane < a.rows) a.y[(size_t)t * a.y_ld + r0 + lane] = keep;
}

template <int FMT, int KCH, int ROWS, bool FULL>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a)
{
    const int lane = threadIdx.x & 63;
    const int r0 = wave_id() * ROWS;
    if (r0 >= a.rows) return;
    for (int t = 0; t < a.nt; t++) gemv_pass<FMT, KCH, ROWS, FULL>(a, t, lane, r0);
}

/* Rows per wave so that a wave keeps sixteen 16-byte chunks per lane (16 KiB)
 * in flight: ROWS x KCH = 16. */
template <int FMT, int KCH>
static hipError_t launch_k(const GemvArgs &a, hipStream_t st)
{
    constexpr int ROWS = 16 / KCH;
    constexpr int WAVES_PER_BLOCK = 4;
    const int waves = (a.rows + ROWS - 1) / ROWS;
    const int blocks = (waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    if (a.row_bytes == KCH * 1024)
        hipLaunchKernelGGL((k_gemv<FMT, KCH, ROWS, true>), dim3(blocks),
                           dim3(64 * WAVES_PER_BLOCK), 0, st, a);
    else
        hipLaunchKernelGGL((k_gemv<FMT, KCH, ROWS, false>), dim3(blocks),
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
    case 5: case 6: return launch_k<FMT, 6>(a, st);
    case 7: case 8: return launch_k<FMT, 8>(a, st);
    default: return hipErrorInvalidValue;
    }
}

/* ------------------------------------------------------------- BF16 --- */

/* One wave per ROWS rows: the rows go to LDS once, then for every token its
 * x goes to LDS and the rows' dot products run from there. ROWS x (1 KiB KCH
 * + 64) bytes of rows (64: a bank offset between rows), then up to 2 KiB
 * KCH of x. */
constexpr int BF16_PAD = 64;
template <int KCH, int ROWS>
__host__ __device__ constexpr size_t bf16_gemv_lds() { return (size_t)ROWS * (KCH * 1024 + BF16_PAD) + 2048 * KCH; }

template <int KCH, int ROWS>
__global__ __launch_bounds__(64) void k_gemv_bf16(GemvBf16Args a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x;
    const int r0 = blockIdx.x * ROWS;
    constexpr int STRIDE = KCH * 1024 + BF16_PAD;
    uint8_t *xl = lds + ROWS * STRIDE;
    bf16_rows_to_lds<KCH>(lds, STRIDE, a.W, r0, ROWS, a.rows - r0, 2 * a.cols, lane);
    const int r = lane >> 4;
    const uint16_t *wl = (const uint16_t *)(lds + (r < ROWS ? r : 0) * STRIDE);
    for (int t = 0; t < a.nt; t++) {
        /* a single wave: its reads of the previous token's x are done */
        bf16_x_to_lds(xl, a.x + (size_t)t * a.x_ld, a.cols, lane);
        __builtin_amdgcn_s_waitcnt(0x0F70);          /* vmcnt(0): rows and x landed */
        asm volatile("" ::: "memory");
        const double acc = bf16_row_dot(wl, (const float *)xl, a.cols, lane);
        if (r < ROWS && (lane & 15) == 0 && r0 + r < a.rows) a.y[(size_t)t * a.y_ld + r0 + r] = (float)acc;
    }
}

template <int KCH, int ROWS>
static hipError_t launch_bf16_k(const GemvBf16Args &a, hipStream_t st)
{
    constexpr size_t lds = bf16_gemv_lds<KCH, ROWS>();
    if constexpr (lds > 64 * 1024) {
        /* set once (not inside a stream capture of a later call) */
        static bool set = false;
        if (!set) {
            const hipError_t e = hipFuncSetAttribute((const void *)k_gemv_bf16<KCH, ROWS>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
            set = true;
        }
    }
    hipLaunchKernelGGL((k_gemv_bf16<KCH, ROWS>), dim3((unsigned)((a.rows + ROWS - 1) / ROWS)), dim3(64), lds,
                       st, a);
    return hipGetLastError();
}

hipError_t gemv_bf16_launch(const GemvBf16Args &a, hipStream_t st)
{
    if (a.rows <= 0 || a.cols <= 0 || a.cols % 8 || a.nt <= 0) return hipErrorInvalidValue;
    switch ((2 * a.cols + 1023) / 1024) {
    case 1: return launch_bf16_k<1, 4>(a, st);
    case 2: return launch_bf16_k<2, 4>(a, st);
    case 3: case 4: return launch_bf16_k<4, 4>(a, st);
    case 5: case 6: case 7: case 8: return launch_bf16_k<8, 4>(a, st);
    case 9: case 10: case 11: case 12: case 13: case 14: case 15: case 16: return launch_bf16_k<16, 4>(a, st);
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

/* ------------------------------------------------- generic geometry --- */

/* Any block geometry (blk_r >= 1 rows x blk_c >= 1 columns per scale, any
 * column count, rows of any width): the reference's generic bodies of fp8_n
 * and fp4_n (src/10_compute/dsv4_matmul_fp8.c:158-176,
 * src/10_compute/dsv4_matmul_fp4.c:143-162), which only fixtures and rows
 * wider than the fast kernels' limits reach. One wave per output row: for
 * each block of blk_c columns the lanes' products are summed (lane order
 * over the block, then a butterfly), the block sum times its scale is added
 * to the row's total in block order. */
template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_generic(GemvGenArgs a)
{
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + wave_in_group();
    if (o >= a.rows) return;
    const int scg = (a.cols + a.blk_c - 1) / a.blk_c;
    const size_t srow = (size_t)(o / a.blk_r) * (size_t)scg;
    const size_t rb = FMT == FMT_GEN_FP4 ? (size_t)a.cols / 2 : (size_t)a.cols;
    const uint8_t *wr = a.W + (size_t)o * rb;
    for (int t = 0; t < a.nt; t++) {
        const float *xt = a.x + (size_t)t * a.cols;
        float total = 0.0f;
        int bi = 0;
        for (int c0 = 0; c0 < a.cols; c0 += a.blk_c, bi++) {
            const int n = min(a.blk_c, a.cols - c0);
            float d = 0.0f;
            for (int i = lane; i < n; i += 64) {
                const int c = c0 + i;
                float w;
                if constexpr (FMT == FMT_GEN_FP4) {
                    const f32x2 p = dev_e2m1x2<0>((uint32_t)wr[c >> 1]);
                    w = (c & 1) ? p.y : p.x;
                } else {
                    w = dev_e4m3x2<false>((uint32_t)wr[c]).x;
                }
                d = fmaf(w, xt[c], d);
            }
#pragma unroll
            for (int sh = 32; sh >= 1; sh >>= 1) d += __shfl_xor(d, sh, 64);
            const float sc = FMT == FMT_GEN_FP8F ? ld_f32(a.S, srow + bi) : dev_e8m0(ld_u8(a.S, srow + bi));
            total = total + d * sc;
        }
        if (lane == 0) a.y[(size_t)t * a.rows + o] = total;
    }
}

hipError_t gemv_generic_launch(int fmt, const GemvGenArgs &a, hipStream_t st)
{
    if (a.rows <= 0 || a.cols <= 0 || a.blk_r <= 0 || a.blk_c <= 0 || a.nt <= 0 ||
        (fmt == FMT_GEN_FP4 && a.cols % 2))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.rows + 3) / 4)), block(256);
    switch (fmt) {
    case FMT_GEN_FP8: hipLaunchKernelGGL(k_gemv_generic<FMT_GEN_FP8>, grid, block, 0, st, a); break;
    case FMT_GEN_FP8F: hipLaunchKernelGGL(k_gemv_generic<FMT_GEN_FP8F>, grid, block, 0, st, a); break;
    case FMT_GEN_FP4: hipLaunchKernelGGL(k_gemv_generic<FMT_GEN_FP4>, grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace dsv4
