/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_gemm.hip - prefill GEMM on block-scaled FP8 weights, CDNA4 MFMA.
 *
 * C[m][n] = sum_k A[m][k] * W[n][k] for an e4m3 weight W with one fp32 (or
 * E8M0) scale per 128 x 128 block and activations quantized to e4m3 with one
 * fp32 scale per 1 x 128 group (k_quant_act_fp8_1x128). What it replaces:
 * the prefill projection seam (src/80_prefill/dsv4_prefill_proj.c:17-27), whose
 * GPU leg is the Vulkan GEMM (src/80_prefill/dsv4_prefill_vk_gemm.c:63-132,
 * src/10_compute/shaders/gemm_fp8.comp) and whose CPU leg is fp8_n with nt > 1
 * (src/10_compute/dsv4_matmul_fp8.c:102-155).
 *
 * SCHEDULE
 *   A workgroup of four waves owns a 128 (tokens) x 256 (features) tile of C;
 *   wave (wm, wn) owns 64 tokens x 128 features. K advances in 128-wide
 *   blocks, one scale block each: the workgroup stages the A block
 *   (128 x 128 B) and the W block (256 x 128 B) in LDS (rows padded to 144 B,
 *   which makes the 16-byte operand reads bank-conflict free), double
 *   buffered so the next block's global loads are in flight while this one
 *   multiplies.
 *   The MFMA is v_mfma_scale_f32_32x32x64_f8f6f4 with both hardware scales
 *   set to 1 (E8M0 127): W rows are its A operand and tokens its B operand,
 *   so each lane's 16 outputs of a 32 x 32 tile share one token and one 128-row
 *   weight block. The product of a 128-K block starts from zero and is then
 *   folded into the fp32 accumulator with the two fp32 block scales,
 *   acc += partial * (s_a[token][kb] * s_w[nb][kb]) -- fp32 scales cannot ride
 *   in the E8M0 hardware scale operands.
 *   Operand layout of the FP8 MFMA (measured on gfx950): lane l supplies row
 *   l % 32 with k in [16 (l/32), +16) in bytes 0-15 and [32 + 16 (l/32), +16) in
 *   bytes 16-31 of each 64-wide k step; accumulator element e of lane l is
 *   row 8 (e/4) + 4 (l/32) + e % 4, column l % 32.
 *
 * Bound: MFMA (2 M N K flops; 68.7 GFLOP at 2048 x 4096 x 4096).
 */
#include <type_traits>

#include "dsv4_internal.h"

namespace dsv4 {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int GM = 128;          /* tokens per workgroup tile            */
constexpr int GN = 256;          /* features per workgroup tile          */
constexpr int GK = 128;          /* k per stage = one scale block        */
constexpr int NSTAGE = 3;        /* LDS ring: stage kb+2 loads while kb multiplies */
/* one stage: A rows and W rows of 128 bytes (16-byte chunks XOR-swizzled),
 * the tile's token scales, the two weight-block scales, a landing pad */
constexpr int ST_A = 0;
constexpr int ST_W = GM * GK;
constexpr int ST_SA = ST_W + GN * GK;
constexpr int ST_SW = ST_SA + GM * 4;
constexpr int ST_PAD = ST_SW + 256;
constexpr int STAGE = ST_PAD + 256;
constexpr int LDS_BYTES = NSTAGE * STAGE;
constexpr int VMEM_PER_STAGE = 13;   /* per wave: 4 A + 8 W + 1 scale load */
constexpr int E8M0_ONE = 127;

/* Physical 16-byte slot of logical chunk c in staged row r. Sixteen lanes
 * reading the same chunk of sixteen consecutive rows hit sixteen different
 * 16-byte bank groups. */
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

__device__ __forceinline__ v8i lds_operand(const uint8_t *rowp, int row, int ks, int g)
{
    const int c0 = 4 * ks + g;
    const u32x4 lo = *(const u32x4 *)(rowp + 16 * swz(row, c0));
    const u32x4 hi = *(const u32x4 *)(rowp + 16 * swz(row, c0 + 2));
    v8i v;
    v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
    v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
    return v;
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;   /* quiet NaN */
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

/* global -> LDS, 16 (or 4) bytes per lane, lane l landing at dst + l * size */
__device__ __forceinline__ void dma16(const void *src, uint8_t *dst)
{
    __builtin_amdgcn_global_load_lds(gptr(src), (lds_void *)dst, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *src, uint8_t *dst)
{
    __builtin_amdgcn_global_load_lds(gptr(src), (lds_void *)dst, 4, 0, 0);
}

} // namespace

/* Issue the direct-to-LDS loads of K block kb into stage buffer `st`:
 * instruction j of the workgroup fills staged rows 8j .. 8j+7 (1 KiB), lane l
 * row 8j + l/8, slot l%8, i.e. logical chunk swz(row, l%8) of that row. */
template <bool WF32S>
__device__ __forceinline__ void issue_stage(const GemmArgs &a, uint8_t *st, int kb,
                                            int m0, int n0, int wave, int lane)
{
    const size_t kofs = (size_t)kb * GK;
    const int r8 = lane >> 3, p = lane & 7;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int j = wave * 4 + i, r = 8 * j + r8;
        int m = m0 + r;
        m = m < a.M ? m : a.M - 1;
        dma16(a.Aq + (size_t)m * a.K + kofs + 16 * swz(r, p), st + ST_A + 1024 * j);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int j = wave * 8 + i, r = 8 * j + r8;
        int n = n0 + r;
        n = n < a.N ? n : a.N - 1;
        dma16(a.W + (size_t)n * a.K + kofs + 16 * swz(r, p), st + ST_W + 1024 * j);
    }
    const int nkb = a.K / GK;
    if (wave < 2) {
        int m = m0 + 64 * wave + lane;
        m = m < a.M ? m : a.M - 1;
        dma4(a.Sa + (size_t)m * nkb + kb, st + ST_SA + 256 * wave);
    } else {
        /* wave 2: the two weight-block scales (lanes 0, 1); wave 3 lands in
         * the pad. An E8M0 scale is a byte: the aligned dword holding it is
         * loaded and the byte picked when read (sw_byte_shift). */
        int nb = n0 / 128 + (lane & 1);
        nb = nb < a.N / 128 ? nb : a.N / 128 - 1;
        const size_t si = (size_t)nb * nkb + kb;
        const uint8_t *src = WF32S ? (const uint8_t *)a.Sw + 4 * si
                                   : (const uint8_t *)a.Sw + (si & ~(size_t)3);
        dma4(src, st + (wave == 2 ? ST_SW : ST_PAD));
    }
}

template <bool WF32S, bool OUT_BF16>
__global__ __launch_bounds__(256) void k_gemm_fp8(GemmArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
    const int nkb = a.K / GK;
    const int col = lane & 31, g = lane >> 5;
    const bool wave_live = n0 + wn * 128 < a.N;

    v16f acc[4][2];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[t][u][e] = 0.0f;
    v16f zero;
#pragma unroll
    for (int e = 0; e < 16; e++) zero[e] = 0.0f;

    issue_stage<WF32S>(a, lds, 0, m0, n0, wave, lane);
    if (nkb > 1) issue_stage<WF32S>(a, lds + STAGE, 1, m0, n0, wave, lane);

    int buf = 0;
    for (int kb = 0; kb < nkb; kb++) {
        /* this wave's loads of stage kb are done once at most the next
         * stage's VMEM_PER_STAGE loads are outstanding; the barrier makes
         * every wave's share visible and frees the buffer of block kb-1 */
        if (kb + 1 < nkb) __builtin_amdgcn_s_waitcnt(0x0F70 | VMEM_PER_STAGE);  /* vmcnt(13) */
        else __builtin_amdgcn_s_waitcnt(0x0F70);                                  /* vmcnt(0)  */
        /* A plain barrier: __syncthreads() would add a release fence that
         * drains every outstanding load, including the next stage's. LDS
         * written by a completed direct load is visible to the whole
         * workgroup, and the loads behind the wait above are this wave's. */
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");   /* keep LDS reads below the barrier */
        if (kb + 2 < nkb) {
            int nbuf = buf + 2;
            nbuf = nbuf >= NSTAGE ? nbuf - NSTAGE : nbuf;
            issue_stage<WF32S>(a, lds + nbuf * STAGE, kb + 2, m0, n0, wave, lane);
        }
        const uint8_t *stage = lds + buf * STAGE;
        const float *sa = (const float *)(stage + ST_SA);
        const uint8_t *As = stage + ST_A + (wm * 64) * GK;
        const uint8_t *Ws = stage + ST_W + (wn * 128) * GK;

        v8i bm[2][2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int u = 0; u < 2; u++)
                bm[ks][u] = lds_operand(As + (u * 32 + col) * GK, u * 32 + col, ks, g);
        float sw;
        if constexpr (WF32S) {
            sw = *(const float *)(stage + ST_SW + 4 * wn);
        } else {
            int nb = n0 / 128 + wn;
            nb = nb < a.N / 128 ? nb : a.N / 128 - 1;
            const int shift = 8 * (int)(((size_t)nb * nkb + kb) & 3);
            sw = dev_e8m0((*(const uint32_t *)(stage + ST_SW + 4 * wn) >> shift) & 0xFFu);
        }
        float cs[2];
#pragma unroll
        for (int u = 0; u < 2; u++) cs[u] = sa[wm * 64 + u * 32 + col] * sw;
        /* Software pipelined: tile t's four MFMAs are issued before tile
         * t-1's promotion FMAs, so the VALU folds one tile while the matrix
         * unit multiplies the next (a wave issues in order; with one wave per
         * SIMD nothing else fills those cycles). */
        v16f p0[2], p1[2];
#pragma unroll
        for (int t = 0; t <= 4; t++) {
            if (t < 4) {
                const v8i an0 = lds_operand(Ws + (t * 32 + col) * GK, t * 32 + col, 0, g);
                const v8i an1 = lds_operand(Ws + (t * 32 + col) * GK, t * 32 + col, 1, g);
                v16f q0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(an0, bm[0][0], zero, 0, 0, 0, E8M0_ONE, 0, E8M0_ONE);
                v16f q1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(an0, bm[0][1], zero, 0, 0, 0, E8M0_ONE, 0, E8M0_ONE);
                p0[t & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(an1, bm[1][0], q0, 0, 0, 0, E8M0_ONE, 0, E8M0_ONE);
                p1[t & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(an1, bm[1][1], q1, 0, 0, 0, E8M0_ONE, 0, E8M0_ONE);
            }
            if (t > 0) {
                const int tp = t - 1;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    acc[tp][0][e] = fmaf(p0[tp & 1][e], cs[0], acc[tp][0][e]);
                    acc[tp][1][e] = fmaf(p1[tp & 1][e], cs[1], acc[tp][1][e]);
                }
            }
        }
        buf = buf + 1 == NSTAGE ? 0 : buf + 1;
    }

    if (!wave_live) return;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int m = m0 + wm * 64 + u * 32 + col;
        if (m >= a.M) continue;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = n0 + wn * 128 + t * 32 + 8 * q + 4 * g;
                const float v0 = acc[t][u][4 * q], v1 = acc[t][u][4 * q + 1];
                const float v2 = acc[t][u][4 * q + 2], v3 = acc[t][u][4 * q + 3];
                if constexpr (OUT_BF16) {
                    uint2 pk;
                    pk.x = f32_to_bf16_bits(v0) | (f32_to_bf16_bits(v1) << 16);
                    pk.y = f32_to_bf16_bits(v2) | (f32_to_bf16_bits(v3) << 16);
                    *(uint2 *)((uint16_t *)a.C + (size_t)m * a.ldc + n) = pk;
                } else {
                    *(f32x4 *)((float *)a.C + (size_t)m * a.ldc + n) = f32x4{v0, v1, v2, v3};
                }
            }
    }
}

template <bool WS, bool OB>
static hipError_t launch_gemm(const GemmArgs &a, hipStream_t st)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm_fp8<WS, OB>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    const dim3 grid((unsigned)((a.N + GN - 1) / GN), (unsigned)((a.M + GM - 1) / GM)), block(256);
    hipLaunchKernelGGL((k_gemm_fp8<WS, OB>), grid, block, LDS_BYTES, st, a);
    return hipGetLastError();
}

hipError_t gemm_fp8_launch(const GemmArgs &a, bool w_f32s, bool out_bf16, hipStream_t st)
{
    if (a.K % GK || a.N % 128 || a.M <= 0) return hipErrorInvalidValue;
    if (w_f32s) return out_bf16 ? launch_gemm<true, true>(a, st) : launch_gemm<true, false>(a, st);
    return out_bf16 ? launch_gemm<false, true>(a, st) : launch_gemm<false, false>(a, st);
}

} // namespace dsv4
