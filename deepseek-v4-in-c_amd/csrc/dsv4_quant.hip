/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_quant.hip - dequantization check kernel, the weight / activation
 * quantizers, and the seeded synthetic-tensor generator.
 *
 * dequant     out[r][c] = decode(W[r][c]) * scale(block of r, c), one fp32
 *             multiply, with the SAME decoders the matmul kernels use
 *             (dsv4_dev.h). For E8M0 scales the product is exact; this is the
 *             reference's dequantized value dsv4_e4m3_to_f32(b) *
 *             dsv4_e8m0_to_f32(s) / dsv4_fp4_at * e8m0
 *             (src/10_compute/dsv4_quant.h:72-172).
 * quantizers  The reference ships pre-quantized weights and never quantizes
 *             activations, so these are this library's own definitions; the
 *             CPU oracle states the same rules and the tests compare the two
 *             byte for byte:
 *               e4m3(v)   round to nearest even, saturate at +-448
 *               e2m1(v)   round to nearest even, saturate at +-6
 *               FP8 weights, fp32 scale per 128x128 = blockmax/448
 *               FP4 weights, E8M0 per 1x32, 2^e the least power of two with
 *                 6 * 2^e >= blockmax (exact, no rounded logarithm)
 *               activations e4m3, fp32 scale per 1x128 = groupmax/448
 *               activations e4m3, E8M0 per 1x32 with 448 * 2^e >= groupmax
 *             Division is IEEE correctly rounded (hipcc's default).
 * synth       counter-based: u64 hash of (seed, index) -> two uniforms ->
 *             Box-Muller in double -> fp32 (optionally rounded to bf16).
 */
#include "dsv4_internal.h"

namespace dsv4 {

/* ------------------------------------------------------------ dequant --- */

template <int FMT>
__global__ __launch_bounds__(256) void k_dequant(DSV4QMat m, float *out)
{
    /* one thread per 16-byte chunk */
    const int row_bytes = FMT == FMT_FP4_E8M0 ? m.cols / 2 : m.cols;
    const int chunks = row_bytes / 16;
    const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (long)m.rows * chunks) return;
    const int r = (int)(id / chunks), ch = (int)(id % chunks);
    const u32x4 w = *(const u32x4 *)((const uint8_t *)m.w + (size_t)r * row_bytes + 16 * ch);
    constexpr int BLK_C = FMT == FMT_FP4_E8M0 ? 32 : 128;
    const int sc_cols = (m.cols + BLK_C - 1) / BLK_C;
    const int c0 = FMT == FMT_FP4_E8M0 ? 32 * ch : 16 * ch;
    const size_t si = (size_t)(r / m.blk_r) * sc_cols + c0 / BLK_C;
    float s;
    if constexpr (FMT == FMT_FP8_F32S) s = ((const float *)m.s)[si];
    else s = dev_e8m0(((const uint8_t *)m.s)[si]);
    float *o = out + (size_t)r * m.cols + c0;
    if constexpr (FMT == FMT_FP4_E8M0) {
        float f[32];
        dev_dec32_e2m1(w, f);
#pragma unroll
        for (int i = 0; i < 32; i++) o[i] = __fmul_rn(f[i], s);
    } else {
        float f[16];
        dev_dec16_e4m3(w, f);
#pragma unroll
        for (int i = 0; i < 16; i++) o[i] = __fmul_rn(f[i], s);
    }
}

hipError_t dequant_launch(int fmt, const DSV4QMat &m, float *out, hipStream_t st)
{
    const int row_bytes = qmat_row_bytes(&m);
    const long n = (long)m.rows * (row_bytes / 16);
    const unsigned blocks = (unsigned)((n + 255) / 256);
    switch (fmt) {
    case FMT_FP8_E8M0: hipLaunchKernelGGL(k_dequant<FMT_FP8_E8M0>, dim3(blocks), dim3(256), 0, st, m, out); break;
    case FMT_FP8_F32S: hipLaunchKernelGGL(k_dequant<FMT_FP8_F32S>, dim3(blocks), dim3(256), 0, st, m, out); break;
    case FMT_FP4_E8M0: hipLaunchKernelGGL(k_dequant<FMT_FP4_E8M0>, dim3(blocks), dim3(256), 0, st, m, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

/* ------------------------------------------------------- element rounding */

__device__ __forceinline__ uint32_t q_e4m3(float v)
{
    const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    if (__builtin_isnan(v)) return sign | 0x7Fu;
    const float a = fabsf(v);
    int code;
    if (a < 0x1p-6f) {
        code = (int)rintf(a * 512.0f);
    } else {
        int e2;
        (void)frexpf(a, &e2);
        const int E = e2 - 1;
        if (E > 8) return sign | 0x7Eu;
        const float frac = ldexpf(a, -E) - 1.0f;
        code = ((E + 7) << 3) + (int)rintf(frac * 8.0f);
    }
    if (code > 0x7E) code = 0x7E;
    return sign | (uint32_t)code;
}

__device__ __forceinline__ uint32_t q_e2m1(float v)
{
    const uint32_t sign = (__float_as_uint(v) >> 28) & 0x08u;
    if (__builtin_isnan(v)) return sign | 0x7u;
    const float a = fabsf(v);
    int code;
    if (a < 1.0f) {
        code = (int)rintf(a * 2.0f);
    } else {
        int e2;
        (void)frexpf(a, &e2);
        const int E = e2 - 1;
        if (E > 2) return sign | 0x7u;
        const float frac = ldexpf(a, -E) - 1.0f;
        code = ((E + 1) << 1) + (int)rintf(frac * 2.0f);
    }
    if (code > 7) code = 7;
    return sign | (uint32_t)code;
}


/* ---------------------------------------------------- FP4 weight quant --- */

/* one thread per 1x32 block */
__global__ __launch_bounds__(256) void k_quant_fp4_mx(uint8_t *W, uint8_t *S,
                                                     const float *w, int rows, int cols)
{
    const int nb = cols / 32;
    const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (long)rows * nb) return;
    const float *src = w + (size_t)id * 32;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        const f32x4 q = *(const f32x4 *)(src + i);
        v[i] = q.x; v[i + 1] = q.y; v[i + 2] = q.z; v[i + 3] = q.w;
    }
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fabsf(v[i]) > amax ? fabsf(v[i]) : amax;
    const uint32_t sb = amax > 0.0f ? e8m0_clamp(pow2_ceil_ratio(amax, 0.75f, 3)) : 127u;
    const int e = (int)sb - 127;
    S[id] = (uint8_t)sb;
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t lo = q_e2m1(ldexpf(v[8 * d + 2 * b], -e));
            const uint32_t hi = q_e2m1(ldexpf(v[8 * d + 2 * b + 1], -e));
            word |= (lo | (hi << 4)) << (8 * b);
        }
        out[d] = word;
    }
    *(u32x4 *)(W + (size_t)id * 16) = out;
}

hipError_t quant_fp4_mx_launch(uint8_t *W, uint8_t *S, const float *w, int rows,
                               int cols, hipStream_t st)
{
    const long n = (long)rows * (cols / 32);
    hipLaunchKernelGGL(k_quant_fp4_mx, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       W, S, w, rows, cols);
    return hipGetLastError();
}

/* ------------------------------------------ FP8 weight quant, fp32 128x128 */

/* one workgroup (256 threads) per 128x128 block */
__global__ __launch_bounds__(256) void k_quant_fp8_blk128(uint8_t *W, float *S,
                                                         const float *w, int rows, int cols)
{
    __shared__ float red[256];
    const int ncb = (cols + 127) / 128;
    const int rb = blockIdx.x / ncb, cb = blockIdx.x % ncb;
    const int r0 = rb * 128, c0 = cb * 128;
    float amax = 0.0f;
    for (int i = threadIdx.x; i < 128 * 128; i += 256) {
        const int r = r0 + i / 128, c = c0 + i % 128;
        if (r < rows && c < cols) {
            const float a = fabsf(w[(size_t)r * cols + c]);
            amax = a > amax ? a : amax;
        }
    }
    red[threadIdx.x] = amax;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float o = red[threadIdx.x + s];
            red[threadIdx.x] = o > red[threadIdx.x] ? o : red[threadIdx.x];
        }
        __syncthreads();
    }
    amax = red[0];
    const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (threadIdx.x == 0) S[(size_t)rb * ncb + cb] = sc;
    for (int i = threadIdx.x; i < 128 * 128; i += 256) {
        const int r = r0 + i / 128, c = c0 + i % 128;
        if (r < rows && c < cols)
            W[(size_t)r * cols + c] = (uint8_t)q_e4m3(w[(size_t)r * cols + c] / sc);
    }
}

hipError_t quant_fp8_blk128_launch(uint8_t *W, float *S, const float *w,
                                   int rows, int cols, hipStream_t st)
{
    const int nblk = ((rows + 127) / 128) * ((cols + 127) / 128);
    hipLaunchKernelGGL(k_quant_fp8_blk128, dim3(nblk), dim3(256), 0, st, W, S, w, rows, cols);
    return hipGetLastError();
}

/* --------------------------------------------- activation quantizers ---- */

/* e4m3(v / s) with v / s correctly rounded (the oracle's rule), without a
 * division in almost every case: q0 = v * (1 / s) lies within 3 * 2^-24 of
 * v / s relative, so the correctly rounded quotient lies between
 * q0 (1 - 2^-21) and q0 (1 + 2^-21); when both ends convert to the same code
 * (the convert rounds to nearest even, monotonically, below 464), so does
 * the quotient. Otherwise -- near a rounding boundary, about 1e-5 of
 * Gaussian inputs, or |q0| >= 448, NaN, infinities -- the division. */
__device__ __forceinline__ uint32_t e4m3_quot(float v, float s, float rs)
{
    const float q0 = v * rs;
    if (fabsf(q0) < 448.0f) {
        const float lo = q0 * (1.0f - 0x1p-21f), hi = q0 * (1.0f + 0x1p-21f);
        const uint32_t pk = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(lo, hi, 0, false);
        if ((pk & 0xFFu) == ((pk >> 8) & 0xFFu)) return pk & 0xFFu;
    }
    return hw_e4m3(v / s);
}

/* v of the lane DPP control CTRL names (every lane of the row active) */
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

/* e4m3_quot of eight elements, the bracketing test done with packed
 * converts: lo = v * RN(rs (1 - 2^-21)) and hi = v * RN(rs (1 + 2^-21))
 * still enclose v / s (the three roundings add at most 3 * 2^-24 relative to
 * a margin of 2^-21), so when the four packed codes of lo equal those of hi,
 * and every |lo| < 460 (finite, and hi below 464, where the convert is the
 * exact rounding), they are the codes of the quotients. Otherwise the lane
 * takes e4m3_quot element by element. */
__device__ __forceinline__ uint2 e4m3_quot8(const float (&v)[8], float s, float rs)
{
    const float rlo = rs * (1.0f - 0x1p-21f), rhi = rs * (1.0f + 0x1p-21f);
    float lo[8], hi[8];
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = v[i] * rlo;
        hi[i] = v[i] * rhi;
        ok = ok && fabsf(lo[i]) < 460.0f;
    }
    uint32_t l[2], h[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        l[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(lo[4 * j], lo[4 * j + 1], 0, false);
        l[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(lo[4 * j + 2], lo[4 * j + 3], (int)l[j], true);
        h[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(hi[4 * j], hi[4 * j + 1], 0, false);
        h[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(hi[4 * j + 2], hi[4 * j + 3], (int)h[j], true);
    }
    uint2 out;
    if (ok && l[0] == h[0] && l[1] == h[1]) {
        out.x = l[0];
        out.y = l[1];
        return out;
    }
    out.x = e4m3_quot(v[0], s, rs) | (e4m3_quot(v[1], s, rs) << 8) | (e4m3_quot(v[2], s, rs) << 16) |
            (e4m3_quot(v[3], s, rs) << 24);
    out.y = e4m3_quot(v[4], s, rs) | (e4m3_quot(v[5], s, rs) << 8) | (e4m3_quot(v[6], s, rs) << 16) |
            (e4m3_quot(v[7], s, rs) << 24);
    return out;
}

/* 16 lanes per 1x128 group, 8 consecutive elements per lane (one 16-byte
 * bf16 load or two fp32 loads, one 8-byte store); a 256-thread block covers
 * 16 groups. s = amax / 448 (1 if the group is all zero), q = e4m3(v / s)
 * with a correctly rounded division -- the oracle's rule (e4m3_quot). The
 * scale of token t, block b goes to S[t][b], or to S[b][t] (S_BLK_MAJOR: one
 * block's scales of consecutive tokens are contiguous, as the GEMM reads
 * them). */
template <bool S_BLK_MAJOR>
__device__ __forceinline__ void quant8_1x128(const float (&v)[8], uint8_t *Q, float *S, size_t e, bool live,
                                             int n, int k)
{
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) m = fmaxf(m, fabsf(v[i]));
    /* maximum over the 16 lanes of the group (one DPP row): quad swaps,
     * then the half-row and row mirrors, every step a VALU operation */
    m = fmaxf(m, dpp_f<DPP_QUAD_1032>(m));
    m = fmaxf(m, dpp_f<DPP_QUAD_2301>(m));
    m = fmaxf(m, dpp_f<DPP_ROW_HALF_MIRROR>(m));
    m = fmaxf(m, dpp_f<DPP_ROW_MIRROR>(m));
    const float sc = m > 0.0f ? m / 448.0f : 1.0f;
    if (!live) return;
    if ((threadIdx.x & 15) == 0) {
        /* group gi = e / 128 of token gi / (k / 128). The wave's four groups
         * are consecutive: the first active lane's group is split into token
         * and block once (a division of wave-uniform values, on the scalar
         * unit), and each lane steps from there (a per-lane division by a
         * runtime divisor is a long instruction sequence every lane runs:
         * 9.3 -> 8.8 us for 2048 x 4096 bf16 with the reciprocal below) */
        const uint32_t gi = (uint32_t)(e >> 7), kb = (uint32_t)k >> 7;
        if (S_BLK_MAJOR) {
            const uint32_t g0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)gi);
            uint32_t t = g0 / kb, b = g0 - t * kb + (gi - g0);
            while (b >= kb) {                          /* at most three steps */
                b -= kb;
                t++;
            }
            S[(size_t)b * (size_t)n + t] = sc;
        } else {
            S[gi] = sc;
        }
    }
    /* the hardware reciprocal (within 1 ulp): the bracketing tests allow
     * 2^-21 and fall back to the exact division */
    const float rs = __builtin_amdgcn_rcpf(sc);
    *(uint2 *)(Q + e) = e4m3_quot8(v, sc, rs);
}

/* Units per thread of the activation quantizers: a thread handles U units
 * of 256-thread blocks (a unit is what one thread of a one-unit grid would
 * do) and issues the loads of all of them before converting any. Measured
 * on the 2048 x 4096 bf16 input: the MXFP8 quantizer 13.2 -> 9.7 us with
 * four (and the packed converts), the 1x128 one 11.1 -> 13.7 us with four
 * and 9.2 -> 10.0 with two, so it keeps one (a grid of eight workgroups per
 * CU walking the units, each thread loading its next unit ahead: 10.5). */
constexpr int QA_U_1X128 = 1, QA_U_MX = 4;

template <bool BF16_IN, bool S_BLK_MAJOR>
__global__ __launch_bounds__(256) void k_quant_act_fp8_1x128(uint8_t *Q, float *S,
                                                            const void *a, int n, int k)
{
    const size_t total = (size_t)n * k;
    size_t e[QA_U_1X128];
    bool live[QA_U_1X128];
    float v[QA_U_1X128][8];
#pragma unroll
    for (int u = 0; u < QA_U_1X128; u++) {
        const size_t e0 = (((size_t)blockIdx.x * QA_U_1X128 + u) * 256 + threadIdx.x) * 8;
        live[u] = e0 < total;
        e[u] = live[u] ? e0 : 0;
        if constexpr (BF16_IN) {
            const u32x4 w = *(const u32x4 *)((const uint16_t *)a + e[u]);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[u][2 * i] = __uint_as_float(ws[i] << 16);
                v[u][2 * i + 1] = __uint_as_float(ws[i] & 0xFFFF0000u);
            }
        } else {
            const f32x4 x0 = *(const f32x4 *)((const float *)a + e[u]);
            const f32x4 x1 = *(const f32x4 *)((const float *)a + e[u] + 4);
            v[u][0] = x0.x; v[u][1] = x0.y; v[u][2] = x0.z; v[u][3] = x0.w;
            v[u][4] = x1.x; v[u][5] = x1.y; v[u][6] = x1.z; v[u][7] = x1.w;
        }
    }
#pragma unroll
    for (int u = 0; u < QA_U_1X128; u++) quant8_1x128<S_BLK_MAJOR>(v[u], Q, S, e[u], live[u], n, k);
}

/* mid = SwiGLU(gate, up) (the reference's clamp, dev_swiglu) of [n][k] fp32
 * rows, quantized by the rule above with block-major scales: the shared
 * expert's mid on its way into the down GEMM. */
__global__ __launch_bounds__(256) void k_swiglu_quant_fp8_1x128(uint8_t *Q, float *S, const float *g,
                                                               const float *u, int n, int k, float limit)
{
    const size_t e0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
    const bool live = e0 < (size_t)n * k;
    const size_t e = live ? e0 : 0;
    const f32x4 g0 = *(const f32x4 *)(g + e), g1 = *(const f32x4 *)(g + e + 4);
    const f32x4 u0 = *(const f32x4 *)(u + e), u1 = *(const f32x4 *)(u + e + 4);
    float v[8];
    v[0] = dev_swiglu(g0.x, u0.x, limit); v[1] = dev_swiglu(g0.y, u0.y, limit);
    v[2] = dev_swiglu(g0.z, u0.z, limit); v[3] = dev_swiglu(g0.w, u0.w, limit);
    v[4] = dev_swiglu(g1.x, u1.x, limit); v[5] = dev_swiglu(g1.y, u1.y, limit);
    v[6] = dev_swiglu(g1.z, u1.z, limit); v[7] = dev_swiglu(g1.w, u1.w, limit);
    quant8_1x128<true>(v, Q, S, e, live, n, k);
}

hipError_t swiglu_quant_fp8_launch(uint8_t *Q, float *S, const float *gate, const float *up, int n, int k,
                                   float limit, hipStream_t st)
{
    if (k % 128 || ((size_t)n * k >> 39)) return hipErrorInvalidValue;   /* 32-bit group indices */
    const size_t lanes = (size_t)n * k / 8;
    hipLaunchKernelGGL(k_swiglu_quant_fp8_1x128, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, st,
                       Q, S, gate, up, n, k, limit);
    return hipGetLastError();
}

hipError_t quant_act_fp8_1x128_launch(uint8_t *Q, float *S, const void *a,
                                      int n, int k, bool bf16_in, bool s_blk_major,
                                      hipStream_t st)
{
    if (k % 128 || ((size_t)n * k >> 39)) return hipErrorInvalidValue;   /* 32-bit group indices */
    const size_t units = ((size_t)n * k / 8 + 255) / 256;
    const dim3 grid((unsigned)((units + QA_U_1X128 - 1) / QA_U_1X128)), block(256);
    if (bf16_in && s_blk_major)
        hipLaunchKernelGGL((k_quant_act_fp8_1x128<true, true>), grid, block, 0, st, Q, S, a, n, k);
    else if (bf16_in)
        hipLaunchKernelGGL((k_quant_act_fp8_1x128<true, false>), grid, block, 0, st, Q, S, a, n, k);
    else if (s_blk_major)
        hipLaunchKernelGGL((k_quant_act_fp8_1x128<false, true>), grid, block, 0, st, Q, S, a, n, k);
    else
        hipLaunchKernelGGL((k_quant_act_fp8_1x128<false, false>), grid, block, 0, st, Q, S, a, n, k);
    return hipGetLastError();
}

/* one unit: the group g's four elements v of lane sub (of eight) */
__device__ __forceinline__ void quant4_mx(const float (&v)[4], long g, int sub, bool live, uint8_t *Q,
                                          uint8_t *S, long s_at)
{
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fabsf(v[i]) > amax ? fabsf(v[i]) : amax;
    /* group maximum over the eight lanes (NaN never wins a > compare): quad
     * swaps and the half-row mirror, DPP operations */
    {
        float o = dpp_f<DPP_QUAD_1032>(amax);
        amax = o > amax ? o : amax;
        o = dpp_f<DPP_QUAD_2301>(amax);
        amax = o > amax ? o : amax;
        o = dpp_f<DPP_ROW_HALF_MIRROR>(amax);
        amax = o > amax ? o : amax;
    }
    if (!live) return;
    const uint32_t sb = mxfp8_scale_byte(amax);
    const int e = (int)sb - 127;
    if (sub == 0) S[s_at] = (uint8_t)sb;
    /* the hardware convert is the exact rounding below 464 (and NaN is
     * mapped explicitly); an infinity takes the software rounding */
    float x[4];
    bool fin = true;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        x[b] = ldexpf(v[b], -e);
        fin = fin && !(fabsf(x[b]) >= 464.0f);
    }
    uint32_t word = 0;
    if (fin) {
#pragma unroll
        for (int b = 0; b < 4; b++) word |= hw_e4m3(x[b]) << (8 * b);
    } else {
#pragma unroll
        for (int b = 0; b < 4; b++) word |= q_e4m3(x[b]) << (8 * b);
    }
    *(uint32_t *)(Q + (size_t)g * 32 + 4 * sub) = word;
}

/* eight lanes per 1x32 group (four elements each), so a wave reads one
 * contiguous run of eight groups; fp32 or bf16 (widened exactly) input.
 * Scale byte of token m, 32-group j: S[m (k / 32) + j] token-major, or
 * S[4 (kb n + m) + j % 4] with kb = j / 4 block-major (one dword per token
 * and 128-wide K block, the K block's tokens contiguous). */
template <bool BF16_IN, bool BLK>
__global__ __launch_bounds__(256) void k_quant_act_mxfp8(uint8_t *Q, uint8_t *S,
                                                        const void *a, int n, int k)
{
    const long groups = (long)n * (k / 32);
    long g[QA_U_MX];
    bool live[QA_U_MX];
    float v[QA_U_MX][4];
#pragma unroll
    for (int u = 0; u < QA_U_MX; u++) {
        const long lid = ((long)blockIdx.x * QA_U_MX + u) * 256 + threadIdx.x;
        g[u] = lid >> 3;
        live[u] = g[u] < groups;
        const size_t off = live[u] ? (size_t)g[u] * 32 + 4 * (lid & 7) : 0;
        if constexpr (BF16_IN) {
            const uint2 q = *(const uint2 *)((const uint16_t *)a + off);
            v[u][0] = __uint_as_float(q.x << 16);
            v[u][1] = __uint_as_float(q.x & 0xFFFF0000u);
            v[u][2] = __uint_as_float(q.y << 16);
            v[u][3] = __uint_as_float(q.y & 0xFFFF0000u);
        } else {
            const f32x4 q = *(const f32x4 *)((const float *)a + off);
            v[u][0] = q.x; v[u][1] = q.y; v[u][2] = q.z; v[u][3] = q.w;
        }
        if (!live[u]) v[u][0] = v[u][1] = v[u][2] = v[u][3] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < QA_U_MX; u++) {
        long at = g[u];
        if constexpr (BLK) {
            /* token m and 32-group j of group g: the wave's eight groups are
             * consecutive, so the first lane's group is split once (a division
             * of wave-uniform values, on the scalar unit) and each lane steps
             * from there; k / 32 >= 4 here, so at most two steps */
            const long gpt = k / 32;
            const long g0 = ((long)__builtin_amdgcn_readfirstlane((int)(g[u] >> 32)) << 32) |
                            (uint32_t)__builtin_amdgcn_readfirstlane((int)g[u]);
            long m = g0 / gpt, j = g0 - m * gpt + (g[u] - g0);
            while (j >= gpt) {
                j -= gpt;
                m++;
            }
            at = 4 * ((j >> 2) * (long)n + m) + (j & 3);
        }
        quant4_mx(v[u], g[u], (int)(threadIdx.x & 7), live[u], Q, S, at);
    }
}

hipError_t quant_act_mxfp8_launch(uint8_t *Q, uint8_t *S, const void *a,
                                  int n, int k, hipStream_t st, bool bf16_in, bool s_blk_major)
{
    if (s_blk_major && k % 128) return hipErrorInvalidValue;
    const long units = ((long)n * (k / 32) * 8 + 255) / 256;
    const dim3 grid((unsigned)((units + QA_U_MX - 1) / QA_U_MX)), block(256);
    if (s_blk_major) {
        if (bf16_in)
            hipLaunchKernelGGL((k_quant_act_mxfp8<true, true>), grid, block, 0, st, Q, S, a, n, k);
        else
            hipLaunchKernelGGL((k_quant_act_mxfp8<false, true>), grid, block, 0, st, Q, S, a, n, k);
    } else if (bf16_in) {
        hipLaunchKernelGGL((k_quant_act_mxfp8<true, false>), grid, block, 0, st, Q, S, a, n, k);
    } else {
        hipLaunchKernelGGL((k_quant_act_mxfp8<false, false>), grid, block, 0, st, Q, S, a, n, k);
    }
    return hipGetLastError();
}

/* -------------------------------------------------------------- synth --- */

__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in (0, 1): 53 random bits + half an ulp */
__device__ __forceinline__ double unif(uint64_t key, uint64_t ctr)
{
    return ((double)(mix64(key ^ mix64(ctr)) >> 11) + 0.5) * 0x1p-53;
}

__global__ __launch_bounds__(256) void k_synth_normal(float *out, size_t n, uint64_t seed,
                                                     float sigma, int round_bf16)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t key = mix64(seed);
    const double u1 = unif(key, 2 * (uint64_t)i), u2 = unif(key, 2 * (uint64_t)i + 1);
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    float v = (float)(z * (double)sigma);
    if (round_bf16) {
        const uint32_t u = __float_as_uint(v);
        v = __uint_as_float(((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16) << 16);
    }
    out[i] = v;
}

hipError_t synth_normal_launch(float *out, size_t n, uint64_t seed, float sigma,
                               int round_bf16, hipStream_t st)
{
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_synth_normal, dim3((unsigned)blocks), dim3(256), 0, st,
                       out, n, seed, sigma, round_bf16);
    return hipGetLastError();
}

} // namespace dsv4
