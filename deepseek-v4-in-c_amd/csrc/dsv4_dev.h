/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_dev.h - gfx950 device helpers shared by every kernel: the exact
 * element decoders, wavefront reductions and the SwiGLU element.
 *
 * One decoder per format, used by the matmul kernels AND the dequant kernel,
 * so the dequantized-weight check exercises the very instructions the matmuls
 * run.
 *
 * Decoders (formats as the reference defines them, src/10_compute/dsv4_quant.h:72-158):
 *   e8m0  byte b -> 2^(b-127); 0 -> 2^-127 (the subnormal 0x00400000),
 *         255 -> NaN. Bit assembly, no table.
 *   e4m3  OCP e4m3fn (bias 7, no infinities, 0x7F/0xFF NaN, max 448) through
 *         v_cvt_scalef32_pk_f32_fp8: two codes per instruction, exact.
 *   e2m1  OCP e2m1 {0,.5,1,1.5,2,3,4,6} with sign, through
 *         v_cvt_scalef32_pk_f32_fp4: one byte (two nibbles, the LOW nibble is
 *         the even element) per instruction, exact.
 */
#ifndef DSV4_DEV_H
#define DSV4_DEV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define DSV4_WAVE 64

__device__ __forceinline__ float dev_e8m0(uint32_t b)
{
    const uint32_t u = (b == 255u) ? 0x7FC00000u
                     : (b == 0u)   ? 0x00400000u : (b << 23);
    return __uint_as_float(u);
}

/* e4m3 codes in bytes 0,1 (HI = false) or 2,3 (HI = true) of v; .x is the
 * lower-addressed byte. */
template <bool HI>
__device__ __forceinline__ f32x2 dev_e4m3x2(uint32_t v)
{
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(v, 1.0f, HI);
}

/* e2m1 nibbles of byte SEL of v; .x is the low nibble (even element). */
template <int SEL>
__device__ __forceinline__ f32x2 dev_e2m1x2(uint32_t v)
{
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, 1.0f, SEL);
}

/* Dot of one 16-byte weight chunk with the lane's matching x slice, decoding
 * one dword at a time so only eight decoded values are live. Two accumulators
 * for instruction-level parallelism, summed in a fixed order.
 *   FP4: 16 bytes = 32 e2m1 columns, xs[0..31]
 *   FP8: 16 bytes = 16 e4m3 columns, xs[0..15] */
__device__ __forceinline__ float dot16_e2m1(const u32x4 w, const float *xs)
{
    float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = dev_e2m1x2<0>(w[d]);
        const f32x2 b = dev_e2m1x2<1>(w[d]);
        const f32x2 c = dev_e2m1x2<2>(w[d]);
        const f32x2 e = dev_e2m1x2<3>(w[d]);
        p0 = fmaf(a.x, xs[8 * d + 0], p0); p1 = fmaf(a.y, xs[8 * d + 1], p1);
        p0 = fmaf(b.x, xs[8 * d + 2], p0); p1 = fmaf(b.y, xs[8 * d + 3], p1);
        p0 = fmaf(c.x, xs[8 * d + 4], p0); p1 = fmaf(c.y, xs[8 * d + 5], p1);
        p0 = fmaf(e.x, xs[8 * d + 6], p0); p1 = fmaf(e.y, xs[8 * d + 7], p1);
    }
    return p0 + p1;
}

__device__ __forceinline__ float dot16_e4m3(const u32x4 w, const float *xs)
{
    float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = dev_e4m3x2<false>(w[d]);
        const f32x2 b = dev_e4m3x2<true>(w[d]);
        p0 = fmaf(a.x, xs[4 * d + 0], p0); p1 = fmaf(a.y, xs[4 * d + 1], p1);
        p0 = fmaf(b.x, xs[4 * d + 2], p0); p1 = fmaf(b.y, xs[4 * d + 3], p1);
    }
    return p0 + p1;
}

/* Sixteen e4m3 codes (one 128-bit load) -> sixteen floats, element order. */
__device__ __forceinline__ void dev_dec16_e4m3(const u32x4 w, float f[16])
{
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = dev_e4m3x2<false>(w[d]);
        const f32x2 b = dev_e4m3x2<true>(w[d]);
        f[4 * d + 0] = a.x; f[4 * d + 1] = a.y;
        f[4 * d + 2] = b.x; f[4 * d + 3] = b.y;
    }
}

/* Sixteen packed bytes (one 128-bit load) -> thirty-two e2m1 floats. */
__device__ __forceinline__ void dev_dec32_e2m1(const u32x4 w, float f[32])
{
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = dev_e2m1x2<0>(w[d]);
        const f32x2 b = dev_e2m1x2<1>(w[d]);
        const f32x2 c = dev_e2m1x2<2>(w[d]);
        const f32x2 e = dev_e2m1x2<3>(w[d]);
        f[8 * d + 0] = a.x; f[8 * d + 1] = a.y;
        f[8 * d + 2] = b.x; f[8 * d + 3] = b.y;
        f[8 * d + 4] = c.x; f[8 * d + 5] = c.y;
        f[8 * d + 6] = e.x; f[8 * d + 7] = e.y;
    }
}

template <int FMT_IS_FP4>
__device__ __forceinline__ float dot16(const u32x4 w, const float *xs)
{
    if constexpr (FMT_IS_FP4) return dot16_e2m1(w, xs);
    else return dot16_e4m3(w, xs);
}

/* Global loads that bypass nothing but are marked non-temporal for streamed
 * weights: each weight byte is read exactly once per call. */
__device__ __forceinline__ u32x4 ld_stream16(const void *p)
{
    return __builtin_nontemporal_load((const u32x4 *)p);
}

__device__ __forceinline__ f32x4 ld_f4(const float *p)
{
    return *(const f32x4 *)p;
}

/* DPP lane moves (GFX9 encodings). */
#define DPP_QUAD_1032 0xB1   /* quad_perm [1,0,3,2] */
#define DPP_QUAD_2301 0x4E   /* quad_perm [2,3,0,1] */
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_BCAST15 0x142
#define DPP_ROW_BCAST31 0x143

#define DPP_ADD(v, CTRL, ROWMASK)                                              \
    (v) = (v) + __int_as_float(__builtin_amdgcn_update_dpp(                    \
              0, __float_as_int(v), (CTRL), (ROWMASK), 0xF, false))

/* Sum over the 64 lanes of a wavefront, in a fixed order (deterministic);
 * the result is returned uniformly to every lane. */
__device__ __forceinline__ float wave_sum(float v)
{
    DPP_ADD(v, DPP_QUAD_1032, 0xF);
    DPP_ADD(v, DPP_QUAD_2301, 0xF);
    DPP_ADD(v, DPP_ROW_HALF_MIRROR, 0xF);
    DPP_ADD(v, DPP_ROW_MIRROR, 0xF);
    DPP_ADD(v, DPP_ROW_BCAST15, 0xA);
    DPP_ADD(v, DPP_ROW_BCAST31, 0xC);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

/* The reference's SwiGLU element (src/10_compute/dsv4_ops.c:61-79): up is
 * clamped to [-limit, limit], gate only from above; limit <= 0 disables the
 * clamp; silu(g) = g / (1 + exp(-g)). Products and sums are explicitly
 * rounded so no contraction changes them. */
__device__ __forceinline__ float dev_swiglu(float g, float u, float limit)
{
    if (limit > 0.0f) {
        u = (u > limit) ? limit : u;
        u = (u < -limit) ? -limit : u;
        g = (g > limit) ? limit : g;      /* deliberately no lower bound */
    }
    const float s = g / __fadd_rn(1.0f, expf(-g));
    return __fmul_rn(s, u);
}

#endif /* DSV4_DEV_H */
