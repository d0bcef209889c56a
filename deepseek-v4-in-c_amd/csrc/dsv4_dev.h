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

/* Pointers read from device memory (descriptor tables) are generic to the
 * compiler, and generic (flat) loads are waited for all at once. Every weight
 * and scale access goes through a global-address-space pointer so loads
 * complete in issue order and are waited for one by one. */
#define DSV4_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const DSV4_GLOBAL T *gptr(const T *p)
{
    return (const DSV4_GLOBAL T *)p;
}

/* Wave-uniform reads (routing ids, descriptor tables) go through the
 * constant address space so they become scalar loads into SGPRs; the data
 * must not be written while the kernel runs. */
#define DSV4_CONST __attribute__((address_space(4)))
template <class T>
__device__ __forceinline__ T ld_uniform(const T *base, int i)
{
    static_assert(sizeof(T) % 4 == 0, "uniform reads move whole dwords");
    const DSV4_CONST uint32_t *p = (const DSV4_CONST uint32_t *)(base + i);
    T r;
    uint32_t *q = (uint32_t *)&r;
#pragma unroll
    for (unsigned k = 0; k < sizeof(T) / 4; k++) q[k] = p[k];
    return r;
}

/* The index of the calling wave in the grid, provably wave-uniform. */
__device__ __forceinline__ int wave_id()
{
    return __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)));
}

/* The index of the calling wave within its workgroup, provably wave-uniform. */
__device__ __forceinline__ int wave_in_group()
{
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

/* Weight chunk loads, marked non-temporal: each weight byte is read exactly
 * once per call. */
__device__ __forceinline__ u32x4 ld_stream16(const void *p)
{
    return __builtin_nontemporal_load(gptr((const u32x4 *)p));
}

/* One scale: an E8M0 byte or an fp32. */
__device__ __forceinline__ uint32_t ld_u8(const void *base, size_t i)
{
    return gptr((const uint8_t *)base)[i];
}
__device__ __forceinline__ float ld_f32(const void *base, size_t i)
{
    return gptr((const float *)base)[i];
}

/* Keep the compiler from moving instructions across this point: the decode
 * kernels use it to pin the issue order of their load groups. */
#define DSV4_ORDER() __builtin_amdgcn_sched_barrier(0)

/* A uniform `true` the compiler cannot see through. Arithmetic placed under
 * `if (dsv4_opaque_true())` lands in its own basic block, so instruction
 * selection cannot hoist it (e.g. a scale-byte decode) in between loads that
 * must all be issued before the wave waits for the first of them. */
__device__ __forceinline__ bool dsv4_opaque_true()
{
    int v;
    asm volatile("s_mov_b32 %0, 1" : "=s"(v));
    return v != 0;
}

/* Chunk geometry of the decode kernels: lane `lane` reads the 16 weight bytes
 * at row byte offset 16 * lane + 1024 * j (j < KCH). A row is FULL when
 * row_bytes == KCH * 1024, i.e. every lane's every chunk is inside the row;
 * otherwise chunks past row_bytes are "out". Loads are never skipped, so no
 * load sits behind a branch: an out chunk loads the row's first chunk
 * instead, its activations read as zero and its scale as zero, so it adds an
 * exact zero (or the NaN that the row's first chunk already contributes). */
__device__ __forceinline__ int chunk_byte(int lane, int j) { return 16 * lane + 1024 * j; }

/* The lane's slice of an fp32 activation row: chunk j covers CPL columns
 * starting at (FP4 ? 2 : 1) * chunk_byte(lane, j); an out chunk reads the
 * row's first CPL columns (its scale is zero). x must be 16-byte aligned and
 * hold at least 32 (FP4) or 16 (FP8) columns. No arithmetic touches the
 * loaded values here, so issuing these loads never waits for them. */
template <bool FP4, int KCH, bool FULL>
__device__ __forceinline__ void load_x_slice(float (&xs)[KCH][FP4 ? 32 : 16],
                                             const float *x, int lane,
                                             int row_bytes)
{
    constexpr int CPL = FP4 ? 32 : 16;
#pragma unroll
    for (int j = 0; j < KCH; j++) {
        const int b = chunk_byte(lane, j);
        const bool in = FULL || b < row_bytes;
        const float *p = x + (in ? (FP4 ? 2 * b : b) : 0);
#pragma unroll
        for (int i = 0; i < CPL; i += 4) {
            const f32x4 v = *(const f32x4 *)(p + i);
            xs[j][i] = v.x; xs[j][i + 1] = v.y; xs[j][i + 2] = v.z; xs[j][i + 3] = v.w;
        }
    }
}

/* Raw scale words: the E8M0 byte or the fp32 bits of one block scale. They
 * are loaded with the other early loads and decoded only at first use, so
 * the weight loads behind them are issued without waiting. */
template <bool F32S>
__device__ __forceinline__ uint32_t ld_scale_raw(const void *S, size_t idx)
{
    if constexpr (F32S) return gptr((const uint32_t *)S)[idx];
    else return gptr((const uint8_t *)S)[idx];
}
template <bool F32S>
__device__ __forceinline__ float scale_from_raw(uint32_t raw)
{
    if constexpr (F32S) return __uint_as_float(raw);
    else return dev_e8m0(raw);
}

/* The lane's KCH weight chunks of one row (row start `wr`). */
template <int KCH, bool FULL>
__device__ __forceinline__ void load_w_row(u32x4 (&w)[KCH], const uint8_t *wr,
                                           int lane, int row_bytes)
{
#pragma unroll
    for (int j = 0; j < KCH; j++) {
        const int b = chunk_byte(lane, j);
        const bool in = FULL || b < row_bytes;
        w[j] = ld_stream16(wr + (in ? b : 0));
    }
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
#define DPP_ROW_ROR8 0x128   /* row_ror:8, lane i of a row of 16 reads lane i ^ 8 */

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

/* ------------------------------------------------ MX scale rounding ---- */

/* least e with (frac_lim * 2^exp_lim) * 2^e >= amax, amax > 0 (448 = 0.875 *
 * 2^9 for e4m3, 6 = 0.75 * 2^3 for e2m1) */
__device__ __forceinline__ int pow2_ceil_ratio(float amax, float frac_lim, int exp_lim)
{
    int e2;
    const float f = frexpf(amax, &e2);
    return (f <= frac_lim) ? e2 - exp_lim : e2 - exp_lim + 1;
}

__device__ __forceinline__ uint32_t e8m0_clamp(int e)
{
    int b = 127 + e;
    b = b < 0 ? 0 : (b > 254 ? 254 : b);
    return (uint32_t)b;
}

/* f32 -> e4m3 by the hardware convert (OCP e4m3fn, round to nearest even).
 * Checked against the software rounding (q_e4m3) over every fp32 bit pattern
 * on gfx950: identical for |v| < 464, which covers every quotient a MX or
 * 1x128 quantizer forms (at most 448 (1 + 2^-22)); NaN is mapped explicitly
 * to the software rule's sign | 0x7F. */
__device__ __forceinline__ uint32_t hw_e4m3(float v)
{
    const uint32_t q = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xFFu;
    return __builtin_isnan(v) ? (((__float_as_uint(v) >> 24) & 0x80u) | 0x7Fu) : q;
}

/* E8M0 scale byte of an MXFP8 block whose largest magnitude is amax (NaN
 * ignored by the caller's max): least 2^e with 448 * 2^e >= amax, clamped to
 * [0, 254]; 127 for an all-zero block. */
__device__ __forceinline__ uint32_t mxfp8_scale_byte(float amax)
{
    return amax > 0.0f ? e8m0_clamp(pow2_ceil_ratio(amax, 0.875f, 9)) : 127u;
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
