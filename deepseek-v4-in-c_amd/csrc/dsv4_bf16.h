/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_bf16.h - the BF16 row dot product of bf16_n on the GPU, shared by the
 * BF16 matvec (dsv4_gemv.hip) and the fused gate + router (dsv4_route.hip). */
#ifndef DSV4_BF16_H
#define DSV4_BF16_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsv4 {

/* Replaces bf16_n (src/10_compute/dsv4_matmul.c:88-113) bit for bit. Its row
 * dot product (BLOCK_DOT_V, src/10_compute/dsv4_dec_common.h:45-61) runs 16
 * fp64 FMA chains over the n - n % 16 leading columns, chain c taking columns
 * c, c + 16, c + 32, ... in increasing order from +0; then
 *   bb[j] = (chain j + chain 4 + j) + (chain 8 + j + chain 12 + j),
 *   acc = (bb[0] + bb[1]) + (bb[2] + bb[3]),
 * the n % 16 trailing columns are added to acc one FMA each, and y = (float)
 * acc. Every product of a bf16 weight and an fp32 activation is exact in
 * fp64 and an fp64 FMA is correctly rounded on both sides, so the same order
 * gives the same bits. Lane 16 r + c of a wave runs chain c of the wave's
 * row r. */
__device__ __forceinline__ double bf16_of(uint16_t h) { return (double)__uint_as_float((uint32_t)h << 16); }

/* chain c over `steps` steps: weights and activations from LDS, the next
 * eight steps' reads issued before this eight's FMAs (a dependent fp64 FMA
 * chain; the reads' latency hides behind it) */
__device__ __forceinline__ double bf16_chain(const uint16_t *wl, const float *xl, int steps, int c)
{
    double acc = 0.0;
    const int full = steps & ~7;
    uint16_t w[8];
    float xv[8];
    if (full) {
#pragma unroll
        for (int i = 0; i < 8; i++) { w[i] = wl[16 * i + c]; xv[i] = xl[16 * i + c]; }
    }
    for (int s = 0; s < full; s += 8) {
        uint16_t wn[8];
        float xn[8];
        const int sn = s + 8 < full ? s + 8 : s;        /* the last round re-reads its own */
#pragma unroll
        for (int i = 0; i < 8; i++) { wn[i] = wl[16 * (sn + i) + c]; xn[i] = xl[16 * (sn + i) + c]; }
#pragma unroll
        for (int i = 0; i < 8; i++) acc = fma(bf16_of(w[i]), (double)xv[i], acc);
#pragma unroll
        for (int i = 0; i < 8; i++) { w[i] = wn[i]; xv[i] = xn[i]; }
    }
    for (int s = full; s < steps; s++) acc = fma(bf16_of(wl[16 * s + c]), (double)xl[16 * s + c], acc);
    return acc;
}

/* The 16 chains of a lane group combined in the reference's order; lane 0 of
 * the group receives acc (before the trailing columns). */
__device__ __forceinline__ double bf16_combine16(double v)
{
    v = v + __shfl_down(v, 4, 16);       /* c < 12: chain c + chain c + 4       */
    v = v + __shfl_down(v, 8, 16);       /* c < 4: bb[c]                        */
    v = v + __shfl_down(v, 1, 16);       /* c = 0, 2: bb[0] + bb[1], bb[2] + bb[3] */
    v = v + __shfl_down(v, 2, 16);       /* c = 0: acc                          */
    return v;
}

/* The whole dot product of one row (wl) with x (xl, fp32), both in LDS, for
 * lane group (row) lane / 16: returns the fp64 acc in lane 16 (lane / 16),
 * the trailing columns included. */
__device__ __forceinline__ double bf16_row_dot(const uint16_t *wl, const float *xl, int cols, int lane)
{
    const int c = lane & 15, steps = cols / 16;
    double acc = bf16_combine16(bf16_chain(wl, xl, steps, c));
    if (c == 0)
        for (int e = 16 * steps; e < cols; e++) acc = fma(bf16_of(wl[e]), (double)xl[e], acc);
    return acc;
}

typedef __attribute__((address_space(3))) void bf_lds_t;

/* Copy `rows` consecutive BF16 rows (row_bytes each, the last row repeated
 * past rows_left) into LDS, stride bytes apart, 1 KiB per instruction; bytes
 * of a row past row_bytes read as zero. The caller waits (vmcnt). */
template <int KCH>
__device__ __forceinline__ void bf16_rows_to_lds(uint8_t *lds, int stride, const uint16_t *W, int row0,
                                                 int rows, int rows_left, int row_bytes, int lane)
{
    for (int r = 0; r < rows; r++) {
        const int row = row0 + min(r, rows_left - 1);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)((const uint8_t *)W + (size_t)row * row_bytes), (short)0, row_bytes, 0x00020000);
#pragma unroll
        for (int k = 0; k < KCH; k++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (bf_lds_t *)(lds + r * stride + 1024 * k), 16,
                                                     1024 * k + 16 * lane, 0, 0, 0);
    }
}

/* x (cols fp32 values) into LDS at xl, 1 KiB per instruction, bytes past
 * cols read as zero; xl_bytes = bf16_x_lds_bytes(cols). The caller waits. */
__host__ __device__ constexpr int bf16_x_lds_bytes(int cols) { return (cols * 4 + 1023) / 1024 * 1024; }

__device__ __forceinline__ void bf16_x_to_lds(uint8_t *xl, const float *x, int cols, int lane)
{
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, cols * 4, 0x00020000);
    for (int k = 0; k < bf16_x_lds_bytes(cols) / 1024; k++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (bf_lds_t *)(xl + 1024 * k), 16, 1024 * k + 16 * lane, 0, 0, 0);
}

} // namespace dsv4

#endif /* DSV4_BF16_H */
