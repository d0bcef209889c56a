/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_moe_grouped.hip - MoE over many tokens at once: batched decode and
 * the prefill MoE layer.
 *
 * What it replaces, in the reference:
 *   - the permutation of (token, k) pairs by expert
 *     (src/80_prefill/dsv4_prefill_union.c:30-66),
 *   - the per-expert bucket: gather, w1 / w3 GEMMs, SwiGLU, w2 GEMM, scatter
 *     (src/80_prefill/dsv4_prefill_experts.c:23-77; its GPU leg, the fused
 *     Vulkan expert, src/80_prefill/dsv4_prefill_vk_expert.c:45-172),
 *   - the combine: per token, out = sum_k w_k * acc_k in k order, then the
 *     shared expert's output added unweighted
 *     (src/80_prefill/dsv4_prefill_union_run.c:109-121).
 * The CPU/GPU bucket scheduler (src/80_prefill/dsv4_prefill_union_sched.c)
 * has no counterpart: every bucket runs in one device-resident pass.
 *
 * PIPELINE (one stream, no host round trip)
 *   k_moe_route     counting sort by expert: first row of each expert's
 *                   bucket (grp_off), prefix of its token tiles (tile_pre),
 *                   each pair's row (pos) and each row's token (row_tok).
 *   k_to_f16        x -> fp16 (round to nearest even).
 *   k_grouped       one wave = one work item: an expert, a slab of output
 *                   features (64 for gate/up with both w1 and w3 rows, 128 for
 *                   down) and a tile of up to 16*TT of its rows. Item ids are
 *                   decoded on the device from tile_pre (binary search), so
 *                   the grid is an upper bound and surplus waves exit.
 *   k_moe_combine   out[t] = sum_k w[t][k] * Y[pos(t, k)] (k order) + shared[t].
 *
 * NUMERICS
 *   v_mfma_f32_16x16x32_f16, fp32 accumulation. Weights are decoded into the
 *   MFMA operand with v_cvt_scalef32_pk_f16_{fp4,fp8}: e2m1 * 2^e is exact in
 *   fp16 for E8M0 scale bytes 104..140 (checked on every block: outside it
 *   the status word gets ST_SCALE_RANGE); e4m3 values enter unscaled (exact)
 *   and the 128x128 block scale, E8M0 or fp32, multiplies each 128-K chunk's
 *   partial sum in fp32, as the reference's fp8_n applies it per block. The
 *   activations and
 *   the SwiGLU output enter the MFMA rounded to fp16 (relative error at most
 *   2^-11 each); everything else is fp32.
 *
 * MFMA OPERANDS (gfx950, measured): lane l supplies row l % 16 of A and of B
 *   with 8 consecutive reduction indices, lane group l / 16 selecting which 8;
 *   accumulator element e of lane l is row 4 (l / 16) + e, column l % 16.
 *   Weights are A (rows = output features), tokens are B. The reduction index
 *   may be permuted freely as long as A and B agree: each lane loads 16
 *   contiguous weight bytes per 128-K chunk (FP4: 32 values, one E8M0 block)
 *   and the B side is fetched in the same order (kmap).
 *
 * Bound: HBM (weights) for small buckets, MFMA for large ones.
 */
#include "dsv4_internal.h"

namespace dsv4 {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int KC = 128;           /* reduction chunk */
constexpr int RB = 8;             /* 16-row weight blocks per item */
constexpr int MAX_ROUTE_EXPERTS = 1024;

/* first reduction index (within a 128-K chunk) of MFMA step j for lane
 * group gq; FP4 lanes hold 32 contiguous values, FP8 lanes two runs of 16 */
template <int WF>
__device__ __forceinline__ int kmap(int gq, int j)
{
    if constexpr (WF == FMT_FP4_E8M0) return 32 * gq + 8 * j;
    else return 64 * (j >> 1) + 16 * gq + 8 * (j & 1);
}

__device__ __forceinline__ uint32_t pk_f16_fp4(uint32_t w, float sc, int sel)
{
    return __builtin_bit_cast(uint32_t, sel == 0 ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 0)
                                       : sel == 1 ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 1)
                                       : sel == 2 ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 2)
                                                  : __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 3));
}

template <bool HI>
__device__ __forceinline__ uint32_t pk_f16_fp8(uint32_t w, float sc)
{
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, sc, HI));
}

/* A operand of step j from one lane's raw weight bytes (whole-word bit casts
 * only: extracting one half of a packed convert result is not reliable) */
template <int WF>
__device__ __forceinline__ h8 a_operand(const u32x4 (&w)[2], float sc, int j)
{
    u32x4 v;
    if constexpr (WF == FMT_FP4_E8M0) {
        const uint32_t d = j == 0 ? w[0].x : j == 1 ? w[0].y : j == 2 ? w[0].z : w[0].w;
        v.x = pk_f16_fp4(d, sc, 0);
        v.y = pk_f16_fp4(d, sc, 1);
        v.z = pk_f16_fp4(d, sc, 2);
        v.w = pk_f16_fp4(d, sc, 3);
    } else {
        const u32x4 &h = w[j >> 1];
        const uint32_t d0 = (j & 1) ? h.z : h.x, d1 = (j & 1) ? h.w : h.y;
        v.x = pk_f16_fp8<false>(d0, sc);
        v.y = pk_f16_fp8<true>(d0, sc);
        v.z = pk_f16_fp8<false>(d1, sc);
        v.w = pk_f16_fp8<true>(d1, sc);
    }
    return __builtin_bit_cast(h8, v);
}

__device__ __forceinline__ f4v mfma16(const h8 &a, const h8 &b, const f4v &c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t f16_bits(float v)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

template <int WF>
__device__ __forceinline__ bool qmat_matches(const DSV4QMat &m, int rows, int cols)
{
    if (m.rows != rows || m.cols != cols || !m.w || !m.s) return false;
    if constexpr (WF == FMT_FP4_E8M0) return m.wdt == DSV4_WFP4 && m.blk_r == 1 && m.blk_c == 32;
    else if constexpr (WF == FMT_FP8_E8M0) return m.wdt == DSV4_WFP8 && m.blk_r == 128 && m.blk_c == 128;
    else return m.wdt == DSV4_WFP8_F32S && m.blk_r == 128 && m.blk_c == 128;
}

} // namespace

/* ------------------------------------------------------------ routing --- */

__global__ __launch_bounds__(1024) void k_moe_route(RouteArgs a)
{
    __shared__ int hist[MAX_ROUTE_EXPERTS];
    __shared__ int cur[MAX_ROUTE_EXPERTS];
    const int tid = threadIdx.x;
    const int E = a.n_experts;
    for (int e = tid; e < E; e += 1024) hist[e] = 0;
    __syncthreads();
    unsigned bad = 0;
    for (int p = tid; p < a.npairs; p += 1024) {
        const int e = a.idx[p];
        if ((unsigned)e < (unsigned)E) atomicAdd(&hist[e], 1);
        else bad = ST_BAD_EXPERT_ID;
    }
    __syncthreads();
    if (tid == 0) {
        int o = 0, tp = 0;
        for (int e = 0; e < E; e++) {
            a.grp_off[e] = o;
            a.tile_pre[e] = tp;
            cur[e] = o;
            o += hist[e];
            tp += (hist[e] + a.tile_rows - 1) / a.tile_rows;
        }
        a.grp_off[E] = o;
        a.tile_pre[E] = tp;
    }
    __syncthreads();
    /* rows inside a bucket are claimed by LDS atomics; a row's result does
     * not depend on its slot, so the order within a bucket does not matter */
    for (int p = tid; p < a.npairs; p += 1024) {
        const int e = a.idx[p];
        if ((unsigned)e < (unsigned)E) {
            const int r = atomicAdd(&cur[e], 1);
            a.pos[p] = r;
            a.row_tok[r] = p / a.topk;
        } else {
            a.pos[p] = -1;
        }
    }
    if (bad) atomicOr(a.status, bad);
}

/* 8 floats -> 8 fp16 per thread */
__global__ __launch_bounds__(256) void k_to_f16(uint16_t *o, const float *x, size_t n8)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const f32x4 a = *(const f32x4 *)(x + 8 * i);
    const f32x4 b = *(const f32x4 *)(x + 8 * i + 4);
    u32x4 v;
    v.x = f16_bits(a.x) | (f16_bits(a.y) << 16);
    v.y = f16_bits(a.z) | (f16_bits(a.w) << 16);
    v.z = f16_bits(b.x) | (f16_bits(b.y) << 16);
    v.w = f16_bits(b.z) | (f16_bits(b.w) << 16);
    *(u32x4 *)(o + 8 * i) = v;
}

/* --------------------------------------------------------- grouped GEMM --- */

template <int WF, bool SWIGLU, int TT>
__global__ __launch_bounds__(256) void k_grouped(GroupedArgs a)
{
    constexpr int FEAT = SWIGLU ? 64 : 128;       /* output features per item */
    constexpr int TROWS = 16 * TT;                /* rows per tile           */
    constexpr bool FP4 = WF == FMT_FP4_E8M0;
    const int lane = threadIdx.x & 63;
    const int rr = lane & 15, gq = lane >> 4;
    const int item = blockIdx.x * 4 + wave_in_group();
    const int nslab = a.N / FEAT;
    const int tile = item / nslab, slab = item - tile * nslab;

    int r0, ntok;
    DSV4QMat m1, m3;
    if (a.table) {
        const int E = a.n_experts;
        if (tile >= ld_uniform(a.tile_pre, E)) return;
        int lo = 0, hi = E;    /* largest g with tile_pre[g] <= tile: a non-empty bucket */
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (ld_uniform(a.tile_pre, mid) <= tile) lo = mid;
            else hi = mid;
        }
        const int grp = lo;
        const int go = ld_uniform(a.grp_off, grp), ge = ld_uniform(a.grp_off, grp + 1);
        r0 = go + (tile - ld_uniform(a.tile_pre, grp)) * TROWS;
        ntok = min(TROWS, ge - r0);
        const DSV4ExpertW e = ld_uniform(a.table, grp);
        m1 = SWIGLU ? e.w1 : e.w2;
        m3 = e.w3;
    } else {
        r0 = tile * TROWS;
        if (r0 >= a.nrows) return;
        ntok = min(TROWS, a.nrows - r0);
        m1 = a.m1;
        m3 = a.m3;
    }
    const int ntt = (ntok + 15) >> 4;              /* live 16-row tiles */
    const int f0 = slab * FEAT;
    const int K = a.K, N = a.N;

    if (!qmat_matches<WF>(m1, N, K) || (SWIGLU && !qmat_matches<WF>(m3, N, K))) {
        if (lane == 0) atomicOr(a.status, ST_BAD_DESCRIPTOR);
        const float nan = __builtin_nanf("");
        for (int t = 0; t < ntok; t++)
            for (int f = lane; f < FEAT; f += 64) {
                const size_t o = (size_t)(r0 + t) * N + f0 + f;
                if constexpr (SWIGLU) ((uint16_t *)a.out)[o] = (uint16_t)f16_bits(nan);
                else ((float *)a.out)[o] = nan;
            }
        return;
    }

    /* this lane's weight rows: SwiGLU items take w1 rows in blocks 0-3 and
     * the matching w3 rows in blocks 4-7 */
    const int rowb = FP4 ? K / 2 : K;              /* bytes per weight row */
    const uint8_t *wrow[RB];
    const uint8_t *srow[RB];                       /* FP4: the row's E8M0 bytes */
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const bool up = SWIGLU && rb >= 4;
        const DSV4QMat &m = up ? m3 : m1;
        const int row = f0 + 16 * (SWIGLU ? (rb & 3) : rb) + rr;
        wrow[rb] = (const uint8_t *)m.w + (size_t)row * rowb + 16 * gq;
        srow[rb] = (const uint8_t *)m.s + (size_t)row * (K / 32);
    }
    /* FP8: one scale per (128-row block, 128-K chunk) per matrix */
    const int nb = f0 / 128, kbn = K / 128;

    /* this lane's B rows (tokens); rows past the tile's end repeat row r0 */
    const uint16_t *brow[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int t = 16 * tt + rr;
        const int r = t < ntok ? r0 + t : r0;
        const int src = a.row_tok ? a.row_tok[r] : r;
        brow[tt] = a.B + (size_t)src * K;
    }

    f4v acc[RB][TT];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) acc[rb][tt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

    unsigned scale_bad = 0;
    const int nchunk = K / KC;
    /* raw weights of the next chunk are in flight while this one multiplies */
    u32x4 wn[RB][2];
    uint32_t sn[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        wn[rb][0] = ld_stream16(wrow[rb]);
        wn[rb][1] = FP4 ? wn[rb][0] : ld_stream16(wrow[rb] + 64);
        sn[rb] = FP4 ? *gptr((const uint32_t *)srow[rb]) : 0u;
    }
    for (int c = 0; c < nchunk; c++) {
        u32x4 wc[RB][2];
        uint32_t sc4[RB];
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            wc[rb][0] = wn[rb][0];
            wc[rb][1] = wn[rb][1];
            sc4[rb] = sn[rb];
        }
        if (c + 1 < nchunk) {
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                const uint8_t *p = wrow[rb] + (size_t)(c + 1) * (FP4 ? 64 : 128);
                wn[rb][0] = ld_stream16(p);
                wn[rb][1] = FP4 ? wn[rb][0] : ld_stream16(p + 64);
                sn[rb] = FP4 ? *gptr((const uint32_t *)(srow[rb] + 4 * (c + 1))) : 0u;
            }
        }
        /* B operands of this chunk */
        h8 bop[TT][4];
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                bop[tt][j] = *gptr((const h8 *)(brow[tt] + c * KC + kmap<WF>(gq, j)));
        /* FP8 chunk scales (wave-uniform), one per matrix */
        float s_lo = 1.0f, s_hi = 1.0f;
        if constexpr (WF == FMT_FP8_E8M0) {
            s_lo = dev_e8m0(ld_u8(m1.s, (size_t)nb * kbn + c));
            if (SWIGLU) s_hi = dev_e8m0(ld_u8(m3.s, (size_t)nb * kbn + c));
        } else if constexpr (WF == FMT_FP8_F32S) {
            s_lo = ld_f32(m1.s, (size_t)nb * kbn + c);
            if (SWIGLU) s_hi = ld_f32(m3.s, (size_t)nb * kbn + c);
        }
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            float cvt_scale;
            if constexpr (FP4) {
                const uint32_t b = (sc4[rb] >> (8 * gq)) & 0xFFu;
                scale_bad |= (b - 104u) > 36u;
                cvt_scale = dev_e8m0(b);
            } else {
                cvt_scale = 1.0f;          /* raw e4m3, exact in fp16 */
            }
            if constexpr (!FP4) {
                f4v part[TT];
#pragma unroll
                for (int tt = 0; tt < TT; tt++) part[tt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const h8 av = a_operand<WF>(wc[rb], cvt_scale, j);
#pragma unroll
                    for (int tt = 0; tt < TT; tt++)
                        if (tt < ntt) part[tt] = mfma16(av, bop[tt][j], part[tt]);
                }
                const float s = (SWIGLU && rb >= 4) ? s_hi : s_lo;
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[rb][tt][e] = fmaf(part[tt][e], s, acc[rb][tt][e]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const h8 av = a_operand<WF>(wc[rb], cvt_scale, j);
#pragma unroll
                    for (int tt = 0; tt < TT; tt++)
                        if (tt < ntt) acc[rb][tt] = mfma16(av, bop[tt][j], acc[rb][tt]);
                }
            }
        }
    }
    if (scale_bad) atomicOr(a.status, ST_SCALE_RANGE);

    /* epilogue: lane holds token rr of each tile, features 4 gq .. 4 gq + 3
     * of each 16-row block */
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int t = 16 * tt + rr;
        if (t >= ntok) continue;
        const size_t orow = (size_t)(r0 + t) * N;
        if constexpr (SWIGLU) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                float m[4];
#pragma unroll
                for (int e = 0; e < 4; e++) m[e] = dev_swiglu(acc[rb][tt][e], acc[rb + 4][tt][e], a.limit);
                uint2 pk;
                pk.x = f16_bits(m[0]) | (f16_bits(m[1]) << 16);
                pk.y = f16_bits(m[2]) | (f16_bits(m[3]) << 16);
                *(uint2 *)((uint16_t *)a.out + orow + f0 + 16 * rb + 4 * gq) = pk;
            }
        } else {
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                *(f4v *)((float *)a.out + orow + f0 + 16 * rb + 4 * gq) = acc[rb][tt];
        }
    }
}

/* ------------------------------------------------------------- combine --- */

/* 4 consecutive outputs of one token per thread */
__global__ __launch_bounds__(256) void k_moe_combine(CombineArgs a)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int q = a.hidden / 4;
    if (i >= (size_t)a.n * q) return;
    const int t = (int)(i / q), c = (int)(i - (size_t)t * q) * 4;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < a.topk; k++) {
        const int p = a.pos[(size_t)t * a.topk + k];
        const float wk = a.w[(size_t)t * a.topk + k];
        f32x4 v;
        if (p >= 0) {
            v = *(const f32x4 *)(a.Y + (size_t)p * a.hidden + c);
        } else {
            const float nan = __builtin_nanf("");
            v = f32x4{nan, nan, nan, nan};
        }
        o.x = __fadd_rn(o.x, __fmul_rn(wk, v.x));
        o.y = __fadd_rn(o.y, __fmul_rn(wk, v.y));
        o.z = __fadd_rn(o.z, __fmul_rn(wk, v.z));
        o.w = __fadd_rn(o.w, __fmul_rn(wk, v.w));
    }
    if (a.YS) {
        const f32x4 s = *(const f32x4 *)(a.YS + (size_t)t * a.hidden + c);
        o.x = __fadd_rn(o.x, s.x);
        o.y = __fadd_rn(o.y, s.y);
        o.z = __fadd_rn(o.z, s.z);
        o.w = __fadd_rn(o.w, s.w);
    }
    *(f32x4 *)(a.out + (size_t)t * a.hidden + c) = o;
}

/* ------------------------------------------------------------ launchers --- */

hipError_t moe_route_launch(const RouteArgs &a, hipStream_t st)
{
    if (a.n_experts < 1 || a.n_experts > MAX_ROUTE_EXPERTS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(1024), 0, st, a);
    return hipGetLastError();
}

hipError_t to_f16_launch(uint16_t *o, const float *x, size_t n, hipStream_t st)
{
    if (n % 8) return hipErrorInvalidValue;
    const size_t n8 = n / 8;
    hipLaunchKernelGGL(k_to_f16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, o, x, n8);
    return hipGetLastError();
}

int grouped_rows_per_tile(int tt) { return 16 * tt; }

template <int WF, bool SW>
static hipError_t grouped_tt(const GroupedArgs &a, int tt, long items, hipStream_t st)
{
    const dim3 grid((unsigned)((items + 3) / 4)), block(256);
    if (tt == 1) hipLaunchKernelGGL((k_grouped<WF, SW, 1>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((k_grouped<WF, SW, 4>), grid, block, 0, st, a);
    return hipGetLastError();
}

hipError_t grouped_launch(int fmt, bool swiglu, int tt, const GroupedArgs &a, long max_tiles,
                          hipStream_t st)
{
    const int feat = swiglu ? 64 : 128;
    if (a.N % feat || a.K % KC || (tt != 1 && tt != 4) || max_tiles <= 0) return hipErrorInvalidValue;
    const long items = max_tiles * (a.N / feat);
    switch (fmt) {
    case FMT_FP4_E8M0:
        return swiglu ? grouped_tt<FMT_FP4_E8M0, true>(a, tt, items, st)
                      : grouped_tt<FMT_FP4_E8M0, false>(a, tt, items, st);
    case FMT_FP8_E8M0:
        return swiglu ? grouped_tt<FMT_FP8_E8M0, true>(a, tt, items, st)
                      : grouped_tt<FMT_FP8_E8M0, false>(a, tt, items, st);
    case FMT_FP8_F32S:
        return swiglu ? grouped_tt<FMT_FP8_F32S, true>(a, tt, items, st)
                      : grouped_tt<FMT_FP8_F32S, false>(a, tt, items, st);
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t moe_combine_launch(const CombineArgs &a, hipStream_t st)
{
    if (a.hidden % 4) return hipErrorInvalidValue;
    const size_t threads = (size_t)a.n * (a.hidden / 4);
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, a);
    return hipGetLastError();
}

} // namespace dsv4
