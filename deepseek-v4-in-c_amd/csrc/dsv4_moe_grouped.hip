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
 *                   each tile's bucket, first row and rows (tile_rec),
 *                   each pair's row (pos) and each row's token (row_tok);
 *                   one launch, each workgroup placing its own chunks of
 *                   1024 pairs after counting all of them.
 *   k_to_f16_rows   x -> fp16 (round to nearest even) after scaling each
 *                   row by the power of two that puts its largest magnitude
 *                   in [2^14, 2^15); the GEMM epilogues undo it exactly.
 *   k_grouped       one wave = one work item: an expert, a slab of output
 *                   features (64 for gate/up with both w1 and w3 rows, 128 for
 *                   down) and a tile of up to 16*TT of its rows, read from
 *                   the tile's record; the grid is an upper bound and
 *                   surplus waves exit.
 *   k_moe_combine   out[t] = sum_k w[t][k] * Y[pos(t, k)] (k order) + shared[t].
 *
 * NUMERICS
 *   v_mfma_f32_16x16x32_f16, fp32 accumulation. Weights are decoded into the
 *   MFMA operand with v_cvt_scalef32_pk_f16_{fp4,fp8}: e2m1 * 2^e is exact in
 *   fp16 for E8M0 scale bytes 104..140 (checked on every block: outside it
 *   the status word gets ST_SCALE_RANGE); e4m3 values enter unscaled (exact)
 *   and the 128x128 block scale, E8M0 or fp32, multiplies each 128-K chunk's
 *   partial sum in fp32, as the reference's fp8_n applies it per block. The
 *   activations (row-scaled by a power of two, so no finite value overflows
 *   and values down to 2^-28 of the row maximum stay normal) and the SwiGLU
 *   output enter the MFMA rounded to fp16 (relative error at most 2^-11
 *   each); a SwiGLU output beyond the fp16 range raises ST_F16_RANGE.
 *   Everything else is fp32.
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
template <int N> struct IC { static constexpr int value = N; };
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

/* The power of two that output row r's B row carries (0 without bexp). */
__device__ __forceinline__ int b_row_exp(const GroupedArgs &a, int r)
{
    if (!a.bexp) return 0;
    return a.bexp[a.row_tok ? a.row_tok[r] : r];
}

/* Four fp32 results of a row that carries 2^ex, brought back to scale
 * (exact: a power-of-two multiply). */
__device__ __forceinline__ f4v unscale4(f4v v, int ex)
{
    if (ex == 0) return v;
    return f4v{ldexpf(v.x, -ex), ldexpf(v.y, -ex), ldexpf(v.z, -ex), ldexpf(v.w, -ex)};
}

/* SwiGLU of four (gate, up) pairs of a row that carries 2^ex, packed as four
 * fp16; a finite result beyond the fp16 range raises ST_F16_RANGE in bad. */
__device__ __forceinline__ uint2 swiglu_f16x4(const f4v &g, const f4v &u, int ex, float limit,
                                              unsigned &bad)
{
    const f4v gs = unscale4(g, ex), us = unscale4(u, ex);
    float m[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        m[e] = dev_swiglu(gs[e], us[e], limit);
        if (__builtin_isfinite(m[e]) && __builtin_fabsf(m[e]) >= 65520.0f) bad |= ST_F16_RANGE;
    }
    uint2 pk;
    pk.x = f16_bits(m[0]) | (f16_bits(m[1]) << 16);
    pk.y = f16_bits(m[2]) | (f16_bits(m[3]) << 16);
    return pk;
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

/* Chunks of 1024 pairs whose routing ids a thread holds in registers at
 * once: their loads are all issued before the first is used, so a pass over
 * them waits out one memory latency instead of one per chunk. */
constexpr int ROUTE_BATCH = 32;
constexpr int ROUTE_MAX_BLOCKS = 256;

__device__ __forceinline__ void route_load(int (&ev)[ROUTE_BATCH], const RouteArgs &a, int c0, int nch,
                                           int tid)
{
#pragma unroll
    for (int i = 0; i < ROUTE_BATCH; i++) {
        const int p = (c0 + i) * 1024 + tid;
        ev[i] = (c0 + i < nch && p < a.npairs) ? a.idx[p] : -1;
    }
}

/* The lanes of the wave whose routing id equals this lane's; ids outside
 * [0, E) (bad ids and pairs past the end) all count as one id of their own:
 * one ballot per bit of the key id + 1 (E <= 1024, so 11 bits). */
__device__ __forceinline__ uint64_t same_id_lanes(int e, int E)
{
    const unsigned key = (unsigned)e < (unsigned)E ? (unsigned)e + 1u : 0u;
    uint64_t peers = ~0ull;
#pragma unroll
    for (int b = 0; b < 11; b++) {
        const bool bit = (key >> b) & 1u;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

/* The wave's count of this lane's expert when this lane is the highest of
 * that expert's lanes, else 0: one LDS add per expert and wave rather than
 * one per pair, so a popular expert's counter is not hammered by every lane.
 * Called by every lane of the wave (it ballots). */
__device__ __forceinline__ int route_leader_count(int e, int E, uint64_t below)
{
    const uint64_t peers = same_id_lanes(e, E);
    const int n = __popcll(peers);
    return ((unsigned)e < (unsigned)E && __popcll(peers & below) == n - 1) ? n : 0;
}

/* Pass one of the two-launch form: workgroup c counts chunk c's pairs per
 * expert into chist[c][E] (and reports bad ids). */
__global__ __launch_bounds__(1024) void k_moe_route_count(RouteArgs a)
{
    __shared__ int hist[MAX_ROUTE_EXPERTS];
    const int tid = threadIdx.x, E = a.n_experts, c = blockIdx.x;
    const int lane = tid & 63;
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    const int p = c * 1024 + tid;
    const int e = p < a.npairs ? a.idx[p] : -1;
    hist[tid] = 0;
    __syncthreads();
    const int n = route_leader_count(e, E, below);
    if (n) atomicAdd(&hist[e], n);
    else if ((unsigned)e >= (unsigned)E && p < a.npairs) atomicOr(a.status, ST_BAD_EXPERT_ID);
    __syncthreads();
    if (tid < E) a.chist[(size_t)c * E + tid] = hist[tid];
}

/* Stable counting sort of the pairs by expert. Pairs go in chunks of 1024;
 * workgroup b places chunks [b * cpb, (b + 1) * cpb). It needs the bucket
 * sizes and how many pairs of each expert precede its first chunk: with
 * PRECOUNT it sums them from the per-chunk counts k_moe_route_count wrote
 * (two launches); without, every workgroup counts every pair itself (one
 * launch, no workgroup waits for another: the form for a few chunks).
 * Workgroup 0 also writes grp_off and tile_pre, every workgroup a share
 * of the tile records; bad ids are
 * reported by workgroup 0 (one launch) or by the counting pass. */
template <bool PRECOUNT>
__global__ __launch_bounds__(1024) void k_moe_route(RouteArgs a, int cpb)
{
    __shared__ int hist[MAX_ROUTE_EXPERTS], before[MAX_ROUTE_EXPERTS];
    __shared__ int cur[MAX_ROUTE_EXPERTS];
    __shared__ int scan_r[MAX_ROUTE_EXPERTS], scan_t[MAX_ROUTE_EXPERTS];
    __shared__ unsigned short wcnt[16][MAX_ROUTE_EXPERTS];
    const int tid = threadIdx.x;
    const int E = a.n_experts;
    const int nch = (a.npairs + 1023) / 1024;
    const int c_lo = blockIdx.x * cpb, c_hi = min(nch, c_lo + cpb);
    int ev[ROUTE_BATCH];
    /* the first batch of routing ids is in flight while the tables clear */
    if (!PRECOUNT) route_load(ev, a, 0, nch, tid);
    if (tid < E) {
        hist[tid] = 0;
        before[tid] = 0;
        for (int w = 0; w < 16; w++) wcnt[w][tid] = 0;
    }
    __syncthreads();
    unsigned bad = 0;
    const int lane = tid & 63, wv = tid >> 6;
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    if constexpr (PRECOUNT) {
        /* expert tid's count in every chunk: sixteen loads in flight per
         * round, summed in chunk order (integers: any order gives the same) */
        if (tid < E) {
            int tot = 0, bef = 0;
            for (int c0 = 0; c0 < nch; c0 += 16) {
                int v[16];
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = c0 + i < nch ? a.chist[(size_t)(c0 + i) * E + tid] : 0;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    tot += v[i];
                    if (c0 + i < c_lo) bef += v[i];
                }
            }
            hist[tid] = tot;
            before[tid] = bef;
        }
    } else
    for (int c0 = 0; c0 < nch; c0 += ROUTE_BATCH) {
        if (c0) route_load(ev, a, c0, nch, tid);
#pragma unroll
        for (int i = 0; i < ROUTE_BATCH; i++) {
            if (c0 + i >= nch) break;                              /* uniform */
            const int p = (c0 + i) * 1024 + tid;
            const int n = route_leader_count(ev[i], E, below);
            if (n) {
                atomicAdd(&hist[ev[i]], n);
                if (c0 + i < c_lo) atomicAdd(&before[ev[i]], n);
            } else if ((unsigned)ev[i] >= (unsigned)E && p < a.npairs) {
                bad = ST_BAD_EXPERT_ID;
            }
        }
    }
    __syncthreads();
    /* inclusive scans of the bucket sizes and tile counts, one expert per
     * thread (E <= 1024): within each wave by shuffles, then the totals of
     * the lower waves added (two barriers) */
    const int cnt = tid < E ? hist[tid] : 0;
    const int tls = (cnt + a.tile_rows - 1) / a.tile_rows;
    {
        /* only the waves that hold experts scan (E / 64 rounded up) */
        __shared__ int wsum[2][16];
        const bool live = wv * 64 < E;
        int ir = cnt, it = tls;
        if (live) {
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int xr = __shfl_up(ir, d, 64), xt = __shfl_up(it, d, 64);
                if (lane >= d) {
                    ir += xr;
                    it += xt;
                }
            }
            if (lane == 63) {
                wsum[0][wv] = ir;
                wsum[1][wv] = it;
            }
        }
        __syncthreads();
        if (live) {
            for (int w = 0; w < wv; w++) {
                ir += wsum[0][w];
                it += wsum[1][w];
            }
            scan_r[tid] = ir;
            scan_t[tid] = it;
        }
        __syncthreads();
    }
    /* each tile's bucket: the first expert whose inclusive tile prefix
     * exceeds it, tiles spread over every workgroup's threads; with the
     * bucket's first row and the tile's rows */
    for (int t = blockIdx.x * 1024 + tid; t < scan_t[E - 1]; t += gridDim.x * 1024) {
        int lo = 0, hi = E - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (scan_t[mid] > t) hi = mid;
            else lo = mid + 1;
        }
        const int go = lo > 0 ? scan_r[lo - 1] : 0, tp = lo > 0 ? scan_t[lo - 1] : 0;
        const int r0 = go + (t - tp) * a.tile_rows;
        TileRec rec;
        rec.grp = lo;
        rec.r0 = r0;
        rec.ntok = min(a.tile_rows, scan_r[lo] - r0);
        rec.pad = 0;
        a.tile_rec[t] = rec;
    }
    if (tid < E) {
        const int o = scan_r[tid] - cnt;
        cur[tid] = o + before[tid];
        if (blockIdx.x == 0) {
            a.grp_off[tid] = o;
            a.tile_pre[tid] = scan_t[tid] - tls;
            if (tid == E - 1) {
                a.grp_off[E] = scan_r[tid];
                a.tile_pre[E] = scan_t[tid];
            }
        }
    }
    __syncthreads();
    /* Rows inside a bucket in pair order (token-major, k-minor), as the
     * reference's counting sort places them: a pair's row is its bucket's
     * start, plus the pairs of the same expert in earlier chunks, plus those
     * in lower waves of its chunk (each expert's per-wave counts turned into
     * exclusive prefixes in place), plus those in lower lanes of its wave.
     * A workgroup that counted every chunk in one batch already holds its
     * routing ids. */
    const bool have_ids = !PRECOUNT && c_lo == 0 && c_hi == nch && nch <= ROUTE_BATCH;
    for (int c0 = c_lo; c0 < c_hi; c0 += ROUTE_BATCH) {
        if (!have_ids) route_load(ev, a, c0, c_hi, tid);
#pragma unroll
        for (int i = 0; i < ROUTE_BATCH; i++) {
            if (c0 + i >= c_hi) break;                             /* uniform */
            const int p = (c0 + i) * 1024 + tid;
            const int e = ev[i];
            const bool ok = (unsigned)e < (unsigned)E;
            const uint64_t peers = same_id_lanes(e, E);
            const int rank = __popcll(peers & below);
            if (ok && rank == __popcll(peers) - 1) wcnt[wv][e] = (unsigned short)(rank + 1);
            __syncthreads();
            int tot = 0;
            if (tid < E) {
                unsigned short c[16];
#pragma unroll
                for (int w = 0; w < 16; w++) c[w] = wcnt[w][tid];
#pragma unroll
                for (int w = 0; w < 16; w++) {
                    wcnt[w][tid] = (unsigned short)tot;
                    tot += c[w];
                }
            }
            __syncthreads();
            if (ok) {
                const int r = cur[e] + wcnt[wv][e] + rank;
                a.pos[p] = r;
                a.row_tok[r] = p / a.topk;
                if (a.row_k) a.row_k[r] = p - (p / a.topk) * a.topk;
            } else if (p < a.npairs) {
                a.pos[p] = -1;
            }
            __syncthreads();
            if (tid < E) {
                cur[tid] += tot;
#pragma unroll
                for (int w = 0; w < 16; w++) wcnt[w][tid] = 0;
            }
            __syncthreads();
        }
    }
    if (!PRECOUNT && bad && blockIdx.x == 0) atomicOr(a.status, bad);
}

/* One workgroup per row: the row's largest finite magnitude (a fixed-order
 * max, order does not matter), then 8 floats -> 8 fp16 per thread and unit,
 * each multiplied by the row's power of two first (exact). The second pass
 * re-reads the row from cache. */
__device__ __forceinline__ float finite_abs(float v)
{
    const float m = __builtin_fabsf(v);
    return __builtin_isfinite(m) ? m : 0.0f;
}

__global__ __launch_bounds__(256) void k_to_f16_rows(uint16_t *o, int *ex, const float *x, int cols)
{
    __shared__ float wmax[4];
    const float *xr = x + (size_t)blockIdx.x * cols;
    uint16_t *orow = o + (size_t)blockIdx.x * cols;
    const int units = cols / 8;
    float m = 0.0f;
    for (int u = threadIdx.x; u < units; u += 256) {
        const f32x4 a = *(const f32x4 *)(xr + 8 * u), b = *(const f32x4 *)(xr + 8 * u + 4);
        m = fmaxf(m, fmaxf(fmaxf(finite_abs(a.x), finite_abs(a.y)), fmaxf(finite_abs(a.z), finite_abs(a.w))));
        m = fmaxf(m, fmaxf(fmaxf(finite_abs(b.x), finite_abs(b.y)), fmaxf(finite_abs(b.z), finite_abs(b.w))));
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const int e = m > 0.0f ? 14 - ilogbf(m) : 0;       /* m * 2^e in [2^14, 2^15) */
    if (threadIdx.x == 0) ex[blockIdx.x] = e;
    for (int u = threadIdx.x; u < units; u += 256) {
        const f32x4 a = *(const f32x4 *)(xr + 8 * u), b = *(const f32x4 *)(xr + 8 * u + 4);
        u32x4 v;
        v.x = f16_bits(ldexpf(a.x, e)) | (f16_bits(ldexpf(a.y, e)) << 16);
        v.y = f16_bits(ldexpf(a.z, e)) | (f16_bits(ldexpf(a.w, e)) << 16);
        v.z = f16_bits(ldexpf(b.x, e)) | (f16_bits(ldexpf(b.y, e)) << 16);
        v.w = f16_bits(ldexpf(b.z, e)) | (f16_bits(ldexpf(b.w, e)) << 16);
        *(u32x4 *)(orow + 8 * u) = v;
    }
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
        const int ntiles = ld_uniform(a.tile_pre, E);
        const TileRec tr = ld_uniform(a.tile_rec, tile);  /* read beside the count: one round trip */
        if ((tile >= ntiles) | (tr.ntok <= 0)) return;
        r0 = tr.r0;
        ntok = tr.ntok;
        const DSV4ExpertW e = ld_uniform(a.table, tr.grp);
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
    /* 32-bit per-lane offsets from the wave-uniform matrix bases (a matrix is
     * below 4 GiB): the weight byte of block rb is base(rb) + wofs[rb], its
     * FP4 scale row base_s(rb) + sofs[rb] */
    const uint8_t *wb1 = (const uint8_t *)m1.w, *wb3 = (const uint8_t *)m3.w;
    const uint8_t *sb1 = (const uint8_t *)m1.s, *sb3 = (const uint8_t *)m3.s;
    uint32_t wofs[RB], sofs[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int row = f0 + 16 * (SWIGLU ? (rb & 3) : rb) + rr;
        wofs[rb] = (uint32_t)row * (uint32_t)rowb + 16u * (uint32_t)gq;
        sofs[rb] = (uint32_t)row * (uint32_t)(K / 32);
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
    /* Raw weights of the next PF chunks are in flight while one multiplies:
     * with 16-row tiles the item is a weight stream and needs several chunks
     * in flight to cover HBM latency; with 64-row tiles one chunk of compute
     * covers it. The B operands (tokens, from L2) are fetched one chunk
     * ahead. */
    constexpr int PF = (TT == 1 && FP4) ? 3 : 1;
    constexpr int CB = FP4 ? 64 : 128;             /* weight bytes per row per chunk */
    struct WChunk {
        u32x4 w[RB][2];
        uint32_t s[RB];                            /* FP4: the lane's 4 E8M0 bytes  */
        float fs[2];                               /* FP8: chunk scale of m1, m3    */
    };
    auto load_w = [&](int c, WChunk &o) {
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const bool up = SWIGLU && rb >= 4;
            const uint8_t *p = (up ? wb3 : wb1) + (wofs[rb] + (uint32_t)(c * CB));
            o.w[rb][0] = ld_stream16(p);
            if constexpr (!FP4) o.w[rb][1] = ld_stream16(p + 64);
            if constexpr (FP4)
                o.s[rb] = *gptr((const uint32_t *)((up ? sb3 : sb1) + (sofs[rb] + 4u * (uint32_t)c)));
        }
        if constexpr (WF == FMT_FP8_E8M0) {
            o.fs[0] = dev_e8m0(ld_u8(m1.s, (size_t)nb * kbn + c));
            o.fs[1] = SWIGLU ? dev_e8m0(ld_u8(m3.s, (size_t)nb * kbn + c)) : 0.0f;
        } else if constexpr (WF == FMT_FP8_F32S) {
            o.fs[0] = ld_f32(m1.s, (size_t)nb * kbn + c);
            o.fs[1] = SWIGLU ? ld_f32(m3.s, (size_t)nb * kbn + c) : 0.0f;
        } else {
            o.fs[0] = o.fs[1] = 1.0f;
        }
    };
    auto load_b = [&](int c, h8 (&b)[TT][4]) {
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                b[tt][j] = *gptr((const h8 *)(brow[tt] + c * KC + kmap<WF>(gq, j)));
    };
    auto compute = [&](const WChunk &wc, const h8 (&bop)[TT][4]) {
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            float cvt_scale = 1.0f;                /* FP8: raw e4m3, exact in fp16 */
            if constexpr (FP4) {
                const uint32_t b = (wc.s[rb] >> (8 * gq)) & 0xFFu;
                scale_bad |= (b - 104u) > 36u;
                cvt_scale = dev_e8m0(b);
            }
            if constexpr (!FP4) {
                f4v part[TT];
#pragma unroll
                for (int tt = 0; tt < TT; tt++) part[tt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const h8 av = a_operand<WF>(wc.w[rb], cvt_scale, j);
#pragma unroll
                    for (int tt = 0; tt < TT; tt++)
                        if (tt < ntt) part[tt] = mfma16(av, bop[tt][j], part[tt]);
                }
                const float sc = (SWIGLU && rb >= 4) ? wc.fs[1] : wc.fs[0];
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[rb][tt][e] = fmaf(part[tt][e], sc, acc[rb][tt][e]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const h8 av = a_operand<WF>(wc.w[rb], cvt_scale, j);
#pragma unroll
                    for (int tt = 0; tt < TT; tt++)
                        if (tt < ntt) acc[rb][tt] = mfma16(av, bop[tt][j], acc[rb][tt]);
                }
            }
        }
    };

    /* Loads are issued unconditionally (past the end they repeat the last
     * chunk, an L2 hit): a load behind a branch makes the wait-count pass
     * drain every outstanding load at the join, prefetches included. */
    const int last = nchunk - 1;
    WChunk ring[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) load_w(min(i, last), ring[i]);
    h8 bnext[TT][4];
    load_b(0, bnext);
    int c = 0;
    for (; c + PF <= nchunk; c += PF) {
#pragma unroll
        for (int i = 0; i < PF; i++) {
            const WChunk wc = ring[i];
            load_w(min(c + i + PF, last), ring[i]);
            h8 bop[TT][4];
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int j = 0; j < 4; j++) bop[tt][j] = bnext[tt][j];
            load_b(min(c + i + 1, last), bnext);
            compute(wc, bop);
        }
    }
    /* at most PF - 1 chunks remain; they are already in the ring */
#pragma unroll
    for (int i = 0; i + 1 < PF; i++) {
        if (c + i < nchunk) {
            h8 bop[TT][4];
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int j = 0; j < 4; j++) bop[tt][j] = bnext[tt][j];
            load_b(min(c + i + 1, last), bnext);
            compute(ring[i], bop);
        }
    }
    if (scale_bad) atomicOr(a.status, ST_SCALE_RANGE);

    /* epilogue: lane holds token rr of each tile, features 4 gq .. 4 gq + 3
     * of each 16-row block */
    unsigned range_bad = 0;
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int t = 16 * tt + rr;
        if (t >= ntok) continue;
        const size_t orow = (size_t)(r0 + t) * N;
        const int ex = b_row_exp(a, r0 + t);
        if constexpr (SWIGLU) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
                *(uint2 *)((uint16_t *)a.out + orow + f0 + 16 * rb + 4 * gq) =
                    swiglu_f16x4(acc[rb][tt], acc[rb + 4][tt], ex, a.limit, range_bad);
        } else {
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                *(f4v *)((float *)a.out + orow + f0 + 16 * rb + 4 * gq) = unscale4(acc[rb][tt], ex);
        }
    }
    if (range_bad) atomicOr(a.status, range_bad);
}

/* ------------------------------------------- LDS-staged grouped GEMM --- */

/* The same work as k_grouped, for K a multiple of 256, with a workgroup per
 * item and every operand staged through LDS by direct loads. Direct global
 * loads in the MFMA layout make each instruction touch 16 rows (64 B each)
 * and keep the texture-address units ~85 % busy; here every 1 KiB load
 * instruction covers whole 128-byte lines of at most 8 rows.
 *
 * Workgroup: 128 weight rows (gate/up: 64 w1 rows + the matching 64 w3 rows;
 * down: 128 w2 rows) x TOK = 16*TT token rows. TT = 1 (a weight stream): 4
 * waves of 32 rows each. TT = 4: 8 waves, 4 x 32 rows by 2 x 32 tokens, two
 * waves per SIMD, so that one wave's LDS operand reads (~27 B/clk each) and
 * conversions overlap the other's MFMAs. A stage is 256 reduction indices: weights (FP4 128 B
 * or FP8 256 B per row), the FP4 rows' eight E8M0 bytes, and the token rows
 * (fp16, 512 B each), in NST ring buffers; stage s+NST-1 is loaded while s
 * multiplies. 16-byte chunks are XOR-swizzled so the operand reads of 16
 * rows hit distinct banks. */
namespace {

typedef __attribute__((address_space(3))) void lds_void;
constexpr int KS = 256;

__device__ __forceinline__ void dma16(const void *src, uint8_t *dst)
{
    __builtin_amdgcn_global_load_lds(gptr(src), (lds_void *)dst, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *src, uint8_t *dst)
{
    __builtin_amdgcn_global_load_lds(gptr(src), (lds_void *)dst, 4, 0, 0);
}

/* Default ring depth: FP4 16-row tiles two stages (2 x 25 KiB, three
 * workgroups per CU overlap each other's pipeline ramp), FP8 16-row tiles
 * three (3 x 40 KiB), 64-row tiles FP4 three, FP8 two. */
template <int WF, int TT>
constexpr int g2_stages() { return TT == 1 ? (WF == FMT_FP4_E8M0 ? 2 : 3) : (WF == FMT_FP4_E8M0 ? 3 : 2); }

template <int WF, int TT, int STAGES = g2_stages<WF, TT>()>
struct G2 {
    static constexpr bool FP4 = WF == FMT_FP4_E8M0;
    static constexpr int WB = FP4 ? KS / 2 : KS;         /* weight bytes per row per stage */
    static constexpr int ROWS = 128;
    static constexpr int TOK = 16 * TT;
    static constexpr int NWAVE = TT == 1 ? 4 : 8;        /* 64-row tiles: 2 waves / SIMD */
    static constexpr int WR = 4;                         /* waves along rows           */
    static constexpr int WT = NWAVE / WR;                /* waves along tokens         */
    static constexpr int RBW = 8 / WR;                   /* 16-row blocks per wave     */
    static constexpr int TTW = TT / WT;                  /* 16-token tiles per wave    */
    static constexpr int OFF_S = ROWS * WB;
    static constexpr int OFF_PAD = OFF_S + (FP4 ? ROWS * 8 : 0);   /* scale loads of waves 4+ */
    static constexpr int OFF_B = OFF_PAD + (FP4 && NWAVE > 4 ? 256 : 0);
    static constexpr int STAGE = OFF_B + TOK * KS * 2;
    static constexpr int NST = STAGES;
    static constexpr int LDS = NST * STAGE;
    static constexpr int NW = ROWS * WB / 1024 / NWAVE;  /* weight loads per wave per stage */
    static constexpr int NS = FP4 ? 1 : 0;               /* scale loads                */
    static constexpr int NB = TOK * KS * 2 / 1024 / NWAVE;   /* token-row loads        */
    static_assert(NW * NWAVE * 1024 == ROWS * WB && NB * NWAVE * 1024 == TOK * KS * 2, "load split");
    static constexpr int VM = NW + NS + NB;
    static_assert(LDS <= 160 * 1024, "LDS ring exceeds 160 KiB");
    static_assert((NST - 2) * VM <= 63, "vmcnt range");
};

/* physical 16-byte slot of logical chunk c in staged row r */
__device__ __forceinline__ int swz_w4(int r, int c) { return c ^ ((r >> 1) & 7); }   /* 8 slots   */
__device__ __forceinline__ int swz_w8(int r, int c) { return c ^ (r & 15); }         /* 16 slots  */
__device__ __forceinline__ int swz_b(int r, int c) { return c ^ (r & 15); }          /* 32 slots  */

/* B chunk (8 halves) of MFMA step sg (0..7) for lane group gq: the token side
 * of the reduction order the weight side is read in */
template <int WF>
__device__ __forceinline__ int bchunk(int gq, int sg)
{
    if constexpr (WF == FMT_FP4_E8M0) return 16 * (sg >> 2) + 4 * gq + (sg & 3);
    else return 8 * (sg >> 1) + 2 * gq + (sg & 1);
}

} // namespace

template <int WF, bool SWIGLU, int TT, int NS>
__global__ __launch_bounds__(512) void k_grouped2(GroupedArgs a)
{
    using C = G2<WF, TT, NS>;
    constexpr bool FP4 = C::FP4;
    constexpr int FEAT = SWIGLU ? 64 : 128;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int rr = lane & 15, gq = lane >> 4;
    const int nslab = a.N / FEAT;
    const int tile = blockIdx.x / nslab, slab = blockIdx.x - tile * nslab;

    int r0, ntok;
    DSV4QMat m1, m3;
    if (a.table) {
        const int E = a.n_experts;
        const int ntiles = ld_uniform(a.tile_pre, E);
        const TileRec tr = ld_uniform(a.tile_rec, tile);  /* read beside the count: one round trip */
        if ((tile >= ntiles) | (tr.ntok <= 0)) return;   /* whole workgroup */
        r0 = tr.r0;
        ntok = tr.ntok;
        const DSV4ExpertW e = ld_uniform(a.table, tr.grp);
        m1 = SWIGLU ? e.w1 : e.w2;
        m3 = e.w3;
    } else {
        r0 = tile * C::TOK;
        if (r0 >= a.nrows) return;
        ntok = min(C::TOK, a.nrows - r0);
        m1 = a.m1;
        m3 = a.m3;
    }
    const int f0 = slab * FEAT;
    const int K = a.K, N = a.N;
    if (!qmat_matches<WF>(m1, N, K) || (SWIGLU && !qmat_matches<WF>(m3, N, K))) {
        if (threadIdx.x == 0) atomicOr(a.status, ST_BAD_DESCRIPTOR);
        const float nan = __builtin_nanf("");
        for (int i = threadIdx.x; i < ntok * FEAT; i += 64 * C::NWAVE) {
            const size_t o = (size_t)(r0 + i / FEAT) * N + f0 + i % FEAT;
            if constexpr (SWIGLU) ((uint16_t *)a.out)[o] = (uint16_t)f16_bits(nan);
            else ((float *)a.out)[o] = nan;
        }
        return;
    }

    /* ---- load plan: per-lane source offsets of this wave's loads ---- */
    const int rowb = FP4 ? K / 2 : K;
    const int nst = K / KS, last = nst - 1;
    const uint8_t *wbase[C::NW];
    int wdst[C::NW];
#pragma unroll
    for (int i = 0; i < C::NW; i++) {
        const int j = wave * C::NW + i;                    /* 1 KiB instruction index */
        const int rpi = 1024 / C::WB;                      /* rows per instruction    */
        const int r = j * rpi + lane / (C::WB / 16);
        const int p = lane % (C::WB / 16);
        const bool up = SWIGLU && r >= 64;
        const int row = f0 + (SWIGLU ? (r & 63) : r);
        const int c = FP4 ? swz_w4(r, p) : swz_w8(r, p);
        wbase[i] = (const uint8_t *)(up ? m3.w : m1.w) + (size_t)row * rowb + 16 * c;
        wdst[i] = 1024 * j;
    }
    const uint8_t *sbase = nullptr;
    if constexpr (FP4) {
        const int r = 32 * (wave & 3) + lane / 2;          /* waves 4+ repeat rows into the pad */
        const bool up = SWIGLU && r >= 64;
        const int row = f0 + (SWIGLU ? (r & 63) : r);
        sbase = (const uint8_t *)(up ? m3.s : m1.s) + (size_t)row * (K / 32) + 4 * (lane & 1);
    }
    const uint16_t *bbase[C::NB];
#pragma unroll
    for (int i = 0; i < C::NB; i++) {
        const int j = wave * C::NB + i;
        const int t = 2 * j + lane / 32, p = lane & 31;
        const int r = t < ntok ? r0 + t : r0;
        const int src = a.row_tok ? a.row_tok[r] : r;
        bbase[i] = a.B + (size_t)src * K + 8 * swz_b(t, p);
    }
    auto issue = [&](int stg, uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < C::NW; i++) dma16(wbase[i] + (size_t)stg * C::WB, buf + wdst[i]);
        if constexpr (FP4)
            dma4(sbase + (size_t)stg * 8, buf + (wave < 4 ? C::OFF_S + 256 * wave : C::OFF_PAD));
#pragma unroll
        for (int i = 0; i < C::NB; i++)
            dma16(bbase[i] + (size_t)stg * KS, buf + C::OFF_B + 1024 * (wave * C::NB + i));
    };

    /* ---- this wave's share ---- */
    const int wr = wave % C::WR, wt = wave / C::WR;
    int blk[C::RBW];
#pragma unroll
    for (int i = 0; i < C::RBW; i++) {
        constexpr int H = C::RBW / 2;
        blk[i] = SWIGLU ? (i < H ? H * wr + i : 4 + H * wr + (i - H)) : C::RBW * wr + i;
    }
    int ntw = 0;                                           /* live tiles of this wave */
#pragma unroll
    for (int u = 0; u < C::TTW; u++) ntw += 16 * (wt * C::TTW + u) < ntok ? 1 : 0;

    f4v acc[C::RBW][C::TTW];
#pragma unroll
    for (int i = 0; i < C::RBW; i++)
#pragma unroll
        for (int u = 0; u < C::TTW; u++) acc[i][u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    unsigned scale_bad = 0;

#pragma unroll
    for (int s0 = 0; s0 < C::NST - 1; s0++) issue(min(s0, last), lds + s0 * C::STAGE);

    /* The main loop, instantiated per count NT of this wave's live 16-token
     * tiles so that the MFMA sequence of a stage is straight-line code (a
     * branch per MFMA splits it into blocks the scheduler cannot overlap). */
    auto run = [&](auto ntc) {
        constexpr int NT = decltype(ntc)::value;
        for (int st = 0; st < nst; st++) {
            __builtin_amdgcn_s_waitcnt(0x0F70 | ((C::NST - 2) * C::VM & 15) | ((((C::NST - 2) * C::VM) >> 4) << 14));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            {
                int nb = st + C::NST - 1;
                nb = nb >= C::NST ? nb - C::NST * (nb / C::NST) : nb;
                issue(min(st + C::NST - 1, last), lds + nb * C::STAGE);
            }
            if constexpr (NT > 0) {
                const uint8_t *buf = lds + (st % C::NST) * C::STAGE;

                /* token operands of this wave's live tiles, all 8 steps */
                h8 bop[NT][8];
#pragma unroll
                for (int u = 0; u < NT; u++) {
                    const int t = 16 * (wt * C::TTW + u) + rr;
                    const uint8_t *brow = buf + C::OFF_B + t * (KS * 2);
#pragma unroll
                    for (int sg = 0; sg < 8; sg++)
                        bop[u][sg] = *(const h8 *)(brow + 16 * swz_b(t, bchunk<WF>(gq, sg)));
                }
                /* FP8 chunk scales: 2 blocks of 128 per stage, per matrix */
                float fs[2][2] = {{1.0f, 1.0f}, {1.0f, 1.0f}};
                if constexpr (!FP4) {
                    const int nb = f0 / 128, kbn = K / 128;
#pragma unroll
                    for (int b = 0; b < 2; b++) {
                        const size_t si = (size_t)nb * kbn + 2 * st + b;
                        if constexpr (WF == FMT_FP8_E8M0) {
                            fs[0][b] = dev_e8m0(ld_u8(m1.s, si));
                            fs[1][b] = SWIGLU ? dev_e8m0(ld_u8(m3.s, si)) : 1.0f;
                        } else {
                            fs[0][b] = ld_f32(m1.s, si);
                            fs[1][b] = SWIGLU ? ld_f32(m3.s, si) : 1.0f;
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < C::RBW; i++) {
                    const int r = 16 * blk[i] + rr;            /* staged row */
                    if constexpr (FP4) {
                        const uint2 sc8 = *(const uint2 *)(buf + C::OFF_S + r * 8);
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const int c = 4 * h + gq;
                            const u32x4 w16 = *(const u32x4 *)(buf + r * C::WB + 16 * swz_w4(r, c));
                            const uint32_t sb = ((c < 4 ? sc8.x : sc8.y) >> (8 * (c & 3))) & 0xFFu;
                            scale_bad |= (sb - 104u) > 36u;
                            const float cs = dev_e8m0(sb);
                            const u32x4 wv[2] = {w16, w16};
#pragma unroll
                            for (int s = 0; s < 4; s++) {
                                const h8 av = a_operand<WF>(wv, cs, s);
#pragma unroll
                                for (int u = 0; u < NT; u++) acc[i][u] = mfma16(av, bop[u][4 * h + s], acc[i][u]);
                            }
                        }
                    } else {
                        const float *fsm = fs[(SWIGLU && blk[i] >= 4) ? 1 : 0];
#pragma unroll
                        for (int b = 0; b < 2; b++) {          /* 128-K block of the stage */
                            f4v part[NT];
#pragma unroll
                            for (int u = 0; u < NT; u++) part[u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                            for (int q2 = 0; q2 < 2; q2++) {
                                const int q = 2 * b + q2;
                                const int c = 4 * q + gq;
                                const u32x4 w16 = *(const u32x4 *)(buf + r * C::WB + 16 * swz_w8(r, c));
                                const u32x4 wv[2] = {w16, w16};
#pragma unroll
                                for (int s = 0; s < 2; s++) {
                                    const h8 av = a_operand<WF>(wv, 1.0f, s);   /* dwords 2s, 2s+1 */
#pragma unroll
                                    for (int u = 0; u < NT; u++) part[u] = mfma16(av, bop[u][2 * q + s], part[u]);
                                }
                            }
#pragma unroll
                            for (int u = 0; u < NT; u++)
#pragma unroll
                                for (int e = 0; e < 4; e++) acc[i][u][e] = fmaf(part[u][e], fsm[b], acc[i][u][e]);
                        }
                    }
                }
            }
        }
    };
    if (ntw >= C::TTW) run(IC<C::TTW>{});
    else if constexpr (C::TTW > 1) {
        if (ntw == 1) run(IC<1>{});
        else run(IC<0>{});
    } else run(IC<0>{});
    __builtin_amdgcn_s_waitcnt(0x0F70);     /* trailing repeat loads drain before exit */
    if (scale_bad) atomicOr(a.status, ST_SCALE_RANGE);

    unsigned range_bad = 0;
#pragma unroll
    for (int u = 0; u < C::TTW; u++) {
        const int t = 16 * (wt * C::TTW + u) + rr;
        if (t >= ntok) continue;
        const size_t orow = (size_t)(r0 + t) * N;
        const int ex = b_row_exp(a, r0 + t);
        if constexpr (SWIGLU) {
            constexpr int H = C::RBW / 2;
#pragma unroll
            for (int i = 0; i < H; i++)
                *(uint2 *)((uint16_t *)a.out + orow + f0 + 16 * blk[i] + 4 * gq) =
                    swiglu_f16x4(acc[i][u], acc[i + H][u], ex, a.limit, range_bad);
        } else {
#pragma unroll
            for (int i = 0; i < C::RBW; i++)
                *(f4v *)((float *)a.out + orow + f0 + 16 * blk[i] + 4 * gq) = unscale4(acc[i][u], ex);
        }
    }
    if (range_bad) atomicOr(a.status, range_bad);
}

/* ------------------------------------------- 128-token FP4 tiles (prefill) --- */

/* For buckets of many tokens (the prefill MoE layer). Workgroup: 8 waves,
 * 256 FP4 weight rows (gate/up: 128 w1 rows + the matching 128 w3 rows;
 * down: 256 w2 rows) x 128 token rows; each wave owns 64 rows x 64 tokens
 * (4 x 4 MFMA tiles), so one converted weight operand feeds 4 MFMAs and one
 * token operand 4 more, which keeps both the conversions (VALU) and the LDS
 * operand reads below the MFMA time.
 *
 * A stage is 128 reduction indices: 256 x 64 weight bytes, the rows' four
 * E8M0 bytes, and 128 x 256 bytes of fp16 token rows; three stages in flight.
 * Every operand arrives by buffer loads straight into LDS; token rows past
 * the end of the bucket use an offset beyond the buffer, which the hardware
 * answers with zeros and no memory traffic. Chunks are XOR-swizzled so that
 * the 16 rows of an MFMA operand read hit distinct banks:
 *   weight row r (64 B):  chunk c at slot c ^ ((r >> 2) & 3)
 *   token row t (256 B):  chunk c at slot c ^ (t & 15)
 * Reduction order: lane group gq's 16 weight bytes of a row (32 values, one
 * E8M0 block) feed MFMA steps s = 0..3, 8 values each; the token side reads
 * the same 8 indices, chunk 4 gq + s of the row. */
namespace {

struct G3 {
    static constexpr int KS = 128;
    static constexpr int ROWS = 256, TOK = 128, NWAVE = 8;
    static constexpr int WB = KS / 2;                        /* FP4 bytes per row per stage */
    static constexpr int OFF_S = ROWS * WB;                  /* E8M0: 256 B per wave        */
    static constexpr int OFF_B = OFF_S + NWAVE * 256;
    static constexpr int STAGE = OFF_B + TOK * KS * 2;
    static constexpr int NST = 3;
    static constexpr int LDS = NST * STAGE;
    static constexpr int NW = ROWS * WB / 1024 / NWAVE;      /* 16-row weight loads per wave */
    static constexpr int NB = TOK * KS * 2 / 1024 / NWAVE;   /* 4-row token loads per wave   */
    static constexpr int VM = NW + 1 + NB;
    static_assert(LDS <= 160 * 1024, "LDS ring exceeds 160 KiB");
    static_assert(NW * NWAVE * 1024 == ROWS * WB && NB * NWAVE * 1024 == TOK * KS * 2, "load split");
};

constexpr uint32_t RSRC_WORD3 = 0x00020000u;      /* raw dword buffer, gfx9 */
constexpr uint32_t OOB_OFFSET = 0x80000000u;      /* beyond every buffer    */

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, (int)RSRC_WORD3);
}
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff, uint8_t *dst)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, (int)voff, soff, 0, 0);
}
__device__ __forceinline__ void bdma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff, uint8_t *dst)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 4, (int)voff, soff, 0, 0);
}

/* 8 e2m1 values (one dword, low nibble first) times 2^e -> fp16 operand */
__device__ __forceinline__ h8 fp4_h8(uint32_t d, float sc)
{
    u32x4 v;
    v.x = pk_f16_fp4(d, sc, 0);
    v.y = pk_f16_fp4(d, sc, 1);
    v.z = pk_f16_fp4(d, sc, 2);
    v.w = pk_f16_fp4(d, sc, 3);
    return __builtin_bit_cast(h8, v);
}

} // namespace

template <bool SWIGLU>
__global__ __launch_bounds__(512) void k_grouped3(GroupedArgs a)
{
    using C = G3;
    constexpr int FEAT = SWIGLU ? 128 : 256;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int rr = lane & 15, gq = lane >> 4;
    const int nslab = a.N / FEAT;
    const int tile = blockIdx.x / nslab, slab = blockIdx.x - tile * nslab;

    int r0, ntok;
    DSV4QMat m1, m3;
    if (a.table) {
        const int E = a.n_experts;
        const int ntiles = ld_uniform(a.tile_pre, E);
        const TileRec tr = ld_uniform(a.tile_rec, tile);  /* read beside the count: one round trip */
        if ((tile >= ntiles) | (tr.ntok <= 0)) return;   /* whole workgroup */
        r0 = tr.r0;
        ntok = tr.ntok;
        const DSV4ExpertW e = ld_uniform(a.table, tr.grp);
        m1 = SWIGLU ? e.w1 : e.w2;
        m3 = e.w3;
    } else {
        r0 = tile * C::TOK;
        if (r0 >= a.nrows) return;
        ntok = min(C::TOK, a.nrows - r0);
        m1 = a.m1;
        m3 = a.m3;
    }
    const int f0 = slab * FEAT;
    const int K = a.K, N = a.N;
    /* buffer loads need 16-byte aligned weights and 4-byte aligned scales */
    const bool aligned = ((uintptr_t)m1.w & 15) == 0 && ((uintptr_t)m1.s & 3) == 0 &&
                         (!SWIGLU || (((uintptr_t)m3.w & 15) == 0 && ((uintptr_t)m3.s & 3) == 0));
    if (!qmat_matches<FMT_FP4_E8M0>(m1, N, K) || (SWIGLU && !qmat_matches<FMT_FP4_E8M0>(m3, N, K)) ||
        !aligned) {
        if (threadIdx.x == 0) atomicOr(a.status, ST_BAD_DESCRIPTOR);
        const float nan = __builtin_nanf("");
        for (int i = threadIdx.x; i < ntok * FEAT; i += 64 * C::NWAVE) {
            const size_t o = (size_t)(r0 + i / FEAT) * N + f0 + i % FEAT;
            if constexpr (SWIGLU) ((uint16_t *)a.out)[o] = (uint16_t)f16_bits(nan);
            else ((float *)a.out)[o] = nan;
        }
        return;
    }

    /* ---- load plan: per-lane byte offsets into the buffers ---- */
    const uint32_t rowb = (uint32_t)K / 2, srow = (uint32_t)K / 32;
    const int nst = K / C::KS, last = nst - 1;
    const __amdgpu_buffer_rsrc_t rw1 = buf_rsrc(m1.w, (uint32_t)N * rowb);
    const __amdgpu_buffer_rsrc_t rs1 = buf_rsrc(m1.s, (uint32_t)N * srow);
    const __amdgpu_buffer_rsrc_t rw3 = SWIGLU ? buf_rsrc(m3.w, (uint32_t)N * rowb) : rw1;
    const __amdgpu_buffer_rsrc_t rs3 = SWIGLU ? buf_rsrc(m3.s, (uint32_t)N * srow) : rs1;
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(a.B, (uint32_t)a.nrows * (uint32_t)K * 2u);
    uint32_t wofs[C::NW];
#pragma unroll
    for (int i = 0; i < C::NW; i++) {
        const int j = wave * C::NW + i;                 /* rows 16 j .. 16 j + 15 */
        const int r = 16 * j + lane / 4;
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        const int row = f0 + (SWIGLU ? (r & 127) : r);
        wofs[i] = (uint32_t)row * rowb + 16u * c;
    }
    uint32_t sofs;
    {
        const int r = 32 * wave + (lane & 31);           /* lanes 32..63 repeat 0..31 */
        const int row = f0 + (SWIGLU ? (r & 127) : r);
        sofs = (uint32_t)row * srow;
    }
    uint32_t bofs[C::NB];
#pragma unroll
    for (int i = 0; i < C::NB; i++) {
        const int j = wave * C::NB + i;                 /* token rows 4 j .. 4 j + 3 */
        const int t = 4 * j + lane / 16;
        const int c = (lane & 15) ^ (t & 15);
        if (t < ntok) {
            const int src = a.row_tok ? a.row_tok[r0 + t] : r0 + t;
            bofs[i] = (uint32_t)src * (uint32_t)K * 2u + 16u * c;
        } else {
            bofs[i] = OOB_OFFSET;
        }
    }
    /* wave-uniform: which matrix each weight load and the scale load read */
    const bool up_s = SWIGLU && wave >= 4;
    auto issue = [&](int stg, uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < C::NW; i++) {
            const bool up = SWIGLU && (wave * C::NW + i) >= 8;
            bdma16(up ? rw3 : rw1, wofs[i], stg * C::WB, buf + 1024 * (wave * C::NW + i));
        }
        bdma4(up_s ? rs3 : rs1, sofs, stg * (C::KS / 32), buf + C::OFF_S + 256 * wave);
#pragma unroll
        for (int i = 0; i < C::NB; i++)
            bdma16(rb, bofs[i], stg * C::KS * 2, buf + C::OFF_B + 1024 * (wave * C::NB + i));
    };

    /* ---- this wave's share: 4 row blocks x 4 token tiles ---- */
    const int wr = wave & 3, wt = wave >> 2;
    int blk[4];
#pragma unroll
    for (int i = 0; i < 4; i++) blk[i] = SWIGLU ? (i < 2 ? 2 * wr + i : 8 + 2 * wr + (i - 2)) : 4 * wr + i;
    int ntw = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) ntw += 64 * wt + 16 * u < ntok ? 1 : 0;

    f4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int u = 0; u < 4; u++) acc[i][u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    unsigned scale_bad = 0;

#pragma unroll
    for (int s0 = 0; s0 < C::NST - 1; s0++) issue(min(s0, last), lds + s0 * C::STAGE);

    auto run = [&](auto ntc) {
        constexpr int NT = decltype(ntc)::value;
        for (int st = 0; st < nst; st++) {
            __builtin_amdgcn_s_waitcnt(0x0F70 | ((C::NST - 2) * C::VM & 15) | ((((C::NST - 2) * C::VM) >> 4) << 14));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            {
                int nb = st + C::NST - 1;
                nb = nb >= C::NST ? nb - C::NST * (nb / C::NST) : nb;
                issue(min(st + C::NST - 1, last), lds + nb * C::STAGE);
            }
            if constexpr (NT > 0) {
                const uint8_t *buf = lds + (st % C::NST) * C::STAGE;
                u32x4 wraw[4];
                float cs[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 16 * blk[i] + rr;
                    wraw[i] = *(const u32x4 *)(buf + r * C::WB + 16 * (gq ^ ((r >> 2) & 3)));
                    const uint32_t sw = *(const uint32_t *)(buf + C::OFF_S + (r >> 5) * 256 + (r & 31) * 4);
                    const uint32_t sb = (sw >> (8 * gq)) & 0xFFu;
                    scale_bad |= (sb - 104u) > 36u;
                    cs[i] = dev_e8m0(sb);
                }
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    h8 bop[NT];
#pragma unroll
                    for (int u = 0; u < NT; u++) {
                        const int t = 64 * wt + 16 * u + rr;
                        bop[u] = *(const h8 *)(buf + C::OFF_B + t * (C::KS * 2) + 16 * ((4 * gq + s) ^ rr));
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t d = s == 0 ? wraw[i].x : s == 1 ? wraw[i].y : s == 2 ? wraw[i].z : wraw[i].w;
                        const h8 av = fp4_h8(d, cs[i]);
#pragma unroll
                        for (int u = 0; u < NT; u++) acc[i][u] = mfma16(av, bop[u], acc[i][u]);
                    }
                }
            }
        }
    };
    switch (ntw) {
    case 4: run(IC<4>{}); break;
    case 3: run(IC<3>{}); break;
    case 2: run(IC<2>{}); break;
    case 1: run(IC<1>{}); break;
    default: run(IC<0>{}); break;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);     /* trailing repeat loads drain before exit */
    if (scale_bad) atomicOr(a.status, ST_SCALE_RANGE);

    unsigned range_bad = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int t = 64 * wt + 16 * u + rr;
        if (t >= ntok) continue;
        const size_t orow = (size_t)(r0 + t) * N;
        const int ex = b_row_exp(a, r0 + t);
        if constexpr (SWIGLU) {
#pragma unroll
            for (int i = 0; i < 2; i++)
                *(uint2 *)((uint16_t *)a.out + orow + f0 + 16 * blk[i] + 4 * gq) =
                    swiglu_f16x4(acc[i][u], acc[i + 2][u], ex, a.limit, range_bad);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                *(f4v *)((float *)a.out + orow + f0 + 16 * blk[i] + 4 * gq) = unscale4(acc[i][u], ex);
        }
    }
    if (range_bad) atomicOr(a.status, range_bad);
}

/* ------------------------------------------------------------- combine --- */

/* 4 consecutive outputs of one token per thread. The positions and weights
 * of all k (topk <= 16) are read first and every Y load is issued before the
 * first is used, so a thread waits one memory latency rather than topk
 * dependent pairs of them; the sum stays in k order. */
__global__ __launch_bounds__(256) void k_moe_combine(CombineArgs a)
{
    constexpr int KMAX = 16;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int q = a.hidden / 4;
    if (i >= (size_t)a.n * q) return;
    const int t = (int)(i / q), c = (int)(i - (size_t)t * q) * 4;
    const int topk = a.topk;
    int p[KMAX];
    float wk[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
        p[k] = k < topk ? a.pos[(size_t)t * topk + k] : -1;
        wk[k] = k < topk ? a.w[(size_t)t * topk + k] : 0.0f;
    }
    f32x4 v[KMAX];
    const float nan = __builtin_nanf("");
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
        if (k < topk && p[k] >= 0) v[k] = *(const f32x4 *)(a.Y + (size_t)p[k] * a.hidden + c);
        else v[k] = f32x4{nan, nan, nan, nan};
    }
    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.YS) s = *(const f32x4 *)(a.YS + (size_t)t * a.hidden + c);
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
        if (k < topk) {
            o.x = __fadd_rn(o.x, __fmul_rn(wk[k], v[k].x));
            o.y = __fadd_rn(o.y, __fmul_rn(wk[k], v[k].y));
            o.z = __fadd_rn(o.z, __fmul_rn(wk[k], v[k].z));
            o.w = __fadd_rn(o.w, __fmul_rn(wk[k], v[k].w));
        }
    }
    if (a.YS) {
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
    const int nch = (a.npairs + 1023) / 1024;
    const int cpb = nch > ROUTE_MAX_BLOCKS ? (nch + ROUTE_MAX_BLOCKS - 1) / ROUTE_MAX_BLOCKS : 1;
    const int blocks = nch > 0 ? (nch + cpb - 1) / cpb : 1;
    if (a.chist && nch >= ROUTE_PRECOUNT_CHUNKS) {
        hipLaunchKernelGGL(k_moe_route_count, dim3(nch), dim3(1024), 0, st, a);
        hipLaunchKernelGGL(k_moe_route<true>, dim3(blocks), dim3(1024), 0, st, a, cpb);
    } else {
        hipLaunchKernelGGL(k_moe_route<false>, dim3(blocks), dim3(1024), 0, st, a, cpb);
    }
    return hipGetLastError();
}

hipError_t to_f16_rows_launch(uint16_t *o, int *ex, const float *x, int rows, int cols,
                              hipStream_t st)
{
    if (rows <= 0 || cols <= 0 || cols % 8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_to_f16_rows, dim3((unsigned)rows), dim3(256), 0, st, o, ex, x, cols);
    return hipGetLastError();
}

int grouped_rows_per_tile(int tt) { return 16 * tt; }

template <int WF, bool SW, int TT, int NS>
static hipError_t grouped2_ns(const GroupedArgs &a, long items, hipStream_t st)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_grouped2<WF, SW, TT, NS>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 G2<WF, TT, NS>::LDS);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    constexpr int lds_bytes = G2<WF, TT, NS>::LDS, threads = 64 * G2<WF, TT, NS>::NWAVE;
    hipLaunchKernelGGL((k_grouped2<WF, SW, TT, NS>), dim3((unsigned)items), dim3(threads), lds_bytes, st, a);
    return hipGetLastError();
}

/* FP8 16-row tiles: when the grid outnumbers the CUs, two stages (2 x 40
 * KiB) so two workgroups share a CU (4096 x 4096 FP8 drop-in matmul, 192
 * tokens in 384 workgroups: 36.1 -> 29.7 us); up to one workgroup per CU the
 * three-stage ring keeps more of a lone workgroup's loads in flight (128
 * tokens 23.7 against 24.3 us, the batched decode's shared expert). */
template <int WF, bool SW, int TT>
static hipError_t grouped2(const GroupedArgs &a, long items, hipStream_t st)
{
    if constexpr (WF != FMT_FP4_E8M0 && TT == 1) {
        static int cus = 0;
        if (cus == 0) {
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
                (void)hipGetLastError();
                cus = 256;
            }
        }
        if (items > cus) return grouped2_ns<WF, SW, TT, 2>(a, items, st);
    }
    return grouped2_ns<WF, SW, TT, g2_stages<WF, TT>()>(a, items, st);
}

template <int WF, bool SW>
static hipError_t grouped_tt(const GroupedArgs &a, int tt, long items, hipStream_t st)
{
    if (a.K % KS == 0) {        /* LDS-staged form: one workgroup per item */
        return tt == 1 ? grouped2<WF, SW, 1>(a, items, st) : grouped2<WF, SW, 4>(a, items, st);
    }
    const dim3 grid((unsigned)((items + 3) / 4)), block(256);
    if (tt == 1) hipLaunchKernelGGL((k_grouped<WF, SW, 1>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((k_grouped<WF, SW, 4>), grid, block, 0, st, a);
    return hipGetLastError();
}

template <bool SW>
static hipError_t grouped3(const GroupedArgs &a, long items, hipStream_t st)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_grouped3<SW>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, G3::LDS);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    constexpr int lds_bytes = G3::LDS, threads = 64 * G3::NWAVE;
    hipLaunchKernelGGL((k_grouped3<SW>), dim3((unsigned)items), dim3(threads), lds_bytes, st, a);
    return hipGetLastError();
}

hipError_t grouped_launch(int fmt, bool swiglu, int tt, const GroupedArgs &a, long max_tiles,
                          hipStream_t st)
{
    if (tt == 8) {
        /* 128-token tiles: FP4 only; byte offsets of every buffer fit 31 bits */
        const int feat = swiglu ? 128 : 256;
        if (fmt != FMT_FP4_E8M0 || a.N % feat || a.K % G3::KS || max_tiles <= 0 || a.nrows <= 0 ||
            (size_t)a.nrows * a.K * 2 >= (1u << 31) || (size_t)a.N * a.K / 2 >= (1u << 31))
            return hipErrorInvalidValue;
        const long items = max_tiles * (a.N / feat);
        return swiglu ? grouped3<true>(a, items, st) : grouped3<false>(a, items, st);
    }
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
