/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_moe_mx.hip - the prefill MoE layer's routed expert GEMMs on CDNA4's
 * block-scaled MFMA: FP4 weights exactly as stored times MXFP8 activations.
 *
 * What it replaces: the per-expert bucket GEMMs of the reference's prefill
 * union path, w1 / w3 -> SwiGLU -> w2 (src/80_prefill/dsv4_prefill_experts.c:
 * 23-77; GPU leg src/80_prefill/dsv4_prefill_vk_expert.c:45-172, whose
 * shaders dequantize through a LUT into fp32).
 *
 * ARITHMETIC
 *   v_mfma_scale_f32_16x16x128_f8f6f4 with the e2m1 weights as the A operand
 *   (cbsz 4) and their E8M0 1x32 scales in the hardware A scale, the tokens
 *   as e4m3 (blgp 0) with one E8M0 scale per 32 reduction indices (MXFP8) in
 *   the hardware B scale: no instruction decodes a weight or an activation,
 *   and the K loop accumulates in the MFMA's fp32 accumulator. FP4 x FP8
 *   issues at the FP8 rate on gfx950 (measured 4.1-4.4 PFLOP/s from
 *   registers, the same as FP8 x FP8). The gate/up form applies SwiGLU (the
 *   reference's asymmetric clamp) to each (w1, w3) pair of results and
 *   quantizes mid to MXFP8 (per token and 32 consecutive features, the rule
 *   of k_quant_act_mxfp8) for the down form's B operand; the down form
 *   writes fp32 rows for the k-order combine. The activations' and mid's
 *   MXFP8 rounding is the only approximation beyond fp32 accumulation: the
 *   oracle for this path quantizes the same activations the same way.
 *
 * SCHEDULE
 *   One workgroup of eight waves per (bucket tile of up to 256 token rows,
 *   slab of 256 weight rows: 128 w1 rows and the matching 128 w3 rows, or
 *   256 w2 rows). Wave (wr, wt) owns weight rows 64 wr .. +63 (gate/up: 32
 *   w1 rows and the same 32 w3 rows) times tokens 128 wt .. +127: 4 x 8
 *   MFMA tiles. K advances in 128-wide stages: 256 weight rows x 64 bytes,
 *   their 256 scale dwords, 256 token rows x 128 bytes and their scale
 *   dwords go global -> LDS by buffer loads straight to LDS (1 KiB per wave
 *   instruction), three stages in flight, 16-byte chunks XOR-swizzled; token
 *   rows past the bucket's end read as zeros (an offset beyond the buffer).
 *   Block b = tile * slabs + slab: the same slab of an expert's consecutive
 *   tiles lands on the same XCD, whose L2 then serves the slab's later reads.
 *
 * OPERANDS (gfx950, measured): of a 128-k stage, A lane l holds row l % 16,
 * k in [32 (l/16), +32) as 16 bytes (low nibble first); B lane l holds token
 * l % 16, k in [16 (l/16), +16) in bytes 0-15 and [64 + 16 (l/16), +16) in
 * bytes 16-31; scale lane l covers row / token l % 16 and the 32-element
 * block l / 16; accumulator element e of lane l is row 4 (l/16) + e, token
 * l % 16.
 *
 * Bound: HBM (the 13.4 MB of each expert's weights) for small buckets, MFMA
 * for large ones.
 */
#include "dsv4_internal.h"

namespace dsv4 {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
template <int N> struct IC { static constexpr int value = N; };

/* Stage geometry for a tile of TOK token rows: 256 weight rows (64 FP4
 * bytes and one scale dword each), TOK token rows (128 e4m3 bytes and one
 * scale dword each) and a 256-byte pad where waves without a scale load
 * land theirs. The fewer the tokens, the smaller a stage and the more stages
 * in flight: a tile of few tokens streams its weights with nothing to hide
 * the latency behind but more loads. */
template <int TOK>
struct GX {
    static constexpr int KS = 128;                     /* reduction indices per stage */
    static constexpr int ROWS = 256, NWAVE = 8;
    static constexpr int WB = KS / 2;                  /* FP4 bytes per weight row per stage */
    static constexpr int OFF_WS = ROWS * WB;
    static constexpr int OFF_B = OFF_WS + ROWS * 4;
    static constexpr int OFF_BS = OFF_B + TOK * KS;
    static constexpr int OFF_PAD = OFF_BS + TOK * 4;
    static constexpr int STAGE = OFF_PAD + 256;
    static constexpr int NST = TOK == 64 ? 6 : TOK == 128 ? 4 : 3;
    static constexpr int LDS = NST * STAGE;
    static constexpr int NW = ROWS * WB / 1024 / NWAVE;   /* 16-row weight loads per wave   */
    static constexpr int NB = TOK * KS / 1024 / NWAVE;    /* 8-row token loads per wave     */
    static constexpr int NBS = TOK / 64;                  /* waves loading token scales     */
    static constexpr int VM = NW + NB + 1;                /* + one scale (or pad) load      */
    static constexpr int NTMAX = TOK / 32;                /* 16-token groups per wave       */
    static_assert(LDS <= 160 * 1024, "LDS ring exceeds 160 KiB");
    static_assert(NW * NWAVE * 1024 == ROWS * WB && NB * NWAVE * 1024 == TOK * KS, "load split");
};
constexpr int GX_TILE = 256;                           /* token rows per bucket tile */
constexpr int GX_LDS = GX<64>::LDS > GX<256>::LDS ? (GX<64>::LDS > GX<128>::LDS ? GX<64>::LDS : GX<128>::LDS)
                                                  : (GX<256>::LDS > GX<128>::LDS ? GX<256>::LDS : GX<128>::LDS);

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

/* LDS slot of logical 16-byte chunk c of staged weight row r / token row t */
__device__ __forceinline__ int wslot(int r, int c) { return c ^ ((r >> 2) & 3); }
__device__ __forceinline__ int bslot(int t, int c) { return c ^ (t & 7); }

__device__ __forceinline__ bool fp4_matches(const DSV4QMat &m, int rows, int cols)
{
    return m.rows == rows && m.cols == cols && m.w && m.s && m.wdt == DSV4_WFP4 && m.blk_r == 1 &&
           m.blk_c == 32 && ((uintptr_t)m.w & 15) == 0 && ((uintptr_t)m.s & 3) == 0;
}

__device__ __forceinline__ f4v mfma_mx(const u32x4 &a, const v8i &b, const f4v &c, int sa, int sb)
{
    v8i av;
    av[0] = (int)a.x; av[1] = (int)a.y; av[2] = (int)a.z; av[3] = (int)a.w;
    av[4] = 0; av[5] = 0; av[6] = 0; av[7] = 0;
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, c, 4, 0, 0, sa, 0, sb);
}

} // namespace

/* One bucket tile (rows r0 .. r0 + ntok - 1, ntok <= TOK) against the
 * workgroup's 256 weight rows from feature f0. */
template <bool SWIGLU, int TOK>
__device__ __forceinline__ void mx_tile(const GroupedMxArgs &a, const DSV4QMat &m1, const DSV4QMat &m3,
                                        int r0, int ntok, int f0, uint8_t *lds)
{
    using C = GX<TOK>;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int rr = lane & 15, gq = lane >> 4;
    const int K = a.K, N = a.N;

    /* ---- load plan: per-lane byte offsets into the buffers ---- */
    const uint32_t rowb = (uint32_t)K / 2, srow = (uint32_t)K / 32;
    const int nst = K / C::KS, last = nst - 1;
    const __amdgpu_buffer_rsrc_t rw1 = buf_rsrc(m1.w, (uint32_t)N * rowb);
    const __amdgpu_buffer_rsrc_t rs1 = buf_rsrc(m1.s, (uint32_t)N * srow);
    const __amdgpu_buffer_rsrc_t rw3 = SWIGLU ? buf_rsrc(m3.w, (uint32_t)N * rowb) : rw1;
    const __amdgpu_buffer_rsrc_t rs3 = SWIGLU ? buf_rsrc(m3.s, (uint32_t)N * srow) : rs1;
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(a.B, (uint32_t)a.nrows * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rbs = buf_rsrc(a.BS, (uint32_t)a.nrows * srow);
    uint32_t wofs[C::NW];
#pragma unroll
    for (int i = 0; i < C::NW; i++) {
        const int j = wave * C::NW + i;                 /* staged rows 16 j .. 16 j + 15 */
        const int r = 16 * j + lane / 4;
        const int row = f0 + (SWIGLU ? (r & 127) : r);
        wofs[i] = (uint32_t)row * rowb + 16u * (uint32_t)wslot(r, lane & 3);
    }
    uint32_t bofs[C::NB];
#pragma unroll
    for (int i = 0; i < C::NB; i++) {
        const int j = wave * C::NB + i;                 /* token rows 8 j .. 8 j + 7 */
        const int t = 8 * j + lane / 8;
        if (t < ntok) {
            const int src = a.row_tok ? a.row_tok[r0 + t] : r0 + t;
            bofs[i] = (uint32_t)src * (uint32_t)K + 16u * (uint32_t)bslot(t, lane & 7);
        } else {
            bofs[i] = OOB_OFFSET;
        }
    }
    /* one 4-byte-per-lane scale load per wave and stage: waves 0-3 the
     * dwords of weight rows 64 w .. +63, waves 4 .. 4 + NBS - 1 those of
     * token rows 64 (w - 4) .. +63, the rest a zero load into the pad (the
     * same count of loads in every wave keeps one vmcnt value for all) */
    uint32_t sofs = OOB_OFFSET;
    bool s_up = false;
    int s_dst = C::OFF_PAD;
    if (wave < 4) {
        const int r = 64 * wave + lane;
        const int row = f0 + (SWIGLU ? (r & 127) : r);
        s_up = SWIGLU && r >= 128;
        sofs = (uint32_t)row * srow;
        s_dst = C::OFF_WS + 256 * wave;
    } else if (wave < 4 + C::NBS) {
        const int t = 64 * (wave - 4) + lane;
        if (t < ntok) sofs = (uint32_t)(a.row_tok ? a.row_tok[r0 + t] : r0 + t) * srow;
        s_dst = C::OFF_BS + 256 * (wave - 4);
    }
    s_up = __builtin_amdgcn_readfirstlane((int)s_up) != 0;
    auto issue = [&](int stg, uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < C::NW; i++) {
            const bool up = SWIGLU && (wave * C::NW + i) >= 8;
            bdma16(up ? rw3 : rw1, wofs[i], stg * C::WB, buf + 1024 * (wave * C::NW + i));
        }
#pragma unroll
        for (int i = 0; i < C::NB; i++)
            bdma16(rb, bofs[i], stg * C::KS, buf + C::OFF_B + 1024 * (wave * C::NB + i));
        if (wave < 4) bdma4(s_up ? rs3 : rs1, sofs, stg * 4, buf + s_dst);
        else bdma4(rbs, sofs, stg * 4, buf + s_dst);
    };

    /* ---- this wave's share: 4 row tiles x NTMAX token groups ---- */
    const int wr = wave & 3, wt = wave >> 2;
    constexpr int HALF = TOK / 2;
    int blk[4];
#pragma unroll
    for (int i = 0; i < 4; i++) blk[i] = SWIGLU ? (i < 2 ? 2 * wr + i : 8 + 2 * wr + (i - 2)) : 4 * wr + i;
    int ntw = 0;
#pragma unroll
    for (int u = 0; u < C::NTMAX; u++) ntw += HALF * wt + 16 * u < ntok ? 1 : 0;

    f4v acc[4][C::NTMAX];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int u = 0; u < C::NTMAX; u++) acc[i][u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
    for (int s0 = 0; s0 < C::NST - 1; s0++) issue(min(s0, last), lds + s0 * C::STAGE);

    auto run = [&](auto ntc) {
        constexpr int NT = decltype(ntc)::value;
        for (int st = 0; st < nst; st++) {
            /* this wave's loads of stage st have landed (the NST - 2 later
             * stages may be in flight); the barrier makes that true for the
             * whole workgroup and frees the stage read in iteration st - 1 */
            __builtin_amdgcn_s_waitcnt(0x0F70 | ((C::NST - 2) * C::VM & 15) |
                                       ((((C::NST - 2) * C::VM) >> 4) << 14));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            {
                int nb = st + C::NST - 1;
                nb = nb >= C::NST ? nb - C::NST * (nb / C::NST) : nb;
                issue(min(st + C::NST - 1, last), lds + nb * C::STAGE);
            }
            if constexpr (NT > 0) {
                const uint8_t *buf = lds + (st % C::NST) * C::STAGE;
                u32x4 aw[4];
                int sa[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 16 * blk[i] + rr;
                    aw[i] = *(const u32x4 *)(buf + r * C::WB + 16 * wslot(r, gq));
                    sa[i] = (int)((*(const uint32_t *)(buf + C::OFF_WS + 4 * r) >> (8 * gq)) & 0xFFu);
                }
#pragma unroll
                for (int u = 0; u < NT; u++) {
                    const int t = HALF * wt + 16 * u + rr;
                    const uint8_t *brow = buf + C::OFF_B + t * C::KS;
                    const u32x4 lo = *(const u32x4 *)(brow + 16 * bslot(t, gq));
                    const u32x4 hi = *(const u32x4 *)(brow + 16 * bslot(t, 4 + gq));
                    const int sb = (int)((*(const uint32_t *)(buf + C::OFF_BS + 4 * t) >> (8 * gq)) & 0xFFu);
                    v8i b;
                    b[0] = (int)lo.x; b[1] = (int)lo.y; b[2] = (int)lo.z; b[3] = (int)lo.w;
                    b[4] = (int)hi.x; b[5] = (int)hi.y; b[6] = (int)hi.z; b[7] = (int)hi.w;
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i][u] = mfma_mx(aw[i], b, acc[i][u], sa[i], sb);
                }
            }
        }
    };
    if constexpr (C::NTMAX >= 8) { if (ntw == 8) run(IC<8>{}); else if (ntw == 7) run(IC<7>{});
                                   else if (ntw == 6) run(IC<6>{}); else if (ntw == 5) run(IC<5>{}); }
    if constexpr (C::NTMAX >= 4) { if (ntw == 4) run(IC<4>{}); else if (ntw == 3) run(IC<3>{}); }
    if constexpr (C::NTMAX >= 2) { if (ntw == 2) run(IC<2>{}); else if (ntw == 1) run(IC<1>{}); }
    if (ntw == 0) run(IC<0>{});
    __builtin_amdgcn_s_waitcnt(0x0F70);     /* trailing repeat loads drain before exit */

#pragma unroll
    for (int u = 0; u < C::NTMAX; u++) {
        const int t = HALF * wt + 16 * u + rr;
        const bool live = t < ntok;
        const size_t row = (size_t)(r0 + (live ? t : 0));
        if constexpr (SWIGLU) {
            /* mid for features f0 + 32 wr + 16 i + 4 gq + e (i = 0, 1) of token
             * row t; its 32-feature MXFP8 block is this wave's whole share of
             * the row, spread over the four lanes rr, rr + 16, rr + 32, rr + 48 */
            float m[2][4];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    m[i][e] = dev_swiglu(acc[i][u][e], acc[i + 2][u][e], a.limit);
                    const float v = __builtin_fabsf(m[i][e]);
                    amax = v > amax ? v : amax;
                }
            amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
            const uint32_t sbyte = mxfp8_scale_byte(amax);
            const int se = (int)sbyte - 127;
            if (live) {
                const int fb = f0 + 32 * wr;
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const uint32_t q = hw_e4m3(ldexpf(m[i][0], -se)) | (hw_e4m3(ldexpf(m[i][1], -se)) << 8) |
                                       (hw_e4m3(ldexpf(m[i][2], -se)) << 16) |
                                       (hw_e4m3(ldexpf(m[i][3], -se)) << 24);
                    *(uint32_t *)((uint8_t *)a.out + row * N + fb + 16 * i + 4 * gq) = q;
                }
                if (gq == 0) a.out_s[row * (size_t)(N / 32) + fb / 32] = (uint8_t)sbyte;
            }
        } else {
            if (live) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    *(f4v *)((float *)a.out + row * N + f0 + 16 * blk[i] + 4 * gq) = acc[i][u];
            }
        }
    }
}

template <bool SWIGLU>
__global__ __launch_bounds__(512) void k_grouped_mx(GroupedMxArgs a)
{
    constexpr int FEAT = SWIGLU ? 128 : 256;           /* output features per workgroup */
    extern __shared__ __align__(16) uint8_t lds[];
    const int nslab = a.N / FEAT;
    const int tile = blockIdx.x / nslab, slab = blockIdx.x - tile * nslab;
    const int E = a.n_experts;
    if (tile >= ld_uniform(a.tile_pre, E)) return;            /* whole workgroup */
    const int grp = ld_uniform(a.tile_grp, tile);
    const int go = ld_uniform(a.grp_off, grp), ge = ld_uniform(a.grp_off, grp + 1);
    const int r0 = go + (tile - ld_uniform(a.tile_pre, grp)) * GX_TILE;
    const int ntok = min(GX_TILE, ge - r0);
    const DSV4ExpertW ex = ld_uniform(a.table, grp);
    const DSV4QMat m1 = SWIGLU ? ex.w1 : ex.w2, m3 = ex.w3;
    const int f0 = slab * FEAT;
    const int K = a.K, N = a.N;

    if (!fp4_matches(m1, N, K) || (SWIGLU && !fp4_matches(m3, N, K))) {
        if (threadIdx.x == 0) atomicOr(a.status, ST_BAD_DESCRIPTOR);
        const float nan = __builtin_nanf("");
        for (int i = threadIdx.x; i < ntok * FEAT; i += 512) {
            const size_t o = (size_t)(r0 + i / FEAT) * N + f0 + i % FEAT;
            if constexpr (SWIGLU) {
                ((uint8_t *)a.out)[o] = 0x7F;                             /* e4m3 NaN */
                if ((i % FEAT) % 32 == 0) a.out_s[o / 32] = 127;
            } else {
                ((float *)a.out)[o] = nan;
            }
        }
        return;
    }
    if (ntok <= 64) mx_tile<SWIGLU, 64>(a, m1, m3, r0, ntok, f0, lds);
    else if (ntok <= 128) mx_tile<SWIGLU, 128>(a, m1, m3, r0, ntok, f0, lds);
    else mx_tile<SWIGLU, 256>(a, m1, m3, r0, ntok, f0, lds);
}

int grouped_mx_rows_per_tile() { return GX_TILE; }

template <bool SW>
static hipError_t grouped_mx_k(const GroupedMxArgs &a, long items, hipStream_t st)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_grouped_mx<SW>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, GX_LDS);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    hipLaunchKernelGGL((k_grouped_mx<SW>), dim3((unsigned)items), dim3(512), GX_LDS, st, a);
    return hipGetLastError();
}

hipError_t grouped_mx_launch(bool swiglu, const GroupedMxArgs &a, long max_tiles, hipStream_t st)
{
    const int feat = swiglu ? 128 : 256;
    if (!a.table || a.N % feat || a.K % 128 || max_tiles <= 0 || a.nrows <= 0 ||
        (swiglu && !a.out_s) || (size_t)a.nrows * a.K >= (1u << 31) ||
        (size_t)a.N * a.K / 2 >= (1u << 31))
        return hipErrorInvalidValue;
    const long items = max_tiles * (a.N / feat);
    return swiglu ? grouped_mx_k<true>(a, items, st) : grouped_mx_k<false>(a, items, st);
}

} // namespace dsv4
