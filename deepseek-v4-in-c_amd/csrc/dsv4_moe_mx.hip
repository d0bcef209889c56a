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
 *   Work item = (bucket tile of up to 256 token rows, slab of 256 weight
 *   rows: 128 w1 rows and the matching 128 w3 rows, or 256 w2 rows). K
 *   advances in 128-wide stages. Two kernels split the tiles by size; each
 *   returns at once from the other's tiles.
 *
 *   Thin tiles (at most 64 token rows: under Zipf routing most experts'
 *   buckets) are bound by streaming the slab's weights, which nothing
 *   reuses. k_grouped_mx_thin runs four waves per workgroup and two
 *   workgroups per CU; wave w owns four 16-row weight tiles and loads their
 *   FP4 bytes and scale dwords global -> VGPR itself, four stages ahead, so
 *   weights never pass through LDS. Only the tile's tokens, which all four
 *   waves multiply, are staged in LDS (buffer loads straight to LDS, a
 *   five-slot ring, one barrier per stage).
 *
 *   Fat tiles (65-256 rows) are bound by the MFMA. k_grouped_mx runs eight
 *   waves: wave (wr, wt) owns weight rows 64 wr .. +63 (gate/up: 32 w1 rows
 *   and the same 32 w3 rows) times half of the tile's tokens. Weights,
 *   tokens and both scale sets of a stage go global -> LDS by buffer loads
 *   straight to LDS (1 KiB per wave instruction), three or four stages in
 *   flight, 16-byte chunks XOR-swizzled.
 *
 *   In both, token rows past the bucket's end read as zeros (an offset
 *   beyond the buffer). Work item b = tile * slabs + slab: workgroups are
 *   dealt to the eight XCDs round robin, so the same slab of an expert's
 *   consecutive tiles lands on one XCD, whose L2 then serves that slab's
 *   weights to the later tiles.
 *
 * OPERANDS (gfx950, measured): of a 128-k stage, A lane l holds row l % 16,
 * k in [32 (l/16), +32) as 16 bytes (low nibble first); B lane l holds token
 * l % 16, k in [16 (l/16), +16) in bytes 0-15 and [64 + 16 (l/16), +16) in
 * bytes 16-31; scale lane l covers row / token l % 16 and the 32-element
 * block l / 16; accumulator element e of lane l is row 4 (l/16) + e, token
 * l % 16.
 *
 * Bound: HBM (the 13.4 MB of each expert's weights) for thin tiles, MFMA
 * for fat ones.
 */
#include "dsv4_internal.h"

namespace dsv4 {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
template <int N> struct IC { static constexpr int value = N; };

/* f(IC<I>{}) for I = B .. E - 1, in order, each a compile-time constant */
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (B < E) {
        f(IC<B>{});
        static_for<B + 1, E>(f);
    }
}

/* Stage geometry of the fat kernel for a tile of TOK token rows: 256 weight
 * rows (64 FP4 bytes and one scale dword each), TOK token rows (128 e4m3
 * bytes and one scale dword each) and a 256-byte pad where waves without a
 * scale load land theirs. */
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
    static constexpr int NST = TOK == 128 ? 4 : 3;
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
constexpr int GX_LDS = GX<256>::LDS > GX<128>::LDS ? GX<256>::LDS : GX<128>::LDS;

/* Thin kernel: tiles of at most TH_TOK rows. A stage covers 256 reduction
 * indices as two 128-wide halves, TH_D stages in flight. LDS holds a ring of
 * TH_D + 1 token stages (two halves of 128 bytes per token) and two groups
 * of the tokens' scale dwords (one dword per half, 2 TH_G per token and
 * group). */
constexpr int TH_TOK = 64;
constexpr int TH_D = 2;                                /* stages in flight             */
constexpr int TH_G = 2;                                /* stages per scale group       */
constexpr int TH_SB = 2;                               /* scale groups per weight-scale block */
constexpr int TH_B = TH_TOK * 128;                     /* token bytes of a half        */
constexpr int TH_SLOT = 2 * TH_B;                      /* token bytes of a stage       */
constexpr int TH_LDS = (TH_D + 1) * TH_SLOT + 2 * 1024;   /* token ring + 2 scale groups */
constexpr int TH_KQ = 256 * TH_G * TH_SB;              /* K granule of the thin kernel */

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

/* s_waitcnt vmcnt(n), other counters untouched (gfx9 encoding, n < 64) */
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

/* LDS slot of logical 16-byte chunk c of staged weight row r / token row t */
__device__ __forceinline__ int wslot(int r, int c) { return c ^ ((r >> 1) & 3); }
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

/* B operand of token row t of a staged stage (128 swizzled bytes per row)
 * and its scale byte for this lane's 32-element block gq */
__device__ __forceinline__ v8i b_operand(const uint8_t *rows, int t, int gq)
{
    const uint8_t *brow = rows + t * 128;
    const u32x4 lo = *(const u32x4 *)(brow + 16 * bslot(t, gq));
    const u32x4 hi = *(const u32x4 *)(brow + 16 * bslot(t, 4 + gq));
    v8i b;
    b[0] = (int)lo.x; b[1] = (int)lo.y; b[2] = (int)lo.z; b[3] = (int)lo.w;
    b[4] = (int)hi.x; b[5] = (int)hi.y; b[6] = (int)hi.z; b[7] = (int)hi.w;
    return b;
}
__device__ __forceinline__ int scale_byte(uint32_t dword, int gq) { return (int)((dword >> (8 * gq)) & 0xFFu); }

} // namespace

/* Bucket tile and slab of this workgroup's work item; false past the last
 * tile (tiles run to tile_pre[E]). */
struct MxItem {
    int r0, ntok, grp, f0;
};
template <int FEAT>
__device__ __forceinline__ bool mx_item(const GroupedMxArgs &a, MxItem &it)
{
    const int nslab = a.N / FEAT;
    const int tile = blockIdx.x / nslab, slab = blockIdx.x - tile * nslab;
    const int E = a.n_experts;
    const int ntiles = ld_uniform(a.tile_pre, E);
    const TileRec tr = ld_uniform(a.tile_rec, tile);      /* read beside the count: one round trip */
    if ((tile >= ntiles) | (tr.ntok <= 0)) return false;
    it.r0 = tr.r0;
    it.ntok = tr.ntok;
    it.grp = tr.grp;
    it.f0 = slab * FEAT;
    return true;
}

/* A tile whose expert fails the descriptor check: flag it, fill its outputs
 * with NaN (e4m3 0x7F with a unit scale for mid). */
template <bool SWIGLU, int FEAT, int NTHR>
__device__ void mx_fill_bad(const GroupedMxArgs &a, const MxItem &it)
{
    if (threadIdx.x == 0) atomicOr(a.status, ST_BAD_DESCRIPTOR);
    const float nan = __builtin_nanf("");
    for (int i = threadIdx.x; i < it.ntok * FEAT; i += NTHR) {
        const size_t o = (size_t)(it.r0 + i / FEAT) * a.N + it.f0 + i % FEAT;
        if constexpr (SWIGLU) {
            ((uint8_t *)a.out)[o] = 0x7F;
            if ((i % FEAT) % 32 == 0) a.out_s[o / 32] = 127;
        } else {
            ((float *)a.out)[o] = nan;
        }
    }
}

/* One wave's results. acc[i][u] element e is token row t0 + 16 u + (lane &
 * 15) of the tile times weight row 4 (lane >> 4) + e of the wave's row tile
 * i. Gate/up: tiles 0, 1 are w1 rows fw + 16 i and tiles 2, 3 the w3 rows of
 * the same features; mid = SwiGLU, quantized to MXFP8 with the 32-feature
 * block fw .. fw + 31 (the wave's whole share of the row, spread over lanes
 * rr, rr + 16, rr + 32, rr + 48). Down: tile i is output features
 * fw + 16 i, written as fp32. */
template <bool SWIGLU, int NU>
__device__ __forceinline__ void mx_store(const GroupedMxArgs &a, const f4v (&acc)[4][NU], int r0, int ntok,
                                         int t0, int fw)
{
    const int lane = threadIdx.x & 63;
    const int rr = lane & 15, gq = lane >> 4;
    const int N = a.N;
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int t = t0 + 16 * u + rr;
        const bool live = t < ntok;
        const size_t row = (size_t)(r0 + (live ? t : 0));
        if constexpr (SWIGLU) {
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
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const uint32_t q = hw_e4m3(ldexpf(m[i][0], -se)) | (hw_e4m3(ldexpf(m[i][1], -se)) << 8) |
                                       (hw_e4m3(ldexpf(m[i][2], -se)) << 16) |
                                       (hw_e4m3(ldexpf(m[i][3], -se)) << 24);
                    *(uint32_t *)((uint8_t *)a.out + row * N + fw + 16 * i + 4 * gq) = q;
                }
                if (gq == 0) a.out_s[row * (size_t)(N / 32) + fw / 32] = (uint8_t)sbyte;
            }
        } else {
            if (live) {
#pragma unroll
                for (int i = 0; i < 4; i++) *(f4v *)((float *)a.out + row * N + fw + 16 * i + 4 * gq) = acc[i][u];
            }
        }
    }
}

/* ------------------------------------------------------------------------
 * Fat tiles: rows r0 .. r0 + ntok - 1 (ntok <= TOK) against the
 * workgroup's 256 weight rows from feature f0, everything staged in LDS.
 * ---------------------------------------------------------------------- */
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
    /* Waves 0-3 stage w1 rows (or w2 rows 0-127), waves 4-7 w3 rows (or w2
     * rows 128-255), so each wave needs one weight descriptor. Descriptors
     * are built from pointers chosen by value: a conditional between two
     * descriptor variables compiles to a select of their addresses, which
     * keeps them in scratch memory, and every buffer load then becomes a
     * readfirstlane loop whose scratch reads wait out all loads in flight. */
    static_assert(C::NW * 16 * 4 == 128, "waves 0-3 stage weight rows 0-127");
    const bool w_up = SWIGLU && wave >= 4;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(w_up ? m3.w : m1.w, (uint32_t)N * rowb);
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(a.B, (uint32_t)a.nrows * (uint32_t)K);
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
    int s_dst = C::OFF_PAD;
    const void *sbase = a.BS;
    uint32_t sbytes = (uint32_t)a.nrows * srow;
    if (wave < 4) {
        const int r = 64 * wave + lane;
        const int row = f0 + (SWIGLU ? (r & 127) : r);
        sbase = SWIGLU && wave >= 2 ? m3.s : m1.s;     /* staged rows 128-255 are w3's */
        sbytes = (uint32_t)N * srow;
        sofs = (uint32_t)row * srow;
        s_dst = C::OFF_WS + 256 * wave;
    } else if (wave < 4 + C::NBS) {
        const int t = 64 * (wave - 4) + lane;
        if (t < ntok) sofs = (uint32_t)(a.row_tok ? a.row_tok[r0 + t] : r0 + t) * srow;
        s_dst = C::OFF_BS + 256 * (wave - 4);
    }
    const __amdgpu_buffer_rsrc_t rsc = buf_rsrc(sbase, sbytes);
    /* Stages past the last are issued as out-of-range loads (zeros, no
     * memory traffic) into a slot nobody reads: every wave and stage keeps
     * the same count of loads. Re-reading the last stage instead cost an
     * L2 fetch per repeat, the lines having been evicted by then. */
    auto issue = [&](int stg, uint8_t *buf) {
        const uint32_t oob = stg > last ? OOB_OFFSET : 0u;
        stg = min(stg, last);
#pragma unroll
        for (int i = 0; i < C::NW; i++)
            bdma16(rw, wofs[i] | oob, stg * C::WB, buf + 1024 * (wave * C::NW + i));
#pragma unroll
        for (int i = 0; i < C::NB; i++)
            bdma16(rb, bofs[i] | oob, stg * C::KS, buf + C::OFF_B + 1024 * (wave * C::NB + i));
        bdma4(rsc, sofs | oob, stg * 4, buf + s_dst);
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
    for (int s0 = 0; s0 < C::NST - 1; s0++) issue(s0, lds + s0 * C::STAGE);

    auto run = [&](auto ntc) {
        constexpr int NT = decltype(ntc)::value;
        for (int st = 0; st < nst; st++) {
            /* this wave's loads of stage st have landed (the NST - 2 later
             * stages may be in flight); the barrier makes that true for the
             * whole workgroup and frees the stage read in iteration st - 1 */
            wait_vm<(C::NST - 2) * C::VM>();
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            {
                int nb = st + C::NST - 1;
                nb = nb >= C::NST ? nb - C::NST * (nb / C::NST) : nb;
                issue(st + C::NST - 1, lds + nb * C::STAGE);
            }
            if constexpr (NT > 0) {
                /* Operands from LDS one token group ahead: the reads of
                 * group u + 1 are issued before the MFMAs of group u, so
                 * those MFMAs wait only for group u's reads. */
                const uint8_t *buf = lds + (st % C::NST) * C::STAGE;
                u32x4 aw[4];
                uint32_t swd[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 16 * blk[i] + rr;
                    aw[i] = *(const u32x4 *)(buf + r * C::WB + 16 * wslot(r, gq));
                    swd[i] = *(const uint32_t *)(buf + C::OFF_WS + 4 * r);
                }
                v8i bq[2];
                uint32_t bsd[2];
                {
                    const int t = HALF * wt + rr;
                    bq[0] = b_operand(buf + C::OFF_B, t, gq);
                    bsd[0] = *(const uint32_t *)(buf + C::OFF_BS + 4 * t);
                }
                DSV4_ORDER();
                int sa[4];
#pragma unroll
                for (int i = 0; i < 4; i++) sa[i] = scale_byte(swd[i], gq);
                static_for<0, NT>([&](auto uc) {
                    constexpr int u = decltype(uc)::value;
                    if constexpr (u + 1 < NT) {
                        const int t = HALF * wt + 16 * (u + 1) + rr;
                        bq[(u + 1) & 1] = b_operand(buf + C::OFF_B, t, gq);
                        bsd[(u + 1) & 1] = *(const uint32_t *)(buf + C::OFF_BS + 4 * t);
                    }
                    DSV4_ORDER();
                    const int sb = scale_byte(bsd[u & 1], gq);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i][u] = mfma_mx(aw[i], bq[u & 1], acc[i][u], sa[i], sb);
                    DSV4_ORDER();
                });
            }
        }
    };
    if constexpr (C::NTMAX >= 8) { if (ntw == 8) run(IC<8>{}); else if (ntw == 7) run(IC<7>{});
                                   else if (ntw == 6) run(IC<6>{}); else if (ntw == 5) run(IC<5>{}); }
    if constexpr (C::NTMAX >= 4) { if (ntw == 4) run(IC<4>{}); else if (ntw == 3) run(IC<3>{}); }
    if constexpr (C::NTMAX >= 2) { if (ntw == 2) run(IC<2>{}); else if (ntw == 1) run(IC<1>{}); }
    if (ntw == 0) run(IC<0>{});
    wait_vm<0>();                           /* trailing repeat loads drain before exit */

    mx_store<SWIGLU, C::NTMAX>(a, acc, r0, ntok, HALF * wt, SWIGLU ? f0 + 32 * wr : f0 + 64 * wr);
}

template <bool SWIGLU>
__global__ __launch_bounds__(512) void k_grouped_mx(GroupedMxArgs a, int thin_rows)
{
    constexpr int FEAT = SWIGLU ? 128 : 256;           /* output features per workgroup */
    extern __shared__ __align__(16) uint8_t lds[];
    MxItem it;
    if (!mx_item<FEAT>(a, it) || it.ntok <= thin_rows) return;     /* whole workgroup */
    const DSV4ExpertW ex = ld_uniform(a.table, it.grp);
    const DSV4QMat m1 = SWIGLU ? ex.w1 : ex.w2, m3 = ex.w3;
    if (!fp4_matches(m1, a.N, a.K) || (SWIGLU && !fp4_matches(m3, a.N, a.K))) {
        mx_fill_bad<SWIGLU, FEAT, 512>(a, it);
        return;
    }
    if (it.ntok <= 128) mx_tile<SWIGLU, 128>(a, m1, m3, it.r0, it.ntok, it.f0, lds);
    else mx_tile<SWIGLU, 256>(a, m1, m3, it.r0, it.ntok, it.f0, lds);
}

/* ------------------------------------------------------------------------
 * Thin tiles: rows r0 .. r0 + ntok - 1, ntok <= 16 NTG <= 64. Wave w owns
 * row tiles i = 0..3: gate/up w1 rows f0 + 32 w + 16 i (i = 0, 1) and the
 * w3 rows of the same features (i = 2, 3); down w2 rows f0 + 64 w + 16 i.
 * A stage is 256 reduction indices, two 128-wide halves: 128 bytes of each
 * weight row, one cache line. A row tile's stage is loaded by two
 * instructions that each read 8 whole lines (rows 2 r' + j of the tile for
 * instruction j; lane 16 g + 2 r' + h takes bytes 64 h + 16 g of its row);
 * a lane-pair exchange (DPP) then forms the MFMA operand of each half, in
 * which lane 16 g + r holds bytes 64 h + 16 g of row r. Half-line loads (16
 * rows x 64 bytes per instruction) made the L2 fetch many lines twice.
 * Weight scales move once per block of TH_SB groups of TH_G stages: lane
 * (rr, gq) loads the 16 scale bytes of group gq of the block for row rr, so
 * one instruction reads 64 contiguous bytes of each of 16 rows. At a group's
 * first stage ds_bpermute hands every lane of row rr the dwords of that
 * group (lane (rr, gq) then takes byte gq of dword c for half c). Loading a
 * group's 16 bytes per row at every group instead touched each row's scale
 * line once per group, and the L2, which turns over several times between
 * two groups, fetched the line again each time (about 0.7 GB of extra reads
 * for the gate/up weights of 194 experts at K = 4096). The tokens' scale
 * dwords are one 4-byte-per-lane load per wave and group (wave w stages
 * dword w of every token).
 * ---------------------------------------------------------------------- */
template <bool SWIGLU, int NTG>
__device__ __forceinline__ void thin_tile(const GroupedMxArgs &a, const DSV4QMat &m1, const DSV4QMat &m3,
                                          int r0, int ntok, int f0, uint8_t *lds)
{
    constexpr int D = TH_D, G = TH_G, SB = TH_SB, U = G * SB;
    static_assert(U % D == 0 && D <= G, "ring depth");
    static_assert(2 * G == 4, "a scale group is four 128-wide halves: 16 scale bytes per row, one dword per wave");
    constexpr int NBL = (2 * NTG + 3) / 4;           /* 8-token loads per wave and half  */
    constexpr int VMW = 8 + 2 * NBL;                 /* VMEM per wave and stage            */
    constexpr int VMG = 1;                           /* + per group: token scales          */
    constexpr int VMB = 4;                           /* + per block: weight scales         */
    static_assert((D - 1) * VMW + VMG + VMB < 64, "vmcnt range");
    const int lane = threadIdx.x & 63, wave = wave_in_group();
    const int rr = lane & 15, gq = lane >> 4;
    const int K = a.K, N = a.N;
    const uint32_t rowb = (uint32_t)K / 2, srow = (uint32_t)K / 32;
    const int nst = K / 256, last = nst - 1, glast = nst / G - 1, blast = nst / U - 1;

    const uint32_t wbytes = (uint32_t)N * rowb, sbytes = (uint32_t)N * srow;
    const uint32_t bbytes = (uint32_t)a.nrows * (uint32_t)K, bsbytes = (uint32_t)a.nrows * srow;
    const void *const w3p = SWIGLU ? m3.w : m1.w, *const s3p = SWIGLU ? m3.s : m1.s;

    /* weights: instruction j of tile i, lane 16 g + 2 r' + h reads 16 bytes
     * of row 2 r' + j at byte 64 h + 16 g of the stage's 128; scales: lane
     * (rr, gq) the 16 scale bytes of group gq of a block of row rr */
    uint32_t wo[4][2], so[4];
    const bool odd = lane & 1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int base = f0 + (SWIGLU ? 32 * wave + 16 * (i & 1) : 64 * wave + 16 * i);
#pragma unroll
        for (int j = 0; j < 2; j++)
            wo[i][j] = (uint32_t)(base + 2 * (rr >> 1) + j) * rowb + 64u * (uint32_t)(lane & 1) +
                       16u * (uint32_t)gq;
        so[i] = (uint32_t)(base + rr) * srow + 16u * (uint32_t)(gq % SB);   /* lanes gq >= SB repeat */
    }
    /* tokens: load q = NBL w + j of a half stages token rows 8 q .. 8 q + 7 */
    uint32_t bo[NBL];
#pragma unroll
    for (int j = 0; j < NBL; j++) {
        const int q = NBL * wave + j;
        const int t = 8 * q + lane / 8;
        bo[j] = OOB_OFFSET;
        if (t < ntok) bo[j] = (uint32_t)(a.row_tok ? a.row_tok[r0 + t] : r0 + t) * (uint32_t)K +
                              16u * (uint32_t)bslot(t, lane & 7);
    }
    /* token scales: lane t, dword w of the group */
    uint32_t bso = OOB_OFFSET;
    if (lane < ntok) bso = (uint32_t)(a.row_tok ? a.row_tok[r0 + lane] : r0 + lane) * srow + 4u * (uint32_t)wave;
    uint8_t *const gs = lds + (D + 1) * TH_SLOT;      /* two group slots of [2 G][64] dwords */

    f4v acc[4][NTG];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int u = 0; u < NTG; u++) acc[i][u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4 aw[D][2][4];                               /* stage s in slot s % D: [instruction][tile] */
    u32x4 wsb[4];                                    /* the weight-scale block being used */
    uint32_t ws[4];                                  /* the current group's scale bytes of lane (rr, gq): byte c for half c */

    /* The loads of stage t: weights into slot t % D (both halves of a row
     * tile back to back), at the first stage of a group that group's scales,
     * then the tokens of both halves into LDS slot lslot. Stages past the
     * last are out-of-range loads (zeros, no memory traffic), so every wave
     * and stage issues the same count of loads without fetching the last
     * stage's lines again. */
    auto issue = [&](int t, int lslot, u32x4 (&w)[2][4], uint8_t *gslot, bool group, bool block) {
        /* past the last stage every buffer is empty: each load is out of range */
        const uint32_t live = t > last ? 0u : 1u;
        const __amdgpu_buffer_rsrc_t rw1 = buf_rsrc(m1.w, live * wbytes), rw3 = buf_rsrc(w3p, live * wbytes);
        const __amdgpu_buffer_rsrc_t rb = buf_rsrc(a.B, live * bbytes);
        const int tc = min(t, last);
        w[0][0] = __builtin_amdgcn_raw_buffer_load_b128(rw1, wo[0][0], tc * 128, 0);
        w[1][0] = __builtin_amdgcn_raw_buffer_load_b128(rw1, wo[0][1], tc * 128, 0);
        w[0][1] = __builtin_amdgcn_raw_buffer_load_b128(rw1, wo[1][0], tc * 128, 0);
        w[1][1] = __builtin_amdgcn_raw_buffer_load_b128(rw1, wo[1][1], tc * 128, 0);
        w[0][2] = __builtin_amdgcn_raw_buffer_load_b128(rw3, wo[2][0], tc * 128, 0);
        w[1][2] = __builtin_amdgcn_raw_buffer_load_b128(rw3, wo[2][1], tc * 128, 0);
        w[0][3] = __builtin_amdgcn_raw_buffer_load_b128(rw3, wo[3][0], tc * 128, 0);
        w[1][3] = __builtin_amdgcn_raw_buffer_load_b128(rw3, wo[3][1], tc * 128, 0);
        if (block) {
            const __amdgpu_buffer_rsrc_t rs1 = buf_rsrc(m1.s, live * sbytes), rs3 = buf_rsrc(s3p, live * sbytes);
            const int b = min(t / U, blast);
            wsb[0] = __builtin_amdgcn_raw_buffer_load_b128(rs1, so[0], b * (16 * SB), 0);
            wsb[1] = __builtin_amdgcn_raw_buffer_load_b128(rs1, so[1], b * (16 * SB), 0);
            wsb[2] = __builtin_amdgcn_raw_buffer_load_b128(rs3, so[2], b * (16 * SB), 0);
            wsb[3] = __builtin_amdgcn_raw_buffer_load_b128(rs3, so[3], b * (16 * SB), 0);
        }
        if (group) bdma4(buf_rsrc(a.BS, live * bsbytes), bso, min(t / G, glast) * 16, gslot + 256 * wave);
        uint8_t *buf = lds + lslot * TH_SLOT;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < NBL; j++)
                bdma16(rb, bo[j], tc * 256 + h * 128, buf + h * TH_B + 1024 * (NBL * wave + j));
    };

#pragma unroll
    for (int t = 0; t < D; t++) {
        issue(t, t, aw[t], gs + ((t / G) & 1) * 1024, t % G == 0, t % U == 0);
        asm volatile("" ::: "memory");
    }

    int slot = 0;                                    /* LDS slot of the stage computed next */
    for (int s0 = 0; s0 < nst; s0 += U) {
        static_for<0, U>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            /* the loads of stage s = s0 + q were issued D stages ago; those
             * of the D - 1 stages after it may still be in flight. After the
             * barrier every wave's tokens of stage s are in LDS and no wave
             * still reads the LDS slot of stage s - 1, which stage s + D
             * reuses (likewise the scale group slot two groups back) */
            wait_vm<(D - 1) * VMW + VMG * (((q % G) + D - 1) / G) + VMB * (((q % U) + D - 1) / U)>();
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            constexpr int p = (q / G) & 1;
            if constexpr (q % G == 0) {
                /* the group's scale dwords of row rr, from lane (rr, group);
                 * of dword c this lane keeps byte gq, packed as byte c */
                const int src = 4 * (rr + 16 * (q / G));
                const uint32_t sel_lo = (uint32_t)gq | (uint32_t)(4 + gq) << 8 | 0x0C0C0000u;
                const uint32_t sel_hi = 0x00000C0Cu | (uint32_t)gq << 16 | (uint32_t)(4 + gq) << 24;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t d[4];
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        uint32_t w = wsb[i][c];
                        asm volatile("" : "+v"(w));
                        d[c] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)w);
                    }
                    ws[i] = __builtin_amdgcn_perm(d[1], d[0], sel_lo) | __builtin_amdgcn_perm(d[3], d[2], sel_hi);
                }
            }
            /* operands of both halves: an even lane keeps its own dword of
             * instruction 0 (half 0) and takes its odd neighbour's (half 1);
             * an odd lane keeps its own of instruction 1 (half 1) and takes
             * its even neighbour's (half 0) */
            u32x4 ah[2][4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const u32x4 &x0 = aw[q % D][0][i], &x1 = aw[q % D][1][i];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t s0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x0[e], DPP_QUAD_1032, 0xF, 0xF, false);
                    const uint32_t s1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x1[e], DPP_QUAD_1032, 0xF, 0xF, false);
                    ah[0][i][e] = odd ? s1 : x0[e];
                    ah[1][i][e] = odd ? x1[e] : s0;
                }
            }
            static_for<0, 2>([&](auto hc) {
                constexpr int h = decltype(hc)::value;
                constexpr int c = 2 * (q % G) + h;   /* 128-wide half within the scale group */
                const uint8_t *bb = lds + slot * TH_SLOT + h * TH_B;
                /* The scale bytes are extracted here and not earlier: an
                 * empty asm that takes each scale dword pins the extraction
                 * (and the wait for its load) behind this stage's barrier,
                 * where the scheduler would otherwise hoist it into an
                 * earlier stage and wait out the loads of the stages
                 * between. */
                int sa[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t w = ws[i];
                    asm volatile("" : "+v"(w));
                    sa[i] = (int)((w >> (8 * c)) & 0xFFu);
                }
                const uint8_t *gsl = gs + p * 1024 + 256 * c;
#pragma unroll
                for (int u = 0; u < NTG; u++) {
                    const int t = 16 * u + rr;
                    const v8i b = b_operand(bb, t, gq);
                    const int sb = scale_byte(*(const uint32_t *)(gsl + 4 * t), gq);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i][u] = mfma_mx(ah[h][i], b, acc[i][u], sa[i], sb);
                }
            });
            asm volatile("" ::: "memory");
            const int nslot = slot == 0 ? D : slot - 1;
            constexpr int qn = q + D;                /* stage s + D within this or the next iteration */
            issue(s0 + qn, nslot, aw[q % D], gs + ((qn / G) & 1) * 1024, qn % G == 0, qn % U == 0);
            asm volatile("" ::: "memory");
            slot = slot == D ? 0 : slot + 1;
        });
    }
    wait_vm<0>();                           /* trailing repeat loads drain before exit */

    mx_store<SWIGLU, NTG>(a, acc, r0, ntok, 0, SWIGLU ? f0 + 32 * wave : f0 + 64 * wave);
}

template <bool SWIGLU>
__global__ __launch_bounds__(256, 2) void k_grouped_mx_thin(GroupedMxArgs a, int thin_rows)
{
    constexpr int FEAT = SWIGLU ? 128 : 256;
    __shared__ __align__(16) uint8_t lds[TH_LDS];
    MxItem it;
    if (!mx_item<FEAT>(a, it) || it.ntok > thin_rows) return;      /* whole workgroup */
    const DSV4ExpertW ex = ld_uniform(a.table, it.grp);
    const DSV4QMat m1 = SWIGLU ? ex.w1 : ex.w2, m3 = ex.w3;
    if (!fp4_matches(m1, a.N, a.K) || (SWIGLU && !fp4_matches(m3, a.N, a.K))) {
        mx_fill_bad<SWIGLU, FEAT, 256>(a, it);
        return;
    }
    const int ntg = (it.ntok + 15) / 16;
    if (ntg == 1) thin_tile<SWIGLU, 1>(a, m1, m3, it.r0, it.ntok, it.f0, lds);
    else if (ntg == 2) thin_tile<SWIGLU, 2>(a, m1, m3, it.r0, it.ntok, it.f0, lds);
    else if (ntg == 3) thin_tile<SWIGLU, 3>(a, m1, m3, it.r0, it.ntok, it.f0, lds);
    else thin_tile<SWIGLU, 4>(a, m1, m3, it.r0, it.ntok, it.f0, lds);
}

int grouped_mx_rows_per_tile() { return GX_TILE; }

template <bool SW>
static hipError_t grouped_mx_k(const GroupedMxArgs &a, long items, int thin_rows, hipStream_t st,
                               hipStream_t st_thin)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_grouped_mx<SW>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, GX_LDS);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    if (thin_rows > 0) hipLaunchKernelGGL((k_grouped_mx_thin<SW>), dim3((unsigned)items), dim3(256), 0, st_thin, a, thin_rows);
    hipLaunchKernelGGL((k_grouped_mx<SW>), dim3((unsigned)items), dim3(512), GX_LDS, st, a, thin_rows);
    return hipGetLastError();
}

hipError_t grouped_mx_launch(bool swiglu, const GroupedMxArgs &a, long max_tiles, hipStream_t st,
                             hipStream_t st_thin)
{
    const int feat = swiglu ? 128 : 256;
    if (!a.table || a.N % feat || a.K % 128 || max_tiles <= 0 || a.nrows <= 0 ||
        (swiglu && !a.out_s) || (size_t)a.nrows * a.K >= (1u << 31) ||
        (size_t)a.N * a.K / 2 >= (1u << 31))
        return hipErrorInvalidValue;
    const long items = max_tiles * (a.N / feat);
    const int thin_rows = a.K % TH_KQ == 0 ? TH_TOK : 0;   /* the thin ring runs whole groups of stages */
    return swiglu ? grouped_mx_k<true>(a, items, thin_rows, st, st_thin)
                  : grouped_mx_k<false>(a, items, thin_rows, st, st_thin);
}

} // namespace dsv4
