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
 *   A workgroup of eight waves (two per SIMD) owns a 128 (tokens) x 256
 *   (features) tile of C; wave (wm, wn) owns tokens 64 wm .. +63 and features
 *   64 wn .. +63. K advances in 128-wide blocks, one scale block each.
 *   Each block's A rows (128 x 128 B), W rows (256 x 128 B) and token scales
 *   travel global -> LDS by direct loads (global_load_lds_dwordx4: 1 KiB per
 *   wave instruction, 8 rows x 128 B, no VGPR round trip) into a three-stage
 *   ring, 16-byte chunks XOR-swizzled so the operand reads are bank-conflict
 *   free. Block kb's MFMAs run from registers. After its first two, every
 *   wave waits for its own loads of stage kb+1 and a plain s_barrier
 *   publishes it and frees stage kb, which the loads of block kb+3 refill one
 *   per MFMA slot; block kb+1's operands are read meanwhile: the token
 *   operands into a second register set, each weight operand into its own
 *   registers right after its last use (feature-group-major MFMA order).
 *   The MFMA is v_mfma_scale_f32_16x16x128_f8f6f4 with both hardware scales
 *   set to 1 (E8M0 127): one instruction per 16 features x 16 tokens x one
 *   128-K block, W rows as its A operand and tokens as its B operand, so each
 *   lane's four outputs share one token and one 128-row weight block. The
 *   product starts from zero and is folded into the fp32 accumulator two
 *   MFMAs later with the two fp32 block scales, acc += p * (s_a[token][kb] *
 *   s_w[nb][kb]) -- fp32 scales cannot ride in the E8M0 hardware scale
 *   operands. Every MFMA slot is fenced, so the promotion never waits on an
 *   MFMA still in the pipe; the other wave of the SIMD fills the matrix
 *   unit while this one promotes, reads LDS or waits at the barrier.
 *   Operand layout of the MFMA (measured on gfx950): lane l supplies row
 *   l % 16 with k in [16 (l/16), +16) in bytes 0-15 and [64 + 16 (l/16), +16)
 *   in bytes 16-31; result element e of lane l is row 4 (l/16) + e, column
 *   l % 16.
 *   The finished tile is staged through LDS and written as whole 16-byte
 *   pieces of contiguous rows.
 *
 * Bound: MFMA (2 M N K flops; 68.7 GFLOP at 2048 x 4096 x 4096).
 *
 * k_gemm_mx is the same schedule for the checkpoint's own FP8 format, E8M0
 * 128 x 128 weight scales, with MXFP8 tokens (E8M0 per 32 reduction
 * indices): both scales go into the MFMA's hardware scale operands, the
 * MFMA accumulates across K blocks, and no product is promoted.
 */
#include "dsv4_internal.h"

namespace dsv4 {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int GM = 128;          /* tokens per workgroup tile                */
constexpr int GN = 256;          /* features per workgroup tile              */
constexpr int GK = 128;          /* k per block = one scale block            */
constexpr int NWAVE = 8;
constexpr int NSTAGE = 3;        /* block kb+3 loads while kb+1 is read      */
/* one stage: A rows and W rows of 128 bytes (16-byte chunks XOR-swizzled),
 * the block's 128 token scales, a pad where the waves without a scale load
 * land theirs */
constexpr int ST_A = 0;
constexpr int ST_W = GM * GK;
constexpr int ST_SA = ST_W + GN * GK;
constexpr int ST_PAD = ST_SA + GM * 4;
constexpr int STAGE = ST_PAD + 256;
constexpr int RING_BYTES = NSTAGE * STAGE;   /* 149,760 B */
constexpr int VM_STAGE = 7;      /* loads per wave per block: 2 A + 4 W + 1 scale */
constexpr int E8M0_ONE = 127;

/* s_waitcnt immediate: vmcnt n (six bits, split 3:0 and 15:14), expcnt 7,
 * lgkmcnt 0 (lgkm0) or 15 (no wait) */
constexpr int waitcnt(int vm, bool lgkm0)
{
    return (vm & 15) | ((vm >> 4) << 14) | 0x70 | (lgkm0 ? 0 : 0xF00);
}

constexpr int lds_bytes(bool out_bf16)
{
    const int stage_out = GM * GN * (out_bf16 ? 2 : 4);
    return RING_BYTES > stage_out ? RING_BYTES : stage_out;
}
static_assert(RING_BYTES <= 160 * 1024 && GM * GN * 4 <= 160 * 1024, "LDS of one CU");

/* Physical 16-byte slot of logical chunk c in staged row r. Sixteen lanes
 * reading the same chunk of sixteen consecutive rows hit sixteen different
 * 16-byte bank groups. */
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;   /* quiet NaN */
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

constexpr uint32_t RSRC_WORD3 = 0x00020000u;      /* raw dword buffer */

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, (int)RSRC_WORD3);
}
/* buffer -> LDS, 16 (or 4) bytes per lane at byte voff + soff, lane l landing
 * at dst + l * size; the per-block offset soff is a scalar, so a load costs
 * no vector instruction for its address */
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint8_t *dst)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, (int)voff, (int)soff, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint8_t *dst)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 4, (int)voff, (int)soff, 0, 0);
}

/* Per-lane offsets, fixed for the whole call; the K block only moves the
 * wave-uniform bases. Direct-load instruction j of the workgroup fills staged
 * rows 8j .. 8j+7 of A (j < 16) or W: lane l row 8j + l/8, slot l%8, which
 * holds logical chunk swz(row, l%8). Wave w issues A instructions 2w, 2w+1
 * and W instructions 4w .. 4w+3. */
struct Plan {
    __amdgpu_buffer_rsrc_t ra, rw, rs;   /* A, W and the token scales          */
    uint32_t a[2], w[4];    /* global byte offsets from column 0            */
    uint32_t s;             /* Sa byte offset of this lane's token (waves 0, 1) */
    int w_lo, w_hi;         /* LDS: chunks l/16, l/16 + 4 of weight row l%16 of the wave */
    int b_lo, b_hi;         /* LDS: the same of token row l%16 of the wave  */
    int sa;                 /* LDS: scale of the wave's token l%16          */
};

__device__ __forceinline__ Plan make_plan(const GemmArgs &a, int m0, int n0, int wave, int lane)
{
    Plan d;
    d.ra = buf_rsrc(a.Aq, (uint32_t)a.M * (uint32_t)a.K);
    d.rw = buf_rsrc(a.W, (uint32_t)a.N * (uint32_t)a.K);
    d.rs = buf_rsrc(a.Sa, (uint32_t)(a.K / GK) * (uint32_t)a.sa_kb * 4u + (uint32_t)a.M * (uint32_t)a.sa_tok * 4u);
    const int r8 = lane >> 3, p = lane & 7;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = 8 * (2 * wave + i) + r8;
        d.a[i] = (uint32_t)min(m0 + r, a.M - 1) * (uint32_t)a.K + 16u * (uint32_t)swz(r, p);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 8 * (4 * wave + i) + r8;
        d.w[i] = (uint32_t)min(n0 + r, a.N - 1) * (uint32_t)a.K + 16u * (uint32_t)swz(r, p);
    }
    d.s = (uint32_t)min(m0 + 64 * (wave & 1) + lane, a.M - 1) * (uint32_t)a.sa_tok * 4u;
    /* operand rows 16q + r16 of a wave share the swizzle of r16 */
    const int wm = wave & 1, wn = wave >> 1, r16 = lane & 15, g = lane >> 4;
    d.w_lo = ST_W + (64 * wn + r16) * GK + 16 * swz(r16, g);
    d.w_hi = ST_W + (64 * wn + r16) * GK + 16 * swz(r16, g + 4);
    d.b_lo = ST_A + (64 * wm + r16) * GK + 16 * swz(r16, g);
    d.b_hi = ST_A + (64 * wm + r16) * GK + 16 * swz(r16, g + 4);
    d.sa = ST_SA + 4 * (64 * wm + r16);
    return d;
}

/* Load j (0..6) of block kb into stage st: A (j < 2), W (2..5), the token
 * scales (6: waves 0, 1 load 64 each; the other waves repeat wave 0's into
 * the pad, so every wave issues the same count and one vmcnt value serves
 * all). */
__device__ __forceinline__ void issue_one(const GemmArgs &a, const Plan &d, uint8_t *st, int kb,
                                          int wave, int j)
{
    const uint32_t kofs = (uint32_t)kb * GK;
    if (j < 2) {
        dma16(d.ra, d.a[j], kofs, st + ST_A + 1024 * (2 * wave + j));
    } else if (j < 6) {
        dma16(d.rw, d.w[j - 2], kofs, st + ST_W + 1024 * (4 * wave + j - 2));
    } else {
        dma4(d.rs, d.s, (uint32_t)kb * (uint32_t)a.sa_kb * 4u, st + (wave < 2 ? ST_SA + 256 * wave : ST_PAD));
    }
}

__device__ __forceinline__ void issue(const GemmArgs &a, const Plan &d, uint8_t *st, int kb, int wave)
{
#pragma unroll
    for (int j = 0; j < VM_STAGE; j++) issue_one(a, d, st, kb, wave, j);
}

__device__ __forceinline__ v8i lds_op(const uint8_t *p_lo, const uint8_t *p_hi)
{
    const u32x4 lo = *(const u32x4 *)p_lo;
    const u32x4 hi = *(const u32x4 *)p_hi;
    v8i v;
    v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
    v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
    return v;
}
/* weight operand of feature group f / token operand of group t (16 rows each) */
__device__ __forceinline__ v8i read_w(const uint8_t *st, const Plan &d, int f)
{
    return lds_op(st + d.w_lo + 2048 * f, st + d.w_hi + 2048 * f);
}
__device__ __forceinline__ v8i read_b(const uint8_t *st, const Plan &d, int t)
{
    return lds_op(st + d.b_lo + 2048 * t, st + d.b_hi + 2048 * t);
}

/* fp32 scale of a 128-row weight block at K block kb (wave-uniform: a scalar
 * load) */
template <bool WF32S>
__device__ __forceinline__ float weight_scale(const GemmArgs &a, int nb, int kb)
{
    const size_t i = (size_t)nb * (size_t)(a.K / GK) + (size_t)kb;
    if constexpr (WF32S) {
        return ld_uniform((const float *)a.Sw + i, 0);
    } else {
        const uintptr_t p = (uintptr_t)a.Sw + i;
        const uint32_t word = ld_uniform((const uint32_t *)(p & ~(uintptr_t)3), 0);
        return dev_e8m0((word >> (8 * (p & 3))) & 0xFFu);
    }
}

__device__ __forceinline__ v4f mfma16(const v8i &w, const v8i &b)
{
    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, b, zero, 0, 0, 0, E8M0_ONE, 0, E8M0_ONE);
}

__device__ __forceinline__ void promote(v4f &acc, const v4f &p, float cs)
{
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = fmaf(p[e], cs, acc[e]);
}

/* What one wave carries from block to block. Values a block hands to the
 * next live in two register sets chosen by the block's parity, so nothing
 * is copied between blocks: block kb (parity P) multiplies with weight
 * group 3 from w3[P] and loads the next block's into w3[1 - P]; it promotes
 * with cs[P] and writes the next block's scales to cs[1 - P]; its last two
 * products land in pc[P], which the next block promotes in its first two
 * slots with cs[P][2..3]. */
struct State {
    v4f acc[4][4];              /* [feature group][token group]                */
    v8i w[3];                   /* weight groups 0-2 (replaced group by group) */
    v8i w3[2];                  /* weight group 3, by block parity             */
    float cs[2][4];             /* s_a * s_w per token group, by block parity  */
    v4f pc[2][2];               /* a block's last two products, by parity      */
    float sw_next;              /* weight scale of the next block              */
};

/* Block kb (parity P): MFMA slot s = 4f + t multiplies weight group f by
 * token group t; behind it the product of slot s-2 is promoted (slots 0, 1
 * promote the previous block's slots 14, 15): an FMA on the product of the
 * MFMA issued just before would stall the matrix pipe. Slots 0 and 1 run
 * from registers; then this wave's loads of stage kb+1 have landed (only
 * block kb+2's are outstanding) and its reads of stage kb are done, and the
 * barrier makes both true for the workgroup: stage kb+1 is read from there
 * on (token groups into bn at slots 2..5, the scales at 6..9, weight group f
 * into w[f] after slot 4f+3, group 3 into w3[1 - P] at slot 10) and stage kb
 * is refilled with block kb+3 (one load per slot, 2..8). */
template <bool WF32S, int P>
__device__ __forceinline__ void kblock(const GemmArgs &a, const Plan &d, uint8_t *lds, State &S,
                                       const v8i (&b)[4], v8i (&bn)[4], int kb, int nkb, int nb,
                                       int wave)
{
    constexpr int Q = 1 - P;
    const int cb = kb % NSTAGE;
    const int nx = cb + 1 == NSTAGE ? 0 : cb + 1;
    const uint8_t *nst = lds + nx * STAGE;
    uint8_t *fill = lds + cb * STAGE;
    const int kl = min(kb + 3, nkb - 1);
    v4f p[14];
    float sa[4];
    float sw2 = 0.0f;
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const int f = s >> 2, t = s & 3;
        const v8i &wop = f < 3 ? S.w[f] : S.w3[P];
        if (s < 14) p[s] = mfma16(wop, b[t]);
        else S.pc[P][s - 14] = mfma16(wop, b[t]);
        DSV4_ORDER();
        if (s < 2) promote(S.acc[3][2 + s], S.pc[Q][s], S.cs[Q][2 + s]);
        else promote(S.acc[(s - 2) >> 2][(s - 2) & 3], p[s - 2], S.cs[P][(s - 2) & 3]);
        if (s == 1) {
            DSV4_ORDER();
            __builtin_amdgcn_s_waitcnt(waitcnt(VM_STAGE, true));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            DSV4_ORDER();
        }
        if (s >= 2 && s < 2 + VM_STAGE) issue_one(a, d, fill, kl, wave, s - 2);
        if (s == 2) sw2 = weight_scale<WF32S>(a, nb, min(kb + 2, nkb - 1));
        if (s >= 2 && s < 6) bn[s - 2] = read_b(nst, d, s - 2);
        if (s >= 6 && s < 10) sa[s - 6] = *(const float *)(nst + d.sa + 64 * (s - 6));
        if (s == 10) S.w3[Q] = read_w(nst, d, 3);
        if (t == 3 && f < 3) S.w[f] = read_w(nst, d, f);
        DSV4_ORDER();
    }
#pragma unroll
    for (int t = 0; t < 4; t++) S.cs[Q][t] = sa[t] * S.sw_next;
    S.sw_next = sw2;
}

/* E8M0 byte of a 128 x 128 weight block (wave-uniform: a scalar load) */
__device__ __forceinline__ int weight_byte(const GemmArgs &a, int nb, int kb)
{
    const uintptr_t p = (uintptr_t)a.Sw + (size_t)nb * (size_t)(a.K / GK) + (size_t)kb;
    const uint32_t word = ld_uniform((const uint32_t *)(p & ~(uintptr_t)3), 0);
    return (int)((word >> (8 * (p & 3))) & 0xFFu);
}

/* What one wave of the hardware-scaled GEMM carries between blocks: the
 * accumulators (the MFMA accumulates across blocks), the operands of weight
 * groups 0-2 and group 3 by block parity, and the E8M0 scales: the token
 * groups' bytes of this lane's 32-element block by parity, the weight
 * block's byte of this block and the next. */
struct StateHw {
    v4f acc[4][4];
    v8i w[3];
    v8i w3[2];
    int tb[2][4];
    int wb, wb_next;
};

/* Block kb (parity P) of the hardware-scaled GEMM: E8M0 weight blocks and
 * MXFP8 tokens both ride in the MFMA's scale operands, so every slot is one
 * MFMA accumulating into its own accumulator and no vector instruction
 * promotes a product. Loads, barrier and operand reads follow kblock. */
template <int P>
__device__ __forceinline__ void kblock_hw(const GemmArgs &a, const Plan &d, uint8_t *lds, StateHw &S,
                                          const v8i (&b)[4], v8i (&bn)[4], int kb, int nkb, int nb,
                                          int wave, int gq)
{
    constexpr int Q = 1 - P;
    const int cb = kb % NSTAGE;
    const int nx = cb + 1 == NSTAGE ? 0 : cb + 1;
    const uint8_t *nst = lds + nx * STAGE;
    uint8_t *fill = lds + cb * STAGE;
    const int kl = min(kb + 3, nkb - 1);
    uint32_t sd[4];
    int wb2 = 0;
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const int f = s >> 2, t = s & 3;
        const v8i &wop = f < 3 ? S.w[f] : S.w3[P];
        S.acc[f][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wop, b[t], S.acc[f][t], 0, 0, 0, S.wb,
                                                                        0, S.tb[P][t]);
        DSV4_ORDER();
        if (s == 1) {
            __builtin_amdgcn_s_waitcnt(waitcnt(VM_STAGE, true));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            DSV4_ORDER();
        }
        if (s >= 2 && s < 2 + VM_STAGE) issue_one(a, d, fill, kl, wave, s - 2);
        if (s == 2) wb2 = weight_byte(a, nb, min(kb + 2, nkb - 1));
        if (s >= 2 && s < 6) bn[s - 2] = read_b(nst, d, s - 2);
        if (s >= 6 && s < 10) sd[s - 6] = *(const uint32_t *)(nst + d.sa + 64 * (s - 6));
        if (s == 10) S.w3[Q] = read_w(nst, d, 3);
        if (t == 3 && f < 3) S.w[f] = read_w(nst, d, f);
        DSV4_ORDER();
    }
#pragma unroll
    for (int t = 0; t < 4; t++) S.tb[Q][t] = (int)((sd[t] >> (8 * gq)) & 0xFFu);
    S.wb = S.wb_next;
    S.wb_next = wb2;
}

template <bool OUT_BF16>
__device__ __forceinline__ void stage_frag(uint8_t *lds, const v4f &acc, int tok, int f)
{
    constexpr int EB = OUT_BF16 ? 2 : 4;
    uint8_t *row = lds + tok * (GN * EB);
    const int c = (f * EB) >> 4, off = (f * EB) & 15;
    uint8_t *dst = row + 16 * (c ^ (tok & 31)) + off;
    if constexpr (OUT_BF16) {
        uint2 pk;
        pk.x = f32_to_bf16_bits(acc[0]) | (f32_to_bf16_bits(acc[1]) << 16);
        pk.y = f32_to_bf16_bits(acc[2]) | (f32_to_bf16_bits(acc[3]) << 16);
        *(uint2 *)dst = pk;
    } else {
        *(f32x4 *)dst = f32x4{acc[0], acc[1], acc[2], acc[3]};
    }
}

/* Output staging: the workgroup's 128 x 256 tile sits in LDS as rows of GN
 * elements, 16-byte chunk c of row r stored at chunk c ^ (r % 32), and is
 * copied to C in whole 16-byte pieces of contiguous rows. The stores are
 * non-temporal (streaming, no L2 allocation): every workgroup of a one-round
 * grid writes its tile at the same moment, after the last K block (measured
 * at 2048 x 4096 x 4096, bf16 out, alternating builds on one device: 40.3 ->
 * 39.8 us). */
template <bool OUT_BF16>
__device__ __forceinline__ void write_tile(const GemmArgs &a, const uint8_t *lds, int m0, int n0)
{
    constexpr int EB = OUT_BF16 ? 2 : 4;
    constexpr int CPR = GN * EB / 16;                  /* 16-byte chunks per row */
    const int live = min(GN, a.N - n0) * EB / 16;       /* a 128-wide N tail uses half */
    for (int i = threadIdx.x; i < GM * CPR; i += NWAVE * 64) {
        const int r = i / CPR, c = i % CPR;
        const int m = m0 + r;
        if (m >= a.M || c >= live) continue;
        const u32x4 v = *(const u32x4 *)(lds + r * (GN * EB) + 16 * (c ^ (r & 31)));
        __builtin_nontemporal_store(v, (u32x4 *)((uint8_t *)a.C + ((size_t)m * a.ldc + n0) * EB + 16 * c));
    }
}

/* Output tile (m0, n0) of this workgroup. Workgroups are dealt to the eight
 * XCDs round robin (linear id % 8); when the grid divides by eight, XCD x
 * takes the x-th eighth of the tiles in grouped order (eight M tiles per
 * group, N tiles within a group one after another), so the workgroups that
 * share an XCD's L2 share A rows and W rows: on 16 x 16 tiles each XCD holds
 * 8 M tiles x 4 N tiles (measured: 36.9 us against 38.2 with row-major
 * tiles, whose XCDs each read all of A). */
__device__ __forceinline__ void tile_of(int &m0, int &n0)
{
    const int gx = gridDim.x, gy = gridDim.y, T = gx * gy;
    int lin = blockIdx.y * gx + blockIdx.x;
    if (T % 8 == 0) lin = (lin % 8) * (T / 8) + lin / 8;
    const int g = lin / (8 * gx), idx = lin - g * 8 * gx;
    const int gm = min(8, gy - 8 * g);
    m0 = (8 * g + idx % gm) * GM;
    n0 = (idx / gm) * GN;
}

} // namespace

template <bool WF32S, bool OUT_BF16>
__global__ __launch_bounds__(512) void k_gemm_fp8(GemmArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int wm = wave & 1, wn = wave >> 1;
    int m0, n0;
    tile_of(m0, n0);
    const int nkb = a.K / GK;
    const int nb = min((n0 + 64 * wn) / 128, a.N / 128 - 1);
    const Plan d = make_plan(a, m0, n0, wave, lane);

    State S;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        S.pc[1][0][e] = 0.0f;
        S.pc[1][1][e] = 0.0f;
#pragma unroll
        for (int f = 0; f < 4; f++)
#pragma unroll
            for (int t = 0; t < 4; t++) S.acc[f][t][e] = 0.0f;
    }
    S.cs[1][2] = 0.0f;
    S.cs[1][3] = 0.0f;

    /* blocks 0, 1, 2 (repeating the last block when K is shorter) */
    issue(a, d, lds, 0, wave);
    DSV4_ORDER();
    issue(a, d, lds + STAGE, min(1, nkb - 1), wave);
    DSV4_ORDER();
    issue(a, d, lds + 2 * STAGE, min(2, nkb - 1), wave);
    DSV4_ORDER();
    const float sw0 = weight_scale<WF32S>(a, nb, 0);
    S.sw_next = weight_scale<WF32S>(a, nb, min(1, nkb - 1));
    __builtin_amdgcn_s_waitcnt(waitcnt(2 * VM_STAGE, true));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    v8i b0[4], b1[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (q < 3) S.w[q] = read_w(lds, d, q);
        else S.w3[0] = read_w(lds, d, 3);
        b0[q] = read_b(lds, d, q);
        S.cs[0][q] = *(const float *)(lds + d.sa + 64 * q) * sw0;
    }
    int kb = 0;
    for (; kb + 1 < nkb; kb += 2) {
        kblock<WF32S, 0>(a, d, lds, S, b0, b1, kb, nkb, nb, wave);
        kblock<WF32S, 1>(a, d, lds, S, b1, b0, kb + 1, nkb, nb, wave);
    }
    if (kb < nkb) {
        kblock<WF32S, 0>(a, d, lds, S, b0, b1, kb, nkb, nb, wave);
        promote(S.acc[3][2], S.pc[0][0], S.cs[0][2]);
        promote(S.acc[3][3], S.pc[0][1], S.cs[0][3]);
    } else {
        promote(S.acc[3][2], S.pc[1][0], S.cs[1][2]);
        promote(S.acc[3][3], S.pc[1][1], S.cs[1][3]);
    }
    /* drain the trailing repeat loads and reads before the ring becomes the
     * output staging area */
    __builtin_amdgcn_s_waitcnt(waitcnt(0, true));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
        for (int t = 0; t < 4; t++)
            stage_frag<OUT_BF16>(lds, S.acc[f][t], 64 * wm + 16 * t + r16, 64 * wn + 16 * f + 4 * g);
    __syncthreads();
    write_tile<OUT_BF16>(a, lds, m0, n0);
}

/* C = A W^T with E8M0 128 x 128 weight blocks (the checkpoint's FP8 format)
 * and MXFP8 tokens (e4m3, one E8M0 per token and 32 reduction indices); the
 * staged scale dword of a token holds its four 32-blocks of a 128-K block. */
template <bool OUT_BF16>
__global__ __launch_bounds__(512) void k_gemm_mx(GemmArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int wm = wave & 1, wn = wave >> 1;
    const int gq = lane >> 4;
    int m0, n0;
    tile_of(m0, n0);
    const int nkb = a.K / GK;
    const int nb = min((n0 + 64 * wn) / 128, a.N / 128 - 1);
    const Plan d = make_plan(a, m0, n0, wave, lane);

    StateHw S;
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
        for (int t = 0; t < 4; t++) S.acc[f][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    issue(a, d, lds, 0, wave);
    DSV4_ORDER();
    issue(a, d, lds + STAGE, min(1, nkb - 1), wave);
    DSV4_ORDER();
    issue(a, d, lds + 2 * STAGE, min(2, nkb - 1), wave);
    DSV4_ORDER();
    S.wb = weight_byte(a, nb, 0);
    S.wb_next = weight_byte(a, nb, min(1, nkb - 1));
    __builtin_amdgcn_s_waitcnt(waitcnt(2 * VM_STAGE, true));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    v8i b0[4], b1[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (q < 3) S.w[q] = read_w(lds, d, q);
        else S.w3[0] = read_w(lds, d, 3);
        b0[q] = read_b(lds, d, q);
        S.tb[0][q] = (int)((*(const uint32_t *)(lds + d.sa + 64 * q) >> (8 * gq)) & 0xFFu);
    }
    int kb = 0;
    for (; kb + 1 < nkb; kb += 2) {
        kblock_hw<0>(a, d, lds, S, b0, b1, kb, nkb, nb, wave, gq);
        kblock_hw<1>(a, d, lds, S, b1, b0, kb + 1, nkb, nb, wave, gq);
    }
    if (kb < nkb) kblock_hw<0>(a, d, lds, S, b0, b1, kb, nkb, nb, wave, gq);
    __builtin_amdgcn_s_waitcnt(waitcnt(0, true));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int r16 = lane & 15;
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
        for (int t = 0; t < 4; t++)
            stage_frag<OUT_BF16>(lds, S.acc[f][t], 64 * wm + 16 * t + r16, 64 * wn + 16 * f + 4 * gq);
    __syncthreads();
    write_tile<OUT_BF16>(a, lds, m0, n0);
}

template <bool OB>
static hipError_t launch_gemm_mx(const GemmArgs &a, hipStream_t st)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm_mx<OB>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 lds_bytes(OB));
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    const dim3 grid((unsigned)((a.N + GN - 1) / GN), (unsigned)((a.M + GM - 1) / GM)), block(512);
    hipLaunchKernelGGL((k_gemm_mx<OB>), grid, block, lds_bytes(OB), st, a);
    return hipGetLastError();
}

template <bool WS, bool OB>
static hipError_t launch_gemm(const GemmArgs &a, hipStream_t st)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm_fp8<WS, OB>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 lds_bytes(OB));
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    const dim3 grid((unsigned)((a.N + GN - 1) / GN), (unsigned)((a.M + GM - 1) / GM)), block(512);
    hipLaunchKernelGGL((k_gemm_fp8<WS, OB>), grid, block, lds_bytes(OB), st, a);
    return hipGetLastError();
}

hipError_t gemm_fp8_launch(const GemmArgs &a, bool w_f32s, bool out_bf16, hipStream_t st)
{
    if (a.K % GK || a.N % 128 || a.M <= 0) return hipErrorInvalidValue;
    /* the loads address A, W and Sa with 32-bit per-lane byte offsets */
    if ((size_t)a.M * a.K > 0xFFFFFFFFull || (size_t)a.N * a.K > 0xFFFFFFFFull ||
        (size_t)a.M * a.sa_tok * 4 + (size_t)(a.K / GK) * a.sa_kb * 4 > 0xFFFFFFFFull)
        return hipErrorInvalidValue;
    if (w_f32s) return out_bf16 ? launch_gemm<true, true>(a, st) : launch_gemm<true, false>(a, st);
    return out_bf16 ? launch_gemm<false, true>(a, st) : launch_gemm<false, false>(a, st);
}

hipError_t gemm_mx_launch(const GemmArgs &a, bool out_bf16, hipStream_t st)
{
    const bool tok_major = a.sa_tok == a.K / GK && a.sa_kb == 1, blk_major = a.sa_tok == 1 && a.sa_kb == a.M;
    if (a.K % GK || a.N % 128 || a.M <= 0 || !(tok_major || blk_major))
        return hipErrorInvalidValue;
    if ((size_t)a.M * a.K > 0xFFFFFFFFull || (size_t)a.N * a.K > 0xFFFFFFFFull)
        return hipErrorInvalidValue;
    return out_bf16 ? launch_gemm_mx<true>(a, st) : launch_gemm_mx<false>(a, st);
}

/* ------------------------------------------------- seam dense GEMM --- */

/* The drop-in seam's dense form for FP8 weights (dsv4_mmq_n with many
 * tokens: src/10_compute/dsv4_matmul_fp8.c:102-155 with nt > 31):
 *   C[m][n] = 2^-ex[m] sum_kb s_w[n / 128][kb] sum_{k in block kb} X[m][k] W[n][k]
 * X fp16 rows scaled by 2^ex[m] (k_to_f16_rows), W e4m3 decoded exactly to
 * fp16 in registers (v_cvt_scalef32_pk_f16_fp8 with scale 1), the block's
 * partial from four v_mfma_f32_16x16x32_f16 steps started from zero, then
 * multiplied by the fp32 (or E8M0) block scale into the fp32 accumulator.
 * The steps' reduction order and the promotion order over blocks are those of
 * the grouped kernel's dense form (kmap / bchunk for FP8), so both give the
 * same bits. Tile and tile order as the FP8 GEMM (128 tokens x 256 features,
 * wave (wm, wn) 64 x 64); a K block stages 256 W rows x 128 B and 128 token
 * rows x 256 B (64 KiB) by direct loads into a two-stage ring. */
namespace {

constexpr int H_XB = GK * 2;                  /* fp16 token bytes per row per block */
constexpr int H_ST_X = GN * GK;               /* after 256 W rows of 128 B          */
constexpr int H_STAGE = H_ST_X + GM * H_XB;   /* 64 KiB                             */
constexpr int H_LDS = 2 * H_STAGE;            /* the fp32 output tile reuses it      */
static_assert(H_LDS >= GM * GN * 4 && H_LDS <= 160 * 1024, "seam GEMM LDS");

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

/* physical 16-byte slot of logical chunk c in staged token row r (16 slots) */
__device__ __forceinline__ int swx(int r, int c) { return c ^ (r & 15); }

/* eight e4m3 (dwords 2 hi, 2 hi + 1 of a 16-byte chunk) to eight fp16, exact */
__device__ __forceinline__ h8v w_f16(const u32x4 &w, int hi)
{
    const uint32_t d0 = hi ? w.z : w.x, d1 = hi ? w.w : w.y;
    u32x4 v;
    v.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, false));
    v.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, true));
    v.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, false));
    v.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, true));
    return __builtin_bit_cast(h8v, v);
}

} // namespace

template <bool WF32S>
__global__ __launch_bounds__(512) void k_gemm_seam(SeamGemmArgs s)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int wm = wave & 1, wn = wave >> 1, rr = lane & 15, gq = lane >> 4;
    int m0, n0;
    tile_of(m0, n0);
    GemmArgs g;                                /* the FP8 GEMM's view: scales, epilogue */
    g.Aq = nullptr; g.Sa = nullptr; g.W = s.W; g.Sw = s.Sw; g.C = s.C;
    g.M = s.M; g.N = s.N; g.K = s.K; g.ldc = s.N; g.sa_tok = 0; g.sa_kb = 0;
    const int nkb = s.K / GK;
    const int nb = min((n0 + 64 * wn) / 128, s.N / 128 - 1);
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(s.W, (uint32_t)s.N * (uint32_t)s.K);
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(s.X, (uint32_t)s.M * (uint32_t)s.K * 2u);
    /* direct loads: W instruction j (4 wave .. + 3) fills W rows 8j .. 8j+7,
     * X instruction j token rows 4j .. 4j+3, lane l landing in physical slot
     * l % 8 (W) or l % 16 (X) of its row */
    uint32_t wo[4], xo[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int j = 4 * wave + i;
        const int rw8 = 8 * j + (lane >> 3), rx4 = 4 * j + (lane >> 4);
        wo[i] = (uint32_t)min(n0 + rw8, s.N - 1) * (uint32_t)s.K + 16u * (uint32_t)swz(rw8, lane & 7);
        xo[i] = (uint32_t)min(m0 + rx4, s.M - 1) * (uint32_t)s.K * 2u + 16u * (uint32_t)swx(rx4, lane & 15);
    }
    auto issue = [&](int kb, uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(rw, wo[i], (uint32_t)kb * GK, buf + 1024 * (4 * wave + i));
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(rx, xo[i], (uint32_t)kb * H_XB, buf + H_ST_X + 1024 * (4 * wave + i));
    };

    v4f acc[4][4];
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[f][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    issue(0, lds);
    for (int kb = 0; kb < nkb; kb++) {
        /* this wave's loads of block kb have landed; after the barrier every
         * wave's have, and no wave still reads the other stage, which the
         * loads of block kb + 1 refill */
        __builtin_amdgcn_s_waitcnt(waitcnt(0, true));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kb + 1 < nkb) issue(kb + 1, lds + ((kb + 1) & 1) * H_STAGE);
        const uint8_t *buf = lds + (kb & 1) * H_STAGE;
        const float sw = weight_scale<WF32S>(g, nb, kb);
        v4f p[4][4];
        u32x4 w16[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            h8v b[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int r = 64 * wm + 16 * t + rr;
                b[t] = *(const h8v *)(buf + H_ST_X + r * H_XB + 16 * swx(r, 8 * (j >> 1) + 2 * gq + (j & 1)));
            }
#pragma unroll
            for (int f = 0; f < 4; f++) {
                if ((j & 1) == 0) {
                    const int r = 64 * wn + 16 * f + rr;
                    w16[f] = *(const u32x4 *)(buf + r * GK + 16 * swz(r, 4 * (j >> 1) + gq));
                }
                const h8v av = w_f16(w16[f], j & 1);
#pragma unroll
                for (int t = 0; t < 4; t++)
                    p[f][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b[t], j == 0 ? v4f{0.0f, 0.0f, 0.0f, 0.0f}
                                                                                  : p[f][t], 0, 0, 0);
            }
        }
#pragma unroll
        for (int f = 0; f < 4; f++)
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[f][t][e] = fmaf(p[f][t][e], sw, acc[f][t][e]);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt(0, true));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int tok = m0 + 64 * wm + 16 * t + rr;
        const int ex = tok < s.M ? s.ex[tok] : 0;
#pragma unroll
        for (int f = 0; f < 4; f++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[f][t][e] = ex ? ldexpf(acc[f][t][e], -ex) : acc[f][t][e];
    }
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
        for (int t = 0; t < 4; t++)
            stage_frag<false>(lds, acc[f][t], 64 * wm + 16 * t + rr, 64 * wn + 16 * f + 4 * gq);
    __syncthreads();
    write_tile<false>(g, lds, m0, n0);
}

template <bool WS>
static hipError_t launch_gemm_seam(const SeamGemmArgs &s, hipStream_t st)
{
    static bool attr_done = false;
    if (!attr_done) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm_seam<WS>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, H_LDS);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    const dim3 grid((unsigned)((s.N + GN - 1) / GN), (unsigned)((s.M + GM - 1) / GM)), block(512);
    hipLaunchKernelGGL((k_gemm_seam<WS>), grid, block, H_LDS, st, s);
    return hipGetLastError();
}

bool gemm_seam_ok(int M, int N, int K)
{
    return M > 0 && N > 0 && K > 0 && K % GK == 0 && N % 128 == 0 &&
           (size_t)N * K <= 0xFFFFFFFFull && (size_t)M * K * 2 <= 0xFFFFFFFFull;
}

hipError_t gemm_seam_launch(const SeamGemmArgs &s, bool w_f32s, hipStream_t st)
{
    if (!gemm_seam_ok(s.M, s.N, s.K) || !s.X || !s.ex || !s.W || !s.Sw || !s.C) return hipErrorInvalidValue;
    return w_f32s ? launch_gemm_seam<true>(s, st) : launch_gemm_seam<false>(s, st);
}

} // namespace dsv4
