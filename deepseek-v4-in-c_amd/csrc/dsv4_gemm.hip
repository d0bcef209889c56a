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
 *   A workgroup of four waves (one per SIMD) owns a 128 (tokens) x 256
 *   (features) tile of C; wave (wm, wn) owns 64 tokens x 128 features. K
 *   advances in 128-wide blocks, one scale block each. Each block's A rows
 *   (128 x 128 B), W rows (256 x 128 B) and scales travel global -> LDS by
 *   direct loads (global_load_lds_dwordx4: 1 KiB per wave instruction, no
 *   VGPR round trip) into a three-buffer ring, 16-byte chunks XOR-swizzled
 *   so the MFMA operand reads are bank-conflict free. Block kb+2's loads are
 *   issued while block kb multiplies, spread over its first three feature
 *   tiles; between tiles 2 and 3 each wave waits for its own share of block
 *   kb+1 (vmcnt) and a plain s_barrier publishes it, so the next block's
 *   first operands are read while tile 3 multiplies.
 *   The MFMA is v_mfma_scale_f32_32x32x64_f8f6f4 with both hardware scales
 *   set to 1 (E8M0 127): W rows are its A operand and tokens its B operand,
 *   so each lane's 16 outputs of a 32 x 32 tile share one token and one 128-row
 *   weight block. The product of a 128-K block starts from zero and is then
 *   folded into the fp32 accumulator with the two fp32 block scales,
 *   acc += partial * (s_a[token][kb] * s_w[nb][kb]) -- fp32 scales cannot ride
 *   in the E8M0 hardware scale operands. Tile t's MFMAs are issued before
 *   tile t-1's promotion, so the VALU works in the matrix unit's shadow.
 *   The finished tile is staged through LDS and written as whole 16-byte
 *   pieces of contiguous rows.
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

/* Output staging. After the K loop the workgroup's 128 x 256 tile is written
 * to LDS (rows of GN elements, 16-byte chunk c of row r stored at chunk
 * c ^ (r % 32), so the 32 tokens of a fragment store and the consecutive
 * chunks of a row read land in distinct banks), then copied to C in whole
 * 16-byte pieces of contiguous rows. */
template <bool OUT_BF16>
__device__ __forceinline__ void stage_frag(uint8_t *lds, const v16f &acc, int t0, int f0, int col, int g)
{
    constexpr int EB = OUT_BF16 ? 2 : 4;
    const int r = t0 + col;
    uint8_t *row = lds + r * (GN * EB);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int f = f0 + 8 * q + 4 * g;              /* 4 consecutive features */
        const int c = (f * EB) >> 4, off = (f * EB) & 15;
        uint8_t *dst = row + 16 * (c ^ (r & 31)) + off;
        if constexpr (OUT_BF16) {
            uint2 pk;
            pk.x = f32_to_bf16_bits(acc[4 * q]) | (f32_to_bf16_bits(acc[4 * q + 1]) << 16);
            pk.y = f32_to_bf16_bits(acc[4 * q + 2]) | (f32_to_bf16_bits(acc[4 * q + 3]) << 16);
            *(uint2 *)dst = pk;
        } else {
            *(f32x4 *)dst = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        }
    }
}

template <bool OUT_BF16>
__device__ __forceinline__ void write_tile(const GemmArgs &a, const uint8_t *lds, int m0, int n0,
                                           int tid, int nthreads)
{
    constexpr int EB = OUT_BF16 ? 2 : 4;
    constexpr int CPR = GN * EB / 16;                  /* 16-byte chunks per row */
    const int live = min(GN, a.N - n0) * EB / 16;       /* a 128-wide N tail uses half */
    for (int i = tid; i < GM * CPR; i += nthreads) {
        const int r = i / CPR, c = i % CPR;
        const int m = m0 + r;
        if (m >= a.M || c >= live) continue;
        const u32x4 v = *(const u32x4 *)(lds + r * (GN * EB) + 16 * (c ^ (r & 31)));
        *(u32x4 *)((uint8_t *)a.C + ((size_t)m * a.ldc + n0) * EB + 16 * c) = v;
    }
}

} // namespace

/* The 13 direct-to-LDS loads a wave issues per K block. Instruction j of the
 * workgroup fills staged rows 8j .. 8j+7 (1 KiB): lane l row 8j + l/8, slot
 * l%8, which holds logical chunk swz(row, l%8). Per-lane byte offsets are
 * fixed; the K block only moves the wave-uniform base. */
struct DmaPlan {
    uint32_t a[4];      /* Aq bytes, from column 0                          */
    uint32_t w[8];      /* W bytes, from column 0                           */
    uint32_t s;         /* Sa (waves 0, 1) or fp32 Sw (waves 2, 3) bytes    */
    int nb;             /* weight block row of this lane's E8M0 scale load  */
};

template <bool WF32S>
__device__ __forceinline__ DmaPlan make_plan(const GemmArgs &a, int m0, int n0, int wave, int lane)
{
    DmaPlan d;
    const int r8 = lane >> 3, p = lane & 7, nkb = a.K / GK;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 8 * (wave * 4 + i) + r8;
        const int m = min(m0 + r, a.M - 1);
        d.a[i] = (uint32_t)m * (uint32_t)a.K + 16u * (uint32_t)swz(r, p);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = 8 * (wave * 8 + i) + r8;
        const int n = min(n0 + r, a.N - 1);
        d.w[i] = (uint32_t)n * (uint32_t)a.K + 16u * (uint32_t)swz(r, p);
    }
    /* waves 0, 1: 64 token scales each; wave 2: the two weight-block scales
     * (lanes 0, 1 land in the stage, the rest in the pad); wave 3: pad only */
    d.nb = min(n0 / 128 + (lane & 1), a.N / 128 - 1);
    if (wave < 2) d.s = (uint32_t)min(m0 + 64 * wave + lane, a.M - 1) * (uint32_t)nkb * 4u;
    else d.s = (uint32_t)d.nb * (uint32_t)nkb * 4u;
    return d;
}

/* Part PART (0: A rows, 1: first half of W rows, 2: second half and the
 * scales) of the loads of K block kb into stage buffer st. */
template <bool WF32S, int PART>
__device__ __forceinline__ void issue_part(const GemmArgs &a, const DmaPlan &d, uint8_t *st,
                                           int kb, int wave)
{
    const size_t kofs = (size_t)kb * GK;
    if constexpr (PART == 0) {
        const uint8_t *base = a.Aq + kofs;
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(base + d.a[i], st + ST_A + 1024 * (wave * 4 + i));
    } else {
        const uint8_t *base = a.W + kofs;
#pragma unroll
        for (int i = 4 * (PART - 1); i < 4 * PART; i++)
            dma16(base + d.w[i], st + ST_W + 1024 * (wave * 8 + i));
    }
    if constexpr (PART == 2) {
        if (wave < 2) {
            dma4((const uint8_t *)a.Sa + 4 * kb + d.s, st + ST_SA + 256 * wave);
        } else if constexpr (WF32S) {
            dma4((const uint8_t *)a.Sw + 4 * kb + d.s, st + (wave == 2 ? ST_SW : ST_PAD));
        } else {
            /* an E8M0 scale is one byte: load the aligned dword holding it and
             * pick the byte when reading (load_ops) */
            const size_t si = (size_t)d.nb * (a.K / GK) + kb;
            dma4((const uint8_t *)a.Sw + (si & ~(size_t)3), st + (wave == 2 ? ST_SW : ST_PAD));
        }
    }
}

/* Operands of one K block that are read before its first MFMA: the wave's
 * token operands (both 64-wide k steps, both 32-token halves), the weight
 * operand of feature tile 0, and the two combined scales s_a * s_w. */
struct Ops {
    v8i b[2][2];        /* [k step][token half]  */
    v8i w0[2];          /* [k step]              */
    float cs[2];        /* [token half]          */
};

template <bool WF32S>
__device__ __forceinline__ void load_ops(Ops &o, const uint8_t *stage, const GemmArgs &a,
                                         int kb, int n0, int wm, int wn, int col, int g)
{
    const uint8_t *As = stage + ST_A + (wm * 64) * GK;
    const uint8_t *Ws = stage + ST_W + (wn * 128) * GK;
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int u = 0; u < 2; u++)
            o.b[ks][u] = lds_operand(As + (u * 32 + col) * GK, u * 32 + col, ks, g);
#pragma unroll
    for (int ks = 0; ks < 2; ks++) o.w0[ks] = lds_operand(Ws + col * GK, col, ks, g);
    float sw;
    if constexpr (WF32S) {
        sw = *(const float *)(stage + ST_SW + 4 * wn);
    } else {
        const int nb = min(n0 / 128 + wn, a.N / 128 - 1);
        const int shift = 8 * (int)(((size_t)nb * (a.K / GK) + kb) & 3);
        sw = dev_e8m0((*(const uint32_t *)(stage + ST_SW + 4 * wn) >> shift) & 0xFFu);
    }
    const float *sa = (const float *)(stage + ST_SA);
#pragma unroll
    for (int u = 0; u < 2; u++) o.cs[u] = sa[wm * 64 + u * 32 + col] * sw;
}

__device__ __forceinline__ v16f mfma(const v8i &w, const v8i &b, const v16f &c)
{
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, b, c, 0, 0, 0, E8M0_ONE, 0, E8M0_ONE);
}

/* acc[u] += p[u] * cs[u] over a tile's 16 outputs per lane */
__device__ __forceinline__ void promote(v16f (&acc)[2], const v16f (&p)[2], const float (&cs)[2])
{
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[u][e] = fmaf(p[u][e], cs[u], acc[u][e]);
}

/* One issue slot pattern per feature tile: the next tile's operand reads
 * first, then MFMA / direct load / eight promotion FMAs, four times, so the
 * vector ALU and the load path work in the shadow of the matrix unit. */
#define GEMM_SLOT(NVM)                                                         \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                         \
    __builtin_amdgcn_sched_group_barrier(0x010, NVM, 0);                       \
    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0)
#define GEMM_STEP_PATTERN(NDS, NVM_LAST)                                       \
    do {                                                                       \
        __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);                   \
        GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(NVM_LAST);         \
    } while (0)

/* One 128-wide K block. On entry `cur` holds block kb's first operands and
 * stage kb is visible; pp / csp are the previous block's tile-3 partial and
 * scales (zero before block 0). Tile t's MFMAs run while tile t-1 is
 * promoted. Between tiles 2 and 3 every wave has finished reading stage kb
 * and waits for its share of stage kb+1; after the barrier `nxt` is read from
 * stage kb+1 while tile 3 multiplies. Loads of block kb+2 go into the buffer
 * freed at the previous block's barrier; past the last block they repeat the
 * last block (harmless traffic that keeps every wait count constant). */
template <bool WF32S>
__device__ __forceinline__ void kblock(const GemmArgs &a, const DmaPlan &d, uint8_t *lds, int &buf,
                                       int kb, int nkb, const Ops &cur, Ops &nxt,
                                       v16f (&acc)[4][2], v16f (&pp)[2], float (&csp)[2],
                                       const v16f &zero, int n0, int wave, int wm, int wn,
                                       int col, int g)
{
    const uint8_t *stage = lds + buf * STAGE;
    const uint8_t *Ws = stage + ST_W + (wn * 128) * GK;
    int b1 = buf + 1; b1 = b1 == NSTAGE ? 0 : b1;
    int b2 = b1 + 1;  b2 = b2 == NSTAGE ? 0 : b2;
    uint8_t *dst = lds + b2 * STAGE;
    const int kl = min(kb + 2, nkb - 1);
    v16f p[2];
    v8i w1[2], w2[2], w3[2];

    /* tile 0 */
#pragma unroll
    for (int ks = 0; ks < 2; ks++) w1[ks] = lds_operand(Ws + (32 + col) * GK, 32 + col, ks, g);
    {
        const v16f q0 = mfma(cur.w0[0], cur.b[0][0], zero);
        const v16f q1 = mfma(cur.w0[0], cur.b[0][1], zero);
        issue_part<WF32S, 0>(a, d, dst, kl, wave);
        promote(acc[3], pp, csp);
        p[0] = mfma(cur.w0[1], cur.b[1][0], q0);
        p[1] = mfma(cur.w0[1], cur.b[1][1], q1);
    }
    /* tile 1 */
    v16f pn[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) w2[ks] = lds_operand(Ws + (64 + col) * GK, 64 + col, ks, g);
    {
        const v16f q0 = mfma(w1[0], cur.b[0][0], zero);
        const v16f q1 = mfma(w1[0], cur.b[0][1], zero);
        issue_part<WF32S, 1>(a, d, dst, kl, wave);
        promote(acc[0], p, cur.cs);
        pn[0] = mfma(w1[1], cur.b[1][0], q0);
        pn[1] = mfma(w1[1], cur.b[1][1], q1);
    }
    /* tile 2 */
#pragma unroll
    for (int ks = 0; ks < 2; ks++) w3[ks] = lds_operand(Ws + (96 + col) * GK, 96 + col, ks, g);
    {
        const v16f q0 = mfma(w2[0], cur.b[0][0], zero);
        const v16f q1 = mfma(w2[0], cur.b[0][1], zero);
        issue_part<WF32S, 2>(a, d, dst, kl, wave);
        promote(acc[1], pn, cur.cs);
        p[0] = mfma(w2[1], cur.b[1][0], q0);
        p[1] = mfma(w2[1], cur.b[1][1], q1);
    }
    GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(1);
    GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(1);
    GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(1); GEMM_SLOT(2);
    DSV4_ORDER();
    /* stage kb fully read by this wave (lgkmcnt 0); stage kb+1 landed for this
     * wave once only block kb+2's 13 loads are outstanding (vmcnt 13). The
     * barrier is a plain s_barrier: __syncthreads() would also drain the
     * loads of block kb+2. */
    __builtin_amdgcn_s_waitcnt(0x0070 | VMEM_PER_STAGE);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    DSV4_ORDER();
    /* tile 3, reading block kb+1's first operands meanwhile */
    load_ops<WF32S>(nxt, lds + b1 * STAGE, a, kb + 1, n0, wm, wn, col, g);
    {
        const v16f q0 = mfma(w3[0], cur.b[0][0], zero);
        const v16f q1 = mfma(w3[0], cur.b[0][1], zero);
        promote(acc[2], p, cur.cs);
        pp[0] = mfma(w3[1], cur.b[1][0], q0);
        pp[1] = mfma(w3[1], cur.b[1][1], q1);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 15, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
    }
    DSV4_ORDER();
    csp[0] = cur.cs[0];
    csp[1] = cur.cs[1];
    buf = b1;
}

template <bool WF32S, bool OUT_BF16>
__global__ __launch_bounds__(256) void k_gemm_fp8(GemmArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
    const int nkb = a.K / GK;
    const int col = lane & 31, g = lane >> 5;
    const DmaPlan d = make_plan<WF32S>(a, m0, n0, wave, lane);

    v16f acc[4][2], pp[2], zero;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        zero[e] = 0.0f;
        pp[0][e] = 0.0f;
        pp[1][e] = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) { acc[t][0][e] = 0.0f; acc[t][1][e] = 0.0f; }
    }
    float csp[2] = {0.0f, 0.0f};

    /* blocks 0 and 1 (block 1 repeats block 0 when K is one block) */
    issue_part<WF32S, 0>(a, d, lds, 0, wave);
    issue_part<WF32S, 1>(a, d, lds, 0, wave);
    issue_part<WF32S, 2>(a, d, lds, 0, wave);
    const int k1 = min(1, nkb - 1);
    issue_part<WF32S, 0>(a, d, lds + STAGE, k1, wave);
    issue_part<WF32S, 1>(a, d, lds + STAGE, k1, wave);
    issue_part<WF32S, 2>(a, d, lds + STAGE, k1, wave);
    __builtin_amdgcn_s_waitcnt(0x0F70 | VMEM_PER_STAGE);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    Ops o0, o1;
    load_ops<WF32S>(o0, lds, a, 0, n0, wm, wn, col, g);
    int buf = 0, kb = 0;
    for (; kb + 1 < nkb; kb += 2) {
        kblock<WF32S>(a, d, lds, buf, kb, nkb, o0, o1, acc, pp, csp, zero, n0, wave, wm, wn, col, g);
        kblock<WF32S>(a, d, lds, buf, kb + 1, nkb, o1, o0, acc, pp, csp, zero, n0, wave, wm, wn, col, g);
    }
    if (kb < nkb)
        kblock<WF32S>(a, d, lds, buf, kb, nkb, o0, o1, acc, pp, csp, zero, n0, wave, wm, wn, col, g);
    promote(acc[3], pp, csp);
    /* drain the trailing repeat loads before the workgroup's LDS is released */
    __builtin_amdgcn_s_waitcnt(0x0F70);

    __builtin_amdgcn_s_barrier();      /* every wave is done with the stage buffers */
    asm volatile("" ::: "memory");
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int u = 0; u < 2; u++)
            stage_frag<OUT_BF16>(lds, acc[t][u], wm * 64 + u * 32, wn * 128 + t * 32, col, g);
    __syncthreads();
    write_tile<OUT_BF16>(a, lds, m0, n0, threadIdx.x, 256);
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
    /* the loads address A and W with 32-bit per-lane byte offsets */
    if ((size_t)a.M * a.K > 0xFFFFFFFFull || (size_t)a.N * a.K > 0xFFFFFFFFull)
        return hipErrorInvalidValue;
    if (w_f32s) return out_bf16 ? launch_gemm<true, true>(a, st) : launch_gemm<true, false>(a, st);
    return out_bf16 ? launch_gemm<false, true>(a, st) : launch_gemm<false, false>(a, st);
}

} // namespace dsv4
