/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_decode_mx.hip - decode matvec, expert gate/up (+ SwiGLU) and routed
 * down (+ k-order combine) on the block-scaled MFMA of gfx950.
 *
 * What it replaces: the nt <= 31 bodies of fp8_n / fp4_n
 * (src/10_compute/dsv4_matmul_fp8.c:55-155, src/10_compute/dsv4_matmul_fp4.c:
 * 51-139), dsv4_expert_forward (src/10_compute/dsv4_ops.c:85-93) and the
 * compute of dsv4_layer_moe (src/70_decode/dsv4_layer.c:57-116).
 *
 * ARITHMETIC
 *   y[o] = sum_k W[o][k] x[k] runs on v_mfma_scale_f32_16x16x128_f8f6f4 with
 *   the packed weights as the A operand exactly as stored (FP4 e2m1 or FP8
 *   e4m3, 16 rows x 128 k per instruction) and their E8M0 block scales in the
 *   hardware scale operand, so no instruction decodes a weight. fp32 block
 *   scales (DSV4_WFP8_F32S) multiply each 128-k partial (one MFMA from zero)
 *   into the fp32 accumulator.
 *   The activations are the B operand. An fp32 activation is split exactly
 *   into NPART e4m3 "parts", each with its own E8M0 scale per 32-element
 *   block: part p is the round-to-nearest-even e4m3 of the block's residual
 *   after parts 0..p-1, at the smallest power-of-two scale that keeps the
 *   block's largest residual at or below 448. Every residual is exact in fp32
 *   and each part removes at least four significant bits, so after four
 *   parts what is left is below 2^-19 of the block maximum. The parts of one
 *   token occupy four of the MFMA's sixteen B columns and the four column
 *   results are added in a fixed order, so up to four tokens share one MFMA.
 *   Every part accumulates in a column of its own, so the hardware's
 *   alignment of products within an MFMA (about 14 bits below the largest
 *   product of a group) is relative to that part's own magnitude.
 *
 * OPERAND LAYOUT (measured on gfx950)
 *   Of a 128-k step, A lane l holds row l % 16: FP4 k in [32 g, +32) as 16
 *   bytes (low nibble first), FP8 k in [16 g, +16) in bytes 0-15 and
 *   [64 + 16 g, +16) in bytes 16-31, g = l / 16. B lane l holds column l % 16
 *   with the FP8 layout. Scale lane l covers row (A) or column (B) l % 16 and
 *   the 32-element block l / 16. Accumulator element e of lane l is row
 *   4 (l / 16) + e, column l % 16. A chunk (128 k) of a row is 64 (FP4) or
 *   128 (FP8) contiguous bytes, so four lanes of a row read it whole.
 *
 * SCHEDULE
 *   A wave owns one 16-row tile and a contiguous range of chunks of K. It
 *   issues its activation loads first, then its scale bytes, then every
 *   weight chunk of its range (loads complete in issue order), splits its
 *   activations into an LDS table in the B-operand layout while the weights
 *   are in flight, and then runs one MFMA per chunk. The four waves of a
 *   workgroup cover the four quarters of K of one tile and add their
 *   partials through LDS in a fixed order.
 *
 * Bound: HBM (each weight byte is read once per call).
 */
#include "dsv4_internal.h"

#include <algorithm>
#include <cstring>

namespace dsv4 {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int NPART = 4;                          /* e4m3 parts per activation */
constexpr int TAB_DATA = 4 * NPART * 32;          /* operand bytes of one chunk */
constexpr int TAB_CHUNK = TAB_DATA + 4 * NPART * 4; /* + one scale dword per (block, part) */
constexpr int TAB_ZERO = 64;                      /* zero operand + unit scale */
/* A mid table (the split of a routed slot's mid, the down projection's B
 * operand): per chunk of 128 the same operand bytes as TAB_DATA, then an E8M0
 * scale dword per (32-element block, 16-element half, part), so that the
 * writer of 16 consecutive mid rows splits them alone. */
constexpr int MTAB_DATA = TAB_DATA;
constexpr int MTAB_CHUNK = MTAB_DATA + 4 * 2 * NPART * 4;
constexpr int E8M0_ONE = 127;
constexpr int KSLICES = 4;                        /* waves per tile along K */

/* The zero B operand and unit scale for columns that carry no token, in
 * kernels whose split tables live in global memory. */
__device__ uint32_t g_zero_operand[16] = {0, 0, 0, 0, 0, 0, 0, 0, E8M0_ONE, 0, 0, 0, 0, 0, 0, 0};

/* Publication of mid's split tables between the workgroups of one launch,
 * without fences: a writer's stores are device-scope (written through the
 * XCD's L2) and acknowledged (vmcnt) before it adds one to the call's item
 * counter; the writer whose add completes the call sets a done flag on
 * another cache line. Readers poll only the flag, then read the tables with
 * device-scope loads, which bypass their CU's L1 and their XCD's L2, so a
 * line cached by the previous call is never used. The last workgroup to
 * leave sets every word back to zero (leave below). */
__device__ __forceinline__ void st_dev32(void *p, uint32_t v)
{
    __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int CPOL_SC1 = 16;                      /* buffer cache policy: device scope */
constexpr uint32_t BUF_WORD3 = 0x00020000u;       /* raw dword buffer */

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, (int)BUF_WORD3);
}

/* The calling workgroup's last access to the publication words: one add to
 * its group's leave counter, issued after every earlier access of the
 * caller has completed (vmcnt(0): stores acknowledged, loads and adds
 * returned). The workgroup whose add completes its group adds one to the top
 * counter; the one whose add completes the top counter is the last of the
 * launch, every other workgroup's accesses are then complete, so it sets all
 * the words back to zero for the next launch. Lane 0 only. */
__device__ __forceinline__ void leave(const OnePub &p)
{
    /* The leave counter is split in ONE_LEAVE_GROUPS group counters (by
     * workgroup id) and a top counter: the last leaver of a group adds once
     * to the top counter, and the last top add does the reset. All the
     * workgroups of a launch end at about the same time; one counter for
     * them all serialised their adds (2.5 us of a 21 us launch). */
    __builtin_amdgcn_s_waitcnt(0x0F70);            /* vmcnt(0) */
    asm volatile("" ::: "memory");
    const unsigned grp = blockIdx.x % ONE_LEAVE_GROUPS;
    const unsigned in_grp = (p.total - grp + ONE_LEAVE_GROUPS - 1) / ONE_LEAVE_GROUPS;
    const unsigned groups = p.total < ONE_LEAVE_GROUPS ? p.total : ONE_LEAVE_GROUPS;
    unsigned *top = p.leave + ONE_LEAVE_GROUPS * ONE_PUB_LINE_WORDS;
    const unsigned old = __hip_atomic_fetch_add(p.leave + grp * ONE_PUB_LINE_WORDS, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if (old != in_grp - 1) return;
    const unsigned told = __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (told != groups - 1) return;
    for (unsigned g = 0; g <= ONE_LEAVE_GROUPS; g++)
        __hip_atomic_store(p.count + g * ONE_PUB_LINE_WORDS, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (unsigned g = 0; g < ONE_LEAVE_GROUPS; g++)
        __hip_atomic_store(p.leave + g * ONE_PUB_LINE_WORDS, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* This wave's stores acknowledged, then one more item counted; the item that
 * completes the call raises the done flag (its add returns after every
 * earlier add, each issued after that item's stores were acknowledged).
 * Then the item leaves. */
__device__ __forceinline__ void publish(const OnePub &p, int lane)
{
    __builtin_amdgcn_s_waitcnt(0x0F70);            /* vmcnt(0) */
    asm volatile("" ::: "memory");
    if (lane == 0) {
        const unsigned old = __hip_atomic_fetch_add(p.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == p.items - 1) __hip_atomic_store(p.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        leave(p);
    }
}

/* Poll the done flag until it is set; false after spin_max polls, and at
 * once, without reading the flag, when spin_max is 0. */
__device__ __forceinline__ bool wait_done(const OnePub &p, unsigned spin_max)
{
    if (spin_max == 0) return false;
    for (unsigned n = 1;; n++) {
        const unsigned v = (unsigned)__builtin_amdgcn_readfirstlane(
            (int)__hip_atomic_load(p.done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (v != 0) break;
        if (n >= spin_max) return false;
        __builtin_amdgcn_s_sleep(16);              /* ~1k cycles between polls */
    }
    asm volatile("" ::: "memory");                 /* the table reads stay after the poll */
    return true;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

/* E8M0 byte of the smallest power of two 2^e with amax / 2^e <= 448
 * (448 = 1.75 * 2^8), for a finite amax >= 0; zero and fp32 subnormals take
 * byte 0 (2^-127). */
__device__ __forceinline__ int part_e8m0(float amax)
{
    const uint32_t b = __float_as_uint(amax);
    const int f = (int)(b >> 23);
    const int E = f - 8 + ((b & 0x7FFFFFu) > 0x600000u ? 1 : 0);
    return f == 0 ? 0 : min(max(E, 0), 254);
}

__device__ __forceinline__ uint32_t e4m3_pk4(float a, float b, float c, float d)
{
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
}

/* Split the eight activations of one lane -- a quarter of a 32-element block
 * whose four quarters sit in the four lanes of a DPP quad -- into NPART e4m3
 * parts: v = sum_p e4m3(code[p]) * 2^(E[p] - 127) + (the final residual).
 * code[p] holds the eight codes in element order, four per dword. */
__device__ __forceinline__ void split8(float (&v)[8], uint32_t (&code)[NPART][2], int (&E)[NPART])
{
#pragma unroll
    for (int p = 0; p < NPART; p++) {
        float m = fabsf(v[0]);
#pragma unroll
        for (int i = 1; i < 8; i++) m = fmaxf(m, fabsf(v[i]));
        m = fmaxf(m, dpp_f<DPP_QUAD_1032>(m));
        m = fmaxf(m, dpp_f<DPP_QUAD_2301>(m));
        E[p] = part_e8m0(m);
        const int e = E[p] - E8M0_ONE;
        float s[8];
#pragma unroll
        for (int i = 0; i < 8; i++) s[i] = ldexpf(v[i], -e);
        code[p][0] = e4m3_pk4(s[0], s[1], s[2], s[3]);
        code[p][1] = e4m3_pk4(s[4], s[5], s[6], s[7]);
        if (p + 1 < NPART) {
#pragma unroll
            for (int d = 0; d < 2; d++) {
                const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)code[p][d], false);
                const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)code[p][d], true);
                v[4 * d + 0] -= ldexpf(lo.x, e);
                v[4 * d + 1] -= ldexpf(lo.y, e);
                v[4 * d + 2] -= ldexpf(hi.x, e);
                v[4 * d + 3] -= ldexpf(hi.y, e);
            }
        }
    }
}

/* The same for a half block: 16 consecutive values, eight in each lane of a
 * lane pair (lanes 2 i, 2 i + 1), one E8M0 scale per part for the 16. */
__device__ __forceinline__ void split8_half(float (&v)[8], uint32_t (&code)[NPART][2], int (&E)[NPART])
{
#pragma unroll
    for (int p = 0; p < NPART; p++) {
        float m = fabsf(v[0]);
#pragma unroll
        for (int i = 1; i < 8; i++) m = fmaxf(m, fabsf(v[i]));
        m = fmaxf(m, dpp_f<DPP_QUAD_1032>(m));
        E[p] = part_e8m0(m);
        const int e = E[p] - E8M0_ONE;
        float s[8];
#pragma unroll
        for (int i = 0; i < 8; i++) s[i] = ldexpf(v[i], -e);
        code[p][0] = e4m3_pk4(s[0], s[1], s[2], s[3]);
        code[p][1] = e4m3_pk4(s[4], s[5], s[6], s[7]);
        if (p + 1 < NPART) {
#pragma unroll
            for (int d = 0; d < 2; d++) {
                const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)code[p][d], false);
                const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)code[p][d], true);
                v[4 * d + 0] -= ldexpf(lo.x, e);
                v[4 * d + 1] -= ldexpf(lo.y, e);
                v[4 * d + 2] -= ldexpf(hi.x, e);
                v[4 * d + 3] -= ldexpf(hi.y, e);
            }
        }
    }
}

/* Byte offsets, inside a chunk of a mid table, of part p's 16 codes of the
 * half block that starts at element k0 of the chunk (k0 % 16 == 0), and of
 * its scale dword. */
__device__ __forceinline__ int mtab_code_off(int k0, int p) { return (((k0 & 63) >> 4) * NPART + p) * 32 + (k0 >> 6) * 16; }
__device__ __forceinline__ int mtab_scale_off(int k0, int p) { return MTAB_DATA + ((k0 >> 4) * NPART + p) * 4; }

/* Split table of one wave's chunks for its tokens (LDS, wave-private).
 * For token t and chunk j (of the wave's ncw) the TAB_CHUNK bytes at
 * (t * ncw + j) * TAB_CHUNK hold:
 *   for lane group h and part p, 32 operand bytes at (h * NPART + p) * 32:
 *     bytes 0-15 = part p of the chunk's elements 16 h .. 16 h + 15,
 *     bytes 16-31 = part p of elements 64 + 16 h .. 64 + 16 h + 15;
 *   for 32-element block b of the chunk and part p, the E8M0 byte as a dword
 *     at TAB_DATA + (b * NPART + p) * 4.
 * After the last token's chunks: TAB_ZERO bytes, a zero operand and a unit
 * scale, read by the columns no token uses.
 * A "unit" is eight consecutive elements; unit u of the wave is token
 * u / (16 ncw), chunk (u / 16) % ncw, elements 8 (u % 16) .. +8 of the chunk. */
template <int UPL>
struct XUnits {
    float v[UPL][8];
};

template <int UPL, int NTHR = 64>
__device__ __forceinline__ void load_units(XUnits<UPL> &xu, const float *x, size_t x_ld,
                                           int ntok, int c0, int ncw, int lane)
{
    const int units = ntok * ncw * 16;
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        int u = NTHR * i + lane;
        u = u < units ? u : 0;
        const int per = ncw > 0 ? ncw * 16 : 16;
        const int t = u / per, rem = u - t * per;
        const float *src = x + (size_t)t * x_ld + (size_t)(c0 + (rem >> 4)) * 128 + 8 * (rem & 15);
        const f32x4 a = *(const f32x4 *)src, b = *(const f32x4 *)(src + 4);
        xu.v[i][0] = a.x; xu.v[i][1] = a.y; xu.v[i][2] = a.z; xu.v[i][3] = a.w;
        xu.v[i][4] = b.x; xu.v[i][5] = b.y; xu.v[i][6] = b.z; xu.v[i][7] = b.w;
    }
}

template <int UPL, int NTHR = 64>
__device__ __forceinline__ void store_units(uint8_t *tab, XUnits<UPL> &xu, int ntok, int ncw, int lane)
{
    const int units = ntok * ncw * 16;
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        const int u = NTHR * i + lane;
        if (u < units) {                            /* whole quads: units % 16 == 0 */
            uint32_t code[NPART][2];
            int E[NPART];
            split8(xu.v[i], code, E);
            const int per = ncw * 16;
            const int t = u / per, rem = u - t * per;
            const int j = rem >> 4, q16 = rem & 15, kk = 8 * q16;
            uint8_t *cb = tab + (size_t)(t * ncw + j) * TAB_CHUNK;
            const int h = (kk & 63) >> 4, half = kk >> 6;
#pragma unroll
            for (int p = 0; p < NPART; p++)
                *(uint2 *)(cb + (h * NPART + p) * 32 + half * 16 + (kk & 15)) =
                    make_uint2(code[p][0], code[p][1]);
            if ((q16 & 3) == 0) {
#pragma unroll
                for (int p = 0; p < NPART; p++)
                    *(int *)(cb + TAB_DATA + ((q16 >> 2) * NPART + p) * 4) = E[p];
            }
        }
    }
    if (lane < TAB_ZERO / 4)
        ((uint32_t *)(tab + (size_t)ntok * ncw * TAB_CHUNK))[lane] = lane == 8 ? E8M0_ONE : 0u;
}

/* B operand source of this lane: column col = 4 t + p is part p of token t. */
struct BSrc {
    const uint8_t *d;   /* operand bytes of chunk 0 */
    const uint8_t *s;   /* scale dword of chunk 0   */
    int step;           /* bytes per chunk          */
    const uint8_t *z;   /* zero operand, unit scale at z + 32 */
};

__device__ __forceinline__ BSrc lds_bsrc(const uint8_t *tab, int ntok, int ncw, int lane)
{
    const int col = lane & 15, h = lane >> 4, t = col >> 2, p = col & 3;
    BSrc b;
    b.z = tab + (size_t)ntok * ncw * TAB_CHUNK;
    if (t < ntok) {
        const uint8_t *cb = tab + (size_t)t * ncw * TAB_CHUNK;
        b.d = cb + (h * NPART + p) * 32;
        b.s = cb + TAB_DATA + (h * NPART + p) * 4;
        b.step = TAB_CHUNK;
    } else {
        b.d = b.z;
        b.s = b.z + 32;
        b.step = 0;
    }
    return b;
}

/* Chunk j's operand; j >= ncw (a wave with fewer chunks than CPW) reads the
 * zero operand, so its MFMA adds zero (the A side re-reads a chunk of the same
 * row, so a NaN weight there is already in the row's sum). */
__device__ __forceinline__ v8i ld_b(const BSrc &b, int j, int ncw)
{
    const uint8_t *p = j < ncw ? b.d + j * b.step : b.z;
    const u32x4 lo = *(const u32x4 *)p;
    const u32x4 hi = *(const u32x4 *)(p + 16);
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
}

__device__ __forceinline__ int ld_bs(const BSrc &b, int j, int ncw)
{
    return *(const int *)(j < ncw ? b.s + j * b.step : b.z + 32);
}

/* A operand of one chunk: FP4 16 bytes, FP8 32 bytes. */
template <bool FP4>
struct AChunk {
    u32x4 q[FP4 ? 1 : 2];
};

/* FP4 chunk c of the lane's row (16 rows x 64 bytes per instruction) */
__device__ __forceinline__ void ld_a(AChunk<true> &a, const uint8_t *wrow, int c, int g)
{
    a.q[0] = ld_stream16(wrow + 64 * c + 16 * g);
}

/* FP8 chunk c of a 16-row tile as whole 128-byte lines: q[0] from rows 0-7
 * (wlo: row r0 + lane % 8), q[1] from rows 8-15 (whi), lane r8 + 8 h + 16 g
 * taking bytes 16 (4 h + g) of its rows' chunk; mfma_a trades halves between
 * lanes i and i ^ 8 to form the operand of row lane % 16. (Loading the
 * operand halves directly, bytes 16 g and 64 + 16 g, read 16 half lines per
 * instruction.) */
__device__ __forceinline__ void ld_a(AChunk<false> &a, const uint8_t *wlo, const uint8_t *whi, int c,
                                     int lane)
{
    const int piece = 16 * (4 * ((lane >> 3) & 1) + (lane >> 4));
    a.q[0] = ld_stream16(wlo + 128 * c + piece);
    a.q[1] = ld_stream16(whi + 128 * c + piece);
}

template <bool FP4>
__device__ __forceinline__ v4f mfma_a(const AChunk<FP4> &a, const v8i &b, const v4f &c, int sa, int sb)
{
    v8i av;
    if constexpr (FP4) {
        av[0] = (int)a.q[0].x; av[1] = (int)a.q[0].y; av[2] = (int)a.q[0].z; av[3] = (int)a.q[0].w;
        av[4] = 0; av[5] = 0; av[6] = 0; av[7] = 0;
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, c, 4, 0, 0, sa, 0, sb);
    } else {
        /* row r8 + 8 h of lane group g wants bytes 16 g (half 0) and
         * 64 + 16 g (half 1) of its chunk: rows 0-7 hold half 0 themselves
         * and take half 1 from lane ^ 8; rows 8-15 the other way round */
        const bool odd = (threadIdx.x >> 3) & 1;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int s0 = __builtin_amdgcn_mov_dpp((int)a.q[0][e], DPP_ROW_ROR8, 0xF, 0xF, false);
            const int s1 = __builtin_amdgcn_mov_dpp((int)a.q[1][e], DPP_ROW_ROR8, 0xF, 0xF, false);
            av[e] = odd ? s1 : (int)a.q[0][e];
            av[4 + e] = odd ? (int)a.q[1][e] : s0;
        }
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, c, 0, 0, 0, sa, 0, sb);
    }
}

/* FP4 A operand with its E8M0 scale in byte SEL of sa4. */
template <int SEL>
__device__ __forceinline__ v4f mfma_f4_sel(const u32x4 &q, const v8i &b, const v4f &c, uint32_t sa4, int sb)
{
    v8i av;
    av[0] = (int)q.x; av[1] = (int)q.y; av[2] = (int)q.z; av[3] = (int)q.w;
    av[4] = 0; av[5] = 0; av[6] = 0; av[7] = 0;
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, c, 4, 0, SEL, (int)sa4, 0, sb);
}

/* The scale side of one matrix for a wave's chunk range: FP4 a byte per lane
 * and chunk (row l % 16, block 4 c + l / 16); FP8 one value per chunk for the
 * whole tile (the 16 rows lie in one row block), E8M0 byte or fp32 bits. */
template <int FMT, int CPW>
struct AScales {
    uint32_t v[CPW];
};

template <int FMT, int CPW>
__device__ __forceinline__ void ld_ascales(AScales<FMT, CPW> &s, const void *S, int sc_cols,
                                           int blk_r, int row, int tile_row0, int c0, int ncw, int g,
                                           int row_max)
{
    if constexpr (FMT == FMT_FP4_E8M0) {
        /* Row r's bytes for the wave's chunks, [4 c0, 4 c0 + 4 CPW), are
         * contiguous: CPW / 4 lanes load them as 16-byte pieces (one load per
         * row piece instead of one per chunk), then every lane fetches the
         * dword of chunk j from the lane holding it and keeps its block's byte.
         * Needs whole pieces inside the row and 16-byte aligned rows. */
        constexpr int NL = CPW / 4;
        const uint8_t *S8 = (const uint8_t *)S;
        bool wide = CPW >= 4 && ncw == CPW && (sc_cols & 15) == 0 && (c0 & 3) == 0 &&
                    ((uintptr_t)S8 & 15u) == 0;
        wide = __builtin_amdgcn_readfirstlane((int)wide) != 0;
        if constexpr (CPW >= 4) {
            if (wide) {
                const int lane = threadIdx.x & 63;
                const int L = lane % (16 * NL);
                const int rl = min(tile_row0 + L / NL, row_max);   /* tile row loaded by this lane */
                const u32x4 piece = *gptr((const u32x4 *)(S8 + (size_t)(rl / blk_r) * sc_cols +
                                                          4 * c0 + 16 * (L % NL)));
#pragma unroll
                for (int j = 0; j < CPW; j++) {
                    const int src = ((lane & 15) * NL + j / 4) * 4;
                    const uint32_t d = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)piece[j & 3]);
                    s.v[j] = (d >> (8 * g)) & 0xFFu;
                }
                return;
            }
        }
#pragma unroll
        for (int j = 0; j < CPW; j++) {
            const int c = c0 + (j < ncw ? j : 0);
            s.v[j] = ld_u8(S, (size_t)(row / blk_r) * sc_cols + 4 * c + g);
        }
    } else {
#pragma unroll
        for (int j = 0; j < CPW; j++) {
            const int c = c0 + (j < ncw ? j : 0);
            if constexpr (FMT == FMT_FP8_E8M0) s.v[j] = ld_u8(S, (size_t)(tile_row0 / blk_r) * sc_cols + c);
            else s.v[j] = gptr((const uint32_t *)S)[(size_t)(tile_row0 / blk_r) * sc_cols + c];
        }
    }
}

/* acc += W[tile rows][chunks] . B over the wave's CPW chunk slots; slots
 * j >= ncw multiply the zero operand. Straight-line: every register index
 * is a compile-time constant. */
template <int FMT, int CPW>
__device__ __forceinline__ v4f mma_rows(const AChunk<FMT == FMT_FP4_E8M0> (&a)[CPW],
                                        const AScales<FMT, CPW> &s, const BSrc &bs, int ncw)
{
    constexpr bool FP4 = FMT == FMT_FP4_E8M0;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        const v8i b = ld_b(bs, j, ncw);
        const int sb = ld_bs(bs, j, ncw);
        if constexpr (FMT == FMT_FP8_F32S) {
            const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
            const v4f p = mfma_a<FP4>(a[j], b, zero, E8M0_ONE, sb);
            const float sw = __uint_as_float(s.v[j]);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = fmaf(p[e], sw, acc[e]);
        } else {
            acc = mfma_a<FP4>(a[j], b, acc, (int)s.v[j], sb);
        }
    }
    return acc;
}

/* Sum the four part columns of every token: afterwards the lane of column
 * 4 t (of each 16-lane group h) holds token t's rows 4 h .. 4 h + 3. */
__device__ __forceinline__ void sum_parts(v4f &acc)
{
#pragma unroll
    for (int e = 0; e < 4; e++) {
        acc[e] = acc[e] + dpp_f<DPP_QUAD_1032>(acc[e]);
        acc[e] = acc[e] + dpp_f<DPP_QUAD_2301>(acc[e]);
    }
}

/* B operand of chunk pair m from a mid table (chunk index relative to `tab`):
 * column c = 8 par + 2 p + hf carries part p of half hf of every 32-element
 * block of chunk c0 + 2 m + par. Lane l (column l % 16, lane group g = l / 16)
 * holds k in [16 g, +16) and [64 + 16 g, +16), which lie in half g % 2 of
 * blocks g / 2 and 2 + g / 2: its bytes are the table's when hf == g % 2 and
 * the zero operand's otherwise. Its scale is the column's scale of block g. */
struct BMid {
    const uint8_t *d, *s;
    int dstep, sstep;
};

__device__ __forceinline__ BMid bmid_src(const uint8_t *tab, int c0, const uint8_t *zero, int lane)
{
    const int col = lane & 15, g = lane >> 4;
    const int par = col >> 3, p = (col >> 1) & 3, hf = col & 1;
    const uint8_t *cb = tab + (size_t)(c0 + par) * MTAB_CHUNK;
    BMid b;
    const bool live = hf == (g & 1);
    b.d = live ? cb + (g * NPART + p) * 32 : zero;
    b.dstep = live ? 2 * MTAB_CHUNK : 0;
    b.s = cb + MTAB_DATA + ((g * 2 + hf) * NPART + p) * 4;
    b.sstep = 2 * MTAB_CHUNK;
    return b;
}

/* Column sums over the eight columns of each chunk of a mid-table pair
 * accumulator ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)), written as 8
 * even-chunk and 8 odd-chunk row partials to dst[0..7], dst[8..15]. */
__device__ __forceinline__ void sum_cols8(v4f &acc)
{
#pragma unroll
    for (int e = 0; e < 4; e++) {
        acc[e] = acc[e] + dpp_f<DPP_QUAD_1032>(acc[e]);
        acc[e] = acc[e] + dpp_f<DPP_QUAD_2301>(acc[e]);
        acc[e] = acc[e] + dpp_f<DPP_ROW_HALF_MIRROR>(acc[e]);
    }
}

__device__ __forceinline__ void store_mid_partials(v4f acc, float *dst, int lane)
{
    sum_cols8(acc);
    const int q = lane >> 4, col = lane & 15;
    if (col == 0 && q < 2) {
#pragma unroll
        for (int e = 0; e < 4; e++) dst[4 * q + e] = acc[e];
    }
    if (col == 8 && q >= 2) {
#pragma unroll
        for (int e = 0; e < 4; e++) dst[8 + 4 * (q - 2) + e] = acc[e];
    }
}

/* The expert of gate/up slot `slot`: by value from the kernel arguments (host
 * routing), the direct descriptor, or table[idx[slot]]; a routing id out of
 * range is reported. */
__device__ __forceinline__ unsigned gateup_expert(const GateUpMxArgs &a, int slot, DSV4ExpertW &e)
{
    if (a.by_value) {
        e = a.routed[slot];
        return 0;
    }
    if (a.use_direct) {
        e = a.direct;
        return 0;
    }
    const int id = ld_uniform(a.idx, slot);
    if (id < 0 || id >= a.n_experts) return ST_BAD_EXPERT_ID;
    e = ld_uniform(a.table, id);
    return 0;
}

/* The down matrix of routed slot k and its routing weight. */
__device__ __forceinline__ unsigned down_expert(const DownMxArgs &a, int k, DSV4QMat &m)
{
    if (a.by_value) {
        m = a.w2v[k];
        return 0;
    }
    const int id = ld_uniform(a.idx, k);
    if (id < 0 || id >= a.n_experts) return ST_BAD_EXPERT_ID;
    m = ld_uniform(a.table, id).w2;
    return 0;
}

__device__ __forceinline__ float route_weight(const DownMxArgs &a, int k)
{
    return a.by_value ? a.wv[k] : ld_uniform(a.w, k);
}

template <int FMT>
__device__ __forceinline__ bool mx_desc_ok(const DSV4QMat &m, int rows, int cols)
{
    const int want = FMT == FMT_FP4_E8M0 ? DSV4_WFP4
                   : FMT == FMT_FP8_F32S ? DSV4_WFP8_F32S : DSV4_WFP8;
    const int blk_c = FMT == FMT_FP4_E8M0 ? 32 : 128;
    const bool br = FMT == FMT_FP4_E8M0 ? m.blk_r > 0 : (m.blk_r > 0 && m.blk_r % 16 == 0);
    return m.wdt == want && m.rows == rows && m.cols == cols && m.blk_c == blk_c && br &&
           m.w != nullptr && m.s != nullptr && ((uintptr_t)m.w & 15u) == 0 &&
           (FMT != FMT_FP8_F32S || ((uintptr_t)m.s & 3u) == 0);
}

__device__ __forceinline__ float qnan_f() { return __uint_as_float(0x7FC00000u); }

/* ------------------------------------------------------------- GEMV --- */

/* x split once for every row block: unit u (eight elements; the four units
 * of a 32-element block in one DPP quad) of token t, chunk c, written where
 * store_units puts it, in token t's table of all nc chunks. */
__global__ __launch_bounds__(256) void k_split_x_tab(uint8_t *tab, const float *x, int x_ld, int nt, int nc)
{
    const int units = nt * nc * 16;                        /* a multiple of 16: whole quads */
    const int u0 = (int)blockIdx.x * 256 + (int)threadIdx.x;
    const bool live = u0 < units;
    const int u = live ? u0 : 0;
    const int per = nc * 16;
    const int t = u / per, rem = u - t * per, c = rem >> 4, q16 = rem & 15, kk = 8 * q16;
    const float *src = x + (size_t)t * x_ld + (size_t)c * 128 + kk;
    const f32x4 a = *(const f32x4 *)src, b = *(const f32x4 *)(src + 4);
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t code[NPART][2];
    int E[NPART];
    split8(v, code, E);
    if (!live) return;
    uint8_t *cb = tab + ((size_t)t * nc + c) * TAB_CHUNK;
    const int h = (kk & 63) >> 4, half = kk >> 6;
#pragma unroll
    for (int p = 0; p < NPART; p++)
        *(uint2 *)(cb + (h * NPART + p) * 32 + half * 16 + (kk & 15)) = make_uint2(code[p][0], code[p][1]);
    if ((q16 & 3) == 0) {
#pragma unroll
        for (int p = 0; p < NPART; p++) *(int *)(cb + TAB_DATA + ((q16 >> 2) * NPART + p) * 4) = E[p];
    }
}

/* This wave's part of token group t0's split tables (ntok tokens, chunks
 * cb0 .. cb0 + ncw - 1) from the table k_split_x_tab wrote, 16 bytes a lane:
 * the loads, then (copy_tab_store) the LDS writes and the zero operand. */
template <int NT, int CPW>
struct TabCopy {
    static constexpr int PER = (CPW * TAB_CHUNK / 16 + 63) / 64;   /* 16-byte pieces per lane and token */
    u32x4 q[NT][PER];
};

template <int NT, int CPW>
__device__ __forceinline__ void copy_tab_load(TabCopy<NT, CPW> &c, const uint8_t *tab, int nc, int t0, int ntok,
                                              int cb0, int ncw, int lane)
{
    const int pieces = ncw * (TAB_CHUNK / 16);
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < TabCopy<NT, CPW>::PER; i++) {
            const int r = 64 * i + lane;
            if (t < ntok && r < pieces)
                c.q[t][i] = *(const u32x4 *)(tab + ((size_t)(t0 + t) * nc + cb0) * TAB_CHUNK + 16 * r);
        }
}

template <int NT, int CPW>
__device__ __forceinline__ void copy_tab_store(uint8_t *lt, const TabCopy<NT, CPW> &c, int ntok, int ncw, int lane)
{
    const int pieces = ncw * (TAB_CHUNK / 16);
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < TabCopy<NT, CPW>::PER; i++) {
            const int r = 64 * i + lane;
            if (t < ntok && r < pieces) *(u32x4 *)(lt + (size_t)t * ncw * TAB_CHUNK + 16 * r) = c.q[t][i];
        }
    if (lane < TAB_ZERO / 4)
        ((uint32_t *)(lt + (size_t)ntok * ncw * TAB_CHUNK))[lane] = lane == 8 ? E8M0_ONE : 0u;
}

/* The small-batch matvec on x split beforehand (k_split_x_tab): a workgroup
 * owns 16 rows and token groups blockIdx.y * gpw .. + gpw - 1 of NT tokens;
 * the rows' weight operands are loaded once and held while it walks its
 * groups, each group's tables copied one group ahead. Every token's MFMA
 * steps are those of k_gemv_mx, so its bits are too. (One token group per
 * workgroup re-read the whole matrix per group: 31 tokens of a 4096 x 4096
 * FP8 matrix in groups of two streamed 268 MB.) */
template <int FMT, int CPW, int NT>
__global__ __launch_bounds__(256) void k_gemv_mx_tab(GemvMxArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool FP4 = FMT == FMT_FP4_E8M0;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int r0 = blockIdx.x * 16;
    const int ngroups = (a.nt + NT - 1) / NT;
    const int g_lo = blockIdx.y * a.gpw, g_hi = min(ngroups, g_lo + a.gpw);
    const int nc = a.cols / 128;
    const int c0 = wave * a.ncw;
    const int ncw = max(0, min(a.ncw, nc - c0));
    const int cb0 = ncw > 0 ? c0 : 0;                      /* loads stay inside the row */
    const int g = lane >> 4;
    const int row = min(r0 + (lane & 15), a.rows - 1);
    const uint8_t *wrow = a.W + (size_t)row * a.row_bytes;
    const uint8_t *wlo = a.W + (size_t)min(r0 + (lane & 7), a.rows - 1) * a.row_bytes;
    const uint8_t *whi = a.W + (size_t)min(r0 + 8 + (lane & 7), a.rows - 1) * a.row_bytes;
    const size_t tab_bytes = (size_t)NT * a.ncw * TAB_CHUNK + TAB_ZERO;
    uint8_t *tab = lds + wave * tab_bytes;
    float *red = (float *)(lds + KSLICES * tab_bytes);     /* [KSLICES][NT][16] */
    auto group_tokens = [&](int tg) { return min(NT, a.nt - tg * NT); };

    TabCopy<NT, CPW> tc;
    copy_tab_load<NT, CPW>(tc, a.tab, nc, g_lo * NT, group_tokens(g_lo), cb0, ncw, lane);
    DSV4_ORDER();
    AScales<FMT, CPW> sc;
    ld_ascales<FMT, CPW>(sc, a.S, a.sc_cols, a.blk_r, row, r0, cb0, ncw, g, a.rows - 1);
    DSV4_ORDER();
    AChunk<FP4> w[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        if constexpr (FP4) ld_a(w[j], wrow, cb0 + (j < ncw ? j : 0), g);
        else ld_a(w[j], wlo, whi, cb0 + (j < ncw ? j : 0), lane);
    }
    DSV4_ORDER();
    for (int tg = g_lo; tg < g_hi; tg++) {
        const int t0 = tg * NT, ntok = group_tokens(tg);
        TabCopy<NT, CPW> tn;
        if (tg + 1 < g_hi) copy_tab_load<NT, CPW>(tn, a.tab, nc, t0 + NT, group_tokens(tg + 1), cb0, ncw, lane);
        copy_tab_store<NT, CPW>(tab, tc, ntok, ncw, lane);
        v4f acc = mma_rows<FMT, CPW>(w, sc, lds_bsrc(tab, ntok, ncw, lane), ncw);
        sum_parts(acc);
        const int col = lane & 15;
        if ((col & 3) == 0 && (col >> 2) < ntok) {
#pragma unroll
            for (int e = 0; e < 4; e++) red[(wave * NT + (col >> 2)) * 16 + 4 * g + e] = acc[e];
        }
        __syncthreads();
        const int tid = threadIdx.x;
        if (tid < ntok * 16) {
            const int t = tid >> 4, rr = tid & 15;
            float s = red[t * 16 + rr];
#pragma unroll
            for (int k = 1; k < KSLICES; k++) s += red[(k * NT + t) * 16 + rr];
            if (r0 + rr < a.rows) a.y[(size_t)(t0 + t) * a.y_ld + r0 + rr] = s;
        }
        __syncthreads();                                   /* red is rewritten next group */
        if (tg + 1 < g_hi) tc = tn;
    }
}

template <int FMT, int CPW, int NT>
__global__ __launch_bounds__(256) void k_gemv_mx(GemvMxArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool FP4 = FMT == FMT_FP4_E8M0;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int r0 = blockIdx.x * 16;
    const int t0 = blockIdx.y * a.tpg;
    const int ntok = min(a.tpg, a.nt - t0);
    const int nc = a.cols / 128;
    const int c0 = wave * a.ncw;
    const int ncw = max(0, min(a.ncw, nc - c0));
    const int cb0 = ncw > 0 ? c0 : 0;                      /* loads stay inside the row */
    const int g = lane >> 4;
    const int row = min(r0 + (lane & 15), a.rows - 1);
    const uint8_t *wrow = a.W + (size_t)row * a.row_bytes;
    const uint8_t *wlo = a.W + (size_t)min(r0 + (lane & 7), a.rows - 1) * a.row_bytes;
    const uint8_t *whi = a.W + (size_t)min(r0 + 8 + (lane & 7), a.rows - 1) * a.row_bytes;
    const size_t tab_bytes = (size_t)a.tpg * a.ncw * TAB_CHUNK + TAB_ZERO;
    uint8_t *tab = lds + wave * tab_bytes;
    float *red = (float *)(lds + KSLICES * tab_bytes);     /* [KSLICES][tpg][16] */
    constexpr int UPL = (NT * CPW * 16 + 63) / 64;

    XUnits<UPL> xu;
    load_units<UPL>(xu, a.x + (size_t)t0 * a.x_ld, a.x_ld, ntok, cb0, ncw, lane);
    DSV4_ORDER();
    AScales<FMT, CPW> sc;
    ld_ascales<FMT, CPW>(sc, a.S, a.sc_cols, a.blk_r, row, r0, cb0, ncw, g, a.rows - 1);
    DSV4_ORDER();
    AChunk<FP4> w[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        if constexpr (FP4) ld_a(w[j], wrow, cb0 + (j < ncw ? j : 0), g);
        else ld_a(w[j], wlo, whi, cb0 + (j < ncw ? j : 0), lane);
    }
    DSV4_ORDER();
    store_units<UPL>(tab, xu, ntok, ncw, lane);
    v4f acc = mma_rows<FMT, CPW>(w, sc, lds_bsrc(tab, ntok, ncw, lane), ncw);
    sum_parts(acc);
    const int col = lane & 15;
    if ((col & 3) == 0 && (col >> 2) < ntok) {
#pragma unroll
        for (int e = 0; e < 4; e++) red[(wave * a.tpg + (col >> 2)) * 16 + 4 * g + e] = acc[e];
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < ntok * 16) {
        const int t = tid >> 4, rr = tid & 15;
        float s = red[t * 16 + rr];
#pragma unroll
        for (int k = 1; k < KSLICES; k++) s += red[(k * a.tpg + t) * 16 + rr];
        if (r0 + rr < a.rows) a.y[(size_t)(t0 + t) * a.y_ld + r0 + rr] = s;
    }
}

/* ----------------------------------------------------- expert gate/up --- */

/* Eight waves: two 16-row tiles of w1 and w3 x four quarters of K. One
 * workgroup per (slot, 32-row group). Writes mid = SwiGLU(w1.x, w3.x) and,
 * when a.msplit is set, the split table of mid for the down projection. */
template <int FMT, int CPW>
__device__ __forceinline__ void gateup_mx_body(const GateUpMxArgs &a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool FP4 = FMT == FMT_FP4_E8M0;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int tile = wave >> 2, slice = wave & 3;
    const int groups = a.inter / 32;
    const int slot = blockIdx.x / groups;
    const int j0 = (blockIdx.x - slot * groups) * 32;        /* first mid row of the group */
    const int nc = a.hidden / 128;
    const int c0 = slice * a.ncw;
    const int ncw = max(0, min(a.ncw, nc - c0));
    const int cb0 = ncw > 0 ? c0 : 0;                      /* loads stay inside the row */
    const int g = lane >> 4;
    const int r0 = j0 + 16 * tile;
    const int row = r0 + (lane & 15);
    const size_t tab_bytes = (size_t)a.ncw * TAB_CHUNK + TAB_ZERO;
    uint8_t *tab = lds + wave * tab_bytes;
    float *red = (float *)(lds + 8 * tab_bytes);               /* [2 tiles][4][2 mats][16] */
    float *mid = a.mid + (size_t)slot * a.mid_ld;
    constexpr int UPL = (CPW * 16 + 63) / 64;

    DSV4ExpertW e;
    unsigned bad = gateup_expert(a, slot, e);
    if (!bad && (!mx_desc_ok<FMT>(e.w1, a.inter, a.hidden) || !mx_desc_ok<FMT>(e.w3, a.inter, a.hidden)))
        bad = ST_BAD_DESCRIPTOR;
    if (bad) {
        if (threadIdx.x == 0) atomicOr(a.status, bad);
        if (threadIdx.x < 32) mid[j0 + threadIdx.x] = qnan_f();
        /* NaN block scales (E8M0 255) make the down projection of this slot NaN */
        if (a.msplit && threadIdx.x < 2 * NPART)
            *(int *)(a.msplit + (size_t)slot * a.msplit_ld + (size_t)(j0 >> 7) * MTAB_CHUNK +
                     mtab_scale_off((j0 & 127) + 16 * (threadIdx.x / NPART), threadIdx.x % NPART)) = 255;
        return;
    }
    const int row_bytes = FP4 ? a.hidden / 2 : a.hidden;
    const int sc_cols = FP4 ? a.hidden / 32 : a.hidden / 128;
    const uint8_t *w1r = (const uint8_t *)e.w1.w + (size_t)row * row_bytes;
    const uint8_t *w3r = (const uint8_t *)e.w3.w + (size_t)row * row_bytes;
    const size_t lo_off = (size_t)(r0 + (lane & 7)) * row_bytes, hi_off = lo_off + (size_t)8 * row_bytes;

    XUnits<UPL> xu;
    load_units<UPL>(xu, a.x, 0, 1, cb0, ncw, lane);
    DSV4_ORDER();
    AScales<FMT, CPW> s1, s3;
    ld_ascales<FMT, CPW>(s1, e.w1.s, sc_cols, e.w1.blk_r, row, r0, cb0, ncw, g, a.inter - 1);
    ld_ascales<FMT, CPW>(s3, e.w3.s, sc_cols, e.w3.blk_r, row, r0, cb0, ncw, g, a.inter - 1);
    DSV4_ORDER();
    AChunk<FP4> w1[CPW], w3[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        const int c = cb0 + (j < ncw ? j : 0);
        if constexpr (FP4) {
            ld_a(w1[j], w1r, c, g);
            ld_a(w3[j], w3r, c, g);
        } else {
            ld_a(w1[j], (const uint8_t *)e.w1.w + lo_off, (const uint8_t *)e.w1.w + hi_off, c, lane);
            ld_a(w3[j], (const uint8_t *)e.w3.w + lo_off, (const uint8_t *)e.w3.w + hi_off, c, lane);
        }
    }
    DSV4_ORDER();
    store_units<UPL>(tab, xu, 1, ncw, lane);
    const BSrc bs = lds_bsrc(tab, 1, ncw, lane);
    v4f gacc = mma_rows<FMT, CPW>(w1, s1, bs, ncw);
    v4f uacc = mma_rows<FMT, CPW>(w3, s3, bs, ncw);
    sum_parts(gacc);
    sum_parts(uacc);
    if ((lane & 15) == 0) {
#pragma unroll
        for (int e2 = 0; e2 < 4; e2++) {
            red[((tile * 4 + slice) * 2 + 0) * 16 + 4 * g + e2] = gacc[e2];
            red[((tile * 4 + slice) * 2 + 1) * 16 + 4 * g + e2] = uacc[e2];
        }
    }
    __syncthreads();
    if (wave != 0) return;

    /* lanes 0..31: mid row j0 + lane; lanes 32..63 carry zeros through the
     * block reductions below */
    float v = 0.0f;
    if (lane < 32) {
        const int t = lane >> 4, rr = lane & 15;
        float gs = red[((t * 4 + 0) * 2 + 0) * 16 + rr], us = red[((t * 4 + 0) * 2 + 1) * 16 + rr];
#pragma unroll
        for (int k = 1; k < 4; k++) {
            gs += red[((t * 4 + k) * 2 + 0) * 16 + rr];
            us += red[((t * 4 + k) * 2 + 1) * 16 + rr];
        }
        v = dev_swiglu(gs, us, a.limit);
        mid[j0 + lane] = v;
    }
    if (!a.msplit) return;

    /* split of the two 16-element halves of block j0 / 32 of mid, each with
     * its own scales, in the down projection's table layout (chunk j0 / 128) */
    uint8_t *cb = a.msplit + (size_t)slot * a.msplit_ld + (size_t)(j0 >> 7) * MTAB_CHUNK;
    const int kk = (j0 & 127) + (lane & 31);
    uint8_t *dst = cb + mtab_code_off(kk & ~15, 0) + (kk & 15);
#pragma unroll
    for (int p = 0; p < NPART; p++) {
        float m = fabsf(v);
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        const int E = part_e8m0(m);
        const int ex = E - E8M0_ONE;
        const uint32_t q = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(v, -ex), 0.0f, 0, false) & 0xFFu;
        if (lane < 32) dst[p * 32] = (uint8_t)q;
        if (lane < 32 && (lane & 15) == 0) *(int *)(cb + mtab_scale_off(kk, p)) = E;
        v -= ldexpf(__builtin_amdgcn_cvt_pk_f32_fp8((int)q, false)[0], ex);
    }
}

/* Four waves per SIMD (two workgroups per CU, every workgroup of a 6-expert
 * decode resident at once) for FP4 with up to eight chunks per wave; the
 * larger variants keep their registers. */
template <int FMT, int CPW>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_gateup_mx(GateUpMxArgs a)
{
    gateup_mx_body<FMT, CPW>(a);
}

template <int FMT, int CPW>
__global__ __launch_bounds__(512) void k_gateup_mx_wide(GateUpMxArgs a)
{
    gateup_mx_body<FMT, CPW>(a);
}

/* ------------------------------------------------- routed down + combine --- */

/* One workgroup per 16 output rows; two waves per routed expert k, each over
 * half of the inter dimension, reading the split table that k_gateup_mx wrote
 * for slot k. After the barrier the first 16 lanes combine in k order:
 * out = 0; out += w[k] * y_k (product and sum separately rounded); out += shared. */
template <int CPW>
__global__ __launch_bounds__(1024) void k_down_mx(DownMxArgs a)
{
    __shared__ float ylds[16][2][16];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int k = wave >> 1, half = wave & 1;
    const int r0 = blockIdx.x * 16;
    const int nc = a.inter / 128;
    const int c0 = half * a.ncw;
    const int ncw = max(0, min(a.ncw, nc - c0));
    const int cb0 = ncw > 0 ? c0 : 0;                      /* loads stay inside the row */
    const int g = lane >> 4, col = lane & 15;
    const int row = min(r0 + col, a.hidden - 1);
    const int row_bytes = a.inter / 2, sc_cols = a.inter / 32;

    unsigned bad = 0;
    DSV4QMat m;
    bad = down_expert(a, k, m);
    if (!bad && !mx_desc_ok<FMT_FP4_E8M0>(m, a.hidden, a.inter)) bad = ST_BAD_DESCRIPTOR;
    float mine[4] = {qnan_f(), qnan_f(), qnan_f(), qnan_f()};
    if (!bad) {
        /* B: column c = 2 p + hf < 8 is part p of half hf of slot k's mid
         * (data in the lanes whose k range lies in half hf, see bmid_src) */
        const uint8_t *tb = a.msplit + (size_t)k * a.msplit_ld;
        const uint8_t *zero = (const uint8_t *)g_zero_operand;
        const int p = (col >> 1) & 3, hf = col & 1;
        const bool live = col < 8 && hf == (g & 1);
        const uint8_t *bd = live ? tb + (g * NPART + p) * 32 : zero;
        const int dstep = live ? MTAB_CHUNK : 0;
        const uint8_t *bsc = col < 8 ? tb + MTAB_DATA + ((g * 2 + hf) * NPART + p) * 4 : zero + 32;
        const int sstep = col < 8 ? MTAB_CHUNK : 0;
        v8i bv[CPW];
        int bsv[CPW];
#pragma unroll
        for (int j = 0; j < CPW; j++) {
            /* slots past the wave's chunks read the zero operand (adds zero) */
            const uint8_t *pd = j < ncw ? bd + (size_t)(cb0 + j) * dstep : zero;
            const uint8_t *ps = j < ncw ? bsc + (size_t)(cb0 + j) * sstep : zero + 32;
            const u32x4 lo = *gptr((const u32x4 *)pd);
            const u32x4 hi = *gptr((const u32x4 *)(pd + 16));
            bv[j][0] = (int)lo.x; bv[j][1] = (int)lo.y; bv[j][2] = (int)lo.z; bv[j][3] = (int)lo.w;
            bv[j][4] = (int)hi.x; bv[j][5] = (int)hi.y; bv[j][6] = (int)hi.z; bv[j][7] = (int)hi.w;
            bsv[j] = *gptr((const int *)ps);
        }
        DSV4_ORDER();
        AScales<FMT_FP4_E8M0, CPW> sc;
        ld_ascales<FMT_FP4_E8M0, CPW>(sc, m.s, sc_cols, m.blk_r, row, r0, cb0, ncw, g, a.hidden - 1);
        DSV4_ORDER();
        AChunk<true> w[CPW];
        const uint8_t *wrow = (const uint8_t *)m.w + (size_t)row * row_bytes;
#pragma unroll
        for (int j = 0; j < CPW; j++) ld_a(w[j], wrow, cb0 + (j < ncw ? j : 0), g);
        DSV4_ORDER();
        v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < CPW; j++) acc = mfma_a<true>(w[j], bv[j], acc, (int)sc.v[j], bsv[j]);
        sum_cols8(acc);
#pragma unroll
        for (int e = 0; e < 4; e++) mine[e] = acc[e];
    } else if (threadIdx.x == 64 * wave && half == 0) {
        atomicOr(a.status, bad);
    }
    if (col == 0) {
#pragma unroll
        for (int e = 0; e < 4; e++) ylds[k][half][4 * g + e] = mine[e];
    }
    __syncthreads();
    if (wave != 0 || lane >= 16 || r0 + lane >= a.hidden) return;
    float o = 0.0f;
    for (int kk = 0; kk < a.topk; kk++) {
        const float y = ylds[kk][0][lane] + ylds[kk][1][lane];
        o = __fadd_rn(o, __fmul_rn(route_weight(a, kk), y));
    }
    if (a.shared) o = __fadd_rn(o, a.shared[r0 + lane]);
    a.out[r0 + lane] = o;
}

/* ------------------------------------------ FP4 chunk-pair kernels --- */

/* One MFMA covers 8 weight rows x 2 chunks: A rows 0-7 are the tile's rows at
 * chunk 2m, A rows 8-15 the same rows at chunk 2m + 1, so each load
 * instruction reads 128 contiguous bytes (one cache line) of 8 rows. B
 * columns 0-3 are the activation parts of chunk 2m, columns 4-7 those of
 * chunk 2m + 1, columns 8-15 zero. Of the 16 x 16 result, rows 0-7 x columns
 * 0-3 (even chunks) and rows 8-15 x columns 4-7 (odd chunks) are the wanted
 * partial dot products; the two cross blocks are discarded. After the
 * column sums, lane 16 q (q = 0, 1) holds rows 4 q + e of the even chunks and
 * lane 16 q + 4 (q = 2, 3) rows 4 (q - 2) + e of the odd chunks.
 * Lane geometry: A row r8 = lane & 7, chunk parity par = (lane >> 3) & 1,
 * 32-element block g = lane >> 4. */

template <int NP>
struct APairs {
    u32x4 q[NP];
    uint32_t s[(NP + 3) / 4];   /* E8M0 scale of pair m in byte m % 4 of s[m / 4] */
    u32x4 piece;                /* this lane's 16 scale bytes on the wide path */
    bool wide;
};

/* E8M0 scales of NP chunk pairs starting at chunk c0 of row `row` (FP4, scale
 * rows sc_cols bytes apart). A row's 2 NP chunks have 8 NP contiguous scale
 * bytes: with NP >= 2 and 16-byte aligned rows, NP / 2 lanes per row load
 * them as 16-byte pieces here and ld_pairs_scales_finish hands every lane its
 * bytes -- called after the weight loads are issued, so waiting for the
 * pieces never delays them. Otherwise each lane loads its bytes directly. */
template <int NP>
__device__ __forceinline__ void ld_pairs_scales(APairs<NP> &a, const uint8_t *S, int sc_cols, int blk_r,
                                                int row, int tile_row0, int row_max, int c0, int lane)
{
    const int par = (lane >> 3) & 1, g = lane >> 4;
    bool wide = NP >= 2 && (sc_cols & 15) == 0 && ((4 * c0) & 15) == 0 && ((uintptr_t)S & 15u) == 0;
    a.wide = __builtin_amdgcn_readfirstlane((int)wide) != 0;
    if constexpr (NP >= 2) {
        if (a.wide) {
            constexpr int NPC = NP / 2;                       /* 16-byte pieces per row */
            const int L = lane % (8 * NPC);
            const int rl = min(tile_row0 + L / NPC, row_max);
            a.piece = *gptr((const u32x4 *)(S + (size_t)(rl / blk_r) * sc_cols + 4 * c0 + 16 * (L % NPC)));
            return;
        }
    }
    uint32_t b[NP];
#pragma unroll
    for (int m = 0; m < NP; m++)
        b[m] = ld_u8(S, (size_t)(row / blk_r) * sc_cols + 4 * (c0 + 2 * m + par) + g);
#pragma unroll
    for (int i = 0; i < (NP + 3) / 4; i++) {
        uint32_t v = 0;
#pragma unroll
        for (int m = 4 * i; m < 4 * i + 4 && m < NP; m++) v |= b[m] << (8 * (m & 3));
        a.s[i] = v;
    }
}

template <int NP>
__device__ __forceinline__ void ld_pairs_scales_finish(APairs<NP> &a, int lane)
{
    if constexpr (NP >= 2) {
        if (a.wide) {
            constexpr int NPC = NP / 2;
            const int par = (lane >> 3) & 1, g = lane >> 4;
#pragma unroll
            for (int i = 0; i < (NP + 3) / 4; i++) a.s[i] = 0;
#pragma unroll
            for (int m = 0; m < NP; m++) {
                const int src = ((lane & 7) * NPC + m / 2) * 4;
                const uint32_t d0 = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)a.piece[2 * (m & 1)]);
                const uint32_t d1 = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)a.piece[2 * (m & 1) + 1]);
                a.s[m >> 2] |= (((par ? d1 : d0) >> (8 * g)) & 0xFFu) << (8 * (m & 3));
            }
        }
    }
}

template <int NP>
__device__ __forceinline__ void ld_pairs_w(APairs<NP> &a, const uint8_t *wrow, int c0, int lane)
{
    const int par = (lane >> 3) & 1, g = lane >> 4;
#pragma unroll
    for (int m = 0; m < NP; m++) a.q[m] = ld_stream16(wrow + 64 * (c0 + 2 * m + par) + 16 * g);
}

/* B operand of pair m from a split table laid out per chunk (TAB_CHUNK bytes
 * per chunk from `tab`, chunk index relative to the table's first chunk). */
struct BPair {
    const uint8_t *d, *s;   /* chunk 0 of this lane's column, or the zero operand */
    int step;               /* bytes per chunk pair (0 for zero columns) */
};

__device__ __forceinline__ BPair bpair_src(const uint8_t *tab, int c0, const uint8_t *zero, int lane)
{
    const int col = lane & 15, h = lane >> 4;
    BPair b;
    if (col < 8) {
        const uint8_t *cb = tab + (size_t)(c0 + (col >> 2)) * TAB_CHUNK;
        b.d = cb + (h * NPART + (col & 3)) * 32;
        b.s = cb + TAB_DATA + (h * NPART + (col & 3)) * 4;
        b.step = 2 * TAB_CHUNK;
    } else {
        b.d = zero;
        b.s = zero + 32;
        b.step = 0;
    }
    return b;
}

/* Column sums of a chunk-pair accumulator and its wanted quadrants, written
 * as 8 even-chunk and 8 odd-chunk row partials to dst[0..7], dst[8..15]. */
__device__ __forceinline__ void store_pair_partials(v4f acc, float *dst, int lane)
{
    sum_parts(acc);
    const int q = lane >> 4, col = lane & 15;
    if (col == 0 && q < 2) {
#pragma unroll
        for (int e = 0; e < 4; e++) dst[4 * q + e] = acc[e];
    }
    if (col == 4 && q >= 2) {
#pragma unroll
        for (int e = 0; e < 4; e++) dst[8 + 4 * (q - 2) + e] = acc[e];
    }
}

/* Gate/up + SwiGLU for FP4 experts with hidden = 512 NP, one item = (slot,
 * 32-row group). Eight waves: four 8-row tiles x two halves of K (NP chunk
 * pairs each). The workgroup splits x once into LDS (one unit of eight
 * elements per thread for hidden 4096) and every wave reads its half from
 * there. Writes mid and, when a.msplit is set, mid's split table. */

template <int NP>
__device__ __forceinline__ void gateup_px_item(const GateUpMxArgs &a, int item, uint8_t *lds,
                                               const OnePub *pub = nullptr)
{
    constexpr int NC = 4 * NP;                         /* chunks of hidden */
    constexpr int UPL = (NC * 16 + 511) / 512;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int tile = wave >> 1, hh = wave & 1;
    const int groups = a.inter / 32;
    const int slot = item / groups;
    const int j0 = (item - slot * groups) * 32;
    const int r0 = j0 + 8 * tile;
    const int row = r0 + (lane & 7);
    const int c0 = hh * 2 * NP;
    uint8_t *tab = lds;                                /* NC chunks + zero operand */
    float *red = (float *)(lds + NC * TAB_CHUNK + TAB_ZERO);   /* [4 tiles][2 halves][2 mats][16] */
    float *vl = red + 4 * 2 * 2 * 16;                  /* the group's 32 mid values */
    float *mid = a.mid + (size_t)slot * a.mid_ld;

    DSV4ExpertW e;
    unsigned bad = gateup_expert(a, slot, e);
    if (!bad && (!mx_desc_ok<FMT_FP4_E8M0>(e.w1, a.inter, a.hidden) ||
                 !mx_desc_ok<FMT_FP4_E8M0>(e.w3, a.inter, a.hidden)))
        bad = ST_BAD_DESCRIPTOR;
    if (bad) {
        if (threadIdx.x == 0) atomicOr(a.status, bad);
        if (threadIdx.x < 32) mid[j0 + threadIdx.x] = qnan_f();
        /* NaN block scales (E8M0 255) make the down projection of this slot NaN */
        if (a.msplit && threadIdx.x < 2 * NPART)
            st_dev32(a.msplit + (size_t)slot * a.msplit_ld + (size_t)(j0 >> 7) * MTAB_CHUNK +
                     mtab_scale_off((j0 & 127) + 16 * (threadIdx.x / NPART), threadIdx.x % NPART), 255u);
    } else {
        const int row_bytes = a.hidden / 2, sc_cols = a.hidden / 32;
        XUnits<UPL> xu;
        load_units<UPL, 512>(xu, a.x, 0, 1, 0, NC, (int)threadIdx.x);
        DSV4_ORDER();
        APairs<NP> w1, w3;
        ld_pairs_scales<NP>(w1, (const uint8_t *)e.w1.s, sc_cols, e.w1.blk_r, row, r0, a.inter - 1, c0, lane);
        ld_pairs_scales<NP>(w3, (const uint8_t *)e.w3.s, sc_cols, e.w3.blk_r, row, r0, a.inter - 1, c0, lane);
        DSV4_ORDER();
        ld_pairs_w<NP>(w1, (const uint8_t *)e.w1.w + (size_t)row * row_bytes, c0, lane);
        ld_pairs_w<NP>(w3, (const uint8_t *)e.w3.w + (size_t)row * row_bytes, c0, lane);
        DSV4_ORDER();
        store_units<UPL, 512>(tab, xu, 1, NC, (int)threadIdx.x);
        ld_pairs_scales_finish<NP>(w1, lane);
        ld_pairs_scales_finish<NP>(w3, lane);
        __builtin_amdgcn_s_waitcnt(0xC07F);            /* lgkmcnt(0): own LDS writes done */
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        const BPair bp = bpair_src(tab, c0, tab + NC * TAB_CHUNK, lane);
        v4f gacc = {0.0f, 0.0f, 0.0f, 0.0f}, uacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < NP; m++) {
            const u32x4 lo = *(const u32x4 *)(bp.d + m * bp.step);
            const u32x4 hi = *(const u32x4 *)(bp.d + m * bp.step + 16);
            const int sb = *(const int *)(bp.s + m * bp.step);
            v8i b;
            b[0] = (int)lo.x; b[1] = (int)lo.y; b[2] = (int)lo.z; b[3] = (int)lo.w;
            b[4] = (int)hi.x; b[5] = (int)hi.y; b[6] = (int)hi.z; b[7] = (int)hi.w;
            switch (m & 3) {       /* compile-time after unrolling: the scale byte select */
            case 0: gacc = mfma_f4_sel<0>(w1.q[m], b, gacc, w1.s[m >> 2], sb);
                    uacc = mfma_f4_sel<0>(w3.q[m], b, uacc, w3.s[m >> 2], sb); break;
            case 1: gacc = mfma_f4_sel<1>(w1.q[m], b, gacc, w1.s[m >> 2], sb);
                    uacc = mfma_f4_sel<1>(w3.q[m], b, uacc, w3.s[m >> 2], sb); break;
            case 2: gacc = mfma_f4_sel<2>(w1.q[m], b, gacc, w1.s[m >> 2], sb);
                    uacc = mfma_f4_sel<2>(w3.q[m], b, uacc, w3.s[m >> 2], sb); break;
            default: gacc = mfma_f4_sel<3>(w1.q[m], b, gacc, w1.s[m >> 2], sb);
                     uacc = mfma_f4_sel<3>(w3.q[m], b, uacc, w3.s[m >> 2], sb); break;
            }
        }
        store_pair_partials(gacc, red + ((tile * 2 + hh) * 2 + 0) * 16, lane);
        store_pair_partials(uacc, red + ((tile * 2 + hh) * 2 + 1) * 16, lane);
        __syncthreads();
        if (wave == 0) {
            if (lane < 32) {
                const int t = lane >> 3, rr = lane & 7;
                const float *p0 = red + ((t * 2 + 0) * 2) * 16, *p1 = red + ((t * 2 + 1) * 2) * 16;
                const float gs = ((p0[rr] + p0[8 + rr]) + p1[rr]) + p1[8 + rr];
                const float us = ((p0[16 + rr] + p0[24 + rr]) + p1[16 + rr]) + p1[24 + rr];
                const float v = dev_swiglu(gs, us, a.limit);
                mid[j0 + lane] = v;
                vl[lane] = v;
            }
            /* the two halves of block j0 / 32 of mid, each in a lane pair of
             * eight values, split with their own scales into the down
             * projection's table (chunk j0 / 128) */
            if (a.msplit && lane < 4) {
                float v8[8];
#pragma unroll
                for (int i = 0; i < 8; i++) v8[i] = vl[8 * lane + i];
                uint32_t code[NPART][2];
                int E[NPART];
                split8_half(v8, code, E);
                uint8_t *cb = a.msplit + (size_t)slot * a.msplit_ld + (size_t)(j0 >> 7) * MTAB_CHUNK;
                const int k0 = (j0 & 127) + 16 * (lane >> 1);
#pragma unroll
                for (int p = 0; p < NPART; p++) {
                    uint8_t *d = cb + mtab_code_off(k0, p) + 8 * (lane & 1);
                    st_dev32(d, code[p][0]);
                    st_dev32(d + 4, code[p][1]);
                }
                if ((lane & 1) == 0) {
#pragma unroll
                    for (int p = 0; p < NPART; p++) st_dev32(cb + mtab_scale_off(k0, p), (uint32_t)E[p]);
                }
            }
        }
    }
    if (pub && wave == 0) publish(*pub, lane);     /* this item's block of slot's table is out */
}

template <int NP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_gateup_px(GateUpMxArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    gateup_px_item<NP>(a, (int)blockIdx.x, lds);
}

/* One wave's share of an 8-row FP8 tile in chunk pairs: rows r0 .. r0 + 7 of
 * a matrix (row pitch row_bytes, scale grid sc_cols wide, blk_r rows high)
 * over chunk pairs starting at chunk c0. A rows 0-7 are the tile's rows at
 * chunk 2 i, rows 8-15 the same rows at chunk 2 i + 1, as in the FP4 pair
 * kernels; B is the workgroup's split of x. E8M0 scales go in the MFMA's
 * scale operand per lane (rows 8-15 take the odd chunk's), fp32 scales
 * multiply each pair's product (one MFMA from zero) row by row. */
template <int FMT, int NP>
struct Px8Tile {
    uint32_t sv[NP];                                   /* E8M0 byte or fp32 bits */
    u32x4 q[NP][2];                                    /* pair i: [0] even chunk, [1] odd chunk */
};

/* Issue the tile's scale loads, then its weight loads (they complete in issue
 * order, behind whatever the wave issued before). Each load instruction reads
 * one chunk of all 8 rows as whole 128-byte lines: lane r8 + 8 h + 16 g takes
 * bytes 16 (4 h + g) of row r8's chunk. (Loading the MFMA operand halves
 * directly, bytes 16 g and 64 + 16 g of each chunk, made every instruction
 * read 16 half lines: a stream of this tile shape took 4.40 us for the
 * 4096 x 4096 FP8 matrix against 3.86 us with whole lines.) px8_mma trades
 * halves between lanes i and i ^ 8 to form the operands. */
template <int FMT, int NP>
__device__ __forceinline__ void px8_load(Px8Tile<FMT, NP> &t, const uint8_t *W, const void *S, int row_bytes,
                                         int sc_cols, int blk_r, int r0, int c0, int lane)
{
    constexpr bool F32S = FMT == FMT_FP8_F32S;
    const int r8 = lane & 7, par = (lane >> 3) & 1, g = lane >> 4;
    const uint8_t *wrow = W + (size_t)(r0 + r8) * row_bytes;
    const size_t srow = (size_t)(r0 / blk_r) * sc_cols;
    /* this lane's chunk scale per pair: E8M0 for the A rows of the lane
     * (rows 8-15, par = 1: the odd chunk), fp32 for its accumulator rows
     * (lanes 32-63 hold rows 8-15) */
#pragma unroll
    for (int i = 0; i < NP; i++) {
        if constexpr (F32S) t.sv[i] = gptr((const uint32_t *)S)[srow + c0 + 2 * i + (lane >> 5)];
        else t.sv[i] = ld_u8(S, srow + c0 + 2 * i + par);
    }
    DSV4_ORDER();
    const int piece = 16 * (4 * par + g);
#pragma unroll
    for (int i = 0; i < NP; i++) {
        t.q[i][0] = ld_stream16(wrow + 128 * (c0 + 2 * i) + piece);
        t.q[i][1] = ld_stream16(wrow + 128 * (c0 + 2 * i + 1) + piece);
    }
}

/* The tile's pair accumulator against x's split table (tab: chunk-major,
 * zero operand after nc chunks). MFMA row r8 + 8 par of lane group g wants
 * bytes 16 g (operand half 0) and 64 + 16 g (half 1) of chunk par of row r8:
 * a lane of the even-chunk rows (par 0) loaded half 0 of the even chunk and
 * its partner lane ^ 8 half 1; for the odd chunk the partner holds half 0. */
template <int FMT, int NP>
__device__ __forceinline__ v4f px8_mma(const Px8Tile<FMT, NP> &t, const uint8_t *tab, int nc, int c0, int lane)
{
    constexpr bool F32S = FMT == FMT_FP8_F32S;
    const BPair bp = bpair_src(tab, c0, tab + (size_t)nc * TAB_CHUNK, lane);
    const bool odd = (lane >> 3) & 1;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NP; i++) {
        u32x4 h0, h1;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t se = (uint32_t)__builtin_amdgcn_mov_dpp((int)t.q[i][0][e], DPP_ROW_ROR8, 0xF, 0xF, false);
            const uint32_t so = (uint32_t)__builtin_amdgcn_mov_dpp((int)t.q[i][1][e], DPP_ROW_ROR8, 0xF, 0xF, false);
            h0[e] = odd ? so : t.q[i][0][e];
            h1[e] = odd ? t.q[i][1][e] : se;
        }
        const u32x4 lo = *(const u32x4 *)(bp.d + i * bp.step);
        const u32x4 hi = *(const u32x4 *)(bp.d + i * bp.step + 16);
        const int sb = *(const int *)(bp.s + i * bp.step);
        v8i b, av;
        b[0] = (int)lo.x; b[1] = (int)lo.y; b[2] = (int)lo.z; b[3] = (int)lo.w;
        b[4] = (int)hi.x; b[5] = (int)hi.y; b[6] = (int)hi.z; b[7] = (int)hi.w;
        av[0] = (int)h0.x; av[1] = (int)h0.y; av[2] = (int)h0.z; av[3] = (int)h0.w;
        av[4] = (int)h1.x; av[5] = (int)h1.y; av[6] = (int)h1.z; av[7] = (int)h1.w;
        if constexpr (F32S) {
            /* accumulator rows 0-7 (lanes 0-31) are the even chunk's, rows
             * 8-15 (lanes 32-63) the odd chunk's: each lane scales its rows */
            const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
            const v4f pr = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, zero, 0, 0, 0, E8M0_ONE, 0, sb);
            const float sw = __uint_as_float(t.sv[i]);
#pragma unroll
            for (int e2 = 0; e2 < 4; e2++) acc[e2] = fmaf(pr[e2], sw, acc[e2]);
        } else {
            acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, acc, 0, 0, 0, (int)t.sv[i], 0, sb);
        }
    }
    return acc;
}

/* Gate/up + SwiGLU of one FP8 expert (E8M0 or fp32 128 x 128 block scales)
 * in 8-row tiles, for the shared expert and single experts, whose mid needs
 * no split table: one workgroup per (slot, 8 rows), so a 2048-row expert
 * spreads over 256 workgroups (32-row groups gave 64, a quarter of the CUs,
 * and ran at 1.2 TB/s). Waves 0-3 take w1, waves 4-7 w3, each over a quarter
 * of K in NP chunk pairs (hidden = 1024 NP <= 4096). */
template <int FMT, int NP>
__global__ __launch_bounds__(512) void k_gateup_px8(GateUpMxArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NC = 8 * NP;                         /* chunks of hidden */
    constexpr int UPL = (NC * 16 + 511) / 512;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int mat = wave >> 2, kq = wave & 3;
    const int tiles = a.inter / 8;
    const int slot = blockIdx.x / tiles;
    const int r0 = (blockIdx.x - slot * tiles) * 8;
    const int c0 = kq * 2 * NP;                        /* the wave's first chunk */
    uint8_t *tab = lds;                                /* NC chunks + zero operand */
    float *red = (float *)(lds + NC * TAB_CHUNK + TAB_ZERO);   /* [2 mats][4 quarters][16] */
    float *mid = a.mid + (size_t)slot * a.mid_ld;

    DSV4ExpertW e;
    unsigned bad = gateup_expert(a, slot, e);
    if (!bad && (!mx_desc_ok<FMT>(e.w1, a.inter, a.hidden) || !mx_desc_ok<FMT>(e.w3, a.inter, a.hidden)))
        bad = ST_BAD_DESCRIPTOR;
    if (bad) {
        if (threadIdx.x == 0) atomicOr(a.status, bad);
        if (threadIdx.x < 8) mid[r0 + threadIdx.x] = qnan_f();
        return;
    }
    const DSV4QMat &m = mat ? e.w3 : e.w1;

    XUnits<UPL> xu;
    load_units<UPL, 512>(xu, a.x, 0, 1, 0, NC, (int)threadIdx.x);
    DSV4_ORDER();
    Px8Tile<FMT, NP> t;
    px8_load<FMT, NP>(t, (const uint8_t *)m.w, m.s, a.hidden, a.hidden / 128, m.blk_r, r0, c0, lane);
    DSV4_ORDER();
    store_units<UPL, 512>(tab, xu, 1, NC, (int)threadIdx.x);
    __builtin_amdgcn_s_waitcnt(0xC07F);                /* lgkmcnt(0): own LDS writes done */
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const v4f acc = px8_mma<FMT, NP>(t, tab, NC, c0, lane);
    store_pair_partials(acc, red + (mat * 4 + kq) * 16, lane);
    __syncthreads();
    if (threadIdx.x < 8) {
        const int rr = threadIdx.x;
        float gs = 0.0f, us = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            gs += red[(0 * 4 + k) * 16 + rr] + red[(0 * 4 + k) * 16 + 8 + rr];
            us += red[(1 * 4 + k) * 16 + rr] + red[(1 * 4 + k) * 16 + 8 + rr];
        }
        mid[r0 + rr] = dev_swiglu(gs, us, a.limit);
    }
}

/* One-token FP8 matvec in the same 8-row chunk-pair tiles: one workgroup per
 * TILES 8-row tiles, KQ waves per tile each over NP chunk pairs (cols =
 * 256 KQ NP), every workgroup splitting x once into LDS. blk: the
 * workgroup's tile group within the matrix. */
template <int FMT, int NP, int KQ, int TILES>
__device__ __forceinline__ void gemv_px8_body(const GemvMxArgs &a, int blk)
{
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NC = 2 * KQ * NP;
    constexpr int NTHR = 64 * KQ * TILES;
    constexpr int UPL = (NC * 16 + NTHR - 1) / NTHR;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int h = wave / KQ, kq = wave % KQ;
    const int r0 = blk * 8 * TILES + 8 * h;
    const int c0 = kq * 2 * NP;
    uint8_t *tab = lds;
    float *red = (float *)(lds + NC * TAB_CHUNK + TAB_ZERO);   /* [TILES][KQ][16] */

    XUnits<UPL> xu;
    load_units<UPL, NTHR>(xu, a.x, 0, 1, 0, NC, (int)threadIdx.x);
    DSV4_ORDER();
    Px8Tile<FMT, NP> t;
    px8_load<FMT, NP>(t, a.W, a.S, a.row_bytes, a.sc_cols, a.blk_r, r0, c0, lane);
    DSV4_ORDER();
    store_units<UPL, NTHR>(tab, xu, 1, NC, (int)threadIdx.x);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const v4f acc = px8_mma<FMT, NP>(t, tab, NC, c0, lane);
    store_pair_partials(acc, red + (h * KQ + kq) * 16, lane);
    __syncthreads();
    if (threadIdx.x < 8 * TILES) {
        const int hh = threadIdx.x >> 3, rr = threadIdx.x & 7;
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < KQ; k++) s += red[(hh * KQ + k) * 16 + rr] + red[(hh * KQ + k) * 16 + 8 + rr];
        a.y[blk * 8 * TILES + threadIdx.x] = s;
    }
}

template <int FMT, int NP, int KQ, int TILES>
__global__ __launch_bounds__(64 * KQ * TILES) void k_gemv_px8(GemvMxArgs a)
{
    gemv_px8_body<FMT, NP, KQ, TILES>(a, (int)blockIdx.x);
}

/* Several one-token matvecs of one geometry class in one launch (the jobs of
 * a multi-job projection): job j owns workgroups first[j] .. first[j + 1] - 1. */
struct Px8Jobs {
    GemvMxArgs job[PX8_MAX_JOBS];
    int first[PX8_MAX_JOBS + 1];
    int nj;
};

template <int FMT, int NP, int KQ, int TILES>
__global__ __launch_bounds__(64 * KQ * TILES) void k_gemv_px8_multi(Px8Jobs m)
{
    int j = 0;
    while (j + 1 < m.nj && (int)blockIdx.x >= m.first[j + 1]) j++;
    gemv_px8_body<FMT, NP, KQ, TILES>(m.job[j], (int)blockIdx.x - m.first[j]);
}

/* Routed FP4 down projections (inter = 256 NP) with the k-order combine. One
 * workgroup per 16 output rows, two waves (8-row tiles) per routed expert k,
 * each over all of inter, reading slot k's split table. */
template <int NP>
__global__ __launch_bounds__(1024) void k_down_px(DownMxArgs a)
{
    __shared__ float ylds[8][2][16];
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int k = wave >> 1, t = wave & 1;
    const int r0 = blockIdx.x * 16 + 8 * t;
    const int row = min(r0 + (lane & 7), a.hidden - 1);
    const int row_bytes = a.inter / 2, sc_cols = a.inter / 32;

    unsigned bad = 0;
    DSV4QMat m;
    bad = down_expert(a, k, m);
    if (!bad && !mx_desc_ok<FMT_FP4_E8M0>(m, a.hidden, a.inter)) bad = ST_BAD_DESCRIPTOR;
    float part[16];
#pragma unroll
    for (int i = 0; i < 16; i++) part[i] = qnan_f();
    if (!bad) {
        const BMid bp = bmid_src(a.msplit + (size_t)k * a.msplit_ld, 0, (const uint8_t *)g_zero_operand, lane);
        v8i bv[NP];
        int bs[NP];
#pragma unroll
        for (int mm = 0; mm < NP; mm++) {
            const u32x4 lo = *gptr((const u32x4 *)(bp.d + (size_t)mm * bp.dstep));
            const u32x4 hi = *gptr((const u32x4 *)(bp.d + (size_t)mm * bp.dstep + 16));
            bv[mm][0] = (int)lo.x; bv[mm][1] = (int)lo.y; bv[mm][2] = (int)lo.z; bv[mm][3] = (int)lo.w;
            bv[mm][4] = (int)hi.x; bv[mm][5] = (int)hi.y; bv[mm][6] = (int)hi.z; bv[mm][7] = (int)hi.w;
            bs[mm] = *gptr((const int *)(bp.s + (size_t)mm * bp.sstep));
        }
        DSV4_ORDER();
        APairs<NP> w;
        ld_pairs_scales<NP>(w, (const uint8_t *)m.s, sc_cols, m.blk_r, row, r0, a.hidden - 1, 0, lane);
        DSV4_ORDER();
        ld_pairs_w<NP>(w, (const uint8_t *)m.w + (size_t)row * row_bytes, 0, lane);
        DSV4_ORDER();
        ld_pairs_scales_finish<NP>(w, lane);
        v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int mm = 0; mm < NP; mm++) {
            switch (mm & 3) {
            case 0: acc = mfma_f4_sel<0>(w.q[mm], bv[mm], acc, w.s[mm >> 2], bs[mm]); break;
            case 1: acc = mfma_f4_sel<1>(w.q[mm], bv[mm], acc, w.s[mm >> 2], bs[mm]); break;
            case 2: acc = mfma_f4_sel<2>(w.q[mm], bv[mm], acc, w.s[mm >> 2], bs[mm]); break;
            default: acc = mfma_f4_sel<3>(w.q[mm], bv[mm], acc, w.s[mm >> 2], bs[mm]); break;
            }
        }
        store_mid_partials(acc, &ylds[k][t][0], lane);
    } else {
        if (lane == 0 && t == 0) atomicOr(a.status, bad);
        if (lane < 16) ylds[k][t][lane] = qnan_f();
    }
    __syncthreads();
    if (wave != 0 || lane >= 16 || blockIdx.x * 16 + lane >= a.hidden) return;
    const int tt = lane >> 3, rr = lane & 7;
    float o = 0.0f;
    for (int kk = 0; kk < a.topk; kk++) {
        const float y = ylds[kk][tt][rr] + ylds[kk][tt][8 + rr];
        o = __fadd_rn(o, __fmul_rn(route_weight(a, kk), y));
    }
    if (a.shared) o = __fadd_rn(o, a.shared[blockIdx.x * 16 + lane]);
    a.out[blockIdx.x * 16 + lane] = o;
}

/* ------------------------------------------- one-launch decode MoE --- */

typedef __attribute__((address_space(3))) void lds_void_t;

/* LDS of a down workgroup of the one-launch form: the partial sums
 * [slot][tile][16], the ready word, then per routed slot its split table in
 * whole 1 KiB DMA rounds and a zero operand. */
constexpr int ONE_YL_BYTES = MX_ROUTED_MAX * 2 * 16 * 4;
constexpr int ONE_HEAD_BYTES = ONE_YL_BYTES + 64;
__host__ __device__ constexpr int one_tab_rounds(int inter) { return (inter / 128 * MTAB_CHUNK + 1023) / 1024; }
__host__ __device__ constexpr int one_slot_lds(int inter) { return one_tab_rounds(inter) * 1024 + TAB_ZERO; }

/* s_waitcnt lgkmcnt(0) + s_barrier: a workgroup barrier that leaves the
 * weight loads in flight (__syncthreads() would drain them). */
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* Down workgroup of the one-launch form: output rows 16 grp .. 16 grp + 15,
 * wave k = routed slot k over both 8-row tiles and all of inter (inter =
 * 256 NP). The down weights load first; wave 0 then waits for every slot's
 * mid; each wave copies its slot's split table into LDS with device-scope
 * loads and runs the MFMA sequence, partial sums and k-order combine of
 * k_down_px. */
template <int NP>
__device__ __forceinline__ void down_one_group(const MoeOneArgs &A, int grp, uint8_t *lds)
{
    const DownMxArgs &a = A.dn;
    constexpr int ROUNDS = one_tab_rounds(256 * NP), SLOT = one_slot_lds(256 * NP);
    float(*yl)[2][16] = (float(*)[2][16])lds;
    int *ready_ok = (int *)(lds + ONE_YL_BYTES);
    const int lane = threadIdx.x & 63;
    const int k = wave_in_group();
    const int r0 = grp * 16;
    const bool live = k < a.topk;
    uint8_t *tab = lds + ONE_HEAD_BYTES + k * SLOT;
    unsigned bad = 0;
    APairs<NP> w0, w1;
    if (live) {
        const int row_bytes = a.inter / 2, sc_cols = a.inter / 32;
        DSV4QMat m;
        bad = down_expert(a, k, m);
        if (!bad && !mx_desc_ok<FMT_FP4_E8M0>(m, a.hidden, a.inter)) bad = ST_BAD_DESCRIPTOR;
        if (!bad) {
            const int row0 = min(r0 + (lane & 7), a.hidden - 1), row1 = min(r0 + 8 + (lane & 7), a.hidden - 1);
            ld_pairs_scales<NP>(w0, (const uint8_t *)m.s, sc_cols, m.blk_r, row0, r0, a.hidden - 1, 0, lane);
            ld_pairs_scales<NP>(w1, (const uint8_t *)m.s, sc_cols, m.blk_r, row1, r0 + 8, a.hidden - 1, 0, lane);
            DSV4_ORDER();
            ld_pairs_w<NP>(w0, (const uint8_t *)m.w + (size_t)row0 * row_bytes, 0, lane);
            ld_pairs_w<NP>(w1, (const uint8_t *)m.w + (size_t)row1 * row_bytes, 0, lane);
            DSV4_ORDER();
            ld_pairs_scales_finish<NP>(w0, lane);
            ld_pairs_scales_finish<NP>(w1, lane);
            if (lane < TAB_ZERO / 4)                   /* zero operand, unit scale */
                ((uint32_t *)(tab + ROUNDS * 1024))[lane] = lane == 8 ? E8M0_ONE : 0u;
        }
    }
    /* One wave waits for every slot's mid (each feeds every output row) and
     * releases the workgroup; the weight loads stay in flight. With fewer
     * than eight slots the poll falls to wave 7, which has no slot: it has
     * issued no weight loads, so its poll returns as soon as the flag is set
     * (a wave's loads return in issue order), and its add to the leave
     * counter runs while the slot waves multiply. */
    const int pw = a.topk < 8 ? 7 : 0;
    if (k == pw) {
        const bool ok = wait_done(A.pub, A.spin_max);
        if (lane == 0) *ready_ok = ok ? 1 : 0;
    }
    lds_barrier();
    if (pw != 0 && k == pw && lane == 0) leave(A.pub);   /* its poll was its last access */
    if (live) {
        if (!bad && !*ready_ok) bad = ST_SYNC_TIMEOUT;
        if (!bad) {
            /* slot k's table, 16 bytes a lane per round (past its end: zeros) */
            const __amdgpu_buffer_rsrc_t rt = dev_rsrc(a.msplit + (size_t)k * a.msplit_ld, (uint32_t)a.msplit_ld);
#pragma unroll
            for (int r = 0; r < ROUNDS; r++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_void_t *)(tab + 1024 * r), 16,
                                                         1024 * r + 16 * lane, 0, 0, CPOL_SC1);
            __builtin_amdgcn_s_waitcnt(0x0F70);        /* vmcnt(0): the copy (and the weights) landed */
            asm volatile("" ::: "memory");
            const BMid bp = bmid_src(tab, 0, tab + ROUNDS * 1024, lane);
            v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int mm = 0; mm < NP; mm++) {
                const u32x4 lo = *(const u32x4 *)(bp.d + mm * bp.dstep);
                const u32x4 hi = *(const u32x4 *)(bp.d + mm * bp.dstep + 16);
                const int sb = *(const int *)(bp.s + mm * bp.sstep);
                v8i b;
                b[0] = (int)lo.x; b[1] = (int)lo.y; b[2] = (int)lo.z; b[3] = (int)lo.w;
                b[4] = (int)hi.x; b[5] = (int)hi.y; b[6] = (int)hi.z; b[7] = (int)hi.w;
                switch (mm & 3) {
                case 0: acc0 = mfma_f4_sel<0>(w0.q[mm], b, acc0, w0.s[mm >> 2], sb);
                        acc1 = mfma_f4_sel<0>(w1.q[mm], b, acc1, w1.s[mm >> 2], sb); break;
                case 1: acc0 = mfma_f4_sel<1>(w0.q[mm], b, acc0, w0.s[mm >> 2], sb);
                        acc1 = mfma_f4_sel<1>(w1.q[mm], b, acc1, w1.s[mm >> 2], sb); break;
                case 2: acc0 = mfma_f4_sel<2>(w0.q[mm], b, acc0, w0.s[mm >> 2], sb);
                        acc1 = mfma_f4_sel<2>(w1.q[mm], b, acc1, w1.s[mm >> 2], sb); break;
                default: acc0 = mfma_f4_sel<3>(w0.q[mm], b, acc0, w0.s[mm >> 2], sb);
                         acc1 = mfma_f4_sel<3>(w1.q[mm], b, acc1, w1.s[mm >> 2], sb); break;
                }
            }
            store_mid_partials(acc0, &yl[k][0][0], lane);
            store_mid_partials(acc1, &yl[k][1][0], lane);
        } else {
            if (lane == 0) atomicOr(a.status, bad);
            if (lane < 32) yl[k][lane >> 4][lane & 15] = qnan_f();
        }
    }
    __syncthreads();
    if (pw == 0 && threadIdx.x == 0) leave(A.pub); /* wave 0's poll has returned */
    if (threadIdx.x >= 16 || r0 + (int)threadIdx.x >= a.hidden) return;
    const int t = threadIdx.x >> 3, rr = threadIdx.x & 7;
    float o = 0.0f;
    for (int kk = 0; kk < a.topk; kk++) {
        const float y = yl[kk][t][rr] + yl[kk][t][8 + rr];
        o = __fadd_rn(o, __fmul_rn(route_weight(a, kk), y));
    }
    if (a.shared) o = __fadd_rn(o, a.shared[r0 + threadIdx.x]);
    a.out[r0 + threadIdx.x] = o;
}

/* Routed FP4 decode MoE in one launch (hidden = 512 NPG, inter = 256 NPD):
 * workgroup b < gu_blocks runs gate/up item b and publishes it; the hidden /
 * 16 down workgroups follow. A workgroup only ever waits on workgroups of
 * lower id, which the hardware dispatches no later than itself and which
 * never wait, so the launch cannot deadlock whatever part of it is resident;
 * every wait is bounded besides. */
template <int NPG, int NPD>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_moe_one(MoeOneArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];
    if ((int)blockIdx.x < a.gu_blocks)
        gateup_px_item<NPG>(a.gu, (int)blockIdx.x, lds, &a.pub);
    else
        down_one_group<NPD>(a, (int)blockIdx.x - a.gu_blocks, lds);
}

/* ------------------------------------- balanced one-launch decode MoE --- */

/* One workgroup per CU, every workgroup resident at once, each doing an equal
 * share of both phases:
 *   - waves 0-11 compute BAL_HB half blocks of gate/up (16 mid rows of one
 *     routed slot each, grid-size apart, so consecutive 32 KB pieces of a
 *     matrix stream to consecutive workgroups): wave u the 8-row tile
 *     (u / 2) % 2 of half block u / 4 for matrix u % 2 (w1, w3), over both
 *     halves of K, in the MFMA sequence of gateup_px_item (the same bits);
 *   - then waves 0-11 load down unit u (routed slot u / 2, 8-row tile u % 2 of
 *     the workgroup's 16 down rows) into registers: the down bytes queue
 *     behind every CU's gate/up bytes;
 *   - waves 12-15 split the workgroup's half blocks of mid (split8_half: the
 *     bytes and scales gateup_px_item writes) into mid_copies replicas of the
 *     slots' mid tables in HBM, then one add per workgroup on grouped
 *     counters; the add that completes the count raises the done flag;
 *   - one wave polls the flag, waves 12-15 copy every slot's table from
 *     replica blockIdx % mid_copies into LDS, waves 0-11 run the MFMA
 *     sequence of down_one_group for their unit, and the first 16 lanes
 *     combine in k order.
 * The workgroups wait on each other, so the host launches this form only when
 * the whole grid fits on the device at once (one workgroup per CU); the wait
 * is bounded (spin_max polls) as in k_moe_one. */
constexpr int BAL_WAVES = 16;
constexpr int BAL_GU_WAVES = 12;
constexpr int BAL_HB = BAL_GU_WAVES / 4;          /* half blocks (16 mid rows) per workgroup */
constexpr int BAL_POLL_WAVE = BAL_GU_WAVES + 1;
constexpr int BAL_HB_DW = 4 * NPART + NPART;      /* table dwords of one half block */

struct BalLds {
    int tab, red, stage, yl, flag, total;
};

/* x's split table, later every slot's mid tables (tab); the gate/up partials
 * (red); the writer waves' staging of the table dwords (stage); the down
 * partials (yl); the ready word (flag). */
__host__ __device__ constexpr BalLds bal_lds(int hidden, int inter, int topk)
{
    BalLds l{};
    const int xt = (hidden / 128) * TAB_CHUNK + TAB_ZERO;
    const int mt = (topk * (inter / 128) * MTAB_CHUNK + 1023) / 1024 * 1024 + TAB_ZERO;   /* whole copy rounds */
    l.tab = 0;
    l.red = xt > mt ? xt : mt;
    l.stage = l.red + 2 * BAL_HB * 2 * 2 * 16 * 4;
    l.yl = l.stage + (BAL_WAVES - BAL_GU_WAVES) * 64 * 4;
    l.flag = l.yl + MX_ROUTED_MAX * 2 * 16 * 4;
    l.total = l.flag + 16;
    return l;
}

template <int NPH, int NPD>
__global__ __launch_bounds__(1024) void k_moe_bal(MoeOneArgs A)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const GateUpMxArgs &a = A.gu;
    const DownMxArgs &d = A.dn;
    constexpr int NC = 4 * NPH;                      /* chunks of hidden */
    constexpr int NCD = 2 * NPD;                     /* chunks of inter  */
    constexpr int GU_THR = BAL_GU_WAVES * 64;
    constexpr int XUPL = (NC * 16 + GU_THR - 1) / GU_THR;
    const int lane = threadIdx.x & 63;
    const int wave = wave_in_group();
    const int topk = d.topk;
    const BalLds L = bal_lds(512 * NPH, 256 * NPD, topk);
    uint8_t *tab = lds + L.tab;
    float *red = (float *)(lds + L.red);             /* [tile 2 j + th][K half][mat][16] */
    float(*yl)[2][16] = (float(*)[2][16])(lds + L.yl);
    int *ready_ok = (int *)(lds + L.flag);
    const int tiles_per_slot = a.inter / 8;
    const int n_hb = topk * tiles_per_slot / 2;
    const int G = (int)gridDim.x;
    const int r0d = (int)blockIdx.x * 16;            /* first down row */
    const int tab_bytes = topk * NCD * MTAB_CHUNK;

    /* ---- gate/up: x, then the tile's scales and weights ---- */
    const int j = wave >> 2, th = (wave >> 1) & 1, mat = wave & 1;
    const int hb = j * G + (int)blockIdx.x;
    const bool live = wave < BAL_GU_WAVES && hb < n_hb;
    unsigned gbad = 0;
    APairs<NPH> gw[2];
    if (wave < BAL_GU_WAVES) {
        /* A wave without a valid tile still issues its loads, from inside x
         * (4 hidden bytes: eight FP4 rows of hidden / 2 bytes, and their
         * scale bytes with every row in scale row 0), so that no branch
         * merges before the x split and its wait counts only the x loads. */
        const int ti = 2 * hb + th;
        const int gslot = live ? ti / tiles_per_slot : 0;
        const int gr0 = live ? (ti - gslot * tiles_per_slot) * 8 : 0;
        const int row_bytes = a.hidden / 2, sc_cols = a.hidden / 32;
        const uint8_t *wb = (const uint8_t *)a.x, *sb = (const uint8_t *)a.x;
        int blk_r = 8, row = lane & 7, trow0 = 0, row_max = 7;
        if (live) {
            DSV4ExpertW e;
            gbad = gateup_expert(a, gslot, e);
            if (!gbad && (!mx_desc_ok<FMT_FP4_E8M0>(e.w1, a.inter, a.hidden) ||
                          !mx_desc_ok<FMT_FP4_E8M0>(e.w3, a.inter, a.hidden)))
                gbad = ST_BAD_DESCRIPTOR;
            if (!gbad) {
                const DSV4QMat &m = mat ? e.w3 : e.w1;
                wb = (const uint8_t *)m.w;
                sb = (const uint8_t *)m.s;
                blk_r = m.blk_r;
                row = gr0 + (lane & 7);
                trow0 = gr0;
                row_max = a.inter - 1;
            }
        }
        XUnits<XUPL> xu;
        load_units<XUPL, GU_THR>(xu, a.x, 0, 1, 0, NC, (int)threadIdx.x);
        DSV4_ORDER();
#pragma unroll
        for (int h = 0; h < 2; h++)
            ld_pairs_scales<NPH>(gw[h], sb, sc_cols, blk_r, row, trow0, row_max, h * 2 * NPH, lane);
        DSV4_ORDER();
#pragma unroll
        for (int h = 0; h < 2; h++) ld_pairs_w<NPH>(gw[h], wb + (size_t)row * row_bytes, h * 2 * NPH, lane);
        DSV4_ORDER();
        store_units<XUPL, GU_THR>(tab, xu, 1, NC, (int)threadIdx.x);
        ld_pairs_scales_finish<NPH>(gw[0], lane);
        ld_pairs_scales_finish<NPH>(gw[1], lane);
    }
    lds_barrier();                                   /* B1: x's table */

    /* ---- gate/up MFMAs: K half h over chunk pairs [h NPH, (h + 1) NPH) ---- */
    if (live) {
        float *rt = red + (size_t)(2 * j + th) * 2 * 2 * 16;
        if (!gbad) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const BPair bp = bpair_src(tab, h * 2 * NPH, tab + NC * TAB_CHUNK, lane);
                v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int m = 0; m < NPH; m++) {
                    const u32x4 lo = *(const u32x4 *)(bp.d + m * bp.step);
                    const u32x4 hi = *(const u32x4 *)(bp.d + m * bp.step + 16);
                    const int sbv = *(const int *)(bp.s + m * bp.step);
                    v8i b;
                    b[0] = (int)lo.x; b[1] = (int)lo.y; b[2] = (int)lo.z; b[3] = (int)lo.w;
                    b[4] = (int)hi.x; b[5] = (int)hi.y; b[6] = (int)hi.z; b[7] = (int)hi.w;
                    switch (m & 3) {
                    case 0: acc = mfma_f4_sel<0>(gw[h].q[m], b, acc, gw[h].s[m >> 2], sbv); break;
                    case 1: acc = mfma_f4_sel<1>(gw[h].q[m], b, acc, gw[h].s[m >> 2], sbv); break;
                    case 2: acc = mfma_f4_sel<2>(gw[h].q[m], b, acc, gw[h].s[m >> 2], sbv); break;
                    default: acc = mfma_f4_sel<3>(gw[h].q[m], b, acc, gw[h].s[m >> 2], sbv); break;
                    }
                }
                store_pair_partials(acc, rt + (h * 2 + mat) * 16, lane);
            }
        } else {
            if (lane == 0 && mat == 0) atomicOr(a.status, gbad);
            if (lane < 16) {
                rt[(0 * 2 + mat) * 16 + lane] = qnan_f();
                rt[(1 * 2 + mat) * 16 + lane] = qnan_f();
            }
        }
    }
    lds_barrier();                                   /* B2: the tiles' partials */

    /* ---- waves 0-11: the down unit's weights; waves 12-15: the mid tables ---- */
    const int uk = wave >> 1, ut = wave & 1;         /* down unit: slot, 8-row tile */
    const bool dlive = wave < BAL_GU_WAVES && uk < topk;
    unsigned dbad = 0;
    APairs<NPD> dw;
    if (dlive) {
        DSV4QMat m;
        dbad = down_expert(d, uk, m);
        if (!dbad && !mx_desc_ok<FMT_FP4_E8M0>(m, d.hidden, d.inter)) dbad = ST_BAD_DESCRIPTOR;
        if (!dbad) {
            const int rt = r0d + 8 * ut;
            const int row = min(rt + (lane & 7), d.hidden - 1);
            ld_pairs_scales<NPD>(dw, (const uint8_t *)m.s, d.inter / 32, m.blk_r, row, rt, d.hidden - 1, 0, lane);
            DSV4_ORDER();
            ld_pairs_w<NPD>(dw, (const uint8_t *)m.w + (size_t)row * (d.inter / 2), 0, lane);
            DSV4_ORDER();
        }
    }
    if (wave >= BAL_GU_WAVES) {
        /* Lanes 2 i and 2 i + 1 (i < BAL_HB) form half block i's 16 mid
         * values, eight each, and split them; its BAL_HB_DW table dwords go
         * through the wave's staging so that lane 20 i + dw stores dword dw
         * (codes of part dw / 4, bytes 4 (dw % 4) .., then the part scales),
         * one store instruction per replica. */
        uint32_t *stg = (uint32_t *)(lds + L.stage) + (wave - BAL_GU_WAVES) * 64;
        const int i = lane >> 1, hl = lane & 1;
        if (lane < 2 * BAL_HB) {
            float v[8];
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const int rr = 8 * hl + r;           /* row of the half block */
                const float *p0 = red + (size_t)(2 * i + (rr >> 3)) * 2 * 2 * 16;
                const int q = rr & 7;
                const float gs = ((p0[q] + p0[8 + q]) + p0[32 + q]) + p0[40 + q];
                const float us = ((p0[16 + q] + p0[24 + q]) + p0[48 + q]) + p0[56 + q];
                v[r] = dev_swiglu(gs, us, a.limit);
            }
            uint32_t code[NPART][2];
            int E[NPART];
            split8_half(v, code, E);
#pragma unroll
            for (int pp = 0; pp < NPART; pp++) {
                stg[BAL_HB_DW * i + 4 * pp + 2 * hl] = code[pp][0];
                stg[BAL_HB_DW * i + 4 * pp + 2 * hl + 1] = code[pp][1];
                if (!hl) stg[BAL_HB_DW * i + 4 * NPART + pp] = (uint32_t)E[pp];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);          /* lgkmcnt(0): the wave's staging is written */
        asm volatile("" ::: "memory");
        const int hi = lane / BAL_HB_DW, dwi = lane - hi * BAL_HB_DW;
        const int hbl = hi * G + (int)blockIdx.x;
        if (hi < BAL_HB && hbl < n_hb) {
            const int k = (hbl % (a.inter / 16)) * 16;                 /* row of the slot's mid */
            const int s2 = hbl / (a.inter / 16);
            const int k0 = k & 127;
            const int off = (s2 * NCD + (k >> 7)) * MTAB_CHUNK +
                            (dwi < 4 * NPART ? mtab_code_off(k0, dwi >> 2) + 4 * (dwi & 3)
                                             : mtab_scale_off(k0, dwi - 4 * NPART));
            const uint32_t val = stg[lane];
            for (int c = wave - BAL_GU_WAVES; c < A.mid_copies; c += BAL_WAVES - BAL_GU_WAVES)
                st_dev32(A.midc + (size_t)c * A.copy_ld + off, val);
        }
        /* the replicas acknowledged before the barrier below */
        __builtin_amdgcn_s_waitcnt(0x0F70);
        asm volatile("" ::: "memory");
    }
    lds_barrier();                                   /* B2b: the workgroup's tables are out */
    if (wave == BAL_GU_WAVES && lane == 0) {
        /* the add that completes the count raises the flag */
        const OnePub &p = A.pub;
        const unsigned grp = blockIdx.x % ONE_LEAVE_GROUPS;
        const unsigned in_grp = (p.items - grp + ONE_LEAVE_GROUPS - 1) / ONE_LEAVE_GROUPS;
        const unsigned groups = p.items < ONE_LEAVE_GROUPS ? p.items : ONE_LEAVE_GROUPS;
        unsigned *top = p.count + ONE_LEAVE_GROUPS * ONE_PUB_LINE_WORDS;
        if (__hip_atomic_fetch_add(p.count + grp * ONE_PUB_LINE_WORDS, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == in_grp - 1 &&
            __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == groups - 1)
            __hip_atomic_store(p.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (wave == BAL_POLL_WAVE) {
        const bool ok = wait_done(A.pub, A.spin_max);
        if (lane == 0) *ready_ok = ok ? 1 : 0;
    }
    lds_barrier();                                   /* B3: every slot's table is out (or the wait gave up) */
    const bool ready = *ready_ok != 0;

    /* ---- every slot's table into LDS (over x's), 1 KiB per instruction ---- */
    if (wave >= BAL_GU_WAVES) {
        if (ready) {
            const __amdgpu_buffer_rsrc_t rt =
                dev_rsrc(A.midc + (size_t)(blockIdx.x % A.mid_copies) * A.copy_ld, (uint32_t)tab_bytes);
            for (int r = wave - BAL_GU_WAVES; r * 1024 < tab_bytes; r += BAL_WAVES - BAL_GU_WAVES)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_void_t *)(tab + 1024 * r), 16,
                                                         1024 * r + 16 * lane, 0, 0, CPOL_SC1);
        }
        if (wave == BAL_GU_WAVES && lane < TAB_ZERO / 4)   /* zero operand, unit scale (past the copies) */
            ((uint32_t *)(tab + (tab_bytes + 1023) / 1024 * 1024))[lane] = lane == 8 ? E8M0_ONE : 0u;
        __builtin_amdgcn_s_waitcnt(0x0F70);          /* the copies landed */
        asm volatile("" ::: "memory");
    }
    lds_barrier();                                   /* B4: the tables */

    /* ---- down MFMAs: wave u = unit (slot u / 2, tile u % 2) ---- */
    if (dlive) {
        unsigned bad = dbad;
        if (!bad && !ready) bad = ST_SYNC_TIMEOUT;
        if (!bad) {
            ld_pairs_scales_finish<NPD>(dw, lane);
            const BMid bp = bmid_src(tab + (size_t)uk * NCD * MTAB_CHUNK, 0,
                                     tab + (tab_bytes + 1023) / 1024 * 1024, lane);
            v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int mm = 0; mm < NPD; mm++) {
                const u32x4 lo = *(const u32x4 *)(bp.d + mm * bp.dstep);
                const u32x4 hi = *(const u32x4 *)(bp.d + mm * bp.dstep + 16);
                const int sbv = *(const int *)(bp.s + mm * bp.sstep);
                v8i bv;
                bv[0] = (int)lo.x; bv[1] = (int)lo.y; bv[2] = (int)lo.z; bv[3] = (int)lo.w;
                bv[4] = (int)hi.x; bv[5] = (int)hi.y; bv[6] = (int)hi.z; bv[7] = (int)hi.w;
                switch (mm & 3) {
                case 0: acc = mfma_f4_sel<0>(dw.q[mm], bv, acc, dw.s[mm >> 2], sbv); break;
                case 1: acc = mfma_f4_sel<1>(dw.q[mm], bv, acc, dw.s[mm >> 2], sbv); break;
                case 2: acc = mfma_f4_sel<2>(dw.q[mm], bv, acc, dw.s[mm >> 2], sbv); break;
                default: acc = mfma_f4_sel<3>(dw.q[mm], bv, acc, dw.s[mm >> 2], sbv); break;
                }
            }
            store_mid_partials(acc, &yl[uk][ut][0], lane);
        } else {
            if (lane == 0 && (ut == 0 || bad == ST_SYNC_TIMEOUT)) atomicOr(a.status, bad);
            if (lane < 16) yl[uk][ut][lane] = qnan_f();
        }
    }
    __syncthreads();                                 /* B5: every slot's partial rows */
    if (threadIdx.x == 0) leave(A.pub);              /* the add and the poll were this workgroup's last */
    if (threadIdx.x >= 16 || r0d + (int)threadIdx.x >= d.hidden) return;
    const int t = threadIdx.x >> 3, rr = threadIdx.x & 7;
    float o = 0.0f;
    for (int kk = 0; kk < topk; kk++) {
        const float y = yl[kk][t][rr] + yl[kk][t][8 + rr];
        o = __fadd_rn(o, __fmul_rn(route_weight(d, kk), y));
    }
    if (d.shared) o = __fadd_rn(o, d.shared[r0d + threadIdx.x]);
    d.out[r0d + threadIdx.x] = o;
}

/* ------------------------------------------------------------ launches --- */

constexpr int cpw_for(int nch) { return nch <= 1 ? 1 : nch <= 2 ? 2 : nch <= 4 ? 4 : nch <= 8 ? 8 : 16; }

/* Tokens per token group: at most four (sixteen B columns), and at most
 * 16 / CPW so the four split tables of a workgroup stay near 37 KiB. */
template <int FMT, int CPW, int NT>
hipError_t gemv_mx_nt(GemvMxArgs a, hipStream_t st)
{
    a.tpg = NT;
    const size_t tab = (size_t)NT * a.ncw * TAB_CHUNK + TAB_ZERO;
    const size_t lds = KSLICES * tab + (size_t)KSLICES * NT * 16 * 4;
    const int row_blocks = (a.rows + 15) / 16, ngroups = (a.nt + NT - 1) / NT;
    if (a.tab) {
        /* token groups split over enough workgroups to fill the device
         * (about 512), each walking its share with the weights held */
        const int parts = max(1, min(ngroups, (512 + row_blocks - 1) / row_blocks));
        a.gpw = (ngroups + parts - 1) / parts;
        const dim3 grid((unsigned)row_blocks, (unsigned)((ngroups + a.gpw - 1) / a.gpw));
        hipLaunchKernelGGL((k_gemv_mx_tab<FMT, CPW, NT>), grid, dim3(256), lds, st, a);
    } else {
        const dim3 grid((unsigned)row_blocks, (unsigned)ngroups);
        hipLaunchKernelGGL((k_gemv_mx<FMT, CPW, NT>), grid, dim3(256), lds, st, a);
    }
    return hipGetLastError();
}


template <int FMT, int CPW>
hipError_t gemv_mx_k(GemvMxArgs a, hipStream_t st)
{
    constexpr int TPG = CPW >= 16 ? 1 : (16 / CPW > 4 ? 4 : 16 / CPW);
    if (a.nt == 1) return gemv_mx_nt<FMT, CPW, 1>(a, st);
    if constexpr (TPG >= 2) {
        if (a.nt == 2 || TPG == 2) return gemv_mx_nt<FMT, CPW, 2>(a, st);
    }
    if constexpr (TPG >= 4) return gemv_mx_nt<FMT, CPW, 4>(a, st);
    return gemv_mx_nt<FMT, CPW, 1>(a, st);
}

template <int FMT>
hipError_t gemv_mx_fmt(GemvMxArgs a, hipStream_t st)
{
    switch (cpw_for(a.ncw)) {
    case 1: return gemv_mx_k<FMT, 1>(a, st);
    case 2: return gemv_mx_k<FMT, 2>(a, st);
    case 4: return gemv_mx_k<FMT, 4>(a, st);
    case 8: return gemv_mx_k<FMT, 8>(a, st);
    default: return gemv_mx_k<FMT, 16>(a, st);
    }
}

template <int FMT, int CPW>
hipError_t gateup_mx_k(const GateUpMxArgs &a, hipStream_t st)
{
    const size_t lds = 8 * ((size_t)a.ncw * TAB_CHUNK + TAB_ZERO) + 2 * 4 * 2 * 16 * 4;
    const dim3 grid((unsigned)(a.nslots * (a.inter / 32)));
    if constexpr (FMT == FMT_FP4_E8M0 && CPW <= 8)
        hipLaunchKernelGGL((k_gateup_mx<FMT, CPW>), grid, dim3(512), lds, st, a);
    else
        hipLaunchKernelGGL((k_gateup_mx_wide<FMT, CPW>), grid, dim3(512), lds, st, a);
    return hipGetLastError();
}

template <int NP>
hipError_t gateup_px_k(const GateUpMxArgs &a, hipStream_t st)
{
    const size_t lds = (size_t)4 * NP * TAB_CHUNK + TAB_ZERO + (4 * 2 * 2 * 16 + 32) * 4;
    const dim3 grid((unsigned)(a.nslots * (a.inter / 32)));
    hipLaunchKernelGGL((k_gateup_px<NP>), grid, dim3(512), lds, st, a);
    return hipGetLastError();
}

template <int FMT, int NP>
hipError_t gateup_px8_k(const GateUpMxArgs &a, hipStream_t st)
{
    const size_t lds = (size_t)8 * NP * TAB_CHUNK + TAB_ZERO + 2 * 4 * 16 * 4;
    const dim3 grid((unsigned)(a.nslots * (a.inter / 8)));
    hipLaunchKernelGGL((k_gateup_px8<FMT, NP>), grid, dim3(512), lds, st, a);
    return hipGetLastError();
}

template <int FMT>
hipError_t gateup_mx_fmt(const GateUpMxArgs &a, hipStream_t st)
{
    if constexpr (FMT != FMT_FP4_E8M0) {
        if (!a.msplit) {                    /* 8-row tiles: hidden = 1024 NP */
            switch (a.hidden) {
            case 1024: return gateup_px8_k<FMT, 1>(a, st);
            case 2048: return gateup_px8_k<FMT, 2>(a, st);
            case 4096: return gateup_px8_k<FMT, 4>(a, st);
            default: break;
            }
        }
    }
    if constexpr (FMT == FMT_FP4_E8M0) {
        switch (a.hidden) {                 /* chunk-pair kernel: hidden = 512 NP */
        case 512: return gateup_px_k<1>(a, st);
        case 1024: return gateup_px_k<2>(a, st);
        case 2048: return gateup_px_k<4>(a, st);
        case 4096: return gateup_px_k<8>(a, st);
        default: break;
        }
    }
    switch (cpw_for(a.ncw)) {
    case 1: return gateup_mx_k<FMT, 1>(a, st);
    case 2: return gateup_mx_k<FMT, 2>(a, st);
    case 4: return gateup_mx_k<FMT, 4>(a, st);
    case 8: return gateup_mx_k<FMT, 8>(a, st);
    default:
        if constexpr (FMT == FMT_FP4_E8M0) return gateup_mx_k<FMT, 16>(a, st);
        return hipErrorInvalidValue;
    }
}

} // namespace

size_t gemv_tab_chunk_bytes() { return TAB_CHUNK; }

hipError_t split_x_tab_launch(uint8_t *tab, const float *x, int x_ld, int nt, int cols, hipStream_t st)
{
    if (nt <= 0 || cols <= 0 || cols % 128 || (long)nt * (cols / 128) * 16 >= (1L << 31))
        return hipErrorInvalidValue;
    const int nc = cols / 128;
    const int units = nt * nc * 16;
    hipLaunchKernelGGL(k_split_x_tab, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, st, tab, x, x_ld, nt, nc);
    return hipGetLastError();
}

/* chunks per wave for a K of `cols` (at most 8192 FP8 or FP4 columns), 0
 * when the MFMA path does not take it */
int gemv_mx_ncw(int fmt, int cols)
{
    (void)fmt;
    if (cols <= 0 || cols % 128) return 0;
    const int ncw = (cols / 128 + KSLICES - 1) / KSLICES;
    return ncw <= 16 ? ncw : 0;
}

/* the gate/up kernels take up to 8 FP8 chunks per wave (4096 columns) */
int gateup_mx_ncw(int fmt, int cols)
{
    const int ncw = gemv_mx_ncw(fmt, cols);
    return fmt == FMT_FP4_E8M0 || ncw <= 8 ? ncw : 0;
}

size_t mx_split_bytes(int inter) { return (size_t)(inter / 128) * MTAB_CHUNK; }

template <int FMT, int NP, int KQ, int TILES>
hipError_t gemv_px8_k(const GemvMxArgs *jobs, int nj, hipStream_t st)
{
    const size_t lds = (size_t)2 * KQ * NP * TAB_CHUNK + TAB_ZERO + TILES * KQ * 16 * 4;
    if (nj == 1) {
        hipLaunchKernelGGL((k_gemv_px8<FMT, NP, KQ, TILES>), dim3((unsigned)(jobs[0].rows / (8 * TILES))),
                           dim3(64 * KQ * TILES), lds, st, jobs[0]);
        return hipGetLastError();
    }
    Px8Jobs m;
    memset(&m, 0, sizeof m);
    m.nj = nj;
    for (int j = 0; j < nj; j++) {
        m.job[j] = jobs[j];
        m.first[j + 1] = m.first[j] + jobs[j].rows / (8 * TILES);
    }
    hipLaunchKernelGGL((k_gemv_px8_multi<FMT, NP, KQ, TILES>), dim3((unsigned)m.first[nj]), dim3(64 * KQ * TILES),
                       lds, st, m);
    return hipGetLastError();
}

/* One token, FP8, rows in whole 16-row groups, scale blocks whole 8-row
 * tiles, 1024 / 2048 / 4096 / 8192 columns: the 8-row chunk-pair matvec.
 * Waves per tile (KQ) and tiles per workgroup by the matrix's shape (the
 * jobs of one launch share it, so each job's bits are its single call's),
 * as measured (us per call, weights cold): 4096 x 4096
 * two tiles x four quarters 5.2 (one tile x eight 5.4); 1024 x 4096 one tile
 * x eight 3.5 (two x four 4.6); 4096 x 2048 one tile x four 3.6; 8192 x 1024
 * one tile x two 3.6; 32768 x 1024 two tiles x two 8.5; 4096 x 8192 two
 * tiles x eight 8.4 (two x four 8.9, the 16-chunk GEMV 11.7); 1024 x 8192
 * one tile x eight 5.3. */
template <int FMT>
hipError_t gemv_px8_fmt(const GemvMxArgs *jobs, int nj, hipStream_t st)
{
    const int rows = jobs[0].rows;
    switch (jobs[0].cols) {
    case 1024:
        return rows >= 16384 ? gemv_px8_k<FMT, 2, 2, 2>(jobs, nj, st) : gemv_px8_k<FMT, 2, 2, 1>(jobs, nj, st);
    case 2048: return gemv_px8_k<FMT, 2, 4, 1>(jobs, nj, st);
    case 8192:
        return rows >= 4096 ? gemv_px8_k<FMT, 4, 8, 2>(jobs, nj, st) : gemv_px8_k<FMT, 4, 8, 1>(jobs, nj, st);
    default:
        return rows >= 4096 ? gemv_px8_k<FMT, 4, 4, 2>(jobs, nj, st) : gemv_px8_k<FMT, 2, 8, 1>(jobs, nj, st);
    }
}

bool gemv_px8_ok(int fmt, const GemvMxArgs &a)
{
    return (fmt == FMT_FP8_E8M0 || fmt == FMT_FP8_F32S) && a.nt == 1 && a.rows % 16 == 0 &&
           a.blk_r % 8 == 0 && a.row_bytes == a.cols &&
           (a.cols == 1024 || a.cols == 2048 || a.cols == 4096 || a.cols == 8192);
}

int gemv_px8_class(const GemvMxArgs &a)
{
    const bool big = a.cols == 1024 ? a.rows >= 16384 : a.cols == 2048 ? false : a.rows >= 4096;
    return a.cols * 2 + (big ? 1 : 0);
}

hipError_t gemv_px8_multi_launch(int fmt, const GemvMxArgs *jobs, int nj, hipStream_t st)
{
    if (nj < 1 || nj > PX8_MAX_JOBS) return hipErrorInvalidValue;
    for (int j = 0; j < nj; j++)
        if (!gemv_px8_ok(fmt, jobs[j]) || gemv_px8_class(jobs[j]) != gemv_px8_class(jobs[0]))
            return hipErrorInvalidValue;
    return fmt == FMT_FP8_E8M0 ? gemv_px8_fmt<FMT_FP8_E8M0>(jobs, nj, st) : gemv_px8_fmt<FMT_FP8_F32S>(jobs, nj, st);
}

hipError_t gemv_mx_launch(int fmt, GemvMxArgs a, hipStream_t st)
{
    a.ncw = gemv_mx_ncw(fmt, a.cols);
    if (!a.ncw || a.nt <= 0) return hipErrorInvalidValue;
    if (gemv_px8_ok(fmt, a))
        return fmt == FMT_FP8_E8M0 ? gemv_px8_fmt<FMT_FP8_E8M0>(&a, 1, st) : gemv_px8_fmt<FMT_FP8_F32S>(&a, 1, st);
    switch (fmt) {
    case FMT_FP8_E8M0: return gemv_mx_fmt<FMT_FP8_E8M0>(a, st);
    case FMT_FP8_F32S: return gemv_mx_fmt<FMT_FP8_F32S>(a, st);
    case FMT_FP4_E8M0: return gemv_mx_fmt<FMT_FP4_E8M0>(a, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t gateup_mx_launch(int fmt, GateUpMxArgs a, hipStream_t st)
{
    a.ncw = gateup_mx_ncw(fmt, a.hidden);
    if (!a.ncw || a.inter % 128) return hipErrorInvalidValue;
    switch (fmt) {
    case FMT_FP8_E8M0: return gateup_mx_fmt<FMT_FP8_E8M0>(a, st);
    case FMT_FP8_F32S: return gateup_mx_fmt<FMT_FP8_F32S>(a, st);
    case FMT_FP4_E8M0: return gateup_mx_fmt<FMT_FP4_E8M0>(a, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t down_mx_launch(DownMxArgs a, hipStream_t st)
{
    if (a.topk < 1 || a.topk > 8 || a.inter % 128 || a.inter > 2048 || a.hidden <= 0)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.hidden + 15) / 16)), block(128 * a.topk);
    switch (a.inter) {                      /* chunk-pair kernel: inter = 256 NP */
    case 256: hipLaunchKernelGGL((k_down_px<1>), grid, block, 0, st, a); return hipGetLastError();
    case 512: hipLaunchKernelGGL((k_down_px<2>), grid, block, 0, st, a); return hipGetLastError();
    case 1024: hipLaunchKernelGGL((k_down_px<4>), grid, block, 0, st, a); return hipGetLastError();
    case 2048: hipLaunchKernelGGL((k_down_px<8>), grid, block, 0, st, a); return hipGetLastError();
    default: break;
    }
    a.ncw = (a.inter / 128 + 1) / 2;
    switch (cpw_for(a.ncw)) {
    case 1: hipLaunchKernelGGL((k_down_mx<1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((k_down_mx<2>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((k_down_mx<4>), grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL((k_down_mx<8>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;      /* inter > 2048: 1024 threads cannot hold 16 chunks */
    }
    return hipGetLastError();
}

bool moe_one_ok(int hidden, int inter, int topk)
{
    if (!(hidden == 512 || hidden == 1024 || hidden == 2048 || hidden == 4096)) return false;
    if (!(inter == 256 || inter == 512 || inter == 1024 || inter == 2048)) return false;
    if (topk < 1 || topk > MX_ROUTED_MAX) return false;
    /* down workgroups: every routed slot's table in LDS, two workgroups per CU */
    return ONE_HEAD_BYTES + (long)topk * one_slot_lds(inter) <= 80L * 1024;
}

template <int NPG, int NPD>
static hipError_t moe_one_k(const MoeOneArgs &a, hipStream_t st)
{
    const size_t lds = std::max<size_t>((size_t)4 * NPG * TAB_CHUNK + TAB_ZERO + (4 * 2 * 2 * 16 + 32) * 4,
                                        (size_t)ONE_HEAD_BYTES + (size_t)a.dn.topk * one_slot_lds(256 * NPD));
    const unsigned grid = (unsigned)(a.gu_blocks + a.dn.hidden / 16);
    /* the largest LDS any launch of this instantiation asks for, set once
     * (not again inside a stream capture of a later call) */
    static int lds_set = 64 * 1024;
    if ((int)lds > lds_set) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_moe_one<NPG, NPD>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)(80 * 1024 + ONE_HEAD_BYTES));
        if (e != hipSuccess) return e;
        lds_set = 80 * 1024 + ONE_HEAD_BYTES;
    }
    hipLaunchKernelGGL((k_moe_one<NPG, NPD>), dim3(grid), dim3(512), lds, st, a);
    return hipGetLastError();
}

template <int NPG>
static hipError_t moe_one_d(const MoeOneArgs &a, hipStream_t st)
{
    switch (a.dn.inter) {
    case 256: return moe_one_k<NPG, 1>(a, st);
    case 512: return moe_one_k<NPG, 2>(a, st);
    case 1024: return moe_one_k<NPG, 4>(a, st);
    default: return moe_one_k<NPG, 8>(a, st);
    }
}

/* Whether the balanced form takes this geometry: every gate/up half block in
 * one round of BAL_HB per workgroup, a down scale row of whole 16-byte pieces
 * (inter >= 512), one gate/up wave per down unit (topk <= 6), the LDS of one
 * workgroup. */
static bool bal_geometry_ok(int hidden, int inter, int topk)
{
    const long half_blocks = (long)topk * inter / 16, groups = hidden / 16;
    return inter >= 512 && half_blocks <= (long)BAL_HB * groups && 2 * topk <= BAL_GU_WAVES &&
           bal_lds(hidden, inter, topk).total <= 160 * 1024;
}

/* Launch k_moe_bal when the whole grid is resident at once (one workgroup of
 * 1024 threads per CU); hipErrorNotSupported otherwise, and the caller takes
 * k_moe_one. The occupancy check and the LDS attribute are set up once per
 * instantiation (not inside a stream capture of a later call). */
template <int NPH, int NPD>
static hipError_t moe_bal_k(const MoeOneArgs &a, hipStream_t st)
{
    static int fits = -1;
    const size_t lds = (size_t)bal_lds(512 * NPH, 256 * NPD, a.dn.topk).total;
    const unsigned grid = (unsigned)(a.dn.hidden / 16);
    if (fits < 0) {
        int dev = 0, cus = 0, per_cu = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)k_moe_bal<NPH, NPD>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e == hipSuccess)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_moe_bal<NPH, NPD>,
                                                             BAL_WAVES * 64, 160 * 1024);
        /* the largest grid of this instantiation is hidden / 16 = 32 NPH; a
         * device that cannot hold it (or a failed query) keeps k_moe_one */
        fits = e == hipSuccess && (long)per_cu * cus >= 32L * NPH ? 1 : 0;
        if (e != hipSuccess) (void)hipGetLastError();
    }
    if (!fits) return hipErrorNotSupported;
    hipLaunchKernelGGL((k_moe_bal<NPH, NPD>), dim3(grid), dim3(BAL_WAVES * 64), lds, st, a);
    return hipGetLastError();
}

template <int NPH>
static hipError_t moe_bal_d(const MoeOneArgs &a, hipStream_t st)
{
    switch (a.dn.inter) {
    case 512: return moe_bal_k<NPH, 2>(a, st);
    case 1024: return moe_bal_k<NPH, 4>(a, st);
    default: return moe_bal_k<NPH, 8>(a, st);
    }
}

static hipError_t moe_bal_launch(MoeOneArgs a, hipStream_t st)
{
    if (!a.midc || a.mid_copies < 1 || a.copy_ld < (size_t)a.dn.topk * mx_split_bytes(a.dn.inter))
        return hipErrorNotSupported;
    a.pub.items = (unsigned)(a.dn.hidden / 16);
    a.pub.total = a.pub.items;
    switch (a.gu.hidden) {
    case 512: return moe_bal_d<1>(a, st);
    case 1024: return moe_bal_d<2>(a, st);
    case 2048: return moe_bal_d<4>(a, st);
    default: return moe_bal_d<8>(a, st);
    }
}

hipError_t moe_one_launch(MoeOneArgs a, hipStream_t st, bool balanced)
{
    if (!moe_one_ok(a.gu.hidden, a.gu.inter, a.gu.nslots) || a.dn.hidden != a.gu.hidden ||
        a.dn.inter != a.gu.inter || a.dn.topk != a.gu.nslots || !a.gu.msplit || !a.pub.count ||
        !a.pub.done || !a.pub.leave)
        return hipErrorInvalidValue;
    if (balanced && bal_geometry_ok(a.gu.hidden, a.gu.inter, a.gu.nslots)) {
        const hipError_t e = moe_bal_launch(a, st);
        if (e != hipErrorNotSupported) return e;
    }
    a.gu_blocks = a.gu.nslots * (a.gu.inter / 32);
    a.pub.items = (unsigned)a.gu_blocks;
    a.pub.total = (unsigned)(a.gu_blocks + a.dn.hidden / 16);
    switch (a.gu.hidden) {
    case 512: return moe_one_d<1>(a, st);
    case 1024: return moe_one_d<2>(a, st);
    case 2048: return moe_one_d<4>(a, st);
    default: return moe_one_d<8>(a, st);
    }
}

} // namespace dsv4
