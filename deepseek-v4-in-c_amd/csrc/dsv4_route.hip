/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_route.hip - the MoE router on the device.
 *
 * Replaces dsv4_route (src/10_compute/dsv4_ops.c:117-157), and, fused with
 * the BF16 gate matvec in front of it (dsv4_mmq at
 * src/70_decode/dsv4_layer.c:52), the decode step's router, so that no host
 * round trip separates the gate from the experts:
 *   orig[e]   = sqrt(softplus(scores[e]))   softplus(x) = x for x > 20
 *   biased[e] = orig[e] + bias[e]            (orig[e] without a bias)
 *   idx       = tid2eid[token] (hash routing), or the topk largest biased
 *               scores, descending, ties to the lower expert id
 *   w[k]      = orig[idx[k]] * inv * route_scale,  inv = (float)(1 / sum_k
 *               (double) orig[idx[k]]), 0 when that sum is 0
 * The bias steers the selection only; the weights come from orig.
 *
 * Selection, one wavefront per token. The reference's loop picks, for each
 * k, the first untaken expert and replaces it by every later untaken one
 * whose biased score is strictly greater. As a closed form: if the first
 * untaken score is NaN it stays; otherwise the pick is the largest non-NaN
 * untaken score, the lowest id among equals (+0 and -0 compare equal, as in
 * the loop). Lane l holds experts l, l + 64, ...; each pick is one wave
 * maximum of 64-bit keys (order-preserving bits of the score above, the
 * complemented id below) over DPP lane moves, with no LDS and no barrier;
 * the first-untaken minimum is taken only when the token has a NaN.
 *
 * orig is the reference's bits: sqrtf, log1pf and expf restated from the
 * host library's algorithms (dsv4_route_math.h; identical to the host's libm
 * on every fp32 input of [-104, 20]), so the picks are the reference's ids.
 *
 * A hash-routed id outside [0, n_experts), or a token id outside [0, n_vocab)
 * (whose ids are then -1), raises ST_BAD_EXPERT_ID; every weight of that
 * token is NaN, and the ids are written as they are so that the experts' own
 * range check catches them too.
 *
 * The fused gate + router (k_gate_route_bf16): one wavefront per gate row
 * computes the row's fp64 dot product in bf16_n's order (16 serial FMA
 * chains and the reference's combine, src/10_compute/dsv4_matmul.c:88-113,
 * dsv4_dec_common.h:45-61; the bits of dsv4_mmq on the host), its orig and
 * biased score, stores
 * them device-scope (written through its XCD's L2); once the workgroup's
 * stores are acknowledged it adds one to a counter (one wave per
 * workgroup, so the rows spread over as many CUs as there are rows). The workgroup whose add
 * completes the count is the last of the launch: every other row's stores
 * are visible to its device-scope loads, so its first wave runs the
 * selection, then sets the counter back to zero for the next launch.
 * Nothing waits on another workgroup.
 *
 * Bound: launch latency; the gate's bytes (n_experts x hidden x 2) are read
 * once, by n_experts waves.
 */
#include "dsv4_internal.h"
#include "dsv4_bf16.h"
#include "dsv4_route_math.h"

namespace dsv4 {

namespace {

constexpr int RT_MAXJ = GATE_ROUTE_MAX_EXPERTS / 64;   /* experts per lane, at most */
constexpr int RT_GROUPS = GATE_ROUTE_GROUPS;           /* arrival counters below the top one */
constexpr int RT_LINE_WORDS = 32;                      /* one 128-byte line per counter */

template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWMASK, 0xF, false);
}

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t min32(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t max32(uint32_t a, uint32_t b) { return a > b ? a : b; }

/* Largest 32-bit value over the wave (each step one DPP-fused max). */
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max32(v, dpp_u32<DPP_QUAD_1032>(v, v));
    v = max32(v, dpp_u32<DPP_QUAD_2301>(v, v));
    v = max32(v, dpp_u32<DPP_ROW_HALF_MIRROR>(v, v));
    v = max32(v, dpp_u32<DPP_ROW_MIRROR>(v, v));
    v = max32(v, dpp_u32<DPP_ROW_BCAST15, 0xA>(v, v));
    v = max32(v, dpp_u32<DPP_ROW_BCAST31, 0xC>(v, v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

/* The largest 64-bit key over the wave: the largest upper half first (one
 * 32-bit reduction), then, among the lanes that hold it (almost always
 * one), the largest lower half. */
__device__ __forceinline__ uint64_t wave_max_key(uint64_t v)
{
    const uint32_t hi = wave_max_u32((uint32_t)(v >> 32));
    const uint64_t at = __builtin_amdgcn_ballot_w64((uint32_t)(v >> 32) == hi);
    uint32_t lo;
    if (__builtin_popcountll(at) == 1)
        lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, (int)__builtin_ctzll(at));
    else
        lo = wave_max_u32((uint32_t)(v >> 32) == hi ? (uint32_t)v : 0u);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
    v = min32(v, dpp_u32<DPP_QUAD_1032>(v, v));
    v = min32(v, dpp_u32<DPP_QUAD_2301>(v, v));
    v = min32(v, dpp_u32<DPP_ROW_HALF_MIRROR>(v, v));
    v = min32(v, dpp_u32<DPP_ROW_MIRROR>(v, v));
    v = min32(v, dpp_u32<DPP_ROW_BCAST15, 0xA>(v, v));
    v = min32(v, dpp_u32<DPP_ROW_BCAST31, 0xC>(v, v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

/* sqrt(softplus(x)) bit for bit as the reference's host libm computes it */
__device__ __forceinline__ float route_orig(float x) { return dsv4_route::route_orig(x); }

/* Order-preserving key of a non-NaN score (-0 as +0) over the complemented
 * expert id: the larger key is the reference's preferred pick. */
__device__ __forceinline__ uint64_t pick_key(float v, int e)
{
    uint32_t u = __float_as_uint(v);
    u = u == 0x80000000u ? 0u : u;
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)e;
}

/* Element j of a lane's register array, for a wave-uniform j. */
template <int NJ>
__device__ __forceinline__ float lane_elem(const float (&a)[NJ], int j)
{
    float r = a[0];
#pragma unroll
    for (int i = 1; i < NJ; i++) r = j == i ? a[i] : r;
    return r;
}

/* The router's picks and weights for one token, by one wavefront. og / bs:
 * the lane's orig and biased scores of experts lane + 64 j, j < NJ. hash:
 * the token's table row (topk ids), or NULL; hash_bad: a token id outside
 * the table. Lane k < topk holds pick k and its orig; the k loop stays
 * rolled so that no per-k value lives in scalar registers. */
template <int NJ>
__device__ __forceinline__ void route_wave(const float (&og)[NJ], const float (&bs)[NJ], int ne,
                                           int topk, const int64_t *hash, bool hash_bad,
                                           float route_scale, int *idx, float *w,
                                           unsigned *status, int lane)
{
    int my_pick = -1;
    float my_o = 0.0f;
    if (hash || hash_bad) {
        if (lane < topk && !hash_bad) my_pick = (int)hash[lane];
    } else {
        bool nan = false;
#pragma unroll
        for (int j = 0; j < NJ; j++) nan |= lane + 64 * j < ne && bs[j] != bs[j];
        const bool any_nan = __builtin_amdgcn_ballot_w64(nan) != 0;
        /* the keys of the lane's non-NaN experts; 0 marks none or taken */
        uint64_t key[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int e = lane + 64 * j;
            key[j] = e < ne && bs[j] == bs[j] ? pick_key(bs[j], e) : 0;
        }
        uint32_t taken = 0;
#pragma clang loop unroll(disable)
        for (int k = 0; k < topk; k++) {
            uint64_t best = key[0];
#pragma unroll
            for (int j = 1; j < NJ; j++) best = max64(best, key[j]);
            best = wave_max_key(best);
            int p = (int)~(uint32_t)best;
            if (any_nan) {
                /* a NaN first candidate is never replaced in the reference's scan */
                uint32_t first = 0xFFFFFFFFu;
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    const int e = lane + 64 * j;
                    first = e < ne && !((taken >> j) & 1u) ? min32(first, (uint32_t)e) : first;
                }
                const uint32_t f = wave_min_u32(first);
                const float fv = __int_as_float(__builtin_amdgcn_readlane(
                    __float_as_int(lane_elem(bs, (int)(f >> 6))), (int)(f & 63u)));
                if (best == 0 || fv != fv) p = (int)f;
            }
            p = __builtin_amdgcn_readfirstlane(p);
            my_pick = lane == k ? p : my_pick;
            const bool mine = (p & 63) == lane;
            taken |= mine ? 1u << (p >> 6) : 0u;
#pragma unroll
            for (int j = 0; j < NJ; j++) key[j] = mine && (p >> 6) == j ? 0 : key[j];
        }
    }
    /* each pick's orig, from the lane that holds it, in k order */
    bool bad = false;
    double sum = 0.0;
#pragma clang loop unroll(disable)
    for (int k = 0; k < topk; k++) {
        const int p = __builtin_amdgcn_readlane(my_pick, k);
        if (p < 0 || p >= ne) { bad = true; continue; }
        const float o = __int_as_float(__builtin_amdgcn_readlane(
            __float_as_int(lane_elem(og, p >> 6)), p & 63));
        my_o = lane == k ? o : my_o;
        sum += (double)o;
    }
    const float inv = sum != 0.0 ? (float)(1.0 / sum) : 0.0f;
    if (lane < topk) {
        idx[lane] = my_pick;
        w[lane] = bad ? __builtin_nanf("") : my_o * inv * route_scale;
    }
    if (bad && lane == 0) atomicOr(status, ST_BAD_EXPERT_ID);
}

/* The token's hash-table row, or NULL with *bad set for a token id outside
 * the table. */
__device__ __forceinline__ const int64_t *hash_row(const GateRouteArgs &a, int tok, bool *bad)
{
    *bad = false;
    if (!a.tid2eid) return nullptr;
    if (tok < 0 || tok >= a.n_vocab) { *bad = true; return nullptr; }
    return a.tid2eid + (int64_t)tok * a.topk;
}

/* dsv4_route for n tokens given their scores: one wavefront per token. */
template <int NJ>
__global__ __launch_bounds__(256) void k_route(GateRouteArgs a)
{
    const int t = wave_id();
    if (t >= a.n) return;
    const int lane = threadIdx.x & 63;
    const int ne = a.n_experts;
    const float *sc = a.scores + (size_t)t * a.scores_ld;
    float og[NJ], bs[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int e = lane + 64 * j;
        og[j] = bs[j] = 0.0f;
        if (e >= ne) continue;
        const float o = route_orig(sc[e]);
        og[j] = o;
        bs[j] = a.bias ? o + a.bias[e] : o;
        if (a.orig) a.orig[(size_t)t * ne + e] = o;
    }
    bool hbad;
    const int64_t *hrow = hash_row(a, a.token_ids ? a.token_ids[t] : a.token_id, &hbad);
    route_wave<NJ>(og, bs, ne, a.topk, hrow, hbad, a.route_scale, a.idx + (size_t)t * a.topk,
                   a.w + (size_t)t * a.topk, a.status, lane);
}

/* Device-scope 32-bit store: written through the XCD's L2, so another
 * XCD's device-scope load sees it. */
__device__ __forceinline__ void st_dev(float *p, float v)
{
    __hip_atomic_store((uint32_t *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Device-scope loads through a buffer resource (sc1: past the CU's L1 and the
 * XCD's L2), issued together rather than one atomic load at a time; bytes
 * beyond the resource read as zero. */
constexpr int RT_CPOL_SC1 = 16;
__device__ __forceinline__ float ld_dev(__amdgpu_buffer_rsrc_t r, int byte_off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, RT_CPOL_SC1));
}

/* The decode step's gate matvec and router in one launch: wave r computes
 * gate row r; the last wave to finish routes the token. KCH 16-byte chunks
 * of the row per lane (row bytes <= 1024 KCH). */
template <int KCH, int NJ>
__global__ __launch_bounds__(64) void k_gate_route_bf16(GateRouteArgs a)
{
    __shared__ unsigned s_old;
    __shared__ __align__(16) uint8_t wrow[KCH * 1024];
    __shared__ __align__(16) uint8_t xl[KCH * 2048];
    const int r = wave_id();
    const int ne = a.n_experts;
    const int lane = threadIdx.x & 63;
    if (r < ne) {
        /* the row and x into LDS, then bf16_n's 16 FMA chains in lanes 0-15 */
        bf16_rows_to_lds<KCH>(wrow, 0, a.gate_w, r, 1, 1, 2 * a.cols, lane);
        bf16_x_to_lds(xl, a.x, a.cols, lane);
        __builtin_amdgcn_s_waitcnt(0x0F70);         /* vmcnt(0): row and x landed */
        asm volatile("" ::: "memory");
        const double acc = bf16_row_dot((const uint16_t *)wrow, (const float *)xl, a.cols, lane);
        if (lane == 0) {
            const float s = (float)acc;
            const float o = route_orig(s);
            st_dev(a.ws_orig + r, o);
            st_dev(a.ws_biased + r, a.bias ? o + a.bias[r] : o);
            if (a.scores_out) a.scores_out[r] = s;
            if (a.orig) a.orig[r] = o;
        }
    }
    /* The workgroup's rows stored and acknowledged, then one add to its
     * group's counter; the last of a group adds one to the top counter, and
     * the last of those is the last workgroup. Adds to one word serialise
     * (one per row cost 3 us, one per workgroup 1.3 us). */
    __builtin_amdgcn_s_waitcnt(0x0F70);            /* vmcnt(0) */
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned grp = blockIdx.x % RT_GROUPS;
        const unsigned in_grp = (gridDim.x - grp + RT_GROUPS - 1) / RT_GROUPS;
        const unsigned groups = gridDim.x < RT_GROUPS ? gridDim.x : RT_GROUPS;
        unsigned last = 0;
        if (__hip_atomic_fetch_add(a.counter + grp * RT_LINE_WORDS, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == in_grp - 1)
            last = __hip_atomic_fetch_add(a.counter + RT_GROUPS * RT_LINE_WORDS, 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == groups - 1;
        s_old = last;
    }
    __syncthreads();
    if (!s_old || wave_in_group() != 0) return;
    /* the last workgroup: every other row's stores were acknowledged before
     * its workgroup's add */
    asm volatile("" ::: "memory");
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(a.ws_orig, (short)0, 4 * ne, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(a.ws_biased, (short)0, 4 * ne, 0x00020000);
    float og[NJ], bs[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        og[j] = ld_dev(ro, 4 * (lane + 64 * j));
        bs[j] = ld_dev(rb, 4 * (lane + 64 * j));
    }
    if (lane <= RT_GROUPS)
        __hip_atomic_store(a.counter + lane * RT_LINE_WORDS, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool hbad;
    const int64_t *hrow = hash_row(a, a.token_id, &hbad);
    route_wave<NJ>(og, bs, ne, a.topk, hrow, hbad, a.route_scale, a.idx, a.w, a.status, lane);
}

template <int NJ>
hipError_t launch_route_nj(const GateRouteArgs &a, hipStream_t st)
{
    if (a.gate_w) {
        /* one wave per workgroup: gate rows spread over as many CUs as there
         * are rows (four waves per workgroup: 0.5 us slower per call) */
        const int grid = a.n_experts;
        switch ((2 * a.cols + 1023) / 1024) {
        case 1: hipLaunchKernelGGL((k_gate_route_bf16<1, NJ>), dim3(grid), dim3(64), 0, st, a); break;
        case 2: hipLaunchKernelGGL((k_gate_route_bf16<2, NJ>), dim3(grid), dim3(64), 0, st, a); break;
        case 3: case 4: hipLaunchKernelGGL((k_gate_route_bf16<4, NJ>), dim3(grid), dim3(64), 0, st, a); break;
        case 5: case 6: case 7: case 8:
            hipLaunchKernelGGL((k_gate_route_bf16<8, NJ>), dim3(grid), dim3(64), 0, st, a); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_route<NJ>, dim3((unsigned)((a.n + 3) / 4)), dim3(256), 0, st, a);
    return hipGetLastError();
}

} // namespace

hipError_t gate_route_launch(const GateRouteArgs &a, hipStream_t st)
{
    if (a.n <= 0 || a.n_experts < 1 || a.n_experts > GATE_ROUTE_MAX_EXPERTS || a.topk < 1 ||
        a.topk > GATE_ROUTE_MAX_TOPK || a.topk > a.n_experts)
        return hipErrorInvalidValue;
    if (a.gate_w ? (a.n != 1 || a.cols <= 0 || a.cols % 8 || a.cols > 4096 || !a.counter ||
                    !a.ws_orig || !a.ws_biased)
                 : a.scores_ld < a.n_experts)
        return hipErrorInvalidValue;
    const int nj = (a.n_experts + 63) / 64;
    if (nj <= 1) return launch_route_nj<1>(a, st);
    if (nj <= 2) return launch_route_nj<2>(a, st);
    if (nj <= 4) return launch_route_nj<4>(a, st);
    if (nj <= 8) return launch_route_nj<8>(a, st);
    return launch_route_nj<RT_MAXJ>(a, st);
}

} // namespace dsv4
