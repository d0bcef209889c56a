/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_route.hip - the MoE router on the device.
 *
 * Replaces dsv4_route (src/10_compute/dsv4_ops.c:117-157) for n tokens, one
 * workgroup per token, so that the decode step's router needs no host round
 * trip between the gate matvec and the experts:
 *   orig[e]   = sqrt(softplus(scores[e]))   softplus(x) = x for x > 20
 *   biased[e] = orig[e] + bias[e]            (orig[e] without a bias)
 *   idx       = tid2eid[token] (hash routing), or the topk largest biased
 *               scores, descending, ties to the lower expert id
 *   w[k]      = orig[idx[k]] * inv * route_scale,  inv = (float)(1 / sum_k
 *               (double) orig[idx[k]]), 0 when that sum is 0
 * The bias steers the selection only; the weights come from orig.
 *
 * Selection. The reference's loop picks, for each k, the first untaken
 * expert and replaces it by every later untaken one whose biased score is
 * strictly greater. Written as a closed form: if the first untaken score is
 * NaN it stays; otherwise the pick is the largest non-NaN untaken score, the
 * lowest id among equals (+0 and -0 compare equal, as in the loop). The
 * workgroup reduces (score, id) pairs under that order in one pass per k.
 *
 * softplus and sqrt are evaluated in fp64 and rounded once to fp32:
 * (float)log1p((double)(float)exp(x)) is the correctly rounded log1pf of the
 * correctly rounded expf. glibc's log1pf is not correctly rounded, so orig
 * may differ from the reference's by one unit in the last place on about 1%
 * of inputs in [-104, 20] (sqrt agrees on all of them); the ids agree unless
 * two biased scores lie within that unit of each other.
 *
 * A hash-routed id outside [0, n_experts), or a token id outside [0, n_vocab)
 * (whose ids are then -1), raises ST_BAD_EXPERT_ID; every weight of that
 * token is NaN, and the ids are written as they are so that the experts' own
 * range check catches them too.
 *
 * Bound: launch latency (n_experts * 4 bytes per token).
 */
#include "dsv4_internal.h"

namespace dsv4 {

namespace {

constexpr int RT_THREADS = 256;

/* the better of two (score, id) candidates; id < 0 is no candidate */
__device__ __forceinline__ void better(float &v, int &e, float v2, int e2)
{
    if (e2 < 0) return;
    if (e < 0 || v2 > v || (v2 == v && e2 < e)) { v = v2; e = e2; }
}

__global__ __launch_bounds__(RT_THREADS) void k_gate_route(GateRouteArgs a)
{
    __shared__ float bs[GATE_ROUTE_MAX_EXPERTS];
    __shared__ float og[GATE_ROUTE_MAX_EXPERTS];
    __shared__ unsigned char taken[GATE_ROUTE_MAX_EXPERTS];
    __shared__ float rv[RT_THREADS / 64];
    __shared__ int re[RT_THREADS / 64], rf[RT_THREADS / 64];
    __shared__ int pick[GATE_ROUTE_MAX_TOPK];

    const int t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int ne = a.n_experts, topk = a.topk;
    const float *sc = a.scores + (size_t)t * a.scores_ld;

    for (int e = tid; e < ne; e += RT_THREADS) {
        const float x = sc[e];
        const float sp = x > 20.0f ? x : (float)log1p((double)(float)exp((double)x));
        const float o = (float)sqrt((double)sp);
        og[e] = o;
        bs[e] = a.bias ? o + a.bias[e] : o;
        taken[e] = 0;
        if (a.orig) a.orig[(size_t)t * ne + e] = o;
    }
    __syncthreads();

    if (a.tid2eid) {
        const int tok = a.token_ids ? a.token_ids[t] : a.token_id;
        if (tid < topk)
            pick[tid] = tok >= 0 && tok < a.n_vocab ? (int)a.tid2eid[(int64_t)tok * topk + tid] : -1;
    } else {
        for (int k = 0; k < topk; k++) {
            float v = 0.0f;
            int e = -1, first = 0x7fffffff;
            for (int j = tid; j < ne; j += RT_THREADS) {
                if (taken[j]) continue;
                if (j < first) first = j;
                const float s = bs[j];
                if (s == s) better(v, e, s, j);
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const float v2 = __shfl_xor(v, off, 64);
                const int e2 = __shfl_xor(e, off, 64);
                const int f2 = __shfl_xor(first, off, 64);
                better(v, e, v2, e2);
                first = f2 < first ? f2 : first;
            }
            if (lane == 0) { rv[wv] = v; re[wv] = e; rf[wv] = first; }
            __syncthreads();
            if (tid == 0) {
                for (int w = 1; w < RT_THREADS / 64; w++) {
                    better(v, e, rv[w], re[w]);
                    first = rf[w] < first ? rf[w] : first;
                }
                /* a NaN first candidate is never replaced in the reference's scan */
                const int p = bs[first] != bs[first] ? first : e;
                pick[k] = p;
                taken[p] = 1;
            }
            __syncthreads();
        }
    }
    __syncthreads();

    if (tid == 0) {
        int bad = 0;
        double sum = 0.0;
        float wk[GATE_ROUTE_MAX_TOPK];
        for (int k = 0; k < topk; k++) {
            const int p = pick[k];
            if (p < 0 || p >= ne) { bad = 1; wk[k] = 0.0f; continue; }
            wk[k] = og[p];
            sum += (double)wk[k];
        }
        const float inv = sum != 0.0 ? (float)(1.0 / sum) : 0.0f;
        for (int k = 0; k < topk; k++) {
            a.idx[(size_t)t * topk + k] = pick[k];
            a.w[(size_t)t * topk + k] = bad ? __builtin_nanf("") : wk[k] * inv * a.route_scale;
        }
        if (bad) atomicOr(a.status, ST_BAD_EXPERT_ID);
    }
}

} // namespace

hipError_t gate_route_launch(const GateRouteArgs &a, hipStream_t st)
{
    if (a.n <= 0 || a.n_experts < 1 || a.n_experts > GATE_ROUTE_MAX_EXPERTS || a.topk < 1 ||
        a.topk > GATE_ROUTE_MAX_TOPK || a.topk > a.n_experts || a.scores_ld < a.n_experts)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gate_route, dim3((unsigned)a.n), dim3(RT_THREADS), 0, st, a);
    return hipGetLastError();
}

} // namespace dsv4
