/* SPDX-License-Identifier: Apache-2.0 */
/* route_math_host.cpp - the router's score transform of the device library
 * (deepseek-v4-in-c_amd/csrc/dsv4_route_math.h), built for the host, against
 * the host C library the reference calls (src/10_compute/dsv4_ops.c:43-46,
 * 121-122: orig = sqrtf(x > 20 ? x : log1pf(expf(x)))).
 *
 *   g++ -O2 -fopenmp -ffp-contract=off route_math_host.cpp -o route_math_host
 *   route_math_host check        every fp32 x in [-104, 20] and the specials:
 *                                prints "expf N log1pf N orig N" mismatches
 *   route_math_host sums LOG2    libm's orig over the same inputs in the order
 *                                of route_input(), per chunk of 2^LOG2 inputs:
 *                                "chunk s1 s2" with s1 = sum of the orig bits,
 *                                s2 = sum of bits * (index in chunk & 63)
 *
 * Inputs in order: -0 down to -104 (bits 0x80000000 .. 0xC2D00000), then +0
 * up to 20 (0 .. 0x41A00000). */
#include <inttypes.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../deepseek-v4-in-c_amd/csrc/dsv4_route_math.h"

using namespace dsv4_route;

static const int64_t N_NEG = 0x42D00001LL;   /* -0 .. -104 */
static const int64_t N_POS = 0x41A00001LL;   /* +0 .. 20   */

static inline uint32_t route_input(int64_t i)
{
    return i < N_NEG ? 0x80000000u + (uint32_t)i : (uint32_t)(i - N_NEG);
}

static inline float libm_orig(float x)
{
    return sqrtf(x > 20.0f ? x : log1pf(expf(x)));
}

static int check(void)
{
    long bad_e = 0, bad_l = 0, bad_o = 0;
    const int64_t n = N_NEG + N_POS;
#pragma omp parallel for reduction(+ : bad_e, bad_l, bad_o) schedule(static, 1 << 16)
    for (int64_t i = 0; i < n; i++) {
        const float x = fof(route_input(i));
        const float e = expf(x);
        bad_e += fbits(expf_lib(x)) != fbits(e);
        bad_l += fbits(log1pf_lib(e)) != fbits(log1pf(e));
        bad_o += fbits(route_orig(x)) != fbits(libm_orig(x));
    }
    /* beyond the range: the threshold's other side, overflow and underflow
     * of expf, infinities and NaN */
    const float sp[] = {20.000002f, 25.0f, 88.0f, 88.8f, 1e30f, -104.00001f, -150.0f, -1e30f,
                        INFINITY, -INFINITY, NAN, 0x1p-149f, -0x1p-149f};
    for (float x : sp) {
        const float o = route_orig(x), w = libm_orig(x);
        if (!(isnan(o) && isnan(w)) && fbits(o) != fbits(w)) {
            bad_o++;
            fprintf(stderr, "orig(%a): %a vs libm %a\n", x, o, w);
        }
        const float e = expf_lib(x), we = expf(x);
        if (!(isnan(e) && isnan(we)) && fbits(e) != fbits(we)) {
            bad_e++;
            fprintf(stderr, "expf(%a): %a vs libm %a\n", x, e, we);
        }
    }
    printf("expf %ld log1pf %ld orig %ld\n", bad_e, bad_l, bad_o);
    return 0;
}

static int sums(int log2)
{
    const int64_t n = N_NEG + N_POS, chunk = (int64_t)1 << log2;
    const int64_t chunks = (n + chunk - 1) / chunk;
    int64_t *s1 = (int64_t *)calloc((size_t)chunks, sizeof(int64_t));
    int64_t *s2 = (int64_t *)calloc((size_t)chunks, sizeof(int64_t));
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < chunks; c++) {
        int64_t a = 0, b = 0;
        const int64_t end = (c + 1) * chunk < n ? (c + 1) * chunk : n;
        for (int64_t i = c * chunk; i < end; i++) {
            const int64_t o = fbits(libm_orig(fof(route_input(i))));
            a += o;
            b += o * ((i - c * chunk) & 63);
        }
        s1[c] = a;
        s2[c] = b;
    }
    for (int64_t c = 0; c < chunks; c++) printf("%" PRId64 " %" PRId64 " %" PRId64 "\n", c, s1[c], s2[c]);
    free(s1);
    free(s2);
    return 0;
}

int main(int argc, char **argv)
{
    if (argc >= 2 && !strcmp(argv[1], "check")) return check();
    if (argc >= 3 && !strcmp(argv[1], "sums")) return sums(atoi(argv[2]));
    fprintf(stderr, "usage: %s check | sums LOG2\n", argv[0]);
    return 2;
}
