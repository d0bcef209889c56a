/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_compute_hip.c - the reference's compute entry points, same names and
 * signatures, running on the gfx950 library.
 *
 *   dsv4_mmq_n            src/10_compute/dsv4_matmul.h:40
 *   dsv4_mmq              src/10_compute/dsv4_matmul.h:43
 *   dsv4_expert_forward   src/10_compute/dsv4_kernels.h:30-32
 *
 * A program written against the reference's src/10_compute links this
 * library instead and runs unchanged, provided the weight arenas were
 * uploaded with dsv4_hip_register() (the loader's job). Error behaviour
 * mirrors the reference's dsv4_mmq_n, which aborts on a matrix it cannot run
 * (src/10_compute/dsv4_matmul.c:110-113): where the GPU path returns -1 these
 * functions print the reason and abort. There is deliberately no CPU
 * fallback here; a build that keeps the CPU bodies calls dsv4_hip_mmq_n()
 * first instead (see the integration notes).
 *
 * The first call initialises device 0 unless dsv4_hip_init() was called.
 */
#include <stdio.h>
#include <stdlib.h>

#include "../../include/dsv4_hip.h"

void dsv4_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt);
void dsv4_mmq(float *y, const float *x, const DSV4QMat *m);
void dsv4_expert_forward(float *out, const float *x, const DSV4ExpertW *e,
                         float *gate, float *up, float *mid, int inter,
                         float limit);

static void ensure_device(void)
{
    static int done;
    if (done) return;
    if (dsv4_hip_init(0) != 0) {
        fprintf(stderr, "dsv4_hip: no usable gfx950 device: %s\n",
                dsv4_hip_last_error());
        abort();
    }
    done = 1;
}

void dsv4_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt)
{
    if (nt <= 0) return;
    ensure_device();
    if (dsv4_hip_mmq_n(y, x, m, nt) != 0) {
        fprintf(stderr, "dsv4_mmq_n: matrix wdt %d (%dx%d) not run on the GPU: %s\n",
                m ? m->wdt : -1, m ? m->rows : 0, m ? m->cols : 0,
                dsv4_hip_last_error());
        abort();
    }
}

void dsv4_mmq(float *y, const float *x, const DSV4QMat *m)
{
    dsv4_mmq_n(y, x, m, 1);
}

/* gate / up / mid are the caller's workspace rows in the reference; here the
 * intermediates live on the device and the rows are left untouched. */
void dsv4_expert_forward(float *out, const float *x, const DSV4ExpertW *e,
                         float *gate, float *up, float *mid, int inter,
                         float limit)
{
    (void)gate; (void)up; (void)mid;
    ensure_device();
    if (dsv4_hip_expert_forward(out, x, e, inter, limit) != 0) {
        fprintf(stderr, "dsv4_expert_forward: not run on the GPU: %s\n",
                dsv4_hip_last_error());
        abort();
    }
}
