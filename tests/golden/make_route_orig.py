# SPDX-License-Identifier: Apache-2.0
"""Write tests/golden/route_orig.npz: checksums of the reference's router
transform orig = sqrtf(x > 20 ? x : log1pf(expf(x)))
(src/10_compute/dsv4_ops.c:43-46, 121-122), evaluated with the host C library
(glibc) over every fp32 input x in [-104, 20], per chunk of 2^24 inputs in the
order of tests/route_math_host.cpp (-0 down to -104, then +0 up to 20):

    s1[c] = sum of the orig bits,  s2[c] = sum of bits * (index in chunk & 63)

    python tests/golden/make_route_orig.py

The GPU test feeds the same inputs to dsv4_hip_route_dev and compares its
orig output chunk by chunk with these sums.
"""
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CHUNK_LOG2 = 24
N_NEG, N_POS = 0x42D00001, 0x41A00001


def build_host_check(out_dir):
    """g++ build of tests/route_math_host.cpp; returns the binary's path."""
    exe = os.path.join(out_dir, "route_math_host")
    src = os.path.join(HERE, "..", "route_math_host.cpp")
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", src, "-o", exe], check=True)
    return exe


def main():
    with tempfile.TemporaryDirectory() as d:
        exe = build_host_check(d)
        out = subprocess.run([exe, "sums", str(CHUNK_LOG2)], check=True, capture_output=True,
                             text=True).stdout
    rows = np.array([[int(v) for v in ln.split()] for ln in out.splitlines()], np.int64)
    assert np.array_equal(rows[:, 0], np.arange(len(rows)))
    np.savez_compressed(os.path.join(HERE, "route_orig.npz"), chunk_log2=np.int64(CHUNK_LOG2),
                        n_neg=np.int64(N_NEG), n_pos=np.int64(N_POS), s1=rows[:, 1], s2=rows[:, 2])
    print(f"{len(rows)} chunks written", file=sys.stderr)


if __name__ == "__main__":
    main()
