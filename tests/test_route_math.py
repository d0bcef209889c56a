# SPDX-License-Identifier: Apache-2.0
"""The device router's score transform (deepseek-v4-in-c_amd/csrc/
dsv4_route_math.h: glibc's expf and log1pf restated operation for operation,
then sqrtf) built for the host and compared with the host's libm over every
fp32 input of [-104, 20] (2.2e9 inputs) and the specials beyond it:
expf, log1pf of expf's results and orig = sqrtf(softplus(x)), bit for bit
(src/10_compute/dsv4_ops.c:43-46, 121-122). Once with gcc and
-ffp-contract=off, once with ROCm's clang under FMA and the contraction mode
the device code is compiled with by default (fast-honor-pragmas): the
header's pragma must keep every unfused multiply-add rounding twice."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from conftest import golden

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "route_math_host.cpp")
CLANG = "/opt/rocm/llvm/bin/clang++"


def _run_check(exe):
    out = subprocess.run([exe, "check"], check=True, capture_output=True, text=True, timeout=600)
    assert out.stdout.split() == ["expf", "0", "log1pf", "0", "orig", "0"], out.stdout + out.stderr


def test_gcc_build_matches_libm(tmp_path):
    exe = str(tmp_path / "rmh_gcc")
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", SRC, "-o", exe], check=True)
    _run_check(exe)


def _host_has_fma():
    try:
        with open("/proc/cpuinfo") as f:
            return " fma " in f.read()
    except OSError:
        return False


@pytest.mark.skipif(not (os.path.exists(CLANG) and _host_has_fma()), reason="needs ROCm clang and FMA")
def test_clang_fma_build_matches_libm(tmp_path):
    exe = str(tmp_path / "rmh_clang")
    libdir = os.path.join(os.path.dirname(os.path.dirname(CLANG)), "lib")
    subprocess.run([CLANG, "-O2", "-mfma", "-mavx2", "-ffp-contract=fast-honor-pragmas", "-fopenmp=libomp",
                    SRC, "-o", exe, "-L" + libdir, "-Wl,-rpath," + libdir], check=True)
    _run_check(exe)


def test_orig_checksum_fixture_shape():
    """The GPU test's fixture: 133 chunks of 2^24 inputs covering [-104, 20];
    the first chunks (x in [-2^-103, -0]) all give orig = sqrtf(log1pf(1))."""
    g = golden("route_orig")
    chunk = 1 << int(g["chunk_log2"])
    total = int(g["n_neg"]) + int(g["n_pos"])
    assert len(g["s1"]) == -(-total // chunk)
    o = np.float32(np.sqrt(np.float32(np.log1p(1.0))))
    ob = int(o.view(np.int32))
    assert int(g["s1"][0]) == ob * chunk
    assert int(g["s2"][0]) == ob * sum(i & 63 for i in range(64)) * (chunk // 64)
