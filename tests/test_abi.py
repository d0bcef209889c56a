# SPDX-License-Identifier: Apache-2.0
"""The C-ABI libraries load and export every entry point include/*.h
declares, and the reference-named mirror exports dsv4_mmq / dsv4_mmq_n /
dsv4_expert_forward. Without a GPU, dsv4_hip_init reports -1 with a reason
and the entry points refuse (return -1) instead of computing anything."""
import ctypes as C
import os
import re

import pytest

from conftest import ROOT, load_pkg


def _declared():
    names = set()
    for h in ("dsv4_hip.h", "dsv4_hip_aux.h"):
        src = open(os.path.join(ROOT, "include", h)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names |= set(re.findall(r"\b(dsv4_hip_\w+)\s*\(", src))
    return names


def test_header_matches_binding_list():
    pkg = load_pkg()
    assert _declared() == set(pkg.EXPORTS)


def test_library_exports_every_declared_symbol():
    pkg = load_pkg()
    lib = C.CDLL(pkg.HIP_SO)
    for name in _declared():
        assert hasattr(lib, name), name
    mirror = C.CDLL(pkg.AMD_SO)
    for name in pkg.MIRROR_EXPORTS:
        assert hasattr(mirror, name), name


def test_disable_switch_forces_cpu_path():
    """DSV4_HIP_DISABLE=1: dsv4_hip_init returns -1 with the reason, before
    any device is touched, so the caller keeps its CPU path (the reference's
    behaviour without a GPU backend, src/80_prefill/dsv4_prefill_vk.h:31-35);
    every entry point then refuses."""
    import subprocess
    import sys
    code = (
        "import sys, numpy as np; sys.path.insert(0, %r); from conftest import load_pkg; "
        "pkg = load_pkg(); L = pkg.Lib(); rc = L.init(0); err = L.error(); "
        "W = np.zeros(128 * 128, np.uint8); S = np.zeros(1, np.uint8); "
        "d = pkg.qmat(pkg.DSV4_WFP8, W.ctypes.data, S.ctypes.data, 128, 128, 128, 128); "
        "rc2 = L.mmq_n_rc(d, np.zeros(128, np.float32)); "
        "print(rc, rc2, err)" % os.path.join(ROOT, "tests"))
    env = dict(os.environ, DSV4_HIP_DISABLE="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    rc, rc2, err = r.stdout.strip().split(" ", 2)
    assert rc == "-1" and rc2 == "-1" and "DSV4_HIP_DISABLE" in err


def test_refuses_without_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the device paths are covered by the gpu tests")
    pkg = load_pkg()
    L = pkg.Lib()
    assert L.init(0) == -1
    assert L.error()
    import numpy as np
    W = np.zeros(128 * 128, np.uint8); S = np.zeros(1, np.uint8)
    d = pkg.qmat(pkg.DSV4_WFP8, W.ctypes.data, S.ctypes.data, 128, 128, 128, 128)
    assert L.mmq_n_rc(d, np.zeros(128, np.float32)) == -1
    assert "init" in L.error()
