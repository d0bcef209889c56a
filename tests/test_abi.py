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
