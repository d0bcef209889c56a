# SPDX-License-Identifier: Apache-2.0
"""Shared fixtures. `gpu`-marked tests need a gfx950 device and the built
library; everything else runs on the CPU. The oracle (oracle/) is imported
here as the checker only."""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)

import pyoracle  # noqa: E402

PKG_DIR = os.path.join(ROOT, "deepseek-v4-in-c_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")

# numerical contract: relative L2 against the oracle
REL_L2_TOL = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


def load_pkg():
    """Import deepseek-v4-in-c_amd/ as module `dsv4_amd`."""
    if "dsv4_amd" in sys.modules:
        return sys.modules["dsv4_amd"]
    spec = importlib.util.spec_from_file_location(
        "dsv4_amd", os.path.join(PKG_DIR, "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["dsv4_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def oracle():
    return pyoracle.Oracle()


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def lib(pkg):
    """The HIP library, initialised on device 0. Fails (does not skip) when
    the device or the library is missing: a gpu test must run native code."""
    L = pkg.load()
    rc = L.init(0)
    if rc != 0:
        pytest.fail(f"dsv4_hip_init(0) failed: {L.error()}")
    return L


@pytest.fixture(autouse=True)
def _drop_registrations(request):
    """After each gpu test, unregister whatever host ranges it left
    registered (a failing test never reaches its own drop calls), so a later
    test's arrays never overlap a stale range."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    mod = sys.modules.get("dsv4_amd")
    if mod is not None and getattr(mod, "_LIB", None) is not None:
        mod._LIB.unregister_all()


def golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.sqrt(np.sum(want * want))
    return float(np.sqrt(np.sum((got - want) ** 2)) / (den if den > 0 else 1.0))


def max_abs(got, want):
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)
