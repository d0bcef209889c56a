# SPDX-License-Identifier: Apache-2.0
"""The allocation-free decode MoE entry point
(dsv4_hip_moe_decode_routed_noalloc_dev) against the entry point it is a
variant of (dsv4_hip_moe_decode_routed_dev): bit-identical outputs on two
calls in a row, the second with a smaller input; no allocation by the
library and the device's free memory unchanged across its calls; a call
beyond the scratch limits returns -1 with the reason."""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import bits
from test_gpu_decode import DEV, bf16_x, dev_f32
from test_gpu_decode_mx import _device_fp4_experts
from test_gpu_decode_one import _device_fp8_shared

pytestmark = pytest.mark.gpu


class _Case:
    def __init__(self, pkg, oracle, seed, inter, hidden, topk, n_exp, shared):
        rng = np.random.default_rng(seed)
        self.inter, self.hidden, self.topk = inter, hidden, topk
        self.descs, _, self.keep = _device_fp4_experts(pkg, oracle, rng, n_exp, inter, hidden)
        self.arr = (pkg.ExpertW * n_exp)(*self.descs)
        self.shared = None
        if shared:
            self.shared, _, k2 = _device_fp8_shared(pkg, oracle, rng, inter, hidden)
            self.keep += k2
        self.idx = rng.choice(n_exp, topk, replace=False).astype(np.int32)
        lg = rng.standard_normal(topk)
        self.w = (np.exp(lg) / np.exp(lg).sum()).astype(np.float32)
        self.x = dev_f32(bf16_x(seed, hidden))
        self.out_ref = torch.empty(hidden, dtype=torch.float32, device=DEV)
        self.out = torch.full((hidden,), float("nan"), dtype=torch.float32, device=DEV)

    def reference(self, lib):
        lib.moe_decode_routed_dev(self.out_ref.data_ptr(), self.x.data_ptr(), self.arr, self.idx, self.w,
                                  self.topk, self.shared, self.hidden, self.inter, 10.0)

    def noalloc_rc(self, lib):
        return lib.moe_decode_routed_noalloc_dev_rc(self.out.data_ptr(), self.x.data_ptr(), self.arr,
                                                    self.idx, self.w, self.topk, self.shared,
                                                    self.hidden, self.inter, 10.0)


def test_noalloc_matches_allocating_entry(lib, pkg, oracle):
    """After a fresh dsv4_hip_init (empty workspaces, scratch address looked
    up again): the allocation-free calls first, at the scratch's maxima
    (topk 8, inter 2048, hidden 4096, shared expert) and then a smaller
    call, with no hipMalloc of the library (its allocation counter) and no
    change of the device's free memory; then the allocating entry point on the
    same inputs, which does allocate its workspaces (the counter's positive
    control), and bit-identical outputs."""
    big = _Case(pkg, oracle, 701, 2048, 4096, 8, 8, True)
    small = _Case(pkg, oracle, 702, 512, 1024, 3, 5, False)
    torch.cuda.synchronize()
    lib.shutdown()
    assert lib.init(0) == 0, lib.error()
    lib.status()
    n0 = lib.alloc_count()
    free0 = torch.cuda.mem_get_info()[0]
    for c in (big, small):
        assert c.noalloc_rc(lib) == 0, lib.error()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert lib.alloc_count() == n0, "the allocation-free entry point allocated"
    assert free1 == free0, f"free device memory changed by {free0 - free1} bytes"
    assert lib.status() == 0
    for c in (big, small):
        c.reference(lib)
    torch.cuda.synchronize()
    assert lib.alloc_count() > n0, "the allocating entry point did not count its workspaces"
    assert lib.status() == 0
    for c in (big, small):
        got = c.out.cpu().numpy()
        assert np.isfinite(got).all()
        assert np.array_equal(bits(got), bits(c.out_ref.cpu().numpy()))


def test_noalloc_rejects_beyond_scratch(lib, pkg, oracle):
    c = _Case(pkg, oracle, 703, 4096, 128, 2, 3, False)
    assert c.noalloc_rc(lib) == -1
    assert "scratch" in lib.error() and "2048" in lib.error()
