# SPDX-License-Identifier: Apache-2.0
"""The reference's asymmetric SwiGLU clamp (src/10_compute/dsv4_ops.c:61-79:
up clamped to [-L, L], gate only from above, L <= 0 disables it; the gate
of tests/unit/test_ops.c:75-122) through every fused gate/up kernel, with
gate and up values far past the limit:

  one launch          k_moe_one (decode MoE, hidden 1024 / inter 512)
  two launches        k_gateup_px + k_down_px (DSV4_HIP_DECODE_LAUNCHES=2)
  one chunk per MFMA  k_gateup_mx (hidden 640; and the FP8 shared expert)
  VALU decode         k_gateup (inter 96, not whole 128-wide chunks)
  grouped, staged     k_grouped2 (<= 4096 pairs, hidden 512)
  grouped, direct     k_grouped (hidden 384, not a multiple of 256)
  grouped, prefill    k_grouped3 (> 4096 pairs)

Each at limit 10, limit 0 and limit -1 against the oracle (rel L2 1e-3)."""
import numpy as np
import pytest
import torch

import pyoracle as P
from conftest import REL_L2_TOL, max_abs, rel_l2
from test_gpu_decode import DEV, check_close, dev_f32
from test_gpu_moe_grouped import DevMat, table_of

pytestmark = pytest.mark.gpu

LIMITS = [10.0, 0.0, -1.0]


class BigExpert:
    """gate/up weights with sigma 25 / sqrt(hidden), so w1.x and w3.x have a
    standard deviation of 25 for N(0, 1) tokens; down weights N(0, 0.02)."""

    def __init__(self, lib, pkg, fmt, inter, hidden, gen):
        s = 25.0 / hidden ** 0.5
        self.m = [DevMat(lib, pkg, fmt, inter, hidden, gen, s), DevMat(lib, pkg, fmt, inter, hidden, gen, s),
                  DevMat(lib, pkg, fmt, hidden, inter, gen, 0.02)]
        self.desc = pkg.ExpertW(self.m[0].desc, self.m[1].desc, self.m[2].desc)
        self.he = P.HostExpert(self.m[0].hm, self.m[1].hm, self.m[2].hm)


def tokens(gen, n, hidden):
    return torch.randn(n, hidden, generator=gen).bfloat16().float().numpy()


def assert_past_limit(oracle, ex, x):
    g = oracle.mmq_n(ex.m[0].hm, np.ascontiguousarray(x[0]), 1)
    u = oracle.mmq_n(ex.m[1].hm, np.ascontiguousarray(x[0]), 1)
    assert g.max() > 40 and g.min() < -40 and np.abs(u).max() > 40


def want_tokens(oracle, experts, x, idx, w, limit, shared=None):
    out = []
    for t in range(x.shape[0]):
        acc = np.stack([oracle.expert_forward(experts[e].he, x[t], limit) for e in idx[t]])
        sh = oracle.expert_forward(shared.he, x[t], limit) if shared is not None else None
        out.append(oracle.moe_combine(acc, w[t], sh))
    return np.stack(out)


@pytest.mark.parametrize("path,hidden,inter", [("one", 1024, 512), ("two", 1024, 512),
                                               ("mx", 640, 256)])
@pytest.mark.parametrize("limit", LIMITS)
def test_decode_moe_clamp(lib, pkg, oracle, monkeypatch, path, hidden, inter, limit):
    gen = torch.Generator(device=DEV).manual_seed(hidden + inter)
    cg = torch.Generator().manual_seed(3)
    ne, topk = 5, 3
    experts = [BigExpert(lib, pkg, "fp4", inter, hidden, gen) for _ in range(ne)]
    x = tokens(cg, 1, hidden)
    assert_past_limit(oracle, experts[0], x)
    idx = np.array([[4, 0, 2]], np.int32)
    w = np.array([[0.5, 0.3, 0.2]], np.float32)
    monkeypatch.setenv("DSV4_HIP_DECODE_LAUNCHES", "2" if path == "two" else "1")
    tbl = table_of(experts)
    di, dw, dx = torch.from_numpy(idx[0]).to(DEV), dev_f32(w[0]), dev_f32(x[0])
    out = torch.empty(hidden, dtype=torch.float32, device=DEV)
    lib.moe_decode_dev(out.data_ptr(), dx.data_ptr(), tbl.data_ptr(), ne, di.data_ptr(), dw.data_ptr(),
                       topk, None, hidden, inter, limit)
    torch.cuda.synchronize()
    assert lib.status() == 0
    check_close(out.cpu().numpy(), want_tokens(oracle, experts, x, idx, w, limit)[0])


@pytest.mark.parametrize("fmt,hidden,inter", [("fp8", 1024, 512), ("fp4", 256, 96)])
@pytest.mark.parametrize("limit", LIMITS)
def test_expert_forward_clamp(lib, pkg, oracle, fmt, hidden, inter, limit):
    """FP8 (the shared expert's format, k_gateup_mx) and FP4 with inter 96
    (the VALU gate/up, k_gateup) through the host-pointer expert entry."""
    gen = torch.Generator(device=DEV).manual_seed(inter)
    ex = BigExpert(lib, pkg, fmt, inter, hidden, gen)
    x = tokens(torch.Generator().manual_seed(4), 1, hidden)
    assert_past_limit(oracle, ex, x)
    keep = []
    for m in ex.m:                         # host copies registered: the host entry point
        W, S = m.hm.W, m.hm.S
        lib.check(lib.register(W), "register")
        lib.check(lib.register(S), "register")
        keep += [W, S]
    d = pkg.ExpertW(*[pkg.qmat(m.hm.wdt, m.hm.W.ctypes.data, m.hm.S.ctypes.data, m.hm.rows, m.hm.cols,
                               m.hm.blk_r, m.hm.blk_c) for m in ex.m])
    check_close(lib.expert_forward(d, x[0], limit), oracle.expert_forward(ex.he, x[0], limit))
    for a in keep:
        lib.unregister(a)


@pytest.mark.parametrize("kind,n,topk,hidden,inter", [
    ("grouped2", 48, 6, 512, 256), ("grouped", 48, 6, 384, 256), ("grouped3", 1024, 6, 512, 256)])
@pytest.mark.parametrize("limit", LIMITS)
def test_grouped_clamp(lib, pkg, oracle, kind, n, topk, hidden, inter, limit):
    """The grouped MoE's three kernels (16-row staged, direct, 128-token
    prefill tiles), with an FP8 shared expert whose gate/up also pass the
    limit. Every checked token against the oracle."""
    gen = torch.Generator(device=DEV).manual_seed(n + hidden)
    ne = 8
    experts = [BigExpert(lib, pkg, "fp4", inter, hidden, gen) for _ in range(ne)]
    shared = BigExpert(lib, pkg, "fp8", inter, hidden, gen)
    x = tokens(torch.Generator().manual_seed(5), n, hidden)
    assert_past_limit(oracle, experts[1], x)
    rng = np.random.default_rng(n)
    idx = np.stack([rng.choice(ne, topk, replace=False) for _ in range(n)]).astype(np.int32)
    lg = rng.standard_normal((n, topk))
    w = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
    tbl = table_of(experts)
    dx = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    di, dw = torch.from_numpy(idx).to(DEV), torch.from_numpy(w).to(DEV)
    out = torch.empty((n, hidden), dtype=torch.float32, device=DEV)
    lib.moe_grouped_dev(out.data_ptr(), dx.data_ptr(), n, tbl.data_ptr(), ne, di.data_ptr(), dw.data_ptr(),
                        topk, shared.desc, hidden, inter, limit)
    torch.cuda.synchronize()
    assert lib.status() == 0
    got = out.cpu().numpy()
    sel = np.arange(n) if n <= 64 else np.random.default_rng(1).choice(n, 48, replace=False)
    want = want_tokens(oracle, experts, x[sel], idx[sel], w[sel], limit, shared)
    assert np.all(np.isfinite(got[sel]))
    for i, t in enumerate(sel):
        e = rel_l2(got[t], want[i])
        assert e <= REL_L2_TOL, f"token {t}: rel L2 {e:.3e} (max abs {max_abs(got[t], want[i]):.3e})"
