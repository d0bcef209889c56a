# SPDX-License-Identifier: Apache-2.0
"""GPU parity for the grouped MoE (dsv4_hip_moe_grouped / _dev): batched
decode and the prefill MoE layer.

The oracle is the reference's per-token path restated: expert_forward
(src/10_compute/dsv4_ops.c:85-93 over fp4_n / fp8_n) for each routed pair and
the shared expert, then the k-order combine
(src/80_prefill/dsv4_prefill_union_run.c:109-121). The reference's bucket
path is bitwise equal to it (tests/unit/test_matmul.c:690-792), so per-token
oracle outputs are the reference's prefill outputs. Tolerance: relative L2
1e-3 (the GPU rounds x and the SwiGLU output to fp16 on the way into the
MFMA)."""
import numpy as np
import pytest
import torch

import pyoracle as P
from conftest import REL_L2_TOL, bits, max_abs, rel_l2

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class DevMat:
    """A quantized matrix generated and quantized on the GPU, with host copies
    for the oracle."""

    def __init__(self, lib, pkg, fmt, rows, cols, gen, sigma=0.02):
        w = torch.randn(rows, cols, generator=gen, device=DEV) * sigma
        if fmt == "fp4":
            W = torch.empty(rows * cols // 2, dtype=torch.uint8, device=DEV)
            S = torch.empty(rows * cols // 32, dtype=torch.uint8, device=DEV)
            lib.quant_fp4_mx_dev(W.data_ptr(), S.data_ptr(), w.data_ptr(), rows, cols)
            wdt, br, bc = pkg.DSV4_WFP4, 1, 32
        else:
            W = torch.empty(rows * cols, dtype=torch.uint8, device=DEV)
            S = torch.empty(((rows + 127) // 128) * ((cols + 127) // 128), dtype=torch.float32, device=DEV)
            lib.quant_fp8_blk128_dev(W.data_ptr(), S.data_ptr(), w.data_ptr(), rows, cols)
            wdt, br, bc = pkg.DSV4_WFP8_F32S, 128, 128
            if fmt == "fp8e8m0":   # power-of-two scales at or above the fp32 ones
                S = torch.clamp(torch.ceil(torch.log2(S)) + 127, 0, 254).to(torch.uint8)
                wdt = pkg.DSV4_WFP8
        torch.cuda.synchronize()
        self.W, self.S = W, S
        self.desc = pkg.qmat(wdt, W.data_ptr(), S.data_ptr(), rows, cols, br, bc)
        self.hm = P.HostMat(wdt, W.cpu().numpy(), S.cpu().numpy(), rows, cols, br, bc)


class DevExpert:
    def __init__(self, lib, pkg, fmt, inter, hidden, gen):
        self.m = [DevMat(lib, pkg, fmt, inter, hidden, gen), DevMat(lib, pkg, fmt, inter, hidden, gen),
                  DevMat(lib, pkg, fmt, hidden, inter, gen)]
        self.desc = pkg.ExpertW(self.m[0].desc, self.m[1].desc, self.m[2].desc)
        self.he = P.HostExpert(self.m[0].hm, self.m[1].hm, self.m[2].hm)


def table_of(experts):
    raw = b"".join(bytes(e.desc) for e in experts)
    return torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(DEV)


def routing(rng, n, topk, ne, zipf=None):
    idx = np.empty((n, topk), np.int32)
    p = None
    if zipf:
        p = 1.0 / np.arange(1, ne + 1) ** zipf
        p /= p.sum()
    for t in range(n):
        idx[t] = rng.choice(ne, topk, replace=False, p=p)
    logits = rng.standard_normal((n, topk))
    w = (np.exp(logits) / np.exp(logits).sum(1, keepdims=True)).astype(np.float32)
    return idx, w


def oracle_tokens(oracle, experts, shared, x, idx, w, tokens, limit=10.0):
    out = []
    for t in tokens:
        acc = np.stack([oracle.expert_forward(experts[e].he, x[t], limit) for e in idx[t]])
        sh = oracle.expert_forward(shared.he, x[t], limit) if shared is not None else None
        out.append(oracle.moe_combine(acc, w[t], sh))
    return np.stack(out)


def run_dev(lib, experts, shared, x, idx, w, hidden, inter, limit=10.0):
    n, topk = idx.shape
    tbl = table_of(experts)
    dx = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV)
    di = torch.from_numpy(idx).to(DEV)
    dw = torch.from_numpy(w).to(DEV)
    out = torch.empty((n, hidden), dtype=torch.float32, device=DEV)
    lib.moe_grouped_dev(out.data_ptr(), dx.data_ptr(), n, tbl.data_ptr(), len(experts), di.data_ptr(),
                        dw.data_ptr(), topk, shared.desc if shared is not None else None, hidden, inter,
                        limit)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def bf16_rows(gen, n, hidden):
    return torch.randn(n, hidden, generator=gen).bfloat16().float().numpy()


@pytest.mark.parametrize("n,topk,ne,shared_fmt", [
    (20, 4, 12, "fp8f32"),      # 16-row tiles, FP8 shared with fp32 block scales
    (7, 6, 16, "fp8e8m0"),      # FP8 shared with E8M0 scales, ragged buckets
    (1100, 4, 8, "fp4"),        # 128-row tiles (more than 4096 pairs), FP4 shared
    (33, 3, 5, None),           # no shared expert
])
def test_grouped_small_shapes(lib, pkg, oracle, n, topk, ne, shared_fmt):
    gen = torch.Generator().manual_seed(n * 7 + ne)
    dgen = torch.Generator(device=DEV).manual_seed(n * 7 + ne)
    rng = np.random.default_rng(n + topk)
    hidden, inter = (256, 128) if n > 500 else (512, 256)
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    shared = DevExpert(lib, pkg, shared_fmt, inter, hidden, dgen) if shared_fmt else None
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne)
    got = run_dev(lib, experts, shared, x, idx, w, hidden, inter)
    tokens = range(n) if n <= 64 else rng.choice(n, 48, replace=False)
    want = oracle_tokens(oracle, experts, shared, x, idx, w, tokens)
    got = got[list(tokens)]
    assert lib.status() == 0
    assert np.all(np.isfinite(got))
    e = rel_l2(got, want)
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e} (max abs {max_abs(got, want):.3e})"


@pytest.mark.parametrize("n,topk,ne,zipf,hidden,inter", [
    (1500, 6, 40, 1.2, 512, 256),   # 128-row tiles: skewed buckets, partial and empty tiles
    (700, 8, 9, None, 768, 384),    # 3 down slabs, K = 384 (3 stages)
    (4100, 1, 3, None, 256, 128),   # single stage (K = 128) down, many full tiles
])
def test_grouped_prefill_tiles(lib, pkg, oracle, n, topk, ne, zipf, hidden, inter):
    """More than 4096 pairs: 128-row tiles, gate/up 128 features and down 256
    features per workgroup; bucket sizes cover every count of live 16-row
    tiles per wave (0..4)."""
    gen = torch.Generator().manual_seed(n + ne)
    dgen = torch.Generator(device=DEV).manual_seed(n + ne)
    rng = np.random.default_rng(n * 3 + topk)
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    shared = DevExpert(lib, pkg, "fp8f32", inter, hidden, dgen)
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne, zipf)
    got = run_dev(lib, experts, shared, x, idx, w, hidden, inter)
    counts = np.bincount(idx.ravel(), minlength=ne)
    assert (counts % 128 > 0).sum() >= 2            # partial tiles exist
    # tokens of the smallest and largest buckets plus a random sample
    small = np.nonzero((idx == np.argmin(np.where(counts > 0, counts, 1 << 30))).any(1))[0][:8]
    big = np.nonzero((idx == np.argmax(counts)).any(1))[0][-8:]
    tokens = np.unique(np.concatenate([small, big, rng.choice(n, 32, replace=False)]))
    want = oracle_tokens(oracle, experts, shared, x, idx, w, tokens)
    got = got[tokens]
    assert lib.status() == 0
    assert np.all(np.isfinite(got))
    e = rel_l2(got, want)
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e} (max abs {max_abs(got, want):.3e})"


def test_grouped_host_entry_point(lib, pkg, oracle):
    """dsv4_hip_moe_grouped with host descriptors inside registered ranges."""
    gen = torch.Generator().manual_seed(5)
    rng = np.random.default_rng(5)
    hidden, inter, ne, n, topk = 256, 128, 6, 10, 3
    host = []
    for _ in range(ne + 1):
        mats = []
        fmt = "fp4" if len(host) < ne else "fp8"
        for (r, c) in ((inter, hidden), (inter, hidden), (hidden, inter)):
            wf = (torch.randn(r, c, generator=gen) * 0.02).numpy()
            if fmt == "fp4":
                W, S = oracle.quant_fp4_mx(wf)
                args = (pkg.DSV4_WFP4, W, S, r, c, 1, 32)
            else:
                W, S = oracle.quant_fp8_blk128(wf)
                args = (pkg.DSV4_WFP8_F32S, W, S, r, c, 128, 128)
            W = np.ascontiguousarray(args[1]); S = np.ascontiguousarray(args[2])
            lib.check(lib.register(W), "register"); lib.check(lib.register(S), "register")
            mats.append((W, S, pkg.qmat(args[0], W.ctypes.data, S.ctypes.data, r, c, args[5], args[6]),
                         P.HostMat(args[0], W, S, r, c, args[5], args[6])))
        host.append(mats)
    descs = [pkg.ExpertW(m[0][2], m[1][2], m[2][2]) for m in host]
    hes = [P.HostExpert(m[0][3], m[1][3], m[2][3]) for m in host]
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne)
    got = lib.moe_grouped(descs[:ne], idx, w, x, descs[ne], 10.0)
    want = []
    for t in range(n):
        acc = np.stack([oracle.expert_forward(hes[e], x[t], 10.0) for e in idx[t]])
        want.append(oracle.moe_combine(acc, w[t], oracle.expert_forward(hes[ne], x[t], 10.0)))
    e = rel_l2(got, np.stack(want))
    for mats in host:
        for W, S, _, _ in mats:
            lib.unregister(W); lib.unregister(S)
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e}"


def test_grouped_deterministic_and_order_free(lib, pkg, oracle):
    """Two calls agree bit for bit, and a token's output does not depend on
    where its rows land in the expert buckets (token order permuted)."""
    gen = torch.Generator().manual_seed(9)
    dgen = torch.Generator(device=DEV).manual_seed(9)
    rng = np.random.default_rng(9)
    hidden, inter, ne, n, topk = 256, 128, 6, 40, 3
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne)
    a = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    b = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    assert np.array_equal(bits(a), bits(b))
    perm = rng.permutation(n)
    c = run_dev(lib, experts, None, x[perm], idx[perm], w[perm], hidden, inter)
    assert np.array_equal(bits(c), bits(a[perm]))


def test_grouped_bad_id_flags_status(lib, pkg, oracle):
    gen = torch.Generator().manual_seed(11)
    dgen = torch.Generator(device=DEV).manual_seed(11)
    rng = np.random.default_rng(11)
    hidden, inter, ne, n, topk = 256, 128, 4, 6, 2
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne)
    lib.status()
    idx[2, 1] = 99
    got = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    assert lib.status() & 1
    assert np.isnan(got[2]).all()
    ok = [t for t in range(n) if t != 2]
    assert np.all(np.isfinite(got[ok]))
    want = oracle_tokens(oracle, experts, None, x, idx, w, ok)
    assert rel_l2(got[ok], want) <= REL_L2_TOL


def test_grouped_scale_range_flag(lib, pkg, oracle):
    """An FP4 scale byte outside 104..140 cannot be decoded exactly into fp16:
    the call raises status bit 2."""
    gen = torch.Generator().manual_seed(13)
    dgen = torch.Generator(device=DEV).manual_seed(13)
    rng = np.random.default_rng(13)
    hidden, inter, ne, n, topk = 256, 128, 2, 4, 1
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne)
    lib.status()
    run_dev(lib, experts, None, x, idx, w, hidden, inter)
    assert lib.status() == 0
    experts[0].m[0].S[5] = 150
    experts[1].m[0].S[5] = 150
    torch.cuda.synchronize()
    run_dev(lib, experts, None, x, idx, w, hidden, inter)
    assert lib.status() & 4


def test_grouped_config2_shape_sampled(lib, pkg, oracle):
    """64 tokens, top-6 of 32 real-size FP4 experts (2048 x 4096) under Zipf
    routing, FP8 shared expert with fp32 scales; 4 tokens checked against the
    oracle."""
    gen = torch.Generator().manual_seed(2)
    dgen = torch.Generator(device=DEV).manual_seed(2)
    rng = np.random.default_rng(2)
    hidden, inter, ne, n, topk = 4096, 2048, 32, 64, 6
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    shared = DevExpert(lib, pkg, "fp8f32", inter, hidden, dgen)
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne, zipf=1.1)
    got = run_dev(lib, experts, shared, x, idx, w, hidden, inter)
    assert lib.status() == 0
    tokens = [0, 17, 40, 63]
    want = oracle_tokens(oracle, experts, shared, x, idx, w, tokens)
    e = rel_l2(got[tokens], want)
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e} (max abs {max_abs(got[tokens], want):.3e})"


@pytest.mark.parametrize("n,topk,ne,zipf,hidden,inter", [
    (60, 4, 5, None, 1024, 512),     # buckets of ~48 rows: several token tiles each
    (64, 8, 8, None, 512, 256),      # 64-row buckets: whole tiles
    (3, 2, 40, None, 2048, 1024),    # one-row buckets, most experts idle
    (50, 6, 24, 1.1, 4096, 2048),    # config-2 geometry, skewed buckets
])
def test_grouped_bucket_shapes(lib, pkg, oracle, n, topk, ne, zipf, hidden, inter):
    """Buckets spanning several token tiles, full tiles, one-row buckets with
    most experts idle, and the real expert geometry under skewed routing:
    against the per-token oracle, and bit-identical across two calls."""
    gen = torch.Generator().manual_seed(n * 13 + ne)
    dgen = torch.Generator(device=DEV).manual_seed(n * 13 + ne)
    rng = np.random.default_rng(n * 5 + topk)
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne, zipf=zipf)
    lib.status()
    got = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    again = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    assert lib.status() == 0
    assert np.array_equal(bits(got), bits(again))
    tokens = list(range(n)) if n <= 8 else sorted(rng.choice(n, 8, replace=False).tolist())
    want = oracle_tokens(oracle, experts, None, x, idx, w, tokens)
    e = rel_l2(got[tokens], want)
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e} (max abs {max_abs(got[tokens], want):.3e})"


def test_grouped_tile_fill_levels(lib, pkg, oracle):
    """Buckets of 4, 5, 1, 16, 17 (a full 16-token tile and a one-token
    tile), 3, 0 and 2 tokens: every token checked against the oracle, and two
    calls bit-identical."""
    counts = [4, 5, 1, 16, 17, 3, 0, 2]
    ne, hidden, inter = len(counts), 512, 256
    gen = torch.Generator().manual_seed(4516)
    dgen = torch.Generator(device=DEV).manual_seed(4516)
    rng = np.random.default_rng(4516)
    ids = np.concatenate([np.full(c, e, np.int32) for e, c in enumerate(counts)])
    rng.shuffle(ids)
    n = len(ids)
    idx = ids.reshape(n, 1)
    w = np.ones((n, 1), np.float32)
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    x = bf16_rows(gen, n, hidden)
    lib.status()
    got = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    again = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    assert lib.status() == 0
    assert np.array_equal(bits(got), bits(again))
    want = oracle_tokens(oracle, experts, None, x, idx, w, list(range(n)))
    e = rel_l2(got, want)
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e} (max abs {max_abs(got, want):.3e})"


def test_grouped_bad_id_real_width(lib, pkg, oracle):
    """A routing id out of range at hidden 512 (whole 256-wide K stages):
    status bit 0, that token NaN, the others exact."""
    gen = torch.Generator().manual_seed(21)
    dgen = torch.Generator(device=DEV).manual_seed(21)
    rng = np.random.default_rng(21)
    hidden, inter, ne, n, topk = 512, 256, 4, 6, 2
    experts = [DevExpert(lib, pkg, "fp4", inter, hidden, dgen) for _ in range(ne)]
    x = bf16_rows(gen, n, hidden)
    idx, w = routing(rng, n, topk, ne)
    lib.status()
    idx[4, 0] = -3
    got = run_dev(lib, experts, None, x, idx, w, hidden, inter)
    assert lib.status() & 1
    assert np.isnan(got[4]).all()
    ok = [t for t in range(n) if t != 4]
    want = oracle_tokens(oracle, experts, None, x, idx, w, ok)
    assert rel_l2(got[ok], want) <= REL_L2_TOL


def _arena_host_expert(bench, arena, e):
    """Host copy of expert e of the benchmark's arena (cache-slot layout:
    s1, s2, s3, w1, w2, w3) as an oracle expert."""
    raw = arena.host_copy(torch, int(e))
    H, I = bench.HIDDEN, bench.INTER
    wb = [I * H // 2, H * I // 2, I * H // 2]
    sb = [I * H // 32, H * I // 32, I * H // 32]
    off_s = [0, sb[0], sb[0] + sb[1]]
    off_w = [sum(sb), sum(sb) + wb[0], sum(sb) + wb[0] + wb[1]]
    shapes = [(I, H), (H, I), (I, H)]
    mats = [P.HostMat(P.DSV4_WFP4, raw[off_w[i]:off_w[i] + wb[i]], raw[off_s[i]:off_s[i] + sb[i]],
                      r, c, 1, 32) for i, (r, c) in enumerate(shapes)]
    return P.HostExpert(mats[0], mats[2], mats[1]), raw


def test_grouped_config4_full_workload_sampled(lib, pkg, oracle):
    """The prefill MoE layer at its full workload, generated exactly as the
    benchmark generates it: 4096 tokens, top-6 of 256 FP4 experts
    (2048 x 4096 / 4096 x 2048) under Zipf(1.1), FP8 shared expert with fp32
    128x128 scales. This runs the 128-token-tile kernels at their real K-loop
    depth and tile counts. Every output row finite; the tokens of the
    smallest bucket, 8 tokens of the largest and 32 random tokens within
    1e-3 of the per-token oracle."""
    import bench
    seed = 0xD5EED004
    n, H, I, topk = 4096, bench.HIDDEN, bench.INTER, bench.TOPK
    arena = bench.ExpertArena(torch, pkg, lib, bench.N_EXPERTS, seed=seed)
    shared, keep = bench.make_shared_fp8(torch, pkg, lib, seed * 7)
    idx, w = bench.zipf_routing(n, seed)
    xs = torch.empty(n * H, dtype=torch.float32, device=DEV)
    lib.synth_normal_dev(xs.data_ptr(), xs.numel(), seed ^ 0x55, 1.0, True)
    di, dw = torch.from_numpy(idx).to(DEV), torch.from_numpy(w).to(DEV)
    out = torch.empty((n, H), dtype=torch.float32, device=DEV)
    lib.status()
    lib.moe_grouped_dev(out.data_ptr(), xs.data_ptr(), n, arena.table.data_ptr(), bench.N_EXPERTS,
                        di.data_ptr(), dw.data_ptr(), topk, shared, H, I, 10.0)
    torch.cuda.synchronize()
    assert lib.status() == 0
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    counts = np.bincount(idx.reshape(-1), minlength=bench.N_EXPERTS)
    used = np.nonzero(counts)[0]
    e_small, e_big = used[np.argmin(counts[used])], int(np.argmax(counts))
    assert counts[e_big] > 1000            # the 128-token tiles run many tiles of one expert
    rng = np.random.default_rng(4)
    toks_small = np.nonzero((idx == e_small).any(1))[0]
    toks_big = rng.choice(np.nonzero((idx == e_big).any(1))[0], 8, replace=False)
    sel = sorted(set(toks_small.tolist()) | set(toks_big.tolist()) |
                 set(rng.choice(n, 32, replace=False).tolist()))
    host = {}
    for e in np.unique(idx[sel]):
        host[int(e)] = _arena_host_expert(bench, arena, e)
    hm = []
    for i, (r, c) in enumerate(((I, H), (I, H), (H, I))):
        hm.append(P.HostMat(P.DSV4_WFP8_F32S, keep[2 * i].cpu().numpy(), keep[2 * i + 1].cpu().numpy(),
                            r, c, 128, 128))
    hshared = P.HostExpert(hm[0], hm[1], hm[2])
    x = xs.view(n, H)[torch.tensor(sel, device=DEV)].cpu().numpy()
    for j, t in enumerate(sel):
        acc = np.stack([oracle.expert_forward(host[int(e)][0], x[j], 10.0) for e in idx[t]])
        want = oracle.moe_combine(acc, w[t], oracle.expert_forward(hshared, x[j], 10.0))
        e = rel_l2(got[t], want)
        assert e <= REL_L2_TOL, f"token {t}: rel L2 {e:.3e} (max abs {max_abs(got[t], want):.3e})"
    _torch_all_tokens_exact(lib, arena, keep, xs.view(n, H), idx, w, got, n, H, I, topk, 10.0)


def _torch_swiglu(g, u, limit):
    """src/10_compute/dsv4_ops.c:61-79 in torch (limit > 0)"""
    u = torch.clamp(u, -limit, limit)
    g = torch.clamp(g, max=limit)
    return (g / (1.0 + torch.exp(-g))) * u


def _torch_all_tokens_exact(lib, arena, keep, x, idx, w, got, n, H, I, topk, limit):
    """Every one of the call's tokens against the unquantized computation in
    float32 torch on the device (TF32 off): each routed expert's weights
    dequantized exactly (dsv4_hip_dequant_dev), SwiGLU, w2, the FP8 shared
    expert on fp32 x with its 128 x 128 scales, the k-order combine; every
    token within 1e-3 (the exact path's contract: only x's and mid's fp16
    rounding, 2^-11 relative, separate the two)."""
    flat = idx.reshape(-1)
    wtmp = torch.empty(H * I, dtype=torch.float32, device=DEV)
    Y = torch.zeros((n * topk, H), dtype=torch.float32, device=DEV)

    def fp8_mat(W, S, r, c):
        return W.view(torch.float8_e4m3fn).float().reshape(r, c) * \
            S.reshape(r // 128, c // 128).repeat_interleave(128, 0).repeat_interleave(128, 1)

    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        for e in np.unique(flat):
            pairs = torch.from_numpy(np.nonzero(flat == e)[0]).to(DEV)
            xe = x[pairs // topk]
            d = arena.descs[int(e)]
            lib.dequant_dev(wtmp.data_ptr(), d.w1)
            g = torch.mm(xe, wtmp.view(I, H).t())
            lib.dequant_dev(wtmp.data_ptr(), d.w3)
            u = torch.mm(xe, wtmp.view(I, H).t())
            lib.dequant_dev(wtmp.data_ptr(), d.w2)
            Y[pairs] = torch.mm(_torch_swiglu(g, u, limit), wtmp.view(H, I).t())
        sg = torch.mm(x, fp8_mat(keep[0], keep[1], I, H).t().contiguous())
        su = torch.mm(x, fp8_mat(keep[2], keep[3], I, H).t().contiguous())
        ys = torch.mm(_torch_swiglu(sg, su, limit), fp8_mat(keep[4], keep[5], H, I).t().contiguous())
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    wd = torch.from_numpy(w).to(DEV)
    out = torch.zeros((n, H), dtype=torch.float32, device=DEV)
    Yk = Y.view(n, topk, H)
    for k in range(topk):
        out = out + wd[:, k:k + 1] * Yk[:, k]
    ref = (out + ys).cpu().numpy().astype(np.float64)
    num = np.sqrt(np.sum((got.astype(np.float64) - ref) ** 2, axis=1))
    den = np.sqrt(np.sum(ref ** 2, axis=1))
    r = num / den
    assert np.all(r <= REL_L2_TOL), f"{int(np.sum(r > REL_L2_TOL))} tokens beyond 1e-3, worst {float(r.max()):.3e}"
