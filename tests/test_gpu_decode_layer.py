# SPDX-License-Identifier: Apache-2.0
"""One decode layer's matrix chain on the device (bench.DecodeLayer: the
dsv4_mmq calls of src/70_decode/dsv4_layer_attn.c:21-106 and
dsv4_layer.c:52-116 at DeepSeek-V4-Flash shapes -- wq_a, wq_b, wkv, the
compressor's and the indexer's matrices, the eight wo_a group slices, wo_b --
then the MoE block with its BF16 gate, router, routed FP4 experts and FP8
shared expert), every launch on one stream with no host round trip.

Eager: every matrix's output against the oracle on the device's own input
(FP8 within 1e-3 relative L2; BF16 bit for bit, bf16_n's fp64 order), the
router's picks and weights bit for bit as dsv4_route gives them on the
oracle's gate scores, and the block's output within 1e-3 of the oracle's
experts combined in k order plus the shared expert. Then the whole chain
captured once in a HIP graph and replayed for three tokens, twice over (x
copied in between, synchronised): every output of every replay bit for bit
the eager call's for the same token."""
import numpy as np
import pytest
import torch

import pyoracle as P
from conftest import bits
from test_gpu_contract import check_bf16
from test_gpu_decode import DEV, bf16_x, check_close, dev_f32
from test_gpu_decode_one import _host_slot_expert

pytestmark = pytest.mark.gpu

OUTS = ("qr", "q", "kv", "comp_kv", "comp_sc", "idx_q", "idx_w", "ogrp", "attn", "moe")


def _host_mats(L):
    import bench
    hm = {}
    for name, r, c, _ in bench.DecodeLayer.FP8 + (("wo_a", 8192, 4096, None), ("wo_b", 4096, 8192, None)):
        W, S = L.keep[name]
        hm[name] = P.HostMat(P.DSV4_WFP8, W.cpu().numpy(), S.cpu().numpy(), r, c, 128, 128)
    for name, r, c in bench.DecodeLayer.BF16:
        W, _ = L.keep[name]
        hm[name] = (W.view(torch.int16).cpu().numpy().view(np.uint16).copy(), r, c)
    W, S = (a.cpu().numpy() for a in L.keep["wo_a"])
    hm["slices"] = [P.HostMat(P.DSV4_WFP8, W[g * 1024 * 4096:(g + 1) * 1024 * 4096],
                              S[g * 256:(g + 1) * 256], 1024, 4096, 128, 128) for g in range(8)]
    sk = L.skeep
    hm["shared"] = P.HostExpert(*[P.HostMat(P.DSV4_WFP8_F32S, sk[2 * i].cpu().numpy(), sk[2 * i + 1].cpu().numpy(),
                                            r, c, 128, 128)
                                  for i, (r, c) in enumerate(((2048, 4096), (2048, 4096), (4096, 2048)))])
    return hm


def _snapshot(L):
    torch.cuda.synchronize()
    d = {k: L.out[k].cpu().numpy().copy() for k in OUTS}
    d["idx"] = L.idx.cpu().numpy().copy()
    d["w"] = L.w.cpu().numpy().copy()
    return d


def _check_against_oracle(oracle, L, hm, xh, got):
    f8 = lambda name, x: check_close(got[name[0]], oracle.mmq_n(hm[name[1]], np.ascontiguousarray(x, np.float32)))
    bf = lambda out, name, x: check_bf16(got[out], oracle.bf16_n(hm[name][0], np.ascontiguousarray(x, np.float32),
                                                                 hm[name][1], hm[name][2]))
    f8(("qr", "wq_a"), xh)
    f8(("q", "wq_b"), got["qr"])
    f8(("kv", "wkv"), xh)
    bf("comp_kv", "comp_wkv", xh)
    bf("comp_sc", "comp_wgate", xh)
    f8(("idx_q", "idx_wq_b"), got["qr"])
    bf("idx_w", "idx_wproj", xh)
    for g in range(8):
        check_close(got["ogrp"][g * 1024:(g + 1) * 1024],
                    oracle.mmq_n(hm["slices"][g], np.ascontiguousarray(got["q"][g * 4096:(g + 1) * 4096])))
    f8(("attn", "wo_b"), got["ogrp"])
    # the MoE block on the device's attention output
    a = got["attn"]
    W16, ne, hid = hm["gate"]
    sc = oracle.bf16_n(W16, a, ne, hid)
    wi, ww, _ = oracle.route(sc, 6, 2.5, bias=L.bias.cpu().numpy())
    assert np.array_equal(got["idx"], wi), f"picks {got['idx']} vs {wi}"
    assert np.array_equal(bits(got["w"]), bits(ww)), "routing weights"
    acc = np.stack([oracle.expert_forward(_host_slot_expert(L.arena.host_copy(torch, int(e))), a, 10.0)
                    for e in wi])
    want = (oracle.moe_combine(acc, ww) + oracle.expert_forward(hm["shared"], a, 10.0)).astype(np.float32)
    check_close(got["moe"], want)


def test_decode_layer_chain_eager_and_graph(lib, pkg, oracle):
    import bench
    arena = bench.ExpertArena(torch, pkg, lib, 256, seed=0x1A7E)
    L = bench.DecodeLayer(torch, pkg, lib, arena, 0x5EED)
    hm = _host_mats(L)
    xs = [bf16_x(900 + i, 4096) for i in range(3)]
    x = dev_f32(xs[0])
    st = torch.cuda.Stream()
    lib.status()
    eager = []
    for i, xh in enumerate(xs):
        x.copy_(torch.from_numpy(xh))
        torch.cuda.synchronize()
        L.run(lib, x.data_ptr(), st.cuda_stream)
        got = _snapshot(L)
        assert lib.status() == 0
        if i < 2:
            _check_against_oracle(oracle, L, hm, xh, got)
        eager.append(got)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        L.run(lib, x.data_ptr(), st.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(2):
        for i, xh in enumerate(xs):
            x.copy_(torch.from_numpy(xh))
            torch.cuda.synchronize()
            graph.replay()
            got = _snapshot(L)
            for k in OUTS + ("w",):
                assert np.array_equal(bits(got[k]), bits(eager[i][k])), f"replay {rep} token {i}: {k}"
            assert np.array_equal(got["idx"], eager[i]["idx"])
    assert lib.status() == 0


def test_bf16_head_full_vocabulary(lib, pkg, oracle):
    """The output head (src/70_decode/dsv4_decode.c:145): BF16 [129280 x
    4096] through dsv4_hip_mmq_n_dev, bit for bit bf16_n."""
    rows, cols = 129280, 4096
    g = torch.Generator(device=DEV).manual_seed(129280)
    W = (torch.randn(rows * cols, generator=g, device=DEV) * 0.02).bfloat16()
    xh = bf16_x(4096, cols)
    x = dev_f32(xh)
    y = torch.empty(rows, dtype=torch.float32, device=DEV)
    m = pkg.qmat(pkg.DSV4_WBF16, W.data_ptr(), None, rows, cols, 0, 0)
    lib.status()
    lib.mmq_n_dev(y.data_ptr(), x.data_ptr(), m, 1)
    torch.cuda.synchronize()
    assert lib.status() == 0
    W16 = W.view(torch.int16).cpu().numpy().view(np.uint16)
    check_bf16(y.cpu().numpy(), oracle.bf16_n(W16, xh, rows, cols))


def test_multi_job_seam_matches_single_calls(lib, pkg, oracle):
    """dsv4_hip_mmq_multi_dev (dsv4_prefill_pm_multi's jobs on the device):
    the eight wo_a slices of one [8192 x 4096] E8M0 arena in one launch, next
    to a 4096-row job, a BF16 job, a three-token FP8 job and an empty one --
    every output bit for bit its single dsv4_hip_mmq_n_dev call's, the
    slices within 1e-3 of the oracle; a refused job (n < 0) returns -1 and
    writes nothing."""
    import bench
    arena = bench.ExpertArena(torch, pkg, lib, 8, seed=0x3A7E)
    L = bench.DecodeLayer(torch, pkg, lib, arena, 0x3ADE)
    hm = _host_mats(L)
    g = torch.Generator(device=DEV).manual_seed(77)
    o = torch.randn(32768, generator=g, device=DEV).bfloat16().float()
    x = torch.randn(4096 * 3, generator=g, device=DEV).bfloat16().float()
    outs = [torch.full((1024,), float("nan"), device=DEV) for _ in range(8)]
    y_b = torch.full((4096,), float("nan"), device=DEV)
    y_bf = torch.full((1024,), float("nan"), device=DEV)
    y_3 = torch.full((3 * 1024,), float("nan"), device=DEV)
    jobs = [(L.slices[gi], o.data_ptr() + 4 * 4096 * gi, outs[gi].data_ptr(), 1) for gi in range(8)]
    shared_w2 = L.shared.w2                                            # FP8 [4096 x 2048], fp32 scales
    x2 = torch.randn(2048, generator=g, device=DEV)
    jobs += [(shared_w2, x2.data_ptr(), y_b.data_ptr(), 1),
             (L.desc["comp_wkv"], x.data_ptr(), y_bf.data_ptr(), 1),
             (L.desc["wq_a"], x.data_ptr(), y_3.data_ptr(), 3),
             (L.desc["wkv"], x.data_ptr(), y_b.data_ptr(), 0)]
    lib.status()
    lib.mmq_multi_dev(jobs)
    torch.cuda.synchronize()
    assert lib.status() == 0
    got = [t.cpu().numpy().copy() for t in outs + [y_b, y_bf, y_3]]
    for (d, xp, yp, n), want_t in zip(jobs[:-1], got):
        single = torch.full((want_t.size,), float("nan"), device=DEV)
        lib.mmq_n_dev(single.data_ptr(), xp, d, n)
        torch.cuda.synchronize()
        assert np.array_equal(bits(single.cpu().numpy()), bits(want_t))
    oh = o.cpu().numpy()
    for gi in range(8):
        check_close(got[gi], oracle.mmq_n(hm["slices"][gi], np.ascontiguousarray(oh[gi * 4096:(gi + 1) * 4096])))
    # a refused job: nothing enqueued
    sentinel = torch.full((1024,), 7.0, device=DEV)
    rc = lib.mmq_multi_dev_rc([(L.slices[0], o.data_ptr(), sentinel.data_ptr(), 1),
                               (L.slices[1], o.data_ptr(), sentinel.data_ptr(), -1)])
    torch.cuda.synchronize()
    assert rc == -1 and "n = -1" in lib.error()
    assert torch.all(sentinel == 7.0)
