# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the block-scaled MFMA decode path (activations split into
four e4m3 parts as the B operand, packed weights as the A operand) against the
oracle: activation edge cases the split must survive (outlier channels, zero
and tiny blocks, fp32 subnormals), 1-7 tokens per call, special scale bytes,
waves without chunks, and the expert / MoE kernels at shapes that take the
MFMA path."""
import zlib

import numpy as np
import pytest
import torch

import pyoracle as P
from conftest import REL_L2_TOL, bits, rel_l2
from test_gpu_decode import (DEV, Resident, _rand_fp8, bf16_x, check_close, dev_f32, dev_u8,
                             make_fp4_expert, make_fp8_shared)

pytestmark = pytest.mark.gpu


def _x_edge(rng, n, kind):
    x = rng.standard_normal(n).astype(np.float32)
    if kind == "outliers":           # a few channels 10^4 x larger than the rest
        x[rng.choice(n, 6, replace=False)] *= 1.0e4
    elif kind == "zero_blocks":      # whole 32-blocks of zeros, and an all-zero chunk
        x[32:64] = 0.0
        x[256:384] = 0.0
    elif kind == "tiny":             # fp32 subnormals and near-underflow blocks
        x[:32] *= 1.0e-41
        x[32:64] *= 1.0e-30
        x[64:96] = np.float32(1.0e-45)
    elif kind == "wide":             # magnitudes spanning 2^-60 .. 2^60 inside each block
        x *= np.exp2(rng.integers(-60, 61, n)).astype(np.float32)
    return x


@pytest.mark.parametrize("kind", ["plain", "outliers", "zero_blocks", "tiny", "wide"])
@pytest.mark.parametrize("fmt", ["fp4", "fp8", "fp8f"])
def test_mx_gemv_activation_edges(lib, pkg, oracle, kind, fmt):
    rows, cols = 256, 1024
    rng = np.random.default_rng(zlib.crc32(f"{kind}/{fmt}".encode()))
    x = _x_edge(rng, cols, kind)
    if fmt == "fp4":
        W = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
        S = rng.integers(118, 134, rows * cols // 32).astype(np.uint8)
        m = Resident(lib, pkg, pkg.DSV4_WFP4, W, S, rows, cols, 1, 32)
        want = oracle.fp4_n(W, S, x, rows, cols, 1, 32, 1)
    elif fmt == "fp8":
        W = _rand_fp8(rng, rows * cols)
        S = rng.integers(118, 134, (rows // 128) * (cols // 128)).astype(np.uint8)
        m = Resident(lib, pkg, pkg.DSV4_WFP8, W, S, rows, cols, 128, 128)
        want = oracle.fp8_n(W, S, x, rows, cols, 128, 128, 1)
    else:
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        W, S = oracle.quant_fp8_blk128(w)
        m = Resident(lib, pkg, pkg.DSV4_WFP8_F32S, W, S, rows, cols, 128, 128)
        want = oracle.fp8f_n(W, S, x, rows, cols, 128, 128, 1)
    y = lib.mmq_n(m.desc, x, 1)
    m.drop()
    check_close(y, want)


@pytest.mark.parametrize("nt", [1, 2, 3, 4, 5, 7])
@pytest.mark.parametrize("fmt,cols", [("fp4", 4096), ("fp8", 4096), ("fp4", 512), ("fp8", 8 * 128)])
def test_mx_gemv_tokens(lib, pkg, oracle, nt, fmt, cols):
    """Token groups of the MFMA GEMV: up to four tokens share the sixteen B
    columns; more tokens are further groups of the grid."""
    rows = 160
    rng = np.random.default_rng(nt * 1000 + cols)
    x = rng.standard_normal(nt * cols).astype(np.float32)
    if fmt == "fp4":
        W = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
        S = rng.integers(118, 134, rows * cols // 32).astype(np.uint8)
        m = Resident(lib, pkg, pkg.DSV4_WFP4, W, S, rows, cols, 1, 32)
        want = oracle.fp4_n(W, S, x, rows, cols, 1, 32, nt)
    else:
        W = _rand_fp8(rng, rows * cols)
        S = rng.integers(118, 134, 2 * (cols // 128)).astype(np.uint8)
        m = Resident(lib, pkg, pkg.DSV4_WFP8, W, S, rows, cols, 128, 128)
        want = oracle.fp8_n(W, S, x, rows, cols, 128, 128, nt)
    y = lib.mmq_n(m.desc, x, nt)
    m.drop()
    for t in range(nt):
        check_close(y[t * rows:(t + 1) * rows], want[t * rows:(t + 1) * rows])


@pytest.mark.parametrize("cols", [128, 384, 640])
def test_mx_gemv_idle_waves(lib, pkg, oracle, cols):
    """K shorter than four waves' worth: some waves of a tile own no chunk."""
    rows = 48
    rng = np.random.default_rng(cols)
    W = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    S = rng.integers(118, 134, rows * cols // 32).astype(np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    m = Resident(lib, pkg, pkg.DSV4_WFP4, W, S, rows, cols, 1, 32)
    y = lib.mmq_n(m.desc, x, 1)
    m.drop()
    check_close(y, oracle.fp4_n(W, S, x, rows, cols, 1, 32, 1))


def test_mx_gemv_special_scales(lib, pkg, oracle):
    """E8M0 scale bytes 0 (2^-127), 254 and 255 (NaN) in the hardware scale
    operand: rows holding a 255 come out NaN, like the oracle's; the others
    match it."""
    rows, cols = 64, 512
    rng = np.random.default_rng(5)
    W = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    S = rng.integers(118, 134, rows * cols // 32).astype(np.uint8).reshape(rows, cols // 32)
    S[3, 2] = 0
    S[7, :] = 0
    S[9, 5] = 254
    S[11, 0] = 255
    S[40, 15] = 255
    S = S.reshape(-1)
    x = rng.standard_normal(cols).astype(np.float32)
    m = Resident(lib, pkg, pkg.DSV4_WFP4, W, S, rows, cols, 1, 32)
    y = lib.mmq_n(m.desc, x, 1)
    m.drop()
    want = oracle.fp4_n(W, S, x, rows, cols, 1, 32, 1)
    nan = np.isnan(want)
    assert list(np.nonzero(nan)[0]) == [11, 40]
    assert np.array_equal(np.isnan(y), nan)
    ok = ~nan & np.isfinite(want)
    assert rel_l2(y[ok], want[ok]) <= REL_L2_TOL


def test_mx_expert_forward_fp8_shared_shape(lib, pkg, oracle):
    """The FP8 (fp32-scale) expert through the MFMA gate/up and GEMV."""
    rng = np.random.default_rng(41)
    e, he, mats = make_fp8_shared(lib, pkg, oracle, rng, inter=512, hidden=1024)
    x = bf16_x(5, 1024)
    y = lib.expert_forward(e, x, 10.0)
    check_close(y, oracle.expert_forward(he, x, 10.0))
    for m in mats:
        m.drop()


@pytest.mark.parametrize("wdt", ["e8m0", "f32s"])
@pytest.mark.parametrize("inter,hidden", [(2048, 4096), (512, 1024), (128, 2048), (256, 640)])
def test_fp8_expert_row_tiles(lib, pkg, oracle, wdt, inter, hidden):
    """FP8 experts (E8M0 or fp32 128 x 128 scales) through the 8-row-tile
    gate/up kernel (hidden 1024, 2048, 4096: chunk pairs, per-lane scales) and
    the 32-row one (hidden 640), with random e4m3 codes and a different scale
    for every block, so the two chunks of every pair scale differently:
    against the oracle's expert_forward."""
    rng = np.random.default_rng(zlib.crc32(wdt.encode()) + inter + hidden)
    mats = []
    for (r, c) in ((inter, hidden), (inter, hidden), (hidden, inter)):
        W = _rand_fp8(rng, r * c)
        nb = ((r + 127) // 128) * (c // 128)
        if wdt == "e8m0":
            S, t = rng.integers(112, 122, nb).astype(np.uint8), pkg.DSV4_WFP8
        else:
            S = (2.0 ** rng.integers(-15, -5, nb) * rng.uniform(0.5, 1.0, nb)).astype(np.float32)
            t = pkg.DSV4_WFP8_F32S
        mats.append(Resident(lib, pkg, t, W, S, r, c, 128, 128))
    e = pkg.ExpertW(mats[0].desc, mats[1].desc, mats[2].desc)
    he = P.HostExpert(mats[0].hm, mats[1].hm, mats[2].hm)
    x = bf16_x(7, hidden)
    y = lib.expert_forward(e, x, 10.0)
    for m in mats:
        m.drop()
    # random codes span 2^-9 .. 448 within a block, the harshest case for the
    # MFMA's alignment of products: the contract's 1e-3 (observed <= 1.5e-4)
    check_close(y, oracle.expert_forward(he, x, 10.0))


@pytest.mark.parametrize("inter,hidden,topk", [(128, 512, 1), (256, 1024, 8), (2048, 4096, 6)])
def test_mx_moe_decode_shapes(lib, pkg, oracle, inter, hidden, topk):
    rng = np.random.default_rng(inter + topk)
    experts = [make_fp4_expert(lib, pkg, oracle, rng, inter, hidden) for _ in range(topk)]
    x = bf16_x(7, hidden)
    lg = rng.standard_normal(topk)
    w = (np.exp(lg) / np.exp(lg).sum()).astype(np.float32)
    y = lib.moe_decode([e for e, _, _ in experts], w, x, None, 10.0)
    acc = np.stack([oracle.expert_forward(he, x, 10.0) for _, he, _ in experts])
    e = check_close(y, oracle.moe_combine(acc, w))
    assert e < 1e-4
    for _, _, mats in experts:
        for m in mats:
            m.drop()


def test_mx_moe_decode_bad_descriptor_poisons(lib, pkg, oracle):
    """A routed slot whose w1 descriptor has the wrong format raises status
    bit 1 and turns the whole output NaN (the down projection reads NaN block
    scales for that slot)."""
    rng = np.random.default_rng(43)
    inter, hidden = 128, 512
    mats = []
    for (r, c) in ((inter, hidden), (inter, hidden), (hidden, inter)):
        W, S = oracle.quant_fp4_mx((rng.standard_normal((r, c)) * 0.02).astype(np.float32))
        mats.append((dev_u8(W), dev_u8(S), r, c))
    good = [pkg.qmat(pkg.DSV4_WFP4, w.data_ptr(), s.data_ptr(), r, c, 1, 32) for w, s, r, c in mats]
    badw1 = pkg.qmat(pkg.DSV4_WFP8, mats[0][0].data_ptr(), mats[0][1].data_ptr(), inter, hidden, 128, 128)
    table = bytes(pkg.ExpertW(good[0], good[1], good[2])) + bytes(pkg.ExpertW(badw1, good[1], good[2]))
    tbl = torch.from_numpy(np.frombuffer(table, np.uint8).copy()).to(DEV)
    x = dev_f32(rng.standard_normal(hidden))
    w = dev_f32(np.array([0.5, 0.5], np.float32))
    out = torch.zeros(hidden, dtype=torch.float32, device=DEV)
    lib.status()
    idx = torch.tensor([0, 0], dtype=torch.int32, device=DEV)
    lib.moe_decode_dev(out.data_ptr(), x.data_ptr(), tbl.data_ptr(), 2, idx.data_ptr(),
                       w.data_ptr(), 2, None, hidden, inter, 10.0)
    assert lib.status() == 0 and torch.isfinite(out).all()
    idx = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    lib.moe_decode_dev(out.data_ptr(), x.data_ptr(), tbl.data_ptr(), 2, idx.data_ptr(),
                       w.data_ptr(), 2, None, hidden, inter, 10.0)
    assert lib.status() & 2
    assert torch.isnan(out).all()


def _device_fp4_experts(pkg, oracle, rng, n, inter, hidden):
    """n FP4 experts with device-resident weights: (device descriptors, host
    experts for the oracle, tensors to keep alive)."""
    descs, host, keep = [], [], []
    for _ in range(n):
        q, hm = [], []
        for (r, c) in ((inter, hidden), (inter, hidden), (hidden, inter)):
            W, S = oracle.quant_fp4_mx((rng.standard_normal((r, c)) * 0.02).astype(np.float32))
            dW, dS = dev_u8(W), dev_u8(S)
            keep += [dW, dS]
            q.append(pkg.qmat(pkg.DSV4_WFP4, dW.data_ptr(), dS.data_ptr(), r, c, 1, 32))
            hm.append(P.HostMat(pkg.DSV4_WFP4, W, S, r, c, 1, 32))
        descs.append(pkg.ExpertW(q[0], q[1], q[2]))          # w1, w3, w2
        host.append(P.HostExpert(hm[0], hm[1], hm[2]))
    return descs, host, keep


@pytest.mark.parametrize("inter,hidden,topk", [(256, 1024, 8), (2048, 4096, 6)])
def test_moe_decode_routed_matches_device_routed(lib, pkg, oracle, inter, hidden, topk):
    """The host-routed entry (descriptors and weights by value in the kernel
    arguments) gives the device-routed entry's output bit for bit, and the
    oracle's within 1e-4."""
    rng = np.random.default_rng(zlib.crc32(b"routed") + inter + topk)
    n_exp = topk + 3
    descs, host, keep = _device_fp4_experts(pkg, oracle, rng, n_exp, inter, hidden)
    idx = rng.choice(n_exp, topk, replace=False).astype(np.int32)
    lg = rng.standard_normal(topk)
    w = (np.exp(lg) / np.exp(lg).sum()).astype(np.float32)
    xh = bf16_x(11, hidden)
    x = dev_f32(xh)
    arr = (pkg.ExpertW * n_exp)(*descs)
    tbl = torch.from_numpy(np.frombuffer(b"".join(bytes(d) for d in descs), np.uint8).copy()).to(DEV)
    didx = torch.from_numpy(idx).to(DEV)
    dw = dev_f32(w)
    out_r = torch.empty(hidden, dtype=torch.float32, device=DEV)
    out_d = torch.empty(hidden, dtype=torch.float32, device=DEV)
    lib.status()
    lib.moe_decode_routed_dev(out_r.data_ptr(), x.data_ptr(), arr, idx, w, topk, None,
                              hidden, inter, 10.0)
    lib.moe_decode_dev(out_d.data_ptr(), x.data_ptr(), tbl.data_ptr(), n_exp, didx.data_ptr(),
                       dw.data_ptr(), topk, None, hidden, inter, 10.0)
    torch.cuda.synchronize()
    assert lib.status() == 0
    got = out_r.cpu().numpy()
    assert np.array_equal(bits(got), bits(out_d.cpu().numpy()))
    acc = np.stack([oracle.expert_forward(host[i], xh, 10.0) for i in idx])
    assert check_close(got, oracle.moe_combine(acc, w)) < 1e-4


def test_moe_decode_routed_rejects_bad_routing(lib, pkg, oracle):
    """A routing id out of range or a routed expert of the wrong format is
    refused on the host before anything is launched; the backend stays usable."""
    rng = np.random.default_rng(zlib.crc32(b"routed-bad"))
    inter, hidden = 128, 512
    descs, host, keep = _device_fp4_experts(pkg, oracle, rng, 2, inter, hidden)
    arr = (pkg.ExpertW * 2)(*descs)
    xh = bf16_x(12, hidden)
    x = dev_f32(xh)
    out = torch.zeros(hidden, dtype=torch.float32, device=DEV)
    w = np.array([0.5, 0.5], np.float32)
    with pytest.raises(Exception, match="routing id 2 of slot 1"):
        lib.moe_decode_routed_dev(out.data_ptr(), x.data_ptr(), arr, [0, 2], w, 2, None,
                                  hidden, inter, 10.0)
    bad = pkg.ExpertW(pkg.qmat(pkg.DSV4_WFP8, descs[0].w1.w, descs[0].w1.s, inter, hidden, 128, 128),
                      descs[0].w3, descs[0].w2)
    arr_bad = (pkg.ExpertW * 2)(descs[0], bad)
    with pytest.raises(Exception, match="moe_decode_routed_dev"):
        lib.moe_decode_routed_dev(out.data_ptr(), x.data_ptr(), arr_bad, [0, 1], w, 2, None,
                                  hidden, inter, 10.0)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0           # nothing ran
    lib.moe_decode_routed_dev(out.data_ptr(), x.data_ptr(), arr, [1, 0], w, 2, None,
                              hidden, inter, 10.0)
    torch.cuda.synchronize()
    acc = np.stack([oracle.expert_forward(host[i], xh, 10.0) for i in (1, 0)])
    assert check_close(out.cpu().numpy(), oracle.moe_combine(acc, w)) < 1e-4
