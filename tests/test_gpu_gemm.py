# SPDX-License-Identifier: Apache-2.0
"""GPU parity for the prefill GEMM (dsv4_hip_gemm_fp8_dev / _fp8q_dev).

The oracle is the reference's fp8_n restated (oracle/dsv4_oracle.c, nt > 1
body of src/10_compute/dsv4_matmul_fp8.c:102-155) run on the activations the
GPU multiplies: quantized with the same 1x128 e4m3 rule and dequantized with
one fp32 multiply (q * s). Tolerance: relative L2 1e-3 on fp32 output; bf16
output is compared with bf16(oracle) at the same bound."""
import zlib

import numpy as np
import pytest
import torch

from conftest import REL_L2_TOL, bits, max_abs, rel_l2

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(DEV)


def e4m3_table(oracle):
    return np.array([oracle.e4m3(b) for b in range(256)], np.float32)


def dequant_act(oracle, Q, S, m, k):
    vals = e4m3_table(oracle)[Q].reshape(m, k)
    return (vals * np.repeat(S.reshape(m, k // 128), 128, axis=1)).astype(np.float32)


def make_weight(oracle, rng, n, k, f32s=True):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    W, S = oracle.quant_fp8_blk128(w)
    if not f32s:
        # E8M0 scales: the power of two at or above each fp32 block scale
        S = np.clip(np.ceil(np.log2(S)) + 127, 0, 254).astype(np.uint8)
    return W, S


def bf16_round(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().float().numpy()


def run_gemm(lib, pkg, A, W, S, n, k, f32s, out_bf16, a_bf16):
    m = A.shape[0]
    dW, dS = dev(W), dev(S)
    wdt = pkg.DSV4_WFP8_F32S if f32s else pkg.DSV4_WFP8
    desc = pkg.qmat(wdt, dW.data_ptr(), dS.data_ptr(), n, k, 128, 128)
    if a_bf16:
        dA = torch.from_numpy(A).to(DEV).bfloat16()
    else:
        dA = dev(A.astype(np.float32))
    C = torch.empty((m, n), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=DEV)
    lib.gemm_fp8_dev(C.data_ptr(), out_bf16, dA.data_ptr(), a_bf16, m, desc)
    torch.cuda.synchronize()
    return C.float().cpu().numpy()


def oracle_gemm(oracle, A, W, S, n, k, f32s):
    m = A.shape[0]
    Q, Sa = oracle.quant_act_fp8_1x128(A)
    x = dequant_act(oracle, Q, Sa, m, k).reshape(-1)
    if f32s:
        return oracle.fp8f_n(W, S, x, n, k, 128, 128, m).reshape(m, n)
    return oracle.fp8_n(W, S, x, n, k, 128, 128, m).reshape(m, n)


@pytest.mark.parametrize("m,n,k,f32s", [
    (256, 512, 1024, True), (200, 384, 512, True), (8, 256, 256, True),
    (130, 640, 768, False), (1, 128, 128, True)])
def test_gemm_fp32_out(lib, pkg, oracle, m, n, k, f32s):
    rng = np.random.default_rng(m * 31 + n + k)
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k, f32s)
    got = run_gemm(lib, pkg, A, W, S, n, k, f32s, out_bf16=0, a_bf16=0)
    want = oracle_gemm(oracle, A, W, S, n, k, f32s)
    e = rel_l2(got, want)
    assert np.all(np.isfinite(got))
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e} (max abs {max_abs(got, want):.3e})"


def test_gemm_bf16_in_equals_fp32_in(lib, pkg, oracle):
    rng = np.random.default_rng(5)
    m, n, k = 160, 256, 512
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k)
    a = run_gemm(lib, pkg, A, W, S, n, k, True, out_bf16=0, a_bf16=0)
    b = run_gemm(lib, pkg, A, W, S, n, k, True, out_bf16=0, a_bf16=1)
    assert np.array_equal(bits(a), bits(b))


def test_gemm_bf16_out(lib, pkg, oracle):
    rng = np.random.default_rng(6)
    m, n, k = 128, 512, 1024
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k)
    got = run_gemm(lib, pkg, A, W, S, n, k, True, out_bf16=1, a_bf16=1)
    want = bf16_round(oracle_gemm(oracle, A, W, S, n, k, True))
    assert rel_l2(got, want) <= REL_L2_TOL


def test_gemm_config_shape_row_sample(lib, pkg, oracle):
    """2048 tokens x 4096 x 4096 (bf16 A, fp32 128x128 weight scales, bf16
    output) on the GPU; 24 seeded rows checked against the oracle (rows are
    independent: each token is quantized and multiplied on its own)."""
    rng = np.random.default_rng(3)
    m, n, k = 2048, 4096, 4096
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k)
    got = run_gemm(lib, pkg, A, W, S, n, k, True, out_bf16=1, a_bf16=1)
    rows = np.sort(rng.choice(m, 24, replace=False))
    want = bf16_round(oracle_gemm(oracle, np.ascontiguousarray(A[rows]), W, S, n, k, True))
    assert np.all(np.isfinite(got))
    assert rel_l2(got[rows], want) <= REL_L2_TOL


def test_gemm_config_shape_every_row_against_torch_fp32(lib, pkg, oracle):
    """The same workload, every one of the 2,048 rows: the GEMM's bf16 output
    against a float32 torch product (TF32 off) of the same e4m3 tokens and
    weights, dequantized exactly (torch's float8_e4m3fn) with their block
    scales, rounded to bf16; each row within 1e-3. The tokens are the device
    quantizer's (dsv4_hip_quant_act_fp8_1x128_dev, whose codes and scales the
    1x128 tests above hold to the oracle's)."""
    rng = np.random.default_rng(33)
    m, n, k = 2048, 4096, 4096
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k)
    got = run_gemm(lib, pkg, A, W, S, n, k, True, out_bf16=1, a_bf16=1)
    dA = dev(A)
    Q = torch.empty(m * k, dtype=torch.uint8, device=DEV)
    Sa = torch.empty(m * k // 128, dtype=torch.float32, device=DEV)
    lib.quant_act_fp8_1x128_dev(Q.data_ptr(), Sa.data_ptr(), dA.data_ptr(), m, k)
    torch.cuda.synchronize()
    Af = Q.view(torch.float8_e4m3fn).float().reshape(m, k) * \
        Sa.reshape(k // 128, m).t().repeat_interleave(128, dim=1)
    Wf = dev(W).view(torch.float8_e4m3fn).float().reshape(n, k) * \
        dev(S).reshape(n // 128, k // 128).repeat_interleave(128, dim=0).repeat_interleave(128, dim=1)
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        ref = torch.mm(Af, Wf.t().contiguous()).bfloat16().float().cpu().numpy()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    assert np.all(np.isfinite(got))
    num = np.sqrt(np.sum((got.astype(np.float64) - ref) ** 2, axis=1))
    den = np.sqrt(np.sum(ref.astype(np.float64) ** 2, axis=1))
    worst = float(np.max(num / den))
    assert worst <= REL_L2_TOL, f"worst row rel L2 {worst:.3e}"


# The prefill attention side's FP8 projections at their real shapes
# (src/00_base/dsv4_weights.h:68-98; called through src/80_prefill/
# dsv4_prefill_proj.c:36-75 and dsv4_prefill_attn.c:26-110), with the
# checkpoint's E8M0 block scales: (rows, cols) = (N, K).
PROJECTIONS = {
    "wq_a": (1024, 4096), "wq_b": (32768, 1024), "wkv": (512, 4096),
    "wo_a_group": (1024, 4096), "wo_b": (4096, 8192), "idx_wq_b": (8192, 1024),
}


@pytest.mark.parametrize("name", sorted(PROJECTIONS))
def test_gemm_prefill_projection_shapes(lib, pkg, oracle, name):
    """300 tokens (not a tile multiple) through each projection, bf16 in and
    out as the prefill path runs them; 12 seeded rows against the oracle."""
    n, k = PROJECTIONS[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    m = 300
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k, f32s=False)
    got = run_gemm(lib, pkg, A, W, S, n, k, False, out_bf16=1, a_bf16=1)
    rows = np.sort(rng.choice(m, 12, replace=False))
    want = bf16_round(oracle_gemm(oracle, np.ascontiguousarray(A[rows]), W, S, n, k, False))
    assert np.all(np.isfinite(got))
    e = rel_l2(got[rows], want)
    assert e <= REL_L2_TOL, f"{name}: rel L2 {e:.3e}"


def test_gemm_prequantized_matches_fused(lib, pkg, oracle):
    rng = np.random.default_rng(8)
    m, n, k = 96, 256, 384
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k)
    fused = run_gemm(lib, pkg, A, W, S, n, k, True, out_bf16=0, a_bf16=0)
    Q, Sa = oracle.quant_act_fp8_1x128(A)
    Sa_blk = np.ascontiguousarray(Sa.reshape(m, k // 128).T)    # the entry point's block-major layout
    dW, dS, dQ, dSa = dev(W), dev(S), dev(Q), dev(Sa_blk)
    desc = pkg.qmat(pkg.DSV4_WFP8_F32S, dW.data_ptr(), dS.data_ptr(), n, k, 128, 128)
    C = torch.empty((m, n), dtype=torch.float32, device=DEV)
    lib.gemm_fp8q_dev(C.data_ptr(), 0, dQ.data_ptr(), dSa.data_ptr(), m, desc)
    torch.cuda.synchronize()
    assert np.array_equal(bits(C.cpu().numpy()), bits(fused))


def test_gemm_deterministic(lib, pkg, oracle):
    rng = np.random.default_rng(9)
    m, n, k = 256, 512, 512
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k)
    a = run_gemm(lib, pkg, A, W, S, n, k, True, 0, 0)
    b = run_gemm(lib, pkg, A, W, S, n, k, True, 0, 0)
    assert np.array_equal(bits(a), bits(b))


def test_gemm_rejects_bad_geometry(lib, pkg):
    W = torch.zeros(100 * 128, dtype=torch.uint8, device=DEV)
    S = torch.zeros(4, dtype=torch.float32, device=DEV)
    A = torch.zeros(128, dtype=torch.float32, device=DEV)
    C = torch.zeros(100, dtype=torch.float32, device=DEV)
    desc = pkg.qmat(pkg.DSV4_WFP8_F32S, W.data_ptr(), S.data_ptr(), 100, 128, 128, 128)
    rc = lib.lib.dsv4_hip_gemm_fp8_dev(C.data_ptr(), 0, A.data_ptr(), 0, 1, desc, None)
    assert rc == -1 and "multiples of 128" in lib.error()


def _e4m3_values():
    v = []
    for c in range(0x7F):
        e, m = c >> 3, c & 7
        v.append((1 + m / 8) * 2.0 ** (e - 7) if e else m / 8 * 2.0 ** -6)
    return np.array(v)


def test_act_quant_1x128_near_rounding_boundaries(lib, pkg, oracle):
    """Elements placed within four fp32 ulps of an e4m3 rounding boundary (the
    midpoint of two codes) times the group's scale, at scales from 2^-40 to
    2^40 and both signs: the quantizer's multiply-by-reciprocal fast path
    must hand every such element to the division, bit-exact against the
    oracle's e4m3(v / s)."""
    rng = np.random.default_rng(23)
    n, k = 64, 1024
    vals = _e4m3_values()
    mids = (vals[:-1] + vals[1:]) / 2
    a = np.empty((n, k), np.float32)
    for t in range(n):
        amax = np.float32(2.0 ** rng.integers(-40, 40) * rng.uniform(0.5, 1.0))
        s = np.float32(amax / np.float32(448.0))
        m = rng.choice(mids, k).astype(np.float32)
        v = (m * s).astype(np.float32).view(np.int32) + rng.integers(-4, 5, k).astype(np.int32)
        row = v.view(np.float32) * np.where(rng.random(k) < 0.5, -1, 1).astype(np.float32)
        row[:: 128] = amax                              # every group's maximum is amax
        a[t] = np.clip(row, -amax, amax)
    da = dev(a)
    Q = torch.empty(n * k, dtype=torch.uint8, device=DEV)
    S = torch.empty(n * (k // 128), dtype=torch.float32, device=DEV)
    lib.quant_act_fp8_1x128_dev(Q.data_ptr(), S.data_ptr(), da.data_ptr(), n, k)
    torch.cuda.synchronize()
    Qo, So = oracle.quant_act_fp8_1x128(a)
    got_q = Q.cpu().numpy()
    bad = np.nonzero(got_q != Qo)[0]
    assert bad.size == 0, f"{bad.size} codes differ, first at {bad[:4]}: {got_q[bad[:4]]} vs {Qo[bad[:4]]}"


def test_act_quant_1x128_edge_cases(lib, pkg, oracle):
    """Bit-exact against the oracle on values the fast path must get right:
    magnitudes from e4m3's subnormal range to its maximum, exact
    round-to-nearest-even ties (amax 448 makes the scale exactly 1), signed
    zeros, an all-zero group and a NaN (ignored by the group max, encoded as
    sign | 0x7F)."""
    rng = np.random.default_rng(17)
    n, k = 12, 512
    a = (rng.standard_normal((n, k)) * np.exp(rng.uniform(-30, 30, (n, k)))).astype(np.float32)
    a[0, :] = 0.0
    a[0, 5] = -0.0
    a[1, :128] = 0.0
    ties = np.array([1.0625, 1.1875, 0.015625 * 1.5, 0.001953125 * 2.5, 240.0 + 8.0, 416.0 + 16.0,
                     -1.0625, -0.0029296875], np.float32)
    a[2, :8] = ties
    a[2, 8] = 448.0
    a[3, 200] = np.float32("nan")
    a[4, :] = (rng.standard_normal(k) * 1e-3).astype(np.float32)
    a[5, :] = np.float32(3.0e38) * np.sign(rng.standard_normal(k)).astype(np.float32)
    da = dev(a)
    Q = torch.empty(n * k, dtype=torch.uint8, device=DEV)
    S = torch.empty(n * (k // 128), dtype=torch.float32, device=DEV)
    lib.quant_act_fp8_1x128_dev(Q.data_ptr(), S.data_ptr(), da.data_ptr(), n, k)
    torch.cuda.synchronize()
    Qo, So = oracle.quant_act_fp8_1x128(a)
    got_q = Q.cpu().numpy()
    got_s = np.ascontiguousarray(S.cpu().numpy().reshape(k // 128, n).T).reshape(-1)   # block-major
    assert np.array_equal(bits(got_s), bits(So))
    bad = np.nonzero(got_q != Qo)[0]
    assert bad.size == 0, f"{bad.size} codes differ, first at {bad[:4]}: {got_q[bad[:4]]} vs {Qo[bad[:4]]}"


# ---------------------------------------------------------------------------
# The checkpoint-format GEMM (dsv4_hip_gemm_mxfp8_dev / _mxfp8q_dev): E8M0
# 128x128 weight scales and MXFP8 activations (e4m3 + E8M0 per 1x32), both in
# the MFMA's hardware scale operands. The oracle is fp8_n on the weights as
# stored, fed the activations quantized by the oracle's MXFP8 rule and
# dequantized (q * 2^(s - 127), exact).

def dequant_mx(oracle, Q, S, m, k):
    vals = e4m3_table(oracle)[Q].reshape(m, k)
    sc = np.ldexp(np.float32(1.0), S.astype(np.int32) - 127).astype(np.float32).reshape(m, k // 32)
    return (vals * np.repeat(sc, 32, axis=1)).astype(np.float32)


def run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16, a_bf16):
    m = A.shape[0]
    dW, dS = dev(W), dev(S)
    desc = pkg.qmat(pkg.DSV4_WFP8, dW.data_ptr(), dS.data_ptr(), n, k, 128, 128)
    dA = torch.from_numpy(A).to(DEV).bfloat16() if a_bf16 else dev(A.astype(np.float32))
    C = torch.empty((m, n), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=DEV)
    lib.gemm_mxfp8_dev(C.data_ptr(), out_bf16, dA.data_ptr(), a_bf16, m, desc)
    torch.cuda.synchronize()
    return C.float().cpu().numpy()


def oracle_gemm_mx(oracle, A, W, S, n, k):
    m = A.shape[0]
    Q, Sa = oracle.quant_act_mxfp8(np.ascontiguousarray(A, np.float32))
    x = dequant_mx(oracle, Q, Sa, m, k).reshape(-1)
    return oracle.fp8_n(W, S, x, n, k, 128, 128, m).reshape(m, n)


@pytest.mark.parametrize("m,n,k", [(256, 512, 1024), (200, 384, 512), (8, 256, 256), (1, 128, 128),
                                   (130, 640, 768)])
def test_gemm_mx_fp32_out(lib, pkg, oracle, m, n, k):
    rng = np.random.default_rng(m * 37 + n + 3 * k)
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k, f32s=False)
    got = run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16=0, a_bf16=0)
    want = oracle_gemm_mx(oracle, A, W, S, n, k)
    e = rel_l2(got, want)
    assert np.all(np.isfinite(got))
    assert e <= REL_L2_TOL, f"rel L2 {e:.3e} (max abs {max_abs(got, want):.3e})"


def test_gemm_mx_outlier_scales(lib, pkg, oracle):
    """Activation groups spanning 2^-40 .. 2^40 and weight blocks whose E8M0
    bytes differ by up to 2^20: every scale is a power of two the hardware
    applies exactly, so the result still meets the bound."""
    rng = np.random.default_rng(44)
    m, n, k = 64, 256, 512
    A = rng.standard_normal((m, k)).astype(np.float32)
    A *= np.exp2(rng.integers(-40, 41, (m, k // 32))).repeat(32, axis=1).astype(np.float32)
    A = bf16_round(A)
    W, S = make_weight(oracle, rng, n, k, f32s=False)
    S = np.clip(S.astype(np.int32) + rng.integers(-10, 11, S.shape), 1, 254).astype(np.uint8)
    got = run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16=0, a_bf16=0)
    want = oracle_gemm_mx(oracle, A, W, S, n, k)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= REL_L2_TOL


def test_gemm_mx_bf16_in_out(lib, pkg, oracle):
    rng = np.random.default_rng(45)
    m, n, k = 160, 512, 1024
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k, f32s=False)
    a = run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16=0, a_bf16=0)
    b = run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16=0, a_bf16=1)
    assert np.array_equal(bits(a), bits(b))
    got = run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16=1, a_bf16=1)
    want = bf16_round(oracle_gemm_mx(oracle, A, W, S, n, k))
    assert rel_l2(got, want) <= REL_L2_TOL


def test_gemm_mx_config_shape_row_sample(lib, pkg, oracle):
    """2048 tokens x 4096 x 4096 with the checkpoint's E8M0 weight scales;
    24 seeded rows against the oracle."""
    rng = np.random.default_rng(46)
    m, n, k = 2048, 4096, 4096
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k, f32s=False)
    got = run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16=1, a_bf16=1)
    rows = np.sort(rng.choice(m, 24, replace=False))
    want = bf16_round(oracle_gemm_mx(oracle, np.ascontiguousarray(A[rows]), W, S, n, k))
    assert np.all(np.isfinite(got))
    assert rel_l2(got[rows], want) <= REL_L2_TOL


def test_gemm_mx_prequantized_matches_fused(lib, pkg, oracle):
    rng = np.random.default_rng(47)
    m, n, k = 96, 256, 384
    A = bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    W, S = make_weight(oracle, rng, n, k, f32s=False)
    fused = run_gemm_mx(lib, pkg, A, W, S, n, k, out_bf16=0, a_bf16=0)
    Q, Sa = oracle.quant_act_mxfp8(A)
    dW, dS, dQ, dSa = dev(W), dev(S), dev(Q), dev(Sa)
    desc = pkg.qmat(pkg.DSV4_WFP8, dW.data_ptr(), dS.data_ptr(), n, k, 128, 128)
    C = torch.empty((m, n), dtype=torch.float32, device=DEV)
    lib.gemm_mxfp8q_dev(C.data_ptr(), 0, dQ.data_ptr(), dSa.data_ptr(), m, desc)
    torch.cuda.synchronize()
    assert np.array_equal(bits(C.cpu().numpy()), bits(fused))


def test_gemm_mx_rejects_fp32_scales(lib, pkg):
    W = torch.zeros(128 * 128, dtype=torch.uint8, device=DEV)
    S = torch.zeros(1, dtype=torch.float32, device=DEV)
    A = torch.zeros(128, dtype=torch.float32, device=DEV)
    C = torch.zeros(128, dtype=torch.float32, device=DEV)
    desc = pkg.qmat(pkg.DSV4_WFP8_F32S, W.data_ptr(), S.data_ptr(), 128, 128, 128, 128)
    rc = lib.lib.dsv4_hip_gemm_mxfp8_dev(C.data_ptr(), 0, A.data_ptr(), 0, 1, desc, None)
    assert rc == -1 and "E8M0" in lib.error()
