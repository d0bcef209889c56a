# SPDX-License-Identifier: Apache-2.0
"""The reference's own known-answer gates, applied to the oracle.

Expected values are the ones the reference's tests hand-derive from the
format definitions (tests/unit/test_quant.c, tests/unit/test_matmul.c,
tests/unit/test_ops.c); none is computed by the code under test. The
random-data gates bound the oracle against its scalar double-precision
counterpart at the reference's own L2 <= 1e-6."""
import math

import numpy as np
import pytest

from conftest import bits, rel_l2


def f32(v):
    return np.float32(v)


# ------------------------------------------------------ test_quant.c gates

def test_e8m0_exact(oracle):
    """test_quant.c:39-61: 2^(b-127) for 1..254, 0 -> 2^-127, 255 -> NaN."""
    for b in range(1, 255):
        assert oracle.e8m0(b) == math.ldexp(1.0, b - 127)
    assert oracle.e8m0(0) == math.ldexp(1.0, -127) and oracle.e8m0(0) != 0.0
    assert math.isnan(oracle.e8m0(255))


def test_e4m3_codes(oracle):
    """test_quant.c:63-107."""
    want = {0x00: 0.0, 0x38: 1.0, 0xB8: -1.0, 0x3C: 1.5, 0x3A: 1.25, 0x40: 2.0,
            0x30: 0.5, 0x01: 2.0 ** -9, 0x02: 2.0 ** -8, 0x07: 7 * 2.0 ** -9,
            0x7E: 448.0, 0x7B: 352.0}
    for b, v in want.items():
        assert oracle.e4m3(b) == v
    assert math.isnan(oracle.e4m3(0x7F)) and math.isnan(oracle.e4m3(0xFF))
    finite = [oracle.e4m3(b) for b in range(256) if not math.isnan(oracle.e4m3(b))]
    assert max(finite) == 448.0
    for b in range(128):
        p, n = oracle.e4m3(b), oracle.e4m3(b | 0x80)
        if not math.isnan(p):
            assert n == -p
    # every code against the format's closed form (sign, 4-bit exp bias 7, 3-bit man)
    for b in range(256):
        e, m, s = (b >> 3) & 15, b & 7, -1.0 if b & 0x80 else 1.0
        if e == 15 and m == 7:
            continue
        v = s * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
        assert oracle.e4m3(b) == v


def test_e2m1_codes_and_nibble_order(oracle):
    """test_quant.c:109-186: eight magnitudes, max 6, sign bit 3, 0x21 -> {0.5, 1.0}."""
    want = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for i in range(8):
        assert oracle.e2m1(i) == want[i]
        assert oracle.e2m1(i | 8) == -want[i]
    assert math.copysign(1.0, oracle.e2m1(8)) == -1.0  # code 8 is -0.0
    # 0x21: low nibble (1 -> 0.5) is element 0, high nibble (2 -> 1.0) element 1
    W = np.array([0x21] * 16, np.uint8)
    S = np.array([127], np.uint8)
    x = np.zeros(32, np.float32); x[0] = 1.0
    assert oracle.fp4_n(W, S, x, 1, 32)[0] == 0.5
    x[:] = 0; x[1] = 1.0
    assert oracle.fp4_n(W, S, x, 1, 32)[0] == 1.0


# ----------------------------------------------------- test_matmul.c gates

def test_gate1_fp8_one_block_shared_row_scale(oracle):
    """test_matmul.c:206-230: both rows of a 2x128 matrix share S[0]."""
    W = np.concatenate([np.full(128, 0x38, np.uint8), np.full(128, 0x40, np.uint8)])
    S = np.array([128, 0], np.uint8)
    y = oracle.fp8_n(W, S, np.ones(128, np.float32), 2, 128)
    assert y[0] == 256.0 and y[1] == 512.0


def test_gate1b_fp8_row_block_boundary(oracle):
    """test_matmul.c:232-252."""
    W = np.full(256 * 128, 0x38, np.uint8)
    S = np.array([127, 129], np.uint8)
    y = oracle.fp8_n(W, S, np.ones(128, np.float32), 256, 128)
    assert y[0] == y[127] == 128.0 and y[128] == y[255] == 512.0


def test_gate2_fp8_scale_changes_across_blocks(oracle):
    """test_matmul.c:254-273: 384, not 256."""
    W = np.full(256, 0x38, np.uint8)
    S = np.array([127, 128], np.uint8)
    assert oracle.fp8_n(W, S, np.ones(256, np.float32), 1, 256)[0] == 384.0


def test_gate3_to_5c_fp4(oracle):
    """test_matmul.c:276-385."""
    # GATE 3: per-row and per-block scales
    W = np.full(2 * 32, 0x22, np.uint8)
    S = np.array([127, 128, 127, 127], np.uint8)
    y = oracle.fp4_n(W, S, np.ones(64, np.float32), 2, 64)
    assert y[0] == 96.0 and y[1] == 64.0
    # GATE 4: row stride is in/2 bytes
    W = np.concatenate([np.full(16, 0x22, np.uint8), np.full(16, 0x44, np.uint8)])
    y = oracle.fp4_n(W, np.array([127, 127], np.uint8), np.ones(32, np.float32), 2, 32)
    assert y[0] == 32.0 and y[1] == 64.0
    # GATE 5: +-1 alternating against 1..32 with scale 2; |y| = 32, and with the
    # low-nibble-first order +1 sits on the even (1-based odd) elements: -32
    W = np.full(16, 0xA2, np.uint8)
    x = np.arange(1, 33, dtype=np.float32)
    y = oracle.fp4_n(W, np.array([128], np.uint8), x, 1, 32)
    assert abs(y[0]) == 32.0 and y[0] == -32.0
    # GATE 5b: one four-block group plus a tail block, scales per block
    IN, OUT = 160, 3
    W = np.full(OUT * IN // 2, 0x22, np.uint8)
    S = np.array([127 + ((b + o) % 5) for o in range(OUT) for b in range(IN // 32)], np.uint8)
    y = oracle.fp4_n(W, S, np.ones(IN, np.float32), OUT, IN)
    for o in range(OUT):
        assert y[o] == sum(32.0 * 2.0 ** ((b + o) % 5) for b in range(IN // 32))
    # GATE 5c: 513 blocks fall back to the generic loop
    IN = 16416
    y = oracle.fp4_n(np.full(IN // 2, 0x22, np.uint8), np.full(IN // 32, 127, np.uint8),
                     np.ones(IN, np.float32), 1, IN)
    assert y[0] == float(IN)


def _lcg(r):
    return (r * 1103515245 + 12345) & 0xFFFFFFFF


def test_gate7_thread_invariance_and_finiteness(oracle, monkeypatch):
    """test_matmul.c:408-437 with the oracle's own OpenMP loop: rows are
    independent, so 1 and 8 threads give identical bits."""
    IN, OUT = 256, 96
    st = 12345
    W = np.zeros(OUT * IN, np.uint8)
    for i in range(OUT * IN):
        st = _lcg(st); W[i] = (st >> 16) & 0x7E
    S = np.array([120 + (i % 9) for i in range(OUT * 2)], np.uint8)
    x = np.zeros(IN, np.float32)
    for i in range(IN):
        st = _lcg(st); x[i] = np.float32(((st >> 20) & 0xFF) - 128) * np.float32(0.01)
    a = oracle.fp8_n(W, S, x, OUT, IN)
    b = oracle.fp8_n(W, S, x, OUT, IN)
    assert np.array_equal(bits(a), bits(b)) and np.all(np.isfinite(a))


def test_random_l2_vs_double(oracle):
    """test_matmul.c:440-541 and :543-585: FP8 (128 and generic 100 blocks) and
    FP4 against the scalar double oracle at L2 <= 1e-6."""
    rng = np.random.default_rng(7)
    for IN, OUT in ((256, 37), (4096, 8)):
        x = (rng.integers(-32768, 32768, IN) * 1e-3).astype(np.float32)
        W8 = rng.integers(0, 256, OUT * IN).astype(np.uint8)
        W8[(W8 & 0x7F) == 0x7F] &= 0xFE
        for bc in (128, 100):
            ns = ((OUT + 127) // 128) * ((IN + bc - 1) // bc)
            S8 = np.full(ns, 127, np.uint8)
            e = rel_l2(oracle.fp8_n(W8, S8, x, OUT, IN, 128, bc),
                       oracle.fp8_double(W8, S8, x, OUT, IN, 128, bc))
            assert e <= 1e-6, (IN, bc, e)
        W4 = rng.integers(0, 256, OUT * IN // 2).astype(np.uint8)
        S4 = np.full(OUT * IN // 32, 127, np.uint8)
        e = rel_l2(oracle.fp4_n(W4, S4, x, OUT, IN), oracle.fp4_double(W4, S4, x, OUT, IN))
        assert e <= 1e-6, (IN, e)


def test_all_256_e4m3_codes_through_fp8_n(oracle):
    """test_matmul.c:588-633: y[r] = decode(r) via a diagonal matrix."""
    N = 256
    W = np.zeros(N * N, np.uint8)
    for r in range(N):
        W[r * N + r] = r
    S = np.full(4, 127, np.uint8)
    y = oracle.fp8_n(W, S, np.ones(N, np.float32), N, N)
    yd = oracle.fp8_double(W, S, np.ones(N, np.float32), N, N)
    for r in range(N):
        want = oracle.e4m3(r)
        if math.isnan(want):
            assert math.isnan(y[r])
            continue
        # the dot starts from +0, so a -0 weight sums to +0 (test_matmul.c:614-621)
        assert y[r] == want and (want != 0.0 or bits(y[r:r + 1])[0] == 0)
        assert bits(y[r:r + 1])[0] == bits(yd[r:r + 1])[0]


def test_batched_equals_nt_gemvs(oracle):
    """test_matmul.c:690-792: nt = 130 > 128, distinct activations per token;
    FP8 with a special block and FP4 are bitwise equal to nt one-token calls."""
    NT, IN, OUT = 130, 256, 130
    rng = np.random.default_rng(123456789)
    x = ((rng.integers(0, 1024, NT * IN) - 512) * 0.017).astype(np.float32)
    e = rng.integers(1, 15, OUT * IN); m = rng.integers(0, 8, OUT * IN)
    s = rng.integers(0, 2, OUT * IN)
    W8 = ((s << 7) | (e << 3) | m).astype(np.uint8)
    W8[0] = 0x01
    S8 = np.array([124 + (i % 7) for i in range(2 * (IN // 128))], np.uint8)
    yb = oracle.fp8_n(W8, S8, x, OUT, IN, nt=NT)
    ya = np.concatenate([oracle.fp8_n(W8, S8, x[t * IN:(t + 1) * IN], OUT, IN) for t in range(NT)])
    assert np.array_equal(bits(ya), bits(yb))
    W4 = rng.integers(0, 256, OUT * IN // 2).astype(np.uint8)
    S4 = np.array([124 + (i % 7) for i in range(OUT * IN // 32)], np.uint8)
    yb = oracle.fp4_n(W4, S4, x, OUT, IN, nt=NT)
    ya = np.concatenate([oracle.fp4_n(W4, S4, x[t * IN:(t + 1) * IN], OUT, IN) for t in range(NT)])
    assert np.array_equal(bits(ya), bits(yb))


# -------------------------------------------------------- test_ops.c gates

def test_swiglu_asymmetric_clamp(oracle):
    """test_ops.c:75-122."""
    lim = 10.0
    silu1 = np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-1.0)))
    y = oracle.swiglu(np.array([1.0], np.float32), np.array([-50.0], np.float32), lim)
    assert abs(y[0] - silu1 * -lim) <= 1e-6
    y = oracle.swiglu(np.array([-50.0], np.float32), np.array([1.0], np.float32), lim)
    unclamped = -50.0 / (1.0 + math.exp(50.0))
    if_clamped = -10.0 / (1.0 + math.exp(10.0))
    assert abs(y[0] - unclamped) <= 1e-12 and abs(y[0]) < abs(if_clamped) * 0.5
    y = oracle.swiglu(np.array([50.0, 10.0], np.float32), np.ones(2, np.float32), lim)
    assert y[0] == y[1]
    y = oracle.swiglu(np.array([50.0], np.float32), np.array([50.0], np.float32), 0.0)
    assert abs(y[0] - (50.0 / (1.0 + math.exp(-50.0))) * 50.0) <= 1e-2


def test_fp8_f32_scale_tag_reduces_to_e8m0(oracle):
    """DSV4_WFP8_F32S has no reference counterpart; with power-of-two fp32
    scales it must give exactly the E8M0 result, since only the widened scale
    row differs (src/10_compute/dsv4_matmul_fp8.c:59-64)."""
    rng = np.random.default_rng(3)
    rows, cols = 200, 512
    W = rng.integers(0, 256, rows * cols).astype(np.uint8)
    W[(W & 0x7F) == 0x7F] &= 0xFE
    Sb = rng.integers(118, 136, 2 * 4).astype(np.uint8)
    Sf = np.array([2.0 ** (int(b) - 127) for b in Sb], np.float32)
    x = rng.standard_normal(3 * cols).astype(np.float32)
    assert np.array_equal(bits(oracle.fp8_n(W, Sb, x, rows, cols, nt=3)),
                          bits(oracle.fp8f_n(W, Sf, x, rows, cols, nt=3)))
