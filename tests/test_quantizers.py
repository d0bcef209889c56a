# SPDX-License-Identifier: Apache-2.0
"""Pins for the quantizers, which have no counterpart in the reference (it
ships pre-quantized weights and never quantizes activations). Each rule is
checked against an independent authority: torch's float8_e4m3fn / bfloat16
casts (round to nearest even), a brute-force nearest search over the 16-entry
e2m1 grid, and the closed-form conditions the scale rules must satisfy."""
import math

import numpy as np
import pytest
import torch


def _e2m1_val(code):
    mag = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0][code & 7]
    return -mag if code & 8 else mag


def test_e4m3_matches_torch_rne(oracle):
    rng = np.random.default_rng(11)
    vals = np.concatenate([
        rng.uniform(-448, 448, 20000),
        rng.standard_normal(20000) * 0.01,
        rng.standard_normal(5000) * 2.0 ** -8,
    ]).astype(np.float32)
    # every midpoint between adjacent finite e4m3 values: ties to even
    pos = sorted({oracle.e4m3(b) for b in range(0x7F)})
    mids = np.array([(a + b) / 2 for a, b in zip(pos[:-1], pos[1:])], np.float32)
    vals = np.concatenate([vals, mids, -mids, np.array(pos, np.float32)])
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.f32_to_e4m3(v) for v in vals], np.uint8)
    assert np.array_equal(got, want)


def test_e4m3_saturates_and_roundtrips(oracle):
    assert oracle.f32_to_e4m3(1e9) == 0x7E and oracle.f32_to_e4m3(-1e9) == 0xFE
    assert oracle.f32_to_e4m3(463.9) == 0x7E
    for b in range(256):
        if (b & 0x7F) == 0x7F:
            continue
        assert oracle.f32_to_e4m3(oracle.e4m3(b)) == b


def test_e2m1_bruteforce_nearest_even(oracle):
    rng = np.random.default_rng(12)
    vals = np.concatenate([rng.uniform(-8, 8, 20000),
                           np.arange(-7.0, 7.0, 0.125)]).astype(np.float32)
    mags = [_e2m1_val(c) for c in range(8)]
    for v in vals:
        code = oracle.f32_to_e2m1(v)
        a = min(abs(float(v)), 6.0)
        # nearest magnitude; on a tie the even code (mantissa bit 0) wins
        best = min(range(8), key=lambda c: (abs(mags[c] - a), c & 1))
        assert (code & 7) == best, (v, code, best)
        assert (code & 8) == (8 if math.copysign(1, v) < 0 else 0)


def test_fp4_mx_scale_rule_and_error(oracle):
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :32] *= 1e-30
    W, S = oracle.quant_fp4_mx(w)
    for r in range(w.shape[0]):
        for b in range(w.shape[1] // 32):
            blk = w[r, b * 32:(b + 1) * 32].astype(np.float64)
            amax = np.max(np.abs(blk))
            e = int(S[r * 8 + b]) - 127
            if amax == 0:
                assert e == 0
                continue
            if 127 + e not in (0, 254):
                assert 6 * 2.0 ** e >= amax and 6 * 2.0 ** (e - 1) < amax
            by = W[r * 128 + b * 16:r * 128 + b * 16 + 16]
            codes = np.stack([by & 15, by >> 4], 1).reshape(-1)
            deq = np.array([_e2m1_val(int(c)) for c in codes]) * 2.0 ** e
            # each element is the nearest grid point: error <= half the local step
            assert np.all(np.abs(deq - blk) <= 2.0 ** e + 1e-300)


def test_fp8_blk128_matches_torch(oracle):
    rng = np.random.default_rng(14)
    w = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    W, S = oracle.quant_fp8_blk128(w)
    for rb in range(2):
        for cb in range(3):
            blk = w[rb * 128:(rb + 1) * 128, cb * 128:(cb + 1) * 128]
            s = np.float32(np.max(np.abs(blk))) / np.float32(448.0)
            assert S[rb * 3 + cb] == s
            q = torch.from_numpy(blk / s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            got = W.reshape(256, 384)[rb * 128:(rb + 1) * 128, cb * 128:(cb + 1) * 128]
            assert np.array_equal(got, q)


def test_act_fp8_1x128_matches_torch(oracle):
    rng = np.random.default_rng(15)
    a = torch.randn(5, 512, generator=torch.Generator().manual_seed(1)).bfloat16().float().numpy()
    a[2, :128] = 0.0
    Q, S = oracle.quant_act_fp8_1x128(a)
    S = S.reshape(5, 4)
    for t in range(5):
        for g in range(4):
            grp = a[t, g * 128:(g + 1) * 128]
            amax = np.float32(np.max(np.abs(grp)))
            s = amax / np.float32(448.0) if amax > 0 else np.float32(1.0)
            assert S[t, g] == s
            q = torch.from_numpy(grp / s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(Q.reshape(5, 512)[t, g * 128:(g + 1) * 128], q)


def test_act_mxfp8_scale_rule(oracle):
    rng = np.random.default_rng(16)
    a = rng.standard_normal((7, 256)).astype(np.float32) * 3
    Q, S = oracle.quant_act_mxfp8(a)
    for t in range(7):
        for g in range(8):
            grp = a[t, g * 32:(g + 1) * 32].astype(np.float64)
            amax = np.max(np.abs(grp))
            e = int(S[t * 8 + g]) - 127
            assert 448 * 2.0 ** e >= amax and 448 * 2.0 ** (e - 1) < amax
            scaled = torch.from_numpy((grp * 2.0 ** -e).astype(np.float32))
            q = scaled.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(Q.reshape(7, 256)[t, g * 32:(g + 1) * 32], q)


def test_bf16_matches_torch(oracle):
    rng = np.random.default_rng(17)
    v = np.concatenate([rng.standard_normal(5000).astype(np.float32),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8], np.float32)])
    want = torch.from_numpy(v).bfloat16().view(torch.uint16).numpy().astype(np.uint16)
    got = np.array([oracle.f32_to_bf16(x) for x in v], np.uint16)
    assert np.array_equal(got, want)
