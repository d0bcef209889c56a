# SPDX-License-Identifier: Apache-2.0
"""Write the golden fixtures under tests/golden/ from the reference's own
hot-path code, compiled unchanged from its sources into oracle/_ref by
oracle/Makefile (needs the reference tree; run in the container that has it):

    make -C oracle ref && python tests/golden/make_golden.py

Each fixture is a small .npz of seeded inputs and the reference's outputs for
fp8_n / fp4_n (src/10_compute/dsv4_matmul_fp8.c:49-177,
dsv4_matmul_fp4.c:46-162), dsv4_swiglu (src/10_compute/dsv4_ops.c:61-79) and
dsv4_expert_forward (dsv4_ops.c:85-93), covering the 128x128 fast path, the
tail blocks, the generic geometry, nt > 1, and special e4m3 codes.
The inputs are generated here with numpy (seeded); no reference source is
stored, only data.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import pyoracle as P  # noqa: E402


def normal_e4m3(rng, n):
    """Random normal e4m3 codes (exponent 1..14), as the reference's
    normal-only gate builds them (tests/unit/test_matmul.c:655-661)."""
    e = rng.integers(1, 15, n)
    m = rng.integers(0, 8, n)
    s = rng.integers(0, 2, n)
    return ((s << 7) | (e << 3) | m).astype(np.uint8)


def any_e4m3_finite(rng, n):
    b = rng.integers(0, 256, n).astype(np.uint8)
    b[(b & 0x7F) == 0x7F] &= 0xFE
    return b


def main():
    R = P.Reference()
    rng = np.random.default_rng(20260412)
    out = {}

    def save(name, **arrs):
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **arrs)
        h = hashlib.sha256()
        for k in sorted(arrs):
            h.update(k.encode())
            h.update(np.ascontiguousarray(arrs[k]).tobytes())
        out[name] = h.hexdigest()[:16]

    # FP8 128x128 fast path, nt = 3, one block forced to the exact gather path.
    rows, cols, nt = 256, 512, 3
    W = normal_e4m3(rng, rows * cols)
    W[0], W[1], W[2], W[3] = 0x01, 0x00, 0x80, 0x06  # subnormal, +-0
    S = rng.integers(118, 134, P.fp8_scale_grid(rows, cols, 128, 128)).astype(np.uint8)
    x = (rng.standard_normal(nt * cols)).astype(np.float32)
    save("fp8_fast", W=W, S=S, x=x, dims=np.array([rows, cols, 128, 128, nt]),
         y=R.fp8_n(W, S, x, rows, cols, 128, 128, nt))

    # FP8 with three 128-blocks per row: one tail block past the 4-group loop.
    rows, cols, nt = 37, 384, 2
    W = any_e4m3_finite(rng, rows * cols)
    S = rng.integers(120, 132, P.fp8_scale_grid(rows, cols, 128, 128)).astype(np.uint8)
    x = (rng.standard_normal(nt * cols) * 0.5).astype(np.float32)
    save("fp8_tail", W=W, S=S, x=x, dims=np.array([rows, cols, 128, 128, nt]),
         y=R.fp8_n(W, S, x, rows, cols, 128, 128, nt))

    # FP8 generic geometry: blk_c = 100 (256 = 100 + 100 + 56), blk_r = 128.
    rows, cols, nt = 37, 256, 1
    W = any_e4m3_finite(rng, rows * cols)
    S = np.full(P.fp8_scale_grid(rows, cols, 128, 100), 127, np.uint8)
    x = (rng.standard_normal(cols)).astype(np.float32)
    save("fp8_generic", W=W, S=S, x=x, dims=np.array([rows, cols, 128, 100, nt]),
         y=R.fp8_n(W, S, x, rows, cols, 128, 100, nt))

    # FP8 4096-wide rows: the cross-block fold over 32 blocks (two full passes
    # of the four accumulator slots).
    rows, cols, nt = 16, 4096, 1
    W = normal_e4m3(rng, rows * cols)
    S = rng.integers(118, 134, P.fp8_scale_grid(rows, cols, 128, 128)).astype(np.uint8)
    x = (rng.standard_normal(cols)).astype(np.float32)
    save("fp8_wide", W=W, S=S, x=x, dims=np.array([rows, cols, 128, 128, nt]),
         y=R.fp8_n(W, S, x, rows, cols, 128, 128, nt))

    # FP4 fast path at Flash width (128 blocks of 32), nt = 2.
    rows, cols, nt = 64, 4096, 2
    W = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    S = rng.integers(118, 134, rows * cols // 32).astype(np.uint8)
    x = (rng.standard_normal(nt * cols)).astype(np.float32)
    save("fp4_wide", W=W, S=S, x=x, dims=np.array([rows, cols, 1, 32, nt]),
         y=R.fp4_n(W, S, x, rows, cols, 1, 32, nt))

    # FP4 with a tail block (160 = one four-block group + one block).
    rows, cols, nt = 9, 160, 3
    W = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    S = rng.integers(120, 132, rows * cols // 32).astype(np.uint8)
    x = (rng.standard_normal(nt * cols)).astype(np.float32)
    save("fp4_tail", W=W, S=S, x=x, dims=np.array([rows, cols, 1, 32, nt]),
         y=R.fp4_n(W, S, x, rows, cols, 1, 32, nt))

    # FP4 generic geometry: blk_c = 64.
    rows, cols, nt = 9, 160, 1
    W = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    S = rng.integers(120, 132, rows * ((cols + 63) // 64)).astype(np.uint8)
    x = (rng.standard_normal(cols)).astype(np.float32)
    save("fp4_generic", W=W, S=S, x=x, dims=np.array([rows, cols, 1, 64, nt]),
         y=R.fp4_n(W, S, x, rows, cols, 1, 64, nt))

    # SwiGLU with the asymmetric clamp and with the clamp disabled.
    g = (rng.standard_normal(4096) * 8).astype(np.float32)
    u = (rng.standard_normal(4096) * 8).astype(np.float32)
    g[:6] = [-50.0, 50.0, 10.0, -10.0, 0.0, -0.0]
    u[:6] = [1.0, 1.0, -50.0, 50.0, 3.0, -3.0]
    save("swiglu", g=g, u=u, y10=R.swiglu(g, u, 10.0), y0=R.swiglu(g, u, 0.0))

    # One small FP4 expert through dsv4_expert_forward (inter 64, hidden 256).
    inter, hidden = 64, 256
    mats = []
    for (r, c) in ((inter, hidden), (inter, hidden), (hidden, inter)):
        Wm = rng.integers(0, 256, r * c // 2).astype(np.uint8)
        Sm = rng.integers(121, 128, r * c // 32).astype(np.uint8)
        mats.append(P.HostMat(P.DSV4_WFP4, Wm, Sm, r, c, 1, 32))
    ex = P.HostExpert(*mats)
    x = (rng.standard_normal(hidden)).astype(np.float32)
    save("expert_fp4", W1=mats[0].W, S1=mats[0].S, W3=mats[1].W, S3=mats[1].S,
         W2=mats[2].W, S2=mats[2].S, x=x, dims=np.array([inter, hidden]),
         y=R.expert_forward(ex, x, 10.0))

    # BF16 (bf16_n, src/10_compute/dsv4_matmul.c:88-113): 4136 columns = 258
    # whole 16-column steps + an 8-column tail, nt = 3; bf16 values from
    # N(0, 0.02) rounded to nearest even, plus +-0, a subnormal and large
    # magnitudes in row 0.
    rows, cols, nt = 70, 4136, 3
    f = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    u = f.view(np.uint32)
    Wb = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    Wb[:6] = [0x0000, 0x8000, 0x0001, 0x7F7F, 0xFF7F, 0x3F80]
    x = (rng.standard_normal(nt * cols)).astype(np.float32)
    x[:6] = [1.0, 1.0, 3.0, 1e-30, 1e-30, -2.0]
    save("bf16", W=Wb, x=x, dims=np.array([rows, cols, nt]), y=R.bf16_n(Wb, x, rows, cols, nt))

    # dsv4_route (src/10_compute/dsv4_ops.c:117-157) over 64 tokens x 256
    # experts: raw gate outputs from -30 to 30 (both sides of softplus's
    # threshold 20), a selection bias, exact ties (duplicated scores; ties go
    # to the lower index), and a hash-routed (tid2eid) call.
    rr = np.random.default_rng(7311)
    ntok, ne, topk, scale = 64, 256, 6, 1.5
    sc = (rr.standard_normal((ntok, ne)) * 4.0).astype(np.float32)
    sc[0, :] = rr.uniform(-30, 30, ne).astype(np.float32)
    sc[1, 10:20] = sc[1, 5]                            # ties
    sc[2, :] = 1.0                                     # all equal
    bias = (rr.standard_normal(ne) * 0.1).astype(np.float32)
    idx_b = np.zeros((ntok, topk), np.int32); w_b = np.zeros((ntok, topk), np.float32)
    idx_n = np.zeros((ntok, topk), np.int32); w_n = np.zeros((ntok, topk), np.float32)
    for t in range(ntok):
        idx_b[t], w_b[t], _ = R.route(sc[t], topk, scale, bias=bias)
        idx_n[t], w_n[t], _ = R.route(sc[t], topk, scale)
    tid2eid = rr.integers(0, ne, (16, topk)).astype(np.int64)
    idx_h = np.zeros((16, topk), np.int32); w_h = np.zeros((16, topk), np.float32)
    for t in range(16):
        idx_h[t], w_h[t], _ = R.route(sc[t], topk, scale, tid2eid=tid2eid, token_id=t)
    save("route", scores=sc, bias=bias, tid2eid=tid2eid, dims=np.array([ntok, ne, topk]),
         scale=np.array([scale], np.float32), idx_b=idx_b, w_b=w_b, idx_n=idx_n, w_n=w_n,
         idx_h=idx_h, w_h=w_h)

    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump({"source": "oracle/_ref/libdsv4ref.so built by oracle/Makefile",
                   "sha256_16": out}, f, indent=1, sort_keys=True)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
