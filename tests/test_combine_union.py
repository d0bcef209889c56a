# SPDX-License-Identifier: Apache-2.0
"""Pins for the two pieces the reference's tests leave numerically open
(test_layer.c checks plumbing only): the k-order weighted combine and the
prefill permutation. Known answers are chosen so a wrong order, a weighted
shared expert, or an unstable permutation gives a different result."""
import numpy as np


def test_combine_is_k_order_with_unweighted_shared(oracle):
    d = 4
    # k order: ((0 + 1e8) + 1) + (-1e8) = 0 in fp32; any other order gives 1
    acc = np.array([[1e8] * d, [1.0] * d, [-1e8] * d], np.float32)
    w = np.ones(3, np.float32)
    assert np.all(oracle.moe_combine(acc, w) == 0.0)
    assert np.all(oracle.moe_combine(acc[[1, 0, 2]], w) == 0.0)  # (1+1e8)-1e8 = 0
    assert np.all(oracle.moe_combine(acc[[0, 2, 1]], w) == 1.0)  # (1e8-1e8)+1 = 1
    # the shared output is added unweighted, after the routed sum
    acc = np.array([[2.0] * d, [4.0] * d], np.float32)
    w = np.array([0.5, 0.25], np.float32)
    sh = np.full(d, 3.0, np.float32)
    assert np.all(oracle.moe_combine(acc, w, sh) == 1.0 + 1.0 + 3.0)
    # product and sum separately rounded (no fused multiply-add): after
    # out = -(1 + 2^-11), w*a = (1+2^-12)^2 = 1 + 2^-11 + 2^-24 rounds to
    # 1 + 2^-11 (tie to even) and the sum is 0; a fused form gives 2^-24
    a = np.float32(1 + 2 ** -12)
    acc = np.array([[-(1 + 2 ** -11)], [a]], np.float32)
    w = np.array([1.0, a], np.float32)
    assert oracle.moe_combine(acc, w)[0] == 0.0


def test_union_prepare_counting_sort(oracle):
    rng = np.random.default_rng(5)
    n, topk, ne = 300, 6, 64
    idx = np.stack([rng.choice(ne, topk, replace=False) for _ in range(n)]).astype(np.int32)
    cnt, off, tok, kk, order = oracle.union_prepare(idx, ne)
    assert cnt.sum() == n * topk and off[0] == 0 and off[-1] == n * topk
    for e in range(ne):
        pairs = [(t, k) for t in range(n) for k in range(topk) if idx[t, k] == e]
        assert cnt[e] == len(pairs)
        got = list(zip(tok[off[e]:off[e + 1]], kk[off[e]:off[e + 1]]))
        assert got == pairs  # stable, token-major
    first = []
    for t in range(n):
        for k in range(topk):
            if idx[t, k] not in first:
                first.append(int(idx[t, k]))
    assert list(order) == first
