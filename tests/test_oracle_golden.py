# SPDX-License-Identifier: Apache-2.0
"""The oracle reproduces, bit for bit, every golden fixture that the
reference's own compiled code wrote (tests/golden/make_golden.py): fp8_n and
fp4_n on their fast, tail and generic paths, nt > 1, SwiGLU with and without
the clamp, and one full dsv4_expert_forward."""
import numpy as np
import pytest

from conftest import bits, golden
import pyoracle as P


@pytest.mark.parametrize("name", ["fp8_fast", "fp8_tail", "fp8_generic", "fp8_wide"])
def test_fp8_fixture_bitexact(oracle, name):
    g = golden(name)
    rows, cols, br, bc, nt = (int(v) for v in g["dims"])
    y = oracle.fp8_n(g["W"], g["S"], g["x"], rows, cols, br, bc, nt)
    assert np.array_equal(bits(y), bits(g["y"]))


@pytest.mark.parametrize("name", ["fp4_wide", "fp4_tail", "fp4_generic"])
def test_fp4_fixture_bitexact(oracle, name):
    g = golden(name)
    rows, cols, br, bc, nt = (int(v) for v in g["dims"])
    y = oracle.fp4_n(g["W"], g["S"], g["x"], rows, cols, br, bc, nt)
    assert np.array_equal(bits(y), bits(g["y"]))


def test_swiglu_fixture_bitexact(oracle):
    g = golden("swiglu")
    assert np.array_equal(bits(oracle.swiglu(g["g"], g["u"], 10.0)), bits(g["y10"]))
    assert np.array_equal(bits(oracle.swiglu(g["g"], g["u"], 0.0)), bits(g["y0"]))


def test_expert_fixture_bitexact(oracle):
    g = golden("expert_fp4")
    inter, hidden = (int(v) for v in g["dims"])
    w1 = P.HostMat(P.DSV4_WFP4, g["W1"], g["S1"], inter, hidden, 1, 32)
    w3 = P.HostMat(P.DSV4_WFP4, g["W3"], g["S3"], inter, hidden, 1, 32)
    w2 = P.HostMat(P.DSV4_WFP4, g["W2"], g["S2"], hidden, inter, 1, 32)
    y = oracle.expert_forward(P.HostExpert(w1, w3, w2), g["x"], 10.0)
    assert np.array_equal(bits(y), bits(g["y"]))


def test_mmq_dispatch_matches_bodies(oracle):
    """orc_mmq_n dispatches on wdt exactly like dsv4_mmq_n
    (src/10_compute/dsv4_matmul.c:96-115)."""
    g = golden("fp4_tail")
    rows, cols, br, bc, nt = (int(v) for v in g["dims"])
    m = P.HostMat(P.DSV4_WFP4, g["W"], g["S"], rows, cols, br, bc)
    assert np.array_equal(bits(oracle.mmq_n(m, g["x"], nt)), bits(g["y"]))
    g = golden("fp8_fast")
    rows, cols, br, bc, nt = (int(v) for v in g["dims"])
    m = P.HostMat(P.DSV4_WFP8, g["W"], g["S"], rows, cols, br, bc)
    assert np.array_equal(bits(oracle.mmq_n(m, g["x"], nt)), bits(g["y"]))
    bad = P.HostMat(P.DSV4_WFP8, g["W"], g["S"], rows, cols, br, bc)
    bad.desc.wdt = P.DSV4_WF32  # the reference's dsv4_mmq_n aborts on F32
    with pytest.raises(ValueError):
        oracle.mmq_n(bad, g["x"], 1)
    g = golden("bf16")
    rows, cols, nt = (int(v) for v in g["dims"])
    m = P.HostMat(P.DSV4_WBF16, g["W"], None, rows, cols, 0, 0)
    assert np.array_equal(bits(oracle.mmq_n(m, g["x"], nt)), bits(g["y"]))


def test_bf16_fixture_bitexact(oracle):
    """bf16_n (src/10_compute/dsv4_matmul.c:88-113): whole 16-column steps,
    an 8-column tail, nt = 3, +-0 / subnormal / large bf16 codes."""
    g = golden("bf16")
    rows, cols, nt = (int(v) for v in g["dims"])
    y = oracle.bf16_n(g["W"], g["x"], rows, cols, nt)
    assert np.array_equal(bits(y), bits(g["y"]))


def test_bf16_exact_integer_sums(oracle):
    """With small-integer weights and activations every product and partial
    sum is exact in double, so the result must be the exact dot product: a
    dropped, repeated or misplaced column (step, lane or tail) changes it."""
    rng = np.random.default_rng(7)
    rows, cols, nt = 5, 16 * 7 + 5, 2
    wi = rng.integers(-8, 9, rows * cols).astype(np.float32)
    W = (wi.view(np.uint32) >> 16).astype(np.uint16)        # small integers are exact in bf16
    x = rng.integers(-16, 17, nt * cols).astype(np.float32)
    x += np.arange(nt * cols, dtype=np.float32) % 3        # breaks column symmetry
    y = oracle.bf16_n(W, x, rows, cols, nt)
    want = (x.reshape(nt, cols).astype(np.float64) @ wi.reshape(rows, cols).T.astype(np.float64))
    assert np.array_equal(y.reshape(nt, rows), want.astype(np.float32))


def test_route_fixture_bitexact(oracle):
    """dsv4_route: biased selection, plain selection and hash routing, with
    ties and scores on both sides of softplus's threshold."""
    g = golden("route")
    ntok, ne, topk = (int(v) for v in g["dims"])
    scale = float(g["scale"][0])
    for t in range(ntok):
        i, w, _ = oracle.route(g["scores"][t], topk, scale, bias=g["bias"])
        assert np.array_equal(i, g["idx_b"][t]) and np.array_equal(bits(w), bits(g["w_b"][t])), t
        i, w, _ = oracle.route(g["scores"][t], topk, scale)
        assert np.array_equal(i, g["idx_n"][t]) and np.array_equal(bits(w), bits(g["w_n"][t])), t
    for t in range(16):
        i, w, _ = oracle.route(g["scores"][t], topk, scale, tid2eid=g["tid2eid"], token_id=t)
        assert np.array_equal(i, g["idx_h"][t]) and np.array_equal(bits(w), bits(g["w_h"][t])), t


def test_route_closed_forms(oracle):
    """What the router's definition fixes: the picks are the top-k of the
    biased scores in descending order with ties to the lower index (a stable
    sort), the weights are the unbiased sqrt(softplus) of the picks summing to
    route_scale, and the bias moves only the selection."""
    rng = np.random.default_rng(9)
    for t in range(50):
        sc = (rng.standard_normal(256) * 3).astype(np.float32)
        sc[rng.integers(0, 256, 8)] = sc[3]                       # ties
        bias = (rng.standard_normal(256) * 0.2).astype(np.float32)
        idx, w, orig = oracle.route(sc, 6, 1.5, bias=bias)
        sp = np.where(sc > 20, sc, np.log1p(np.exp(sc.astype(np.float64)))).astype(np.float32)
        assert np.allclose(orig, np.sqrt(sp), rtol=1e-6)
        biased = orig + bias
        want = np.argsort(-biased, kind="stable")[:6]
        assert np.array_equal(idx, want)
        assert abs(float(w.astype(np.float64).sum()) - 1.5) < 1e-5
        assert np.allclose(w, orig[idx] / orig[idx].astype(np.float64).sum() * 1.5, rtol=1e-6)
