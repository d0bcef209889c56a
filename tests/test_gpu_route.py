# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the device router (dsv4_hip_route_dev) and of the decode
step's MoE block on the device (dsv4_hip_moe_layer_dev: gate matvec, router,
routed experts and shared expert with no host round trip).

The router's fixture comes from the reference's own dsv4_route compiled from
its sources (src/10_compute/dsv4_ops.c:117-157); the edge cases run through
the oracle's restatement, which that fixture pins. Tolerances: none for the
index work. ids, orig = sqrtf(softplus(score)) and the weights are bit for
bit the reference's (the device restates glibc's expf and log1pf operation
for operation; the host check of that restatement over every fp32 input is
tests/test_route_math.py), and so are the BF16 gate's scores (bf16_n's fp64
sums in the same order). The MoE block's output is within 1e-4 relative L2
of the oracle's pipeline (FP4/FP8 expert arithmetic in another order)."""
import zlib

import numpy as np
import pytest
import torch

import pyoracle as P
from conftest import bits, golden
from test_gpu_decode import DEV, bf16_x, check_close, dev_f32
from test_gpu_decode_one import _host_slot_expert

pytestmark = pytest.mark.gpu


def _assert_bits(got, want, what):
    """fp32 arrays equal bit for bit (any NaN matching any NaN)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), f"{what}: NaN pattern"
    diff = np.nonzero(bits(got[~nan]) != bits(want[~nan]))[0]
    assert diff.size == 0, f"{what}: {diff.size} values differ, first {got[~nan][diff[0]]!r} vs {want[~nan][diff[0]]!r}"


def _assert_ids(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{what}: id {got[tuple(bad[0])]} vs {want[tuple(bad[0])]} at {tuple(bad[0])}"


def _route_gpu(lib, scores, topk, scale, bias=None, tid2eid=None, tokens=None, n_vocab=0):
    n, ne = scores.shape
    ds = dev_f32(scores)
    di = torch.full((n * topk,), -7, dtype=torch.int32, device=DEV)
    dw = torch.empty(n * topk, dtype=torch.float32, device=DEV)
    do = torch.empty(n * ne, dtype=torch.float32, device=DEV)
    db = dev_f32(bias) if bias is not None else None
    dt = torch.from_numpy(np.ascontiguousarray(tid2eid, np.int64).reshape(-1)).to(DEV) \
        if tid2eid is not None else None
    dk = torch.from_numpy(np.ascontiguousarray(tokens, np.int32)).to(DEV) if tokens is not None else None
    lib.route_dev(di.data_ptr(), dw.data_ptr(), do.data_ptr(), ds.data_ptr(), n, ne, topk, scale,
                  bias_ptr=db.data_ptr() if db is not None else None,
                  tid2eid_ptr=dt.data_ptr() if dt is not None else None, n_vocab=n_vocab,
                  token_ids_ptr=dk.data_ptr() if dk is not None else None)
    torch.cuda.synchronize()
    return (di.cpu().numpy().reshape(n, topk), dw.cpu().numpy().reshape(n, topk),
            do.cpu().numpy().reshape(n, ne))


def test_route_golden_fixture(lib, oracle):
    """64 tokens x 256 experts from the compiled reference: biased selection,
    plain selection and hash routing; ids, weights and orig bit for bit."""
    g = golden("route")
    ntok, ne, topk = (int(v) for v in g["dims"])
    scale = float(g["scale"][0])
    sc, bias = g["scores"], g["bias"]
    lib.status()
    orig_o = np.stack([oracle.route(sc[t], topk, scale)[2] for t in range(ntok)])
    i, w, o = _route_gpu(lib, sc, topk, scale, bias=bias)
    _assert_bits(o, orig_o, "orig")
    _assert_ids(i, g["idx_b"], "biased")
    _assert_bits(w, g["w_b"], "biased")
    i, w, _ = _route_gpu(lib, sc, topk, scale)
    _assert_ids(i, g["idx_n"], "plain")
    _assert_bits(w, g["w_n"], "plain")
    i, w, _ = _route_gpu(lib, sc[:16], topk, scale, tid2eid=g["tid2eid"], tokens=np.arange(16),
                         n_vocab=16)
    _assert_ids(i, g["idx_h"], "hash")
    _assert_bits(w, g["w_h"], "hash")
    assert lib.status() == 0


def _edge_cases():
    rng = np.random.default_rng(zlib.crc32(b"route-edges"))
    cases = []
    ne = 256
    cases.append(("all equal", np.full((2, ne), 0.37, np.float32), None, 6, 1.0))
    s = rng.standard_normal((4, ne)).astype(np.float32)
    s[0, 0] = np.nan                                # first untaken is NaN: kept
    s[1, [0, 1, 2]] = np.nan                        # three leading NaNs
    s[2, rng.integers(1, ne, 9)] = np.nan           # NaNs inside: never picked
    s[3, :] = np.nan                                # all NaN
    cases.append(("NaN", s, None, 6, 1.0))
    s = rng.standard_normal((3, ne)).astype(np.float32)
    s[0, [3, 50, 200]] = np.inf
    s[1, :40] = -np.inf
    s[2, ::3] = 25.0                                # above softplus's threshold, tied
    s[2, 1::7] = 19.999998
    cases.append(("inf and threshold", s, None, 8, 2.5))
    s = np.repeat(rng.standard_normal((1, 32)).astype(np.float32), 8, axis=0).reshape(1, ne)
    s = np.concatenate([s, np.round(rng.standard_normal((3, ne)) * 2, 1).astype(np.float32)])
    b = np.round(rng.standard_normal(ne) * 0.5, 1).astype(np.float32)
    b[::5] = -np.inf
    cases.append(("ties with bias", s, b, 6, 1.5))
    cases.append(("1024 experts top 16", (rng.standard_normal((3, 1024)) * 4).astype(np.float32),
                  (rng.standard_normal(1024) * 0.1).astype(np.float32), 16, 2.5))
    cases.append(("topk == n_experts", rng.standard_normal((2, 16)).astype(np.float32), None, 16, 1.0))
    cases.append(("300 experts", rng.standard_normal((5, 300)).astype(np.float32),
                  (rng.standard_normal(300) * 0.3).astype(np.float32), 8, 1.0))
    cases.append(("one expert", rng.standard_normal((2, 1)).astype(np.float32), None, 1, 3.0))
    s = np.full((1, ne), -200.0, np.float32)         # orig 0 everywhere: weights 0
    cases.append(("zero sum", s, None, 6, 1.0))
    return cases


@pytest.mark.parametrize("case", _edge_cases(), ids=lambda c: c[0])
def test_route_edges(lib, oracle, case):
    """NaN (first untaken kept, others skipped), infinities, the softplus
    threshold, exact ties with and without a bias (-inf included), 1 to 1024
    experts, topk up to 16 and topk == n_experts, a zero weight sum: ids and
    weights bit for bit as the oracle's loop gives them."""
    name, sc, bias, topk, scale = case
    lib.status()
    i, w, o = _route_gpu(lib, sc, topk, scale, bias=bias)
    want = [oracle.route(sc[t], topk, scale, bias=bias) for t in range(sc.shape[0])]
    wi = np.stack([r[0] for r in want])
    ww = np.stack([r[1] for r in want])
    wo = np.stack([r[2] for r in want])
    _assert_bits(o, wo, name)
    _assert_ids(i, wi, name)
    _assert_bits(w, ww, name)
    assert lib.status() == 0


def test_route_orig_every_input(lib):
    """orig of dsv4_hip_route_dev for every fp32 score in [-104, 20] (2.2e9
    inputs, 1024 experts a token, 2^24 a call) against per-chunk checksums of
    glibc's sqrtf(log1pf(expf(x))) (tests/golden/route_orig.npz, written by
    make_route_orig.py): every chunk's two sums equal."""
    g = golden("route_orig")
    chunk, n_neg, n_pos = 1 << int(g["chunk_log2"]), int(g["n_neg"]), int(g["n_pos"])
    total = n_neg + n_pos
    ne = 1024
    di = torch.empty(chunk // ne, dtype=torch.int32, device=DEV)
    dw = torch.empty(chunk // ne, dtype=torch.float32, device=DEV)
    do = torch.empty(chunk, dtype=torch.float32, device=DEV)
    pos = torch.arange(chunk, dtype=torch.int64, device=DEV)
    w64 = pos & 63
    lib.status()
    bad = []
    for c in range(len(g["s1"])):
        cnt = min(chunk, total - c * chunk)
        i = pos[:cnt] + c * chunk
        u = torch.where(i < n_neg, 0x80000000 + i, i - n_neg)
        u = torch.where(u >= 1 << 31, u - (1 << 32), u).to(torch.int32)
        sc = torch.zeros(-(-cnt // ne) * ne, dtype=torch.int32, device=DEV)
        sc[:cnt] = u
        n = sc.numel() // ne
        lib.route_dev(di.data_ptr(), dw.data_ptr(), do.data_ptr(), sc.data_ptr(), n, ne, 1, 1.0)
        ob = do[:cnt].view(torch.int32).to(torch.int64)
        s1, s2 = int(ob.sum()), int((ob * w64[:cnt]).sum())
        if s1 != int(g["s1"][c]) or s2 != int(g["s2"][c]):
            bad.append(c)
    torch.cuda.synchronize()
    assert lib.status() == 0
    assert not bad, f"chunks {bad[:8]} differ ({len(bad)} of {len(g['s1'])})"


def test_route_bad_ids_raise_status(lib, oracle):
    """A token id outside the hash table, or a table entry outside the experts:
    status bit 0, NaN weights, the ids written as they are (-1 for the token)."""
    rng = np.random.default_rng(5)
    sc = rng.standard_normal((3, 64)).astype(np.float32)
    t2e = np.stack([rng.choice(64, 4, replace=False) for _ in range(8)]).astype(np.int64)
    t2e[5, 2] = 64
    lib.status()
    i, w, _ = _route_gpu(lib, sc, 4, 1.0, tid2eid=t2e, tokens=np.array([1, 8, 5]), n_vocab=8)
    assert lib.status() & 1
    assert np.array_equal(i[0], t2e[1]) and np.all(np.isfinite(w[0]))
    assert np.array_equal(i[1], [-1] * 4) and np.all(np.isnan(w[1]))
    assert np.array_equal(i[2], t2e[5]) and np.all(np.isnan(w[2]))
    assert lib.status() == 0


def test_route_rejects_bad_arguments(lib):
    """Sizes the kernel does not take are refused before any launch."""
    d = torch.zeros(4096, dtype=torch.float32, device=DEV)
    p = d.data_ptr()
    for ne, topk in ((1025, 6), (256, 17), (8, 9), (0, 1)):
        with pytest.raises(Exception):
            lib.route_dev(p, p, None, p, 1, ne, topk, 1.0)
    with pytest.raises(Exception):          # hash routing without token ids
        lib.route_dev(p, p, None, p, 1, 64, 4, 1.0, tid2eid_ptr=p, n_vocab=4)
    lib.route_dev(p, p, None, p, 0, 64, 4, 1.0)       # n == 0: nothing to do
    torch.cuda.synchronize()


class _Layer:
    """One decode MoE block at the released shape: BF16 gate [256 x 4096], a
    bias, 256 FP4 experts [2048 x 4096] in one device arena, the FP8 shared
    expert, top-6."""

    def __init__(self, pkg, lib, seed, gate_fmt="bf16"):
        import bench
        self.hidden, self.inter, self.ne, self.topk, self.scale = 4096, 2048, 256, 6, 2.5
        rng = np.random.default_rng(seed)
        self.arena = bench.ExpertArena(torch, pkg, lib, self.ne, seed=seed)
        self.shared, self.skeep = bench.make_shared_fp8(torch, pkg, lib, seed + 1)
        g32 = (rng.standard_normal((self.ne, self.hidden)) * 0.02).astype(np.float32)
        if gate_fmt == "bf16":
            W16 = (g32.view(np.uint32) >> 16).astype(np.uint16)   # bf16 by truncation
            self.gkeep = [torch.from_numpy(W16.view(np.int16).reshape(-1).copy()).to(DEV)]
            self.gate = pkg.qmat(pkg.DSV4_WBF16, self.gkeep[0].data_ptr(), None, self.ne,
                                 self.hidden, 0, 0)
            self.hgate = P.HostMat(P.DSV4_WBF16, W16, None, self.ne, self.hidden, 0, 0)
        else:
            W, S = P.Oracle().quant_fp8_blk128(g32)
            self.gkeep = [torch.from_numpy(np.ascontiguousarray(W, np.uint8).reshape(-1)).to(DEV),
                          dev_f32(S)]
            self.gate = pkg.qmat(pkg.DSV4_WFP8_F32S, self.gkeep[0].data_ptr(),
                                 self.gkeep[1].data_ptr(), self.ne, self.hidden, 128, 128)
            self.hgate = P.HostMat(P.DSV4_WFP8_F32S, W, S, self.ne, self.hidden, 128, 128)
        self.bias = (rng.standard_normal(self.ne) * 0.05).astype(np.float32)
        self.dbias = dev_f32(self.bias)
        self.t2e = np.stack([rng.choice(self.ne, self.topk, replace=False)
                             for _ in range(32)]).astype(np.int64)
        self.dt2e = torch.from_numpy(self.t2e.reshape(-1)).to(DEV)
        I, H = self.inter, self.hidden
        self.hshared = P.HostExpert(*[P.HostMat(P.DSV4_WFP8_F32S, self.skeep[2 * i].cpu().numpy(),
                                                self.skeep[2 * i + 1].cpu().numpy(), r, c, 128, 128)
                                      for i, (r, c) in enumerate(((I, H), (I, H), (H, I)))])
        self._host = {}

    def run(self, lib, x, out, idx, w, hash_tok=None, stream=None):
        lib.moe_layer_dev(out.data_ptr(), x.data_ptr(), self.gate, self.arena.table.data_ptr(),
                          self.ne, self.topk, self.scale, self.shared, self.hidden, self.inter, 10.0,
                          bias_ptr=None if hash_tok is not None else self.dbias.data_ptr(),
                          tid2eid_ptr=self.dt2e.data_ptr() if hash_tok is not None else None,
                          n_vocab=len(self.t2e), token_id=hash_tok or 0,
                          idx_ptr=idx.data_ptr(), w_ptr=w.data_ptr(), stream=stream)

    def expert(self, e):
        if e not in self._host:
            self._host[e] = _host_slot_expert(self.arena.host_copy(torch, e))
        return self._host[e]

    def want(self, oracle, xh, idx, w):
        acc = np.stack([oracle.expert_forward(self.expert(int(e)), xh, 10.0) for e in idx])
        return (oracle.moe_combine(acc, w) + oracle.expert_forward(self.hshared, xh, 10.0)).astype(np.float32)


@pytest.mark.parametrize("hash_tok,gate_fmt", [(None, "bf16"), (17, "bf16"), (None, "fp8")])
def test_moe_layer_matches_oracle_pipeline(lib, pkg, oracle, hash_tok, gate_fmt):
    """The device block against the reference's sequence run by the oracle:
    gate scores (dsv4_mmq: bf16_n with fp64 sums bit for bit, or the FP8
    matvec within 1e-4 relative L2), the router's picks and weights bit for bit
    as dsv4_route gives them on the oracle's scores (BF16 gate) or the
    device's (FP8 gate), and the block's output within 1e-4
    relative L2 of the oracle's experts combined in k order plus the shared
    expert. Biased routing and hash routing (token 17); the BF16 gate runs
    fused with the router, the FP8 gate through the matvec kernels first."""
    L = _Layer(pkg, lib, (zlib.crc32(b"layer") & 0xFFFF) + len(gate_fmt), gate_fmt)
    lib.status()
    for seed in (3, 4):
        xh = bf16_x(seed, L.hidden)
        x = dev_f32(xh)
        out = torch.empty(L.hidden, dtype=torch.float32, device=DEV)
        di = torch.empty(L.topk, dtype=torch.int32, device=DEV)
        dw = torch.empty(L.topk, dtype=torch.float32, device=DEV)
        L.run(lib, x, out, di, dw, hash_tok)
        sc = torch.empty(L.ne, dtype=torch.float32, device=DEV)
        lib.mmq_n_dev(sc.data_ptr(), x.data_ptr(), L.gate, 1)
        torch.cuda.synchronize()
        assert lib.status() == 0
        sc_o = oracle.mmq_n(L.hgate, xh)
        if gate_fmt == "bf16":
            _assert_bits(sc.cpu().numpy(), sc_o, "gate scores")
        else:
            check_close(sc.cpu().numpy(), sc_o, 1e-4)
        # the router on the device's scores: the oracle's for the BF16 gate;
        # the FP8 matvec sums in another order than fp8_n
        bias = None if hash_tok is not None else L.bias
        wi, ww, wo = oracle.route(sc.cpu().numpy(), L.topk, L.scale, bias=bias,
                                  tid2eid=L.t2e if hash_tok is not None else None,
                                  token_id=hash_tok or 0)
        gi, gw = di.cpu().numpy(), dw.cpu().numpy()
        _assert_ids(gi, wi, "layer")
        _assert_bits(gw, ww, "layer")
        check_close(out.cpu().numpy(), L.want(oracle, xh, gi, gw), 1e-4)


def test_moe_layer_graph_replays(lib, pkg, oracle):
    """The whole block captured once in a HIP graph and replayed for four
    tokens (new x copied in between, synchronised): output, ids and weights
    of every replay bit for bit the eager call's, status clean."""
    L = _Layer(pkg, lib, 0x6A7E)
    xs = [bf16_x(70 + i, L.hidden) for i in range(4)]
    out = torch.empty(L.hidden, dtype=torch.float32, device=DEV)
    di = torch.empty(L.topk, dtype=torch.int32, device=DEV)
    dw = torch.empty(L.topk, dtype=torch.float32, device=DEV)
    x = dev_f32(xs[0])
    st = torch.cuda.Stream()
    want = []
    lib.status()
    for xh in xs:
        x.copy_(torch.from_numpy(xh))
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            L.run(lib, x, out, di, dw, stream=st.cuda_stream)
        torch.cuda.synchronize()
        want.append((bits(out.cpu().numpy()), di.cpu().numpy().copy(), bits(dw.cpu().numpy())))
    assert lib.status() == 0
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        L.run(lib, x, out, di, dw, stream=st.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        for i, xh in enumerate(xs):
            x.copy_(torch.from_numpy(xh))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(out.cpu().numpy()), want[i][0]), f"replay {rep} token {i}"
            assert np.array_equal(di.cpu().numpy(), want[i][1])
            assert np.array_equal(bits(dw.cpu().numpy()), want[i][2])
    assert lib.status() == 0
    check_close(out.cpu().numpy(), L.want(oracle, xs[-1], want[-1][1], want[-1][2].view(np.float32)), 1e-4)


def test_moe_layer_rejects_bad_gate(lib, pkg):
    """A gate whose shape is not [n_experts x hidden] is refused on the host,
    before anything is launched."""
    d = torch.zeros(1 << 20, dtype=torch.float32, device=DEV)
    p = d.data_ptr()
    gate = pkg.qmat(pkg.DSV4_WBF16, p, None, 128, 4096, 0, 0)
    with pytest.raises(Exception, match="gate"):
        lib.moe_layer_dev(p, p, gate, p, 256, 6, 1.0, None, 4096, 2048, 10.0)
    torch.cuda.synchronize()


@pytest.mark.parametrize("ne,hidden,topk", [(64, 1024, 8), (300, 2048, 6), (1024, 512, 16), (8, 4096, 8),
                                           (16, 8192, 4)])
def test_fused_gate_router_shapes(lib, pkg, oracle, ne, hidden, topk):
    """The fused gate matvec + router launch at other geometries (1 to 16
    experts per lane, 1 to 8 row chunks per lane, 8 to 1024 workgroups), and
    a gate too wide for it (8192 columns: the BF16 matvec, then the router):
    the picks and weights of `dsv4_hip_moe_layer_dev` against dsv4_route on
    the oracle's bf16_n scores, bit for bit, over four
    tokens in a row so the arrival counters' reset is exercised; small FP4
    experts behind it."""
    rng = np.random.default_rng(ne * 7 + hidden)
    inter = 256
    descs, host, keep = [], [], []
    for _ in range(ne):
        q, hm = [], []
        for (r, c) in ((inter, hidden), (inter, hidden), (hidden, inter)):
            W, S = oracle.quant_fp4_mx((rng.standard_normal((r, c)) * 0.02).astype(np.float32))
            dW, dS = (torch.from_numpy(np.ascontiguousarray(a, np.uint8).reshape(-1)).to(DEV) for a in (W, S))
            keep += [dW, dS]
            q.append(pkg.qmat(pkg.DSV4_WFP4, dW.data_ptr(), dS.data_ptr(), r, c, 1, 32))
            hm.append(P.HostMat(pkg.DSV4_WFP4, W, S, r, c, 1, 32))
        descs.append(pkg.ExpertW(q[0], q[1], q[2]))
        host.append(P.HostExpert(hm[0], hm[1], hm[2]))
    tbl = torch.from_numpy(np.frombuffer(b"".join(bytes(d) for d in descs), np.uint8).copy()).to(DEV)
    g32 = (rng.standard_normal((ne, hidden)) * 0.05).astype(np.float32)
    W16 = (g32.view(np.uint32) >> 16).astype(np.uint16)
    dW16 = torch.from_numpy(W16.view(np.int16).reshape(-1).copy()).to(DEV)
    gate = pkg.qmat(pkg.DSV4_WBF16, dW16.data_ptr(), None, ne, hidden, 0, 0)
    bias = (rng.standard_normal(ne) * 0.05).astype(np.float32)
    dbias = dev_f32(bias)
    out = torch.empty(hidden, dtype=torch.float32, device=DEV)
    di = torch.empty(topk, dtype=torch.int32, device=DEV)
    dw = torch.empty(topk, dtype=torch.float32, device=DEV)
    lib.status()
    for tkn in range(4):
        xh = bf16_x(100 + tkn, hidden)
        x = dev_f32(xh)
        lib.moe_layer_dev(out.data_ptr(), x.data_ptr(), gate, tbl.data_ptr(), ne, topk, 1.5, None,
                          hidden, inter, 10.0, bias_ptr=dbias.data_ptr(), idx_ptr=di.data_ptr(),
                          w_ptr=dw.data_ptr())
        torch.cuda.synchronize()
        assert lib.status() == 0
        sc_o = oracle.bf16_n(W16, xh, ne, hidden)
        wi, ww, wo = oracle.route(sc_o, topk, 1.5, bias=bias)
        gi, gw = di.cpu().numpy(), dw.cpu().numpy()
        _assert_ids(gi, wi, f"token {tkn}")
        _assert_bits(gw, ww, f"token {tkn}")
        acc = np.stack([oracle.expert_forward(host[int(i)], xh, 10.0) for i in gi])
        check_close(out.cpu().numpy(), oracle.moe_combine(acc, gw), 1e-4)


@pytest.mark.parametrize("n,mx,hashed", [(64, False, False), (300, True, False), (48, False, True)])
def test_moe_layer_n_matches_router_and_grouped(lib, pkg, oracle, n, mx, hashed):
    """The many-token MoE layer with the router on the device
    (dsv4_hip_moe_layer_n_dev, dsv4_prefill_moe's sequence for n tokens):
    the picks and weights of every token as dsv4_route gives them on the gate
    scores of dsv4_hip_mmq_n_dev for the same tokens, bit for bit, and the layer's output bit for bit the grouped entry point's
    (exact fp16 path, or the block-scaled path when mx) run on those picks.
    Two tokens also against the oracle's experts (exact path only)."""
    L = _Layer(pkg, lib, 0x4E00 + n)
    rng = np.random.default_rng(n)
    xh = np.stack([bf16_x(200 + t, L.hidden) for t in range(n)]).astype(np.float32)
    x = dev_f32(xh)
    toks = rng.integers(0, len(L.t2e), n).astype(np.int32)
    dtok = torch.from_numpy(toks).to(DEV)
    out = torch.empty(n * L.hidden, dtype=torch.float32, device=DEV)
    di = torch.full((n * L.topk,), -1, dtype=torch.int32, device=DEV)
    dw = torch.empty(n * L.topk, dtype=torch.float32, device=DEV)
    lib.status()
    lib.moe_layer_n_dev(out.data_ptr(), x.data_ptr(), n, L.gate, L.arena.table.data_ptr(), L.ne,
                        L.topk, L.scale, L.shared, L.hidden, L.inter, 10.0, mx=mx,
                        bias_ptr=None if hashed else L.dbias.data_ptr(),
                        tid2eid_ptr=L.dt2e.data_ptr() if hashed else None,
                        n_vocab=len(L.t2e) if hashed else 0,
                        token_ids_ptr=dtok.data_ptr() if hashed else None,
                        idx_ptr=di.data_ptr(), w_ptr=dw.data_ptr())
    sc = torch.empty(n * L.ne, dtype=torch.float32, device=DEV)
    lib.mmq_n_dev(sc.data_ptr(), x.data_ptr(), L.gate, n)
    ref = torch.empty_like(out)
    grouped = lib.moe_grouped_mx_dev if mx else lib.moe_grouped_dev
    grouped(ref.data_ptr(), x.data_ptr(), n, L.arena.table.data_ptr(), L.ne, di.data_ptr(),
            dw.data_ptr(), L.topk, L.shared, L.hidden, L.inter, 10.0)
    torch.cuda.synchronize()
    assert lib.status() == 0
    scores = sc.cpu().numpy().reshape(n, L.ne)
    gi = di.cpu().numpy().reshape(n, L.topk)
    gw = dw.cpu().numpy().reshape(n, L.topk)
    bias = None if hashed else L.bias
    for t in range(n):
        wi, ww, wo = oracle.route(scores[t], L.topk, L.scale, bias=bias,
                                  tid2eid=L.t2e if hashed else None, token_id=int(toks[t]))
        _assert_ids(gi[t], wi, f"token {t}")
        _assert_bits(gw[t], ww, f"token {t}")
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.array_equal(bits(got), bits(ref.cpu().numpy())), "layer output differs from the grouped entry"
    if not mx:
        go = got.reshape(n, L.hidden)
        for t in (0, n - 1):
            check_close(go[t], L.want(oracle, xh[t], gi[t], gw[t]), 1e-3)
