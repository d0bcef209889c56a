"""The one-launch decode MoE (gate/up and down workgroups of one grid, mid's
split tables published through an item counter and a done flag) against the
two-launch form of the same kernels and against the oracle.

The reference decodes one token's MoE as six `dsv4_expert_forward` calls
summed in k order (src/70_decode/dsv4_layer.c:57-116, src/10_compute/dsv4_ops.c:85-93);
both GPU forms compute the same MFMA sequence, so they must agree bit for bit.
Consecutive calls reuse the split-table buffers and the counters: a stale
cached table line or a wrong counter target shows up as a mismatch in a later
call, not the first."""
import zlib

import numpy as np
import pytest
import torch

import pyoracle as P
from conftest import bits
from test_gpu_decode import DEV, bf16_x, check_close, dev_f32, dev_u8
from test_gpu_decode_mx import _device_fp4_experts

pytestmark = pytest.mark.gpu

ENV = "DSV4_HIP_DECODE_LAUNCHES"


def _device_fp8_shared(pkg, oracle, rng, inter, hidden):
    q, hm, keep = [], [], []
    for (r, c) in ((inter, hidden), (inter, hidden), (hidden, inter)):
        W, S = oracle.quant_fp8_blk128((rng.standard_normal((r, c)) * 0.02).astype(np.float32))
        dW, dS = dev_u8(W), dev_f32(S)
        keep += [dW, dS]
        q.append(pkg.qmat(pkg.DSV4_WFP8_F32S, dW.data_ptr(), dS.data_ptr(), r, c, 128, 128))
        hm.append(P.HostMat(pkg.DSV4_WFP8_F32S, W, S, r, c, 128, 128))
    return pkg.ExpertW(q[0], q[1], q[2]), P.HostExpert(hm[0], hm[1], hm[2]), keep


class _Setup:
    def __init__(self, pkg, oracle, seed, inter, hidden, topk, n_exp, shared=False):
        self.rng = np.random.default_rng(seed)
        self.inter, self.hidden, self.topk, self.n_exp = inter, hidden, topk, n_exp
        self.descs, self.host, self.keep = _device_fp4_experts(pkg, oracle, self.rng, n_exp, inter, hidden)
        self.tbl = torch.from_numpy(np.frombuffer(b"".join(bytes(d) for d in self.descs),
                                                  np.uint8).copy()).to(DEV)
        self.shared = self.hshared = None
        if shared:
            self.shared, self.hshared, k2 = _device_fp8_shared(pkg, oracle, self.rng, inter, hidden)
            self.keep += k2

    def draw(self, seed):
        idx = self.rng.choice(self.n_exp, self.topk, replace=False).astype(np.int32)
        lg = self.rng.standard_normal(self.topk)
        w = (np.exp(lg) / np.exp(lg).sum()).astype(np.float32)
        return idx, w, bf16_x(seed, self.hidden)

    def run(self, lib, idx, w, xh, out=None):
        didx = torch.from_numpy(idx).to(DEV)
        dw, x = dev_f32(w), dev_f32(xh)
        if out is None:
            out = torch.empty(self.hidden, dtype=torch.float32, device=DEV)
        lib.moe_decode_dev(out.data_ptr(), x.data_ptr(), self.tbl.data_ptr(), self.n_exp,
                           didx.data_ptr(), dw.data_ptr(), self.topk, self.shared, self.hidden,
                           self.inter, 10.0)
        return out, (didx, dw, x)

    def want(self, oracle, idx, w, xh):
        acc = np.stack([oracle.expert_forward(self.host[i], xh, 10.0) for i in idx])
        y = oracle.moe_combine(acc, w)
        if self.hshared is not None:
            y = (y + oracle.expert_forward(self.hshared, xh, 10.0)).astype(np.float32)
        return y


# DSV4_HIP_DECODE_LAUNCHES: "0" the balanced one-launch form (the default where
# it takes the geometry), "1" the grid-ordered one-launch form, "2" two launches.
FORMS = ("0", "1", "2")


@pytest.mark.parametrize("inter,hidden,topk", [(2048, 4096, 6), (256, 1024, 8), (512, 2048, 3),
                                               (1024, 512, 1), (1024, 2048, 8), (2048, 2048, 2)])
def test_one_launch_matches_two_launch(lib, pkg, oracle, monkeypatch, inter, hidden, topk):
    """Twelve calls enqueued back to back on each one-launch form, each with
    its own routing and token, then the same twelve on the two-launch form:
    bit for bit equal, status clear, and the first and last against the
    oracle. (1024, 2048, 8) has more gate/up tiles than the balanced form
    takes in one round, so its default is the grid-ordered form."""
    s = _Setup(pkg, oracle, zlib.crc32(b"one") + inter + topk, inter, hidden, topk, topk + 4)
    calls = [s.draw(100 + i) for i in range(12)]
    lib.status()
    outs = {}
    for form in FORMS:
        monkeypatch.setenv(ENV, form)
        res = [s.run(lib, *c) for c in calls]
        torch.cuda.synchronize()
        assert lib.status() == 0, f"form {form}"
        outs[form] = [o.cpu().numpy() for o, _ in res]
    for form in ("0", "1"):
        for i in range(len(calls)):
            assert np.array_equal(bits(outs[form][i]), bits(outs["2"][i])), f"form {form} call {i}"
    for i in (0, len(calls) - 1):
        assert check_close(outs["0"][i], s.want(oracle, *calls[i])) < 1e-4


def test_one_launch_with_shared_expert(lib, pkg, oracle, monkeypatch):
    """An FP8 shared expert (fp32 128x128 scales) added in the combine: every
    form agrees bit for bit and matches the oracle."""
    s = _Setup(pkg, oracle, zlib.crc32(b"one-shared"), 2048, 4096, 6, 10, shared=True)
    c = s.draw(7)
    outs = {}
    for form in FORMS:
        monkeypatch.setenv(ENV, form)
        o, _ = s.run(lib, *c)
        torch.cuda.synchronize()
        outs[form] = o.cpu().numpy()
    assert lib.status() == 0
    for form in ("0", "1"):
        assert np.array_equal(bits(outs[form]), bits(outs["2"])), f"form {form}"
    assert check_close(outs["0"], s.want(oracle, *c)) < 1e-4


def test_one_launch_bad_id_then_good(lib, pkg, oracle, monkeypatch):
    """A routing id out of range on the device: status bit 0 and a NaN output;
    the gate/up items of that slot still publish, so the next call's counter
    targets hold and its output is exact."""
    monkeypatch.delenv(ENV, raising=False)
    s = _Setup(pkg, oracle, zlib.crc32(b"one-bad"), 512, 2048, 4, 6)
    idx, w, xh = s.draw(3)
    bad = idx.copy()
    bad[2] = s.n_exp + 5
    lib.status()
    o, _ = s.run(lib, bad, w, xh)
    torch.cuda.synchronize()
    assert lib.status() & 1
    assert np.isnan(o.cpu().numpy()).all()
    o, _ = s.run(lib, idx, w, xh)
    torch.cuda.synchronize()
    assert lib.status() == 0
    assert check_close(o.cpu().numpy(), s.want(oracle, idx, w, xh)) < 1e-4


def test_one_launch_host_routed(lib, pkg, oracle, monkeypatch):
    """The host-routed entry (descriptors by value) on the one-launch form
    equals its two-launch form bit for bit over consecutive calls."""
    s = _Setup(pkg, oracle, zlib.crc32(b"one-routed"), 2048, 4096, 6, 9)
    arr = (pkg.ExpertW * s.n_exp)(*s.descs)
    calls = [s.draw(40 + i) for i in range(4)]
    outs = {}
    for mode in FORMS:
        monkeypatch.setenv(ENV, mode)
        res = []
        for idx, w, xh in calls:
            x = dev_f32(xh)
            out = torch.empty(s.hidden, dtype=torch.float32, device=DEV)
            lib.moe_decode_routed_dev(out.data_ptr(), x.data_ptr(), arr, idx, w, s.topk, None,
                                      s.hidden, s.inter, 10.0)
            res.append((out, x))
        torch.cuda.synchronize()
        outs[mode] = [bits(o.cpu().numpy()) for o, _ in res]
    assert lib.status() == 0
    for form in ("0", "1"):
        for i in range(len(calls)):
            assert np.array_equal(outs[form][i], outs["2"][i]), f"form {form} call {i}"
    assert check_close(outs["0"][0].view(np.float32), s.want(oracle, *calls[0])) < 1e-4


@pytest.mark.parametrize("form", ["0", "1"])
def test_one_launch_wait_timeout_then_recovers(lib, pkg, oracle, monkeypatch, form):
    """The down phase's wait forced to give up from the host
    (DSV4_HIP_DECODE_SPIN=0: every down workgroup gives up without polling,
    and every kernel still exits normally): status bit 3, and every output
    row NaN. The hand-off words are reset by the launch's last workgroup
    whatever the waits did, so the next calls with the default limit are
    bit-identical to the two-launch form."""
    s = _Setup(pkg, oracle, zlib.crc32(b"one-timeout"), 2048, 4096, 6, 8)
    idx, w, xh = s.draw(5)
    monkeypatch.setenv(ENV, "2")
    ref, _ = s.run(lib, idx, w, xh)
    torch.cuda.synchronize()
    want = bits(ref.cpu().numpy())
    monkeypatch.setenv(ENV, form)
    assert lib.status() == 0
    monkeypatch.setenv("DSV4_HIP_DECODE_SPIN", "0")
    o, _ = s.run(lib, idx, w, xh)
    torch.cuda.synchronize()
    assert lib.status() == 8
    assert np.isnan(o.cpu().numpy()).all()
    monkeypatch.delenv("DSV4_HIP_DECODE_SPIN")
    for _ in range(3):
        o, _ = s.run(lib, idx, w, xh)
        torch.cuda.synchronize()
        assert lib.status() == 0
        assert np.array_equal(bits(o.cpu().numpy()), want)


def test_one_launch_timeout_through_host_entry_returns_minus1(lib, pkg, oracle, monkeypatch):
    """The host-pointer decode MoE reads its status word after the sync: a
    wait that gave up makes the call -1 (its output is NaN), and the next call
    is 0 and exact."""
    rng = np.random.default_rng(88)
    from test_gpu_decode import make_fp4_expert
    mats, ex, hx = [], [], []
    for _ in range(3):
        e, he, m = make_fp4_expert(lib, pkg, oracle, rng)
        ex.append(e)
        hx.append(he)
        mats += m
    w = np.array([0.5, 0.3, 0.2], np.float32)
    x = bf16_x(9, 4096)
    monkeypatch.setenv("DSV4_HIP_DECODE_SPIN", "0")
    with pytest.raises(pkg.Dsv4Error, match="timed out"):
        lib.moe_decode(ex, w, x, None, 10.0)
    monkeypatch.delenv("DSV4_HIP_DECODE_SPIN")
    got = lib.moe_decode(ex, w, x, None, 10.0)
    acc = np.stack([oracle.expert_forward(h, x, 10.0) for h in hx])
    check_close(got, oracle.moe_combine(acc, w))
    assert lib.status() == 0
    for m in mats:
        m.drop()


@pytest.mark.parametrize("shared", [False, True])
def test_one_launch_graph_replays(lib, pkg, oracle, monkeypatch, shared):
    """One device-routed decode MoE call captured in a HIP graph (through
    torch's graph capture, on the capture stream) and replayed three times
    for each of four routings, with eager copies of the new inputs and
    synchronisations between replays: every replay bit-identical to the
    eager two-launch form, status clean; an eager call afterwards too."""
    s = _Setup(pkg, oracle, zlib.crc32(b"one-graph") + int(shared), 2048, 4096, 6, 16, shared=shared)
    calls = [s.draw(40 + i) for i in range(4)]
    monkeypatch.setenv(ENV, "2")
    want = []
    for c in calls:
        o, _ = s.run(lib, *c)
        torch.cuda.synchronize()
        want.append(bits(o.cpu().numpy()))
    monkeypatch.delenv(ENV, raising=False)
    assert lib.status() == 0
    idx0, w0, x0 = calls[0]
    didx = torch.from_numpy(idx0.copy()).to(DEV)
    dw, dx = dev_f32(w0), dev_f32(x0)
    out = torch.empty(s.hidden, dtype=torch.float32, device=DEV)
    st = torch.cuda.Stream()

    def call(stream):
        lib.moe_decode_dev(out.data_ptr(), dx.data_ptr(), s.tbl.data_ptr(), s.n_exp, didx.data_ptr(),
                           dw.data_ptr(), s.topk, s.shared, s.hidden, s.inter, 10.0,
                           stream.cuda_stream)

    with torch.cuda.stream(st):
        call(st)                     # workspaces exist before the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        call(st)
    torch.cuda.synchronize()
    for rep in range(3):
        for i, (idx, w, xh) in enumerate(calls):
            didx.copy_(torch.from_numpy(idx))
            dw.copy_(torch.from_numpy(w))
            dx.copy_(torch.from_numpy(xh))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(out.cpu().numpy()), want[i]), f"replay {rep} call {i}"
    assert lib.status() == 0
    with torch.cuda.stream(st):
        call(st)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), want[len(calls) - 1])
    assert lib.status() == 0


def _host_slot_expert(raw):
    """A device-arena expert copied to the host: scales s1 s2 s3 then weights
    w1 w2 w3 (the reference's cache slot layout)."""
    I, H = 2048, 4096
    wb = [I * H // 2, H * I // 2, I * H // 2]
    sb = [I * H // 32, H * I // 32, I * H // 32]
    off_s = [0, sb[0], sb[0] + sb[1]]
    off_w = [sum(sb), sum(sb) + wb[0], sum(sb) + wb[0] + wb[1]]
    shapes = [(I, H), (H, I), (I, H)]
    m = [P.HostMat(P.DSV4_WFP4, raw[off_w[i]:off_w[i] + wb[i]], raw[off_s[i]:off_s[i] + sb[i]], r, c, 1, 32)
         for i, (r, c) in enumerate(shapes)]
    return P.HostExpert(m[0], m[2], m[1])


def test_one_launch_soak(lib, pkg, oracle, monkeypatch):
    """A bounded soak of the one-launch hand-off: 2,000 consecutive calls,
    each with fresh routing (top-6 of 32 full-size FP4 experts), a fresh
    token and the FP8 shared expert, enqueued back to back on the one-launch
    form; then the same 2,000 on the two-launch form. Every output bit for bit
    equal (the first mismatch is reported by its call index) and the status
    clean after each form; the first and the last call against the oracle."""
    import bench
    n_calls, n_exp, topk, hidden, inter = 2000, 32, 6, 4096, 2048
    arena = bench.ExpertArena(torch, pkg, lib, n_exp, seed=0x50A4)
    shared, keep = bench.make_shared_fp8(torch, pkg, lib, 0x50A5)
    rng = np.random.default_rng(0x50A6)
    idx = np.stack([rng.choice(n_exp, topk, replace=False) for _ in range(n_calls)]).astype(np.int32)
    lg = rng.standard_normal((n_calls, topk))
    w = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
    didx, dw = torch.from_numpy(idx).to(DEV), torch.from_numpy(w).to(DEV)
    xs = torch.empty(n_calls * hidden, dtype=torch.float32, device=DEV)
    lib.synth_normal_dev(xs.data_ptr(), xs.numel(), 0x50A7, 1.0, True)
    outs = {}
    lib.status()
    for mode in FORMS:
        monkeypatch.setenv(ENV, mode)
        o = torch.empty((n_calls, hidden), dtype=torch.float32, device=DEV)
        for i in range(n_calls):
            lib.moe_decode_dev(o[i].data_ptr(), xs.data_ptr() + 4 * hidden * i, arena.table.data_ptr(),
                               n_exp, didx.data_ptr() + 4 * topk * i, dw.data_ptr() + 4 * topk * i, topk,
                               shared, hidden, inter, 10.0)
        torch.cuda.synchronize()
        assert lib.status() == 0, f"status after form {mode}"
        outs[mode] = bits(o.cpu().numpy())
    for form in ("0", "1"):
        same = (outs[form] == outs["2"]).all(1)
        assert same.all(), f"form {form}: first mismatch at call {int(np.argmin(same))} of {n_calls}"
    hsh = P.HostExpert(*[P.HostMat(P.DSV4_WFP8_F32S, keep[2 * i].cpu().numpy(), keep[2 * i + 1].cpu().numpy(),
                                   r, c, 128, 128)
                         for i, (r, c) in enumerate(((inter, hidden), (inter, hidden), (hidden, inter)))])
    for i in (0, n_calls - 1):
        xh = xs[i * hidden:(i + 1) * hidden].cpu().numpy()
        acc = np.stack([oracle.expert_forward(_host_slot_expert(arena.host_copy(torch, int(e))), xh, 10.0)
                        for e in idx[i]])
        want = (oracle.moe_combine(acc, w[i]) + oracle.expert_forward(hsh, xh, 10.0)).astype(np.float32)
        assert check_close(outs["1"][i].view(np.float32), want) < 1e-4
