# SPDX-License-Identifier: Apache-2.0
"""Loader residency: the host-descriptor entry points running from an expert
arena laid out exactly as the reference's expert cache builds it.

The reference's cache allocates its slots as one 4096-aligned arena
(src/60_cache/dsv4_cache_init.c:70-101), each slot expert_bytes +
DSV4_SLOT_SLACK (6 x 4096, src/60_cache/dsv4_cache.h:14) bytes. Its geometry
(src/60_cache/dsv4_cache_geom.c:14-31) packs an FP4 expert as the three 1x32
scale arrays s1, s2, s3 followed by the weights w1, w2, w3; dsv4_cache_bind_slot
(:33-50) points each DSV4QMat at slot + toff[3 + i] (weights) and
slot + toff[i] (scales). toff is that compact layout until a load places the
tensors where O_DIRECT lands them: each run at the slot offset with the same
residue mod 4096 as its file offset (src/60_cache/dsv4_cache_load.c:85-137).

The loader's side of the boundary is one dsv4_hip_register of the arena;
dsv4_hip_moe_decode and dsv4_hip_moe_grouped then take the cache's host
descriptors unchanged. Both are checked against the oracle (relative L2 1e-3
per token), for the compact layout and for an O_DIRECT placement, with the
experts scattered over the slots as an LRU cache leaves them.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import pyoracle as P
from conftest import REL_L2_TOL, max_abs, rel_l2

HIDDEN, INTER, N_EXPERTS, TOPK = 4096, 2048, 256, 6
SLOT_SLACK = 6 * 4096
# dsv4_cache_expert_geometry: w1 [inter x hidden], w2 [hidden x inter],
# w3 [inter x hidden], FP4 (half a byte per value), one E8M0 byte per 1x32
WB = [INTER * (HIDDEN // 2), HIDDEN * (INTER // 2), INTER * (HIDDEN // 2)]
SB = [INTER * (HIDDEN // 32), HIDDEN * (INTER // 32), INTER * (HIDDEN // 32)]
ROWS = [INTER, HIDDEN, INTER]
COLS = [HIDDEN, INTER, HIDDEN]
EXPERT_BYTES = sum(WB) + sum(SB)
SLOT_BYTES = EXPERT_BYTES + SLOT_SLACK


def compact_toff():
    """toff[0..2] = scale offsets, toff[3..5] = weight offsets, in the
    geometry's order (scales first)."""
    off, toff = 0, [0] * 6
    for i in range(3):
        toff[i] = off
        off += SB[i]
    for i in range(3):
        toff[3 + i] = off
        off += WB[i]
    return toff


def odirect_toff(file_offsets, direct_only=False):
    """Where dsv4_cache_load places single-tensor runs read with O_DIRECT
    (src/60_cache/dsv4_cache_load.c:85-137): at the first slot offset whose
    residue mod 4096 equals the file offset's and whose widened read window
    (starting `pad` bytes earlier) does not reach back into the previous run,
    so the window lands in the slot without a copy; when that window would
    run past the slot, through the bounce buffer at the cursor instead. Runs
    in the order s1 s2 s3 w1 w2 w3 (file_offsets in that order)."""
    lens = SB + WB
    cursor, toff = 0, [0] * 6
    for k in range(6):
        pad = file_offsets[k] & 4095
        base = cursor + pad
        soff = base + ((pad - base) & 4095)
        wlen = (pad + lens[k] + 4095) & ~4095
        if soff - pad + wlen <= SLOT_BYTES:
            place = soff
        else:
            assert not direct_only, "placement must fit the slot slack"
            assert cursor + lens[k] <= SLOT_BYTES
            place = cursor
        toff[k] = place
        cursor = place + lens[k]
    return toff


class SlotArena:
    """N_EXPERTS slots in one 4096-aligned host allocation; expert e lives in
    slot perm[e] with tensor offsets toff. Scale bytes 116..119 (|w| up to
    6 * 2^-8) keep every activation well inside fp16 for the grouped path."""

    def __init__(self, toff, seed):
        rng = np.random.default_rng(seed)
        raw = np.empty(N_EXPERTS * SLOT_BYTES + 4096, np.uint8)
        start = (-raw.ctypes.data) % 4096
        self.buf = raw[start:start + N_EXPERTS * SLOT_BYTES]
        self.raw = raw
        self.toff = toff
        self.perm = rng.permutation(N_EXPERTS)
        # 4 random weight sets, each expert one of them XOR a byte of its own,
        # so every expert differs without drawing 3.4 GB of random numbers
        pool_w = [rng.integers(0, 256, sum(WB), dtype=np.uint8) for _ in range(4)]
        for e in range(N_EXPERTS):
            s = self.slot(e)
            s[:] = 0
            wsrc = pool_w[e % 4]
            at = 0
            for i in range(3):
                np.bitwise_xor(wsrc[at:at + WB[i]], np.uint8((e * 37) & 0xFF),
                               out=s[toff[3 + i]:toff[3 + i] + WB[i]])
                at += WB[i]
                s[toff[i]:toff[i] + SB[i]] = 116 + ((np.arange(SB[i]) * 7 + e + i) % 4)

    def slot(self, e):
        o = int(self.perm[e]) * SLOT_BYTES
        return self.buf[o:o + SLOT_BYTES]

    def host_descs(self, pkg, e):
        """dsv4_cache_bind_slot: w = slot + toff[3 + i], s = slot + toff[i];
        returned in DSV4ExpertW order (w1, w3, w2)."""
        base = self.slot(e).ctypes.data
        m = [pkg.qmat(pkg.DSV4_WFP4, base + self.toff[3 + i], base + self.toff[i], ROWS[i], COLS[i], 1, 32)
             for i in range(3)]
        return pkg.ExpertW(m[0], m[2], m[1])

    def oracle_expert(self, e):
        s = self.slot(e)
        m = [P.HostMat(P.DSV4_WFP4, s[self.toff[3 + i]:self.toff[3 + i] + WB[i]],
                       s[self.toff[i]:self.toff[i] + SB[i]], ROWS[i], COLS[i], 1, 32) for i in range(3)]
        return P.HostExpert(m[0], m[2], m[1])


LAYOUTS = {
    "compact": compact_toff,
    # file offsets of a checkpoint's six tensors (safetensors data, 16-byte
    # aligned, arbitrary residues mod 4096)
    "odirect": lambda: odirect_toff([0x2A5F0, 0x9B3C10, 0x1D2E00, 0x5C7A30, 0x3FF0, 0x777B60],
                                    direct_only=True),
}


@pytest.mark.gpu
@pytest.mark.parametrize("layout", sorted(LAYOUTS))
def test_arena_decode_and_grouped(lib, pkg, oracle, layout):
    toff = LAYOUTS[layout]()
    for i in range(3):
        assert toff[3 + i] % 16 == 0 and toff[i] % 4 == 0
    arena = SlotArena(toff, seed=0xCAC4E + len(layout))
    lib.check(lib.register(arena.buf), "register the slot arena")
    try:
        rng = np.random.default_rng(11)
        descs = [arena.host_descs(pkg, e) for e in range(N_EXPERTS)]
        cache = {}

        def ref_expert(e):
            if e not in cache:
                cache[e] = arena.oracle_expert(e)
            return cache[e]

        # decode: the router's top-6 per token, descriptors straight from the slots
        for t in range(4):
            ids = rng.choice(N_EXPERTS, TOPK, replace=False)
            lg = rng.standard_normal(TOPK)
            w = (np.exp(lg) / np.exp(lg).sum()).astype(np.float32)
            x = rng.standard_normal(HIDDEN).astype(np.float32)
            got = lib.moe_decode([descs[e] for e in ids], w, x, None, 10.0)
            acc = np.stack([oracle.expert_forward(ref_expert(e), x, 10.0) for e in ids])
            want = oracle.moe_combine(acc, w)
            assert np.all(np.isfinite(got))
            err = rel_l2(got, want)
            assert err <= REL_L2_TOL, f"decode token {t}: rel L2 {err:.3e} (max abs {max_abs(got, want):.3e})"

        # prefill: 64 tokens, top-6 under Zipf(1.1), the full descriptor table
        n = 64
        p = 1.0 / np.arange(1, N_EXPERTS + 1) ** 1.1
        p /= p.sum()
        idx = np.stack([rng.choice(N_EXPERTS, TOPK, replace=False, p=p) for _ in range(n)]).astype(np.int32)
        lg = rng.standard_normal((n, TOPK))
        w = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
        x = rng.standard_normal((n, HIDDEN)).astype(np.float32)
        got = lib.moe_grouped(descs, idx, w, x, None, 10.0)
        assert np.all(np.isfinite(got))
        for t in range(n):
            acc = np.stack([oracle.expert_forward(ref_expert(int(e)), x[t], 10.0) for e in idx[t]])
            want = oracle.moe_combine(acc, w[t])
            err = rel_l2(got[t], want)
            assert err <= REL_L2_TOL, f"grouped token {t}: rel L2 {err:.3e}"
        assert lib.status() == 0
    finally:
        lib.unregister(arena.buf)


def test_odirect_placement_rule():
    """The placement restated above: a tensor read in place keeps its file
    offset's residue mod 4096 and its read window starts at or after the
    previous run's end; one that falls back sits at the cursor; every slot
    holds all six tensors, and both layouts used here keep the alignment the
    kernels need (16 bytes for weights, 4 for scales)."""
    rng = np.random.default_rng(3)
    lens = SB + WB
    direct = 0
    for _ in range(500):
        fo = [int(v) * 16 for v in rng.integers(0, 1 << 24, 6)]
        toff = odirect_toff(fo)
        end = 0
        for k in range(6):
            if toff[k] % 4096 == fo[k] % 4096 and toff[k] - (fo[k] & 4095) >= end:
                direct += 1
            else:
                assert toff[k] == end, "a copied run sits at the cursor"
            assert toff[k] >= end
            end = toff[k] + lens[k]
        assert end <= SLOT_BYTES
    assert direct > 0
    for make in LAYOUTS.values():
        toff = make()
        assert all(toff[3 + i] % 16 == 0 and toff[i] % 4 == 0 for i in range(3))


# ---------------------------------------------------------------------------
# Straight from the checkpoint files: dsv4_hip_load_experts reads the packer's
# experts.idx and the shards (tests/ckpt_writer.py writes a synthetic pair in
# that format) into one device arena of cache-layout slots; the MoE runs from
# the descriptors it returns.

@pytest.mark.gpu
def test_load_experts_from_checkpoint(lib, pkg, oracle, tmp_path):
    from ckpt_writer import write_checkpoint

    hidden, inter, ne, layers = 512, 256, 8, 2
    model_dir, index_dir, hosts = write_checkpoint(oracle, str(tmp_path), layers, ne, hidden, inter, seed=11)
    arena, table, n = lib.load_experts(model_dir, index_dir, 1, hidden, inter)
    try:
        assert n == ne
        # every matrix bit-exact after dequantization
        for e in (0, 5, 7):
            he = hosts[(1, e)]
            for desc, hm in ((table[e].w1, he.w1), (table[e].w3, he.w3), (table[e].w2, he.w2)):
                out = torch.empty(hm.rows * hm.cols, dtype=torch.float32, device="cuda:0")
                lib.dequant_dev(out.data_ptr(), desc)
                torch.cuda.synchronize()
                want = oracle.dequant(hm) if hasattr(oracle, "dequant") else None
                got = out.cpu().numpy().reshape(hm.rows, hm.cols)
                if want is not None:
                    assert np.array_equal(got.view(np.uint32), want.reshape(hm.rows, hm.cols).view(np.uint32))
                else:
                    x = np.eye(hm.cols, dtype=np.float32)[:8]          # rows of the dequantized matrix
                    ref = oracle.mmq_n(hm, np.ascontiguousarray(x.reshape(-1)), 8).reshape(8, hm.rows).T
                    assert np.array_equal(got[:, :8], ref)
        # the decode MoE through the loaded table against the oracle
        raw = bytes(C.string_at(C.addressof(table), C.sizeof(pkg.ExpertW) * n))
        dtab = torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to("cuda:0")
        rng = np.random.default_rng(5)
        for t in range(4):
            ids = rng.choice(ne, 6, replace=False).astype(np.int32)
            w = rng.dirichlet(np.ones(6)).astype(np.float32)
            x = rng.standard_normal(hidden).astype(np.float32)
            dx, di, dw = (torch.from_numpy(a).to("cuda:0") for a in (x, ids, w))
            out = torch.empty(hidden, dtype=torch.float32, device="cuda:0")
            lib.moe_decode_dev(out.data_ptr(), dx.data_ptr(), dtab.data_ptr(), ne, di.data_ptr(), dw.data_ptr(),
                               6, None, hidden, inter, 10.0)
            torch.cuda.synchronize()
            acc = np.stack([oracle.expert_forward(hosts[(1, int(e))], x, 10.0) for e in ids])
            want = oracle.moe_combine(acc, w)
            got = out.cpu().numpy()
            assert rel_l2(got, want) <= REL_L2_TOL, f"token {t}: {rel_l2(got, want):.3e}"
        assert lib.status() == 0
    finally:
        lib.free_experts(arena)
