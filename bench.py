# SPDX-License-Identifier: Apache-2.0
"""Benchmark of the gfx950 quantized-matmul hot path on one MI355X.

Default workload (--config 1): one decode token through a DeepSeek-V4-Flash
MoE layer's routed experts -- 256 FP4 experts resident in HBM (gate/up
2048x4096, down 4096x2048, e2m1 packed two per byte, E8M0 scale per 1x32),
top-6 uniform routing with softmax weights, SwiGLU (limit 10), k-order
weighted combine. One step = one token. Every step routes to a fresh set of
six experts, so the weights stream from HBM rather than from the 256 MB
Infinity Cache. Metric: algorithmic HBM GB/s (6 x 13,369,344 B of expert
weights and scales + 8 KiB bf16 x + 16 KiB fp32 out per token).

--config 0: one 4096x4096 e4m3 matvec with fp32 128x128 scales, x bf16;
weights rotated over 40 copies (672 MB) so each step reads from HBM.

--config 2: batched decode MoE, 64 tokens per step, top-6 of the 256 FP4
experts under Zipf(1.1) popularity (fresh routing every step), plus an FP8
shared expert (fp32 128x128 scales), through the grouped MoE. Metric:
algorithmic HBM GB/s (distinct routed experts x 13,369,344 B + shared
25,171,968 B + bf16 x + fp32 out per step).

--config 3: prefill GEMM, 2048 tokens x 4096 (bf16 A, quantized on the fly to
e4m3 with an fp32 scale per 1x128) times a 4096x4096 e4m3 weight with fp32
128x128 scales, bf16 output, on FP8 MFMA. Metric: TFLOP/s (2 M N K per step).

--config 4: the prefill MoE layer, 4096 tokens, top-6 Zipf(1.1) routing over
the 256 FP4 experts plus the FP8 shared expert, permute -> grouped MFMA GEMMs
with SwiGLU -> combine. Metric: TFLOP/s of the routed + shared FLOPs.

Prints ONE JSON line. Synthetic data (seeded), random-init weights.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0          # MI355X dense FP8 MFMA
FP16_PEAK_TFLOPS = 2500.0         # MI355X dense fp16 / bf16 MFMA
SHARED_BYTES = 3 * (2048 * 4096 + 16 * 32 * 4)   # FP8 gate/up/down + fp32 128x128 scales

EXPERT_BYTES = 13_369_344          # w1,w3: 2048x4096 FP4 + scales; w2: 4096x2048
HIDDEN, INTER, N_EXPERTS, TOPK = 4096, 2048, 256, 6


def load_pkg():
    spec = importlib.util.spec_from_file_location(
        "dsv4_amd", os.path.join(ROOT, "deepseek-v4-in-c_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["dsv4_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_for(cfg):
    """HBM bytes per launch of the config's measured call, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/traffic.json), each
    counter scaled by what it reads for a plain 256 MiB device copy. None when
    the summary is absent."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            t = json.load(f)
        return int(t["configs"][str(cfg)]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


# ------------------------------------------------------------ workloads ----

class ExpertArena:
    """256 FP4 experts in one device arena, each laid out like the reference's
    cache slot (src/60_cache/dsv4_cache_geom.c:14-31): scales s1, s2, s3 then
    weights w1, w2, w3."""

    def __init__(self, torch, pkg, lib, n_experts, seed):
        self.n = n_experts
        dev = "cuda:0"
        self.buf = torch.empty(n_experts * EXPERT_BYTES, dtype=torch.uint8, device=dev)
        wb = [INTER * HIDDEN // 2, HIDDEN * INTER // 2, INTER * HIDDEN // 2]
        sb = [INTER * HIDDEN // 32, HIDDEN * INTER // 32, INTER * HIDDEN // 32]
        shapes = [(INTER, HIDDEN), (HIDDEN, INTER), (INTER, HIDDEN)]   # w1, w2, w3
        off_s = [0, sb[0], sb[0] + sb[1]]
        off_w = [sum(sb), sum(sb) + wb[0], sum(sb) + wb[0] + wb[1]]
        tmp = torch.empty(INTER * HIDDEN, dtype=torch.float32, device=dev)
        base = self.buf.data_ptr()
        descs = []
        for e in range(n_experts):
            eb = base + e * EXPERT_BYTES
            q = []
            for i, (r, c) in enumerate(shapes):
                lib.synth_normal_dev(tmp.data_ptr(), r * c, seed * 1000003 + e * 3 + i, 0.02)
                lib.quant_fp4_mx_dev(eb + off_w[i], eb + off_s[i], tmp.data_ptr(), r, c)
                q.append(pkg.qmat(pkg.DSV4_WFP4, eb + off_w[i], eb + off_s[i], r, c, 1, 32))
            descs.append(pkg.ExpertW(q[0], q[2], q[1]))   # (w1, w3, w2)
        torch.cuda.synchronize()
        raw = b"".join(bytes(d) for d in descs)
        self.descs = descs
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(dev)

    def host_copy(self, torch, e):
        return self.buf[e * EXPERT_BYTES:(e + 1) * EXPERT_BYTES].cpu().numpy()


def routing(n_steps, seed):
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.choice(N_EXPERTS, TOPK, replace=False) for _ in range(n_steps)])
    lg = rng.standard_normal((n_steps, TOPK))
    w = np.exp(lg) / np.exp(lg).sum(1, keepdims=True)
    return idx.astype(np.int32), w.astype(np.float32)


def zipf_routing(n_tokens, seed, s=1.1):
    """top-6 of 256 experts per token, expert e drawn with weight (e+1)^-s
    without replacement within a token; softmax weights of N(0,1) logits."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, N_EXPERTS + 1) ** s
    p /= p.sum()
    idx = np.stack([rng.choice(N_EXPERTS, TOPK, replace=False, p=p) for _ in range(n_tokens)])
    lg = rng.standard_normal((n_tokens, TOPK))
    w = np.exp(lg) / np.exp(lg).sum(1, keepdims=True)
    return idx.astype(np.int32), w.astype(np.float32)


def make_shared_fp8(torch, pkg, lib, seed):
    """The shared expert: e4m3 gate/up [2048 x 4096] and down [4096 x 2048],
    fp32 scale per 128 x 128 block."""
    dev = "cuda:0"
    tmp = torch.empty(INTER * HIDDEN, dtype=torch.float32, device=dev)
    keep, q = [], []
    for i, (r, c) in enumerate(((INTER, HIDDEN), (INTER, HIDDEN), (HIDDEN, INTER))):
        W = torch.empty(r * c, dtype=torch.uint8, device=dev)
        S = torch.empty((r // 128) * (c // 128), dtype=torch.float32, device=dev)
        lib.synth_normal_dev(tmp.data_ptr(), r * c, seed + i, 0.02)
        lib.quant_fp8_blk128_dev(W.data_ptr(), S.data_ptr(), tmp.data_ptr(), r, c)
        keep += [W, S]
        q.append(pkg.qmat(pkg.DSV4_WFP8_F32S, W.data_ptr(), S.data_ptr(), r, c, 128, 128))
    torch.cuda.synchronize()
    return pkg.ExpertW(q[0], q[1], q[2]), keep


class DecodeLayer:
    """The matrices of one decode layer at DeepSeek-V4-Flash shapes
    (src/00_base/dsv4_weights.h:44-112), run on the device in the order
    src/70_decode/dsv4_layer_attn.c:21-106 and dsv4_layer.c:52-116 call
    dsv4_mmq: wq_a, wq_b, wkv, the compressor's wkv and wgate (BF16, ratio-4
    layer), the indexer's wq_b and weights_proj (BF16), the eight wo_a group
    slices of one [8192 x 4096] arena (dsv4_wo_a_group) as one multi-job call
    (dsv4_hip_mmq_multi_dev, as dsv4_prefill_oproj hands them to
    dsv4_prefill_pm_multi), wo_b [4096 x 8192],
    then the MoE block (dsv4_hip_moe_layer_dev: BF16 gate 256 x 4096, the
    router with a bias, six of the 256 FP4 experts, the FP8 shared expert).
    FP8 matrices carry E8M0 128 x 128 scales as the checkpoint's do. The
    steps between the matrices (norms, RoPE, the compressor's pooling, the
    indexer's scores, sparse attention) are not on the matmul path and are
    left out: a matrix takes the previous one's output where the layer
    feeds it one (qr into wq_b and the indexer's wq_b; the attention output,
    here q itself, 64 heads x 512, into wo_a; the group outputs into wo_b;
    wo_b's output into the MoE block), else x."""

    FP8 = (("wq_a", 1024, 4096, "x"), ("wq_b", 32768, 1024, "qr"), ("wkv", 512, 4096, "x"),
           ("idx_wq_b", 8192, 1024, "qr"))
    BF16 = (("comp_wkv", 1024, 4096), ("comp_wgate", 1024, 4096), ("idx_wproj", 64, 4096),
            ("gate", N_EXPERTS, HIDDEN))

    def __init__(self, torch, pkg, lib, arena, seed):
        dev = "cuda:0"
        self.arena = arena
        self.keep = {}
        self.desc = {}
        tmp = torch.empty(8192 * 4096, dtype=torch.float32, device=dev)

        def fp8(name, r, c, sd):
            W = torch.empty(r * c, dtype=torch.uint8, device=dev)
            S32 = torch.empty((r // 128) * (c // 128), dtype=torch.float32, device=dev)
            lib.synth_normal_dev(tmp.data_ptr(), r * c, sd, 0.02)
            lib.quant_fp8_blk128_dev(W.data_ptr(), S32.data_ptr(), tmp.data_ptr(), r, c)
            S = torch.clamp(torch.ceil(torch.log2(S32)) + 127, 0, 254).to(torch.uint8)
            self.keep[name] = (W, S)
            return pkg.qmat(pkg.DSV4_WFP8, W.data_ptr(), S.data_ptr(), r, c, 128, 128)

        for i, (name, r, c, _) in enumerate(self.FP8):
            self.desc[name] = fp8(name, r, c, seed * 97 + i)
        self.desc["wo_a"] = fp8("wo_a", 8192, 4096, seed * 97 + 10)
        self.desc["wo_b"] = fp8("wo_b", 4096, 8192, seed * 97 + 11)
        for i, (name, r, c) in enumerate(self.BF16):
            lib.synth_normal_dev(tmp.data_ptr(), r * c, seed * 97 + 20 + i, 0.02)
            W = tmp[:r * c].bfloat16()
            self.keep[name] = (W, None)
            self.desc[name] = pkg.qmat(pkg.DSV4_WBF16, W.data_ptr(), None, r, c, 0, 0)
        W, S = self.keep["wo_a"]
        self.slices = [pkg.qmat(pkg.DSV4_WFP8, W.data_ptr() + g * 1024 * 4096, S.data_ptr() + g * 8 * 32,
                                1024, 4096, 128, 128) for g in range(8)]
        self.bias = torch.empty(N_EXPERTS, dtype=torch.float32, device=dev)
        lib.synth_normal_dev(self.bias.data_ptr(), N_EXPERTS, seed * 97 + 30, 0.05)
        self.shared, self.skeep = make_shared_fp8(torch, pkg, lib, seed * 97 + 31)
        f = lambda n: torch.empty(n, dtype=torch.float32, device=dev)
        self.out = {"qr": f(1024), "q": f(32768), "kv": f(512), "comp_kv": f(1024), "comp_sc": f(1024),
                    "idx_q": f(8192), "idx_w": f(64), "ogrp": f(8192), "attn": f(HIDDEN), "moe": f(HIDDEN)}
        self.idx = torch.empty(TOPK, dtype=torch.int32, device=dev)
        self.w = torch.empty(TOPK, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        del tmp

    # bytes one token reads: every matrix once, the six routed experts
    def bytes_per_token(self):
        b = sum(r * c + (r // 128) * (c // 128) for _, r, c, _ in self.FP8)
        b += 2 * (8192 * 4096 + 32 * 32 * 2)
        b += sum(2 * r * c for _, r, c in self.BF16)
        return b + TOPK * EXPERT_BYTES + SHARED_BYTES

    def run(self, lib, x_ptr, sp):
        """Enqueue the layer's matrices for the token at x_ptr on stream sp."""
        o = self.out
        mm = lambda y, x, name: lib.mmq_n_dev(o[y].data_ptr(), x, self.desc[name], 1, sp)
        mm("qr", x_ptr, "wq_a")
        mm("q", o["qr"].data_ptr(), "wq_b")
        mm("kv", x_ptr, "wkv")
        mm("comp_kv", x_ptr, "comp_wkv")
        mm("comp_sc", x_ptr, "comp_wgate")
        mm("idx_q", o["qr"].data_ptr(), "idx_wq_b")
        mm("idx_w", x_ptr, "idx_wproj")
        lib.mmq_multi_dev([(self.slices[g], o["q"].data_ptr() + 4 * 4096 * g, o["ogrp"].data_ptr() + 4 * 1024 * g, 1)
                           for g in range(8)], sp)
        mm("attn", o["ogrp"].data_ptr(), "wo_b")
        lib.moe_layer_dev(o["moe"].data_ptr(), o["attn"].data_ptr(), self.desc["gate"],
                          self.arena.table.data_ptr(), N_EXPERTS, TOPK, 2.5, self.shared, HIDDEN, INTER,
                          10.0, bias_ptr=self.bias.data_ptr(), idx_ptr=self.idx.data_ptr(),
                          w_ptr=self.w.data_ptr(), stream=sp)


def bench_decode_layer(torch, pkg, lib, arena, xs, n_layers=4, graph_calls=16, reps=8):
    """One decode layer's whole matrix chain per token (DecodeLayer), replayed
    from a HIP graph of graph_calls tokens that cycle through n_layers layers
    with their own weights (so the attention matrices, 129 MB a layer, do not
    stay in the 256 MB memory-side cache between a layer's tokens), each
    token its own x and so its own experts."""
    layers = [DecodeLayer(torch, pkg, lib, arena, 0xDEC0 + i) for i in range(n_layers)]
    n_x = xs.numel() // HIDDEN
    st = torch.cuda.Stream()
    ss = st.cuda_stream

    def token(i):
        layers[i % n_layers].run(lib, xs.data_ptr() + 4 * HIDDEN * (i % n_x), ss)

    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        for i in range(2 * n_layers):
            token(i)
        torch.cuda.synchronize()
        assert lib.status() == 0
        eager = time_events(torch, st, token, graph_calls)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for i in range(graph_calls):
                token(i)
        torch.cuda.synchronize()
        g.replay()                                   # replays go to the current stream, st
        torch.cuda.synchronize()
        per_tok = time_events(torch, st, lambda i: g.replay(), reps) / graph_calls
    assert lib.status() == 0
    nb = layers[0].bytes_per_token()
    return {"entry": "one decode layer's matrices: 8 FP8 projections incl. 8 wo_a slices and wo_b, "
                     "4 BF16 matrices, then dsv4_hip_moe_layer_dev with the FP8 shared expert",
            "bytes_per_token": nb, "layers_cycled": n_layers,
            "eager_us": round(eager * 1e6, 3), "graph_us": round(per_tok * 1e6, 3),
            "graph_GBs": round(nb / per_tok / 1e9, 1),
            "graph_hbm_frac": round(nb / per_tok / 1e9 / HBM_PEAK_GBS, 4)}


def time_events(torch, stream, fn, n):
    """Average duration of one fn() call over n calls enqueued back to back on
    `stream` (the stream the kernels are launched on), from one pair of HIP
    events around the n calls. Events around every single call would add a
    drain and a release between calls that back-to-back calls do not pay
    (about 2 us on a 21 us call), and would disagree with the kernel
    durations rocprofv3 reports."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(n):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / n


# --------------------------------------------------------- CPU baseline ----
#
# The reference's CPU path (its src/10_compute objects compiled unchanged into
# oracle/_ref, else this repo's C restatement) timed on the host of the GPU.
# Each measurement runs in a child process started with OMP_NUM_THREADS,
# OMP_PROC_BIND=spread and OMP_PLACES=cores in its environment: libgomp reads
# them once, when it initialises, so they cannot be set from inside a process
# that has loaded it. One child runs one thread, one all physical cores of
# this process's CPU set; each does one warm-up unit and then at least five
# timed units (more while the time bound allows) and reports their median.
# The inputs are the GPU run's own tensors, handed over as .npy files.

def host_cpu():
    """CPU model, sockets and cores (lscpu), and the physical cores of the CPU
    set this process may run on."""
    info = {}
    env = dict(os.environ, LC_ALL="C")
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, env=env, timeout=20).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "Model name":
                info["model"] = v
            elif k == "Socket(s)":
                info["sockets"] = int(v)
            elif k == "Core(s) per socket":
                info["cores_per_socket"] = int(v)
            elif k == "Thread(s) per core":
                info["threads_per_core"] = int(v)
        allowed = os.sched_getaffinity(0)
        par = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"], capture_output=True, text=True,
                             env=env, timeout=20).stdout
        cores = set()
        for line in par.splitlines():
            if line.startswith("#"):
                continue
            f = line.split(",")
            if len(f) >= 3 and f[0].isdigit() and int(f[0]) in allowed:
                cores.add((f[2], f[1]))
        info["cpus_allowed"] = len(allowed)
        info["cores_allowed"] = len(cores) if cores else len(allowed)
    except (OSError, ValueError, subprocess.SubprocessError):
        info.setdefault("cpus_allowed", os.cpu_count() or 1)
        info.setdefault("cores_allowed", info["cpus_allowed"])
    return info


def all_core_threads(info):
    """All physical cores of the CPU set, at most the OMP_NUM_THREADS the
    environment grants (the per-GPU share of the host)."""
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    n = info.get("cores_allowed") or 1
    return max(1, min(n, cap) if cap > 0 else n)


def cpu_baseline(work, arrays, params, per_unit, unit, sample, seconds, threads=0):
    """Runs `work` in two child processes (1 thread; all cores, or `threads`
    when given) on `arrays` (name -> ndarray, written to a temporary
    directory) and returns the cpu_baseline record: value = per_unit / median
    unit time at all cores."""
    info = host_cpu()
    threads = threads or all_core_threads(info)
    tmp = tempfile.mkdtemp(prefix="dsv4_cpu_")
    try:
        for k, a in arrays.items():
            np.save(os.path.join(tmp, k + ".npy"), np.ascontiguousarray(a), allow_pickle=False)
        runs = {}
        for label, nthr, budget in (("one_thread", 1, 0.5 * seconds), ("all_cores", threads, 0.5 * seconds)):
            spec = dict(params, work=work, dir=tmp, seconds=budget, min_runs=5, max_runs=200)
            spath = os.path.join(tmp, f"spec_{label}.json")
            with open(spath, "w") as f:
                json.dump(spec, f)
            env = dict(os.environ, OMP_NUM_THREADS=str(nthr), OMP_PROC_BIND="spread",
                       OMP_PLACES="cores")
            log(f"CPU baseline {work}: {label} ({nthr} threads)")
            p = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-worker", spath],
                               capture_output=True, text=True, env=env, timeout=600)
            if p.returncode != 0:
                raise RuntimeError(f"CPU worker {work}/{label} failed: {p.stderr[-2000:]}")
            r = json.loads(p.stdout.strip().splitlines()[-1])
            r["threads"] = nthr
            r["value"] = round(per_unit / r["median_s"], 5)
            runs[label] = r
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    a = runs["all_cores"]
    return {"value": a["value"], "unit": unit, "cores": threads, "kind": a["kind"],
            "sample": f"{sample}; median of {a['runs']} timed units after 1 warm-up",
            "one_thread": runs["one_thread"], "all_cores": a,
            "omp": {"OMP_PROC_BIND": "spread", "OMP_PLACES": "cores"}, "host": info}


def _cpu_worker(spec_path):
    """Child side of cpu_baseline: builds the work unit named in the spec,
    runs it once untimed, then times units until min_runs are done and the
    time bound is spent (or max_runs), and prints the median."""
    with open(spec_path) as f:
        spec = json.load(f)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as P
    kind = "reference"
    try:
        impl = P.Reference()
    except (FileNotFoundError, OSError):
        impl, kind = P.Oracle(), "port"
    orc = P.Oracle()
    d = spec["dir"]

    def ld(name):
        return np.load(os.path.join(d, name + ".npy"), mmap_mode="r", allow_pickle=False)

    wb = [INTER * HIDDEN // 2, HIDDEN * INTER // 2, INTER * HIDDEN // 2]
    sb = [INTER * HIDDEN // 32, HIDDEN * INTER // 32, INTER * HIDDEN // 32]
    off_s = [0, sb[0], sb[0] + sb[1]]
    off_w = [sum(sb), sum(sb) + wb[0], sum(sb) + wb[0] + wb[1]]
    shapes = [(INTER, HIDDEN), (HIDDEN, INTER), (INTER, HIDDEN)]

    def host_expert(raw):
        """An expert in the reference's slot layout (scales s1 s2 s3, then
        w1 w2 w3) as host descriptors over the slot's bytes."""
        m = [P.HostMat(P.DSV4_WFP4, raw[off_w[i]:off_w[i] + wb[i]], raw[off_s[i]:off_s[i] + sb[i]],
                       r, c, 1, 32) for i, (r, c) in enumerate(shapes)]
        return P.HostExpert(m[0], m[2], m[1])

    def fp4_tiles(mat, X, rows, cols, nt):
        """dsv4_mmq_n's tiling: the fp4_n body takes at most 128 tokens
        (DSV4_MAX_BATCH, src/10_compute/dsv4_matmul.c:63-73)"""
        out = np.empty(nt * rows, np.float32)
        for o in range(0, nt, 128):
            t = min(128, nt - o)
            out[o * rows:(o + t) * rows] = impl.fp4_n(mat.W, mat.S, X[o * cols:(o + t) * cols],
                                                      rows, cols, 1, 32, t)
        return out

    def fp4_bucket(e, X, nt):
        g = fp4_tiles(e.w1, X, INTER, HIDDEN, nt)
        u = fp4_tiles(e.w3, X, INTER, HIDDEN, nt)
        return fp4_tiles(e.w2, impl.swiglu(g, u, 10.0), HIDDEN, INTER, nt)

    def shared_fp8(X, nt):
        """The FP8 shared expert through fp8_n (E8M0 block scales)."""
        S = [ld(f"sh_s{i}") for i in range(3)]
        Wm = [ld(f"sh_w{i}") for i in range(3)]
        g = impl.fp8_n(Wm[0], S[0], X, INTER, HIDDEN, 128, 128, nt)
        u = impl.fp8_n(Wm[1], S[1], X, INTER, HIDDEN, 128, 128, nt)
        return impl.fp8_n(Wm[2], S[2], impl.swiglu(g, u, 10.0), HIDDEN, INTER, 128, 128, nt)

    work = spec["work"]
    if work == "fp8_matvec":
        Wq, Se, x = ld("w"), ld("s"), np.ascontiguousarray(ld("x"))
        def unit(i):
            impl.fp8_n(Wq, Se, x, 4096, 4096, 128, 128, 1)
    elif work == "fp8_gemm":
        Wq, Se, X = ld("w"), ld("s"), np.ascontiguousarray(ld("x")).reshape(-1)
        nt = X.size // 4096
        def unit(i):
            impl.fp8_n(Wq, Se, X, 4096, 4096, 128, 128, nt)
    elif work == "decode_token":
        slots = ld("experts")
        experts = [host_expert(slots[e]) for e in range(slots.shape[0])]
        x = np.ascontiguousarray(ld("x"))
        rng = np.random.default_rng(7)
        plans = [(rng.choice(len(experts), TOPK, replace=False), rng.standard_normal(TOPK))
                 for _ in range(spec["max_runs"] + 1)]
        def unit(i):
            ids, lg = plans[i]
            w = (np.exp(lg) / np.exp(lg).sum()).astype(np.float32)
            acc = np.stack([impl.expert_forward(experts[k], x, 10.0) for k in ids])
            orc.moe_combine(acc, w)
    elif work == "buckets":
        slots = ld("experts")
        experts = [host_expert(slots[e]) for e in range(slots.shape[0])]
        Xs = [np.ascontiguousarray(ld(f"x{e}")).reshape(-1) for e in range(slots.shape[0])]
        Xsh = np.ascontiguousarray(ld("x_shared")).reshape(-1)
        nsh = Xsh.size // HIDDEN
        def unit(i):
            for e, X in zip(experts, Xs):
                fp4_bucket(e, X, X.size // HIDDEN)
            shared_fp8(Xsh, nsh)
    else:
        raise SystemExit(f"unknown CPU work {work}")

    unit(0)                                   # warm-up
    times = []
    t_end = time.perf_counter() + spec["seconds"]
    while len(times) < spec["min_runs"] or (time.perf_counter() < t_end and len(times) < spec["max_runs"]):
        t0 = time.perf_counter()
        unit(len(times) + 1)
        times.append(time.perf_counter() - t0)
    print(json.dumps({"kind": kind, "runs": len(times), "median_s": float(np.median(times)),
                      "min_s": float(np.min(times)), "max_s": float(np.max(times))}), flush=True)


def fp8_e8m0(torch, S):
    """E8M0 block scales (the power of two at or above each fp32 scale): the
    reference's CPU fp8_n stores E8M0 scales only."""
    return torch.clamp(torch.ceil(torch.log2(S)) + 127, 0, 254).to(torch.uint8).cpu().numpy()


def shared_host(torch, keep):
    """The FP8 shared expert's weights (gate, up, down) and E8M0 scales on the host."""
    out = {}
    for i in range(3):
        out[f"sh_w{i}"] = keep[2 * i].cpu().numpy()
        out[f"sh_s{i}"] = fp8_e8m0(torch, keep[2 * i + 1])
    return out


def bench_grouped(args, torch, pkg, lib, stream, sp, K, W, cfg):
    """Configs 2 (64 tokens per step) and 4 (4096 tokens per step)."""
    n = 64 if cfg == 2 else 4096
    dev = "cuda:0"
    seed = 0xD5EED000 + cfg
    log("generating 256 FP4 experts and the FP8 shared expert on the device")
    arena = ExpertArena(torch, pkg, lib, N_EXPERTS, seed=seed)
    shared, keep = make_shared_fp8(torch, pkg, lib, seed * 7)
    # fresh routing and tokens for every step (config 2: K + W steps; config
    # 4: four rotating token blocks, a block being 4096 x 4096 fp32)
    nsets = K + W if cfg == 2 else 4
    idx_h, w_h = zipf_routing(n * nsets, seed)
    idx = torch.from_numpy(idx_h).to(dev)
    wts = torch.from_numpy(w_h).to(dev)
    xs = torch.empty(n * nsets * HIDDEN, dtype=torch.float32, device=dev)
    lib.synth_normal_dev(xs.data_ptr(), xs.numel(), seed ^ 0x55, 1.0, True)
    out = torch.empty(n * HIDDEN, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    # config 4 runs the routed experts on the block-scaled MFMA (FP4 weights x
    # MXFP8 tokens and mid: within 1e-3 relative L2 of the reference fed the
    # same quantized tokens and mid, a few 1e-2 from the unquantized one, both
    # reported); config 2 (and config 4 with --exact) the exact fp16 path
    mx = cfg == 4 and not args.exact

    def call(fn, i):
        j = i % nsets
        fn(out.data_ptr(), xs.data_ptr() + 4 * HIDDEN * n * j, n,
           arena.table.data_ptr(), N_EXPERTS, idx.data_ptr() + 4 * TOPK * n * j,
           wts.data_ptr() + 4 * TOPK * n * j, TOPK, shared, HIDDEN, INTER, 10.0, sp)

    def step(i):
        call(lib.moe_grouped_mx_dev if mx else lib.moe_grouped_dev, i)

    def step_other(i):
        call(lib.moe_grouped_dev if mx else lib.moe_grouped_mx_dev, i)

    def step_bytes(j):
        d = len(np.unique(idx_h[n * j:n * (j + 1)]))
        return d * EXPERT_BYTES + SHARED_BYTES + n * HIDDEN * 2 + n * HIDDEN * 4

    flops_step = 2.0 * n * TOPK * 3 * INTER * HIDDEN + 2.0 * n * 3 * INTER * HIDDEN
    for i in range(W):
        step(i)
    torch.cuda.synchronize()
    assert lib.status() == 0
    log(f"timing {K} steps")
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(K):
        step(W + i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_step = e0.elapsed_time(e1) * 1e-3 / K
    t_launch = time_events(torch, stream, lambda i: step(W + i), K)
    other = None
    if cfg == 4 and not args.no_other:
        # the other precision path of the same call, timed the same way, and
        # the block-scaled path's error against the exact one on one step
        for i in range(W):
            step_other(i)
        t_other = time_events(torch, stream, lambda i: step_other(W + i), K)
        call(lib.moe_grouped_dev, W)
        exact_out = out.clone()
        call(lib.moe_grouped_mx_dev, W)
        torch.cuda.synchronize()
        e = (out.double() - exact_out.double()).norm() / exact_out.double().norm()
        rel = float(e)
        other = {"entry": "dsv4_hip_moe_grouped_dev" if mx else "dsv4_hip_moe_grouped_mx_dev",
                 "path": "exact: fp16 MFMA on exactly decoded weights" if mx
                 else "block-scaled MFMA, MXFP8 tokens and mid",
                 "launch_us": round(t_other * 1e6, 3),
                 "tflops": round(flops_step / t_other / 1e12, 2),
                 "mx_rel_l2_vs_exact": float(f"{rel:.3e}"),
                 "mx_error_note": "the block-scaled path rounds tokens and mid to MXFP8 (e4m3, "
                                  "E8M0 per 32): rel L2 <= 1e-3 per token against the reference "
                                  "fed the same quantized tokens and mid (tests/test_gpu_moe_mx.py); "
                                  "mx_rel_l2_vs_exact against the unquantized computation, beyond "
                                  "1e-3; the exact path is within 1e-3 of the unquantized reference"}
    assert lib.status() == 0
    bytes_avg = float(np.mean([step_bytes((W + i) % nsets) for i in range(K)]))
    d_avg = (bytes_avg - SHARED_BYTES - n * HIDDEN * 6) / EXPERT_BYTES
    cpu = None
    if not args.no_cpu:
        # the reference's bucket path (src/80_prefill/dsv4_prefill_experts.c:60-69):
        # per expert, its routed tokens through fp4_n (nt = bucket size, in
        # tiles of 128) for w1 and w3, SwiGLU, fp4_n for w2; then the shared
        # expert through fp8_n. Unit: the 8 most-loaded buckets of step 0 and
        # the shared expert over its 64 tokens (config 2); the 2 most-loaded
        # buckets cut to 128 tokens each and the shared expert over 128 tokens
        # (config 4).
        counts = np.bincount(idx_h[:n].reshape(-1), minlength=N_EXPERTS)
        nsel, cap = (8, n) if cfg == 2 else (2, 128)
        sel = np.argsort(-counts, kind="stable")[:nsel]
        x_host = xs[:n * HIDDEN].view(n, HIDDEN).cpu().numpy()
        arrays = {"experts": np.stack([arena.host_copy(torch, int(e)) for e in sel])}
        ntoks = []
        for j, e in enumerate(sel):
            toks = np.nonzero((idx_h[:n] == e).any(1))[0][:cap]
            arrays[f"x{j}"] = x_host[toks]
            ntoks.append(len(toks))
        nsh = min(n, cap)
        arrays["x_shared"] = x_host[:nsh]
        arrays.update(shared_host(torch, keep))
        if cfg == 2:
            per_unit, unit = (nsel * EXPERT_BYTES + SHARED_BYTES) / 1e9, "GB/s"
        else:
            per_unit, unit = 2.0 * (sum(ntoks) + nsh) * 3 * INTER * HIDDEN / 1e12, "TFLOP/s"
        cpu = cpu_baseline("buckets", arrays, {}, per_unit, unit,
                           f"buckets of {nsel} experts (tokens {','.join(map(str, ntoks))}) through "
                           f"fp4_n/SwiGLU/fp4_n plus the shared expert over {nsh} tokens through fp8_n",
                           args.cpu_seconds, args.cpu_threads)
    res = {
        "metric": "quant matvec HBM GB/s (% peak); prefill FP4/FP8 GEMM TFLOP/s (% MFMA peak)",
        "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": round(t_step * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ("fp4 e2m1 weights x mxfp8 e4m3 tokens and mid on block-scaled MFMA (routed), fp8 "
                  "e4m3 weights x e4m3 1x128 tokens and mid on the FP8 GEMM (shared), fp32 accumulate")
                 if mx else
                 "fp16 MFMA on exactly decoded FP4 (routed) / FP8 (shared) weights, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) experts, bf16 N(0,1) tokens, Zipf(1.1) top-6 routing), "
                "random-init",
        "tokens_per_s": round(n / t_step, 1),
        "cpu_baseline": cpu,
        "wall_s": round(wall, 4),
    }
    if cfg == 2:
        value = bytes_avg / t_step / 1e9
        achieved = bytes_avg / t_launch / 1e9
        res.update({
            "value": round(value, 2), "unit": "GB/s",
            "config": {"workload": "batched decode MoE: 64 tokens x top-6 of 256 FP4 experts "
                                   "(Zipf 1.1) + FP8 shared expert, grouped GEMM, SwiGLU, combine",
                       "tokens_per_step": n, "distinct_experts_avg": round(d_avg, 1),
                       "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic_for(cfg),
                         "kernel": "moe_grouped_dev call (route, fp16 convert, grouped gate/up, "
                                   "grouped down, shared gate/up + down, combine)",
                         "bytes_per_launch": round(bytes_avg), "launch_us": round(t_launch * 1e6, 3)},
        })
    else:
        value = flops_step / t_step / 1e12
        achieved = flops_step / t_launch / 1e12
        # composite bound: each distinct expert (and the shared one) at
        # max(bytes / HBM, flops / MFMA peak); the FP4 x FP8 and FP8 x FP8
        # block-scaled MFMA both issue at the FP8 rate on gfx950
        peak = FP8_PEAK_TFLOPS if mx else FP16_PEAK_TFLOPS
        j = (W) % nsets
        cnt = np.bincount(idx_h[n * j:n * (j + 1)].reshape(-1), minlength=N_EXPERTS)
        t_roof = sum(max(EXPERT_BYTES / (HBM_PEAK_GBS * 1e9),
                         2.0 * c * 3 * INTER * HIDDEN / (FP8_PEAK_TFLOPS * 1e12)) for c in cnt if c)
        t_roof += max(SHARED_BYTES / (HBM_PEAK_GBS * 1e9),
                      2.0 * n * 3 * INTER * HIDDEN / (FP8_PEAK_TFLOPS * 1e12))
        res.update({
            "value": round(value, 2), "unit": "TFLOP/s",
            "config": {"workload": "prefill MoE layer: 4096 tokens x top-6 of 256 FP4 experts "
                                   "(Zipf 1.1) + FP8 shared expert, permute, grouped GEMM with "
                                   "SwiGLU, combine",
                       "tokens_per_step": n, "distinct_experts_avg": round(d_avg, 1),
                       "parallelism": "single GPU"},
            "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
                         "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                         "traffic": traffic_for(cfg),
                         "kernel": ("moe_grouped_mx_dev call (route, MXFP8 quantize, block-scaled "
                                    "grouped gate/up, grouped down, shared 1x128 FP8 quantize, gate and up "
                                    "GEMMs, SwiGLU + quantize, down GEMM on the side stream, combine)") if mx else
                                   ("moe_grouped_dev call (route, fp16 convert, grouped gate/up, "
                                    "grouped down, shared gate/up + down, combine)"),
                         "flops_per_launch": flops_step, "launch_us": round(t_launch * 1e6, 3),
                         "composite_t_roof_us": round(t_roof * 1e6, 1),
                         "composite_frac": round(t_roof / t_launch, 4)},
            "other_path": other,
        })
    return res


def bench_cfg3(args, torch, pkg, lib, stream, sp, K, W):
    M, N, KD = 2048, 4096, 4096
    flops = 2.0 * M * N * KD
    dev = "cuda:0"
    log("generating the 4096x4096 FP8 weight and 2048x4096 bf16 activations")
    tmp = torch.empty(N * KD, dtype=torch.float32, device=dev)
    Wd = torch.empty(N * KD, dtype=torch.uint8, device=dev)
    Sd = torch.empty((N // 128) * (KD // 128), dtype=torch.float32, device=dev)
    lib.synth_normal_dev(tmp.data_ptr(), tmp.numel(), 0xD5EED003, 0.02)
    lib.quant_fp8_blk128_dev(Wd.data_ptr(), Sd.data_ptr(), tmp.data_ptr(), N, KD)
    af = torch.empty(M * KD, dtype=torch.float32, device=dev)
    lib.synth_normal_dev(af.data_ptr(), af.numel(), 0xD5EED003 ^ 0x55, 1.0, True)
    A = af.bfloat16()
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    Aq = torch.empty(M * KD, dtype=torch.uint8, device=dev)
    Sa = torch.empty(M * KD // 128, dtype=torch.float32, device=dev)
    lib.quant_act_fp8_1x128_dev(Aq.data_ptr(), Sa.data_ptr(), af.data_ptr(), M, KD)
    desc = pkg.qmat(pkg.DSV4_WFP8_F32S, Wd.data_ptr(), Sd.data_ptr(), N, KD, 128, 128)
    torch.cuda.synchronize()

    def step(i):
        lib.gemm_fp8_dev(C.data_ptr(), 1, A.data_ptr(), 1, M, desc, sp)

    def gemm_only(i):
        lib.gemm_fp8q_dev(C.data_ptr(), 1, Aq.data_ptr(), Sa.data_ptr(), M, desc, sp)

    for i in range(W):
        step(i)
    torch.cuda.synchronize()
    log(f"timing {K} steps")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(K):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_step = e0.elapsed_time(e1) * 1e-3 / K
    t_gemm = time_events(torch, stream, gemm_only, K)
    value = flops / t_step / 1e12
    achieved = flops / t_gemm / 1e12
    # the same GEMM in the checkpoint's own FP8 format: E8M0 128x128 weight
    # scales (the power of two at or above each fp32 scale) and MXFP8 tokens,
    # both in the MFMA's hardware scale operands (dsv4_hip_gemm_mxfp8_dev)
    Se = torch.from_numpy(fp8_e8m0(torch, Sd)).to(dev)
    desc_e = pkg.qmat(pkg.DSV4_WFP8, Wd.data_ptr(), Se.data_ptr(), N, KD, 128, 128)
    Aqm = torch.empty(M * KD, dtype=torch.uint8, device=dev)
    Asm = torch.empty(M * KD // 32, dtype=torch.uint8, device=dev)
    lib.quant_act_mxfp8_dev(Aqm.data_ptr(), Asm.data_ptr(), af.data_ptr(), M, KD)

    def step_mx(i):
        lib.gemm_mxfp8_dev(C.data_ptr(), 1, A.data_ptr(), 1, M, desc_e, sp)

    def gemm_only_mx(i):
        lib.gemm_mxfp8q_dev(C.data_ptr(), 1, Aqm.data_ptr(), Asm.data_ptr(), M, desc_e, sp)

    for i in range(W):
        step_mx(i)
    t_step_mx = time_events(torch, stream, step_mx, K)
    t_gemm_mx = time_events(torch, stream, gemm_only_mx, K)
    checkpoint = {"entry": "dsv4_hip_gemm_mxfp8_dev",
                  "format": "e4m3 W with E8M0 128x128 scales, bf16 A quantized on the fly to MXFP8 "
                            "(e4m3 + E8M0 per 1x32), bf16 out",
                  "ms_per_step": round(t_step_mx * 1e3, 5),
                  "tflops_step": round(flops / t_step_mx / 1e12, 2),
                  "gemm_launch_us": round(t_gemm_mx * 1e6, 3),
                  "gemm_tflops": round(flops / t_gemm_mx / 1e12, 2),
                  "gemm_frac": round(flops / t_gemm_mx / 1e12 / FP8_PEAK_TFLOPS, 4)}
    # the drop-in seam: dsv4_mmq_n's own form (fp32 x and y, no quantization
    # of x beyond the exact power-of-two row scaling and fp16 rounding) on the
    # same weight, as the prefill projections call it (src/80_prefill/
    # dsv4_prefill_proj.c:21-24); the dense fp16-MFMA GEMM plus its x converter
    y32 = torch.empty(M * N, dtype=torch.float32, device=dev)

    def seam(i):
        lib.mmq_n_dev(y32.data_ptr(), af.data_ptr(), desc, M, sp)

    for i in range(W):
        seam(i)
    t_seam = time_events(torch, stream, seam, K)
    seam_rec = {"entry": "dsv4_hip_mmq_n_dev (fp32 x [2048x4096], fp32 y)",
                "path": "x rows scaled by a power of two and rounded to fp16 (k_to_f16_rows), then "
                        "k_gemm_seam: 128x256 tiles, e4m3 weights decoded exactly to fp16 in "
                        "registers, fp16 MFMA, fp32 block-scale promotion",
                "ms_per_call": round(t_seam * 1e3, 5),
                "tflops": round(flops / t_seam / 1e12, 2),
                "frac_of_fp16_peak": round(flops / t_seam / 1e12 / FP16_PEAK_TFLOPS, 4)}
    cpu = None
    if not args.no_cpu:
        # the reference's fp8_n, nt > 1 body (src/10_compute/dsv4_matmul_fp8.c:
        # 102-155), on the same weight with E8M0 block scales; unit: one
        # 128-token tile (dsv4_mmq_n's tile) of the activations
        cpu = cpu_baseline("fp8_gemm", {"w": Wd.cpu().numpy(), "s": fp8_e8m0(torch, Sd),
                                        "x": A.view(M, KD)[:128].float().cpu().numpy()},
                           {}, 2.0 * 128 * N * KD / 1e12, "TFLOP/s",
                           "128 tokens x 4096x4096 e4m3 (E8M0 block scales) through fp8_n",
                           args.cpu_seconds, args.cpu_threads)
    return {
        "metric": "quant matvec HBM GB/s (% peak); prefill FP4/FP8 GEMM TFLOP/s (% MFMA peak)",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(t_step * 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8 e4m3 x e4m3 (fp32 block scales), fp32 accumulate, bf16 out",
        "data": "synthetic (seeded bf16 N(0,1) activations, N(0,0.02) weight), random-init",
        "config": {"workload": "prefill FP8 GEMM 2048x4096x4096: bf16 A quantized on the fly "
                               "(e4m3, fp32 1x128 scales), e4m3 W (fp32 128x128 scales), bf16 out",
                   "tokens": M, "n": N, "k": KD, "parallelism": "single GPU"},
        "tokens_per_s": round(M / t_step, 1),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP8_PEAK_TFLOPS, 4),
                     "traffic": traffic_for(3), "kernel": "k_gemm_fp8<true,true>",
                     "flops_per_launch": flops, "launch_us": round(t_gemm * 1e6, 3)},
        "step_includes": "activation quantization kernel + GEMM kernel",
        "checkpoint_format": checkpoint,
        "drop_in_seam": seam_rec,
        "cpu_baseline": cpu,
        "wall_s": round(wall, 4),
    }


# ------------------------------------------------------------------ main ----

def bench_layer(torch, pkg, lib, arena, xs, K, W, graph_calls=16):
    """The decode step's MoE block with the router on the device
    (dsv4_hip_moe_layer_dev: BF16 gate 256 x 4096 matvec, sqrt-softplus
    top-6 with a bias, the six routed experts): per-token time enqueued
    eagerly, and replayed from a HIP graph of `graph_calls` consecutive tokens
    captured on a side stream. Each token is its own x, so each picks its own
    experts from the 3.4 GB arena. Then the same block with the FP8 shared
    expert, which runs beside the gate and the router, next to the routed
    experts plus the shared expert with the routing already known
    (dsv4_hip_moe_decode_dev)."""
    dev = "cuda:0"
    tmp = torch.empty(N_EXPERTS * HIDDEN, dtype=torch.float32, device=dev)
    lib.synth_normal_dev(tmp.data_ptr(), tmp.numel(), 0x6A7E, 0.02)
    gw = tmp.bfloat16()
    gate = pkg.qmat(pkg.DSV4_WBF16, gw.data_ptr(), None, N_EXPERTS, HIDDEN, 0, 0)
    bias = torch.empty(N_EXPERTS, dtype=torch.float32, device=dev)
    lib.synth_normal_dev(bias.data_ptr(), N_EXPERTS, 0x6A7F, 0.05)
    shared, keep = make_shared_fp8(torch, pkg, lib, 0x6A80)
    out = torch.empty(HIDDEN, dtype=torch.float32, device=dev)
    di = torch.empty(TOPK, dtype=torch.int32, device=dev)
    dw = torch.empty(TOPK, dtype=torch.float32, device=dev)
    st = torch.cuda.Stream()
    n_x = xs.numel() // HIDDEN
    idx_h, w_h = routing(n_x, seed=0x6A81)
    didx = torch.from_numpy(idx_h).to(dev)
    dwts = torch.from_numpy(w_h).to(dev)

    def call(i, s=None, sh=None):
        lib.moe_layer_dev(out.data_ptr(), xs.data_ptr() + 4 * HIDDEN * (i % n_x), gate,
                          arena.table.data_ptr(), N_EXPERTS, TOPK, 2.5, sh, HIDDEN, INTER, 10.0,
                          bias_ptr=bias.data_ptr(), idx_ptr=di.data_ptr(), w_ptr=dw.data_ptr(),
                          stream=s)

    def known(i, s=None):
        j = i % n_x
        lib.moe_decode_dev(out.data_ptr(), xs.data_ptr() + 4 * HIDDEN * j, arena.table.data_ptr(),
                           N_EXPERTS, didx.data_ptr() + 4 * TOPK * j, dwts.data_ptr() + 4 * TOPK * j,
                           TOPK, shared, HIDDEN, INTER, 10.0, s)

    torch.cuda.synchronize()
    ss = st.cuda_stream
    with torch.cuda.stream(st):
        for i in range(W):
            call(i, ss)
            call(i, ss, shared)
            known(i, ss)
        torch.cuda.synchronize()
        t_eager = time_events(torch, st, lambda i: call(W + i, ss), K)
        t_shared = time_events(torch, st, lambda i: call(W + i, ss, shared), K)
        t_known = time_events(torch, st, lambda i: known(W + i, ss), K)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            for i in range(graph_calls):
                call(W + K + i, ss)
        torch.cuda.synchronize()
        reps = max(1, K // graph_calls)
        graph.replay()
        torch.cuda.synchronize()
        t_graph = time_events(torch, st, lambda i: graph.replay(), reps) / graph_calls
    assert lib.status() == 0
    b = TOPK * EXPERT_BYTES + N_EXPERTS * HIDDEN * 2 + 8192 + 16384
    return {"entry": "dsv4_hip_moe_layer_dev (gate matvec + router + routed experts, no host "
                     "round trip)",
            "bytes_per_token": b,
            "eager_us": round(t_eager * 1e6, 3), "graph_us": round(t_graph * 1e6, 3),
            "graph_calls": graph_calls,
            "eager_GBs": round(b / t_eager / 1e9, 1), "graph_GBs": round(b / t_graph / 1e9, 1),
            "with_shared_us": round(t_shared * 1e6, 3),
            "known_routing_with_shared_us": round(t_known * 1e6, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=[0, 1, 2, 3, 4])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-other", action="store_true",
                    help="config 4: skip timing the other precision path (counter runs)")
    ap.add_argument("--no-others", action="store_true",
                    help="config 1: do not run configs 0, 2, 3 and 4 as child processes "
                         "(their lines go into other_configs)")
    ap.add_argument("--exact", action="store_true",
                    help="config 4: time the exact fp16-MFMA grouped path as the value instead "
                         "of the block-scaled one")
    ap.add_argument("--cpu-worker", metavar="SPEC",
                    help="internal: run one CPU-baseline measurement described by SPEC and exit")
    ap.add_argument("--copy-calib", action="store_true",
                    help="run only a plain 256 MiB device copy (the HBM-counter calibration "
                         "kernel for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.cpu_worker:
        _cpu_worker(args.cpu_worker)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calib:
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_read": n, "copy_calib_bytes_written": n,
                          "calls": args.steps}), flush=True)
        return
    pkg = load_pkg()
    lib = pkg.load()
    lib.check(lib.init(0), "dsv4_hip_init")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    K, W = args.steps, args.warmup

    if args.config == 1:
        log("generating 256 FP4 experts on the device")
        arena = ExpertArena(torch, pkg, lib, N_EXPERTS, seed=0xD5EED001)
        idx_h, w_h = routing(K + W + K, seed=0xD5EED001)
        idx = torch.from_numpy(idx_h).to("cuda:0")
        wts = torch.from_numpy(w_h).to("cuda:0")
        xs = torch.empty((K + W + K) * HIDDEN, dtype=torch.float32, device="cuda:0")
        lib.synth_normal_dev(xs.data_ptr(), xs.numel(), 0xD5EED001 ^ 0x55, 1.0, True)
        out = torch.empty(HIDDEN, dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()

        # The router of the reference runs on the host (src/70_decode/dsv4_layer.c:57-116):
        # the timed path takes each token's top-6 ids and weights from the host and
        # passes the six descriptors by value (dsv4_hip_moe_decode_routed_dev). The
        # device-routed form (ids / weights in HBM, dsv4_hip_moe_decode_dev) is timed too.
        ex_arr = (pkg.ExpertW * N_EXPERTS)(*arena.descs)
        ids_c = [(C.c_int * TOPK)(*[int(v) for v in idx_h[i]]) for i in range(K + W + K)]
        wts_c = [(C.c_float * TOPK)(*[float(v) for v in w_h[i]]) for i in range(K + W + K)]
        routed_fn = lib.lib.dsv4_hip_moe_decode_routed_dev

        def step(i):
            if routed_fn(out.data_ptr(), xs.data_ptr() + 4 * HIDDEN * i, ex_arr, N_EXPERTS,
                         ids_c[i], wts_c[i], TOPK, None, HIDDEN, INTER, C.c_float(10.0), sp):
                lib.check(-1, "dsv4_hip_moe_decode_routed_dev")

        def step_dev(i):
            lib.moe_decode_dev(out.data_ptr(), xs.data_ptr() + 4 * HIDDEN * i,
                               arena.table.data_ptr(), N_EXPERTS,
                               idx.data_ptr() + 4 * TOPK * i, wts.data_ptr() + 4 * TOPK * i,
                               TOPK, None, HIDDEN, INTER, 10.0, sp)

        for i in range(W):
            step(i)
            step_dev(i)
        torch.cuda.synchronize()
        assert lib.status() == 0
        log(f"timing {K} steps")

        def timed(fn):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(K):
                fn(W + i)
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e-3 / K

        t0 = time.perf_counter()
        t_step = timed(step)
        wall = time.perf_counter() - t0
        t_step_dev = timed(step_dev)
        # average launch durations on fresh weight sets
        t_launch = time_events(torch, stream, lambda i: step(W + K + i), K)
        t_launch_dev = time_events(torch, stream, lambda i: step_dev(W + K + i), K)
        assert lib.status() == 0
        layer = bench_layer(torch, pkg, lib, arena, xs, K, W)
        dlayer = bench_decode_layer(torch, pkg, lib, arena, xs)
        bytes_step = TOPK * EXPERT_BYTES + 8192 + 16384
        value = bytes_step / t_step / 1e9
        achieved = bytes_step / t_launch / 1e9
        cpu = None
        if not args.no_cpu:
            # the reference's decode path on the host: dsv4_expert_forward x 6
            # (src/10_compute/dsv4_ops.c:85-93) and the k-order combine, each
            # unit a token routed to 6 of 64 host-resident experts (856 MB,
            # beyond the host LLC), copied in the reference's slot layout
            nh = 64
            slots = arena.buf[:nh * EXPERT_BYTES].cpu().numpy().reshape(nh, EXPERT_BYTES)
            cpu = cpu_baseline("decode_token", {"experts": slots, "x": xs[:HIDDEN].cpu().numpy()},
                               {}, (TOPK * EXPERT_BYTES + 8192 + 16384) / 1e9, "GB/s",
                               f"one token x top-6 of {nh} host-resident FP4 experts through "
                               f"dsv4_expert_forward and the combine",
                               args.cpu_seconds, args.cpu_threads)
        res = {
            "metric": "quant matvec HBM GB/s (% peak); prefill FP4/FP8 GEMM TFLOP/s (% MFMA peak)",
            "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": W,
            "ms_per_step": round(t_step * 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp4 e2m1 weights, fp32 accumulate",
            "data": "synthetic (seeded N(0,0.02) experts, bf16 N(0,1) token), random-init",
            "config": {"workload": "single-token FP4 MoE expert FFN decode: 256 resident experts, "
                                   "top-6, gate/up 2048x4096 + down 4096x2048, SwiGLU, combine",
                       "tokens_per_step": 1, "hidden": HIDDEN, "moe_inter": INTER,
                       "n_experts": N_EXPERTS, "topk": TOPK, "parallelism": "single GPU"},
            "tokens_per_s": round(1.0 / t_step, 1),
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic_for(1),
                         "kernel": "moe_decode_routed_dev call (k_moe_one: gate/up and down workgroups in one launch)",
                         "bytes_per_launch": bytes_step,
                         "launch_us": round(t_launch * 1e6, 3)},
            "device_routed": {"entry": "dsv4_hip_moe_decode_dev (ids and weights in HBM)",
                              "ms_per_step": round(t_step_dev * 1e3, 5),
                              "value": round(bytes_step / t_step_dev / 1e9, 2),
                              "launch_us": round(t_launch_dev * 1e6, 3)},
            "moe_layer": layer,
            "decode_layer": dlayer,
            "cpu_baseline": cpu,
            "wall_s": round(wall, 4),
        }
    elif args.config in (2, 4):
        if args.config == 4 and K > 50:
            K, W = 50, min(W, 5)      # about 1 ms per step; keeps the timed region short
        res = bench_grouped(args, torch, pkg, lib, stream, sp, K, W, args.config)
    elif args.config == 3:
        res = bench_cfg3(args, torch, pkg, lib, stream, sp, K, W)
    else:
        ncopy = 40
        log(f"generating {ncopy} copies of a 4096x4096 FP8 matrix")
        Wd = torch.empty(ncopy * 4096 * 4096, dtype=torch.uint8, device="cuda:0")
        Sd = torch.empty(ncopy * 32 * 32, dtype=torch.float32, device="cuda:0")
        tmp = torch.empty(4096 * 4096, dtype=torch.float32, device="cuda:0")
        for c in range(ncopy):
            lib.synth_normal_dev(tmp.data_ptr(), tmp.numel(), 0xD5EED000 + c, 0.02)
            lib.quant_fp8_blk128_dev(Wd.data_ptr() + c * 4096 * 4096,
                                     Sd.data_ptr() + 4 * c * 1024, tmp.data_ptr(), 4096, 4096)
        xs = torch.empty(4096, dtype=torch.float32, device="cuda:0")
        lib.synth_normal_dev(xs.data_ptr(), 4096, 0xD5EED000 ^ 0x55, 1.0, True)
        y = torch.empty(4096, dtype=torch.float32, device="cuda:0")
        descs = [pkg.qmat(pkg.DSV4_WFP8_F32S, Wd.data_ptr() + c * 4096 * 4096,
                          Sd.data_ptr() + 4 * c * 1024, 4096, 4096, 128, 128) for c in range(ncopy)]
        torch.cuda.synchronize()

        def step(i):
            lib.mmq_n_dev(y.data_ptr(), xs.data_ptr(), descs[i % ncopy], 1, sp)

        for i in range(W):
            step(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(K):
            step(i)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        t_step = e0.elapsed_time(e1) * 1e-3 / K
        t_launch = time_events(torch, stream, step, K)
        bytes_step = 16_805_888
        value = bytes_step / t_step / 1e9
        cpu = None
        if not args.no_cpu:
            # the reference's fp8_n with nt = 1 (src/10_compute/dsv4_matmul_fp8.c:
            # 57-99) on the first weight copy (16.8 MB, beyond the host LLC)
            cpu = cpu_baseline("fp8_matvec", {"w": Wd[:4096 * 4096].cpu().numpy(),
                                              "s": fp8_e8m0(torch, Sd[:1024]),
                                              "x": xs.cpu().numpy()},
                               {}, bytes_step / 1e9, "GB/s",
                               "one 4096x4096 e4m3 matvec (E8M0 block scales) through fp8_n",
                               args.cpu_seconds, args.cpu_threads)
        res = {
            "metric": "quant matvec HBM GB/s (% peak); prefill FP4/FP8 GEMM TFLOP/s (% MFMA peak)",
            "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": W,
            "ms_per_step": round(t_step * 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp8 e4m3 weights, fp32 accumulate",
            "data": "synthetic (seeded), random-init",
            "config": {"workload": "FP8 matvec 4096x4096, fp32 128x128 scales, bf16 x",
                       "copies_rotated": ncopy, "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "achieved": round(bytes_step / t_launch / 1e9, 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(bytes_step / t_launch / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": traffic_for(0), "kernel": "k_gemv_px8<FP8_F32S,4,4,2>",
                         "bytes_per_launch": bytes_step, "launch_us": round(t_launch * 1e6, 3)},
            "cpu_baseline": cpu,
            "wall_s": round(wall, 4),
        }
    if args.config == 1 and not args.no_others:
        res["other_configs"] = other_configs(args)
    print(json.dumps(res), flush=True)


def other_configs(args):
    """Configs 0, 2, 3 and 4, each in a child process of this one (its own
    data and HIP context, nothing else on the GPU meanwhile), so that the
    default run times every workload: their JSON lines keyed by config, each
    with its CPU baseline (a shorter sample than config 1's) unless --no-cpu."""
    out = {}
    for c, steps in ((0, 200), (2, 50), (3, 100), (4, 30)):
        cmd = [sys.executable, os.path.abspath(__file__), "--config", str(c),
               "--steps", str(steps), "--warmup", str(min(args.warmup, 5))]
        cmd += ["--no-cpu"] if args.no_cpu else ["--cpu-seconds", str(min(args.cpu_seconds, 4.0))]
        if args.cpu_threads:
            cmd += ["--cpu-threads", str(args.cpu_threads)]
        log(f"config {c} in a child process")
        r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=600)
        lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
        if r.returncode != 0 or not lines:
            out[str(c)] = {"error": f"exit {r.returncode}"}
            continue
        out[str(c)] = json.loads(lines[-1])
    return out


if __name__ == "__main__":
    main()
