# SPDX-License-Identifier: Apache-2.0
"""Python binding of the gfx950 quantized-matmul library (lib/libdsv4_hip.so).

The product is the C ABI declared in include/dsv4_hip.h and
include/dsv4_hip_aux.h; this module binds it with ctypes for tests and the
benchmark. Host-pointer calls take numpy arrays; _dev calls take device
addresses (e.g. torch tensors' data_ptr()) and a HIP stream handle.

Importing fails loudly when the library has not been built: there is no
fallback implementation behind this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
HIP_SO = os.path.join(LIB_DIR, "libdsv4_hip.so")
AMD_SO = os.path.join(LIB_DIR, "libdsv4_amd.so")

# src/00_base/dsv4.h:86 plus this library's DSV4_WFP8_F32S
DSV4_WF32, DSV4_WBF16, DSV4_WFP8, DSV4_WFP4, DSV4_WFP8_F32S = 0, 1, 2, 3, 4

# every symbol include/*.h declares
EXPORTS = (
    "dsv4_hip_init", "dsv4_hip_shutdown", "dsv4_hip_last_error",
    "dsv4_hip_register", "dsv4_hip_unregister", "dsv4_hip_device_ptr",
    "dsv4_hip_mmq_n", "dsv4_hip_mmq", "dsv4_hip_mmq_n_dev",
    "dsv4_hip_expert_forward", "dsv4_hip_moe_decode", "dsv4_hip_moe_decode_dev",
    "dsv4_hip_moe_decode_routed_dev", "dsv4_hip_moe_decode_routed_noalloc_dev",
    "dsv4_hip_moe_grouped", "dsv4_hip_moe_grouped_dev", "dsv4_hip_moe_grouped_mx_dev",
    "dsv4_hip_status", "dsv4_hip_gemm_fp8_dev", "dsv4_hip_gemm_fp8q_dev",
    "dsv4_hip_gemm_mxfp8_dev", "dsv4_hip_gemm_mxfp8q_dev",
    "dsv4_hip_load_experts", "dsv4_hip_free_experts",
    "dsv4_hip_dequant_dev", "dsv4_hip_quant_fp8_blk128_dev",
    "dsv4_hip_quant_fp4_mx_dev", "dsv4_hip_quant_act_fp8_1x128_dev",
    "dsv4_hip_quant_act_mxfp8_dev", "dsv4_hip_synth_normal_dev", "dsv4_hip_moe_route_dev",
    "dsv4_hip_moe_grouped_mx_mid_dev", "dsv4_hip_shared_fp8q_mid_dev",
    "dsv4_hip_route_dev", "dsv4_hip_moe_layer_dev", "dsv4_hip_moe_layer_n_dev",
    "dsv4_hip_alloc_count", "dsv4_hip_mmq_multi_dev",
)
# the reference-named C mirror (host/dsv4_compute_hip.c)
MIRROR_EXPORTS = ("dsv4_mmq_n", "dsv4_mmq", "dsv4_expert_forward")


class QMat(C.Structure):
    """DSV4QMat (src/00_base/dsv4_weights.h:34-40)."""
    _fields_ = [("w", C.c_void_p), ("s", C.c_void_p), ("wdt", C.c_int),
                ("rows", C.c_int), ("cols", C.c_int),
                ("blk_r", C.c_int), ("blk_c", C.c_int)]


class HipJob(C.Structure):
    """DSV4HipJob: DSV4PMJob's fields (src/80_prefill/dsv4_prefill_int.h:21-28)."""
    _fields_ = [("m", C.POINTER(QMat)), ("x", C.c_void_p), ("y", C.c_void_p), ("n", C.c_int)]


class ExpertW(C.Structure):
    """DSV4ExpertW (src/00_base/dsv4_weights.h:103-106)."""
    _fields_ = [("w1", QMat), ("w3", QMat), ("w2", QMat)]


_P, _I, _F = C.c_void_p, C.c_int, C.c_float


def weight_bytes(wdt, rows, cols):
    return rows * (cols // 2) if wdt == DSV4_WFP4 else rows * cols


def scale_entries(rows, cols, blk_r, blk_c):
    return ((rows + blk_r - 1) // blk_r) * ((cols + blk_c - 1) // blk_c)


def scale_bytes(wdt, rows, cols, blk_r, blk_c):
    n = scale_entries(rows, cols, blk_r, blk_c)
    return 4 * n if wdt == DSV4_WFP8_F32S else n


class Dsv4Error(RuntimeError):
    pass


class Lib:
    """ctypes view of libdsv4_hip.so."""

    def __init__(self, path: str = HIP_SO):
        if not os.path.exists(path):
            raise Dsv4Error(f"{path} is not built: run __graft_entry__.build()")
        self.path = path
        self._registered = {}
        L = self.lib = C.CDLL(path)
        L.dsv4_hip_init.restype = _I; L.dsv4_hip_init.argtypes = [_I]
        L.dsv4_hip_shutdown.restype = None; L.dsv4_hip_shutdown.argtypes = []
        L.dsv4_hip_last_error.restype = C.c_char_p; L.dsv4_hip_last_error.argtypes = []
        L.dsv4_hip_alloc_count.restype = C.c_ulonglong; L.dsv4_hip_alloc_count.argtypes = []
        L.dsv4_hip_register.restype = _I; L.dsv4_hip_register.argtypes = [_P, C.c_size_t]
        L.dsv4_hip_unregister.restype = _I; L.dsv4_hip_unregister.argtypes = [_P]
        L.dsv4_hip_device_ptr.restype = _P; L.dsv4_hip_device_ptr.argtypes = [_P]
        L.dsv4_hip_mmq_n.restype = _I
        L.dsv4_hip_mmq_n.argtypes = [_P, _P, C.POINTER(QMat), _I]
        L.dsv4_hip_mmq.restype = _I; L.dsv4_hip_mmq.argtypes = [_P, _P, C.POINTER(QMat)]
        L.dsv4_hip_mmq_n_dev.restype = _I
        L.dsv4_hip_mmq_n_dev.argtypes = [_P, _P, C.POINTER(QMat), _I, _P]
        L.dsv4_hip_mmq_multi_dev.restype = _I
        L.dsv4_hip_mmq_multi_dev.argtypes = [C.POINTER(HipJob), _I, _P]
        L.dsv4_hip_expert_forward.restype = _I
        L.dsv4_hip_expert_forward.argtypes = [_P, _P, C.POINTER(ExpertW), _I, _F]
        L.dsv4_hip_moe_decode.restype = _I
        L.dsv4_hip_moe_decode.argtypes = [_P, _P, C.POINTER(C.POINTER(ExpertW)), _P, _I,
                                          C.POINTER(ExpertW), _F]
        L.dsv4_hip_moe_decode_dev.restype = _I
        L.dsv4_hip_moe_decode_dev.argtypes = [_P, _P, _P, _I, _P, _P, _I,
                                              C.POINTER(ExpertW), _I, _I, _F, _P]
        for n in ("dsv4_hip_moe_decode_routed_dev", "dsv4_hip_moe_decode_routed_noalloc_dev"):
            getattr(L, n).restype = _I
            getattr(L, n).argtypes = [_P, _P, C.POINTER(ExpertW), _I, C.POINTER(_I),
                                      C.POINTER(_F), _I, C.POINTER(ExpertW), _I, _I, _F, _P]
        L.dsv4_hip_moe_grouped.restype = _I
        L.dsv4_hip_moe_grouped.argtypes = [_P, _P, _I, _P, _P, _I, C.POINTER(ExpertW), _I,
                                           C.POINTER(ExpertW), _F]
        for n in ("dsv4_hip_moe_grouped_dev", "dsv4_hip_moe_grouped_mx_dev"):
            getattr(L, n).restype = _I
            getattr(L, n).argtypes = [_P, _P, _I, _P, _I, _P, _P, _I, C.POINTER(ExpertW), _I, _I,
                                      _F, _P]
        L.dsv4_hip_status.restype = _I; L.dsv4_hip_status.argtypes = [C.POINTER(C.c_uint)]
        L.dsv4_hip_gemm_fp8_dev.restype = _I
        L.dsv4_hip_gemm_fp8_dev.argtypes = [_P, _I, _P, _I, _I, C.POINTER(QMat), _P]
        L.dsv4_hip_gemm_fp8q_dev.restype = _I
        L.dsv4_hip_gemm_fp8q_dev.argtypes = [_P, _I, _P, _P, _I, C.POINTER(QMat), _P]
        L.dsv4_hip_gemm_mxfp8_dev.restype = _I
        L.dsv4_hip_gemm_mxfp8_dev.argtypes = [_P, _I, _P, _I, _I, C.POINTER(QMat), _P]
        L.dsv4_hip_gemm_mxfp8q_dev.restype = _I
        L.dsv4_hip_gemm_mxfp8q_dev.argtypes = [_P, _I, _P, _P, _I, C.POINTER(QMat), _P]
        L.dsv4_hip_load_experts.restype = _P
        L.dsv4_hip_load_experts.argtypes = [C.c_char_p, C.c_char_p, _I, _I, _I, _P, _I, C.POINTER(_I)]
        L.dsv4_hip_free_experts.restype = _I
        L.dsv4_hip_free_experts.argtypes = [_P]
        L.dsv4_hip_dequant_dev.restype = _I
        L.dsv4_hip_dequant_dev.argtypes = [_P, C.POINTER(QMat), _P]
        for n in ("dsv4_hip_quant_fp8_blk128_dev", "dsv4_hip_quant_fp4_mx_dev",
                  "dsv4_hip_quant_act_fp8_1x128_dev", "dsv4_hip_quant_act_mxfp8_dev"):
            getattr(L, n).restype = _I
            getattr(L, n).argtypes = [_P, _P, _P, _I, _I, _P]
        L.dsv4_hip_synth_normal_dev.restype = _I
        L.dsv4_hip_synth_normal_dev.argtypes = [_P, C.c_size_t, C.c_uint64, _F, _I, _P]
        L.dsv4_hip_moe_route_dev.restype = _I
        L.dsv4_hip_moe_route_dev.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _P]
        L.dsv4_hip_route_dev.restype = _I
        L.dsv4_hip_route_dev.argtypes = [_P, _P, _P, _P, _I, _P, _P, _I, _P, _I, _I, _F, _P]
        L.dsv4_hip_moe_layer_n_dev.restype = _I
        L.dsv4_hip_moe_layer_n_dev.argtypes = [_P, _P, _I, C.POINTER(QMat), _P, _P, _I, _P, _F,
                                               _P, _I, _I, C.POINTER(ExpertW), _I, _I, _F, _I,
                                               _P, _P, _P]
        L.dsv4_hip_moe_layer_dev.restype = _I
        L.dsv4_hip_moe_layer_dev.argtypes = [_P, _P, C.POINTER(QMat), _P, _P, _I, _I, _F,
                                             _P, _I, _I, C.POINTER(ExpertW), _I, _I, _F,
                                             _P, _P, _P]
        L.dsv4_hip_moe_grouped_mx_mid_dev.restype = _I
        L.dsv4_hip_moe_grouped_mx_mid_dev.argtypes = [_P, _P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I,
                                                      _F, _P]
        L.dsv4_hip_shared_fp8q_mid_dev.restype = _I
        L.dsv4_hip_shared_fp8q_mid_dev.argtypes = [_P, _P, _P, _I, _P, _I, _F, _P]

    # ------------------------------------------------------------ basics
    def alloc_count(self) -> int:
        """hipMalloc calls the library has made since it was loaded."""
        return int(self.lib.dsv4_hip_alloc_count())

    def error(self) -> str:
        return (self.lib.dsv4_hip_last_error() or b"").decode()

    def check(self, rc: int, what: str):
        if rc != 0:
            raise Dsv4Error(f"{what}: {self.error()}")

    def init(self, device: int = 0) -> int:
        return self.lib.dsv4_hip_init(device)

    def shutdown(self):
        self.lib.dsv4_hip_shutdown()

    def register(self, arr: np.ndarray) -> int:
        """Upload arr once; the array is kept alive (its address cannot be
        reused) until it is unregistered."""
        assert arr.flags["C_CONTIGUOUS"]
        rc = self.lib.dsv4_hip_register(arr.ctypes.data, arr.nbytes)
        if rc == 0:
            self._registered[arr.ctypes.data] = arr
        return rc

    def unregister(self, arr: np.ndarray) -> int:
        self._registered.pop(arr.ctypes.data, None)
        return self.lib.dsv4_hip_unregister(arr.ctypes.data)

    def unregister_all(self) -> int:
        """Drop every range this binding registered; returns how many."""
        live = list(self._registered.values())
        for a in live:
            self.unregister(a)
        return len(live)

    def status(self) -> int:
        v = C.c_uint(0)
        self.check(self.lib.dsv4_hip_status(C.byref(v)), "status")
        return v.value

    # ------------------------------------------------ host-pointer entry points
    def mmq_n(self, desc: QMat, x: np.ndarray, nt: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        assert x.size >= nt * desc.cols
        y = np.zeros(nt * desc.rows, np.float32)
        self.check(self.lib.dsv4_hip_mmq_n(y.ctypes.data, x.ctypes.data, C.byref(desc), nt),
                   "dsv4_hip_mmq_n")
        return y

    def mmq_n_rc(self, desc: QMat, x: np.ndarray, nt: int = 1) -> int:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(max(nt, 1) * desc.rows, np.float32)
        return self.lib.dsv4_hip_mmq_n(y.ctypes.data, x.ctypes.data, C.byref(desc), nt)

    def expert_forward(self, e: ExpertW, x: np.ndarray, limit: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(e.w1.cols, np.float32)
        self.check(self.lib.dsv4_hip_expert_forward(out.ctypes.data, x.ctypes.data,
                                                    C.byref(e), e.w1.rows, float(limit)),
                   "dsv4_hip_expert_forward")
        return out

    def moe_decode(self, experts, w, x, shared=None, limit=10.0) -> np.ndarray:
        topk = len(experts)
        arr = (C.POINTER(ExpertW) * topk)(*[C.pointer(e) for e in experts])
        w = np.ascontiguousarray(w, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(experts[0].w1.cols, np.float32)
        sp = C.pointer(shared) if shared is not None else None
        self.check(self.lib.dsv4_hip_moe_decode(out.ctypes.data, x.ctypes.data, arr,
                                                w.ctypes.data, topk, sp, float(limit)),
                   "dsv4_hip_moe_decode")
        return out

    def moe_grouped(self, experts, idx, w, x, shared=None, limit=10.0) -> np.ndarray:
        """experts: list of ExpertW (host pointers inside registered ranges);
        idx, w: [n][topk]; x: [n][hidden] fp32. Returns out [n][hidden]."""
        idx = np.ascontiguousarray(idx, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        n, topk = idx.shape
        arr = (ExpertW * len(experts))(*experts)
        out = np.zeros((n, experts[0].w1.cols), np.float32)
        sp = C.pointer(shared) if shared is not None else None
        self.check(self.lib.dsv4_hip_moe_grouped(out.ctypes.data, x.ctypes.data, n,
                                                 idx.ctypes.data, w.ctypes.data, topk, arr,
                                                 len(experts), sp, float(limit)),
                   "dsv4_hip_moe_grouped")
        return out

    # ---------------------------------------------------------- _dev entry points
    def mmq_n_dev(self, y_ptr, x_ptr, desc: QMat, nt, stream=None):
        self.check(self.lib.dsv4_hip_mmq_n_dev(y_ptr, x_ptr, C.byref(desc), nt, stream),
                   "dsv4_hip_mmq_n_dev")

    def mmq_multi_dev_rc(self, jobs, stream=None) -> int:
        """jobs: (QMat, x_ptr, y_ptr, n) tuples; returns the C return code. The
        descriptors must stay alive until the call returns."""
        descs = [d for d, _, _, _ in jobs]
        arr = (HipJob * max(1, len(jobs)))(*[HipJob(C.pointer(d), x, y, n) for d, (_, x, y, n) in zip(descs, jobs)])
        return self.lib.dsv4_hip_mmq_multi_dev(arr, len(jobs), stream)

    def mmq_multi_dev(self, jobs, stream=None):
        self.check(self.mmq_multi_dev_rc(jobs, stream), "dsv4_hip_mmq_multi_dev")

    def moe_decode_dev(self, out_ptr, x_ptr, table_ptr, n_experts, idx_ptr, w_ptr, topk,
                       shared: ExpertW | None, hidden, inter, limit, stream=None):
        sp = C.pointer(shared) if shared is not None else None
        self.check(self.lib.dsv4_hip_moe_decode_dev(out_ptr, x_ptr, table_ptr, n_experts,
                                                    idx_ptr, w_ptr, topk, sp, hidden, inter,
                                                    float(limit), stream),
                   "dsv4_hip_moe_decode_dev")

    def moe_decode_routed_dev(self, out_ptr, x_ptr, experts, idx, w, topk,
                              shared: ExpertW | None, hidden, inter, limit, stream=None):
        """experts: a ctypes array of ExpertW (device pointers); idx, w: host
        sequences of topk routing ids and weights."""
        sp = C.pointer(shared) if shared is not None else None
        ia = (_I * topk)(*[int(i) for i in idx[:topk]])
        wa = (_F * topk)(*[float(v) for v in w[:topk]])
        self.check(self.lib.dsv4_hip_moe_decode_routed_dev(out_ptr, x_ptr, experts, len(experts),
                                                           ia, wa, topk, sp, hidden, inter,
                                                           float(limit), stream),
                   "dsv4_hip_moe_decode_routed_dev")

    def moe_decode_routed_noalloc_dev_rc(self, out_ptr, x_ptr, experts, idx, w, topk,
                                         shared: ExpertW | None, hidden, inter, limit,
                                         stream=None) -> int:
        """The allocation-free twin; returns the C return code."""
        sp = C.pointer(shared) if shared is not None else None
        ia = (_I * topk)(*[int(i) for i in idx[:topk]])
        wa = (_F * topk)(*[float(v) for v in w[:topk]])
        return self.lib.dsv4_hip_moe_decode_routed_noalloc_dev(out_ptr, x_ptr, experts, len(experts),
                                                               ia, wa, topk, sp, hidden, inter,
                                                               float(limit), stream)

    def moe_grouped_dev(self, out_ptr, x_ptr, n, table_ptr, n_experts, idx_ptr, w_ptr, topk,
                        shared: ExpertW | None, hidden, inter, limit, stream=None):
        sp = C.pointer(shared) if shared is not None else None
        self.check(self.lib.dsv4_hip_moe_grouped_dev(out_ptr, x_ptr, n, table_ptr, n_experts,
                                                     idx_ptr, w_ptr, topk, sp, hidden, inter,
                                                     float(limit), stream),
                   "dsv4_hip_moe_grouped_dev")

    def moe_grouped_mx_dev(self, out_ptr, x_ptr, n, table_ptr, n_experts, idx_ptr, w_ptr, topk,
                           shared: ExpertW | None, hidden, inter, limit, stream=None):
        sp = C.pointer(shared) if shared is not None else None
        self.check(self.lib.dsv4_hip_moe_grouped_mx_dev(out_ptr, x_ptr, n, table_ptr, n_experts,
                                                        idx_ptr, w_ptr, topk, sp, hidden, inter,
                                                        float(limit), stream),
                   "dsv4_hip_moe_grouped_mx_dev")

    def moe_grouped_mx_mid_dev(self, mid_ptr, mids_ptr, row_tok_ptr, row_k_ptr, x_ptr, n, table_ptr,
                               n_experts, idx_ptr, topk, hidden, inter, limit, stream=None):
        self.check(self.lib.dsv4_hip_moe_grouped_mx_mid_dev(mid_ptr, mids_ptr, row_tok_ptr, row_k_ptr,
                                                            x_ptr, n, table_ptr, n_experts, idx_ptr,
                                                            topk, hidden, inter, float(limit), stream),
                   "dsv4_hip_moe_grouped_mx_mid_dev")

    def shared_fp8q_mid_dev(self, mid_ptr, mids_ptr, x_ptr, n, shared: ExpertW, hidden, limit, stream=None):
        self.check(self.lib.dsv4_hip_shared_fp8q_mid_dev(mid_ptr, mids_ptr, x_ptr, n, C.byref(shared), hidden,
                                                         float(limit), stream),
                   "dsv4_hip_shared_fp8q_mid_dev")

    def gemm_fp8_dev(self, c_ptr, out_bf16, a_ptr, a_bf16, m, desc: QMat, stream=None):
        self.check(self.lib.dsv4_hip_gemm_fp8_dev(c_ptr, int(bool(out_bf16)), a_ptr,
                                                  int(bool(a_bf16)), m, C.byref(desc), stream),
                   "dsv4_hip_gemm_fp8_dev")

    def gemm_fp8q_dev(self, c_ptr, out_bf16, aq_ptr, sa_ptr, m, desc: QMat, stream=None):
        self.check(self.lib.dsv4_hip_gemm_fp8q_dev(c_ptr, int(bool(out_bf16)), aq_ptr, sa_ptr,
                                                   m, C.byref(desc), stream),
                   "dsv4_hip_gemm_fp8q_dev")

    def load_experts(self, model_dir, index_dir, layer, hidden, inter, max_experts=1024):
        """(arena, ctypes array of ExpertW with device pointers, n_experts)"""
        table = (ExpertW * max_experts)()
        n = _I(0)
        arena = self.lib.dsv4_hip_load_experts(model_dir.encode(), index_dir.encode(), layer, hidden, inter,
                                               C.cast(table, C.c_void_p), max_experts, C.byref(n))
        if not arena:
            raise Dsv4Error(f"dsv4_hip_load_experts: {self.error()}")
        return arena, table, n.value

    def free_experts(self, arena):
        self.check(self.lib.dsv4_hip_free_experts(arena), "dsv4_hip_free_experts")

    def gemm_mxfp8_dev(self, c_ptr, out_bf16, a_ptr, a_bf16, m, desc: QMat, stream=None):
        self.check(self.lib.dsv4_hip_gemm_mxfp8_dev(c_ptr, int(bool(out_bf16)), a_ptr,
                                                    int(bool(a_bf16)), m, C.byref(desc), stream),
                   "dsv4_hip_gemm_mxfp8_dev")

    def gemm_mxfp8q_dev(self, c_ptr, out_bf16, aq_ptr, as_ptr, m, desc: QMat, stream=None):
        self.check(self.lib.dsv4_hip_gemm_mxfp8q_dev(c_ptr, int(bool(out_bf16)), aq_ptr, as_ptr,
                                                     m, C.byref(desc), stream),
                   "dsv4_hip_gemm_mxfp8q_dev")

    def dequant_dev(self, out_ptr, desc: QMat, stream=None):
        self.check(self.lib.dsv4_hip_dequant_dev(out_ptr, C.byref(desc), stream),
                   "dsv4_hip_dequant_dev")

    def quant_fp8_blk128_dev(self, W, S, w, rows, cols, stream=None):
        self.check(self.lib.dsv4_hip_quant_fp8_blk128_dev(W, S, w, rows, cols, stream),
                   "quant_fp8_blk128_dev")

    def quant_fp4_mx_dev(self, W, S, w, rows, cols, stream=None):
        self.check(self.lib.dsv4_hip_quant_fp4_mx_dev(W, S, w, rows, cols, stream),
                   "quant_fp4_mx_dev")

    def quant_act_fp8_1x128_dev(self, Q, S, a, n, k, stream=None):
        self.check(self.lib.dsv4_hip_quant_act_fp8_1x128_dev(Q, S, a, n, k, stream),
                   "quant_act_fp8_1x128_dev")

    def quant_act_mxfp8_dev(self, Q, S, a, n, k, stream=None):
        self.check(self.lib.dsv4_hip_quant_act_mxfp8_dev(Q, S, a, n, k, stream),
                   "quant_act_mxfp8_dev")

    def synth_normal_dev(self, out_ptr, n, seed, sigma, round_bf16=False, stream=None):
        self.check(self.lib.dsv4_hip_synth_normal_dev(out_ptr, n, seed, float(sigma),
                                                      int(bool(round_bf16)), stream),
                   "synth_normal_dev")

    def moe_route_dev(self, ex_off_ptr, ex_tok_ptr, ex_k_ptr, pos_ptr, idx_ptr, n, topk,
                      n_experts, stream=None):
        self.check(self.lib.dsv4_hip_moe_route_dev(ex_off_ptr, ex_tok_ptr, ex_k_ptr, pos_ptr,
                                                   idx_ptr, n, topk, n_experts, stream),
                   "dsv4_hip_moe_route_dev")


    def route_dev(self, idx_ptr, w_ptr, orig_ptr, scores_ptr, n, n_experts, topk, route_scale,
                  bias_ptr=None, tid2eid_ptr=None, n_vocab=0, token_ids_ptr=None, stream=None):
        self.check(self.lib.dsv4_hip_route_dev(idx_ptr, w_ptr, orig_ptr, scores_ptr, n, bias_ptr,
                                               tid2eid_ptr, n_vocab, token_ids_ptr, n_experts,
                                               topk, float(route_scale), stream),
                   "dsv4_hip_route_dev")

    def moe_layer_dev(self, out_ptr, x_ptr, gate: QMat, table_ptr, n_experts, topk, route_scale,
                      shared: ExpertW | None, hidden, inter, limit, bias_ptr=None,
                      tid2eid_ptr=None, n_vocab=0, token_id=0, idx_ptr=None, w_ptr=None,
                      stream=None):
        sp = C.pointer(shared) if shared is not None else None
        self.check(self.lib.dsv4_hip_moe_layer_dev(out_ptr, x_ptr, C.byref(gate), bias_ptr,
                                                   tid2eid_ptr, n_vocab, token_id,
                                                   float(route_scale), table_ptr, n_experts,
                                                   topk, sp, hidden, inter, float(limit),
                                                   idx_ptr, w_ptr, stream),
                   "dsv4_hip_moe_layer_dev")


    def moe_layer_n_dev(self, out_ptr, x_ptr, n, gate: QMat, table_ptr, n_experts, topk,
                        route_scale, shared: ExpertW | None, hidden, inter, limit, mx=False,
                        bias_ptr=None, tid2eid_ptr=None, n_vocab=0, token_ids_ptr=None,
                        idx_ptr=None, w_ptr=None, stream=None):
        sp = C.pointer(shared) if shared is not None else None
        self.check(self.lib.dsv4_hip_moe_layer_n_dev(out_ptr, x_ptr, n, C.byref(gate), bias_ptr,
                                                     tid2eid_ptr, n_vocab, token_ids_ptr,
                                                     float(route_scale), table_ptr, n_experts, topk,
                                                     sp, hidden, inter, float(limit), int(bool(mx)),
                                                     idx_ptr, w_ptr, stream),
                   "dsv4_hip_moe_layer_n_dev")


class Mirror:
    """ctypes view of libdsv4_amd.so: the reference's own compute entry points
    (dsv4_mmq_n, dsv4_mmq, dsv4_expert_forward) running on the GPU library,
    as a program written against src/10_compute would call them."""

    def __init__(self, path: str = AMD_SO):
        if not os.path.exists(path):
            raise Dsv4Error(f"{path} is not built: run __graft_entry__.build()")
        L = self.lib = C.CDLL(path)
        L.dsv4_mmq_n.restype = None
        L.dsv4_mmq_n.argtypes = [_P, _P, C.POINTER(QMat), _I]
        L.dsv4_mmq.restype = None
        L.dsv4_mmq.argtypes = [_P, _P, C.POINTER(QMat)]
        L.dsv4_expert_forward.restype = None
        L.dsv4_expert_forward.argtypes = [_P, _P, C.POINTER(ExpertW), _P, _P, _P, _I, _F]

    def mmq(self, desc: QMat, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(desc.rows, np.float32)
        self.lib.dsv4_mmq(y.ctypes.data, x.ctypes.data, C.byref(desc))
        return y

    def mmq_n(self, desc: QMat, x: np.ndarray, nt: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(nt * desc.rows, np.float32)
        self.lib.dsv4_mmq_n(y.ctypes.data, x.ctypes.data, C.byref(desc), nt)
        return y

    def expert_forward(self, e: ExpertW, x: np.ndarray, limit: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        inter = e.w1.rows
        out = np.zeros(e.w1.cols, np.float32)
        g, u, m = (np.zeros(inter, np.float32) for _ in range(3))
        self.lib.dsv4_expert_forward(out.ctypes.data, x.ctypes.data, C.byref(e), g.ctypes.data,
                                     u.ctypes.data, m.ctypes.data, inter, float(limit))
        return out


def qmat(wdt, w_ptr, s_ptr, rows, cols, blk_r, blk_c) -> QMat:
    return QMat(w_ptr, s_ptr, wdt, rows, cols, blk_r, blk_c)


_LIB: Lib | None = None


def load() -> Lib:
    """The process-wide binding (raises Dsv4Error when not built)."""
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
