# SPDX-License-Identifier: Apache-2.0
"""ctypes bindings for the CPU oracle (liboracle.so) and, where it was built,
the reference's own hot path compiled unchanged (_ref/libdsv4ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and bench.py's
CPU-baseline leg as the checker; the product never imports it.

Arrays are numpy; every wrapper checks dtype, contiguity and size before the
call so a C routine never reads past a buffer.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libdsv4ref.so")

DSV4_WF32, DSV4_WBF16, DSV4_WFP8, DSV4_WFP4, DSV4_WFP8_F32S = 0, 1, 2, 3, 4


class QMat(C.Structure):
    """DSV4QMat (src/00_base/dsv4_weights.h:34-40)."""
    _fields_ = [("w", C.c_void_p), ("s", C.c_void_p), ("wdt", C.c_int),
                ("rows", C.c_int), ("cols", C.c_int),
                ("blk_r", C.c_int), ("blk_c", C.c_int)]


class ExpertW(C.Structure):
    """DSV4ExpertW (src/00_base/dsv4_weights.h:103-106)."""
    _fields_ = [("w1", QMat), ("w3", QMat), ("w2", QMat)]


_P = C.c_void_p
_I = C.c_int
_F = C.c_float


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data


def _need(a, dtype, n, what):
    if not isinstance(a, np.ndarray) or a.dtype != np.dtype(dtype):
        raise TypeError(f"{what}: expected {np.dtype(dtype)} ndarray")
    if a.size < n:
        raise ValueError(f"{what}: needs {n} elements, has {a.size}")
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError(f"{what}: must be C-contiguous")


def fp8_scale_grid(rows, cols, blk_r, blk_c):
    return ((rows + blk_r - 1) // blk_r) * ((cols + blk_c - 1) // blk_c)


def scale_count(wdt, rows, cols, blk_r, blk_c):
    if wdt == DSV4_WBF16:
        return 0
    if wdt in (DSV4_WFP8, DSV4_WFP8_F32S):
        return fp8_scale_grid(rows, cols, blk_r, blk_c)
    if wdt == DSV4_WFP4:
        return ((rows + blk_r - 1) // blk_r) * ((cols + blk_c - 1) // blk_c)
    raise ValueError(wdt)


def weight_bytes(wdt, rows, cols):
    if wdt == DSV4_WBF16:
        return 2 * rows * cols
    return rows * (cols // 2) if wdt == DSV4_WFP4 else rows * cols


class _Lib:
    def __init__(self, path):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run __graft_entry__.build())")
        self.lib = C.CDLL(path)


class Oracle(_Lib):
    """The C restatement (oracle/dsv4_oracle.c)."""

    def __init__(self, path=ORACLE_SO):
        super().__init__(path)
        L = self.lib
        L.orc_e8m0.restype = _F; L.orc_e8m0.argtypes = [C.c_uint8]
        L.orc_e4m3.restype = _F; L.orc_e4m3.argtypes = [C.c_uint8]
        L.orc_e2m1.restype = _F; L.orc_e2m1.argtypes = [C.c_uint8]
        for n in ("orc_fp8_n", "orc_fp8f_n", "orc_fp4_n"):
            getattr(L, n).restype = None
            getattr(L, n).argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I]
        for n in ("orc_fp8_double", "orc_fp4_double"):
            getattr(L, n).restype = None
            getattr(L, n).argtypes = [_P, _P, _P, _P, _I, _I, _I, _I]
        L.orc_bf16_n.restype = None
        L.orc_bf16_n.argtypes = [_P, _P, _P, _I, _I, _I]
        L.orc_mmq_n.restype = _I; L.orc_mmq_n.argtypes = [_P, _P, C.POINTER(QMat), _I]
        L.orc_swiglu.restype = None; L.orc_swiglu.argtypes = [_P, _P, _P, _I, _F]
        L.orc_route.restype = None
        L.orc_route.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F]
        L.orc_expert_forward.restype = _I
        L.orc_expert_forward.argtypes = [_P, _P, C.POINTER(ExpertW), _P, _P, _P, _I, _F]
        L.orc_moe_combine.restype = None
        L.orc_moe_combine.argtypes = [_P, _P, _P, _I, _P, _I]
        L.orc_union_prepare.restype = _I
        L.orc_union_prepare.argtypes = [_P, _I, _I, _I, _P, _P, _P, _P, _P]
        L.orc_f32_to_e4m3.restype = C.c_uint8; L.orc_f32_to_e4m3.argtypes = [_F]
        L.orc_f32_to_e2m1.restype = C.c_uint8; L.orc_f32_to_e2m1.argtypes = [_F]
        L.orc_f32_to_bf16.restype = C.c_uint16; L.orc_f32_to_bf16.argtypes = [_F]
        L.orc_quant_fp8_blk128.restype = None
        L.orc_quant_fp8_blk128.argtypes = [_P, _P, _P, _I, _I]
        L.orc_quant_fp4_mx.restype = None
        L.orc_quant_fp4_mx.argtypes = [_P, _P, _P, _I, _I]
        L.orc_quant_act_fp8_1x128.restype = None
        L.orc_quant_act_fp8_1x128.argtypes = [_P, _P, _P, _I, _I]
        L.orc_quant_act_mxfp8.restype = None
        L.orc_quant_act_mxfp8.argtypes = [_P, _P, _P, _I, _I]

    # -- decoders
    def e8m0(self, b): return self.lib.orc_e8m0(int(b))
    def e4m3(self, b): return self.lib.orc_e4m3(int(b))
    def e2m1(self, b): return self.lib.orc_e2m1(int(b))

    # -- matmul bodies
    def _body(self, name, W, S, x, rows, cols, blk_r, blk_c, nt, wdt, sdtype):
        _need(W, np.uint8, weight_bytes(wdt, rows, cols), "W")
        _need(S, sdtype, scale_count(wdt, rows, cols, blk_r, blk_c), "S")
        _need(x, np.float32, nt * cols, "x")
        y = np.zeros(nt * rows, np.float32)
        getattr(self.lib, name)(_ptr(y), _ptr(x), _ptr(W), _ptr(S),
                                cols, rows, blk_r, blk_c, nt)
        return y

    def fp8_n(self, W, S, x, rows, cols, blk_r=128, blk_c=128, nt=1):
        return self._body("orc_fp8_n", W, S, x, rows, cols, blk_r, blk_c, nt,
                          DSV4_WFP8, np.uint8)

    def fp8f_n(self, W, S, x, rows, cols, blk_r=128, blk_c=128, nt=1):
        return self._body("orc_fp8f_n", W, S, x, rows, cols, blk_r, blk_c, nt,
                          DSV4_WFP8_F32S, np.float32)

    def bf16_n(self, W, x, rows, cols, nt=1):
        """W: uint16 bf16 bits [rows][cols]."""
        _need(W, np.uint16, rows * cols, "W")
        _need(x, np.float32, nt * cols, "x")
        y = np.zeros(nt * rows, np.float32)
        self.lib.orc_bf16_n(_ptr(y), _ptr(x), _ptr(W), cols, rows, nt)
        return y

    def fp4_n(self, W, S, x, rows, cols, blk_r=1, blk_c=32, nt=1):
        return self._body("orc_fp4_n", W, S, x, rows, cols, blk_r, blk_c, nt,
                          DSV4_WFP4, np.uint8)

    def fp8_double(self, W, S, x, rows, cols, blk_r=128, blk_c=128):
        _need(W, np.uint8, rows * cols, "W"); _need(x, np.float32, cols, "x")
        _need(S, np.uint8, fp8_scale_grid(rows, cols, blk_r, blk_c), "S")
        assert blk_c <= 1024
        y = np.zeros(rows, np.float32)
        self.lib.orc_fp8_double(_ptr(y), _ptr(x), _ptr(W), _ptr(S), cols, rows, blk_r, blk_c)
        return y

    def fp4_double(self, W, S, x, rows, cols, blk_r=1, blk_c=32):
        _need(W, np.uint8, rows * cols // 2, "W"); _need(x, np.float32, cols, "x")
        _need(S, np.uint8, scale_count(DSV4_WFP4, rows, cols, blk_r, blk_c), "S")
        assert blk_c <= 1024
        y = np.zeros(rows, np.float32)
        self.lib.orc_fp4_double(_ptr(y), _ptr(x), _ptr(W), _ptr(S), cols, rows, blk_r, blk_c)
        return y

    def route(self, scores, topk, route_scale, bias=None, tid2eid=None, token_id=0):
        """(idx, wts, orig) of dsv4_route on one token's raw gate outputs"""
        sc = np.array(scores, np.float32)
        ne = sc.size
        orig = np.zeros(ne, np.float32)
        idx = np.zeros(topk, np.int32)
        wts = np.zeros(topk, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        t = None if tid2eid is None else np.ascontiguousarray(tid2eid, np.int64)
        self.lib.orc_route(_ptr(idx), _ptr(wts), _ptr(sc), _ptr(orig), _ptr(b) if b is not None else None,
                           _ptr(t) if t is not None else None, token_id, ne, topk, float(route_scale))
        return idx, wts, orig

    def swiglu(self, gate, up, limit):
        _need(gate, np.float32, gate.size, "gate"); _need(up, np.float32, gate.size, "up")
        y = np.zeros(gate.size, np.float32)
        self.lib.orc_swiglu(_ptr(y), _ptr(gate), _ptr(up), gate.size, float(limit))
        return y

    def expert_forward(self, expert: "HostExpert", x, limit):
        inter = expert.inter
        _need(x, np.float32, expert.hidden, "x")
        out = np.zeros(expert.hidden, np.float32)
        g = np.zeros(inter, np.float32); u = np.zeros(inter, np.float32)
        m = np.zeros(inter, np.float32)
        rc = self.lib.orc_expert_forward(_ptr(out), _ptr(x), C.byref(expert.desc),
                                         _ptr(g), _ptr(u), _ptr(m), inter, float(limit))
        assert rc == 0
        return out

    def moe_combine(self, acc, w, shared=None):
        topk, d = acc.shape
        acc = np.ascontiguousarray(acc, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.zeros(d, np.float32)
        sp = None
        if shared is not None:
            shared = np.ascontiguousarray(shared, np.float32)
            _need(shared, np.float32, d, "shared")
            sp = _ptr(shared)
        self.lib.orc_moe_combine(_ptr(out), _ptr(acc), _ptr(w), topk, sp, d)
        return out

    def union_prepare(self, topk_idx, ne):
        topk_idx = np.ascontiguousarray(topk_idx, np.int32)
        n, topk = topk_idx.shape
        assert topk_idx.min() >= 0 and topk_idx.max() < ne
        cnt = np.zeros(ne, np.int32); off = np.zeros(ne + 1, np.int32)
        tok = np.zeros(n * topk, np.int32); kk = np.zeros(n * topk, np.int32)
        order = np.zeros(ne, np.int32)
        nord = self.lib.orc_union_prepare(_ptr(topk_idx), n, topk, ne, _ptr(cnt),
                                          _ptr(off), _ptr(tok), _ptr(kk), _ptr(order))
        return cnt, off, tok, kk, order[:nord]

    # -- quantizers
    def f32_to_e4m3(self, v): return self.lib.orc_f32_to_e4m3(float(v))
    def f32_to_e2m1(self, v): return self.lib.orc_f32_to_e2m1(float(v))
    def f32_to_bf16(self, v): return self.lib.orc_f32_to_bf16(float(v))

    def quant_fp8_blk128(self, w):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        W = np.zeros(rows * cols, np.uint8)
        S = np.zeros(fp8_scale_grid(rows, cols, 128, 128), np.float32)
        self.lib.orc_quant_fp8_blk128(_ptr(W), _ptr(S), _ptr(w), rows, cols)
        return W, S

    def quant_fp4_mx(self, w):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        assert cols % 32 == 0
        W = np.zeros(rows * cols // 2, np.uint8)
        S = np.zeros(rows * cols // 32, np.uint8)
        self.lib.orc_quant_fp4_mx(_ptr(W), _ptr(S), _ptr(w), rows, cols)
        return W, S

    def quant_act_fp8_1x128(self, a):
        a = np.ascontiguousarray(a, np.float32)
        n, k = a.shape
        assert k % 128 == 0
        Q = np.zeros(n * k, np.uint8); S = np.zeros(n * k // 128, np.float32)
        self.lib.orc_quant_act_fp8_1x128(_ptr(Q), _ptr(S), _ptr(a), n, k)
        return Q, S

    def quant_act_mxfp8(self, a):
        a = np.ascontiguousarray(a, np.float32)
        n, k = a.shape
        assert k % 32 == 0
        Q = np.zeros(n * k, np.uint8); S = np.zeros(n * k // 32, np.uint8)
        self.lib.orc_quant_act_mxfp8(_ptr(Q), _ptr(S), _ptr(a), n, k)
        return Q, S

    def mmq_n(self, m: "HostMat", x, nt=1):
        _need(x, np.float32, nt * m.cols, "x")
        y = np.zeros(nt * m.rows, np.float32)
        rc = self.lib.orc_mmq_n(_ptr(y), _ptr(x), C.byref(m.desc), nt)
        if rc:
            raise ValueError(f"oracle: unsupported wdt {m.wdt}")
        return y


class Reference(_Lib):
    """The reference's own src/10_compute objects (oracle/_ref), present only
    where /root/reference was there to build them."""

    def __init__(self, path=REF_SO):
        super().__init__(path)
        L = self.lib
        for n in ("fp8_n", "fp4_n"):
            getattr(L, n).restype = None
            getattr(L, n).argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I]
        L.dsv4_mmq_n.restype = None
        L.dsv4_mmq_n.argtypes = [_P, _P, C.POINTER(QMat), _I]
        L.dsv4_swiglu.restype = None; L.dsv4_swiglu.argtypes = [_P, _P, _P, _I, _F]
        L.dsv4_expert_forward.restype = None
        L.dsv4_expert_forward.argtypes = [_P, _P, C.POINTER(ExpertW), _P, _P, _P, _I, _F]
        L.dsv4_matmul_fp8_f32.restype = None
        L.dsv4_matmul_fp8_f32.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I]
        L.bf16_n.restype = None
        L.bf16_n.argtypes = [_P, _P, _P, _I, _I, _I]

    def bf16_n(self, W, x, rows, cols, nt=1):
        _need(W, np.uint16, rows * cols, "W"); _need(x, np.float32, nt * cols, "x")
        y = np.zeros(nt * rows, np.float32)
        self.lib.bf16_n(_ptr(y), _ptr(x), _ptr(W), cols, rows, nt)
        return y

    def fp8_n(self, W, S, x, rows, cols, blk_r=128, blk_c=128, nt=1):
        _need(W, np.uint8, rows * cols, "W"); _need(x, np.float32, nt * cols, "x")
        _need(S, np.uint8, fp8_scale_grid(rows, cols, blk_r, blk_c), "S")
        y = np.zeros(nt * rows, np.float32)
        self.lib.fp8_n(_ptr(y), _ptr(x), _ptr(W), _ptr(S), cols, rows, blk_r, blk_c, nt)
        return y

    def fp4_n(self, W, S, x, rows, cols, blk_r=1, blk_c=32, nt=1):
        _need(W, np.uint8, rows * cols // 2, "W"); _need(x, np.float32, nt * cols, "x")
        _need(S, np.uint8, scale_count(DSV4_WFP4, rows, cols, blk_r, blk_c), "S")
        y = np.zeros(nt * rows, np.float32)
        self.lib.fp4_n(_ptr(y), _ptr(x), _ptr(W), _ptr(S), cols, rows, blk_r, blk_c, nt)
        return y

    def swiglu(self, gate, up, limit):
        y = np.zeros(gate.size, np.float32)
        self.lib.dsv4_swiglu(_ptr(y), _ptr(gate), _ptr(up), gate.size, float(limit))
        return y

    def route(self, scores, topk, route_scale, bias=None, tid2eid=None, token_id=0):
        sc = np.array(scores, np.float32)
        ne = sc.size
        orig = np.zeros(ne, np.float32)
        idx = np.zeros(topk, np.int32)
        wts = np.zeros(topk, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        t = None if tid2eid is None else np.ascontiguousarray(tid2eid, np.int64)
        f = self.lib.dsv4_route
        f.restype = None
        f.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F]
        f(_ptr(idx), _ptr(wts), _ptr(sc), _ptr(orig), _ptr(b) if b is not None else None,
          _ptr(t) if t is not None else None, token_id, ne, topk, float(route_scale))
        return idx, wts, orig

    def expert_forward(self, expert: "HostExpert", x, limit):
        inter = expert.inter
        out = np.zeros(expert.hidden, np.float32)
        g = np.zeros(inter, np.float32); u = np.zeros(inter, np.float32)
        m = np.zeros(inter, np.float32)
        self.lib.dsv4_expert_forward(_ptr(out), _ptr(x), C.byref(expert.desc),
                                     _ptr(g), _ptr(u), _ptr(m), inter, float(limit))
        return out


class HostMat:
    """A packed matrix in host memory plus its DSV4QMat descriptor. Keeps the
    numpy buffers alive as long as the descriptor."""

    def __init__(self, wdt, W, S, rows, cols, blk_r, blk_c):
        self.wdt, self.rows, self.cols = wdt, rows, cols
        self.blk_r, self.blk_c = blk_r, blk_c
        if wdt == DSV4_WBF16:
            # a plain BF16 matrix: uint16 bits, no scales (s = NULL, blk 0)
            self.W = np.ascontiguousarray(W, np.uint16)
            _need(self.W, np.uint16, rows * cols, "W")
            self.S = None
            self.desc = QMat(_ptr(self.W), None, wdt, rows, cols, 0, 0)
            return
        self.W = np.ascontiguousarray(W, np.uint8)
        sd = np.float32 if wdt == DSV4_WFP8_F32S else np.uint8
        self.S = np.ascontiguousarray(S, sd)
        _need(self.W, np.uint8, weight_bytes(wdt, rows, cols), "W")
        _need(self.S, sd, scale_count(wdt, rows, cols, blk_r, blk_c), "S")
        self.desc = QMat(_ptr(self.W), _ptr(self.S), wdt, rows, cols, blk_r, blk_c)


class HostExpert:
    def __init__(self, w1: HostMat, w3: HostMat, w2: HostMat):
        self.w1, self.w3, self.w2 = w1, w3, w2
        self.inter, self.hidden = w1.rows, w1.cols
        assert w3.rows == self.inter and w2.cols == self.inter and w2.rows == self.hidden
        self.desc = ExpertW(w1.desc, w3.desc, w2.desc)
