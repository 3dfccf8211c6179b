"""TEST INFRASTRUCTURE ONLY: ctypes bindings for the oracle.

* ``Oracle`` wraps liboracle.so, the scalar C restatement of sycl-infer's CPU
  integer path (miq_oracle.c).
* ``Ref`` wraps _ref/libsiref.so, sycl-infer's own CPU kernels compiled from
  the reference sources (Makefile target ``ref``); present only where it was
  built.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this
module -- as the checker, never as the thing measured or shipped.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libsiref.so")

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
_VB = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
_BB = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}

_vp, _i32, _u32, _f32, _u16 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_float, ctypes.c_uint16


def row_bytes(qtype: int, K: int) -> int:
    return K // _VB[qtype] * _BB[qtype]


def _ptr(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class _SegC(ctypes.Structure):
    _fields_ = [("w", _vp), ("type", _u32), ("K", ctypes.c_int32), ("n_rows", ctypes.c_int32), ("out", _vp),
                ("out_stride", ctypes.c_int32), ("residual", _vp), ("alpha", _f32), ("x8", _vp), ("xmeta", _vp),
                ("xsumq", _vp)]


class _MoeC(ctypes.Structure):
    _fields_ = [("gate", _vp), ("up", _vp), ("down", _vp), ("gate_type", _u32), ("up_type", _u32),
                ("down_type", _u32), ("gate_plane", ctypes.c_size_t), ("up_plane", ctypes.c_size_t),
                ("down_plane", ctypes.c_size_t), ("n_embd", _i32), ("n_ff", _i32), ("n_expert", _i32)]


class Oracle:
    """The C restatement (miq_oracle.c)."""

    def __init__(self, path: str = ORACLE_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle)")
        L = self.L = ctypes.CDLL(path)
        L.miqo_half_to_float.restype, L.miqo_half_to_float.argtypes = _f32, [_u16]
        L.miqo_float_to_half.restype, L.miqo_float_to_half.argtypes = _u16, [_f32]
        L.miqo_get_scale_min_k4.argtypes = [_i32, _vp, _vp, _vp]
        L.miqo_dequantize_row.argtypes = [_u32, _vp, _vp, _i32]
        L.miqo_xq.argtypes = [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _i32]
        L.miqo_group_dots.argtypes = [_u32, _vp, _i32, _i32, _vp, _i32, _vp]
        L.miqo_i8_gemv.argtypes = [ctypes.POINTER(_SegC)]
        L.miqo_i8_gemm.argtypes = [ctypes.POINTER(_SegC), _i32]
        L.miqo_moe_route.argtypes = [_vp, _i32, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]
        L.miqo_moe_experts.argtypes = [ctypes.POINTER(_MoeC), _vp, _i32, _i32, _i32, _vp, _vp, _i32, _vp]
        L.miqo_moe_reduce.argtypes = [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _i32]
        L.miqo_silu.restype, L.miqo_silu.argtypes = _f32, [_f32]
        L.miqo_expf_mismatches.restype = ctypes.c_uint64
        L.miqo_expf_mismatches.argtypes = [_u32, _u32, _vp, ctypes.POINTER(_u32)]
        L.miqo_expf_method.restype, L.miqo_expf_method.argtypes = _f32, [_f32]
        L.miqo_expf_method_mismatches.restype = ctypes.c_uint64
        L.miqo_expf_method_mismatches.argtypes = [_u32, _u32, ctypes.POINTER(_u32)]
        L.miqo_float_to_half_rne.restype, L.miqo_float_to_half_rne.argtypes = _u16, [_f32]
        L.miqo_w4_pack_q4k.restype, L.miqo_w4_pack_q4k.argtypes = _i32, [_vp, _i32, _i32, _vp, _vp, _vp]
        L.miqo_w4_act.argtypes = [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp]
        L.miqo_w4_gemv.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f32, _i32, _i32]
        L.miqo_k5_pack.restype, L.miqo_k5_pack.argtypes = _i32, [_vp, _i32, _i32, _vp, _vp, _vp, _vp]
        L.miqo_k5_gemv.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f32, _i32, _i32]

    def half_to_float(self, h: int) -> float:
        return self.L.miqo_half_to_float(h)

    def float_to_half(self, f: float) -> int:
        return self.L.miqo_float_to_half(f)

    def get_scale_min_k4(self, j: int, scales: np.ndarray):
        s = _c(scales, np.uint8)
        d, m = ctypes.c_uint8(), ctypes.c_uint8()
        self.L.miqo_get_scale_min_k4(j, s.ctypes.data, ctypes.addressof(d), ctypes.addressof(m))
        return d.value, m.value

    def dequantize(self, qtype: int, w: np.ndarray, K: int) -> np.ndarray:
        w = _c(w, np.uint8).reshape(-1, row_bytes(qtype, K))
        y = np.empty((w.shape[0], K), dtype=np.float32)
        for r in range(w.shape[0]):
            self.L.miqo_dequantize_row(qtype, w[r].ctypes.data, y[r].ctypes.data, K)
        return y

    def xq(self, x: np.ndarray, up: np.ndarray | None = None):
        x = _c(x, np.float32)
        TB, K = x.shape
        up = None if up is None else _c(up, np.float32)
        x8 = np.empty((K // 32, TB, 32), np.int8)
        xm = np.empty((K // 32, TB, 2), np.float32)
        xs = np.empty((K // 32, TB, 2), np.int32)
        self.L.miqo_xq(x.ctypes.data, _ptr(up), K, K, x8.ctypes.data, xm.ctypes.data, xs.ctypes.data, TB, K)
        return x8, xm, xs

    def group_dots(self, qtype: int, w: np.ndarray, K: int, n_rows: int, x8: np.ndarray) -> np.ndarray:
        w = _c(w, np.uint8)
        x8 = _c(x8, np.int8)
        TB = x8.shape[1]
        S = K // 16 if qtype == Q6_K else K // 32
        out = np.empty((TB, n_rows, S), np.int32)
        self.L.miqo_group_dots(qtype, w.ctypes.data, K, n_rows, x8.ctypes.data, TB, out.ctypes.data)
        return out

    def _seg(self, qtype, w, K, n_rows, act, out, out_stride, residual, alpha):
        s = _SegC()
        s.w, s.type, s.K, s.n_rows = w.ctypes.data, qtype, K, n_rows
        s.out, s.out_stride, s.residual, s.alpha = out.ctypes.data, out_stride, _ptr(residual), alpha
        s.x8, s.xmeta, s.xsumq = act[0].ctypes.data, act[1].ctypes.data, act[2].ctypes.data
        return s

    def gemm(self, qtype: int, w: np.ndarray, K: int, n_rows: int, act, residual=None, alpha: float = 1.0):
        """cpu_i8_gemv for TB == 1, cpu_i8_gemm otherwise; out [TB, n_rows]."""
        w = _c(w, np.uint8)
        act = tuple(_c(a, d) for a, d in zip(act, (np.int8, np.float32, np.int32)))
        TB = act[0].shape[1]
        out = np.empty((TB, n_rows), np.float32)
        res = None if residual is None else _c(residual, np.float32)
        s = self._seg(qtype, w, K, n_rows, act, out, n_rows, res, alpha)
        if TB == 1:
            self.L.miqo_i8_gemv(ctypes.byref(s))
        else:
            self.L.miqo_i8_gemm(ctypes.byref(s), TB)
        return out

    def float_to_half_rne(self, f: float) -> int:
        return self.L.miqo_float_to_half_rne(f)

    def w4_pack(self, w: np.ndarray, K: int, N: int):
        """pack_q4_K: (vals [N, K/2] u8, scale [K/32, N] u16, off [K/32, N] u16)."""
        w = _c(w, np.uint8)
        vals = np.empty((N, K // 2), np.uint8)
        sc = np.empty((K // 32, N), np.uint16)
        of = np.empty((K // 32, N), np.uint16)
        if self.L.miqo_w4_pack_q4k(w.ctypes.data, K, N, vals.ctypes.data, sc.ctypes.data, of.ctypes.data):
            raise ValueError("w4_pack: K must be a multiple of 256")
        return vals, sc, of

    def w4_act(self, x: np.ndarray, up: np.ndarray | None = None):
        """act_quant_grp with the even/odd split: (xq [M,K], asa [M,K/32] u16, xs [M,K/32], axe, axo [M,K/2])."""
        x = _c(x, np.float32)
        M, K = x.shape
        up = None if up is None else _c(up, np.float32)
        xq = np.empty((M, K), np.int8)
        asa = np.empty((M, K // 32), np.uint16)
        xs = np.empty((M, K // 32), np.float32)
        axe = np.empty((M, K // 2), np.int8)
        axo = np.empty((M, K // 2), np.int8)
        self.L.miqo_w4_act(x.ctypes.data, _ptr(up), M, K, xq.ctypes.data, asa.ctypes.data, xs.ctypes.data,
                           axe.ctypes.data, axo.ctypes.data)
        return xq, asa, xs, axe, axo

    def w4_gemv(self, store, act, residual=None, alpha: float = 1.0):
        """w4_gemv_impl for one activation row; store = w4_pack(...), act = w4_act(...) (row 0)."""
        vals, sc, of = (_c(a, d) for a, d in zip(store, (np.uint8, np.uint16, np.uint16)))
        N, K = vals.shape[0], vals.shape[1] * 2
        _, asa, xs, axe, axo = act
        asa, xs = _c(asa.reshape(-1)[: K // 32], np.uint16), _c(xs.reshape(-1)[: K // 32], np.float32)
        axe, axo = _c(axe.reshape(-1)[: K // 2], np.int8), _c(axo.reshape(-1)[: K // 2], np.int8)
        res = None if residual is None else _c(residual, np.float32)
        out = np.empty(N, np.float32)
        self.L.miqo_w4_gemv(vals.ctypes.data, sc.ctypes.data, of.ctypes.data, axe.ctypes.data, axo.ctypes.data,
                            asa.ctypes.data, xs.ctypes.data, out.ctypes.data, _ptr(res), alpha, K, N)
        return out

    def k5_pack(self, w: np.ndarray, K: int, N: int):
        """pack_q5_K: (vals [N, K/2] u8, hi [N, K/8] u8, scale [K/32, N] u16, off [K/32, N] u16)."""
        w = _c(w, np.uint8)
        vals = np.empty((N, K // 2), np.uint8)
        hi = np.empty((N, K // 8), np.uint8)
        sc = np.empty((K // 32, N), np.uint16)
        of = np.empty((K // 32, N), np.uint16)
        if self.L.miqo_k5_pack(w.ctypes.data, K, N, vals.ctypes.data, hi.ctypes.data, sc.ctypes.data,
                               of.ctypes.data):
            raise ValueError("k5_pack: K must be a multiple of 256")
        return vals, hi, sc, of

    def k5_gemv(self, store, act, residual=None, alpha: float = 1.0):
        """k5_gemv_impl for one activation row; store = k5_pack(...), act = w4_act(...) (row 0)."""
        vals, hi, sc, of = (_c(a, d) for a, d in zip(store, (np.uint8, np.uint8, np.uint16, np.uint16)))
        N, K = vals.shape[0], vals.shape[1] * 2
        _, asa, xs, axe, axo = act
        asa, xs = _c(asa.reshape(-1)[: K // 32], np.uint16), _c(xs.reshape(-1)[: K // 32], np.float32)
        axe, axo = _c(axe.reshape(-1)[: K // 2], np.int8), _c(axo.reshape(-1)[: K // 2], np.int8)
        res = None if residual is None else _c(residual, np.float32)
        out = np.empty(N, np.float32)
        self.L.miqo_k5_gemv(vals.ctypes.data, hi.ctypes.data, sc.ctypes.data, of.ctypes.data, axe.ctypes.data,
                            axo.ctypes.data, asa.ctypes.data, xs.ctypes.data, out.ctypes.data, _ptr(res), alpha, K, N)
        return out

    def moe_route(self, logits: np.ndarray, top_k: int, x=None, gate_inp=None):
        lg = _c(logits, np.float32).copy()
        n_tok, n_expert = lg.shape
        ids = np.empty((n_tok, top_k), np.int32)
        wts = np.empty((n_tok, top_k), np.float32)
        xx = None if x is None else _c(x, np.float32)
        gi = None if gate_inp is None else _c(gate_inp, np.float32)
        n_embd = gi.shape[1] if gi is not None else 0
        self.L.miqo_moe_route(_ptr(xx), n_embd, _ptr(gi), n_tok, n_embd, n_expert, top_k, lg.ctypes.data,
                              ids.ctypes.data, wts.ctypes.data)
        return ids, wts, lg

    def moe_experts(self, qtype, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids, down_type=None,
                    want_h=False):
        dt = qtype if down_type is None else down_type
        gate, up, down = _c(gate, np.uint8), _c(up, np.uint8), _c(down, np.uint8)
        m = _MoeC()
        m.gate, m.up, m.down = gate.ctypes.data, up.ctypes.data, down.ctypes.data
        m.gate_type = m.up_type = qtype
        m.down_type = dt
        m.gate_plane = m.up_plane = n_ff * row_bytes(qtype, n_embd)
        m.down_plane = n_embd * row_bytes(dt, n_ff)
        m.n_embd, m.n_ff, m.n_expert = n_embd, n_ff, n_expert
        x = _c(x, np.float32)
        ids = _c(ids, np.int32)
        n_tok = x.shape[0]
        acc = np.empty((n_tok * top_k, n_embd), np.float32)
        h = np.empty((n_tok * top_k, n_ff), np.float32) if want_h else None
        self.L.miqo_moe_experts(ctypes.byref(m), x.ctypes.data, n_embd, n_tok, top_k, ids.ctypes.data,
                                acc.ctypes.data, n_embd, _ptr(h))
        return (acc, h) if want_h else acc

    def moe_experts_grouped(self, qtype, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids, down_type=None):
        """The grouped expert flow of moe_experts_grouped_i8 (moe.cpp:147-334) composed from the pinned
        pieces: per expert, its pairs' activation rows gathered (at least two, so the batched GEMM's
        continuous accumulation across blocks applies, i8.cpp:316-349, as in the reference's tiled GEMM on
        rows padded to 32), gate/up GEMM, h = silu(g)*u, h requantised, the down GEMM on the gathered h rows.
        Pairs with an expert id out of range give zero rows."""
        dt = qtype if down_type is None else down_type
        x = _c(x, np.float32)
        ids = np.asarray(ids, np.int32).reshape(-1)
        n_tok = x.shape[0]
        rb_g, rb_d = row_bytes(qtype, n_embd), row_bytes(dt, n_ff)
        gate = _c(gate, np.uint8).reshape(n_expert, n_ff * rb_g)
        up = _c(up, np.uint8).reshape(n_expert, n_ff * rb_g)
        down = _c(down, np.uint8).reshape(n_expert, n_embd * rb_d)
        acc = np.zeros((ids.size, n_embd), np.float32)
        silu = np.vectorize(lambda v: self.L.miqo_silu(float(v)), otypes=[np.float32])
        for e in range(n_expert):
            pairs = np.nonzero(ids == e)[0]
            if pairs.size == 0:
                continue
            rows = np.zeros((max(2, pairs.size), n_embd), np.float32)
            rows[: pairs.size] = x[pairs // top_k]
            gg = self.gemm(qtype, gate[e], n_embd, n_ff, self.xq(rows))
            uu = self.gemm(qtype, up[e], n_embd, n_ff, self.xq(rows))
            h = np.zeros((rows.shape[0], n_ff), np.float32)
            h[: pairs.size] = silu(gg[: pairs.size]) * uu[: pairs.size]
            acc[pairs] = self.gemm(dt, down[e], n_ff, n_embd, self.xq(h))[: pairs.size]
        return acc

    def moe_reduce(self, acc, wts, top_k, out):
        acc, wts = _c(acc, np.float32), _c(wts, np.float32)
        out = _c(out, np.float32).copy()
        n_tok, n_embd = out.shape
        self.L.miqo_moe_reduce(acc.ctypes.data, wts.ctypes.data, top_k, n_tok, n_embd, n_embd, out.ctypes.data,
                               n_embd)
        return out

    def silu(self, x: float) -> float:
        return self.L.miqo_silu(x)

    def expf_mismatches(self, first: int, y: np.ndarray):
        """(count, first bad input bits) of y against the host expf over bits first.."""
        y = _c(y, np.float32)
        fb = _u32(0)
        n = self.L.miqo_expf_mismatches(first, y.size, y.ctypes.data, ctypes.byref(fb))
        return int(n), int(fb.value)

    def expf_method_mismatches(self, first: int, count: int):
        fb = _u32(0)
        n = self.L.miqo_expf_method_mismatches(first, count, ctypes.byref(fb))
        return int(n), int(fb.value)


class Ref:
    """sycl-infer's own CPU kernels (oracle/_ref/libsiref.so, built from the reference sources)."""

    def __init__(self, path: str = REF_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle ref, needs /root/reference)")
        L = self.L = ctypes.CDLL(path)
        L.ref_half_to_float.restype, L.ref_half_to_float.argtypes = _f32, [_u16]
        L.ref_float_to_half.restype, L.ref_float_to_half.argtypes = _u16, [_f32]
        L.ref_silu.restype, L.ref_silu.argtypes = _f32, [_f32]
        L.ref_thread_count.restype = _i32
        L.ref_i8_supported.restype = _i32
        L.ref_dequantize_row.argtypes = [_u32, _vp, _vp, _i32]
        L.ref_xq.argtypes = [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _i32]
        L.ref_i8_gemv.argtypes = [_vp, _u32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _f32]
        L.ref_i8_gemm.argtypes = [_vp, _u32, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _f32, _i32]
        L.ref_q8_0_gemm.argtypes = [_vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _i32]
        L.ref_moe_route.argtypes = [_vp, _i32, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]
        L.ref_moe_reduce.argtypes = [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _i32]
        L.ref_moe_experts.argtypes = [_vp, _vp, _vp, _u32, _u32, _u32, ctypes.c_size_t, ctypes.c_size_t,
                                      ctypes.c_size_t, _i32, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _i32]
        L.ref_moe_experts_grouped.argtypes = [_vp, _vp, _vp, _u32, _u32, _u32, ctypes.c_size_t, ctypes.c_size_t,
                                      ctypes.c_size_t, _i32, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _i32]

        L.ref_w4_pack.restype, L.ref_w4_pack.argtypes = _i32, [_u32, _vp, _i32, _i32, _vp, _vp, _vp]
        L.ref_k5_pack.restype, L.ref_k5_pack.argtypes = _i32, [_u32, _vp, _i32, _i32, _vp, _vp, _vp, _vp]
        L.ref_gguf_dump.restype, L.ref_gguf_dump.argtypes = ctypes.c_size_t, [ctypes.c_char_p, _vp, ctypes.c_size_t]

    def ggml_geom(self, t: int):
        """(name, block size, block bytes) of ggml type t; sizes None where the reference throws."""
        b, z, nm = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_char_p()
        rc = self.L.ref_ggml_geom(t, ctypes.byref(b), ctypes.byref(z), ctypes.byref(nm))
        return nm.value.decode(), (None if rc else b.value), (None if rc else z.value)

    def gguf_dump(self, path: str) -> str:
        """gguf_file::load (src/model/gguf.cpp:345) of `path`, as the text lines of ref_gguf_dump."""
        n = self.L.ref_gguf_dump(os.fsencode(path), None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        self.L.ref_gguf_dump(os.fsencode(path), buf, n + 1)
        return buf.value.decode("utf-8", "surrogateescape")

    def thread_count(self) -> int:
        return self.L.ref_thread_count()

    def isa_spec(self) -> str:
        """the reference's ISA choice for its CPU kernels (si::cpu_isa_spec)"""
        self.L.ref_isa_spec.restype = ctypes.c_char_p
        return self.L.ref_isa_spec().decode()

    def w4_pack(self, w: np.ndarray, K: int, N: int, qtype: int = Q4_K):
        """si::w4_pack (src/common/w4.cpp:416); None where the reference declines."""
        w = _c(w, np.uint8)
        vals = np.empty((N, K // 2), np.uint8)
        sc = np.empty((K // 32, N), np.uint16)
        of = np.empty((K // 32, N), np.uint16)
        rc = self.L.ref_w4_pack(qtype, w.ctypes.data, K, N, vals.ctypes.data, sc.ctypes.data, of.ctypes.data)
        return None if rc else (vals, sc, of)

    def k5_pack(self, w: np.ndarray, K: int, N: int, qtype: int = Q5_K):
        """si::k5_pack (src/common/w4.cpp:409); None where the reference declines."""
        w = _c(w, np.uint8)
        vals = np.empty((N, K // 2), np.uint8)
        hi = np.empty((N, K // 8), np.uint8)
        sc = np.empty((K // 32, N), np.uint16)
        of = np.empty((K // 32, N), np.uint16)
        rc = self.L.ref_k5_pack(qtype, w.ctypes.data, K, N, vals.ctypes.data, hi.ctypes.data, sc.ctypes.data,
                                of.ctypes.data)
        return None if rc else (vals, hi, sc, of)

    def half_to_float(self, h: int) -> float:
        return self.L.ref_half_to_float(h)

    def float_to_half(self, f: float) -> int:
        return self.L.ref_float_to_half(f)

    def dequantize(self, qtype: int, w: np.ndarray, K: int) -> np.ndarray:
        w = _c(w, np.uint8).reshape(-1, row_bytes(qtype, K))
        y = np.empty((w.shape[0], K), dtype=np.float32)
        for r in range(w.shape[0]):
            self.L.ref_dequantize_row(qtype, w[r].ctypes.data, y[r].ctypes.data, K)
        return y

    def xq(self, x: np.ndarray, up: np.ndarray | None = None):
        x = _c(x, np.float32)
        TB, K = x.shape
        up = None if up is None else _c(up, np.float32)
        x8 = np.empty((K // 32, TB, 32), np.int8)
        xm = np.empty((K // 32, TB, 2), np.float32)
        xs = np.empty((K // 32, TB, 2), np.int32)
        self.L.ref_xq(x.ctypes.data, _ptr(up), K, K, x8.ctypes.data, xm.ctypes.data, xs.ctypes.data, TB, K)
        return x8, xm, xs

    def gemm(self, qtype: int, w: np.ndarray, K: int, n_rows: int, act, residual=None, alpha: float = 1.0):
        """cpu_i8_gemv (TB == 1) / cpu_i8_gemm (TB >= 2) for K-quants; Q8_0 via
        cpu_q8_0_down_grouped (no alpha/residual there)."""
        w = _c(w, np.uint8)
        act = tuple(_c(a, d) for a, d in zip(act, (np.int8, np.float32, np.int32)))
        TB = act[0].shape[1]
        out = np.empty((TB, n_rows), np.float32)
        res = None if residual is None else _c(residual, np.float32)
        if qtype == Q8_0:
            assert residual is None and alpha == 1.0
            self.L.ref_q8_0_gemm(w.ctypes.data, K, n_rows, act[0].ctypes.data, act[1].ctypes.data,
                                 act[2].ctypes.data, TB, out.ctypes.data, n_rows)
        elif TB == 1:
            self.L.ref_i8_gemv(w.ctypes.data, qtype, K, n_rows, act[0].ctypes.data, act[1].ctypes.data,
                               act[2].ctypes.data, out.ctypes.data, _ptr(res), alpha)
        else:
            self.L.ref_i8_gemm(w.ctypes.data, qtype, K, n_rows, act[0].ctypes.data, act[1].ctypes.data,
                               act[2].ctypes.data, out.ctypes.data, n_rows, _ptr(res), alpha, TB)
        return out

    def moe_route(self, logits: np.ndarray, top_k: int, x=None, gate_inp=None):
        """cpu_moe_route; with gate_inp None an identity-free path is emulated by
        passing the logits through a one-hot router (x = logits, gate = I)."""
        lg = _c(logits, np.float32)
        n_tok, n_expert = lg.shape
        if gate_inp is None:
            x = lg
            gate_inp = np.eye(n_expert, dtype=np.float32)
        x = _c(x, np.float32)
        gi = _c(gate_inp, np.float32)
        n_embd = gi.shape[1]
        out_lg = np.empty((n_tok, n_expert), np.float32)
        ids = np.empty((n_tok, top_k), np.int32)
        wts = np.empty((n_tok, top_k), np.float32)
        self.L.ref_moe_route(x.ctypes.data, n_embd, gi.ctypes.data, n_tok, n_embd, n_expert, top_k,
                             out_lg.ctypes.data, ids.ctypes.data, wts.ctypes.data)
        return ids, wts, out_lg

    def moe_experts(self, qtype, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids, down_type=None):
        dt = qtype if down_type is None else down_type
        gate, up, down = _c(gate, np.uint8), _c(up, np.uint8), _c(down, np.uint8)
        x = _c(x, np.float32)
        ids = _c(ids, np.int32)
        n_tok = x.shape[0]
        acc = np.empty((n_tok * top_k, n_embd), np.float32)
        gp = n_ff * row_bytes(qtype, n_embd)
        dp = n_embd * row_bytes(dt, n_ff)
        self.L.ref_moe_experts(gate.ctypes.data, up.ctypes.data, down.ctypes.data, qtype, qtype, dt, gp, gp, dp,
                               n_embd, n_ff, n_expert, x.ctypes.data, n_embd, n_tok, top_k, ids.ctypes.data,
                               acc.ctypes.data, n_embd)
        return acc

    def moe_experts_grouped(self, qtype, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids, down_type=None):
        """The reference's grouped expert flow (moe.cpp:147-334; K-quant down banks through the same tiled GEMM)."""
        dt = qtype if down_type is None else down_type
        gate, up, down = _c(gate, np.uint8), _c(up, np.uint8), _c(down, np.uint8)
        x = _c(x, np.float32)
        ids = _c(ids, np.int32)
        n_tok = x.shape[0]
        acc = np.empty((n_tok * top_k, n_embd), np.float32)
        gp = n_ff * row_bytes(qtype, n_embd)
        dp = n_embd * row_bytes(dt, n_ff)
        self.L.ref_moe_experts_grouped(gate.ctypes.data, up.ctypes.data, down.ctypes.data, qtype, qtype, dt, gp, gp,
                                       dp, n_embd, n_ff, n_expert, x.ctypes.data, n_embd, n_tok, top_k,
                                       ids.ctypes.data, acc.ctypes.data, n_embd)
        return acc

    def moe_reduce(self, acc, wts, top_k, out):
        acc, wts = _c(acc, np.float32), _c(wts, np.float32)
        out = _c(out, np.float32).copy()
        n_tok, n_embd = out.shape
        self.L.ref_moe_reduce(acc.ctypes.data, wts.ctypes.data, top_k, n_tok, n_embd, n_embd, out.ctypes.data,
                              n_embd)
        return out
