"""Python host mirror of miq's C ABI (include/miq.h) over ctypes.

The product is the C-ABI library ``libmiq.so`` next to this file (HIP kernels
for gfx950).  This module binds its entry points with the reference's names
and argument meaning -- ``xq``, ``i8_gemv``, ``i8_gemm`` (compute_backend,
src/backend/backend.h:104-114 of sycl-infer) and the MoE launchers -- taking
torch tensors for device buffers.  There is no fallback: if the library is
missing or a call fails, it raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmiq.so")

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
TYPE_NAMES = {Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

MIQ_OK, MIQ_UNSUPPORTED = 0, 1

# every symbol include/miq.h declares
EXPORTS = (
    "miq_version", "miq_last_error", "miq_row_bytes", "miq_xq", "miq_i8_gemv", "miq_i8_gemm",
    "miq_quant_gemm", "miq_group_dots", "miq_moe_route", "miq_moe_csr", "miq_moe_workspace_bytes",
    "miq_moe_experts", "miq_moe_reduce", "miq_quantize_rows",
    "miq_ggml_type_name", "miq_ggml_blck_size", "miq_ggml_type_size", "miq_ggml_row_bytes",
    "miq_gguf_open", "miq_gguf_close", "miq_gguf_describe", "miq_gguf_shard", "miq_gguf_find", "miq_gguf_tensor",
    "miq_gguf_kv_key", "miq_gguf_meta", "miq_gguf_val_read", "miq_gguf_val_elem", "miq_gguf_get_u32",
    "miq_gguf_get_f32", "miq_gguf_get_str", "miq_gguf_drop_cache", "miq_gguf_upload",
    "miq_w4_pack", "miq_w4_act", "miq_w4_gemv", "miq_k5_pack", "miq_k5_gemv", "miq_w4_quant_gemv",
    "miq_w4_gemm", "miq_nat_gemm", "miq_expf_range", "miq_set_switch",
    "miq_i8_gemm_noalloc", "miq_i8_gemv_multi", "miq_quant_gemm_multi",
)


class MiqError(RuntimeError):
    pass


class Seg(ctypes.Structure):
    """miq_seg (include/miq.h) == gemv_seg / cpu_gemv_seg on the integer path."""
    _fields_ = [
        ("w", ctypes.c_void_p), ("type", ctypes.c_uint32), ("K", ctypes.c_int32), ("n_rows", ctypes.c_int32),
        ("x", ctypes.c_void_p), ("x_stride", ctypes.c_int32), ("act_up", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("out_stride", ctypes.c_int32), ("residual", ctypes.c_void_p),
        ("alpha", ctypes.c_float), ("x8", ctypes.c_void_p), ("xmeta", ctypes.c_void_p), ("xsumq", ctypes.c_void_p),
    ]


class W4SegC(ctypes.Structure):
    """miq_w4_seg (include/miq.h) == w4_grp_seg (src/backend/gpu/kernels/kernels.h:226-234)."""
    _fields_ = [
        ("vals", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("off", ctypes.c_void_p), ("n_rows", ctypes.c_int32),
        ("out", ctypes.c_void_p), ("alpha", ctypes.c_float), ("residual", ctypes.c_void_p),
    ]


class Moe(ctypes.Structure):
    """miq_moe (include/miq.h)."""
    _fields_ = [
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("gate_type", ctypes.c_uint32), ("up_type", ctypes.c_uint32), ("down_type", ctypes.c_uint32),
        ("gate_plane", ctypes.c_size_t), ("up_plane", ctypes.c_size_t), ("down_plane", ctypes.c_size_t),
        ("n_embd", ctypes.c_int32), ("n_ff", ctypes.c_int32), ("n_expert", ctypes.c_int32),
    ]


class GgufDesc(ctypes.Structure):
    """miq_gguf_desc (include/miq.h)."""
    _fields_ = [
        ("version", ctypes.c_uint32), ("n_shards", ctypes.c_int32), ("n_tensors", ctypes.c_int64),
        ("n_kv", ctypes.c_int64), ("split_count", ctypes.c_int32), ("split_no", ctypes.c_int32),
        ("map_base", ctypes.c_void_p), ("map_size", ctypes.c_size_t), ("data_offset", ctypes.c_size_t),
    ]


class GgufShardInfo(ctypes.Structure):
    """miq_gguf_shard_info (include/miq.h)."""
    _fields_ = [("base", ctypes.c_void_p), ("size", ctypes.c_size_t), ("data_offset", ctypes.c_size_t)]


class GgufTensorInfo(ctypes.Structure):
    """miq_gguf_tensor_info (include/miq.h)."""
    _fields_ = [
        ("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
        ("dims", ctypes.POINTER(ctypes.c_uint64)), ("n_elements", ctypes.c_uint64), ("n_rows", ctypes.c_uint64),
        ("nbytes", ctypes.c_uint64), ("offset", ctypes.c_uint64), ("data", ctypes.c_void_p),
        ("map_offset", ctypes.c_uint64), ("shard", ctypes.c_int32),
    ]


class GgufKv(ctypes.Structure):
    """miq_gguf_kv (include/miq.h)."""
    _fields_ = [
        ("type", ctypes.c_uint32), ("arr_type", ctypes.c_uint32), ("u64", ctypes.c_uint64), ("i64", ctypes.c_int64),
        ("f64", ctypes.c_double), ("str", ctypes.c_void_p), ("str_len", ctypes.c_uint64), ("n", ctypes.c_uint64),
    ]


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise MiqError(f"{path} is not built: run __graft_entry__.build() (make -C sycl-infer_amd/csrc)")
    lib = ctypes.CDLL(path)
    vp, i32, u32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_float, ctypes.c_size_t
    sig = {
        "miq_version": (ctypes.c_char_p, []),
        "miq_last_error": (ctypes.c_char_p, []),
        "miq_row_bytes": (sz, [u32, i32]),
        "miq_xq": (i32, [vp, vp, vp, i32, i32, vp, vp, vp, i32, i32]),
        "miq_i8_gemv": (i32, [vp, ctypes.POINTER(Seg)]),
        "miq_i8_gemm": (i32, [vp, ctypes.POINTER(Seg), i32]),
        "miq_quant_gemm": (i32, [vp, ctypes.POINTER(Seg), i32]),
        "miq_group_dots": (i32, [vp, vp, u32, i32, i32, vp, vp, i32, vp, i32]),
        "miq_expf_range": (i32, [vp, u32, u32, vp]),
        "miq_set_switch": (i32, [ctypes.c_char_p, i32]),
        "miq_i8_gemm_noalloc": (i32, [vp, ctypes.POINTER(Seg), i32]),
        "miq_i8_gemv_multi": (i32, [vp, ctypes.POINTER(Seg), i32, i32]),
        "miq_quant_gemm_multi": (i32, [vp, ctypes.POINTER(Seg), i32, i32]),
        "miq_moe_route": (i32, [vp, vp, i32, vp, i32, i32, i32, i32, vp, vp, vp]),
        "miq_moe_csr": (i32, [vp, vp, i32, i32, vp, vp, vp, vp]),
        "miq_moe_workspace_bytes": (sz, [ctypes.POINTER(Moe), i32, i32]),
        "miq_moe_experts": (i32, [vp, ctypes.POINTER(Moe), vp, i32, i32, i32, vp, vp, i32, vp, sz]),
        "miq_moe_reduce": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, i32]),
        "miq_quantize_rows": (i32, [u32, vp, vp, ctypes.c_int64, i32, i32]),
        "miq_ggml_type_name": (ctypes.c_char_p, [u32]),
        "miq_ggml_blck_size": (sz, [u32]),
        "miq_ggml_type_size": (sz, [u32]),
        "miq_ggml_row_bytes": (sz, [u32, ctypes.c_uint64]),
        "miq_gguf_open": (vp, [ctypes.c_char_p]),
        "miq_gguf_close": (None, [vp]),
        "miq_gguf_describe": (i32, [vp, ctypes.POINTER(GgufDesc)]),
        "miq_gguf_shard": (i32, [vp, i32, ctypes.POINTER(GgufShardInfo)]),
        "miq_gguf_find": (ctypes.c_int64, [vp, ctypes.c_char_p]),
        "miq_gguf_tensor": (i32, [vp, ctypes.c_int64, ctypes.POINTER(GgufTensorInfo)]),
        "miq_gguf_kv_key": (ctypes.c_char_p, [vp, ctypes.c_int64]),
        "miq_gguf_meta": (vp, [vp, ctypes.c_char_p]),
        "miq_gguf_val_read": (i32, [vp, ctypes.POINTER(GgufKv)]),
        "miq_gguf_val_elem": (vp, [vp, ctypes.c_uint64]),
        "miq_gguf_get_u32": (u32, [vp, ctypes.c_char_p, u32]),
        "miq_gguf_get_f32": (f32, [vp, ctypes.c_char_p, f32]),
        "miq_gguf_get_str": (ctypes.c_char_p, [vp, ctypes.c_char_p]),
        "miq_gguf_drop_cache": (i32, [vp, ctypes.c_uint64, ctypes.c_uint64]),
        "miq_gguf_upload": (i32, [vp, vp, ctypes.c_uint64, ctypes.c_uint64, vp]),
        "miq_w4_pack": (i32, [vp, u32, vp, i32, i32, vp, vp, vp]),
        "miq_w4_act": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp]),
        "miq_w4_gemv": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, f32, i32, i32]),
        "miq_k5_pack": (i32, [vp, u32, vp, i32, i32, vp, vp, vp, vp]),
        "miq_k5_gemv": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, f32, i32, i32]),
        "miq_w4_quant_gemv": (i32, [vp, ctypes.POINTER(W4SegC), i32, i32, vp, vp, i32]),
        "miq_w4_gemm": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, f32, i32, i32, i32]),
        "miq_nat_gemm": (i32, [vp, i32] + [vp] * 13 + [i32, vp, f32, i32, i32, i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != MIQ_OK:
        raise MiqError(f"{what} -> {rc}: {lib().miq_last_error().decode()}")


def _p(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


def row_bytes(qtype: int, K: int) -> int:
    return int(lib().miq_row_bytes(qtype, K))


# ------------------------------------------------------------------ host encoder
def quantize_rows(qtype: int, x, n_threads: int = 0):
    """fp32 numpy [n_rows, K] -> uint8 numpy [n_rows, row_bytes] of GGUF blocks."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, K = x.shape
    out = np.empty((n, row_bytes(qtype, K)), dtype=np.uint8)
    _check(lib().miq_quantize_rows(qtype, x.ctypes.data, out.ctypes.data, n, K, n_threads), "miq_quantize_rows")
    return out


# ------------------------------------------------------------------ activations
@dataclass
class QAct:
    """Quantized activation of TB tokens (cpu_xq layout, group-major)."""
    x8: object      # int8 [K/32, TB, 32]
    xmeta: object   # float32 [K/32, TB, 2]
    xsumq: object   # int32 [K/32, TB, 2]
    TB: int
    K: int


def alloc_act(TB: int, K: int, device="cuda") -> QAct:
    import torch
    G = K // 32
    return QAct(torch.empty((G, TB, 32), dtype=torch.int8, device=device),
                torch.empty((G, TB, 2), dtype=torch.float32, device=device),
                torch.empty((G, TB, 2), dtype=torch.int32, device=device), TB, K)


def xq(x, up=None, out: QAct | None = None, stream=None) -> QAct:
    """compute_backend::xq: x fp32 [TB, >=K] (row stride = x.stride(0))."""
    TB, K = x.shape[0], x.shape[1]
    a = out if out is not None else alloc_act(TB, K, x.device)
    _check(lib().miq_xq(_stream(stream), x.data_ptr(), _p(up), x.stride(0), up.stride(0) if up is not None else 0,
                        a.x8.data_ptr(), a.xmeta.data_ptr(), a.xsumq.data_ptr(), TB, K), "miq_xq")
    return a


def make_seg(w, qtype: int, K: int, n_rows: int, act: QAct, out, out_stride: int | None = None, residual=None,
             alpha: float = 1.0, x=None, act_up=None) -> Seg:
    s = Seg()
    s.w = w.data_ptr()
    s.type = qtype
    s.K = K
    s.n_rows = n_rows
    s.x = _p(x)
    s.x_stride = x.stride(0) if x is not None else 0
    s.act_up = _p(act_up)
    s.out = out.data_ptr()
    s.out_stride = n_rows if out_stride is None else out_stride
    s.residual = _p(residual)
    s.alpha = alpha
    s.x8, s.xmeta, s.xsumq = act.x8.data_ptr(), act.xmeta.data_ptr(), act.xsumq.data_ptr()
    return s


def i8_gemv(seg: Seg, stream=None) -> None:
    _check(lib().miq_i8_gemv(_stream(stream), ctypes.byref(seg)), "miq_i8_gemv")


def i8_gemm(seg: Seg, TB: int, stream=None) -> None:
    _check(lib().miq_i8_gemm(_stream(stream), ctypes.byref(seg), TB), "miq_i8_gemm")


def i8_gemm_noalloc(seg: Seg, TB: int, stream=None) -> None:
    """miq_i8_gemm with the split-K scratch in the library's static device array (no allocation)."""
    _check(lib().miq_i8_gemm_noalloc(_stream(stream), ctypes.byref(seg), TB), "miq_i8_gemm_noalloc")


def i8_gemv_multi(segs, TB: int, stream=None) -> None:
    """compute_backend::i8_row_gemv_multi: every segment of one activation (segs[0]'s) in one call."""
    arr = (Seg * len(segs))(*segs)
    _check(lib().miq_i8_gemv_multi(_stream(stream), arr, len(segs), TB), "miq_i8_gemv_multi")


def quant_gemm_multi(segs, TB: int, stream=None) -> None:
    """The fused quantize + multi-segment form (i8_grp_quant_gemv_launch)."""
    arr = (Seg * len(segs))(*segs)
    _check(lib().miq_quant_gemm_multi(_stream(stream), arr, len(segs), TB), "miq_quant_gemm_multi")


def quant_gemm(seg: Seg, TB: int, stream=None) -> None:
    _check(lib().miq_quant_gemm(_stream(stream), ctypes.byref(seg), TB), "miq_quant_gemm")


def group_dots(w, qtype: int, K: int, n_rows: int, act: QAct, path: int = 0, stream=None):
    import torch
    S = K // 16 if qtype == Q6_K and path != 2 else K // 32
    out = torch.empty((act.TB, n_rows, S), dtype=torch.int32, device=w.device)
    _check(lib().miq_group_dots(_stream(stream), w.data_ptr(), qtype, K, n_rows, act.x8.data_ptr(),
                                act.xsumq.data_ptr(), act.TB, out.data_ptr(), path), "miq_group_dots")
    return out


SWITCH_DEFAULT = -(2 ** 31)  # INT_MIN: back to the environment / built-in default


def set_switch(name: str, value: int) -> None:
    """Set the tuning switch `name` (miq_set_switch); SWITCH_DEFAULT restores it."""
    _check(lib().miq_set_switch(name.encode(), value), "miq_set_switch")


def expf_range(first: int, count: int, y, stream=None) -> None:
    """y[i] = the device expf of the float with bits first + i (a parity hook)."""
    _check(lib().miq_expf_range(_stream(stream), first, count, y.data_ptr()), "miq_expf_range")


# ------------------------------------------------------------------ u4 store
@dataclass
class W4Store:
    """The u4 native-width store (w4t, src/common/w4.h:55-66) on the device."""
    vals: object    # uint8 [N, K/2]
    scale: object   # int16 (f16 bits) [K/32, N]
    off: object     # int16 (f16 bits) [K/32, N]
    K: int
    N: int


@dataclass
class W4Act:
    """act_quant_grp's output (src/backend/dnnl_gemm.cpp:100-146) for M rows."""
    xq: object      # int8 [M, K]
    asa: object     # int16 (f16 bits) [M, K/32]
    xs: object      # float32 [M, K/32]
    axe: object     # int8 [M, K/2]
    axo: object     # int8 [M, K/2]
    M: int
    K: int


def w4_pack(w, K: int, N: int, qtype: int = Q4_K, stream=None) -> W4Store:
    """w4_pack (src/common/w4.cpp:416) of a device Q4_K tensor [N, row_bytes]."""
    import torch
    st = W4Store(torch.empty((N, K // 2), dtype=torch.uint8, device=w.device),
                 torch.empty((K // 32, N), dtype=torch.int16, device=w.device),
                 torch.empty((K // 32, N), dtype=torch.int16, device=w.device), K, N)
    _check(lib().miq_w4_pack(_stream(stream), qtype, w.data_ptr(), K, N, st.vals.data_ptr(), st.scale.data_ptr(),
                             st.off.data_ptr()), "miq_w4_pack")
    return st


def w4_act(x, up=None, out: W4Act | None = None, stream=None) -> W4Act:
    """act_quant_grp_launch with do_split: x fp32 [M, >=K] (row stride = x.stride(0))."""
    import torch
    M, K = x.shape
    d = x.device
    a = out if out is not None else W4Act(
        torch.empty((M, K), dtype=torch.int8, device=d), torch.empty((M, K // 32), dtype=torch.int16, device=d),
        torch.empty((M, K // 32), dtype=torch.float32, device=d), torch.empty((M, K // 2), dtype=torch.int8, device=d),
        torch.empty((M, K // 2), dtype=torch.int8, device=d), M, K)
    _check(lib().miq_w4_act(_stream(stream), x.data_ptr(), _p(up), x.stride(0), up.stride(0) if up is not None else 0,
                            M, K, _p(a.xq), a.asa.data_ptr(), a.xs.data_ptr(), _p(a.axe), _p(a.axo)), "miq_w4_act")
    return a


def w4_gemv(st: W4Store, act: W4Act, out, residual=None, alpha: float = 1.0, row: int = 0, stream=None) -> None:
    """w4_gemv_launch (src/backend/gpu/kernels/kernels.h:240) on activation row `row`: out [N] fp32."""
    K, N = st.K, st.N
    _check(lib().miq_w4_gemv(_stream(stream), st.vals.data_ptr(), st.scale.data_ptr(), st.off.data_ptr(),
                             act.axe[row].data_ptr(), act.axo[row].data_ptr(), act.asa[row].data_ptr(),
                             act.xs[row].data_ptr(), out.data_ptr(), N, _p(residual), alpha, K, N), "miq_w4_gemv")


def w4_gemm(st: W4Store, act: W4Act, out, residual=None, alpha: float = 1.0, stream=None) -> None:
    """w4_gemm_launch (src/backend/gpu/kernels/kernels.h:237): all act.M rows; out [M, >=N] fp32."""
    _check(lib().miq_w4_gemm(_stream(stream), st.vals.data_ptr(), st.scale.data_ptr(), st.off.data_ptr(),
                             act.axe.data_ptr(), act.axo.data_ptr(), act.asa.data_ptr(), act.xs.data_ptr(),
                             out.data_ptr(), out.stride(0), _p(residual), alpha, act.M, st.K, st.N), "miq_w4_gemm")


def w4_quant_gemv(segs, x, up=None, stream=None) -> None:
    """w4_grp_quant_gemv_launch (src/backend/gpu/kernels/kernels.h:235): one token x [K] (or [1, K])
    quantized in the launch, then every segment; segs = [(W4Store, out, alpha, residual)]."""
    arr = (W4SegC * len(segs))()
    rows = 0
    for i, (st, out, alpha, res) in enumerate(segs):
        arr[i].vals, arr[i].scale, arr[i].off = st.vals.data_ptr(), st.scale.data_ptr(), st.off.data_ptr()
        arr[i].n_rows, arr[i].out, arr[i].alpha, arr[i].residual = st.N, out.data_ptr(), alpha, _p(res)
        rows += st.N
    K = segs[0][0].K
    _check(lib().miq_w4_quant_gemv(_stream(stream), arr, len(segs), rows, x.data_ptr(), _p(up), K),
           "miq_w4_quant_gemv")


@dataclass
class K5Store:
    """The k5 native 5-bit store (k5t, src/common/w4.h:104-132) on the device."""
    vals: object    # uint8 [N, K/2]
    hi: object      # uint8 [N, K/8]
    scale: object   # int16 (f16 bits) [K/32, N]
    off: object     # int16 (f16 bits) [K/32, N]
    K: int
    N: int


def k5_pack(w, K: int, N: int, qtype: int = Q5_K, stream=None) -> K5Store:
    """k5_pack (src/common/w4.cpp:409) of a device Q5_K tensor [N, row_bytes]."""
    import torch
    st = K5Store(torch.empty((N, K // 2), dtype=torch.uint8, device=w.device),
                 torch.empty((N, K // 8), dtype=torch.uint8, device=w.device),
                 torch.empty((K // 32, N), dtype=torch.int16, device=w.device),
                 torch.empty((K // 32, N), dtype=torch.int16, device=w.device), K, N)
    _check(lib().miq_k5_pack(_stream(stream), qtype, w.data_ptr(), K, N, st.vals.data_ptr(), st.hi.data_ptr(),
                             st.scale.data_ptr(), st.off.data_ptr()), "miq_k5_pack")
    return st


def k5_gemv(st: K5Store, act: W4Act, out, residual=None, alpha: float = 1.0, row: int = 0, stream=None) -> None:
    """k5_gemv_launch (src/backend/gpu/kernels/kernels.h:267) on activation row `row`: out [N] fp32."""
    _check(lib().miq_k5_gemv(_stream(stream), st.vals.data_ptr(), st.hi.data_ptr(), st.scale.data_ptr(),
                             st.off.data_ptr(), act.axe[row].data_ptr(), act.axo[row].data_ptr(),
                             act.asa[row].data_ptr(), act.xs[row].data_ptr(), out.data_ptr(), _p(residual), alpha,
                             st.K, st.N), "miq_k5_gemv")


def nat_gemm(st, act: W4Act, out, residual=None, alpha: float = 1.0, stream=None) -> None:
    """nat_gemm_launch (src/backend/gpu/kernels/kernels.h:250-262) over a W4Store (fmt 0) or a K5Store
    (fmt 1): all act.M rows (2..32; k5 2..13); out [M, >=N] fp32."""
    k5 = isinstance(st, K5Store)
    _check(lib().miq_nat_gemm(_stream(stream), 1 if k5 else 0, st.vals.data_ptr(), st.hi.data_ptr() if k5 else None,
                              None, st.scale.data_ptr(), st.off.data_ptr(), None, None, act.axe.data_ptr(),
                              act.axo.data_ptr(), None, act.asa.data_ptr(), act.xs.data_ptr(), out.data_ptr(),
                              out.stride(0), _p(residual), alpha, act.M, st.K, st.N), "miq_nat_gemm")


# ------------------------------------------------------------------ MoE
def moe_route(logits, top_k: int, x=None, gate_inp=None, stream=None):
    """Router over [n_tok, n_expert] logits (filled in place when gate_inp is given)."""
    import torch
    n_tok, n_expert = logits.shape
    ids = torch.empty((n_tok, top_k), dtype=torch.int32, device=logits.device)
    wts = torch.empty((n_tok, top_k), dtype=torch.float32, device=logits.device)
    n_embd = gate_inp.shape[1] if gate_inp is not None else 0
    _check(lib().miq_moe_route(_stream(stream), _p(x), x.stride(0) if x is not None else 0, _p(gate_inp), n_tok,
                               n_embd, n_expert, top_k, logits.data_ptr(), ids.data_ptr(), wts.data_ptr()),
           "miq_moe_route")
    return ids, wts


def moe_csr(ids, n_expert: int, stream=None):
    import torch
    n_pairs = ids.numel()
    dev = ids.device
    off = torch.empty(n_expert + 1, dtype=torch.int32, device=dev)
    pair = torch.empty(n_pairs, dtype=torch.int32, device=dev)
    active = torch.empty(n_expert, dtype=torch.int32, device=dev)
    n_active = torch.empty(1, dtype=torch.int32, device=dev)
    _check(lib().miq_moe_csr(_stream(stream), ids.data_ptr(), n_pairs, n_expert, off.data_ptr(), pair.data_ptr(),
                             active.data_ptr(), n_active.data_ptr()), "miq_moe_csr")
    return off, pair, active, n_active


def make_moe(gate, up, down, qtype: int, n_embd: int, n_ff: int, n_expert: int, down_type: int | None = None) -> Moe:
    m = Moe()
    dt = qtype if down_type is None else down_type
    m.gate, m.up, m.down = gate.data_ptr(), up.data_ptr(), down.data_ptr()
    m.gate_type = m.up_type = qtype
    m.down_type = dt
    m.gate_plane = m.up_plane = n_ff * row_bytes(qtype, n_embd)
    m.down_plane = n_embd * row_bytes(dt, n_ff)
    m.n_embd, m.n_ff, m.n_expert = n_embd, n_ff, n_expert
    return m


def moe_workspace(m: Moe, n_tok: int, top_k: int, device="cuda"):
    import torch
    nbytes = int(lib().miq_moe_workspace_bytes(ctypes.byref(m), n_tok, top_k))
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def moe_experts(m: Moe, x, top_k: int, ids, acc, ws, stream=None) -> None:
    n_tok = x.shape[0]
    _check(lib().miq_moe_experts(_stream(stream), ctypes.byref(m), x.data_ptr(), x.stride(0), n_tok, top_k,
                                 ids.data_ptr(), acc.data_ptr(), acc.stride(0), ws.data_ptr(), ws.numel()),
           "miq_moe_experts")


def moe_reduce(acc, wts, top_k: int, out, stream=None) -> None:
    n_tok, n_embd = out.shape
    _check(lib().miq_moe_reduce(_stream(stream), acc.data_ptr(), wts.data_ptr(), top_k, n_tok, n_embd, acc.stride(0),
                                out.data_ptr(), out.stride(0)), "miq_moe_reduce")


# ------------------------------------------------------------------ GGUF files
@dataclass
class GgufTensor:
    """gguf_tensor_info (src/model/gguf.h:64-93) of an open GgufFile."""
    name: str
    type: int
    dims: tuple
    n_elements: int
    n_rows: int
    nbytes: int
    offset: int        # within its shard's data section
    map_offset: int    # from the start of the (whole-model) mapping
    shard: int
    data: int          # host address inside the mapping


class GgufValue:
    """One kv value, widened as gguf_kv (src/model/gguf.h:38-62)."""
    __slots__ = ("type", "arr_type", "u64", "i64", "f64", "str", "arr")

    def __init__(self, h):
        kv = GgufKv()
        _check(lib().miq_gguf_val_read(h, ctypes.byref(kv)), "miq_gguf_val_read")
        self.type, self.arr_type = kv.type, kv.arr_type
        self.u64, self.i64, self.f64 = kv.u64, kv.i64, kv.f64
        self.str = ctypes.string_at(kv.str, kv.str_len) if kv.str else b""
        self.arr = [GgufValue(lib().miq_gguf_val_elem(h, i)) for i in range(kv.n)] if kv.type == 9 else []

    def as_u32(self) -> int:
        return self.u64 & 0xFFFFFFFF

    def as_f32(self) -> float:
        return float(ctypes.c_float(self.f64).value)

    def is_arr(self) -> bool:
        return self.type == 9


class GgufFile:
    """A GGUF model opened by libmiq (mirror of gguf_file, src/model/gguf.h:102-158):
    `find`, `meta`, `get_u32`, `get_f32`, `get_str` keep the reference's names and
    defaults; `tensor_bytes` views a tensor in the mapping; `upload` copies a
    tensor (or any mapping range) into device memory.  Load errors raise MiqError
    with the reference's exception text."""

    def __init__(self, path: str):
        self._h = lib().miq_gguf_open(os.fsencode(path))
        if not self._h:
            raise MiqError(lib().miq_last_error().decode())
        d = GgufDesc()
        _check(lib().miq_gguf_describe(self._h, ctypes.byref(d)), "miq_gguf_describe")
        self.version, self.split_count, self.split_no = d.version, d.split_count, d.split_no
        self.map_base, self.map_size, self.data_offset = d.map_base, d.map_size, d.data_offset
        self.shards = []
        for i in range(d.n_shards):
            s = GgufShardInfo()
            _check(lib().miq_gguf_shard(self._h, i, ctypes.byref(s)), "miq_gguf_shard")
            self.shards.append((s.base, s.size, s.data_offset))
        self.tensors = []
        for i in range(d.n_tensors):
            t = GgufTensorInfo()
            _check(lib().miq_gguf_tensor(self._h, i, ctypes.byref(t)), "miq_gguf_tensor")
            self.tensors.append(GgufTensor(t.name.decode(), t.type, tuple(t.dims[k] for k in range(t.n_dims)),
                                           t.n_elements, t.n_rows, t.nbytes, t.offset, t.map_offset, t.shard,
                                           t.data))
        self.keys = [lib().miq_gguf_kv_key(self._h, i).decode() for i in range(d.n_kv)]

    def close(self) -> None:
        if self._h:
            lib().miq_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def is_split(self) -> bool:
        return len(self.shards) > 1

    def find(self, name: str) -> GgufTensor | None:
        i = lib().miq_gguf_find(self._h, name.encode())
        return None if i < 0 else self.tensors[i]

    def meta(self, key: str) -> GgufValue | None:
        h = lib().miq_gguf_meta(self._h, key.encode())
        return GgufValue(h) if h else None

    def get_u32(self, key: str, default: int = 0) -> int:
        return int(lib().miq_gguf_get_u32(self._h, key.encode(), default))

    def get_f32(self, key: str, default: float = 0.0) -> float:
        return float(lib().miq_gguf_get_f32(self._h, key.encode(), default))

    def get_str(self, key: str) -> str | None:
        r = lib().miq_gguf_get_str(self._h, key.encode())
        return None if r is None else r.decode("utf-8", "surrogateescape")

    def tensor_bytes(self, t: GgufTensor):
        """uint8 numpy view of the tensor's bytes in the mapping (read-only, valid while open)."""
        import numpy as np
        buf = (ctypes.c_uint8 * t.nbytes).from_address(t.data)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def drop_cache(self, off: int, length: int) -> None:
        _check(lib().miq_gguf_drop_cache(self._h, off, length), "miq_gguf_drop_cache")

    def upload(self, dst, off: int, length: int, stream=None) -> None:
        """Copy mapping bytes [off, off+length) into the device tensor `dst`."""
        if dst.numel() * dst.element_size() < length:
            raise MiqError("upload: destination too small")
        _check(lib().miq_gguf_upload(_stream(stream), self._h, off, length, dst.data_ptr()), "miq_gguf_upload")

    def upload_tensor(self, t: GgufTensor, device="cuda", stream=None):
        """The tensor's bytes as a uint8 device tensor [n_rows, nbytes/n_rows]."""
        import torch
        rows = max(int(t.n_rows), 1)
        out = torch.empty((rows, t.nbytes // rows), dtype=torch.uint8, device=device)
        self.upload(out, t.map_offset, t.nbytes, stream)
        return out
