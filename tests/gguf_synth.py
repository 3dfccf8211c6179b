"""TEST INFRASTRUCTURE: writes GGUF files from Python for the reader's tests.

Written from the published GGUF layout (little-endian): magic 'GGUF', u32
version, u64 n_tensors, u64 n_kv; kv pairs (string key, u32 value type,
value); tensor infos (string name, u32 n_dims, u64 dims[n_dims], u32 ggml
type, u64 offset into the data section); zero padding to `general.alignment`
(32 by default); the data section.  Strings are a u64 length plus bytes.
The same layout is what src/model/gguf.cpp:104-289 of sycl-infer parses.
"""
from __future__ import annotations

import struct

# GGUF value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(b) -> bytes:
    if isinstance(b, str):
        b = b.encode()
    return struct.pack("<Q", len(b)) + b


def value(vtype: int, v) -> bytes:
    """Encoded value of type vtype.  ARR takes (elem_type, [values])."""
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def header(kv, infos, version: int = 3, n_tensors: int | None = None) -> bytes:
    """kv: [(key, vtype, value)]; infos: [(name, dims, ggml_type, offset)]."""
    out = [b"GGUF", struct.pack("<IQQ", version, len(infos) if n_tensors is None else n_tensors, len(kv))]
    for key, vt, v in kv:
        out += [_str(key), struct.pack("<I", vt), value(vt, v)]
    for name, dims, gt, off in infos:
        out += [_str(name), struct.pack("<I", len(dims)), struct.pack(f"<{len(dims)}Q", *dims),
                struct.pack("<IQ", gt, off)]
    return b"".join(out)


def build(kv, tensors, alignment: int | None = None, version: int = 3) -> tuple[bytes, dict]:
    """A whole file.  tensors: [(name, dims, ggml_type, bytes)]; each tensor's
    data starts at a multiple of the alignment inside the data section.
    Returns the file bytes and {name: absolute file offset of its data}."""
    al = 32 if alignment is None else alignment
    kv = list(kv)
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    infos, blobs, off = [], [], 0
    for name, dims, gt, data in tensors:
        infos.append((name, dims, gt, off))
        blobs.append((off, data))
        off = (off + len(data) + al - 1) // al * al
    head = header(kv, infos, version)
    data_off = (len(head) + al - 1) // al * al
    body = bytearray(off if tensors else 0)
    for o, d in blobs:
        body[o:o + len(d)] = d
    where = {name: data_off + o for (name, _, _, _), (o, _) in zip(tensors, blobs)}
    raw = head + b"\0" * (data_off - len(head)) + bytes(body) if tensors else head
    return raw, where


def shard_name(stem: str, i: int, n: int) -> str:
    return f"{stem}-{i:05d}-of-{n:05d}.gguf"
