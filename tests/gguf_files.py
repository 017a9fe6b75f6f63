"""Small GGUF files for the reader's tests, written from the published GGUF
layout (little-endian): magic "GGUF", version, tensor count, metadata count,
metadata (key string, u32 type, value), tensor infos (name, u32 n_dims, u64
extents, u32 ggml type, u64 offset), padding to the alignment, then the
tensor data.  Strings are u64 length + bytes.  The layout is the one
src/gguf/mod.rs:459-532 reads."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}
# ggml type -> (elements, bytes) per block, for the types the tests use
BLOCK = {0: (1, 4), 1: (1, 2), 12: (256, 144), 13: (256, 176), 14: (256, 210), 8: (32, 34)}


def gstr(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def meta_value(ty: int, value, array_type: int | None = None) -> bytes:
    if ty == STRING:
        return gstr(value)
    if ty == ARRAY:
        out = struct.pack("<IQ", array_type, len(value))
        for v in value:
            out += gstr(v) if array_type == STRING else struct.pack(_SCALAR[array_type], v)
        return out
    return struct.pack(_SCALAR[ty], value)


def build(tensors, meta=(), alignment: int | None = None, version: int = 3, magic: bytes = b"GGUF",
          tensor_count: int | None = None):
    """tensors: [(name, ggml_type, shape, data bytes)]; meta: [(key, type,
    value[, array_type])].  Offsets are laid out at the alignment.  Returns
    (file bytes, {name: (offset, nbytes)}, data_offset)."""
    align = alignment or 32
    meta = list(meta)
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
    head = magic + struct.pack("<IQQ", version, len(tensors) if tensor_count is None else tensor_count, len(meta))
    for m in meta:
        key, ty, value = m[0], m[1], m[2]
        head += gstr(key) + struct.pack("<I", ty) + meta_value(ty, value, m[3] if len(m) > 3 else None)
    offsets, off = {}, 0
    infos = b""
    for name, ty, shape, data in tensors:
        off = (off + align - 1) // align * align
        infos += gstr(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        infos += struct.pack("<IQ", ty, off)
        offsets[name] = (off, len(data))
        off += len(data)
    desc = head + infos
    data_offset = (len(desc) + align - 1) // align * align
    blob = bytearray(desc + b"\0" * (data_offset - len(desc)))
    for name, ty, shape, data in tensors:
        o, n = offsets[name]
        end = data_offset + o
        blob += b"\0" * (end - len(blob))
        blob += data
    return bytes(blob), offsets, data_offset


def tensor_bytes(ty: int, shape, seed: int) -> bytes:
    """Random bytes of the tensor's size (F32: finite normals)."""
    elems = int(np.prod(shape))
    be, bb = BLOCK[ty]
    rng = np.random.default_rng(seed)
    if ty == 0:
        return rng.standard_normal(elems).astype(np.float32).tobytes()
    return rng.integers(0, 256, elems // be * bb, dtype=np.uint8).tobytes()
