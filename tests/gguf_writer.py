"""Minimal GGUF v3 writer for tests (written from the published GGUF layout,
independently of the library's reader).

Layout: little-endian u32 magic 0x46554747 ("GGUF"), u32 version 3,
u64 n_tensors, u64 n_kv, then the key/value pairs (string key, u32 type, value),
the tensor infos (string name, u32 ndim, u64 ne[ndim], u32 type, u64 offset)
and the data section at the next multiple of general.alignment (default 32).
"""
import struct

import numpy as np

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
        T_BOOL: "<B", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _val(t, v):
    if t == T_STR:
        return _str(v)
    if t == T_ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_val(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(kv, tensors, alignment=32, version=3, magic=0x46554747):
    """kv: [(key, type, value)]; tensors: [(name, ggml_type, ne, payload bytes)].
    Payloads are placed in order, each at an alignment boundary."""
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(kv))
    head += b"".join(_str(k) + struct.pack("<I", t) + _val(t, v) for k, t, v in kv)
    offsets, off = [], 0
    for _, _, _, payload in tensors:
        offsets.append(off)
        off += (len(payload) + alignment - 1) // alignment * alignment
    for (name, gt, ne, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gt, o)
    pad = (-len(head)) % alignment
    data = bytearray()
    for (_, _, _, payload), o in zip(tensors, offsets):
        data += b"\0" * (o - len(data))
        data += bytes(payload)
    return head + b"\0" * pad + bytes(data), len(head) + pad


def write_gguf(path, kv, tensors, **kw):
    blob, data_offset = gguf_bytes(kv, tensors, **kw)
    with open(path, "wb") as f:
        f.write(blob)
    return data_offset


def random_kquant(seed, N, K, block_bytes):
    """Random k-quant blocks with finite fp16 scale fields (d, dmin for Q5_K at
    bytes 0..3; d for Q6_K at bytes 208..209)."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(N, K // 256, block_bytes), dtype=np.uint8)
    h = rng.uniform(1e-3, 2e-2, size=(N, K // 256, 2)).astype(np.float16).view(np.uint8)
    if block_bytes == 176:
        b[..., 0:4] = h.reshape(N, K // 256, 4)
    else:
        b[..., 208:210] = h[..., 0:2]
    return b.reshape(N, -1)
