"""Minimal GGUF v3 writer for the tests: small checkpoints whose tensors the tests generate themselves (weights
quantised with the oracle's restatement of ggml's reference quantisers). The layout is the public GGUF format
(llama.cpp docs/gguf.md): header, typed key/values, tensor table, data section aligned to general.alignment.

kv entries are (key, type, value) with type one of the GGUF_* codes; arrays are (key, GGUF_ARRAY, (elem_type, values)).
tensors are (name, ggml_type, ne, data) with ne in ggml order (ne[0] contiguous) and data the raw bytes.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL = 0, 1, 2, 3, 4, 5, 6, 7
GGUF_STRING, GGUF_ARRAY, GGUF_U64, GGUF_I64, GGUF_F64 = 8, 9, 10, 11, 12

F32, BF16 = 0, 30
_SCALAR = {GGUF_U8: "<B", GGUF_I8: "<b", GGUF_U16: "<H", GGUF_I16: "<h", GGUF_U32: "<I", GGUF_I32: "<i",
           GGUF_F32: "<f", GGUF_BOOL: "<B", GGUF_U64: "<Q", GGUF_I64: "<q", GGUF_F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == GGUF_STRING:
        return _str(v)
    if t == GGUF_ARRAY:
        et, vals = v
        out = struct.pack("<IQ", et, len(vals))
        return out + b"".join(_value(et, x) for x in vals)
    return struct.pack(_SCALAR[t], int(v) if t not in (GGUF_F32, GGUF_F64) else float(v))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def write_gguf(path: str | Path, kv: list, tensors: list, alignment: int = 32, version: int = 3) -> None:
    kv = list(kv)
    if alignment != 32:
        kv.append(("general.alignment", GGUF_U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    blobs, off = [], 0
    for name, gtype, ne, data in tensors:
        raw = bytes(np.ascontiguousarray(data).view(np.uint8).tobytes())
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gtype, off)
        pad = (-len(raw)) % alignment
        blobs.append(raw + b"\0" * pad)
        off += len(raw) + pad
    head += b"\0" * ((-len(head)) % alignment)
    Path(path).write_bytes(head + b"".join(blobs))
