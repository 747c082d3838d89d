"""A minimal GGUF writer for tests (the GGUF v2/v3 container: header, metadata,
tensor table, aligned data section).  It builds the files the loader tests parse:
edge-case metadata, shared experts, dense FFN layers, truncated files, and the
GPU test's model file made from the committed layer-0 fixture of the reference's
toy model."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "?", U64: "Q", I64: "q", F64: "d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack("<" + _FMT[t], v)


def write_gguf(path: str, metadata: list, tensors: list, version: int = 3, alignment: int = 32) -> None:
    """metadata: [(key, type, value)]; tensors: [(name, dims, ggml_type, raw bytes)] in file order.
    Tensor data are laid out in order, each at a multiple of `alignment` inside the data section."""
    kv = b""
    for key, t, v in metadata:
        kv += _str(key) + struct.pack("<I", t) + _value(t, v)
    infos, blobs, off = b"", [], 0
    for name, dims, ty, raw in tensors:
        raw = bytes(np.asarray(raw, np.uint8).tobytes()) if not isinstance(raw, (bytes, bytearray)) else bytes(raw)
        infos += _str(name) + struct.pack("<I", len(dims)) + struct.pack("<" + "Q" * len(dims), *dims)
        infos += struct.pack("<IQ", ty, off)
        pad = (-len(raw)) % alignment
        blobs.append(raw + b"\0" * pad)
        off += len(raw) + pad
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata)) + kv + infos
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        for b in blobs:
            f.write(b)
