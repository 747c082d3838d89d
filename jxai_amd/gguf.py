"""GGUF model files feeding the MoE layer upload (host side of libjxmoe.so).

    f = GGUFFile(path)                  # ModelFile::open / parse_gguf (src/gguf.cpp:810-889)
    f.tensors()                         # name -> (type, dims, file offset, bytes)
    f.get_u32("qwen2moe.expert_used_count", 2)
    layer = f.moe_layer(0)              # bind_tensors for blk.0 (src/transformer.cpp:2116-2199)
                                        # then jx_moe_layer_create: one upload to HBM
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import JxError, LayerDesc, lib  # noqa: F401  (JxError: the error callers catch)
from . import moe as _moe


def _check(rc, what):
    if rc != 0:
        raise JxError(f"{what} failed: {lib().jx_gguf_last_error().decode(errors='replace')}")


class GGUFFile:
    def __init__(self, path: str):
        self.path = path
        self.handle = C.c_void_p()
        _check(lib().jx_gguf_open(path.encode(), C.byref(self.handle)), "jx_gguf_open")

    def tensor_count(self) -> int:
        return int(lib().jx_gguf_tensor_count(self.handle))

    def tensor(self, i: int) -> dict:
        name = C.c_char_p()
        t, nd = C.c_int32(), C.c_int32()
        dims = (C.c_uint64 * 4)()
        off, nb = C.c_uint64(), C.c_uint64()
        data = C.c_void_p()
        _check(lib().jx_gguf_tensor_info(self.handle, i, C.byref(name), C.byref(t), C.byref(nd), dims, C.byref(off),
                                         C.byref(nb), C.byref(data)), "jx_gguf_tensor_info")
        return {"name": name.value.decode(), "type": t.value, "n_dims": nd.value, "dims": list(dims),
                "offset": off.value, "bytes": nb.value, "data": data.value}

    def tensors(self) -> dict:
        return {t["name"]: t for t in (self.tensor(i) for i in range(self.tensor_count()))}

    def find(self, name: str) -> int:
        return int(lib().jx_gguf_find_tensor(self.handle, name.encode()))

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A copy of one tensor's bytes."""
        t = self.tensor(self.find(name))
        return np.ctypeslib.as_array((C.c_uint8 * t["bytes"]).from_address(t["data"])).copy()

    def get_u32(self, key: str, default: int = 0) -> int:
        v = C.c_uint32()
        _check(lib().jx_gguf_get_u32(self.handle, key.encode(), default, C.byref(v)), "jx_gguf_get_u32")
        return v.value

    def get_f32(self, key: str, default: float = 0.0) -> float:
        v = C.c_float()
        _check(lib().jx_gguf_get_f32(self.handle, key.encode(), default, C.byref(v)), "jx_gguf_get_f32")
        return v.value

    def get_str(self, key: str):
        v = C.c_char_p()
        _check(lib().jx_gguf_get_str(self.handle, key.encode(), C.byref(v)), "jx_gguf_get_str")
        return None if v.value is None else v.value.decode()

    def layer_desc(self, layer: int) -> LayerDesc:
        d = LayerDesc()
        _check(lib().jx_gguf_moe_layer_desc(self.handle, layer, C.byref(d)), "jx_gguf_moe_layer_desc")
        return d

    def moe_layer(self, layer: int, device: int = 0) -> "_moe.MoELayer":
        """Layer `layer`'s MoE block uploaded to the device (the file may be closed afterwards)."""
        return _moe.MoELayer.from_desc(self.layer_desc(layer), device)

    def close(self) -> None:
        if self.handle:
            lib().jx_gguf_close(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
