"""ctypes binding of libjxmoe.so (declarations in include/jxmoe.h).

Loading fails loudly: there is no CPU fallback for the MoE path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libjxmoe.so")

JX_OK = 0
ERRORS = {1: "JX_ERR_INVALID", 2: "JX_ERR_UNSUPPORTED", 3: "JX_ERR_HIP", 4: "JX_ERR_NOMEM", 5: "JX_ERR_NODEVICE"}

JX_FWD_DEVICE_PTRS = 1 << 0
JX_FWD_ASYNC = 1 << 1
JX_FWD_FORCE_GEMV = 1 << 2
JX_FWD_FORCE_MFMA = 1 << 3
JX_FWD_RESIDUAL = 1 << 4
JX_FWD_UNFUSED = 1 << 5
JX_FWD_TEST_GIVEUP = 1 << 6  # test hook: the fused one-token step's waits give up (outputs invalid)

JX_ACT_SILU = 0
JX_ACT_GELU_TANH = 1

# Every symbol include/jxmoe.h declares.
EXPORTS = [
    "jx_moe_init", "jx_moe_layer_create", "jx_moe_layer_destroy", "jx_moe_forward", "jx_moe_last_logits",
    "jx_moe_last_xq8",
    "jx_moe_profile", "jx_moe_profile_read", "jx_qmatrix_create", "jx_qmatrix_destroy", "jx_matmul_quant_f32",
    "jx_matmul_swiglu_quant_f32", "jx_quantize_row_q8_0", "jx_matmul_quant_f32_noalloc", "jx_dev_alloc", "jx_dev_free", "jx_memcpy_htod",
    "jx_memcpy_dtoh", "jx_device_synchronize", "jx_moe_last_error", "jx_tier_record", "jx_tier_lfru_score",
    "jx_gguf_open", "jx_gguf_close", "jx_gguf_tensor_count", "jx_gguf_find_tensor", "jx_gguf_tensor_info",
    "jx_gguf_get_u32", "jx_gguf_get_f32", "jx_gguf_get_str", "jx_gguf_moe_layer_desc", "jx_gguf_last_error",
    "jx_matmul_quant_f32_dev", "jx_matmul_qkv_quant_f32_dev", "jx_moe_layer_status",
    "jx_build_id",
]

_fp = C.POINTER(C.c_float)
_vp = C.c_void_p


class LayerDesc(C.Structure):
    """jx_moe_layer_desc."""
    _fields_ = [
        ("n_experts", C.c_int32), ("top_k", C.c_int32), ("d_model", C.c_int32), ("d_ff", C.c_int32),
        ("gate_type", C.c_int32), ("up_type", C.c_int32), ("down_type", C.c_int32),
        ("router", _vp), ("router_bias", _vp),
        ("gate_exps", _vp), ("up_exps", _vp), ("down_exps", _vp),
        ("d_ff_shared", C.c_int32),
        ("sh_gate_type", C.c_int32), ("sh_up_type", C.c_int32), ("sh_down_type", C.c_int32),
        ("sh_gate", _vp), ("sh_up", _vp), ("sh_down", _vp),
        ("sh_gate_inp", _vp),
        ("activation", C.c_int32), ("router_type", C.c_int32),
        ("ffn_norm", _vp), ("post_ffw_norm", _vp), ("rms_norm_eps", C.c_float),
    ]


class JxError(RuntimeError):
    pass


_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise JxError(f"{LIB_PATH} is missing: build it with `python -m jxai_amd.build` "
                      "(the MoE path has no CPU fallback)")
    L = C.CDLL(LIB_PATH)
    L.jx_moe_last_error.restype = C.c_char_p
    L.jx_build_id.restype = C.c_char_p
    L.jx_moe_init.argtypes = [C.c_int32]
    L.jx_moe_layer_create.argtypes = [C.POINTER(LayerDesc), C.POINTER(_vp)]
    L.jx_moe_layer_destroy.argtypes = [_vp]
    L.jx_moe_layer_destroy.restype = None
    L.jx_moe_forward.argtypes = [_vp, _vp, C.c_int32, _vp, _vp, _vp, _vp, _vp, C.c_uint32]
    L.jx_moe_last_logits.argtypes = [_vp, _vp, C.c_int32]
    L.jx_moe_layer_status.argtypes = [_vp, C.c_int32]
    L.jx_moe_last_xq8.argtypes = [_vp, _vp, C.c_int32]
    L.jx_moe_profile.argtypes = [_vp, C.c_int32]
    L.jx_moe_profile_read.argtypes = [_vp, C.c_char_p, C.c_size_t, C.POINTER(C.c_double), C.POINTER(C.c_int64),
                                      C.c_int32, C.POINTER(C.c_int32)]
    L.jx_qmatrix_create.argtypes = [C.c_int32, C.c_int64, C.c_int64, _vp, C.POINTER(_vp)]
    L.jx_qmatrix_destroy.argtypes = [_vp]
    L.jx_qmatrix_destroy.restype = None
    L.jx_matmul_quant_f32.argtypes = [_vp, _vp, _vp]
    L.jx_matmul_quant_f32_noalloc.argtypes = [_vp, _vp, _vp, _vp]
    L.jx_matmul_quant_f32_dev.argtypes = [_vp, _vp, _vp, _vp]
    L.jx_matmul_qkv_quant_f32_dev.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    L.jx_matmul_swiglu_quant_f32.argtypes = [_vp, _vp, _vp, _vp, C.c_int32]
    L.jx_quantize_row_q8_0.argtypes = [_vp, _vp, C.c_int64]
    L.jx_dev_alloc.argtypes = [C.c_size_t, C.POINTER(_vp)]
    L.jx_dev_free.argtypes = [_vp]
    L.jx_memcpy_htod.argtypes = [_vp, _vp, C.c_size_t]
    L.jx_memcpy_dtoh.argtypes = [_vp, _vp, C.c_size_t]
    L.jx_device_synchronize.argtypes = []
    L.jx_tier_record.argtypes = [C.c_uint32, C.c_uint32, _vp, _vp, C.c_int32, C.c_int32, C.c_uint32, _vp, _vp, _vp,
                                 C.c_size_t]
    L.jx_tier_lfru_score.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
    L.jx_tier_lfru_score.restype = C.c_uint32
    L.jx_gguf_open.argtypes = [C.c_char_p, C.POINTER(_vp)]
    L.jx_gguf_close.argtypes = [_vp]
    L.jx_gguf_close.restype = None
    L.jx_gguf_tensor_count.argtypes = [_vp]
    L.jx_gguf_tensor_count.restype = C.c_int64
    L.jx_gguf_find_tensor.argtypes = [_vp, C.c_char_p]
    L.jx_gguf_find_tensor.restype = C.c_int64
    L.jx_gguf_tensor_info.argtypes = [_vp, C.c_int64, C.POINTER(C.c_char_p), C.POINTER(C.c_int32),
                                      C.POINTER(C.c_int32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                      C.POINTER(C.c_uint64), C.POINTER(_vp)]
    L.jx_gguf_get_u32.argtypes = [_vp, C.c_char_p, C.c_uint32, C.POINTER(C.c_uint32)]
    L.jx_gguf_get_f32.argtypes = [_vp, C.c_char_p, C.c_float, C.POINTER(C.c_float)]
    L.jx_gguf_get_str.argtypes = [_vp, C.c_char_p, C.POINTER(C.c_char_p)]
    L.jx_gguf_moe_layer_desc.argtypes = [_vp, C.c_int32, C.POINTER(LayerDesc)]
    L.jx_gguf_last_error.restype = C.c_char_p
    _lib = L
    return L


def check(rc: int, what: str) -> None:
    if rc != JX_OK:
        msg = lib().jx_moe_last_error().decode(errors="replace")
        raise JxError(f"{what} failed: {ERRORS.get(rc, rc)}: {msg}")
