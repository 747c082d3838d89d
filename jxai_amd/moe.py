"""Host-side mirror of the reference's MoE-path interfaces over libjxmoe.so.

  MoELayer.forward          the MoE block of forward_token
                            (src/transformer.cpp:2589-2757), batched over tokens
  matmul_quant_f32          include/quant.h:336-343
  matmul_swiglu_quant_f32   include/quant.h:354-362
  quantize_row_q8_0         include/quant.h:112

Arguments keep the reference's meaning (GGML type codes, row-major block
matrices [rows][cols], fp32 activations); errors raise JxError instead of the
reference's warn-and-return-zero.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import formats as F
from ._lib import (JX_FWD_DEVICE_PTRS, JX_FWD_ASYNC, JX_FWD_FORCE_GEMV, JX_FWD_FORCE_MFMA, JX_FWD_RESIDUAL,  # noqa: F401
                   JX_FWD_UNFUSED, JX_FWD_TEST_GIVEUP,
                   JxError, LayerDesc, check, lib)

_inited = {}


def init(device: int = 0) -> None:
    if device not in _inited:
        check(lib().jx_moe_init(device), "jx_moe_init")
        _inited[device] = True


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


class DeviceBuffer:
    """A device allocation owned by the library's allocator."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = C.c_void_p()
        check(lib().jx_dev_alloc(max(self.nbytes, 1), C.byref(self.ptr)), "jx_dev_alloc")

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().jx_memcpy_htod(self.ptr, _p(a), a.nbytes), "jx_memcpy_htod")
        return self

    def download(self, out: np.ndarray) -> np.ndarray:
        assert out.flags.c_contiguous and out.nbytes <= self.nbytes
        check(lib().jx_memcpy_dtoh(_p(out), self.ptr, out.nbytes), "jx_memcpy_dtoh")
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib().jx_dev_free(self.ptr), "jx_dev_free")
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class MoELayer:
    """One MoE layer resident in HBM (jx_moe_layer)."""

    def __init__(self, *, n_experts, top_k, d_model, d_ff, gate_type, up_type, down_type, router,
                 gate_exps, up_exps, down_exps, router_bias=None, d_ff_shared=0, sh_gate_type=None,
                 sh_up_type=None, sh_down_type=None, sh_gate=None, sh_up=None, sh_down=None,
                 sh_gate_inp=None, activation: int = 0, router_type: int = F.F32, ffn_norm=None,
                 post_ffw_norm=None, rms_norm_eps: float = 1e-5, device: int = 0):
        init(device)
        keep = [np.ascontiguousarray(a) if a is not None else None
                for a in (router, router_bias, gate_exps, up_exps, down_exps, sh_gate, sh_up, sh_down, sh_gate_inp,
                          ffn_norm, post_ffw_norm)]
        (router, router_bias, gate_exps, up_exps, down_exps, sh_gate, sh_up, sh_down, sh_gate_inp, ffn_norm,
         post_ffw_norm) = keep
        if router.size != n_experts * d_model or router.dtype != (np.float32 if router_type == F.F32 else np.uint16):
            raise JxError("router must hold E x d_model fp32 values (F32) or half / bfloat16 bits (F16 / BF16)")
        for name, a, t, rows, cols in (("gate", gate_exps, gate_type, d_ff, d_model),
                                       ("up", up_exps, up_type, d_ff, d_model),
                                       ("down", down_exps, down_type, d_model, d_ff)):
            want = n_experts * F.matrix_bytes(t, rows, cols)
            if a.nbytes != want:
                raise JxError(f"{name}_exps holds {a.nbytes} bytes, expected {want}")
        D = LayerDesc(n_experts, top_k, d_model, d_ff, gate_type, up_type, down_type,
                      _p(router), _p(router_bias), _p(gate_exps), _p(up_exps), _p(down_exps),
                      d_ff_shared, sh_gate_type or 0, sh_up_type or 0, sh_down_type or 0,
                      _p(sh_gate), _p(sh_up), _p(sh_down), _p(sh_gate_inp), activation, router_type,
                      _p(ffn_norm), _p(post_ffw_norm), rms_norm_eps)
        self.handle = C.c_void_p()
        check(lib().jx_moe_layer_create(C.byref(D), C.byref(self.handle)), "jx_moe_layer_create")
        self.E, self.k, self.d, self.F = n_experts, top_k, d_model, d_ff

    @classmethod
    def from_desc(cls, desc: LayerDesc, device: int = 0) -> "MoELayer":
        """From a filled jx_moe_layer_desc (e.g. jxai_amd.gguf's binding of a model file)."""
        init(device)
        self = cls.__new__(cls)
        self.handle = C.c_void_p()
        check(lib().jx_moe_layer_create(C.byref(desc), C.byref(self.handle)), "jx_moe_layer_create")
        self.E, self.k, self.d, self.F = desc.n_experts, desc.top_k, desc.d_model, desc.d_ff
        return self

    @classmethod
    def from_weights(cls, lw, device: int = 0) -> "MoELayer":
        """From a jxai_amd.synth.LayerWeights."""
        cfg = lw.cfg
        gt, ut, dt = lw.types
        kw = {}
        if cfg.has_shared:
            sgt, sut, sdt = lw.sh_types
            kw = dict(d_ff_shared=cfg.d_ff_shared, sh_gate_type=sgt, sh_up_type=sut, sh_down_type=sdt,
                      sh_gate=lw.sh_gate, sh_up=lw.sh_up, sh_down=lw.sh_down, sh_gate_inp=lw.sh_gate_inp)
        return cls(n_experts=cfg.n_experts, top_k=cfg.top_k, d_model=cfg.d_model, d_ff=cfg.d_ff,
                   gate_type=gt, up_type=ut, down_type=dt, router=lw.router, router_bias=lw.router_bias,
                   gate_exps=lw.gate, up_exps=lw.up, down_exps=lw.down, activation=cfg.act,
                   ffn_norm=lw.ffn_norm, post_ffw_norm=lw.post_ffw_norm, rms_norm_eps=cfg.rms_eps,
                   router_type=cfg.router_type, device=device, **kw)

    def forward(self, x: np.ndarray, regime: str | None = None, residual: bool = False, fused: bool = True):
        """MoE block over host activations [n][d] -> (out [n][d], topk_ids, topk_w, counts).
        residual: x is the residual stream and out = x + the block on rms_norm(x) (JX_FWD_RESIDUAL).
        fused=False: a one-token step as separate launches (JX_FWD_UNFUSED; same results)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        out = np.empty((n, self.d), np.float32)
        ids = np.empty((n, self.k), np.int32)
        w = np.empty((n, self.k), np.float32)
        counts = np.empty(self.E, np.int32)
        flags = {None: 0, "gemv": JX_FWD_FORCE_GEMV, "mfma": JX_FWD_FORCE_MFMA}[regime]
        flags |= JX_FWD_RESIDUAL if residual else 0
        flags |= 0 if fused else JX_FWD_UNFUSED
        check(lib().jx_moe_forward(self.handle, _p(x), n, _p(out), _p(ids), _p(w), _p(counts), None, flags),
              "jx_moe_forward")
        return out, ids, w, counts

    def forward_device(self, x: DeviceBuffer, n: int, out: DeviceBuffer, sync: bool = True, regime=None,
                       stream=None, fused: bool = True, extra_flags: int = 0) -> None:
        """MoE block over device-resident activations (no host copies), enqueued on `stream`
        (a hipStream_t as an integer; None: the layer's own stream)."""
        flags = JX_FWD_DEVICE_PTRS | (0 if sync else JX_FWD_ASYNC) | (0 if fused else JX_FWD_UNFUSED) | extra_flags
        flags |= {None: 0, "gemv": JX_FWD_FORCE_GEMV, "mfma": JX_FWD_FORCE_MFMA}[regime]
        st = None if stream is None else C.c_void_p(stream)
        check(lib().jx_moe_forward(self.handle, x.ptr, n, out.ptr, None, None, None, st, flags), "jx_moe_forward")

    def status(self, wait: bool = True) -> None:
        """Raise JxError if a fused one-token step of this layer gave up a wait between its blocks since
        the last report (jx_moe_layer_status; wait: synchronize the last forward's stream first)."""
        check(lib().jx_moe_layer_status(self.handle, 1 if wait else 0), "jx_moe_layer_status")

    def last_logits(self, n: int) -> np.ndarray:
        out = np.empty((n, self.E), np.float32)
        check(lib().jx_moe_last_logits(self.handle, _p(out), n), "jx_moe_last_logits")
        return out

    def last_xq8(self, n: int) -> np.ndarray:
        """Q8_0 blocks of the last forward's activations as the router kernels wrote them."""
        out = np.empty(n * (self.d // 32) * 34, np.uint8)
        check(lib().jx_moe_last_xq8(self.handle, _p(out), n), "jx_moe_last_xq8")
        return out.reshape(n, -1)

    def profile(self, enable: bool = True) -> None:
        check(lib().jx_moe_profile(self.handle, 1 if enable else 0), "jx_moe_profile")

    def profile_read(self) -> dict:
        buf = C.create_string_buffer(4096)
        ms = (C.c_double * 32)()
        cnt = (C.c_int64 * 32)()
        n = C.c_int32()
        check(lib().jx_moe_profile_read(self.handle, buf, 4096, ms, cnt, 32, C.byref(n)), "jx_moe_profile_read")
        names = buf.value.decode().split(";")[: n.value]
        return {nm: (ms[i], cnt[i]) for i, nm in enumerate(names)}

    def close(self) -> None:
        if self.handle:
            lib().jx_moe_layer_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QMatrix:
    """A quantized [rows][cols] weight matrix resident on the device (jx_qmatrix)."""

    def __init__(self, qtype: int, W: np.ndarray, rows: int, cols: int, device: int = 0):
        init(device)
        W = np.ascontiguousarray(W, dtype=np.uint8)
        if W.nbytes != F.matrix_bytes(qtype, rows, cols):
            raise JxError("W size does not match rows x cols")
        self.qtype, self.rows, self.cols = qtype, rows, cols
        self.handle = C.c_void_p()
        check(lib().jx_qmatrix_create(qtype, rows, cols, _p(W), C.byref(self.handle)), "jx_qmatrix_create")

    def close(self):
        if self.handle:
            lib().jx_qmatrix_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matmul_quant_f32(qtype: int, W, x, rows: int, cols: int) -> np.ndarray:
    """out[r] = W[r] . x on the GPU (reference: matmul_quant_f32)."""
    m = W if isinstance(W, QMatrix) else QMatrix(qtype, W, rows, cols)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows, np.float32)
    check(lib().jx_matmul_quant_f32(m.handle, _p(x), _p(out)), "jx_matmul_quant_f32")
    return out


def matmul_swiglu_quant_f32(gate_type: int, W_gate, up_type: int, W_up, x, exp_dim: int, cols: int,
                            use_gelu: bool = False) -> np.ndarray:
    """act(W_gate x) * (W_up x), act = SiLU or GELU-tanh, on the GPU (reference: matmul_swiglu_quant_f32)."""
    g = W_gate if isinstance(W_gate, QMatrix) else QMatrix(gate_type, W_gate, exp_dim, cols)
    u = W_up if isinstance(W_up, QMatrix) else QMatrix(up_type, W_up, exp_dim, cols)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(exp_dim, np.float32)
    check(lib().jx_matmul_swiglu_quant_f32(g.handle, u.handle, _p(x), _p(out), 1 if use_gelu else 0),
          "jx_matmul_swiglu_quant_f32")
    return out


def quantize_row_q8_0(x) -> np.ndarray:
    """Q8_0 blocks (34 bytes per 32 values) computed on the GPU."""
    init(0)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 34, np.uint8)
    check(lib().jx_quantize_row_q8_0(_p(x), _p(out), x.size), "jx_quantize_row_q8_0")
    return out
