"""Seeded synthetic MoE layers and token batches.

One generator feeds the GPU path, the oracle and the golden-vector script, so
all three see identical bytes.  Everything derives from SplitMix64 streams:

  * sub-seed  = splitmix64(base_seed XOR fnv1a64("<config>/<tensor>"))
  * uniform   = (u64 >> 11) * 2**-53                      in [0, 1)
  * normal    = Box-Muller in float64 on (1-u0, u1) pairs, rounded to fp32
  * fp16 scale= float16(lo + (hi-lo)*u)  (round to nearest even)
  * bytes     = the little-endian bytes of consecutive u64 outputs
  * int8      = (byte mod 255) - 127

Weight tensors are produced in the reference's on-disk block layout
(include/quant.h:10-33), packed over experts the way GGUF stores
``ffn_{gate,up,down}_exps`` (expert e's slice at e * bytes/E,
src/transformer.cpp:2166-2185).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import formats as F

BASE_SEED = 20261201
_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first ``n`` outputs of SplitMix64 started at ``seed``."""
    out = np.empty(n, dtype=np.uint64)
    s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    tmp = np.empty(min(n, _CHUNK), dtype=np.uint64)
    with np.errstate(over="ignore"):
        for lo in range(0, n, _CHUNK):
            hi = min(n, lo + _CHUNK)
            z = out[lo:hi]
            t = tmp[: hi - lo]
            z[:] = np.arange(lo + 1, hi + 1, dtype=np.uint64)
            z *= _GOLD
            z += s
            np.right_shift(z, np.uint64(30), out=t)
            z ^= t
            z *= _M1
            np.right_shift(z, np.uint64(27), out=t)
            z ^= t
            z *= _M2
            np.right_shift(z, np.uint64(31), out=t)
            z ^= t
    return out


def _fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for b in text.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def sub_seed(config: str, tensor: str, base: int = BASE_SEED) -> int:
    return int(splitmix64(base ^ _fnv1a64(f"{config}/{tensor}"), 1)[0])


def uniform01(seed: int, n: int) -> np.ndarray:
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal_f32(seed: int, n: int, std: float) -> np.ndarray:
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m)
    r = np.sqrt(-2.0 * np.log(1.0 - u[0::2]))
    t = 2.0 * math.pi * u[1::2]
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    return (std * z[:n]).astype(np.float32)


def random_bytes(seed: int, n: int) -> np.ndarray:
    w = (n + 7) // 8
    return splitmix64(seed, w).view(np.uint8)[:n].copy()


def fp16_uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    return (lo + (hi - lo) * uniform01(seed, n)).astype(np.float16)


def int8_pm127(seed: int, n: int) -> np.ndarray:
    """int8 in [-127, 127] as (b mod 255) - 127 of random bytes b, as uint8 bytes."""
    b = random_bytes(seed, n)
    np.remainder(b, np.uint8(255), out=b)
    b += np.uint8(129)  # wraps: t + 129 mod 256 is the two's complement of t - 127
    return b


# ---------------------------------------------------------------------------
# block-format matrices


def quant_matrix(seed: int, qtype: int, rows: int, cols: int,
                 scale_lo: float = 0.005, scale_hi: float = 0.02) -> np.ndarray:
    """A [rows][cols] matrix in GGML block layout as raw bytes."""
    blk, bsz = F.BLOCK[qtype]
    nb = (cols + blk - 1) // blk
    nblocks = rows * nb
    out = np.empty((nblocks, bsz), dtype=np.uint8)
    if qtype == F.Q4_0:
        d = fp16_uniform(seed ^ 0x1, nblocks, scale_lo, scale_hi)
        out[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
        out[:, 2:18] = random_bytes(seed ^ 0x2, nblocks * 16).reshape(nblocks, 16)
    elif qtype == F.Q8_0:
        d = fp16_uniform(seed ^ 0x1, nblocks, scale_lo, scale_hi)
        out[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
        out[:, 2:34] = int8_pm127(seed ^ 0x2, nblocks * 32).reshape(nblocks, 32)
    elif qtype in (F.Q4_K, F.Q5_K):
        # Q5_K quants reach 31: half the scale range keeps the weights' spread near Q4_K's
        k = 0.5 if qtype == F.Q5_K else 1.0
        d = fp16_uniform(seed ^ 0x1, nblocks, k * scale_lo, k * scale_hi)
        dmin = fp16_uniform(seed ^ 0x3, nblocks, k * scale_lo, k * scale_hi)
        out[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
        out[:, 2:4] = dmin.view(np.uint8).reshape(nblocks, 2)
        out[:, 4:16] = random_bytes(seed ^ 0x4, nblocks * 12).reshape(nblocks, 12)
        q0 = 48 if qtype == F.Q5_K else 16
        out[:, q0:q0 + 128] = random_bytes(seed ^ 0x2, nblocks * 128).reshape(nblocks, 128)
        if qtype == F.Q5_K:
            out[:, 16:48] = random_bytes(seed ^ 0x5, nblocks * 32).reshape(nblocks, 32)
    elif qtype == F.Q6_K:
        # ql[128], qh[64], int8 scales[16] over the full range (sign and |sc| > 64 included), d
        out[:, 0:192] = random_bytes(seed ^ 0x2, nblocks * 192).reshape(nblocks, 192)
        out[:, 192:208] = random_bytes(seed ^ 0x4, nblocks * 16).reshape(nblocks, 16)
        d = fp16_uniform(seed ^ 0x1, nblocks, scale_lo / 16, scale_hi / 16)
        out[:, 208:210] = d.view(np.uint8).reshape(nblocks, 2)
    elif qtype == F.Q5_0:
        d = fp16_uniform(seed ^ 0x1, nblocks, scale_lo / 2, scale_hi / 2)
        out[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
        out[:, 2:22] = random_bytes(seed ^ 0x2, nblocks * 20).reshape(nblocks, 20)
    else:
        raise ValueError(f"unsupported expert weight type {qtype}")
    return out.reshape(-1)


# ---------------------------------------------------------------------------
# layer configurations


@dataclass(frozen=True)
class LayerConfig:
    name: str
    d_model: int
    n_experts: int
    top_k: int
    d_ff: int
    wtype: int
    d_ff_shared: int = 0
    down_wtype: int | None = None     # routed down type when it differs (Q4_K_M files: Q6_K / Q5_0 downs)
    sh_down_wtype: int | None = None  # shared down type (default: the routed down type)
    shared_gate: bool = False
    zipf_gamma: float = 0.0
    act: int = 0  # gated activation: 0 SiLU, 1 GELU-tanh (the reference's use_gelu)
    norms: bool = False  # ffn_norm and post_ffw_norm weights for the residual-stream form
    router_type: int = F.F32  # F16 / BF16: the router rows stored as half / bfloat16 bits
    rms_eps: float = 1e-5
    decode_tokens: tuple = field(default_factory=tuple)
    describe: str = ""

    @property
    def has_shared(self) -> bool:
        return self.d_ff_shared > 0

    @property
    def down_t(self) -> int:
        return self.wtype if self.down_wtype is None else self.down_wtype

    @property
    def sh_down_t(self) -> int:
        return self.down_t if self.sh_down_wtype is None else self.sh_down_wtype


CONFIGS = {
    "toy": LayerConfig("toy", 512, 8, 2, 1024, F.Q4_0, decode_tokens=(1,),
                       describe="Toy MoE FFN d512 E8 top-2 F1024 Q4_0"),
    # the toy layer with the gemma family's GELU-tanh gate (the reference's use_gelu)
    "toy_gelu": LayerConfig("toy_gelu", 512, 8, 2, 1024, F.Q4_0, act=1, decode_tokens=(1, 64),
                            describe="Toy MoE FFN d512 E8 top-2 F1024 Q4_0, GELU-tanh gate"),
    # a GELU-tanh layer with a sigmoid-gated shared expert: the routed experts take GELU, the shared expert
    # SiLU (the reference's shared-expert call never passes use_gelu)
    "toy_gelu_sh": LayerConfig("toy_gelu_sh", 512, 8, 2, 1024, F.Q4_0, d_ff_shared=1024, shared_gate=True, act=1,
                               decode_tokens=(1, 64),
                               describe="Toy MoE FFN d512 E8 top-2 F1024 Q4_0, GELU-tanh gate, shared 1024 "
                                        "(SiLU, sigmoid gate)"),
    # the toy layer in its residual-stream form: ffn_norm before, post_ffw_norm and the residual add after
    "toy_norm": LayerConfig("toy_norm", 512, 8, 2, 1024, F.Q4_0, norms=True, decode_tokens=(1, 64),
                            describe="Toy MoE FFN d512 E8 top-2 F1024 Q4_0 with ffn_norm / post_ffw_norm"),
    "qwen15moe": LayerConfig("qwen15moe", 2048, 60, 4, 1408, F.Q4_0, d_ff_shared=5632,
                             shared_gate=True, decode_tokens=(1, 64),
                             describe="Qwen1.5-MoE-A2.7B-shaped d2048 E60 top-4 F1408 Q4_0 + shared 5632 (sigmoid gate)"),
    "mixtral": LayerConfig("mixtral", 4096, 8, 2, 14336, F.Q4_K, decode_tokens=(1, 512, 2048),
                           describe="Mixtral-8x7B-shaped d4096 E8 top-2 F14336 Q4_K"),
    "qwen3moe": LayerConfig("qwen3moe", 2048, 128, 8, 768, F.Q8_0, zipf_gamma=0.75,
                            decode_tokens=(2048,),
                            describe="Qwen3-30B-A3B-shaped d2048 E128 top-8 F768 Q8_0, Zipf-skewed routing"),
    "dsv2lite": LayerConfig("dsv2lite", 2048, 64, 6, 1408, F.Q4_K, d_ff_shared=2816,
                            decode_tokens=(32,),
                            describe="DeepSeek-V2-Lite-shaped d2048 E64 top-6 F1408 Q4_K + 2x1408 shared"),
    # the mixed-type layers of real Q4_K_M files: Q6_K downs on the layers llama.cpp gives more bits,
    # Q5_0 where d_ff % 256 != 0 rules out the K-quants (its fallback for Q4_K), Q6_K shared down
    "mixtral_q6k": LayerConfig("mixtral_q6k", 4096, 8, 2, 14336, F.Q4_K, down_wtype=F.Q6_K,
                               decode_tokens=(1, 512, 2048),
                               describe="Mixtral-8x7B-shaped Q4_K_M layer: Q4_K gate/up, Q6_K down"),
    "dsv2lite_q50": LayerConfig("dsv2lite_q50", 2048, 64, 6, 1408, F.Q4_K, d_ff_shared=2816,
                                down_wtype=F.Q5_0, sh_down_wtype=F.Q6_K, decode_tokens=(1, 32, 512),
                                describe="DeepSeek-V2-Lite-shaped Q4_K_M layer: Q4_K gate/up, Q5_0 routed down "
                                         "(fp32 activations), Q6_K shared down"),
    # single-format toy layers: every kernel form of each type (Q5_0 gate/up takes fp32 x)
    "toy_q5k": LayerConfig("toy_q5k", 512, 8, 2, 1024, F.Q5_K, decode_tokens=(1, 2, 64, 512),
                           describe="Toy MoE FFN d512 E8 top-2 F1024 Q5_K"),
    "toy_q6k": LayerConfig("toy_q6k", 512, 8, 2, 1024, F.Q6_K, decode_tokens=(1, 2, 64, 512),
                           describe="Toy MoE FFN d512 E8 top-2 F1024 Q6_K"),
    "toy_q50": LayerConfig("toy_q50", 512, 8, 2, 1024, F.Q5_0, decode_tokens=(1, 2, 64, 512),
                           describe="Toy MoE FFN d512 E8 top-2 F1024 Q5_0 (fp32 activations throughout)"),
    # routers stored as F16 / BF16 (the reference's matmul_quant_f32 takes any router type): the toy
    # layer, and a 24-expert layer (split routers) with a sigmoid-gated shared expert whose fp32 gate
    # keeps vec_dot_f32's order beside the BF16 router rows
    "toy_f16r": LayerConfig("toy_f16r", 512, 8, 2, 1024, F.Q4_0, router_type=F.F16, decode_tokens=(1, 64),
                            describe="Toy MoE FFN d512 E8 top-2 F1024 Q4_0, F16 router"),
    "toy_bf16r_sh": LayerConfig("toy_bf16r_sh", 512, 24, 4, 512, F.Q4_K, d_ff_shared=512, shared_gate=True,
                                router_type=F.BF16, decode_tokens=(1, 64),
                                describe="d512 E24 top-4 F512 Q4_K + shared 512 (sigmoid gate), BF16 router"),
}


def zipf_bias(cfg: LayerConfig, seed: int = BASE_SEED) -> np.ndarray:
    """Per-expert router bias -1.1*gamma*ln(rank_e) with a seeded rank permutation."""
    keys = splitmix64(sub_seed(cfg.name, "zipf_rank", seed), cfg.n_experts)
    order = np.argsort(keys, kind="stable")
    rank = np.empty(cfg.n_experts, dtype=np.int64)
    rank[order] = np.arange(1, cfg.n_experts + 1)
    return np.array([-1.1 * cfg.zipf_gamma * math.log(float(r)) for r in rank], dtype=np.float32)


def to_f16_bits(v: np.ndarray) -> np.ndarray:
    """fp32 -> IEEE half bits, round to nearest even (numpy's conversion)."""
    return np.ascontiguousarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


def to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """fp32 -> bfloat16 bits, round to nearest even (fp32_to_bf16, src/quant.cpp:934-939; finite inputs)."""
    b = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


@dataclass
class LayerWeights:
    cfg: LayerConfig
    router: np.ndarray              # [E][d]: fp32, or uint16 half / bfloat16 bits (cfg.router_type)
    router_bias: np.ndarray | None  # fp32 [E]
    gate: np.ndarray                # bytes, [E][F] rows of d
    up: np.ndarray
    down: np.ndarray                # bytes, [E][d] rows of F
    sh_gate: np.ndarray | None = None
    sh_up: np.ndarray | None = None
    sh_down: np.ndarray | None = None
    sh_gate_inp: np.ndarray | None = None  # fp32 [d]
    ffn_norm: np.ndarray | None = None      # fp32 [d]
    post_ffw_norm: np.ndarray | None = None  # fp32 [d]

    @property
    def types(self):
        t = self.cfg.wtype
        return t, t, self.cfg.down_t

    @property
    def sh_types(self):
        t = self.cfg.wtype
        return t, t, self.cfg.sh_down_t


def make_layer(cfg: LayerConfig, seed: int = BASE_SEED) -> LayerWeights:
    d, E, Fd = cfg.d_model, cfg.n_experts, cfg.d_ff
    s = lambda name: sub_seed(cfg.name, name, seed)  # noqa: E731
    router = normal_f32(s("router"), E * d, 0.02).reshape(E, d)
    if cfg.router_type == F.F16:
        router = to_f16_bits(router)
    elif cfg.router_type == F.BF16:
        router = to_bf16_bits(router)
    bias = zipf_bias(cfg, seed) if cfg.zipf_gamma > 0 else None
    gate = quant_matrix(s("gate_exps"), cfg.wtype, E * Fd, d)
    up = quant_matrix(s("up_exps"), cfg.wtype, E * Fd, d)
    down = quant_matrix(s("down_exps"), cfg.down_t, E * d, Fd)
    lw = LayerWeights(cfg, router, bias, gate, up, down)
    if cfg.has_shared:
        Fs = cfg.d_ff_shared
        lw.sh_gate = quant_matrix(s("gate_shexp"), cfg.wtype, Fs, d)
        lw.sh_up = quant_matrix(s("up_shexp"), cfg.wtype, Fs, d)
        lw.sh_down = quant_matrix(s("down_shexp"), cfg.sh_down_t, d, Fs)
        if cfg.shared_gate:
            lw.sh_gate_inp = normal_f32(s("gate_inp_shexp"), d, 0.02)
    if cfg.norms:  # RMSNorm weights around 1
        lw.ffn_norm = (1.0 + normal_f32(s("ffn_norm"), d, 0.1)).astype(np.float32)
        lw.post_ffw_norm = (1.0 + normal_f32(s("post_ffw_norm"), d, 0.1)).astype(np.float32)
    return lw


def make_tokens(cfg: LayerConfig, n: int, seed: int = BASE_SEED) -> np.ndarray:
    """``n`` post-norm activations ~N(0,1), fp32 [n][d]."""
    return normal_f32(sub_seed(cfg.name, f"x@{n}", seed), n * cfg.d_model, 1.0).reshape(n, cfg.d_model)


def expert_bytes(cfg: LayerConfig) -> int:
    """gate+up+down bytes of one routed expert."""
    t = cfg.wtype
    return 2 * F.matrix_bytes(t, cfg.d_ff, cfg.d_model) + F.matrix_bytes(cfg.down_t, cfg.d_model, cfg.d_ff)


def shared_bytes(cfg: LayerConfig) -> int:
    if not cfg.has_shared:
        return 0
    t = cfg.wtype
    Fs = cfg.d_ff_shared
    return 2 * F.matrix_bytes(t, Fs, cfg.d_model) + F.matrix_bytes(cfg.sh_down_t, cfg.d_model, Fs)
