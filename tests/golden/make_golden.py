"""Write the golden vectors in tests/golden/*.npz.

The expected values come from the reference engine's own arithmetic: its
src/quant.cpp and src/tier.cpp compiled in place by ``make -C oracle ref``
(oracle/_ref/libjxref.so), driven through oracle/ref_driver.cpp, which replays
the MoE block of src/transformer.cpp:2589-2757.  Inputs are the seeded
synthetics of jxai_amd.synth; each fixture stores SHA-256 digests of its inputs
so a drift in the generator is reported instead of silently compared.

Run in a container that has the reference tree:
    python tests/golden/make_golden.py            # AVX2 dot order (MOE_AVX512=0)
The AVX-512 variant of the toy fixture is produced by a child process, since
the reference caches MOE_AVX512 on its first dot call.
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from jxai_amd import formats as F  # noqa: E402
from jxai_amd import synth  # noqa: E402
from oracle.oracle import Oracle, build  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# (config, n tokens, tokens whose full output row is stored, or the tile granularity the rows must cover:
# ("tiles", routed pairs per tile, shared-expert tokens per tile) -- 32 where the library takes the
# matrix-core GEMMs (their 32-pair MFMA tiles), 16 where it takes the 16-token matrix-core GEMV)
CASES = [
    ("toy", 1, [0]),
    ("qwen15moe", 1, [0]),
    ("qwen15moe", 64, ("tiles", 16, 32)),
    ("mixtral", 1, [0]),
    ("mixtral", 512, ("tiles", 32, 0)),
    ("mixtral", 2048, ("tiles", 32, 0)),
    ("qwen3moe", 2048, ("tiles", 32, 0)),
    ("dsv2lite", 32, ("tiles", 16, 16)),
    ("toy_gelu", 1, [0]),
    ("toy_gelu", 64, ("tiles", 32, 0)),
]
# the five- and six-bit formats (Q4_K_M mixes; whole toy layers of each type, every row stored)
F3_CASES = [
    ("toy_q5k", 1, [0]),
    ("toy_q5k", 64, list(range(64))),
    ("toy_q6k", 1, [0]),
    ("toy_q6k", 64, list(range(64))),
    ("toy_q50", 1, [0]),
    ("toy_q50", 64, list(range(64))),
    ("mixtral_q6k", 1, [0]),
    ("mixtral_q6k", 512, ("tiles", 32, 0)),
    ("dsv2lite_q50", 1, [0]),
    ("dsv2lite_q50", 32, ("tiles", 16, 16)),
]
# a GELU layer with a sigmoid-gated shared expert (GELU on the routed experts only, SiLU on the shared one):
# 64 tokens take the routed GEMMs (32-pair tiles) and the shared expert's 16-token GEMV
GELU_SH_CASES = [
    ("toy_gelu_sh", 1, [0]),
    ("toy_gelu_sh", 64, ("tiles", 32, 16)),
]
# the residual-stream form (rms_norm before, post_ffw_norm and the residual add after the block)
RESID_CASES = [
    ("toy_norm", 1, [0]),
    ("toy_norm", 64, ("tiles", 32, 0)),
]

# F16 / BF16 routers (the router GEMV through matmul_quant_f32 of the router's own type)
ROUTER16_CASES = [
    ("toy_f16r", 1, [0]),
    ("toy_f16r", 64, list(range(64))),
    ("toy_bf16r_sh", 1, [0]),
    ("toy_bf16r_sh", 64, list(range(64))),
]


def covering_rows(ids: np.ndarray, n_experts: int, g_routed: int, g_shared: int) -> list[int]:
    """Tokens whose output rows together touch every tile of the grouped kernels.

    The dispatch is a stable counting sort, so expert e's pairs are its tokens in token order and the
    j-th of them sits in tile j // g_routed of that expert; the shared expert's tile of token t is
    t // g_shared.  Greedy set cover over those (expert, tile) units, seeded with the first and last
    token: every tile, each expert's last partial one included, holds at least one checked row."""
    n, k = ids.shape
    seen = np.zeros(n_experts, np.int64)
    units = [set() for _ in range(n)]
    for t in range(n):
        for s in range(k):
            e = int(ids[t, s])
            units[t].add((e, int(seen[e]) // g_routed))
            seen[e] += 1
        if g_shared:
            units[t].add((-1, t // g_shared))
    want = set().union(*units)
    rows = sorted({0, n - 1})
    covered = set().union(*(units[t] for t in rows))
    while covered != want:
        best = max(range(n), key=lambda t: (len(units[t] - covered), -t))
        rows.append(best)
        covered |= units[best]
    return sorted(rows)


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def layer_digest(lw) -> str:
    return digest(lw.router, lw.router_bias, lw.gate, lw.up, lw.down,
                  lw.sh_gate, lw.sh_up, lw.sh_down, lw.sh_gate_inp)


def make_case(ref: Oracle, name: str, n: int, rows, tag: str = "", residual: bool = False) -> str:
    cfg = synth.CONFIGS[name]
    lw = synth.make_layer(cfg)
    x = synth.make_tokens(cfg, n)
    # the router sees rms_norm(x) in the residual form (restated from transformer.cpp:67-73 on the
    # reference build's own vec_dot_f32)
    xr = x
    if residual:
        xr = np.empty_like(x)
        for t in range(n):
            ss = np.float32(ref.vec_dot_f32(x[t], x[t]))
            inv = np.float32(1.0) / np.sqrt(ss / np.float32(cfg.d_model) + np.float32(cfg.rms_eps))
            xr[t] = x[t] * inv * lw.ffn_norm
    ids_all = np.zeros((n, cfg.top_k), np.int32)
    w_all = np.zeros((n, cfg.top_k), np.float32)
    lg_all = np.zeros((n, cfg.n_experts), np.float32)
    for t in range(n):
        logits = ref.matmul_quant_f32(cfg.router_type, lw.router.view(np.uint8).reshape(-1), xr[t],
                                      cfg.n_experts, cfg.d_model)
        if lw.router_bias is not None:
            logits = (logits + lw.router_bias).astype(np.float32)
        i, p, _ = ref.select_experts(logits, cfg.top_k)
        ids_all[t], w_all[t], lg_all[t] = i, p, logits
    if isinstance(rows, tuple):  # ("tiles", routed, shared): rows covering every tile of the dispatch
        rows = covering_rows(ids_all, cfg.n_experts, rows[1], rows[2])
    # full MoE-block outputs for `rows`
    out, ids_r, w_r, lg_r = ref.moe_forward(lw, x, np.asarray(rows, dtype=np.int32), residual=residual)
    assert np.array_equal(ids_all[rows], ids_r) and np.array_equal(w_all[rows].view(np.uint32), w_r.view(np.uint32))
    counts = np.bincount(ids_all.reshape(-1), minlength=cfg.n_experts).astype(np.int32)
    path = os.path.join(OUT, f"{name}_n{n}{tag}.npz")
    np.savez_compressed(
        path,
        config=name, n=n, rows=np.asarray(rows, np.int32), residual=residual,
        out=out, topk_ids=ids_all, topk_w=w_all, logits_rows=lg_all[rows], counts=counts,
        layer_sha256=layer_digest(lw), x_sha256=digest(x),
    )
    return path


def make_units(ref: Oracle) -> str:
    """Function-level vectors: fp16 truncation, Q8_0 quantization, block dots."""
    rng_f = synth.normal_f32(synth.sub_seed("units", "f"), 4096, 3.0)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05,
                        6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 1e-12, np.inf, -np.inf,
                        0.33333334, 2.0 / 3.0, 0.1, 1.0009765625, 1.00048828125], np.float32)
    f = np.concatenate([special, rng_f, rng_f * np.float32(1e-5)]).astype(np.float32)
    h = np.array([ref.fp32_to_fp16(float(v)) for v in f], np.uint16)

    # Q8_0 activations: random blocks, a zero block, exact .5 ties, one huge block
    xs = synth.normal_f32(synth.sub_seed("units", "xq"), 32 * 64, 1.0)
    xs[0:32] = 0.0
    xs[32:64] = np.arange(32, dtype=np.float32) - 15.5          # amax 15.5 -> ties
    xs[64:96] = np.linspace(-127.0, 127.0, 32, dtype=np.float32)  # q == x exactly
    xs[96:128] = xs[96:128] * np.float32(1e4)
    xq = ref.quantize_row_q8_0(xs)

    dots = {}
    for qt, cols in ((F.Q4_0, 2048), (F.Q8_0, 2048), (F.Q4_K, 4096), (F.Q4_K, 896)):
        rows = 16
        w = synth.quant_matrix(synth.sub_seed("units", f"w{qt}_{cols}"), qt, rows, cols)
        y = synth.normal_f32(synth.sub_seed("units", f"y{qt}_{cols}"), cols, 1.0)
        out_q8 = ref.matmul_quant_f32(qt, w, y, rows, cols)
        yq = ref.quantize_row_q8_0(np.concatenate([y, np.zeros((-cols) % 256, np.float32)]))
        rb = F.row_bytes(qt, cols)
        direct = np.array([ref.vec_dot_q8(qt, w[r * rb:(r + 1) * rb], yq, cols) for r in range(rows)], np.float32)
        dots[f"{qt}_{cols}"] = (w, y, out_q8, direct)
    # Q4_K fp32-activation dot with a partial super-block (DeepSeek down rows)
    w14 = synth.quant_matrix(synth.sub_seed("units", "w14"), F.Q4_K, 16, 1408)
    y14 = synth.normal_f32(synth.sub_seed("units", "y14"), 1408, 1.0)
    o14 = ref.matmul_quant_f32(F.Q4_K, w14, y14, 16, 1408)
    sw_g = synth.quant_matrix(synth.sub_seed("units", "swg"), F.Q4_0, 64, 512)
    sw_u = synth.quant_matrix(synth.sub_seed("units", "swu"), F.Q4_0, 64, 512)
    sw_x = synth.normal_f32(synth.sub_seed("units", "swx"), 512, 1.0)
    sw_o = ref.matmul_swiglu_quant_f32(F.Q4_0, sw_g, F.Q4_0, sw_u, sw_x, 64, 512)
    path = os.path.join(OUT, "units.npz")
    kw = {}
    for key, (w, y, o, dd) in dots.items():
        kw[f"dot_w_{key}"], kw[f"dot_y_{key}"], kw[f"dot_out_{key}"], kw[f"dot_direct_{key}"] = w, y, o, dd
    np.savez_compressed(path, f=f, h=h, xs=xs, xq=xq, w14=w14, y14=y14, o14=o14,
                        sw_g=sw_g, sw_u=sw_u, sw_x=sw_x, sw_o=sw_o, **kw)
    return path


def make_units_f3(ref: Oracle) -> str:
    """Function-level vectors of the five- and six-bit formats (Q5_0, Q5_K, Q6_K) and of the fp32-activation
    dots of every expert format: dequantize_row, vec_dot_quant_f32, the Q8_0-activation dots and the two
    matmul dispatchers over both activation forms."""
    kw = {}
    for qt in (F.Q5_0, F.Q5_K, F.Q6_K):  # dequantize_row, two rows (all scale bytes / fifth bits exercised)
        cols = 512
        w = synth.quant_matrix(synth.sub_seed("units_f3", f"deq{qt}"), qt, 2, cols)
        kw[f"deq_w_{qt}"] = w
        kw[f"deq_o_{qt}"] = np.concatenate([ref.dequantize_row(qt, w[r * F.row_bytes(qt, cols):], cols) for r in range(2)])
    # matmul_quant_f32: K-quants at 2048 (Q8_0 activations) and 896 / 1408 (fp32, partial super-block);
    # Q5_0 (fp32 always); Q4_0 / Q8_0 with 4 rows (fp32: matmul_quant_f32 quantizes x only from 8 rows)
    for qt, rows, cols in ((F.Q5_K, 16, 2048), (F.Q6_K, 16, 2048), (F.Q5_K, 16, 896), (F.Q6_K, 16, 1408),
                           (F.Q5_0, 16, 1408), (F.Q4_0, 4, 512), (F.Q8_0, 4, 512), (F.Q4_K, 4, 512)):
        key = f"{qt}_{rows}_{cols}"
        w = synth.quant_matrix(synth.sub_seed("units_f3", f"w{key}"), qt, rows, cols)
        y = synth.normal_f32(synth.sub_seed("units_f3", f"y{key}"), cols, 1.0)
        kw[f"mm_w_{key}"], kw[f"mm_y_{key}"] = w, y
        kw[f"mm_o_{key}"] = ref.matmul_quant_f32(qt, w, y, rows, cols)
        rb = F.row_bytes(qt, cols)
        kw[f"f32_o_{key}"] = np.array([ref.vec_dot_quant_f32(qt, w[r * rb:(r + 1) * rb], y) for r in range(rows)],
                                      np.float32)
        if qt in (F.Q5_K, F.Q6_K):  # the Q8_0-activation block dot directly, partial super-block included
            yq = ref.quantize_row_q8_0(np.concatenate([y, np.zeros((-cols) % 256, np.float32)]))
            kw[f"q8_o_{key}"] = np.array([ref.vec_dot_q8(qt, w[r * rb:(r + 1) * rb], yq, cols) for r in range(rows)],
                                         np.float32)
    # matmul_swiglu_quant_f32 with fp32 x (Q5_0) and Q8_0 x (Q6_K, Q5_K)
    for qt in (F.Q5_0, F.Q6_K, F.Q5_K):
        g = synth.quant_matrix(synth.sub_seed("units_f3", f"swg{qt}"), qt, 64, 512)
        u = synth.quant_matrix(synth.sub_seed("units_f3", f"swu{qt}"), qt, 64, 512)
        x = synth.normal_f32(synth.sub_seed("units_f3", f"swx{qt}"), 512, 1.0)
        kw[f"sw_g_{qt}"], kw[f"sw_u_{qt}"], kw[f"sw_x_{qt}"] = g, u, x
        kw[f"sw_o_{qt}"] = ref.matmul_swiglu_quant_f32(qt, g, qt, u, x, 64, 512)
    path = os.path.join(OUT, "units_f3.npz")
    np.savez_compressed(path, **kw)
    return path


def make_units_router16(ref: Oracle) -> str:
    """vec_dot_f16_f32 / vec_dot_bf16_f32 (src/quant.cpp:3015-3055) through vec_dot_quant_f32, with and
    without a scalar tail (k % 8 != 0), and matmul_quant_f32 over an E x d router of each type."""
    kw = {}
    for t in (F.F16, F.BF16):
        for k in (37, 512, 4101):
            v = synth.normal_f32(synth.sub_seed("units_r16", f"w{t}_{k}"), k, 0.05)
            w = synth.to_f16_bits(v) if t == F.F16 else synth.to_bf16_bits(v)
            y = synth.normal_f32(synth.sub_seed("units_r16", f"y{t}_{k}"), k, 1.0)
            kw[f"dot_w_{t}_{k}"], kw[f"dot_y_{t}_{k}"] = w, y
            kw[f"dot_o_{t}_{k}"] = np.float32(ref.vec_dot_quant_f32(t, w.view(np.uint8), y))
        E, d = 24, 2048
        v = synth.normal_f32(synth.sub_seed("units_r16", f"router{t}"), E * d, 0.02)
        w = synth.to_f16_bits(v) if t == F.F16 else synth.to_bf16_bits(v)
        x = synth.normal_f32(synth.sub_seed("units_r16", f"x{t}"), d, 1.0)
        kw[f"mm_w_{t}"], kw[f"mm_x_{t}"] = w, x
        kw[f"mm_o_{t}"] = ref.matmul_quant_f32(t, w.view(np.uint8), x, E, d)
    path = os.path.join(OUT, "units_router16.npz")
    np.savez_compressed(path, **kw)
    return path


TOY_GGUF = "/root/reference/models/qwen_run.gguf"


def make_gguf_case(ref: Oracle) -> str:
    """Layer 0 of the reference's toy model file (models/qwen_run.gguf, written by its
    src/model_forge.cpp:135-339): the layer's tensors as stored in the file (router F32 [128, 8],
    Q4_0 experts [128, 128, 8], ffn_norm) with their metadata, seeded tokens, and the reference
    build's MoE block on them -- the fixture the GPU test rebuilds a GGUF file from."""
    from jxai_amd.gguf import GGUFFile
    f = GGUFFile(TOY_GGUF)
    names = ["blk.0.ffn_gate_inp.weight", "blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
             "blk.0.ffn_down_exps.weight", "blk.0.ffn_norm.weight"]
    t = f.tensors()
    kw = {}
    for i, nm in enumerate(names):
        kw[f"t{i}_name"] = nm
        kw[f"t{i}_dims"] = np.array(t[nm]["dims"][: t[nm]["n_dims"]], np.int64)
        kw[f"t{i}_type"] = t[nm]["type"]
        kw[f"t{i}_bytes"] = f.tensor_bytes(nm)
    arch = f.get_str("general.architecture")
    meta = {"arch": arch, "top_k": f.get_u32(f"{arch}.expert_used_count"),
            "n_experts": f.get_u32(f"{arch}.expert_count"),
            "eps": f.get_f32(f"{arch}.attention.layer_norm_rms_epsilon")}
    d, E, Fd = 128, 8, 128
    cfg = synth.LayerConfig("qwen_run_l0", d, E, meta["top_k"], Fd, F.Q4_0)
    lw = synth.LayerWeights(cfg, kw["t0_bytes"].view(np.float32).reshape(E, d).copy(), None, kw["t1_bytes"],
                            kw["t2_bytes"], kw["t3_bytes"])
    n = 64
    x = synth.make_tokens(cfg, n, seed=5)
    out, ids, w, lg = ref.moe_forward(lw, x)
    f.close()
    path = os.path.join(OUT, "qwen_run_layer0.npz")
    np.savez_compressed(path, n_tensors=len(names), arch=arch, top_k=meta["top_k"], n_experts=meta["n_experts"],
                        eps=np.float32(meta["eps"]), x=x, out=out, topk_ids=ids, topk_w=w, logits=lg,
                        file_sha256=hashlib.sha256(open(TOY_GGUF, "rb").read()).hexdigest(), **kw)
    return path


def main() -> None:
    build(ref=True)
    if "--gguf" in sys.argv:  # only the toy-model fixture
        print(make_gguf_case(Oracle("reference", avx512=False)))
        return
    if "--f3" in sys.argv:  # only the five- and six-bit format fixtures
        ref = Oracle("reference", avx512=False)
        print(make_units_f3(ref))
        for name, n, rows in F3_CASES:
            print(make_case(ref, name, n, rows))
        return
    if "--router16" in sys.argv:  # only the F16 / BF16 router fixtures
        ref = Oracle("reference", avx512=False)
        print(make_units_router16(ref))
        for name, n, rows in ROUTER16_CASES:
            print(make_case(ref, name, n, rows))
        return
    if "--resid" in sys.argv:  # only the residual-stream cases
        ref = Oracle("reference", avx512=False)
        for name, n, rows in RESID_CASES:
            print(make_case(ref, name, n, rows, tag="_resid", residual=True))
        return
    if "--gelu-sh" in sys.argv:  # only the GELU + shared-expert cases
        ref = Oracle("reference", avx512=False)
        for name, n, rows in GELU_SH_CASES:
            print(make_case(ref, name, n, rows))
        return
    if "--avx512-child" in sys.argv:
        ref = Oracle("reference", avx512=True)
        print(make_case(ref, "toy", 1, [0], tag="_avx512"))
        print(make_case(ref, "qwen3moe", 2048, [0, 5], tag="_avx512"))
        return
    ref = Oracle("reference", avx512=False)
    print(make_units(ref))
    print(make_gguf_case(ref))
    for name, n, rows in CASES:
        print(make_case(ref, name, n, rows))
    for name, n, rows in GELU_SH_CASES:
        print(make_case(ref, name, n, rows))
    for name, n, rows in RESID_CASES:
        print(make_case(ref, name, n, rows, tag="_resid", residual=True))
    print(make_units_f3(ref))
    for name, n, rows in F3_CASES:
        print(make_case(ref, name, n, rows))
    print(make_units_router16(ref))
    for name, n, rows in ROUTER16_CASES:
        print(make_case(ref, name, n, rows))
    subprocess.run([sys.executable, os.path.abspath(__file__), "--avx512-child"], check=True)


if __name__ == "__main__":
    main()
