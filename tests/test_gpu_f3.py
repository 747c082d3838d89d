"""GPU parity of the five- and six-bit formats (Q5_0, Q5_K, Q6_K) against the oracle and the golden vectors.

The layers mix types as llama.cpp's Q4_K_M files do: Q6_K downs on the layers that get more bits, Q5_0
where a K-quant cannot hold a row (d_ff % 256 != 0; fp32 activations, as the reference's
vec_dot_q5_0_f32), a Q6_K shared down; plus single-type toy layers that run every kernel form of each type
(Q5_0 gate/up over fp32 x, Q6_K gate/up on the GEMVs at every token count).  Bar as in test_gpu.py:
routing bit-exact, outputs within 1e-3 relative per token.
"""
import os

import numpy as np
import pytest

from jxai_amd import formats as F
from jxai_amd import synth
from tests.conftest import GOLDEN
from tests.test_gpu import REL_TOL, rel_err, say

pytestmark = pytest.mark.gpu

_LAYERS = {}

EXTRA = {
    # Q5_K gate/up and down with a sigmoid-gated shared expert whose down is Q6_K
    "q5k_shared": synth.LayerConfig("q5k_shared", 512, 8, 2, 768, F.Q5_K, d_ff_shared=512, shared_gate=True,
                                    sh_down_wtype=F.Q6_K),
    # fp32 x for a K-quant gate/up (d_model % 256 != 0) and a Q5_0 shared expert
    "kq_f32x": synth.LayerConfig("kq_f32x", 384, 8, 2, 512, F.Q6_K, d_ff_shared=256, down_wtype=F.Q5_K,
                                 sh_down_wtype=F.Q5_0),
    # Q6_K down projection with the GELU gate; d_ff 1408 (fp32 activations, partial super-block)
    "q6k_f32h": synth.LayerConfig("q6k_f32h", 512, 8, 2, 1408, F.Q4_K, down_wtype=F.Q6_K, act=1),
}


@pytest.fixture(scope="module")
def moe():
    from jxai_amd import moe as M
    M.init(0)
    return M


def layer(name):
    if name not in _LAYERS:
        cfg = synth.CONFIGS[name] if name in synth.CONFIGS else EXTRA[name]
        _LAYERS.clear()
        _LAYERS[name] = (cfg, synth.make_layer(cfg))
    return _LAYERS[name]


F3_GOLDEN = ["toy_q5k_n1", "toy_q5k_n64", "toy_q6k_n1", "toy_q6k_n64", "toy_q50_n1", "toy_q50_n64",
             "mixtral_q6k_n1", "mixtral_q6k_n512", "dsv2lite_q50_n1", "dsv2lite_q50_n32"]


@pytest.mark.parametrize("case", F3_GOLDEN)
def test_layer_vs_golden_f3(moe, case):
    z = np.load(os.path.join(GOLDEN, case + ".npz"))
    name, n = str(z["config"]), int(z["n"])
    say(f"layer {case}: building")
    cfg, lw = layer(name)
    x = synth.make_tokens(cfg, n)
    L = moe.MoELayer.from_weights(lw)
    say(f"layer {case}: forward")
    out, ids, w, counts = L.forward(x)
    assert np.array_equal(ids, z["topk_ids"]), "routing differs"
    assert np.array_equal(counts, z["counts"])
    np.testing.assert_allclose(w, z["topk_w"], rtol=2e-6, atol=0)
    err = rel_err(out[z["rows"]], z["out"])
    say(f"layer {case}: max rel err {err:.2e} over {len(z['rows'])} rows")
    assert err <= REL_TOL
    L.close()


# every kernel form: one token (folded combine on top-2 layers), two tokens, groups of 4, the 16-token
# matrix-core GEMV, the GEMMs (Q6_K / Q5_0 gate/up staying on the GEMVs), and both forced regimes
F3_REGIMES = [("toy_q5k", n, r) for n, r in ((1, None), (2, None), (3, None), (24, None), (40, "gemv"),
                                             (300, None), (300, "gemv"), (8, "mfma"))] + \
             [("toy_q6k", n, r) for n, r in ((1, None), (2, None), (3, None), (24, None), (40, "gemv"),
                                             (300, None), (8, "mfma"))] + \
             [("toy_q50", n, r) for n, r in ((1, None), (2, None), (3, None), (24, None), (300, None),
                                             (300, "gemv"), (8, "mfma"))] + \
             [("mixtral_q6k", 1, None), ("mixtral_q6k", 2, None), ("mixtral_q6k", 32, None),
              ("mixtral_q6k", 64, "mfma"), ("dsv2lite_q50", 1, None), ("dsv2lite_q50", 2, None),
              ("dsv2lite_q50", 7, "gemv"), ("dsv2lite_q50", 64, None), ("dsv2lite_q50", 300, None),
              ("q5k_shared", 1, None), ("q5k_shared", 3, None), ("q5k_shared", 100, None), ("q5k_shared", 200, "gemv"),
              ("kq_f32x", 1, None), ("kq_f32x", 2, None), ("kq_f32x", 5, None), ("kq_f32x", 100, None),
              ("q6k_f32h", 1, None), ("q6k_f32h", 2, None), ("q6k_f32h", 20, "gemv"), ("q6k_f32h", 200, None)]


@pytest.mark.parametrize("name,n,regime", F3_REGIMES)
def test_layer_regimes_vs_oracle_f3(moe, port, name, n, regime):
    say(f"{name} n={n} regime={regime}")
    cfg, lw = layer(name)
    x = synth.make_tokens(cfg, n, seed=7)
    L = moe.MoELayer.from_weights(lw)
    out, ids, w, counts = L.forward(x, regime=regime)
    lg_o, ids_o, w_o = port.route(lw, x)
    assert np.array_equal(ids, ids_o)
    assert np.array_equal(counts, np.bincount(ids_o.reshape(-1), minlength=cfg.n_experts))
    np.testing.assert_allclose(w, w_o, rtol=2e-6, atol=0)
    sel = np.unique(np.linspace(0, n - 1, min(n, 6)).astype(np.int32))
    want = port.moe_forward(lw, x, sel)[0]
    err = rel_err(out[sel], want)
    say(f"{name} n={n} regime={regime}: max rel err {err:.2e}")
    assert err <= REL_TOL
    L.close()


def test_q6k_extreme_scales(moe, port):
    """Q6_K down rows whose sub-block scales are all -128 or 127 with quants at 0 or 63: sc * (q - 32) up to
    4096, past fp16's exact integers (the down GEMM's one rounding, 2^-12 relative), in both regimes."""
    cfg = synth.LayerConfig("q6k_ext", 512, 4, 2, 1024, F.Q4_K, down_wtype=F.Q6_K)
    lw = synth.make_layer(cfg)
    dn = lw.down.reshape(-1, 210)
    dn[:, 192:208] = np.where(np.arange(16) % 2, 0x80, 0x7F).astype(np.uint8)
    dn[0::3, 0:192] = 0xFF
    dn[1::3, 0:192] = 0x00
    lw.down = dn.reshape(-1)
    for n, regime in ((1, None), (64, "gemv"), (256, "mfma")):
        x = synth.make_tokens(cfg, n, seed=3)
        L = moe.MoELayer.from_weights(lw)
        out = L.forward(x, regime=regime)[0]
        L.close()
        sel = np.unique(np.linspace(0, n - 1, min(n, 6)).astype(np.int32))
        err = rel_err(out[sel], port.moe_forward(lw, x, sel)[0])
        say(f"q6k extremes n={n} {regime}: max rel err {err:.2e}")
        assert err <= REL_TOL


# ------------------------------------------------------------------ the drop-ins
@pytest.mark.parametrize("qt,rows,cols", [(F.Q5_K, 512, 2048), (F.Q6_K, 512, 4096), (F.Q6_K, 256, 1408),
                                          (F.Q5_K, 256, 896), (F.Q5_0, 512, 1408), (F.Q5_0, 1000, 896),
                                          (F.Q4_0, 4, 512), (F.Q8_0, 5, 768), (F.Q4_K, 3, 512), (F.Q6_K, 7, 2048)])
def test_matmul_quant_f32_f3(moe, port, qt, rows, cols):
    """Q8_0 activations from 8 rows where the type allows, fp32 otherwise (Q5_0 always; fewer than 8 rows;
    K-quants with cols % 256 != 0, partial super-block)."""
    say(f"matmul_quant_f32 type={qt} {rows}x{cols}")
    W = synth.quant_matrix(synth.sub_seed("gpu_f3", f"mm{qt}_{rows}_{cols}"), qt, rows, cols)
    x = synth.normal_f32(synth.sub_seed("gpu_f3", f"mx{cols}"), cols, 1.0)
    got = moe.matmul_quant_f32(qt, W, x, rows, cols)
    want = port.matmul_quant_f32(qt, W, x, rows, cols)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("use_gelu", [False, True])
@pytest.mark.parametrize("qt,rows,cols", [(F.Q5_0, 1024, 896), (F.Q6_K, 512, 2048), (F.Q5_K, 768, 2048),
                                          (F.Q6_K, 256, 1408)])
def test_matmul_swiglu_quant_f32_f3(moe, port, qt, rows, cols, use_gelu):
    say(f"matmul_swiglu_quant_f32 type={qt} {rows}x{cols} gelu={use_gelu}")
    Wg = synth.quant_matrix(synth.sub_seed("gpu_f3", f"g{qt}_{cols}"), qt, rows, cols)
    Wu = synth.quant_matrix(synth.sub_seed("gpu_f3", f"u{qt}_{cols}"), qt, rows, cols)
    x = synth.normal_f32(synth.sub_seed("gpu_f3", f"sx{cols}"), cols, 1.0)
    got = moe.matmul_swiglu_quant_f32(qt, Wg, qt, Wu, x, rows, cols, use_gelu=use_gelu)
    want = port.matmul_swiglu_quant_f32(qt, Wg, qt, Wu, x, rows, cols, use_gelu=use_gelu)
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()
