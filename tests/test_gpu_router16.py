"""GPU parity of F16 / BF16 routers (the reference's router GEMV is matmul_quant_f32 of the router
tensor's own type, src/transformer.cpp:2591, so F16 / BF16 rows take vec_dot_{f16,bf16}_f32's 8-lane
order, src/quant.cpp:3015-3055, while the shared expert's fp32 gate keeps vec_dot_f32's).

Every router kernel is reached: the one-block few-token router (1-2 tokens), the row-per-block one (up
to 4 tokens), the many-token router with and without row splits (24 experts + the shared gate: 25
rows), from one token per block to four.  Bar: router logits bit-exact against the reference build's
golden vectors and the oracle, routing identical, outputs within 1e-3 relative per token.
"""
import os

import numpy as np
import pytest

from jxai_amd import synth
from tests.conftest import GOLDEN
from tests.test_gpu import REL_TOL, rel_err, say

pytestmark = pytest.mark.gpu

_LAYERS = {}


@pytest.fixture(scope="module")
def moe():
    from jxai_amd import moe as M
    M.init(0)
    return M


def layer(name):
    if name not in _LAYERS:
        _LAYERS.clear()
        cfg = synth.CONFIGS[name]
        _LAYERS[name] = (cfg, synth.make_layer(cfg))
    return _LAYERS[name]


@pytest.mark.parametrize("case", ["toy_f16r_n1", "toy_f16r_n64", "toy_bf16r_sh_n1", "toy_bf16r_sh_n64"])
def test_layer_vs_golden_router16(moe, case):
    z = np.load(os.path.join(GOLDEN, case + ".npz"))
    name, n = str(z["config"]), int(z["n"])
    say(f"layer {case}: building")
    cfg, lw = layer(name)
    x = synth.make_tokens(cfg, n)
    L = moe.MoELayer.from_weights(lw)
    say(f"layer {case}: forward")
    out, ids, w, counts = L.forward(x)
    lg = L.last_logits(n)
    assert np.array_equal(lg[z["rows"]].view(np.uint32), z["logits_rows"].view(np.uint32)), "logits not bit-exact"
    assert np.array_equal(ids, z["topk_ids"]), "routing differs"
    assert np.array_equal(counts, z["counts"])
    np.testing.assert_allclose(w, z["topk_w"], rtol=2e-6, atol=0)
    err = rel_err(out[z["rows"]], z["out"])
    say(f"layer {case}: max rel err {err:.2e}")
    assert err <= REL_TOL
    L.close()


@pytest.mark.parametrize("name,n", [("toy_f16r", n) for n in (1, 2, 3, 24, 300, 700)] +
                                   [("toy_bf16r_sh", n) for n in (1, 2, 3, 24, 300, 700)])
def test_router16_logits_vs_oracle(moe, port, name, n):
    say(f"{name} n={n}")
    cfg, lw = layer(name)
    x = synth.make_tokens(cfg, n, seed=9)
    L = moe.MoELayer.from_weights(lw)
    out, ids, w, counts = L.forward(x)
    lg = L.last_logits(n)
    lg_o, ids_o, w_o = port.route(lw, x)
    assert np.array_equal(lg.view(np.uint32), lg_o.view(np.uint32)), "logits not bit-exact"
    assert np.array_equal(ids, ids_o)
    np.testing.assert_allclose(w, w_o, rtol=2e-6, atol=0)
    sel = np.unique(np.linspace(0, n - 1, min(n, 5)).astype(np.int32))
    err = rel_err(out[sel], port.moe_forward(lw, x, sel)[0])
    say(f"{name} n={n}: max rel err {err:.2e}")
    assert err <= REL_TOL
    L.close()
