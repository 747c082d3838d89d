"""f4 on the GPU: host telemetry fed from the GPU's routing.

A configured layer routes a batch on the GPU; its topk_ids / topk_w go to jx_tier_record (the side
effects of select_experts_cache_aware, src/tier.cpp:186-194), and the result is compared with the
reference's own LFRUTierManager (oracle/_ref) routing the same logits one token at a time and read back
through snapshot_telemetry (src/tier.cpp:233-263).  The GPU's logits are bit-exact, so activation
counts, last steps and LFRU scores must match exactly.  last_prob is the GPU's softmax weight, whose
exp differs from glibc's expf by at most a few ulp: it is held to 2e-6 relative.
"""
import numpy as np
import pytest

from jxai_amd import synth
from tests.test_gpu import say
from tests.test_telemetry import ref_replay

pytestmark = pytest.mark.gpu

PROB_RTOL = 2e-6


@pytest.fixture(scope="module")
def moe():
    from jxai_amd import moe as M
    M.init(0)
    return M


@pytest.mark.parametrize("name,n,ticks", [("toy", 1, 0), ("mixtral", 1, 3), ("qwen15moe", 64, 10),
                                          ("qwen3moe", 300, 250), ("dsv2lite", 32, 0), ("qwen3moe", 1, 1)])
def test_gpu_routing_feeds_reference_telemetry(moe, ref, name, n, ticks):
    from jxai_amd import telemetry
    cfg = synth.CONFIGS[name]
    say(f"telemetry {name} n={n}")
    L = moe.MoELayer.from_weights(synth.make_layer(cfg))
    x = synth.make_tokens(cfg, n, seed=61)
    _, ids, w, counts = L.forward(x)
    lg = L.last_logits(n)
    L.close()
    E, k, layer, n_layers = cfg.n_experts, cfg.top_k, 1, 2
    T = telemetry.ExpertTelemetry(n_layers, E)
    T.step_tick(ticks)
    first = T.current_step + 1
    T.record(layer, ids, w)
    act, score, lp = ref_replay(ref, lg, k, layer, n_layers, ticks)
    assert np.array_equal(T.activation_counts, act)
    assert np.array_equal(T.activation_counts[layer * E:(layer + 1) * E], counts)
    snap = T.snapshot()
    assert [s["lfru_score"] for s in snap] == score.tolist()
    # last step of each expert: the step of the last token that selected it (tokens are steps first, ...)
    want_step = np.zeros(n_layers * E, np.uint32)
    for t in range(n):
        want_step[layer * E + ids[t]] = first + t
    assert np.array_equal(T.last_step, want_step)
    used = lp != 0
    assert np.array_equal(used, T.last_prob != 0)
    np.testing.assert_allclose(T.last_prob[used], lp[used], rtol=PROB_RTOL, atol=0)
