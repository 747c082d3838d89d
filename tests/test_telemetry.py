"""Host telemetry (jx_tier_record, jx_tier_lfru_score) against the reference's own LFRUTierManager:
the same logits routed one token at a time through select_experts_cache_aware in the reference build
(oracle/_ref) and read back with snapshot_telemetry must give the counters, last probabilities and LFRU
scores that the library replays from the batch's topk_ids / topk_w."""
import ctypes as C

import numpy as np
import pytest

from jxai_amd import synth


@pytest.fixture(scope="module")
def tel():
    from jxai_amd import _lib, telemetry
    import os
    if not os.path.exists(_lib.LIB_PATH):
        from jxai_amd import build
        build.build(verbose=False)
    return telemetry


def ref_replay(ref, logits, k, layer, n_layers, ticks_before):
    n, E = logits.shape
    m = n_layers * E
    act = np.zeros(m, np.uint32)
    score = np.zeros(m, np.uint32)
    lp = np.zeros(m, np.float32)
    L = ref.lib
    L.jxr_tier_replay.restype = C.c_int32
    L.jxr_tier_replay.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                  C.c_void_p, C.c_void_p, C.c_void_p]
    lg = np.ascontiguousarray(logits, np.float32)
    got = L.jxr_tier_replay(lg.ctypes.data, n, E, k, layer, n_layers, ticks_before, act.ctypes.data,
                            score.ctypes.data, lp.ctypes.data)
    assert got == m
    return act, score, lp


@pytest.mark.parametrize("E,k,n,ticks", [(8, 2, 37, 0), (60, 4, 300, 5), (128, 8, 64, 400), (8, 2, 1, 0)])
def test_tier_record_matches_reference(tel, port, ref, E, k, n, ticks):
    logits = synth.normal_f32(synth.sub_seed("tier", f"{E}_{n}"), n * E, 0.7).reshape(n, E)
    ids = np.zeros((n, k), np.int32)
    probs = np.zeros((n, k), np.float32)
    for t in range(n):
        ids[t], probs[t], _ = port.select_experts(logits[t], k)
    n_layers, layer = 3, 1
    T = tel.ExpertTelemetry(n_layers, E)
    T.step_tick(ticks)
    T.record(layer, ids, probs)
    act, score, lp = ref_replay(ref, logits, k, layer, n_layers, ticks)
    assert np.array_equal(T.activation_counts, act)
    assert np.array_equal(T.last_prob.view(np.uint32), lp.view(np.uint32))
    snap = T.snapshot()
    assert [s["lfru_score"] for s in snap] == score.tolist()
    assert sum(s["activations"] for s in snap) == n * k


def test_tier_record_rejects_bad_ids(tel):
    from jxai_amd._lib import JxError
    T = tel.ExpertTelemetry(1, 4)
    with pytest.raises(JxError):
        T.record(0, np.array([[5, 1]], np.int32), np.array([[0.5, 0.5]], np.float32))
