"""GPU parity of the fused one-token steps (k_decode1: router rows, gate/up, down and the folded
combine in one launch whose blocks hand over through device-coherent words; k_decode_p: the same
step as one block per CU for layers with many gate/up tiles) against the separate launches
(JX_FWD_UNFUSED).  Both run the same arithmetic in the same order, so the bar is bit-exact:
outputs, router logits, ids, weights, counts and the Q8_0 of x.  The layer's launch count tags each
launch's logits and h's scale words (blocks poll for the tag), so the cases run many fused steps in
a row, interleaved with separate and multi-token calls, on one layer.  The layer outputs
themselves are held to the reference by the golden and oracle tests of test_gpu.py, whose one-token
cases take the fused launch where it is chosen (gate/up blocks at most one per CU); here JX_FUSED=1
forces it on every shape it is built for, the Mixtral-sized ones included.
"""
import numpy as np
import pytest

from jxai_amd import formats as F
from jxai_amd import synth
from tests.test_gpu import REL_TOL, rel_err, say

pytestmark = pytest.mark.gpu

_LAYERS = {}

EXTRA = {
    # the residual-stream form (combine after the fused launch) at a Mixtral-sized d_model
    "mixtral_norm": synth.LayerConfig("mixtral_norm", 4096, 8, 2, 1024, F.Q4_K, norms=True),
    # top-4 without a shared expert: two gate/up block pairs, the combine after the fused launch
    "toy_k4": synth.LayerConfig("toy_k4", 512, 16, 4, 768, F.Q8_0),
    # shared experts: GELU gate with a sigmoid-gated shared expert, and the residual-stream form
    "gelu_q4k": synth.LayerConfig("gelu_q4k", 512, 8, 2, 768, F.Q4_K, d_ff_shared=512, shared_gate=True, act=1),
    "qwen15_norm": synth.LayerConfig("qwen15_norm", 512, 12, 4, 384, F.Q4_0, d_ff_shared=768, shared_gate=True,
                                     norms=True),
    # a shared expert without a gate (weight 1) and of an odd row-tile count (17: one shared gate/up
    # block runs a single tile)
    "toy_sh_nogate": synth.LayerConfig("toy_sh_nogate", 512, 8, 2, 1024, F.Q8_0, d_ff_shared=544),
    # fp32 h at d_ff = 1408 (no Q8_0 form for a K-quant or Q5_0 down): h as tagged fp32 words, the folded
    # combine (top-2, no shared expert)
    "toy_f32dn_q4k": synth.LayerConfig("toy_f32dn_q4k", 512, 8, 2, 1408, F.Q4_K),
    "toy_f32dn_q50": synth.LayerConfig("toy_f32dn_q50", 512, 8, 2, 1408, F.Q4_K, down_wtype=F.Q5_0),
}

FUSED = ["toy", "toy_gelu", "toy_gelu_sh", "toy_f16r", "toy_q5k", "toy_q6k", "toy_k4", "qwen3moe", "gelu_q4k", "qwen15_norm",
         "toy_sh_nogate", "toy_bf16r_sh", "qwen15moe", "mixtral_norm", "mixtral", "mixtral_q6k",
         # fp32-activation routed downs, with shared experts of the routed or another down format
         "toy_f32dn_q4k", "toy_f32dn_q50", "dsv2lite", "dsv2lite_q50"]


@pytest.fixture(scope="module")
def moe():
    from jxai_amd import moe as M
    M.init(0)
    return M


def layer(name):
    if name not in _LAYERS:
        _LAYERS.clear()
        cfg = synth.CONFIGS[name] if name in synth.CONFIGS else EXTRA[name]
        _LAYERS[name] = (cfg, synth.make_layer(cfg))
    return _LAYERS[name]


def same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.fixture(autouse=True)
def force_fused(monkeypatch):
    monkeypatch.setenv("JX_FUSED", "1")  # read when a layer is created


def took_fused(L, x, residual):
    L.profile(True)
    L.forward(x, residual=residual)
    names = set(L.profile_read())
    L.profile(False)
    return bool(names & {"decode_fused", "decode_fused_y", "decode_fused_cu"})


def took_cu(L, x):
    L.profile(True)
    L.forward(x)
    names = set(L.profile_read())
    L.profile(False)
    return "decode_fused_cu" in names


def step(L, x, fused, residual):
    out, ids, w, counts = L.forward(x, fused=fused, residual=residual)
    return out, ids, w, counts, L.last_logits(x.shape[0]), L.last_xq8(x.shape[0])


@pytest.mark.parametrize("name", FUSED)
def test_fused_step_matches_separate_launches(moe, port, name):
    cfg, lw = layer(name)
    residual = cfg.norms
    L = moe.MoELayer.from_weights(lw)
    xs = synth.make_tokens(cfg, 6, seed=23)
    x2 = synth.make_tokens(cfg, 2, seed=29)
    assert took_fused(L, xs[:1], residual)
    for i in range(6):
        x = xs[i:i + 1]
        say(f"{name} token {i}: fused vs separate")
        got = step(L, x, True, residual)
        want = step(L, x, False, residual)
        for g, w_, what in zip(got, want, ("out", "ids", "weights", "counts", "logits", "xq8")):
            assert same(g, w_) if g.dtype != np.uint8 else np.array_equal(g, w_), f"token {i}: {what}"
        if i == 2:  # a two-token step (the separate few-token launches) between fused ones
            L.forward(x2, residual=residual)
    # the fused path against the reference's algorithm (the CPU restatement) on the last token
    x = xs[5:6]
    out = L.forward(x, residual=residual)[0]
    want, ids_o, _, _ = port.moe_forward(lw, x, np.array([0], np.int32), residual=residual)
    err = rel_err(out, want)
    say(f"{name}: fused step vs oracle max rel err {err:.2e}")
    assert err <= REL_TOL
    L.close()


@pytest.mark.parametrize("name", ["toy", "qwen15moe", "mixtral", "dsv2lite_q50"])
def test_fused_steps_back_to_back(moe, name):
    """Hundreds of fused launches queued without host synchronization (the launch count, and with
    it the tags of the logits and of h's scales, advances every step), then the last outputs against
    separate-launch steps."""
    cfg, lw = layer(name)
    L = moe.MoELayer.from_weights(lw)
    xs = synth.make_tokens(cfg, 2, seed=41)
    assert took_fused(L, xs[:1], False)
    xa, xb_ = xs[0:1], xs[1:2]
    want_a = L.forward(xa, fused=False)[0]
    want_b = L.forward(xb_, fused=False)[0]
    da = moe.DeviceBuffer(xa.nbytes).upload(xa)
    db = moe.DeviceBuffer(xb_.nbytes).upload(xb_)
    oa = moe.DeviceBuffer(xa.nbytes)
    ob = moe.DeviceBuffer(xb_.nbytes)
    say(f"{name}: 400 fused steps back to back")
    for i in range(200):
        L.forward_device(da, 1, oa, sync=False)
        L.forward_device(db, 1, ob, sync=False)
    moe.lib().jx_device_synchronize()
    assert same(oa.download(np.empty_like(xa)), want_a)
    assert same(ob.download(np.empty_like(xb_)), want_b)
    # a synchronous fused step reports no timed-out wait
    assert same(L.forward(xa)[0], want_a)
    for buf in (da, db, oa, ob):
        buf.free()
    L.close()


# k_decode_p: one block per CU (every block routes the token itself; the down tiles start once h's
# tagged scale words say their slot is complete); taken by itself on the Mixtral-shaped layers.  It
# needs at least as many gate/up row tiles as CUs (d_ff >= 32 * 256 here), so the smaller shapes keep
# Mixtral's d_ff at d_model 512, in each format it is built for (an F16 router on one).
EXTRA.update({
    "cu_q4_0": synth.LayerConfig("cu_q4_0", 512, 8, 2, 14336, F.Q4_0),
    "cu_q8_0": synth.LayerConfig("cu_q8_0", 512, 8, 2, 14336, F.Q8_0, router_type=F.F16),
    "cu_q5k": synth.LayerConfig("cu_q5k", 512, 8, 2, 14336, F.Q5_K),
    "cu_q6k": synth.LayerConfig("cu_q6k", 512, 8, 2, 14336, F.Q6_K),
    "cu_q4k": synth.LayerConfig("cu_q4k", 512, 8, 2, 14336, F.Q4_K),
})
CU = ["cu_q4_0", "cu_q8_0", "cu_q5k", "cu_q6k", "cu_q4k", "mixtral", "mixtral_q6k"]


@pytest.mark.parametrize("name", CU)
def test_fused_cu_step_matches_separate_launches(moe, port, monkeypatch, name):
    monkeypatch.setenv("JX_DECP", "1")
    cfg, lw = layer(name)
    L = moe.MoELayer.from_weights(lw)
    xs = synth.make_tokens(cfg, 4, seed=31)
    x2 = synth.make_tokens(cfg, 2, seed=37)
    assert took_cu(L, xs[:1])
    for i in range(4):
        x = xs[i:i + 1]
        say(f"{name} token {i}: one block per CU vs separate")
        got = step(L, x, True, False)
        want = step(L, x, False, False)
        for g, w_, what in zip(got, want, ("out", "ids", "weights", "counts", "logits", "xq8")):
            assert same(g, w_) if g.dtype != np.uint8 else np.array_equal(g, w_), f"token {i}: {what}"
        if i == 1:
            L.forward(x2)
    x = xs[3:4]
    out = L.forward(x)[0]
    want, _, _, _ = port.moe_forward(lw, x, np.array([0], np.int32))
    err = rel_err(out, want)
    say(f"{name}: one-block-per-CU step vs oracle max rel err {err:.2e}")
    assert err <= REL_TOL
    L.close()


# ------------------------------------------------------------------ a wait that gives up is reported
@pytest.mark.parametrize("name,cu", [("toy", False), ("qwen15moe", False), ("cu_q4k", True), ("dsv2lite_q50", False)])
def test_fused_giveup_is_reported(moe, monkeypatch, name, cu):
    """JX_FWD_TEST_GIVEUP makes every wait of the fused launch give up after a few polls (the kernels
    end normally; the outputs are invalid).  The failure must reach the caller on every path: the
    synchronous call returns an error; after an asynchronous call, jx_moe_layer_status reports it once,
    and otherwise the layer's next forward does, without running.  The step after a report is
    bit-identical to the separate launches (the launch count goes on, so nothing left by the failed
    launch can pass a later wait)."""
    if cu:
        monkeypatch.setenv("JX_DECP", "1")
    cfg, lw = layer(name)
    L = moe.MoELayer.from_weights(lw)
    xs = synth.make_tokens(cfg, 2, seed=53)
    x = xs[:1]
    assert (took_cu(L, x) if cu else took_fused(L, x, False))
    want = L.forward(x, fused=False)[0]
    dx = moe.DeviceBuffer(x.nbytes).upload(x)
    do = moe.DeviceBuffer(x.nbytes)
    giveup = moe.JX_FWD_TEST_GIVEUP

    def fused_ok():
        L.forward_device(dx, 1, do)
        return same(do.download(np.empty_like(x)), want)

    say(f"{name}: synchronous step whose waits give up")
    with pytest.raises(moe.JxError, match="timed out"):
        L.forward_device(dx, 1, do, extra_flags=giveup)
    assert fused_ok()
    say(f"{name}: asynchronous step whose waits give up, then jx_moe_layer_status")
    L.forward_device(dx, 1, do, sync=False, extra_flags=giveup)
    with pytest.raises(moe.JxError, match="timed out"):
        L.status(wait=True)
    L.status(wait=True)  # reported once
    assert fused_ok()
    say(f"{name}: asynchronous step whose waits give up, then the next forward")
    L.forward_device(dx, 1, do, sync=False, extra_flags=giveup)
    moe.lib().jx_device_synchronize()
    with pytest.raises(moe.JxError, match="timed out"):
        L.forward(xs[1:2])
    assert fused_ok()
    assert same(L.forward(x)[0], want)
    dx.free()
    do.free()
    L.close()


def test_fused_shared_first_step_after_recreate(moe):
    """A layer with a shared expert, created where a destroyed layer of the same shape ran fused steps:
    its first fused step must not take the old layer's tagged h scale words (the shared h's scale words
    start untagged), so it equals the separate launches bit for bit."""
    cfg, lw = layer("qwen15_norm")
    cfg2 = synth.LayerConfig("qwen15_norm2", cfg.d_model, cfg.n_experts, cfg.top_k, cfg.d_ff, cfg.wtype,
                             d_ff_shared=cfg.d_ff_shared, shared_gate=True)
    lw2 = synth.make_layer(cfg2, seed=77)
    x = synth.make_tokens(cfg, 1, seed=59)
    for rnd in range(3):
        say(f"recreate round {rnd}")
        L = moe.MoELayer.from_weights(lw if rnd % 2 == 0 else lw2)
        first = L.forward(x)[0]
        assert took_fused(L, x, False)
        assert same(first, L.forward(x, fused=False)[0])
        L.close()


def test_fused_cu_steps_on_several_streams(moe, monkeypatch):
    """One-block-per-CU steps of three layers queued asynchronously, each on the layer's own stream: two of
    them running at once could each hold CUs the other waits for, so the library orders them across
    streams.  Every step completes its waits (jx_moe_layer_status) and the outputs equal the separate
    launches bit for bit."""
    monkeypatch.setenv("JX_DECP", "1")
    cfg, lw = layer("cu_q4k")
    Ls = [moe.MoELayer.from_weights(lw) for _ in range(3)]
    x = synth.make_tokens(cfg, 1, seed=71)
    assert took_cu(Ls[0], x)
    want = Ls[0].forward(x, fused=False)[0]
    dx = moe.DeviceBuffer(x.nbytes).upload(x)
    outs = [moe.DeviceBuffer(x.nbytes) for _ in Ls]
    say("three layers, 300 steps, each on its own stream")
    for i in range(300):
        j = i % 3
        Ls[j].forward_device(dx, 1, outs[j], sync=False)
    moe.lib().jx_device_synchronize()
    for L, o in zip(Ls, outs):
        L.status(wait=True)
        assert same(o.download(np.empty_like(x)), want)
    dx.free()
    for o in outs:
        o.free()
    for L in Ls:
        L.close()
