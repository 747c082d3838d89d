"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the GPU checker.

Each oracle function is checked three ways where possible:
  * against the reference's own known answers (README.md:70 self-test KATs);
  * bit-for-bit against golden vectors written by tests/golden/make_golden.py
    from a build of the reference's src/quant.cpp + src/tier.cpp, and live
    against that build when it is present (this container);
  * against what the mathematics fixes, independently of lane order: the block
    formats' closed-form dequantization (include/quant.h:10-33) with float64
    sums, round-toward-zero for the fp16 store, brute-force top-k, and a
    float64 restatement of the whole MoE block.
"""
import os

import numpy as np
import pytest

from jxai_amd import formats as F
from jxai_amd import synth
from tests.conftest import GOLDEN


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


# --------------------------------------------------------------- numpy decode of the block formats
def deq_q8_blocks(b: np.ndarray) -> np.ndarray:
    blk = b.reshape(-1, 34)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)
    q = blk[:, 2:].view(np.int8).astype(np.float64)
    return (q * d).reshape(-1)


def deq_matrix(qt: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Closed-form dequantization of a [rows][cols] block matrix, float64."""
    blk, bsz = F.BLOCK[qt]
    nb = (cols + blk - 1) // blk
    b = w.reshape(rows, nb, bsz)
    if qt == F.Q4_0:
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)
        qs = b[:, :, 2:18].astype(np.int64)
        vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=2).astype(np.float64)
        return (vals * d).reshape(rows, nb * 32)[:, :cols]
    if qt == F.Q8_0:
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)
        return (b[:, :, 2:34].view(np.int8).astype(np.float64) * d).reshape(rows, nb * 32)[:, :cols]
    if qt == F.Q5_0:  # d, qh (u32 LE: bit j = fifth bit of element j), qs: low nibbles 0..15, high 16..31
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)
        qh = b[:, :, 2:6].copy().view("<u4").astype(np.int64)
        qs = b[:, :, 6:22].astype(np.int64)
        bits = (qh >> np.arange(32)) & 1
        vals = np.concatenate([qs & 15, qs >> 4], axis=2) + 16 * bits - 16
        return (vals * d).reshape(rows, nb * 32)[:, :cols]
    if qt == F.Q6_K:  # ql[128], qh[64], int8 scales[16], d; element 128n + 32r + l
        ql = b[:, :, 0:128].astype(np.int64).reshape(rows, nb, 2, 2, 32)   # [n][r % 2][l]
        qh = b[:, :, 128:192].astype(np.int64).reshape(rows, nb, 2, 1, 32)  # [n][l]
        sc = b[:, :, 192:208].view(np.int8).astype(np.float64)
        d = b[:, :, 208:210].copy().view(np.float16).astype(np.float64)
        r = np.arange(4).reshape(1, 1, 1, 4, 1)
        nib = (np.take_along_axis(ql, np.broadcast_to(r % 2, (rows, nb, 2, 4, 1)), axis=3) >> (4 * (r // 2))) & 15
        q = (nib | (((qh >> (2 * r)) & 3) << 4)) - 32  # [rows][nb][n][r][l]
        vals = q.reshape(rows, nb, 256) * np.repeat(sc, 16, axis=2) * d
        return vals.reshape(rows, nb * 256)[:, :cols]
    # Q4_K / Q5_K: d, dmin, 12 bytes of 6-bit (scale, min) pairs (Q5_K: then qh[32]), 128 bytes of nibbles
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    dmin = b[:, :, 2:4].copy().view(np.float16).astype(np.float64)[..., 0]
    s = b[:, :, 4:16].astype(np.int64)
    sc = np.empty((rows, nb, 8), np.int64)
    mn = np.empty((rows, nb, 8), np.int64)
    sc[..., :4] = s[..., 0:4] & 63
    mn[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    q0 = 48 if qt == F.Q5_K else 16
    qs = b[:, :, q0:q0 + 128].astype(np.int64).reshape(rows, nb, 4, 32)
    nib = np.stack([qs & 15, qs >> 4], axis=3).reshape(rows, nb, 8, 32)  # sub-block 2j: low, 2j+1: high
    if qt == F.Q5_K:  # fifth bit of element l of sub-block j: bit j of qh[l]
        qh = b[:, :, 16:48].astype(np.int64)
        nib = nib + 16 * ((qh[:, :, None, :] >> np.arange(8).reshape(1, 1, 8, 1)) & 1)
    w_ = d[..., None, None] * sc[..., None] * nib - dmin[..., None, None] * mn[..., None]
    return w_.reshape(rows, nb * 256)[:, :cols]


# --------------------------------------------------------------- known answers from the reference
def test_readme_kats(port):
    """README.md:70 (src/main.cpp:166-182): fp32 dot 0.150863, Q8_0 dot 0.152989 (K=128)."""
    i = np.arange(128, dtype=np.float32)
    x = np.sin(i * np.float32(0.1)).astype(np.float32)
    y = np.cos(i * np.float32(0.2)).astype(np.float32)
    assert f"{port.vec_dot_f32(x, y):.6f}" == "0.150863"
    q8dot = float(np.dot(deq_q8_blocks(port.quantize_row_q8_0(x)), y.astype(np.float64)))
    assert abs(q8dot - 0.152989) < 1e-6


# --------------------------------------------------------------- fp16 store: round toward zero
def test_fp16_truncation_is_round_toward_zero(port):
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.standard_normal(3000) * 10 ** rng.uniform(-9, 5, 3000),
                         [0.0, 65504.0, 65535.9, 65536.0, 1e30, 2.0 ** -24, 2.0 ** -25, 2.0 ** -26]]).astype(np.float32)
    for x in xs:
        h = port.fp32_to_fp16(float(x))
        v = float(np.uint16(h).view(np.float16))
        ax = abs(float(x))
        if ax >= 65536.0:
            assert np.isinf(v)
            continue
        assert abs(v) <= ax and (v == 0 or np.sign(v) == np.sign(x))
        nxt = float((np.uint16(h & 0x7FFF) + np.uint16(1)).view(np.float16))
        assert nxt > ax  # nothing on the fp16 grid between the result and |x|
        assert port.fp16_to_fp32(h) == np.float32(v)


def test_fp16_golden(port):
    z = load("units.npz")
    got = np.array([port.fp32_to_fp16(float(v)) for v in z["f"]], np.uint16)
    assert np.array_equal(got, z["h"])


# --------------------------------------------------------------- Q8_0 activation quantization
def test_quantize_q8_0_properties(port):
    x = synth.normal_f32(77, 32 * 256, 2.0)
    x[:32] = 0
    x[32:64] = np.arange(32, dtype=np.float32) - 15.5
    q = port.quantize_row_q8_0(x).reshape(-1, 34)
    xb = x.reshape(-1, 32)
    for b in range(xb.shape[0]):
        amax = np.float32(np.abs(xb[b]).max())
        d = np.float32(amax / np.float32(127.0))
        d16 = float(q[b, 0:2].copy().view(np.float16)[0])
        assert d16 <= d and (d == 0 or d16 > d * (1 - 2 ** -10))
        qs = q[b, 2:].view(np.int8).astype(np.int64)
        if d == 0:
            assert not qs.any()
            continue
        v = (xb[b] * (np.float32(1.0) / d)).astype(np.float64)  # fp32 product, exact in float64
        assert np.all(np.abs(v - qs) <= 0.5)
        ties = np.abs(np.abs(v - np.trunc(v)) - 0.5) == 0
        assert np.all(np.abs(qs[ties]) == np.ceil(np.abs(v[ties])))  # half away from zero
        assert np.abs(qs).max() <= 127


def test_quantize_q8_0_golden(port):
    z = load("units.npz")
    assert np.array_equal(port.quantize_row_q8_0(z["xs"]), z["xq"])


# --------------------------------------------------------------- block dots
@pytest.mark.parametrize("key", ["2_2048", "8_2048", "12_4096", "12_896"])
def test_dots_golden_and_float64(port, key):
    z = load("units.npz")
    qt, cols = map(int, key.split("_"))
    w, y = z[f"dot_w_{key}"], z[f"dot_y_{key}"]
    rows = 16
    got = port.matmul_quant_f32(qt, w, y, rows, cols)
    assert np.array_equal(got.view(np.uint32), z[f"dot_out_{key}"].view(np.uint32))
    # float64 from the closed-form block decode, with the same Q8_0 activations
    # (or fp32 activations when the reference's rule says so)
    W = deq_matrix(qt, w, rows, cols)
    if F.supports_q8_activation(qt, cols):
        ya = deq_q8_blocks(port.quantize_row_q8_0(y))
    else:
        ya = y.astype(np.float64)
    exact = W @ ya
    bound = np.abs(W) @ np.abs(ya)
    assert np.all(np.abs(got - exact) <= 2e-6 * bound + 1e-30)
    # the direct block dot (incl. the partial super-block path at cols=896)
    yq = port.quantize_row_q8_0(np.concatenate([y, np.zeros((-cols) % 256, np.float32)]))
    rb = F.row_bytes(qt, cols)
    direct = np.array([port.vec_dot_q8(qt, w[r * rb:(r + 1) * rb], yq, cols) for r in range(rows)], np.float32)
    assert np.array_equal(direct.view(np.uint32), z[f"dot_direct_{key}"].view(np.uint32))


def test_q4_K_fp32_partial_superblock(port):
    z = load("units.npz")
    got = port.matmul_quant_f32(F.Q4_K, z["w14"], z["y14"], 16, 1408)
    assert np.array_equal(got.view(np.uint32), z["o14"].view(np.uint32))
    W = deq_matrix(F.Q4_K, z["w14"], 16, 1408)
    exact = W @ z["y14"].astype(np.float64)
    assert np.all(np.abs(got - exact) <= 2e-6 * (np.abs(W) @ np.abs(z["y14"].astype(np.float64))))


def test_swiglu_golden(port):
    z = load("units.npz")
    got = port.matmul_swiglu_quant_f32(F.Q4_0, z["sw_g"], F.Q4_0, z["sw_u"], z["sw_x"], 64, 512)
    assert np.array_equal(got.view(np.uint32), z["sw_o"].view(np.uint32))
    xa = deq_q8_blocks(port.quantize_row_q8_0(z["sw_x"]))
    g = deq_matrix(F.Q4_0, z["sw_g"], 64, 512) @ xa
    u = deq_matrix(F.Q4_0, z["sw_u"], 64, 512) @ xa
    np.testing.assert_allclose(got, g / (1 + np.exp(-g)) * u, rtol=1e-5, atol=1e-6)


def _gelu64(g):
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))


@pytest.mark.parametrize("qt,rows,cols", [(F.Q4_0, 256, 512), (F.Q4_K, 128, 1024), (F.Q8_0, 128, 2048)])
def test_gelu_gate_float64(port, qt, rows, cols):
    """use_gelu (src/quant.cpp:3999-4003): GELU-tanh of the gate times up, against a float64 closed form."""
    Wg = synth.quant_matrix(synth.sub_seed("gelu", f"g{qt}"), qt, rows, cols)
    Wu = synth.quant_matrix(synth.sub_seed("gelu", f"u{qt}"), qt, rows, cols)
    x = synth.normal_f32(synth.sub_seed("gelu", f"x{qt}"), cols, 3.0)
    got = port.matmul_swiglu_quant_f32(qt, Wg, qt, Wu, x, rows, cols, use_gelu=True)
    xa = deq_q8_blocks(port.quantize_row_q8_0(x))
    g, u = deq_matrix(qt, Wg, rows, cols) @ xa, deq_matrix(qt, Wu, rows, cols) @ xa
    want = _gelu64(g) * u
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    assert not np.array_equal(got, port.matmul_swiglu_quant_f32(qt, Wg, qt, Wu, x, rows, cols))


@pytest.mark.parametrize("qt,rows,cols", [(F.Q4_0, 256, 512), (F.Q4_K, 128, 1024), (F.Q8_0, 128, 2048)])
def test_gelu_gate_live_vs_reference(port, ref, qt, rows, cols):
    """Bit-exact against the reference build, gates spread over |g| up to ~100 (the fma the build
    contracts the cubic's sum into changes the bits of ~16% of such sums)."""
    Wg = synth.quant_matrix(synth.sub_seed("gelu", f"g{qt}"), qt, rows, cols)
    Wu = synth.quant_matrix(synth.sub_seed("gelu", f"u{qt}"), qt, rows, cols)
    for scale in (0.3, 3.0, 30.0):
        x = synth.normal_f32(synth.sub_seed("gelu", f"x{qt}_{scale}"), cols, scale)
        a = port.matmul_swiglu_quant_f32(qt, Wg, qt, Wu, x, rows, cols, use_gelu=True)
        b = ref.matmul_swiglu_quant_f32(qt, Wg, qt, Wu, x, rows, cols, use_gelu=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# --------------------------------------------------------------- the five- and six-bit formats
F3_MM = ["13_16_2048", "14_16_2048", "13_16_896", "14_16_1408", "6_16_1408", "2_4_512", "8_4_512", "12_4_512"]


@pytest.mark.parametrize("qt", [F.Q5_0, F.Q5_K, F.Q6_K])
def test_f3_dequantize_golden(port, qt):
    """dequantize_row_q5_0 / _q5_K / _q6_K (src/quant.cpp:1585-1600, 1345-1387, 1389-1428) bit for bit
    against the reference build's vectors and exactly against the closed-form decode (every value is
    exact in fp32: d * sc * q products of at most 22 bits)."""
    z = load("units_f3.npz")
    w, cols = z[f"deq_w_{qt}"], 512
    rb = F.row_bytes(qt, cols)
    got = np.concatenate([port.dequantize_row(qt, w[r * rb:], cols) for r in range(2)])
    assert np.array_equal(got.view(np.uint32), z[f"deq_o_{qt}"].view(np.uint32))
    assert np.array_equal(got.astype(np.float64), deq_matrix(qt, w, 2, cols).reshape(-1))


@pytest.mark.parametrize("key", F3_MM)
def test_f3_dots_golden_and_float64(port, key):
    """matmul_quant_f32 (Q8_0 x from 8 rows where the type allows, fp32 otherwise), vec_dot_quant_f32 and
    the Q5_K / Q6_K Q8_0-activation dots (src/quant.cpp:3648-3818) against the reference build's vectors,
    then against the float64 closed form with the activations each path uses."""
    z = load("units_f3.npz")
    qt, rows, cols = map(int, key.split("_"))
    w, y = z[f"mm_w_{key}"], z[f"mm_y_{key}"]
    got = port.matmul_quant_f32(qt, w, y, rows, cols)
    assert np.array_equal(got.view(np.uint32), z[f"mm_o_{key}"].view(np.uint32))
    rb = F.row_bytes(qt, cols)
    f32 = np.array([port.vec_dot_quant_f32(qt, w[r * rb:(r + 1) * rb], y) for r in range(rows)], np.float32)
    assert np.array_equal(f32.view(np.uint32), z[f"f32_o_{key}"].view(np.uint32))
    W = deq_matrix(qt, w, rows, cols)
    y64 = y.astype(np.float64)
    assert np.all(np.abs(f32 - W @ y64) <= 2e-6 * (np.abs(W) @ np.abs(y64)) + 1e-30)
    if qt in (F.Q5_K, F.Q6_K):
        yq = port.quantize_row_q8_0(np.concatenate([y, np.zeros((-cols) % 256, np.float32)]))
        q8 = np.array([port.vec_dot_q8(qt, w[r * rb:(r + 1) * rb], yq, cols) for r in range(rows)], np.float32)
        assert np.array_equal(q8.view(np.uint32), z[f"q8_o_{key}"].view(np.uint32))
        ya = deq_q8_blocks(yq)[:cols]
        assert np.all(np.abs(q8 - W @ ya) <= 2e-6 * (np.abs(W) @ np.abs(ya)) + 1e-30)
    # the dispatcher's activation form (supports_q8_activation, quant.cpp:3881-3893, from 8 rows): here
    # every case without Q8_0 activations must equal the fp32 dots, and every Q5_K / Q6_K one with them
    # the Q8_0 dots
    if not (rows >= 8 and F.supports_q8_activation(qt, cols)):
        assert np.array_equal(got.view(np.uint32), f32.view(np.uint32))
    elif qt in (F.Q5_K, F.Q6_K):
        assert np.array_equal(got.view(np.uint32), q8.view(np.uint32))


def _h16_values(t, w):
    """Half / bfloat16 bits -> exact float64 values."""
    if t == F.F16:
        return w.view(np.float16).astype(np.float64)
    return (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("t", [F.F16, F.BF16])
def test_router16_dots_golden_and_float64(port, t):
    """vec_dot_f16_f32 / vec_dot_bf16_f32 (src/quant.cpp:3015-3055): the reference build's values bit for
    bit (with and without the scalar tail), the float64 closed form of the widened weights, and the
    lane structure itself: the 16-lane vec_dot_f32 order over the same values differs from the golden
    (so a router kernel left in the fp32 order would be caught)."""
    z = load("units_router16.npz")
    for k in (37, 512, 4101):
        w, y = z[f"dot_w_{t}_{k}"], z[f"dot_y_{t}_{k}"]
        got = np.float32(port.vec_dot_quant_f32(t, w.view(np.uint8), y))
        assert got.view(np.uint32) == z[f"dot_o_{t}_{k}"].view(np.uint32), (t, k)
        w64 = _h16_values(t, w)
        assert abs(float(got) - float(w64 @ y.astype(np.float64))) <= 2e-6 * float(np.abs(w64) @ np.abs(y)) + 1e-30
    w, y = z[f"dot_w_{t}_4101"], z[f"dot_y_{t}_4101"]
    wrong = np.float32(port.vec_dot_f32(_h16_values(t, w).astype(np.float32), y))
    assert wrong.view(np.uint32) != z[f"dot_o_{t}_4101"].view(np.uint32)
    E, d = 24, 2048
    mw, mx = z[f"mm_w_{t}"], z[f"mm_x_{t}"]
    got = port.matmul_quant_f32(t, mw.view(np.uint8), mx, E, d)
    assert np.array_equal(got.view(np.uint32), z[f"mm_o_{t}"].view(np.uint32))


@pytest.mark.parametrize("t", [F.F16, F.BF16])
def test_router16_live_vs_reference(port, ref, t):
    """Seeded rows of assorted lengths through both builds, bit for bit, and a layer's routing."""
    import dataclasses
    rng = np.random.default_rng(11 + t)
    for k in (8, 24, 64, 136, 1000, 2048, 8192):
        v = (rng.standard_normal(k) * 0.05).astype(np.float32)
        w = synth.to_f16_bits(v) if t == F.F16 else synth.to_bf16_bits(v)
        y = rng.standard_normal(k).astype(np.float32)
        a = np.float32(port.vec_dot_quant_f32(t, w.view(np.uint8), y))
        b = np.float32(ref.vec_dot_quant_f32(t, w.view(np.uint8), y))
        assert a.view(np.uint32) == b.view(np.uint32), (t, k)
    cfg = dataclasses.replace(synth.CONFIGS["toy"], name="toy_live_r16", router_type=t)
    lw, x = synth.make_layer(cfg), synth.make_tokens(synth.CONFIGS["toy"], 6)
    o1, i1, w1, l1 = port.moe_forward(lw, x)
    o2, i2, w2, l2 = ref.moe_forward(lw, x)
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32)) and np.array_equal(i1, i2)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))


@pytest.mark.parametrize("qt", [F.Q5_0, F.Q6_K, F.Q5_K])
def test_f3_swiglu_golden(port, qt):
    """matmul_swiglu_quant_f32 over fp32 x (Q5_0: no Q8_0 form) and Q8_0 x (Q5_K, Q6_K)."""
    z = load("units_f3.npz")
    g, u, x = z[f"sw_g_{qt}"], z[f"sw_u_{qt}"], z[f"sw_x_{qt}"]
    got = port.matmul_swiglu_quant_f32(qt, g, qt, u, x, 64, 512)
    assert np.array_equal(got.view(np.uint32), z[f"sw_o_{qt}"].view(np.uint32))
    xa = x.astype(np.float64) if qt == F.Q5_0 else deq_q8_blocks(port.quantize_row_q8_0(x))
    gv, uv = deq_matrix(qt, g, 64, 512) @ xa, deq_matrix(qt, u, 64, 512) @ xa
    np.testing.assert_allclose(got, gv / (1 + np.exp(-gv)) * uv, rtol=1e-5, atol=1e-6 * np.abs(got).max())


def test_f3_q6k_scale_extremes(port, ref):
    """Q6_K with every sub-block scale at -128 or 127 and quants at 0 / 63 (the largest |sc * (q - 32)|),
    both dots, against the reference build."""
    rows, cols = 8, 512
    w = synth.quant_matrix(synth.sub_seed("q6x", "w"), F.Q6_K, rows, cols).reshape(rows * 2, 210)
    w[:, 192:208] = np.where(np.arange(16) % 2, 0x80, 0x7F).astype(np.uint8)
    w[0::2, 0:192] = 0xFF
    w[1::2, 0:192] = 0x00
    w = w.reshape(-1)
    y = synth.normal_f32(synth.sub_seed("q6x", "y"), cols, 50.0)
    for rr in (rows, 4):  # Q8_0 and fp32 activations
        a = port.matmul_quant_f32(F.Q6_K, w, y, rr, cols)
        b = ref.matmul_quant_f32(F.Q6_K, w, y, rr, cols)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("qt,cols", [(F.Q4_0, 512), (F.Q8_0, 512), (F.Q4_K, 1024)])
def test_dequantize_row(port, qt, cols):
    """dequantize_row_q4_0 / _q8_0 / _q4_K (src/quant.cpp:1014-1057, 1209-1249) against the formats'
    closed form, and against the reference build when it is present."""
    w = synth.quant_matrix(synth.sub_seed("deq", f"{qt}"), qt, 1, cols)
    got = port.dequantize_row(qt, w, cols)
    exact = deq_matrix(qt, w, 1, cols)[0]
    # Q4_0 / Q8_0 values are exact in fp32; Q4_K's d * sc * q - dmin * m rounds in fp32
    tol = 0.0 if qt != F.Q4_K else 2.0 ** -22 * np.abs(exact).max()
    assert np.abs(got.astype(np.float64) - exact).max() <= tol
    from oracle import oracle as O
    if O.available("reference"):
        want = O.Oracle("reference").dequantize_row(qt, w, cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("d,scale,weighted", [(512, 1.0, True), (4096, 3.0, True), (128, 1e-3, False), (2048, 0.0, True)])
def test_rms_norm(port, ref, d, scale, weighted):
    """MoETransformerEngine::rms_norm (transformer.cpp:67-73): against the same three steps in
    float32 on the reference build's own vec_dot_f32 (bit for bit: IEEE division and square root),
    and against a float64 closed form (a few ulp)."""
    x = (synth.normal_f32(synth.sub_seed("rms", f"{d}_{scale}"), d, 1.0) * np.float32(scale)).astype(np.float32)
    w = (1.0 + synth.normal_f32(synth.sub_seed("rmsw", str(d)), d, 0.1)).astype(np.float32) if weighted else None
    eps = np.float32(1e-5)
    got = port.rms_norm(x, w, float(eps))
    ss = np.float32(ref.vec_dot_f32(x, x))
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(d) + eps)
    want = x * inv * (w if w is not None else np.float32(1.0))
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    x64 = x.astype(np.float64)
    exact = x64 / np.sqrt((x64 @ x64) / d + 1e-5) * (w.astype(np.float64) if w is not None else 1.0)
    assert np.abs(got - exact).max() <= 4 * np.finfo(np.float32).eps * max(np.abs(exact).max(), 1e-30)


@pytest.mark.parametrize("name", ["toy_norm", "qwen15_norm"])
def test_moe_block_residual_live_vs_reference(port, ref, name):
    """The residual-stream form (rms_norm, block, post_ffw_norm, residual add) bit-exact against the
    reference build's functions."""
    cfg = RESID_CFGS[name]
    lw = synth.make_layer(cfg, seed=5)
    x = synth.make_tokens(cfg, 5, seed=5)
    a = port.moe_forward(lw, x, residual=True)
    b = ref.moe_forward(lw, x, residual=True)
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    plain = port.moe_forward(lw, x)[0]
    assert not np.array_equal(a[0], plain)


RESID_CFGS = {
    "toy_norm": synth.CONFIGS["toy_norm"],
    "qwen15_norm": synth.LayerConfig("qwen15_norm", 512, 12, 4, 384, F.Q4_0, d_ff_shared=768, shared_gate=True,
                                     norms=True),
}


QKV_CASES = [((F.Q4_K, F.Q4_0, F.Q8_0), 512, (256, 4, 4)),   # k, v alone under 8 rows: x quantized for all
             ((F.Q4_K, F.Q4_K, F.Q4_K), 1408, (64, 32, 32)),  # cols % 256 != 0: fp32 Q4_K dots
             ((F.Q4_K, F.Q4_K, F.Q4_K), 256, (2, 2, 2))]      # 6 rows in all: no quantization


@pytest.mark.parametrize("types,cols,rows", QKV_CASES)
def test_qkv_live_vs_reference(port, ref, types, cols, rows):
    """matmul_qkv_quant_f32 (src/quant.cpp:3924-3968) bit-exact against the reference build."""
    mats = [(t, synth.quant_matrix(synth.sub_seed("qkv", f"{i}{cols}"), t, r, cols), r)
            for i, (t, r) in enumerate(zip(types, rows))]
    x = synth.normal_f32(synth.sub_seed("qkv", f"x{cols}"), cols, 1.0)
    for u, v in zip(port.matmul_qkv_quant_f32(mats, x), ref.matmul_qkv_quant_f32(mats, x)):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    # the k and v rows of the first case take the Q8_0 dot as part of the q/k/v set, unlike alone
    if rows[1] < 8 and sum(rows) >= 8 and cols % 32 == 0:
        alone = port.matmul_quant_f32(types[2], mats[2][1], x, rows[2], cols) if types[2] == F.Q4_K else None
        assert alone is None or not np.array_equal(alone, port.matmul_qkv_quant_f32(mats, x)[2])


# --------------------------------------------------------------- top-k + softmax
@pytest.mark.parametrize("E,k", [(8, 2), (60, 4), (128, 8), (64, 6), (5, 5)])
def test_select_experts_bruteforce(port, E, k):
    rng = np.random.default_rng(E * 31 + k)
    for _ in range(50):
        logits = (rng.standard_normal(E) * 0.7).astype(np.float32)
        ids, probs, ties = port.select_experts(logits, k)
        assert ties == 0
        assert list(ids) == list(np.argsort(-logits.astype(np.float64), kind="stable")[:k])
        sel = logits[ids].astype(np.float64)
        p = np.exp(sel - sel.max())
        np.testing.assert_allclose(probs, p / p.sum(), rtol=2e-6)


def test_select_experts_live_vs_reference(port, ref):
    rng = np.random.default_rng(5)
    for E, k in [(8, 2), (60, 4), (128, 8), (64, 6)]:
        for _ in range(200):
            logits = (rng.standard_normal(E) * 0.5).astype(np.float32)
            a = port.select_experts(logits, k)
            b = ref.select_experts(logits, k)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))


# --------------------------------------------------------------- whole MoE block vs the golden vectors
F3_GOLDEN_CASES = ["toy_q5k_n1", "toy_q5k_n64", "toy_q6k_n1", "toy_q6k_n64", "toy_q50_n1", "toy_q50_n64",
                   "mixtral_q6k_n1", "mixtral_q6k_n512", "dsv2lite_q50_n1", "dsv2lite_q50_n32"]
ROUTER16_GOLDEN_CASES = ["toy_f16r_n1", "toy_f16r_n64", "toy_bf16r_sh_n1", "toy_bf16r_sh_n64"]
GOLDEN_CASES = F3_GOLDEN_CASES + ROUTER16_GOLDEN_CASES + ["toy_n1", "qwen15moe_n1", "qwen15moe_n64", "mixtral_n1", "mixtral_n512",
                "mixtral_n2048", "qwen3moe_n2048", "dsv2lite_n32", "toy_gelu_n1", "toy_gelu_n64",
                "toy_gelu_sh_n1", "toy_gelu_sh_n64", "toy_norm_n1_resid", "toy_norm_n64_resid"]


def _layer(name, n):
    cfg = synth.CONFIGS[name]
    return cfg, synth.make_layer(cfg), synth.make_tokens(cfg, n)


@pytest.mark.parametrize("case", GOLDEN_CASES)
def test_moe_block_golden(port, case):
    z = load(case + ".npz")
    name, n = str(z["config"]), int(z["n"])
    cfg, lw, x = _layer(name, n)
    from tests.golden.make_golden import digest, layer_digest
    assert layer_digest(lw) == str(z["layer_sha256"]), "synthetic generator drifted"
    assert digest(x) == str(z["x_sha256"]), "synthetic generator drifted"
    # routing of every token: bit-exact ids, order, probabilities and counts
    xr = np.stack([port.rms_norm(v, lw.ffn_norm, cfg.rms_eps) for v in x]) if bool(z["residual"]) else x
    lg, ids, w = port.route(lw, xr)
    assert np.array_equal(ids, z["topk_ids"])
    assert np.array_equal(w.view(np.uint32), z["topk_w"].view(np.uint32))
    assert np.array_equal(np.bincount(ids.reshape(-1), minlength=cfg.n_experts), z["counts"])
    assert int(z["counts"].sum()) == n * cfg.top_k
    # full block output for the stored rows
    out, ids_r, w_r, lg_r = port.moe_forward(lw, x, z["rows"], residual=bool(z["residual"]))
    assert np.array_equal(out.view(np.uint32), z["out"].view(np.uint32))
    assert np.array_equal(lg_r.view(np.uint32), z["logits_rows"].view(np.uint32))


@pytest.mark.parametrize("case", ["toy_n1_avx512", "qwen3moe_n2048_avx512"])
def test_moe_block_golden_avx512_order(case):
    from oracle.oracle import Oracle
    o = Oracle("port", avx512=True)
    z = load(case + ".npz")
    cfg, lw, x = _layer(str(z["config"]), int(z["n"]))
    out = o.moe_forward(lw, x, z["rows"])[0]
    assert np.array_equal(out.view(np.uint32), z["out"].view(np.uint32))


def test_moe_block_live_vs_reference(port, ref):
    """Bit-exact against the reference build on fresh seeds (small shapes of every format)."""
    for qt, E, k, d, Fd, Fs, gate, act in [(F.Q4_0, 8, 2, 512, 1024, 0, False, 0),
                                           (F.Q8_0, 16, 4, 256, 320, 0, False, 0),
                                           (F.Q4_K, 8, 3, 512, 768, 512, True, 0),
                                           (F.Q4_K, 6, 2, 256, 1408, 1408, False, 0),
                                           (F.Q4_K, 8, 2, 512, 768, 512, True, 1),
                                           (F.Q5_K, 8, 2, 512, 768, 512, True, 0),
                                           (F.Q6_K, 8, 3, 256, 640, 0, False, 1),
                                           (F.Q5_0, 8, 2, 256, 640, 320, True, 0)]:
        cfg = synth.LayerConfig(f"live{qt}_{Fd}_{act}", d, E, k, Fd, qt, d_ff_shared=Fs, shared_gate=gate, act=act)
        lw = synth.make_layer(cfg, seed=99)
        x = synth.make_tokens(cfg, 6, seed=99)
        a = port.moe_forward(lw, x)
        b = ref.moe_forward(lw, x)
        for u, v in zip(a, b):
            assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


# --------------------------------------------------------------- float64 restatement of the block
def _block_float64(port, lw, x, ids, probs):
    cfg = lw.cfg
    d, Fd, E = cfg.d_model, cfg.d_ff, cfg.n_experts
    t, td, tsd = cfg.wtype, cfg.down_t, cfg.sh_down_t
    G = deq_matrix(t, lw.gate, E * Fd, d).reshape(E, Fd, d)
    U = deq_matrix(t, lw.up, E * Fd, d).reshape(E, Fd, d)
    D = deq_matrix(td, lw.down, E * d, Fd).reshape(E, d, Fd)

    def act_in(v, qt, k):  # the activations each path uses: Q8_0 where the type allows, fp32 otherwise
        return deq_q8_blocks(port.quantize_row_q8_0(v)) if F.supports_q8_activation(qt, k) else v.astype(np.float64)

    out = np.zeros((x.shape[0], d))
    for i in range(x.shape[0]):
        xa = act_in(x[i], t, d)
        for s in range(cfg.top_k):
            e = ids[i, s]
            g, u = G[e] @ xa, U[e] @ xa
            h = ((_gelu64(g) if cfg.act else g / (1 + np.exp(-g))) * u).astype(np.float32)
            out[i] += probs[i, s] * (D[e] @ act_in(h, td, Fd))
        if cfg.has_shared:
            Fs = cfg.d_ff_shared
            g = deq_matrix(t, lw.sh_gate, Fs, d) @ xa
            u = deq_matrix(t, lw.sh_up, Fs, d) @ xa
            h = (g / (1 + np.exp(-g)) * u).astype(np.float32)  # SiLU whatever cfg.act (transformer.cpp:2741-2745)
            sh = 1.0
            if lw.sh_gate_inp is not None:
                sh = 1 / (1 + np.exp(-(lw.sh_gate_inp.astype(np.float64) @ x[i].astype(np.float64))))
            out[i] += sh * (deq_matrix(tsd, lw.sh_down, d, Fs) @ act_in(h, tsd, Fs))
    return out


@pytest.mark.parametrize("name,n", [("toy", 3), ("dsv2lite", 2), ("qwen15moe", 2), ("toy_gelu", 3), ("toy_gelu_sh", 3),
                                    ("toy_q5k", 3),
                                    ("toy_q6k", 3), ("toy_q50", 3), ("dsv2lite_q50", 2)])
def test_moe_block_float64_restatement(port, name, n):
    cfg, lw, x = _layer(name, 64 if name == "qwen15moe" else n)
    x = x[:n]
    out, ids, w, lg = port.moe_forward(lw, x)
    # the router in float64 agrees on the selection wherever the top-k margin is clear
    lg64 = x.astype(np.float64) @ lw.router.astype(np.float64).T
    for i in range(n):
        srt = np.sort(lg64[i])[::-1]
        if srt[cfg.top_k - 1] - srt[cfg.top_k] > 1e-4:
            assert set(ids[i]) == set(np.argsort(-lg64[i])[:cfg.top_k])
    ref64 = _block_float64(port, lw, x, ids, w)
    rel = np.abs(out - ref64).max(axis=1) / np.abs(ref64).max(axis=1)
    assert rel.max() < 2e-4, rel


def test_shared_expert_is_silu_in_gelu_layer(port):
    """A GELU-tanh layer's shared expert is SwiGLU: transformer.cpp:2741-2745 calls matmul_swiglu_quant_f32
    without use_gelu (default false, quant.h:361); only the routed experts take the layer's GELU (2721-2724).
    The block output must equal the routed-only output plus fma(sigmoid(gate), down(SiLU h)), and must not
    equal the same sum with GELU h, which differs here by far more than the bar."""
    cfg, lw, x = _layer("toy_gelu_sh", 4)
    from dataclasses import replace
    import copy
    routed_cfg = replace(cfg, d_ff_shared=0, shared_gate=False)
    routed_lw = copy.copy(lw)
    routed_lw.cfg, routed_lw.sh_gate, routed_lw.sh_up, routed_lw.sh_down, routed_lw.sh_gate_inp = \
        routed_cfg, None, None, None, None
    full = port.moe_forward(lw, x)[0]
    routed = port.moe_forward(routed_lw, x)[0]
    d, Fs = cfg.d_model, cfg.d_ff_shared
    for t in range(x.shape[0]):
        sh = np.float32(1.0) / (np.float32(1.0) + np.exp(-np.float32(port.vec_dot_f32(lw.sh_gate_inp, x[t]))))
        ys = {}
        for gelu in (False, True):
            h = port.matmul_swiglu_quant_f32(cfg.wtype, lw.sh_gate, cfg.wtype, lw.sh_up, x[t], Fs, d, use_gelu=gelu)
            y = port.matmul_quant_f32(cfg.sh_down_t, lw.sh_down, h, d, Fs)
            ys[gelu] = (sh.astype(np.float64) * y + routed[t]).astype(np.float32)
        assert np.array_equal(full[t].view(np.uint32), ys[False].view(np.uint32))
        gap = np.abs(ys[True] - ys[False]).max() / np.abs(ys[False]).max()
        assert gap > 1e-3, gap
