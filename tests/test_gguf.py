"""The GGUF loader (jx_gguf_*) against the reference's own parser, ModelFile::open
(src/gguf.cpp, built into oracle/_ref): the reference's toy model file
models/qwen_run.gguf when the reference tree is present, and files written here
with edge-case metadata, shared experts, a dense FFN, another alignment, and
broken headers.  Then the layer binding of bind_tensors (transformer.cpp:2116-2199)."""
import ctypes as C
import os

import numpy as np
import pytest

from jxai_amd import formats as F
from jxai_amd import synth
from tests import gguf_writer as W

TOY = "/root/reference/models/qwen_run.gguf"


@pytest.fixture(scope="module")
def gg():
    from jxai_amd import _lib, gguf
    if not os.path.exists(_lib.LIB_PATH):
        from jxai_amd import build
        build.build(verbose=False)
    return gguf


class RefParser:
    """ModelFile through the reference build's jxr_gguf_* exports."""

    def __init__(self, ref, path):
        L = self.L = ref.lib
        L.jxr_gguf_open.restype = C.c_void_p
        L.jxr_gguf_open.argtypes = [C.c_char_p]
        L.jxr_gguf_close.argtypes = [C.c_void_p]
        L.jxr_gguf_tensor_count.restype = C.c_int64
        L.jxr_gguf_tensor_count.argtypes = [C.c_void_p]
        L.jxr_gguf_tensor_name.restype = C.c_char_p
        L.jxr_gguf_tensor_name.argtypes = [C.c_void_p, C.c_int64]
        L.jxr_gguf_tensor.restype = C.c_int32
        L.jxr_gguf_tensor.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                      C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
        L.jxr_gguf_get_u32.restype = C.c_uint32
        L.jxr_gguf_get_u32.argtypes = [C.c_void_p, C.c_char_p, C.c_uint32]
        L.jxr_gguf_get_f32.restype = C.c_float
        L.jxr_gguf_get_f32.argtypes = [C.c_void_p, C.c_char_p, C.c_float]
        self.h = L.jxr_gguf_open(path.encode())

    def ok(self):
        return bool(self.h)

    def tensors(self):
        out = {}
        for i in range(self.L.jxr_gguf_tensor_count(self.h)):
            name = self.L.jxr_gguf_tensor_name(self.h, i)
            t, nd = C.c_int32(), C.c_int32()
            dims = (C.c_uint64 * 4)()
            off, nb = C.c_uint64(), C.c_uint64()
            assert self.L.jxr_gguf_tensor(self.h, name, C.byref(t), C.byref(nd), dims, C.byref(off), C.byref(nb)) == 0
            out[name.decode()] = {"type": t.value, "n_dims": nd.value, "dims": list(dims), "offset": off.value,
                                  "bytes": nb.value}
        return out

    def close(self):
        if self.h:
            self.L.jxr_gguf_close(self.h)


def compare(gg, ref, path, keys):
    mine = gg.GGUFFile(path)
    theirs = RefParser(ref, path)
    assert theirs.ok()
    a = {n: {k: t[k] for k in ("type", "n_dims", "dims", "offset", "bytes")} for n, t in mine.tensors().items()}
    assert a == theirs.tensors()
    assert [mine.tensor(i)["name"] for i in range(mine.tensor_count())] == list(theirs.tensors())  # file order
    for key in keys:
        assert mine.get_u32(key, 77) == theirs.L.jxr_gguf_get_u32(theirs.h, key.encode(), 77), key
        assert mine.get_f32(key, 0.5) == theirs.L.jxr_gguf_get_f32(theirs.h, key.encode(), 0.5), key
    theirs.close()
    return mine


def test_toy_model_file(gg, ref):
    """models/qwen_run.gguf (the reference's forge toy, src/model_forge.cpp:135-339): 43 tensors in
    1,328,288 bytes, everything as ModelFile reads it; layer 0: router F32 [128, 8], Q4_0 experts
    [128, 128, 8]."""
    if not os.path.exists(TOY):
        pytest.skip("the reference tree is not present")
    assert os.path.getsize(TOY) == 1328288
    keys = ["qwen2moe.embedding_length", "qwen2moe.expert_count", "qwen2moe.expert_used_count",
            "qwen2moe.expert_feed_forward_length", "qwen2moe.block_count", "general.alignment",
            "qwen2moe.attention.layer_norm_rms_epsilon", "qwen2moe.rope.freq_base", "no.such.key",
            "general.architecture", "tokenizer.ggml.scores"]
    f = compare(gg, ref, TOY, keys)
    assert f.tensor_count() == 43
    t = f.tensors()
    assert t["blk.0.ffn_gate_inp.weight"]["dims"][:2] == [128, 8] and t["blk.0.ffn_gate_inp.weight"]["type"] == F.F32
    for p in ("gate", "up", "down"):
        assert t[f"blk.0.ffn_{p}_exps.weight"]["dims"][:3] == [128, 128, 8]
        assert t[f"blk.0.ffn_{p}_exps.weight"]["type"] == F.Q4_0
    for layer in range(4):
        d = f.layer_desc(layer)
        assert (d.n_experts, d.top_k, d.d_model, d.d_ff) == (8, 2, 128, 128)
        assert d.gate_exps == t[f"blk.{layer}.ffn_gate_exps.weight"]["data"]
        assert d.down_exps == t[f"blk.{layer}.ffn_down_exps.weight"]["data"]
        assert d.router == t[f"blk.{layer}.ffn_gate_inp.weight"]["data"]
        assert d.d_ff_shared == 0 and d.activation == 0 and d.router_type == F.F32
    f.close()


def _moe_file(path, arch="qwen2moe", shared=True, version=3, alignment=32, dense=False, extra_meta=()):
    d, E, k, Fd, Fs = 256, 4, 2, 512, 256
    cfg = synth.LayerConfig("gguf_t", d, E, k, Fd, F.Q4_K, d_ff_shared=Fs, shared_gate=True)
    lw = synth.make_layer(cfg, seed=11)
    meta = [("general.architecture", W.STR, arch), ("general.alignment", W.U32, alignment),
            (f"{arch}.expert_used_count", W.U32, k), (f"{arch}.expert_count", W.U32, E),
            (f"{arch}.attention.layer_norm_rms_epsilon", W.F32, 1e-6), ("x.i8", W.I8, -3), ("x.u16", W.U16, 513),
            ("x.i64", W.I64, -5), ("x.f64", W.F64, 0.25), ("x.bool", W.BOOL, True),
            ("x.strs", W.ARR, (W.STR, ["a", "bc", ""])), ("x.u8s", W.ARR, (W.U8, [1, 2, 3])),
            ("x.nested", W.ARR, (W.ARR, [(W.I32, [1, 2]), (W.F32, [0.5])]))] + list(extra_meta)
    tens = [("token_embd.weight", [d, 8], F.F32, np.zeros(d * 8 * 4, np.uint8)),
            ("blk.0.ffn_norm.weight", [d], F.F32, np.ones(d, np.float32).view(np.uint8))]
    if dense:
        tens += [("blk.0.ffn_gate.weight", [d, Fd], F.Q4_K, lw.gate[: lw.gate.size // E]),
                 ("blk.0.ffn_up.weight", [d, Fd], F.Q4_K, lw.up[: lw.up.size // E]),
                 ("blk.0.ffn_down.weight", [Fd, d], F.Q4_K, lw.down[: lw.down.size // E])]
    else:
        tens += [("blk.0.ffn_gate_inp.weight", [d, E], F.F32, lw.router.view(np.uint8)),
                 ("blk.0.ffn_gate_exps.weight", [d, Fd, E], F.Q4_K, lw.gate),
                 ("blk.0.ffn_up_exps.weight", [d, Fd, E], F.Q4_K, lw.up),
                 ("blk.0.ffn_down_exps.weight", [Fd, d, E], F.Q4_K, lw.down)]
    if shared:
        tens += [("blk.0.ffn_gate_shexp.weight", [d, Fs], F.Q4_K, lw.sh_gate),
                 ("blk.0.ffn_up_shexp.weight", [d, Fs], F.Q4_K, lw.sh_up),
                 ("blk.0.ffn_down_shexp.weight", [Fs, d], F.Q4_K, lw.sh_down),
                 ("blk.0.ffn_gate_inp_shexp.weight", [d], F.F32, lw.sh_gate_inp.view(np.uint8))]
    W.write_gguf(path, meta, tens, version=version, alignment=alignment)
    return lw


KEYS = ["x.i8", "x.u16", "x.i64", "x.f64", "x.bool", "x.strs", "gemma2.expert_used_count",
        "qwen2moe.expert_used_count", "general.alignment", "qwen2moe.attention.layer_norm_rms_epsilon"]


@pytest.mark.parametrize("version,alignment", [(3, 32), (2, 64), (3, 256)])
def test_written_files_match_reference(gg, ref, tmp_path, version, alignment):
    path = str(tmp_path / "m.gguf")
    lw = _moe_file(path, version=version, alignment=alignment)
    f = compare(gg, ref, path, KEYS)
    d = f.layer_desc(0)
    assert (d.n_experts, d.top_k, d.d_model, d.d_ff, d.d_ff_shared) == (4, 2, 256, 512, 256)
    assert d.gate_type == F.Q4_K and d.sh_down_type == F.Q4_K and d.activation == 0
    got = np.ctypeslib.as_array((C.c_uint8 * lw.down.size).from_address(d.down_exps))
    assert np.array_equal(got, lw.down)
    sg = np.ctypeslib.as_array((C.c_float * 256).from_address(C.cast(d.sh_gate_inp, C.c_void_p).value))
    assert np.array_equal(sg, lw.sh_gate_inp)
    f.close()


def test_gemma_gates_with_gelu_and_dense_ffn_is_one_expert(gg, ref, tmp_path):
    path = str(tmp_path / "g.gguf")
    _moe_file(path, arch="gemma2", shared=False)
    f = compare(gg, ref, path, KEYS)
    assert f.layer_desc(0).activation == 1
    f.close()
    path2 = str(tmp_path / "dense.gguf")
    _moe_file(path2, shared=False, dense=True)
    f = compare(gg, ref, path2, KEYS)
    d = f.layer_desc(0)
    assert (d.n_experts, d.top_k, d.d_ff) == (1, 1, 512)
    assert not np.any(np.ctypeslib.as_array((C.c_float * 256).from_address(C.cast(d.router, C.c_void_p).value)))
    f.close()


def test_broken_files_are_refused_like_the_reference(gg, ref, tmp_path):
    path = str(tmp_path / "ok.gguf")
    _moe_file(path, shared=False)
    raw = open(path, "rb").read()
    cases = {"magic": b"GGUX" + raw[4:], "version": raw[:4] + (4).to_bytes(4, "little") + raw[8:],
             "header": raw[:20], "metadata": raw[:120], "table": raw[:raw.index(b"blk.0.ffn_up_exps") + 8],
             "data": raw[:-100]}
    for name, blob in cases.items():
        p = str(tmp_path / f"{name}.gguf")
        open(p, "wb").write(blob)
        with pytest.raises(gg.JxError):
            gg.GGUFFile(p)
        assert not RefParser(ref, p).ok(), name


def test_missing_layer_is_refused(gg, tmp_path):
    path = str(tmp_path / "m.gguf")
    _moe_file(path, shared=False)
    f = gg.GGUFFile(path)
    with pytest.raises(gg.JxError, match="no FFN tensors"):
        f.layer_desc(3)
    f.close()


def fixture_file(path):
    """A GGUF file holding layer 0 of the reference's toy model, rebuilt from the committed fixture."""
    from tests.conftest import GOLDEN
    z = np.load(os.path.join(GOLDEN, "qwen_run_layer0.npz"), allow_pickle=False)
    arch = str(z["arch"])
    meta = [("general.architecture", W.STR, arch), (f"{arch}.expert_used_count", W.U32, int(z["top_k"])),
            (f"{arch}.expert_count", W.U32, int(z["n_experts"])),
            (f"{arch}.attention.layer_norm_rms_epsilon", W.F32, float(z["eps"]))]
    tens = [(str(z[f"t{i}_name"]), [int(v) for v in z[f"t{i}_dims"]], int(z[f"t{i}_type"]), z[f"t{i}_bytes"])
            for i in range(int(z["n_tensors"]))]
    W.write_gguf(path, meta, tens)
    return z


def test_toy_layer0_fixture_on_the_oracle(gg, port, tmp_path):
    """The fixture's bytes bound through the loader give the reference build's outputs through the
    oracle bit for bit (routing and outputs of all 64 tokens)."""
    path = str(tmp_path / "l0.gguf")
    z = fixture_file(path)
    f = gg.GGUFFile(path)
    d = f.layer_desc(0)
    assert (d.n_experts, d.top_k, d.d_model, d.d_ff) == (8, 2, 128, 128)
    cfg = synth.LayerConfig("l0", 128, 8, 2, 128, F.Q4_0)
    rd = lambda p, n, t: np.ctypeslib.as_array((t * n).from_address(C.cast(p, C.c_void_p).value)).copy()  # noqa: E731
    lw = synth.LayerWeights(cfg, rd(d.router, 1024, C.c_float).reshape(8, 128), None,
                            rd(d.gate_exps, 73728, C.c_uint8), rd(d.up_exps, 73728, C.c_uint8),
                            rd(d.down_exps, 73728, C.c_uint8))
    out, ids, w, lg = port.moe_forward(lw, z["x"])
    assert np.array_equal(ids, z["topk_ids"]) and np.array_equal(w.view(np.uint32), z["topk_w"].view(np.uint32))
    assert np.array_equal(out.view(np.uint32), z["out"].view(np.uint32))
    f.close()
