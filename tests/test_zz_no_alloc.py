"""jx_matmul_quant_f32_noalloc: the device-pointer matmul that allocates nothing
(static per-GPU scratch) against jx_matmul_quant_f32 (per-call allocation), bit
for bit: the same kernels on the same inputs.  Two calls in a row with the
second smaller, through the C ABI; a fp32-activation (Q4_K, cols % 256 != 0)
call after a wider Q8_0-activation one, so stale scratch past the new row would
show; a matrix wider than the scratch is refused before any work."""
import ctypes as C
import sys

import numpy as np
import pytest

from jxai_amd import formats as F
from jxai_amd import synth

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def moe():
    from jxai_amd import moe as M
    M.init(0)
    return M


def noalloc(moe, m, x):
    lib = moe.lib()
    xb = moe.DeviceBuffer(x.nbytes).upload(x)
    ob = moe.DeviceBuffer(m.rows * 4)
    rc = lib.jx_matmul_quant_f32_noalloc(m.handle, xb.ptr, ob.ptr, None)
    assert rc == 0, lib.jx_moe_last_error()
    assert lib.jx_device_synchronize() == 0
    out = ob.download(np.empty(m.rows, np.float32))
    xb.free()
    ob.free()
    return out


CALLS = [  # (type, rows, cols): each call smaller than the one before it
    (F.Q4_K, 512, 8192),   # Q8_0 activations, 8192 columns
    (F.Q4_K, 256, 1408),   # fp32 activations zero-padded to 1536 (scratch held 8192 columns of Q8_0)
    (F.Q4_0, 128, 1024),   # Q8_0 activations again, smaller still
]


def test_noalloc_matches_allocating_entry_point(moe, port):
    for i, (qt, rows, cols) in enumerate(CALLS):
        say(f"noalloc call {i}: type={qt} {rows}x{cols}")
        W = synth.quant_matrix(synth.sub_seed("noalloc", f"w{i}"), qt, rows, cols)
        x = synth.normal_f32(synth.sub_seed("noalloc", f"x{i}"), cols, 1.0)
        m = moe.QMatrix(qt, W, rows, cols)
        got = noalloc(moe, m, x)
        want = moe.matmul_quant_f32(qt, m, x, rows, cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {i}"
        ref = port.matmul_quant_f32(qt, W, x, rows, cols)
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
        m.close()


def test_noalloc_refuses_wide_matrix(moe):
    cols = 65536 + 256
    W = synth.quant_matrix(synth.sub_seed("noalloc", "wide"), F.Q4_0, 32, cols)
    m = moe.QMatrix(F.Q4_0, W, 32, cols)
    lib = moe.lib()
    rc = lib.jx_matmul_quant_f32_noalloc(m.handle, C.c_void_p(1), C.c_void_p(1), None)  # refused before any use
    assert rc == 2 and b"no-allocation scratch" in lib.jx_moe_last_error()
    m.close()


def _hip():
    h = C.CDLL("libamdhip64.so")
    h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
    h.hipStreamDestroy.argtypes = [C.c_void_p]
    h.hipStreamSynchronize.argtypes = [C.c_void_p]
    h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    h.hipGraphExecDestroy.argtypes = [C.c_void_p]
    h.hipGraphDestroy.argtypes = [C.c_void_p]
    h.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    return h


def test_noalloc_graph_capture_and_no_allocation(moe):
    """Captured into a HIP graph (global capture mode, where an allocation inside the call would be an
    error), replayed with new inputs and eager calls between the replays: every replay equals the eager
    call on the same input bit for bit.  Free device memory is unchanged across 200 calls."""
    h = _hip()
    lib = moe.lib()
    qt, rows, cols = F.Q4_K, 256, 4096
    W = synth.quant_matrix(synth.sub_seed("noalloc", "graph_w"), qt, rows, cols)
    m = moe.QMatrix(qt, W, rows, cols)
    xs = [synth.normal_f32(synth.sub_seed("noalloc", f"graph_x{i}"), cols, 1.0) for i in range(4)]
    xb = moe.DeviceBuffer(cols * 4).upload(xs[0])
    ob = moe.DeviceBuffer(rows * 4)
    eb = moe.DeviceBuffer(rows * 4)
    st = C.c_void_p()
    assert h.hipStreamCreate(C.byref(st)) == 0
    say("noalloc: capture into a graph")
    assert h.hipStreamBeginCapture(st, 0) == 0  # hipStreamCaptureModeGlobal
    rc = lib.jx_matmul_quant_f32_noalloc(m.handle, xb.ptr, ob.ptr, st)
    g = C.c_void_p()
    assert h.hipStreamEndCapture(st, C.byref(g)) == 0
    assert rc == 0, lib.jx_moe_last_error()
    ex = C.c_void_p()
    assert h.hipGraphInstantiate(C.byref(ex), g, None, None, 0) == 0
    for i, x in enumerate(xs):
        say(f"noalloc: replay {i}")
        xb.upload(x)
        assert lib.jx_matmul_quant_f32_noalloc(m.handle, xb.ptr, eb.ptr, st) == 0  # eager, same input
        assert h.hipStreamSynchronize(st) == 0
        want = eb.download(np.empty(rows, np.float32))
        assert h.hipGraphLaunch(ex, st) == 0
        assert h.hipStreamSynchronize(st) == 0
        got = ob.download(np.empty(rows, np.float32))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {i}"
    h.hipGraphExecDestroy(ex)
    h.hipGraphDestroy(g)
    say("noalloc: free memory across 200 calls")
    free0, free1, total = C.c_size_t(), C.c_size_t(), C.c_size_t()
    assert h.hipStreamSynchronize(st) == 0
    assert h.hipMemGetInfo(C.byref(free0), C.byref(total)) == 0
    for _ in range(200):
        assert lib.jx_matmul_quant_f32_noalloc(m.handle, xb.ptr, ob.ptr, st) == 0
    assert h.hipStreamSynchronize(st) == 0
    assert h.hipMemGetInfo(C.byref(free1), C.byref(total)) == 0
    assert free1.value == free0.value
    h.hipStreamDestroy(st)
    for b in (xb, ob, eb):
        b.free()
    m.close()
