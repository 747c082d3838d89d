"""The C-ABI library builds, loads and exports every entry point of
include/jxmoe.h; host-side argument checks work without a GPU."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "jxmoe.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def jxlib():
    from jxai_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from jxai_amd import build
        build.build(verbose=False)
    return _lib.lib()


def test_header_lists_the_bound_symbols():
    from jxai_amd import _lib
    assert header_symbols() == sorted(_lib.EXPORTS)


def test_library_exports_every_header_symbol(jxlib):
    for s in header_symbols():
        assert hasattr(jxlib, s), s


def test_errors_without_device_or_init(jxlib):
    from jxai_amd import _lib
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present; the no-device path is not reachable")
    assert jxlib.jx_moe_init(0) == 5  # JX_ERR_NODEVICE
    assert b"device" in jxlib.jx_moe_last_error()
    # layer creation before init is refused, not crashed
    D = _lib.LayerDesc()
    h = C.c_void_p()
    assert jxlib.jx_moe_layer_create(C.byref(D), C.byref(h)) == 5
    # null arguments are rejected on the host side
    assert jxlib.jx_moe_forward(None, None, 1, None, None, None, None, None, 0) == 1
    assert jxlib.jx_quantize_row_q8_0(None, None, 32) == 1
    x = np.zeros(31, np.float32)
    out = np.zeros(34, np.uint8)
    assert jxlib.jx_quantize_row_q8_0(C.c_void_p(x.ctypes.data), C.c_void_p(out.ctypes.data), 31) == 1


def test_python_mirror_fails_loudly_without_library(monkeypatch, tmp_path):
    from jxai_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.JxError, match="no CPU fallback"):
        _lib.lib()


def build_caller(out_dir) -> str:
    """g++ build of tests/abi_caller.cpp against include/jxmoe.h and libjxmoe.so."""
    from jxai_amd import _lib
    exe = os.path.join(str(out_dir), "abi_caller")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "abi_caller.cpp"), "-o", exe, _lib.LIB_PATH,
                    "-Wl,-rpath," + os.path.dirname(_lib.LIB_PATH)], check=True)
    return exe


def test_compiled_caller_without_device(jxlib, tmp_path):
    """A C++ program that sees only include/jxmoe.h compiles, links and gets JX_ERR_NODEVICE here."""
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present; the no-device path is not reachable")
    exe = build_caller(tmp_path)
    r = subprocess.run([exe, "nodevice"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "-> 5" in r.stdout
