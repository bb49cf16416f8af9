"""CPU-side checks of libloom_accel_amd.so: it loads, exports every symbol the
headers declare, and honours loom's plugin-loader contract without a GPU
(poly/accel/plugin_linux.go:45-92, 184-212; error handling as
accel/apple/src/loom_accel_apple.cpp:145-205).  No compute runs here.
"""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    names = []
    for h in ("loom_accel.h", "loom_accel_amd.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(loom_(?:accel|amd)_\w+)\s*\(", text)
    return sorted(set(names))


def gpu_visible() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def test_library_exports_every_declared_symbol(amd_lib):
    syms = header_symbols()
    assert len(syms) >= 12 + 14
    for name in syms:
        assert hasattr(amd_lib, name), f"{name} declared in include/ but not exported"
    from loom_amd import _lib
    assert set(syms) == set(_lib.SIGNATURES), "ctypes signature table out of sync with headers"


def test_v2_identity(amd_lib):
    assert amd_lib.loom_accel_api_version() == 2
    assert amd_lib.loom_accel_vendor_id() == b"amd"
    assert amd_lib.loom_accel_npu_available() in (0, 1)


def test_open_errors(amd_lib):
    assert not amd_lib.loom_accel_plugin_open(b"CPU")
    assert b"CPU" in amd_lib.loom_accel_last_error(None)
    assert not amd_lib.loom_accel_plugin_open(b"TPU")
    assert b"unknown device" in amd_lib.loom_accel_last_error(None)
    if not gpu_visible():
        assert not amd_lib.loom_accel_plugin_open(b"GPU")
        assert b"gfx950" in amd_lib.loom_accel_last_error(None)


def test_weight_bytes_contract(amd_lib):
    from loom_amd import _lib

    def wb(name, dtype, label):
        d = _lib.LayerDesc(name.encode(), dtype.encode(), label.encode())
        return amd_lib.loom_accel_weight_bytes(C.byref(d))

    assert wb("BitNetLinear", "TERNARY", "m=1,k=2560,n=6912") == 24 + 6912 * 160 * 4
    assert wb("BitNetLinear", "TERNARY", "m=3,k=17,n=3") == 24 + 3 * 2 * 4
    assert wb("BitNetSwiGLU", "TERNARY", "m=1,k=2560,n=6912") == (
        2 * (24 + 6912 * 160 * 4) + 24 + 2560 * 432 * 4 + 6912 * 4)
    # bias=1: the Master-tail biases [gate | up | down] follow the norm weights
    assert wb("BitNetSwiGLU", "TERNARY", "m=1,k=2560,n=6912,bias=1") == (
        2 * (24 + 6912 * 160 * 4) + 24 + 2560 * 432 * 4 + 6912 * 4 + (2 * 6912 + 2560) * 4)
    assert wb("BitNetSwiGLU", "TERNARY", "m=1,k=2560,n=6912,bias=0") == wb(
        "BitNetSwiGLU", "TERNARY", "m=1,k=2560,n=6912")
    for bad in [("Dense", "TERNARY", "m=1,k=4,n=4"), ("BitNetLinear", "INT8", "m=1,k=4,n=4"),
                ("BitNetLinear", "TERNARY", "medium"), ("BitNetLinear", "TERNARY", "m=1,k=4"),
                ("BitNetLinear", "TERNARY", "m=0,k=4,n=4"), ("BitNetLinear", "TERNARY",
                                                             "m=1,k=4,n=4,norm=loose"),
                ("BitNetLinear", "TERNARY", "m=1,k=4,n=4,bias=1"),  # loom's Dense has no bias
                ("BitNetSwiGLU", "TERNARY", "m=1,k=4,n=4,bias=2")]:
        assert wb(*bad) == 0, bad
    assert amd_lib.loom_accel_weight_bytes(None) == 0


def test_amd_extension_errors_without_gpu(amd_lib):
    if gpu_visible():
        pytest.skip("checks the no-device path")
    assert amd_lib.loom_amd_device_count() == 0
    out = C.c_void_p()
    words = (C.c_uint32 * 4)()
    assert amd_lib.loom_amd_matrix_create(0, words, 4, 1, 64, 4, 1.0, C.byref(out)) == -1
    assert b"not visible" in amd_lib.loom_amd_last_error()
    assert amd_lib.loom_amd_kernel_variant(1) == b"skinny_m16_fusedq"
    assert amd_lib.loom_amd_kernel_variant(5) == b"skinny_m16_fusedq"
    assert amd_lib.loom_amd_kernel_variant(8) == b"skinny_m16_fusedq"
    assert amd_lib.loom_amd_kernel_variant(9) == b"skinny_m16"
    assert amd_lib.loom_amd_kernel_variant(56) == b"skinny_m64"
    assert amd_lib.loom_amd_kernel_variant(64) == b"gemm_m64"
    assert amd_lib.loom_amd_kernel_variant(65) == b"gemm"


def test_python_accel_mirror_refuses_cpu(amd_lib):
    from loom_amd import accel
    with pytest.raises(accel.AccelError, match="open device CPU"):
        accel.open_amd(device="CPU")
    with pytest.raises(accel.ErrUnavailable):
        accel.open_amd(path="/nonexistent/libloom_accel_amd.so")
    assert accel.npu_available() == gpu_visible()


def test_c_loader_conformance(amd_lib, tmp_path):
    from loom_amd import _lib
    exe = tmp_path / "abi_conformance"
    subprocess.run(["gcc", "-O1", "-Wall", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "abi_conformance.c"), "-o", str(exe), "-ldl"],
                   check=True)
    proc = subprocess.run([str(exe), _lib.LIB_PATH, "1" if gpu_visible() else "0"],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_drift_spectrum_classifier():
    # classifyDrift's buckets (lucy/examples/apple/spectrum.go:37-58) at and
    # either side of each edge; maxAbsDiffTensor's NaN rule and size mismatch
    # (lucy/examples/apple/dispatch.go:205-238)
    import numpy as np
    from tests import spectrum as sp
    tol = 1e-7
    cases = [(0.0, sp.EXACT), (5e-8, sp.INDUS), (1e-7, sp.INDUS), (1.0000001e-7, sp.LOWBIT),
             (1e-6, sp.LOWBIT), (1.01e-6, sp.DRIFT), (0.1, sp.DRIFT), (0.10001, sp.H_DRIFT),
             (1.0, sp.H_DRIFT), (1.5, sp.BROKE), (float("nan"), sp.FATAL),
             (float("inf"), sp.FATAL)]
    for diff, want in cases:
        assert sp.classify(diff, tol) == want, (diff, sp.LABELS[want])
    assert sp.infer_tolerance("FP32") == 1e-7 and sp.infer_tolerance("TERNARY") == 1e-7
    assert sp.gpu_parity_tolerance("FP32") == 0.1
    a = np.array([1.0, np.nan, 3.0], np.float32)
    b = np.array([1.0, 2.0, 3.5], np.float32)
    assert sp.max_abs_diff(a, b) == 0.5          # NaN difference skipped
    assert sp.max_abs_diff(a, b[:2]) == np.finfo(np.float64).max
    assert sp.histogram(a, b, tol) == [1, 0, 0, 0, 1, 0, 1]
