"""loom_amd_dense_forward_noalloc (no counterpart in loom: for callers that
cannot allocate device memory) against loom_amd_dense_forward and the oracle,
through the C ABI.

Bar: bit-exact fp32 outputs (the same kernels; the quantized rows are staged
in the library's fixed per-GPU array instead of its scratch arena), on two
calls in a row, the second with a smaller input, so the second call reuses the
array the first one filled.  Calls past the array's size fail with a message.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from loom_amd import _lib
    assert _lib.lib().loom_amd_device_count() >= 1, "no gfx950 device visible to the library"
    return torch


def _noalloc(torch, w, x, activation=-1, residual=None):
    from loom_amd import _lib
    m = x.shape[0]
    pre = torch.full((m, w.rows), float("nan"), dtype=torch.float32, device="cuda")
    post = torch.full((m, w.rows), float("nan"), dtype=torch.float32, device="cuda")
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = _lib.lib().loom_amd_dense_forward_noalloc(
        w.handle, C.c_void_p(x.data_ptr()), m, activation, C.c_void_p(pre.data_ptr()),
        C.c_void_p(post.data_ptr()) if activation != -1 else None,
        C.c_void_p(residual.data_ptr()) if residual is not None else None, s)
    if rc != 0:
        raise _lib.AMDError(_lib.lib().loom_amd_last_error().decode())
    torch.cuda.synchronize()
    return pre, post


@pytest.mark.parametrize("shape,rows", [((6912, 2560), (300, 40)), ((2560, 6912), (130, 65)),
                                        ((384, 640), (8, 3)), ((1000, 2570), (77, 5))])
def test_noalloc_equals_dense_forward(orc, torch_dev, shape, rows):
    # two calls in a row on the same GPU: the second (fewer rows) reuses the
    # fixed array the first one filled
    from loom_amd import bitnet as bn
    torch = torch_dev
    n, k = shape
    m = orc.random_matrix(n, k, seed=n + k)
    w = bn.TernaryMatrix.from_words(m.words, n, k, m.scale)
    for i, M in enumerate(rows):
        x = orc.normal_f32(M * k, seed=100 * i + M).reshape(M, k)
        xd = torch.from_numpy(x).cuda()
        got, _ = _noalloc(torch, w, xd)
        want, _ = bn.dense_forward_packed_ternary(w, xd)
        torch.cuda.synchronize()
        assert got.cpu().numpy().tobytes() == want.cpu().numpy().tobytes(), (shape, M)
        ref = orc.dense_forward(m, x, simd=True)
        assert got.cpu().numpy().tobytes() == ref.pre.tobytes(), (shape, M)
    w.release()


def test_noalloc_activation_and_residual(orc, torch_dev):
    from loom_amd import bitnet as bn
    torch = torch_dev
    n, k, M = 512, 768, 100
    m = orc.random_matrix(n, k, seed=7)
    w = bn.TernaryMatrix.from_words(m.words, n, k, m.scale)
    x = torch.from_numpy(orc.normal_f32(M * k, seed=8).reshape(M, k)).cuda()
    r = torch.from_numpy(orc.normal_f32(M * n, seed=9).reshape(M, n)).cuda()
    for act in (0, 1, 2, 3, 4, 5, 6):  # every Activate id (poly/poly.go:90-97): same kernels, same bytes
        got_pre, got_post = _noalloc(torch, w, x, activation=act, residual=r)
        want_pre, want_post = bn.dense_forward_packed_ternary(w, x, activation=act, residual=r)
        torch.cuda.synchronize()
        assert got_pre.cpu().numpy().tobytes() == want_pre.cpu().numpy().tobytes()
        assert got_post.cpu().numpy().tobytes() == want_post.cpu().numpy().tobytes()
    w.release()


def test_noalloc_refuses_more_than_its_array(orc, torch_dev):
    from loom_amd import _lib, bitnet as bn
    torch = torch_dev
    n, k = 64, 6912
    m = orc.random_matrix(n, k, seed=11)
    w = bn.TernaryMatrix.from_words(m.words, n, k, m.scale)
    def need(M):  # int8 rows, amax and sum(xq), each 256-byte aligned
        def a(b):
            return (b + 255) // 256 * 256
        return a(M * bn.padded_cols(k)) + 2 * a(4 * M)

    fit = max(M for M in range(1, 2000) if need(M) <= 8 << 20)
    assert need(fit + 1) > 8 << 20
    x = torch.zeros((fit + 1, k), dtype=torch.float32, device="cuda")
    with pytest.raises(_lib.AMDError, match="more than the fixed"):
        _noalloc(torch, w, x)
    # the largest call that fits still runs, and matches the oracle on sampled rows
    M = fit
    xs = orc.normal_f32(M * k, seed=12).reshape(M, k)
    got, _ = _noalloc(torch, w, torch.from_numpy(xs).cuda())
    rows = [0, M // 2, M - 1]
    ref = orc.dense_forward(m, xs[rows], simd=True)
    assert got.cpu().numpy()[rows].tobytes() == ref.pre.tobytes()
    w.release()
