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


def test_noalloc_allocates_nothing(orc, torch_dev):
    # The promise itself: once its kernels are loaded, a call that stages
    # quantized rows (300 rows: past the fused prologue's 4) leaves the
    # device's free memory unchanged -- while a call through
    # loom_amd_dense_forward at a size its arena has not seen grows the arena,
    # which the same measurement sees -- and the call can be captured into a
    # HIP graph (global capture mode refuses allocations) whose replays, with
    # eager work and synchronizations between them, equal eager calls.
    from loom_amd import _lib, bitnet as bn
    torch = torch_dev
    n, k, M = 2560, 6912, 300
    m = orc.random_matrix(n, k, seed=21)
    w = bn.TernaryMatrix.from_words(m.words, n, k, m.scale)
    xs = [torch.from_numpy(orc.normal_f32(M * k, seed=22 + i).reshape(M, k)).cuda() for i in range(4)]
    got, _ = _noalloc(torch, w, xs[0])                 # loads the kernels, looks up the array
    want, _ = bn.dense_forward_packed_ternary(w, xs[0])
    torch.cuda.synchronize()
    assert got.cpu().numpy().tobytes() == want.cpu().numpy().tobytes()
    free0 = torch.cuda.mem_get_info()[0]
    for x in xs[1:]:
        _noalloc(torch, w, x)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0, "the no-allocation entry point allocated"
    # more rows than any other test stages through the arena (config 4's
    # 16384), so the arena grows whatever ran before in this process
    big = torch.zeros((24576, k), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    bn.dense_forward_packed_ternary(w, big)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] < free1, "the measurement does not see the arena grow"
    # graph capture of the call on fixed buffers, replayed on new inputs
    x_in = xs[0].clone()
    pre = torch.empty((M, n), dtype=torch.float32, device="cuda")
    lib = _lib.lib()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.loom_amd_dense_forward_noalloc(w.handle, C.c_void_p(x_in.data_ptr()), M, -1,
                                                C.c_void_p(pre.data_ptr()), None, None, s)
    assert rc == 0, lib.loom_amd_last_error()
    for i, x in enumerate(xs[1:] + xs[:1]):
        x_in.copy_(x)
        eager, _ = bn.dense_forward_packed_ternary(w, x)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert pre.cpu().numpy().tobytes() == eager.cpu().numpy().tobytes(), f"replay {i}"
    del g
    w.release()
