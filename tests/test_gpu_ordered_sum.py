"""The library's wave-parallel form of the reference's sequential fp64 sum.

loom forms every sum of squares (and the softmax exp sums) as one left-to-right
fp64 chain, `sumSq += f * f` (poly/bitnet_cpu.go:901-905, poly/norm.go,
poly/mha.go).  The strict norm kernels form that chain with a whole wavefront
(exact integer arithmetic in units of the running sum's ulp, half-ulp ties
resolved from the running parity); `loom_amd_ordered_sum_rows` exposes it.

Bar: bit-exact against the sequential chain (numpy's `add.accumulate`, which
adds strictly left to right; pinned below against a Python loop), on rows built
to hit each branch: half-ulp ties, binade crossings, zero runs, tiny and huge
running sums, negative terms, NaN and Inf.
"""
import ctypes as C

import numpy as np
import pytest


def sequential(t, s0):
    """s0 + t[:, 0] + t[:, 1] + ... row by row, one rounding per addition."""
    t = np.asarray(t, np.float64)
    full = np.concatenate([np.full((t.shape[0], 1), s0, np.float64), t], axis=1)
    return np.add.accumulate(full, axis=1)[:, -1]


def test_checker_is_the_sequential_chain():
    rng = np.random.default_rng(7)
    t = np.concatenate([rng.standard_normal((3, 300)) ** 2,
                        rng.integers(0, 9, (3, 300)) * 0.5,
                        np.exp(-rng.random((3, 300)) * 40)])
    t[:, 0] = 1.0 + 2.0 ** -51
    for s0 in (0.0, 1.5):
        want = []
        for row in t:
            s = s0
            for v in row:
                s = s + float(v)
            want.append(s)
        got = sequential(t, s0)
        assert np.array_equal(np.array(want).view(np.uint64), got.view(np.uint64))
    # the chain is not the pairwise or exactly rounded sum on these rows
    assert not np.array_equal(sequential(t, 0.0), t.sum(axis=1))


def rows_of_kind(kind, n, rng, m=8):
    if kind == "squares":
        x = rng.standard_normal((m, n)).astype(np.float32)
        return x.astype(np.float64) ** 2
    if kind == "squares_wide_range":
        x = (rng.standard_normal((m, n)) * np.exp(rng.uniform(-30, 30, (m, n)))).astype(np.float32)
        return x.astype(np.float64) ** 2
    if kind == "squares_fine":  # 20-bit fractions: many half-ulp ties
        return (rng.integers(1, 2 ** 20, (m, n)).astype(np.float64) * 2.0 ** -20) ** 2
    if kind == "integers":
        return rng.integers(0, 5, (m, n)).astype(np.float64)
    if kind == "halves":
        return rng.integers(0, 9, (m, n)).astype(np.float64) * 0.5
    if kind == "powers_of_two":
        return 2.0 ** rng.integers(-60, 60, (m, n)).astype(np.float64)
    if kind == "ties":  # a running sum of 1 + 2^-51 followed by half-ulp terms
        t = np.full((m, n), 2.0 ** -52)
        t[:, 0] = 1.0 + 2.0 ** -51
        return t
    if kind == "sparse":
        t = np.zeros((m, n))
        for r in range(m):
            t[r, rng.integers(0, n, 3)] = rng.random(3)
        return t
    if kind == "zeros":
        return np.zeros((m, n))
    if kind == "nan":
        t = rng.random((m, n))
        t[np.arange(m), rng.integers(0, n, m)] = np.nan
        return t
    if kind == "inf":
        t = rng.random((m, n))
        t[np.arange(m), rng.integers(0, n, m)] = np.inf
        return t
    if kind == "mixed_sign":
        return rng.standard_normal((m, n))
    if kind == "tiny":
        return rng.random((m, n)) * 1e-300
    if kind == "huge":
        return rng.random((m, n)) * 1e300
    if kind == "exps":
        return np.exp(-rng.random((m, n)) * 40)
    raise ValueError(kind)


KINDS = ["squares", "squares_wide_range", "squares_fine", "integers", "halves",
         "powers_of_two", "ties", "sparse", "zeros", "nan", "inf", "mixed_sign", "tiny",
         "huge", "exps"]
WIDTHS = [1, 5, 63, 64, 65, 255, 256, 257, 1000, 2560, 6912, 8064]


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from loom_amd import _lib
    assert _lib.lib().loom_amd_device_count() >= 1, "no gfx950 device visible to the library"
    return torch


def gpu_ordered_sums(torch, t, s0, threads):
    from loom_amd import _lib
    lib = _lib.lib()
    td = torch.from_numpy(np.ascontiguousarray(t, np.float64)).cuda()
    out = torch.empty(t.shape[0], dtype=torch.float64, device="cuda")
    rc = lib.loom_amd_ordered_sum_rows(C.c_void_p(td.data_ptr()), t.shape[0], t.shape[1],
                                       C.c_double(s0), C.c_void_p(out.data_ptr()), threads, None)
    assert rc == 0, lib.loom_amd_last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def same_bits(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    both_nan = np.isnan(a) & np.isnan(b)
    return np.all(both_nan | (a.view(np.uint64) == b.view(np.uint64)))


@pytest.mark.gpu
@pytest.mark.parametrize("threads", [64, 256, 512])
@pytest.mark.parametrize("kind", KINDS)
def test_ordered_sum_rows_bit_exact(torch_dev, kind, threads):
    rng = np.random.default_rng(101 + KINDS.index(kind))
    for n in WIDTHS:
        t = rows_of_kind(kind, n, rng)
        for s0 in (0.0, 1.5, -2.0, 1e-310):
            got = gpu_ordered_sums(torch_dev, t, s0, threads)
            want = sequential(t, s0)
            bad = np.nonzero(~(np.isnan(got) & np.isnan(want))
                             & (got.view(np.uint64) != want.view(np.uint64)))[0]
            assert bad.size == 0, (kind, n, s0, bad[:4], got[bad[:4]], want[bad[:4]])


@pytest.mark.gpu
def test_ordered_sum_rows_many_rows(torch_dev):
    # BitNet-2B widths, 512 rows each (the strict norms' inputs: fp32 squares)
    rng = np.random.default_rng(3)
    for n in (2560, 6912):
        x = (rng.standard_normal((512, n)) * rng.uniform(0.01, 10, (512, 1))).astype(np.float32)
        t = x.astype(np.float64) ** 2
        for threads in (64, 256, 512):
            assert same_bits(gpu_ordered_sums(torch_dev, t, 0.0, threads), sequential(t, 0.0))


@pytest.mark.gpu
def test_ordered_sum_rows_rejects_bad_shapes(torch_dev):
    from loom_amd import _lib
    lib = _lib.lib()
    torch = torch_dev
    buf = torch.zeros(8065, dtype=torch.float64, device="cuda")
    out = torch.zeros(1, dtype=torch.float64, device="cuda")
    p, o = C.c_void_p(buf.data_ptr()), C.c_void_p(out.data_ptr())
    assert lib.loom_amd_ordered_sum_rows(p, 1, 8065, C.c_double(0.0), o, 256, None) == -1
    assert b"8064" in lib.loom_amd_last_error()
    assert lib.loom_amd_ordered_sum_rows(p, 1, 0, C.c_double(0.0), o, 256, None) == -1
    assert lib.loom_amd_ordered_sum_rows(None, 1, 4, C.c_double(0.0), o, 256, None) == -1
    assert lib.loom_amd_ordered_sum_rows(p, 1, 4, C.c_double(0.0), o, 128, None) == -1
    assert lib.loom_amd_ordered_sum_rows(p, 0, 4, C.c_double(0.0), o, 256, None) == 0
