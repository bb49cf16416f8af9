"""Parity of the gfx950 HIP path against the CPU oracle (loom's CPU path restated).

Bar (stated per test):
  * int8 activations, per-row amax, int32 accumulators: bit-exact;
  * fp32 Dense outputs: bit-exact -- the rescale is loom's fp64 multiply in its
    operation order, then one fp64 -> fp32 rounding;
  * SwiGLU: every integer stage bit-exact; the gate product uses exp(), whose
    last fp64 bit differs between libraries (Go math.Exp, glibc, ROCm ocml), so
    the normalized rows h are compared within 1 fp32 ulp and the stages after
    h are checked bit-exact against the oracle fed the GPU's own h.
Citations are relative to the loom v0.83.0 tree.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# loom's parity shapes rows x cols (poly/tests/bitnet_packed_test.go:19-21,
# poly/tests/bitnet_cpu_test.go:217) plus the BitNet-2B FFN shapes.
LOOM_SHAPES = [(40, 70), (8, 64), (33, 65), (16, 128), (64, 2560), (128, 6912), (7, 191), (3, 17)]
M_EDGES = [1, 2, 4, 5, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200]


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from loom_amd import _lib
    assert _lib.lib().loom_amd_device_count() >= 1, "no gfx950 device visible to the library"
    return torch


@pytest.fixture(scope="module")
def bn(torch_dev):
    from loom_amd import bitnet
    return bitnet


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_matrix(bn, m):
    return bn.TernaryMatrix.from_words(m.words, m.rows, m.cols, m.scale)


def ulp_diff_f32(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


# ---------------------------------------------------------------- quantization
def test_quantize_rows_bit_exact(orc, torch_dev, bn):
    torch = torch_dev
    k = 2560
    rows = [orc.normal_f32(k, 100 + i) for i in range(6)]
    rows.append(np.zeros(k, np.float32))                       # amax floor 1e-5
    rows.append(np.full(k, 3e-6, np.float32))                  # below the floor
    spike = orc.normal_f32(k, 7) * np.float32(1e-3)
    spike[17] = np.float32(-50.0)
    rows.append(spike)
    nan_row = orc.normal_f32(k, 8)
    nan_row[5] = np.nan                                        # NaN -> -128, ignored by amax
    rows.append(nan_row)
    inf_row = orc.normal_f32(k, 9)
    inf_row[3] = np.inf                                        # amax = inf, scale 0
    rows.append(inf_row)
    half = np.arange(k, dtype=np.float32) - np.float32(k / 2)  # exact .5 ties
    rows.append(half)
    x = np.stack(rows)
    q = bn.quantize_activation(to_dev(torch, x))
    torch.cuda.synchronize()
    xq = q.unpadded().cpu().numpy()
    for i, r in enumerate(rows):
        eq, eamax = orc.quant_act(r)
        assert np.array_equal(xq[i], eq), f"row {i}"
        assert np.float32(q.amax[i].item()).tobytes() == np.float32(eamax).tobytes(), f"row {i}"
        assert int(q.xsum[i].item()) == int(eq.astype(np.int64).sum()), f"row {i}"
    assert not q.xq[:, k:].any().item() if q.xq.shape[1] > k else True


@pytest.mark.parametrize("k", [64, 2048, 2560, 4096, 6912, 8192, 1001])
def test_quantize_rows_group_kernel(orc, torch_dev, bn, tuning, k):
    # fp32 rows with k % 4 == 0 take the 16-byte group quantizer (two, three,
    # four or eight float4 a thread); LOOM_AMD_QUANT_GROUPS=0 keeps the
    # value-per-thread kernel, which k = 1001 always takes.  Both against the
    # oracle: normal rows, ties (amax 127: scale 1), near-ties, NaN, inf, zero.
    torch = torch_dev
    rows = [orc.normal_f32(k, 500 + i) for i in range(3)]
    t = orc.normal_f32(k, 510) * np.float32(20.0)
    t[0] = np.float32(127.0)
    t[1 % k] = np.float32(2.5)
    t[2 % k] = np.nextafter(np.float32(-6.5), np.float32(0.0))
    rows.append(t)
    r = orc.normal_f32(k, 511)
    r[k // 2] = np.nan
    rows.append(r)
    r = orc.normal_f32(k, 512)
    r[k - 1] = -np.inf
    rows.append(r)
    rows.append(np.zeros(k, np.float32))
    x = np.stack(rows)
    outs = {}
    for mode in ("groups", "values"):
        tuning("LOOM_AMD_QUANT_GROUPS", None if mode == "groups" else "0")
        q = bn.quantize_activation(to_dev(torch, x))
        torch.cuda.synchronize()
        outs[mode] = [a.cpu().numpy().tobytes() for a in (q.xq, q.amax, q.xsum)]
        xq = q.unpadded().cpu().numpy()
        for i, row in enumerate(rows):
            eq, eamax = orc.quant_act(row)
            assert np.array_equal(xq[i], eq), (mode, i)
            assert np.float32(q.amax[i].item()).tobytes() == np.float32(eamax).tobytes(), (mode, i)
            assert int(q.xsum[i].item()) == int(eq.astype(np.int64).sum()), (mode, i)
        if q.xq.shape[1] > k:
            assert not q.xq[:, k:].any().item(), mode
    assert outs["groups"] == outs["values"]


def test_quantize_rows_f64_bit_exact(orc, torch_dev, bn):
    torch = torch_dev
    k = 640
    x = np.stack([orc.normal_f32(k, 300 + i).astype(np.float64) * 1.000000001 for i in range(5)])
    q = bn.quantize_activation(to_dev(torch, x))
    torch.cuda.synchronize()
    for i in range(x.shape[0]):
        eq, eamax = orc.quant_act(x[i])
        assert np.array_equal(q.unpadded()[i].cpu().numpy(), eq)
        assert np.float32(q.amax[i].item()) == np.float32(eamax)


# ---------------------------------------------------------------- matvec KATs
def _manual_rows(torch, bn, xq_rows, amax):
    xq_rows = np.atleast_2d(np.asarray(xq_rows, np.int8))
    m, k = xq_rows.shape
    pad = np.zeros((m, bn.padded_cols(k)), np.int8)
    pad[:, :k] = xq_rows
    return bn.QuantizedRows(to_dev(torch, pad), to_dev(torch, np.asarray(amax, np.float32)),
                            to_dev(torch, xq_rows.astype(np.int32).sum(axis=1).astype(np.int32)), k)


def test_microsoft_offline_kat(orc, torch_dev, bn):
    # TestMicrosoftOfflinePackedBitNetRowsDecode (poly/tests/bitnet_cpu_test.go:334-362):
    # 8x2, Scale 0.5, xq {2,-3}, amax 127 -> {1.5,-2.5,-2.5,-2.5,1,1.5,2.5,2.5}
    torch = torch_dev
    packed = np.array([0b10100001, 0b00011000, 0b10010000, 0b00001010], np.float32)
    m = orc.pack_ms_offline_float_slots(packed, 8, 2, scale=0.5)
    w = gpu_matrix(bn, m)
    out, acc = bn.ternary_matvec_quantized(w, _manual_rows(torch, bn, [2, -3], [127.0]), want_acc=True)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy()[0],
                          np.array([1.5, -2.5, -2.5, -2.5, 1, 1.5, 2.5, 2.5], np.float32))
    assert np.array_equal(acc.cpu().numpy()[0], [3, -5, -5, -5, 2, 3, 5, 5])


def test_tail_columns_brute_force(orc, torch_dev, bn):
    # Tail-column closed form (poly/tests/bitnet_cpu_test.go:216-247): 3x17.
    torch = torch_dev
    rows, cols = 3, 17
    master = orc.deterministic_weights(rows * cols)
    m = orc.pack_float32(master, rows, cols)
    x = orc.deterministic_weights(cols + 5)[5:]
    xq, amax = orc.quant_act(x)
    w = gpu_matrix(bn, m)
    out, acc = bn.ternary_matvec_quantized(w, _manual_rows(torch, bn, xq, [amax]), want_acc=True)
    torch.cuda.synchronize()
    codes = np.array([[orc.quant_value(v, m.scale) for v in master[r * cols:(r + 1) * cols]]
                      for r in range(rows)], np.int64)
    brute = codes @ xq.astype(np.int64)
    assert np.array_equal(acc.cpu().numpy()[0], brute)
    os_ = orc.output_scale(m.scale, amax)
    assert np.array_equal(out.cpu().numpy()[0], (brute.astype(np.float64) * os_).astype(np.float32))


# ---------------------------------------------------------------- dense
def _check_dense(orc, torch, bn, m, x, activation=-1, residual=None):
    w = gpu_matrix(bn, m)
    pre, post, taps = bn.dense_forward_packed_ternary(
        w, to_dev(torch, x), activation=activation,
        residual=None if residual is None else to_dev(torch, residual), taps=True)
    torch.cuda.synchronize()
    ref = orc.dense_forward(m, x, activation=activation, simd=True)
    M = x.shape[0]
    assert np.array_equal(taps.xq.cpu().numpy(), ref.xq), "int8 activations"
    assert taps.amax.cpu().numpy().tobytes() == ref.amax.tobytes(), "amax"
    acc = taps.acc.cpu().numpy()
    assert np.array_equal(acc, ref.acc), f"int32 accumulators ({np.count_nonzero(acc != ref.acc)} differ of {acc.size})"
    want_pre = ref.pre if residual is None else (ref.pre + residual).astype(np.float32)
    assert pre.cpu().numpy().tobytes() == want_pre.tobytes(), "fp32 pre-activation (bit-exact)"
    # without debug taps the kernels take their plain epilogue: same bytes
    pre2, _ = bn.dense_forward_packed_ternary(
        w, to_dev(torch, x), activation=activation,
        residual=None if residual is None else to_dev(torch, residual))
    torch.cuda.synchronize()
    assert pre2.cpu().numpy().tobytes() == want_pre.tobytes(), "fp32 output without taps"
    if activation != -1:
        if residual is None:
            check_activation(activation, ref.pre, post.cpu().numpy(), ref.post)
    return M


def check_activation(act, pre, got, want):
    """loom's Activate (poly/poly.go:167-200) on the device against the oracle.

    ReLU (0), LeakyReLU (5), ReLU2 (6) and linear use IEEE basic operations
    only: bit-exact.  SiLU (1), Tanh (3) and Sigmoid (4) round an exp/tanh
    value to fp32, whose last fp64 bit differs between libraries: <= 1 fp32 ulp.
    GELU (2) also forms 1 + tanh(z), which cancels for pre < 0: <= 1 fp32 ulp,
    or, where the cancellation leaves fewer than 24 correct bits in loom's own
    fp64 arithmetic, within 0.5*|pre|*4*2^-53 (tanh's last bits times the
    factor 0.5*pre) plus one fp32 rounding."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    if act in (-1, 0, 5, 6) or act > 6 or act < -1:
        assert got.tobytes() == want.tobytes(), f"activation {act}: bit-exact"
        return
    d = ulp_diff_f32(got, want)
    if act != 2:
        assert d.max() <= 1, f"activation {act}: {int(d.max())} ulps"
        return
    p64 = np.asarray(pre, np.float64)
    bound = 0.5 * np.abs(p64) * 4 * 2.0**-53 + np.abs(want.astype(np.float64)) * 2.0**-23
    far = np.abs(got.astype(np.float64) - want.astype(np.float64)) > bound
    assert not np.any((d > 1) & far), f"GELU: {int(np.count_nonzero((d > 1) & far))} outside the bar"


@pytest.mark.parametrize("rows,cols", LOOM_SHAPES)
def test_dense_loom_shapes_bit_exact(orc, torch_dev, bn, rows, cols):
    m = orc.random_matrix(rows, cols, seed=rows * 1000 + cols)
    for M in (1, 7, 64, 130):
        x = orc.normal_f32(M * cols, seed=M + rows).reshape(M, cols)
        _check_dense(orc, torch_dev, bn, m, x)


def test_dense_deterministic_weights(orc, torch_dev, bn):
    # deterministicWeights inputs (poly/tests/bitnet_cpu_test.go:10-20), 512x512
    # as BenchmarkPackedTernaryDenseForward, several batch sizes.
    rows = cols = 512
    m = orc.pack_float32(orc.deterministic_weights(rows * cols), rows, cols)
    for M in (1, 3, 96):
        x = orc.deterministic_weights(M * cols + 11)[11:].reshape(M, cols)
        _check_dense(orc, torch_dev, bn, m, x)


@pytest.mark.parametrize("M", M_EDGES)
def test_dense_batch_edges(orc, torch_dev, bn, M):
    # every kernel variant boundary (skinny 16/32/64, gemm) on a ragged shape
    m = orc.random_matrix(200, 300, seed=77)
    x = orc.normal_f32(M * 300, seed=M).reshape(M, 300)
    _check_dense(orc, torch_dev, bn, m, x)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_dense_fused_quant_edge_rows(orc, torch_dev, bn, M):
    # M <= 8 with K % 4 == 0 (K <= 4096 from M = 5 on, one row per wave)
    # quantizes inside the matmul launch: the same loom edge semantics as the
    # standalone quantizer (zero row -> 1e-5 floor, NaN ignored by amax and
    # quantized to -128, inf amax -> scale 0).
    assert bn._lib.lib().loom_amd_kernel_variant(M) == b"skinny_m16_fusedq"
    k = 2560
    m = orc.random_matrix(96, k, seed=12)
    specials = [np.zeros(k, np.float32), np.full(k, 2e-6, np.float32)]
    r = orc.normal_f32(k, 3)
    r[10] = np.nan
    specials.append(r)
    r = orc.normal_f32(k, 4)
    r[11] = -np.inf
    specials.append(r)
    for start in range(0, len(specials)):
        rows = [specials[(start + i) % len(specials)] for i in range(M)]
        x = np.stack(rows)
        with np.errstate(invalid="ignore"):
            ref = orc.dense_forward(m, x, simd=True)
        w = gpu_matrix(bn, m)
        pre, _, taps = bn.dense_forward_packed_ternary(w, to_dev(torch_dev, x), taps=True)
        torch_dev.cuda.synchronize()
        assert np.array_equal(taps.xq.cpu().numpy(), ref.xq)
        assert taps.amax.cpu().numpy().tobytes() == ref.amax.tobytes()
        assert np.array_equal(taps.acc.cpu().numpy(), ref.acc)
        assert pre.cpu().numpy().tobytes() == ref.pre.tobytes()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_dense_fused_quant_rounding_ties(orc, torch_dev, bn, M):
    # The fused prologue rounds in fp32 and takes loom's fp64 rounding for any
    # thread holding a product within 3.1e-5 of a boundary j + 1/2.  With a
    # row maximum of 127 the scale is exactly 1, so x = j + 1/2 is a tie
    # (math.Round: away from zero, where rintf would pick the even neighbour);
    # rows hold single ties, a run of ties, and near-ties on either side.
    k = 2560
    m = orc.random_matrix(96, k, seed=21)
    rows = []
    for i in range(M):
        r = orc.normal_f32(k, 40 + i) * np.float32(20.0)
        r[0] = np.float32(127.0)
        r[7 + 64 * i] = np.float32(2.5)
        r[900 + i] = np.float32(-0.5)
        r[1500 + i] = np.nextafter(np.float32(6.5), np.float32(7.0))
        r[1700 + i] = np.nextafter(np.float32(-6.5), np.float32(0.0))
        if i % 2:
            r[1000:1100] = np.arange(100, dtype=np.float32) - np.float32(49.5)
        rows.append(r)
    x = np.stack(rows)
    assert np.abs(x).max() == np.float32(127.0)
    ref = orc.dense_forward(m, x, simd=True)
    assert ref.xq[0, 7] == 3 and ref.xq[0, 900] == -1  # the ties went away from zero
    w = gpu_matrix(bn, m)
    pre, _, taps = bn.dense_forward_packed_ternary(w, to_dev(torch_dev, x), taps=True)
    torch_dev.cuda.synchronize()
    assert np.array_equal(taps.xq.cpu().numpy(), ref.xq)
    assert taps.amax.cpu().numpy().tobytes() == ref.amax.tobytes()
    assert np.array_equal(taps.acc.cpu().numpy(), ref.acc)
    assert pre.cpu().numpy().tobytes() == ref.pre.tobytes()


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4, 5, 6])
def test_dense_activation_and_residual(orc, torch_dev, bn, act):
    m = orc.random_matrix(96, 160, seed=5)
    x = orc.normal_f32(9 * 160, seed=6).reshape(9, 160)
    _check_dense(orc, torch_dev, bn, m, x, activation=act)
    res = orc.normal_f32(9 * 96, seed=8).reshape(9, 96)
    _check_dense(orc, torch_dev, bn, m, x, residual=res)


@pytest.mark.parametrize("act", [-1, 0, 1, 2, 3, 4, 5, 6, 9])
@pytest.mark.parametrize("M", [1, 9, 40, 256, 300])
def test_dense_every_activation_on_every_kernel(orc, torch_dev, bn, act, M):
    # Activate(pre) for every id of poly/poly.go:90-97 (and an unknown id,
    # which loom treats as linear) through each matmul family: the fused
    # M = 1 GEMV, the small-M kernels, the GEMM's full-tile epilogue (M = 256
    # of 128-token tiles, N = 512 of 256-row tiles) and its ragged edge
    # (M = 300).  Inputs scaled by 30 put pre in about [-8, 8], across the
    # curved parts of every activation.
    m = orc.random_matrix(512, 640, seed=40 + M)
    x = orc.normal_f32(M * 640, seed=41 + M).reshape(M, 640) * np.float32(30.0)
    _check_dense(orc, torch_dev, bn, m, x, activation=act)


def test_config0_gemv_bit_exact(orc, torch_dev, bn):
    # M=1, K=2560, N=6912.
    m = orc.random_matrix(6912, 2560, seed=0xC0)
    x = orc.normal_f32(2560, seed=0xC1).reshape(1, 2560)
    _check_dense(orc, torch_dev, bn, m, x)


@pytest.mark.parametrize("shape", [(6912, 2560), (2560, 6912)], ids=["up_gate", "down"])
@pytest.mark.parametrize("M", [1, 8, 64, 512, 4096])
def test_config1_sweep_bit_exact(orc, torch_dev, bn, shape, M):
    # M in {1,8,64,512,4096} on both FFN shapes, int32 bit-exact.
    n, k = shape
    m = orc.random_matrix(n, k, seed=n + k)
    x = orc.normal_f32(M * k, seed=M * 31 + k).reshape(M, k)
    _check_dense(orc, torch_dev, bn, m, x)


# ---------------------------------------------------------------- norm + requant
@pytest.mark.parametrize("n", [160, 2560, 6912])
def test_norm_quant_strict_bit_exact(orc, torch_dev, bn, n):
    torch = torch_dev
    M = 5
    h = orc.normal_f32(M * n, seed=n).reshape(M, n) * np.float32(3.0)
    wt = orc.uniform_f32(n, 0.5, 1.5, seed=n + 1)
    for weight in (None, wt):
        hd = to_dev(torch, h.copy())
        q = bn.norm_quant_rows(hd, None if weight is None else to_dev(torch, weight), eps=1e-5,
                               norm="strict")
        torch.cuda.synchronize()
        got = hd.cpu().numpy()
        for i in range(M):
            want = orc.bitnet_rmsnorm_row(h[i], weight, 1e-5)
            assert got[i].tobytes() == want.tobytes(), f"row {i} normalized values"
            eq, eamax = orc.quant_act(want)
            assert np.array_equal(q.unpadded()[i].cpu().numpy(), eq)
            assert np.float32(q.amax[i].item()) == np.float32(eamax)


@pytest.mark.parametrize("M", [300, 1100])
def test_norm_quant_strict_many_rows(orc, torch_dev, bn, M):
    # below 1024 rows each workgroup forms its row's ordered sum of squares
    # (the workgroup-parallel exact form); from 1024 rows one lane per row
    # adds the row in order.  Sampled rows, bit-exact against the oracle.
    torch = torch_dev
    n = 2560
    h = orc.normal_f32(M * n, seed=M + 7).reshape(M, n) * np.float32(2.0)
    h[:, ::97] *= np.float32(40.0)  # a few large values per row
    hd = to_dev(torch, h.copy())
    q = bn.norm_quant_rows(hd, None, eps=1e-5, norm="strict")
    torch.cuda.synchronize()
    got = hd.cpu().numpy()
    qn = q.unpadded().cpu().numpy()
    for i in sorted({0, 1, M // 2, M - 2, M - 1} | set(range(3, M, 61))):
        want = orc.bitnet_rmsnorm_row(h[i], None, 1e-5)
        assert got[i].tobytes() == want.tobytes(), f"row {i} normalized values"
        assert np.array_equal(qn[i], orc.quant_act(want)[0]), f"row {i} codes"


def test_norm_quant_fast_within_one_ulp(orc, torch_dev, bn):
    torch = torch_dev
    n, M = 6912, 16
    h = orc.normal_f32(M * n, seed=99).reshape(M, n)
    hd = to_dev(torch, h.copy())
    q = bn.norm_quant_rows(hd, None, eps=1e-5, norm="fast")
    torch.cuda.synchronize()
    got = hd.cpu().numpy()
    want = np.stack([orc.bitnet_rmsnorm_row(h[i], None, 1e-5) for i in range(M)])
    assert ulp_diff_f32(got, want).max() <= 1
    # requantization of the GPU's own rows is bit-exact
    for i in range(M):
        eq, _ = orc.quant_act(got[i])
        assert np.array_equal(q.unpadded()[i].cpu().numpy(), eq)


# ---------------------------------------------------------------- SwiGLU
def _swiglu_case(orc, torch, bn, hidden, inter, M, seed, norm, with_norm_w, act=1,
                 with_bias=False):
    g = orc.random_matrix(inter, hidden, seed=seed)
    u = orc.random_matrix(inter, hidden, seed=seed + 1)
    d = orc.random_matrix(hidden, inter, seed=seed + 2)
    wn = orc.uniform_f32(inter, 0.5, 1.5, seed=seed + 3) if with_norm_w else None
    x = orc.normal_f32(M * hidden, seed=seed + 4).reshape(M, hidden)
    # loom's Master-tail biases [gate inter | up inter | down hidden]
    # (poly/swiglu.go:276-281, poly/bitnet_cpu.go:521-526)
    bias = orc.normal_f32(2 * inter + hidden, seed=seed + 5) * np.float32(0.25) if with_bias else None
    G, U, D = gpu_matrix(bn, g), gpu_matrix(bn, u), gpu_matrix(bn, d)
    h, out, t = bn.swiglu_forward_packed_ternary(
        G, U, D, to_dev(torch, x), inner_norm=None if wn is None else to_dev(torch, wn),
        eps=1e-5, activation=act, norm=norm, taps=True,
        bias=None if bias is None else to_dev(torch, bias))
    torch.cuda.synchronize()
    ref = orc.swiglu_forward(g, u, d, x, inner_norm=wn, bias=bias, eps=1e-5, activation=act,
                             simd=True)
    # integer stages before the gate: bit-exact
    assert np.array_equal(t.xq.cpu().numpy(), ref.xq)
    assert t.amax.cpu().numpy().tobytes() == ref.amax.tobytes()
    assert np.array_equal(t.acc_gate.cpu().numpy(), ref.acc_gate)
    assert np.array_equal(t.acc_up.cpu().numpy(), ref.acc_up)
    # normalized gate product: <= 1 fp32 ulp (exp last bit; fast-mode sum order)
    hg = h.cpu().numpy()
    assert ulp_diff_f32(hg, ref.h).max() <= 1
    # stages after h, against the oracle fed the GPU's own h: bit-exact
    hq_ref, hamax_ref = orc.quant_act_rows(hg)
    assert np.array_equal(t.hq.cpu().numpy(), hq_ref)
    assert t.hamax.cpu().numpy().tobytes() == hamax_ref.tobytes()
    acc_down_ref = np.stack([orc.matvec_scalar(d, hq_ref[i], orc.output_scale(d.scale, hamax_ref[i]))[1]
                             for i in range(M)])
    assert np.array_equal(t.acc_down.cpu().numpy(), acc_down_ref)
    bias_d = 0.0 if bias is None else bias[2 * inter:].astype(np.float64)
    out_ref = np.stack([(acc_down_ref[i].astype(np.float64) * orc.output_scale(d.scale, hamax_ref[i])
                         + bias_d).astype(np.float32) for i in range(M)])
    assert out.cpu().numpy().tobytes() == out_ref.tobytes()
    return hg, ref


@pytest.mark.parametrize("norm", ["strict", "fast"])
@pytest.mark.parametrize("M", [1, 5, 64, 100])
def test_swiglu_small(orc, torch_dev, bn, norm, M):
    _swiglu_case(orc, torch_dev, bn, hidden=64, inter=160, M=M, seed=11 + M, norm=norm,
                 with_norm_w=True)


@pytest.mark.parametrize("act", [1, 6])
def test_swiglu_relu2_and_silu(orc, torch_dev, bn, act):
    _swiglu_case(orc, torch_dev, bn, hidden=128, inter=320, M=3, seed=21, norm="strict",
                 with_norm_w=False, act=act)


@pytest.mark.parametrize("norm", ["strict", "fast"])
@pytest.mark.parametrize("act", [1, 6])
@pytest.mark.parametrize("M", [1, 3, 40, 100])
def test_swiglu_biases(orc, torch_dev, bn, norm, act, M):
    # gate/up biases enter in fp64 before the gate product, the down bias
    # after the down matvec (poly/swiglu.go:303-320): through the fused M = 1
    # GEMV, the small-M kernels and the GEMM epilogue
    _swiglu_case(orc, torch_dev, bn, hidden=256, inter=640, M=M, seed=70 + M, norm=norm,
                 with_norm_w=True, act=act, with_bias=True)


@pytest.mark.parametrize("M", [1, 256])
def test_swiglu_biases_bitnet_2b_shape(orc, torch_dev, bn, M):
    _swiglu_case(orc, torch_dev, bn, hidden=2560, inter=6912, M=M, seed=90 + M, norm="strict",
                 with_norm_w=True, with_bias=True)


@pytest.mark.parametrize("norm", ["strict", "fast"])
@pytest.mark.parametrize("shape", [(64, 160), (2560, 6912)])
def test_swiglu_row_norm_in_down(orc, torch_dev, bn, norm, shape, tuning):
    # One row: the down projection's workgroups normalize and quantize h
    # themselves and write the normalized rows to h_out; with
    # LOOM_AMD_UNFUSED_NORM=1 the separate inner-norm launch does it.  Both
    # pass every stage check against the oracle; strict sums give the same
    # normalized rows byte for byte.
    hidden, inter = shape
    got = {}
    for unfused in (None, "1"):
        tuning("LOOM_AMD_UNFUSED_NORM", unfused)
        got[unfused] = _swiglu_case(orc, torch_dev, bn, hidden=hidden, inter=inter, M=1, seed=1310 + hidden,
                                    norm=norm, with_norm_w=True, with_bias=True)[0]
    tuning("LOOM_AMD_UNFUSED_NORM", None)
    if norm == "strict":
        assert got[None].tobytes() == got["1"].tobytes()


@pytest.mark.parametrize("M", [1, 8, 64, 256])
def test_swiglu_bitnet_2b_shape(orc, torch_dev, bn, M):
    hg, ref = _swiglu_case(orc, torch_dev, bn, hidden=2560, inter=6912, M=M, seed=1234 + M,
                           norm="strict", with_norm_w=True)
    # with strict summation the only freedom is exp's last fp64 bit, which
    # essentially never survives the fp32 cast: report how many h differ
    assert np.count_nonzero(hg != ref.h) <= max(1, hg.size // 100000)


# ---------------------------------------------------------------- plugin ABI on the GPU
def test_plugin_bitnet_linear(orc, torch_dev):
    from loom_amd import accel
    m = orc.random_matrix(384, 512, seed=3)
    M = 4
    x = orc.normal_f32(M * 512, seed=4).reshape(M, 512)
    p = accel.open_amd(device="GPU")
    try:
        assert p.vendor_id() == "amd"
        desc = accel.LayerDesc("BitNetLinear", "TERNARY", f"m={M},k=512,n=384")
        blob = m.entity_blob()
        assert p.weight_bytes(desc) == len(blob)
        res = p.compile_layer(desc, blob)
        assert (res.in_bytes, res.out_bytes) == (M * 512 * 4, M * 384 * 4)
        out = bytearray(res.out_bytes)
        r = res.layer.infer(x.tobytes(), out)
        assert r.infer_ms >= 0
        ref = orc.dense_forward(m, x, simd=True)
        assert bytes(out) == ref.pre.tobytes()
        with pytest.raises(accel.AccelError, match="input byte size mismatch|buffer size mismatch"):
            res.layer.infer(x[:1].tobytes(), out)
        res.layer.release()
    finally:
        p.close()


@pytest.mark.parametrize("act", [1, 2, 3, 4, 5])
def test_plugin_bitnet_linear_activations(orc, torch_dev, act):
    # the size label's act=<id> reaches Activate (poly/dense.go:94-98): the
    # plugin hands back postAct, as DispatchAccelForward does
    # (poly/accel_intel.go:223-225)
    from loom_amd import accel
    n, k, M = 384, 512, 5
    m = orc.random_matrix(n, k, seed=60 + act)
    x = orc.normal_f32(M * k, seed=61 + act).reshape(M, k) * np.float32(30.0)
    p = accel.open_amd(device="GPU")
    try:
        res = p.compile_layer(accel.LayerDesc("BitNetLinear", "TERNARY", f"m={M},k={k},n={n},act={act}"),
                              m.entity_blob())
        out = bytearray(res.out_bytes)
        res.layer.infer(x.tobytes(), out)
        ref = orc.dense_forward(m, x, activation=act, simd=True)
        check_activation(act, ref.pre, np.frombuffer(bytes(out), np.float32).reshape(M, n), ref.post)
        res.layer.release()
    finally:
        p.close()


def test_plugin_bitnet_swiglu(orc, torch_dev):
    from loom_amd import accel
    hidden, inter, M = 128, 320, 3
    g = orc.random_matrix(inter, hidden, seed=31)
    u = orc.random_matrix(inter, hidden, seed=32)
    d = orc.random_matrix(hidden, inter, seed=33)
    wn = orc.uniform_f32(inter, 0.5, 1.5, seed=34)
    x = orc.normal_f32(M * hidden, seed=35).reshape(M, hidden)
    p = accel.open_amd(device="GPU")
    try:
        desc = accel.LayerDesc("BitNetSwiGLU", "TERNARY", f"m={M},k={hidden},n={inter},eps=1e-5")
        blob = g.entity_blob() + u.entity_blob() + d.entity_blob() + wn.tobytes()
        assert p.weight_bytes(desc) == len(blob)
        res = p.compile_layer(desc, blob)
        out = bytearray(res.out_bytes)
        res.layer.infer(x.tobytes(), out)
        ref = orc.swiglu_forward(g, u, d, x, inner_norm=wn, eps=1e-5, simd=True)
        got = np.frombuffer(bytes(out), np.float32).reshape(M, hidden)
        assert ulp_diff_f32(got, ref.out).max() <= 1 or np.array_equal(got, ref.out)
        res.layer.release()
    finally:
        p.close()


@pytest.mark.parametrize("with_norm", [True, False])
def test_plugin_bitnet_swiglu_biases(orc, torch_dev, with_norm):
    # bias=1: the blob ends with loom's Master-tail biases [gate | up | down]
    # (poly/swiglu.go:276-281), after the optional inner-norm weights
    from loom_amd import accel
    hidden, inter, M = 128, 320, 2
    g = orc.random_matrix(inter, hidden, seed=41)
    u = orc.random_matrix(inter, hidden, seed=42)
    d = orc.random_matrix(hidden, inter, seed=43)
    wn = orc.uniform_f32(inter, 0.5, 1.5, seed=44) if with_norm else None
    bias = orc.normal_f32(2 * inter + hidden, seed=45) * np.float32(0.25)
    x = orc.normal_f32(M * hidden, seed=46).reshape(M, hidden)
    p = accel.open_amd(device="GPU")
    try:
        desc = accel.LayerDesc("BitNetSwiGLU", "TERNARY", f"m={M},k={hidden},n={inter},bias=1")
        blob = g.entity_blob() + u.entity_blob() + d.entity_blob()
        blob += (wn.tobytes() if with_norm else b"") + bias.tobytes()
        res = p.compile_layer(desc, blob)
        out = bytearray(res.out_bytes)
        res.layer.infer(x.tobytes(), out)
        ref = orc.swiglu_forward(g, u, d, x, inner_norm=wn, bias=bias, eps=1e-5, simd=True)
        got = np.frombuffer(bytes(out), np.float32).reshape(M, hidden)
        assert ulp_diff_f32(got, ref.out).max() <= 1
        # the biases are not ignored: without them the output differs
        ref0 = orc.swiglu_forward(g, u, d, x, inner_norm=wn, eps=1e-5, simd=True)
        assert ulp_diff_f32(got, ref0.out).max() > 1
        res.layer.release()
    finally:
        p.close()


@pytest.mark.parametrize("force", ["1", ""])
@pytest.mark.parametrize("n,k", [(6912, 2560), (2560, 6912), (6900, 2570), (1000, 1792),
                                 (70000, 2560)])
def test_stream_gemv_matches_oracle(orc, torch_dev, bn, tuning, force, n, k):
    # The streaming GEMV (fixed grid of waves, each walking its 16-row tiles'
    # K tiles through a ring of in-flight loads): forced on every shape
    # (LOOM_AMD_GEMV_STREAM=1) and by default (large N only).  Fused
    # quantization (Dense forward) and pre-quantized rows, M = 1..4: int8 rows,
    # amax and fp32 outputs bit-exact against the oracle.
    torch = torch_dev
    if force:
        tuning("LOOM_AMD_GEMV_STREAM", force)
    m = orc.random_matrix(n, k, seed=n + 3 * k)
    w = gpu_matrix(bn, m)
    for M in (1, 2, 3, 4):
        x = orc.normal_f32(M * k, seed=900 + M).reshape(M, k)
        ref = orc.dense_forward(m, x, simd=True)
        xd = to_dev(torch, x)
        pre, _ = bn.dense_forward_packed_ternary(w, xd)
        q = bn.quantize_activation(xd)
        out = bn.ternary_matvec_quantized(w, q)
        torch.cuda.synchronize()
        assert pre.cpu().numpy().tobytes() == ref.pre.tobytes(), (n, k, M, "fused")
        assert out.cpu().numpy().tobytes() == ref.pre.tobytes(), (n, k, M, "pre-quantized")
    w.release()


def test_c_loader_replays_glue_on_gpu(orc, torch_dev, tmp_path):
    # tests/abi_conformance.c replays the AMD Go glue's sequence (INTEGRATION.md
    # section 1: dlopen + 12 dlsyms + version + open GPU, weight_bytes, compile,
    # io_bytes, first_infer, infer x3, release, close) on the GPU box; the
    # outputs must equal the oracle's Dense forward bytes (linear and ReLU).
    import os
    import struct
    import subprocess
    from loom_amd import _lib
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = tmp_path / "abi_conformance"
    subprocess.run(["gcc", "-O1", "-Wall", "-I", os.path.join(root, "include"),
                    os.path.join(root, "tests", "abi_conformance.c"), "-o", str(exe), "-ldl"],
                   check=True)
    cases = []
    for i, (n, k, M, act) in enumerate([(384, 640, 3, -1), (2560, 6912, 1, 0), (6912, 2560, 70, -1)]):
        m = orc.random_matrix(n, k, seed=800 + i)
        x = orc.normal_f32(M * k, seed=810 + i).reshape(M, k)
        ref = orc.dense_forward(m, x, activation=act, simd=True)
        want = (ref.pre if act == -1 else ref.post).tobytes()
        label = f"m={M},k={k},n={n},act={act}"
        fields = [b"BitNetLinear", label.encode(), m.entity_blob(), x.tobytes(), want]
        path = tmp_path / f"case{i}.bin"
        path.write_bytes(b"".join(struct.pack("<I", len(f)) + f for f in fields))
        cases.append(str(path))
    proc = subprocess.run([str(exe), _lib.LIB_PATH, "1", *cases], capture_output=True, text=True)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.count("ok   infer output == oracle bytes") == 3 * len(cases)


def test_plugin_concurrent_infer_two_threads(orc, torch_dev):
    # loom's Go glue takes no lock around infer, and two goroutines may run
    # two compiled layers at once.  Every layer on a device shares the
    # device's quantization scratch and split-K workspace, so the plugin
    # serializes infer per device: both threads' outputs must stay equal to
    # the oracle over many interleaved calls.  Layer A is a split-K GEMM
    # (M = 128 rows through the down shape), layer B a SwiGLU FFN.
    import threading

    from loom_amd import accel
    ma = orc.random_matrix(2560, 6912, seed=51)
    xa = orc.normal_f32(128 * 6912, seed=52).reshape(128, 6912)
    want_a = orc.dense_forward(ma, xa, simd=True).pre.tobytes()
    hidden, inter, mb = 512, 1024, 4
    g, u, d = (orc.random_matrix(r, c, seed=s) for r, c, s in
               ((inter, hidden, 53), (inter, hidden, 54), (hidden, inter, 55)))
    xb = orc.normal_f32(mb * hidden, seed=56).reshape(mb, hidden)
    p = accel.open_amd(device="GPU")
    try:
        la = p.compile_layer(accel.LayerDesc("BitNetLinear", "TERNARY", "m=128,k=6912,n=2560"),
                             ma.entity_blob()).layer
        lb = p.compile_layer(accel.LayerDesc("BitNetSwiGLU", "TERNARY",
                                             f"m={mb},k={hidden},n={inter},norm=strict"),
                             g.entity_blob() + u.entity_blob() + d.entity_blob()).layer
        out_b0 = bytearray(mb * hidden * 4)
        lb.infer(xb.tobytes(), out_b0)  # single-threaded reference for B
        ref_b = orc.swiglu_forward(g, u, d, xb, eps=1e-5, simd=True)
        got_b = np.frombuffer(bytes(out_b0), np.float32).reshape(mb, hidden)
        assert ulp_diff_f32(got_b, ref_b.out).max() <= 1
        want_b = bytes(out_b0)
        bad = []

        def worker(layer, x, want, name):
            out = bytearray(len(want))
            for i in range(40):
                layer.infer(x.tobytes(), out)
                if bytes(out) != want:
                    bad.append((name, i))

        ts = [threading.Thread(target=worker, args=(la, xa, want_a, "dense")),
              threading.Thread(target=worker, args=(lb, xb, want_b, "swiglu"))]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        assert not bad, f"outputs changed under concurrent infer: {bad[:5]}"
        la.release()
        lb.release()
    finally:
        p.close()


def test_entity_blob_upload_matches_words(orc, torch_dev, bn):
    torch = torch_dev
    m = orc.random_matrix(48, 300, seed=41)
    a = bn.TernaryMatrix.from_entity_blob(m.entity_blob(offset=10000))
    b = gpu_matrix(bn, m)
    assert (a.rows, a.cols, a.scale) == (b.rows, b.cols, b.scale)
    q = bn.quantize_activation(to_dev(torch, orc.normal_f32(300, 1).reshape(1, 300)))
    oa = bn.ternary_matvec_quantized(a, q)
    ob = bn.ternary_matvec_quantized(b, q)
    torch.cuda.synchronize()
    assert torch.equal(oa, ob)
    # and the blob-built matrix's Dense forward equals the oracle bit for bit
    x = orc.normal_f32(3 * 300, 5).reshape(3, 300)
    pre, _ = bn.dense_forward_packed_ternary(a, to_dev(torch, x))
    torch.cuda.synchronize()
    assert pre.cpu().numpy().tobytes() == orc.dense_forward(m, x, simd=True).pre.tobytes()


def test_library_errors_are_loud(orc, torch_dev, bn):
    from loom_amd import _lib
    torch = torch_dev
    m = orc.random_matrix(16, 32, seed=1)
    w = gpu_matrix(bn, m)
    with pytest.raises(ValueError):
        bn.dense_forward_packed_ternary(w, torch.zeros((2, 31), device="cuda"))
    with pytest.raises(_lib.AMDError, match="word count"):
        bn.TernaryMatrix.from_words(m.words[:3], 16, 32, 1.0)
    with pytest.raises(_lib.AMDError, match="truncated"):
        bn.TernaryMatrix.from_entity_blob(m.entity_blob()[:-4])
    assert _lib.lib().loom_amd_ternary_matmul(None, None, 256, None, None, 1, None, None, None) == -1


@pytest.mark.parametrize("path", ["skinny", "stream"])
def test_fused_quant_near_ties(orc, torch_dev, bn, tuning, path):
    # The quantizers decide in fp32 when the fp32 product lies farther than
    # 3.1e-5 from a rounding boundary k + 1/2 (it is within 1.52e-5 of loom's
    # fp64 product) and take loom's fp64 path otherwise: rows built on exact
    # ties, inside the band, at its edge and just outside it must quantize
    # exactly like loom's fp64 path -- through the fused matmul prologue
    # (skinny or streaming kernel) and the stand-alone quantization kernel.
    torch = torch_dev
    if path == "stream":
        tuning("LOOM_AMD_GEMV_STREAM", "1")
    rng = np.random.default_rng(7)
    K = 4096
    m = orc.random_matrix(32, K, seed=71)
    bands = [0.0, 1e-7, -1e-7, 1.5e-5, -1.5e-5, 2.5e-5, -2.5e-5, 3.1e-5, -3.1e-5, 3.5e-5,
             -3.5e-5, 5e-5, -5e-5, 3e-4, -3e-4, 9.9e-4, -9.9e-4, 0.2, -0.3]
    for amax in (127.0, 63.5, 3.0, 1.0, 300.0, 0.001, 7.3):
        scale = 127.0 / float(np.float32(amax))
        rows = []
        for _ in range(4):
            k = rng.integers(-127, 127, K).astype(np.float64)
            eps = rng.choice(bands, K)
            row = ((k + 0.5 + eps) / scale).astype(np.float32)
            row[rng.integers(0, K)] = np.float32(amax) * rng.choice([1.0, -1.0])
            rows.append(row)
        x = np.stack(rows)
        _check_dense(orc, torch, bn, m, x)
        q = bn.quantize_activation(to_dev(torch, x))
        torch.cuda.synchronize()
        xq_ref, am_ref = orc.quant_rows(x)
        assert np.array_equal(q.unpadded().cpu().numpy(), xq_ref), amax


# ---------------------------------------------------------------- large-M GEMM (32x32x32 MFMA) paths
def test_gemm_ragged_rows_and_tiles(orc, torch_dev, bn):
    # M and N not multiples of the 128-token / 32-row blocks: clamped loads
    # must only ever feed outputs that are not stored.
    m = orc.random_matrix(6900, 2560, seed=91)
    x = orc.normal_f32(4100 * 2560, seed=92).reshape(4100, 2560)
    _check_dense(orc, torch_dev, bn, m, x)


def test_gemm_general_epilogue(orc, torch_dev, bn):
    # residual + activation force the general epilogue of the large-M kernel
    m = orc.random_matrix(4096, 512, seed=93)
    x = orc.normal_f32(4096 * 512, seed=94).reshape(4096, 512)
    res = orc.normal_f32(4096 * 4096, seed=95).reshape(4096, 4096)
    _check_dense(orc, torch_dev, bn, m, x, activation=0)
    _check_dense(orc, torch_dev, bn, m, x, residual=res)


def test_swiglu_large_tiles(orc, torch_dev, bn):
    # gate|up at M=4096 x inter=4096 runs the two-matrix large-M kernel
    _swiglu_case(orc, torch_dev, bn, hidden=640, inter=4096, M=4096, seed=97, norm="fast",
                 with_norm_w=True)


def test_swiglu_large_ragged(orc, torch_dev, bn):
    # 63 weight tiles (inter 1000) against 8-tile workgroups, 300 tokens against
    # 128-token tiles: the partial blocks of both matrices
    _swiglu_case(orc, torch_dev, bn, hidden=768, inter=1000, M=300, seed=98, norm="strict",
                 with_norm_w=True)


@pytest.mark.parametrize("shape,M", [((2560, 6912), 300), ((6912, 2560), 200), ((2560, 6912), 65),
                                     ((1000, 2000), 129), ((2560, 6912), 512)])
def test_gemm_split_k(orc, torch_dev, bn, shape, M):
    # 64-token tiles split over K (the last K range shorter than the others),
    # with the general epilogue (taps, residual) and the plain one, back to back
    # on the same arrival counters
    n, k = shape
    m = orc.random_matrix(n, k, seed=n + M)
    x = orc.normal_f32(M * k, seed=M + 5).reshape(M, k)
    _check_dense(orc, torch_dev, bn, m, x)
    res = orc.normal_f32(M * n, seed=M + 6).reshape(M, n)
    _check_dense(orc, torch_dev, bn, m, x, residual=res)


@pytest.mark.parametrize("tile,split", [("64", "1"), ("64", "2"), ("64", "3"), ("64", "27"),
                                        ("128", "0")])
def test_gemm_forced_plans(orc, torch_dev, bn, tuning, tile, split):
    # every tile height and split width, including one K tile per workgroup
    # (27 ranges of the down shape), against the oracle
    tuning("LOOM_AMD_GEMM_TILE", tile)
    tuning("LOOM_AMD_GEMM_SPLIT", split)
    m = orc.random_matrix(2560, 6912, seed=3)
    x = orc.normal_f32(70 * 6912, seed=4).reshape(70, 6912)
    _check_dense(orc, torch_dev, bn, m, x)


@pytest.mark.parametrize("nj,split", [("1", "1"), ("1", "2"), ("1", "3"), ("2", "1")])
@pytest.mark.parametrize("rows,cols,M", [(6912, 2560, 512), (2560, 6912, 200), (6900, 2560, 130),
                                         (1000, 2000, 129)])
def test_gemm_half_width_tiles(orc, torch_dev, bn, tuning, nj, split, rows, cols, M):
    # 64-token tiles of 128 (half width) or 256 weight rows per workgroup, with
    # and without split K (ranges of unequal length), ragged weight rows
    # (6900 = 431.25 tiles, 1000 = 62.5) and token rows, plain and with
    # residual + ReLU: bit-exact
    tuning("LOOM_AMD_GEMM_NJ", nj)
    tuning("LOOM_AMD_GEMM_SPLIT", split)
    m = orc.random_matrix(rows, cols, seed=rows + cols + M)
    x = orc.normal_f32(M * cols, seed=M + 11).reshape(M, cols)
    res = orc.normal_f32(M * rows, seed=M + 12).reshape(M, rows)
    _check_dense(orc, torch_dev, bn, m, x)
    _check_dense(orc, torch_dev, bn, m, x, activation=0, residual=res)


@pytest.mark.parametrize("n", [2560, 6912, 1000, 260, 8192, 4, 1001])
def test_norm_quant_rows_one_wave_equal_workgroup(orc, torch_dev, bn, tuning, n):
    # fast inner norm + requantization of 1024 or more rows, one wave per row,
    # against the one-workgroup-per-row kernel (LOOM_AMD_ROWNORM_WAVE=0): the
    # same normalized rows, codes (zero padding included), amax and sum(xq),
    # on rows with NaN, +-Inf, zeros, tiny and huge values; n = 1001 (not a
    # multiple of 4) takes the workgroup kernel in both runs
    torch = torch_dev
    m = 1030
    h0 = orc.normal_f32(m * n, seed=n + 70).reshape(m, n) * np.float32(3.0)
    h0[1, :] = 0.0
    h0[2, n // 2] = np.nan
    h0[3, 0] = np.inf
    h0[4, -1] = -np.inf
    h0[5, :] *= np.float32(1e-30)
    h0[6, :] *= np.float32(1e30)
    wt = orc.uniform_f32(n, 0.5, 1.5, seed=n + 71)
    outs = {}
    for mode in ("wave", "workgroup"):
        tuning("LOOM_AMD_ROWNORM_WAVE", None if mode == "wave" else "0")
        for weight in (wt, None):
            h = to_dev(torch, h0)
            q = bn.norm_quant_rows(h, None if weight is None else to_dev(torch, weight), eps=1e-5, norm="fast")
            outs[(mode, weight is None)] = [a.cpu().numpy().tobytes() for a in (h, q.xq, q.amax, q.xsum)]
    for unit in (False, True):
        for name, a, b in zip(("rows", "codes", "amax", "xsum"), outs[("wave", unit)], outs[("workgroup", unit)]):
            assert a == b, (name, unit)


@pytest.mark.parametrize("group", ["0", "3", "8"])
def test_gemm_tile_order_groups(orc, torch_dev, bn, tuning, group):
    # the GEMM's tile order: weight-row group fastest (0), or groups of 3
    # token tiles (the last group partial: 5 token tiles) or 8
    tuning("LOOM_AMD_GEMM_GROUP", group)
    m = orc.random_matrix(6900, 2560, seed=61)
    x = orc.normal_f32(300 * 2560, seed=62).reshape(300, 2560)
    _check_dense(orc, torch_dev, bn, m, x)


@pytest.mark.parametrize("ntr", ["default", "1", "2", "4"])
@pytest.mark.parametrize("rows,cols", [(6912, 2560), (2560, 6912), (1000, 2560), (40, 1000), (33, 260)])
def test_fused_row_tiles_per_workgroup(orc, torch_dev, bn, tuning, ntr, rows, cols):
    # M = 1 with the quantization fused: the dispatcher's choice, or one, two
    # or four 16-row weight tiles per workgroup (ragged last groups: 63 and 3
    # tiles, a partial last tile of 33 rows), plain and with residual + ReLU:
    # bit-exact
    if ntr != "default":
        tuning("LOOM_AMD_FUSED_NTR", ntr)
    if ntr == "4":
        tuning("LOOM_AMD_FUSED_WAVES", "8")  # four tiles: eight-wave workgroups
    m = orc.random_matrix(rows, cols, seed=rows + cols)
    x = orc.normal_f32(cols, seed=cols + 1).reshape(1, cols)
    res = orc.normal_f32(rows, seed=rows + 2).reshape(1, rows)
    _check_dense(orc, torch_dev, bn, m, x)
    _check_dense(orc, torch_dev, bn, m, x, activation=0, residual=res)


@pytest.mark.parametrize("ntr", ["1", "2"])
@pytest.mark.parametrize("rows,cols,M", [(6912, 2560, 5), (6912, 2560, 16), (1000, 2560, 8), (40, 1000, 13)])
def test_prequantized_row_tiles_per_workgroup(orc, torch_dev, bn, tuning, ntr, rows, cols, M):
    # 4 < M <= 16 (quantized by its own kernel, then the skinny GEMV on the
    # int8 rows, read branch-free: rows past M fall past the buffer's end):
    # one or two 16-row weight tiles per workgroup (ragged last groups of 63
    # and 3 tiles), plain and with residual + ReLU: bit-exact
    tuning("LOOM_AMD_SKINNY_NTR", ntr)
    m = orc.random_matrix(rows, cols, seed=rows + M)
    x = orc.normal_f32(M * cols, seed=M + 3).reshape(M, cols)
    res = orc.normal_f32(M * rows, seed=M + 4).reshape(M, rows)
    _check_dense(orc, torch_dev, bn, m, x)
    _check_dense(orc, torch_dev, bn, m, x, activation=0, residual=res)


@pytest.mark.parametrize("nt", ["default", "gemm", "split", "1", "2", "4"])
@pytest.mark.parametrize("rows,cols,M", [(6912, 2560, 64), (2560, 6912, 40), (1000, 2570, 17),
                                         (6900, 2560, 33), (40000, 512, 20), (2560, 6912, 64),
                                         (6900, 6912, 57)])
def test_small_m_tiles_per_workgroup(orc, torch_dev, bn, tuning, nt, rows, cols, M):
    # 16 < M <= 64: the default choice, the GEMM kernel on one partial
    # 64-token tile (LOOM_AMD_SMALLM=2: half-width tiles split over K, rows
    # past M never stored), the K-split kernel (40000 rows exceed its
    # workspace and take the single-workgroup kernels), and the skinny kernels
    # with one, two or four 16-row tiles per workgroup (ragged last group and
    # K slice included): int32 accumulators and fp32 outputs bit-exact
    if nt == "default":
        pass
    elif nt == "gemm":
        tuning("LOOM_AMD_SMALLM", "2")
    elif nt == "split":
        tuning("LOOM_AMD_SMALLM", "1")
    else:
        tuning("LOOM_AMD_SMALLM", "0")
        tuning("LOOM_AMD_SKINNY_NT", nt)
    m = orc.random_matrix(rows, cols, seed=rows + M)
    x = orc.normal_f32(M * cols, seed=M + 7).reshape(M, cols)
    _check_dense(orc, torch_dev, bn, m, x)


def test_small_m_split_repeatable(orc, torch_dev, bn, tuning):
    # the K-split kernel leaves its accumulators and arrival counters at zero:
    # back-to-back launches of two shapes (different row groups and slices),
    # residual epilogue included, all give the oracle's bytes
    tuning("LOOM_AMD_SMALLM", "1")
    torch = torch_dev
    cases = []
    for rows, cols, M in ((2560, 6912, 64), (6912, 2560, 29)):
        m = orc.random_matrix(rows, cols, seed=rows + 3)
        x = orc.normal_f32(M * cols, seed=cols + M).reshape(M, cols)
        res = orc.normal_f32(M * rows, seed=M).reshape(M, rows)
        ref = (orc.dense_forward(m, x, simd=True).pre + res).astype(np.float32)
        cases.append((gpu_matrix(bn, m), to_dev(torch, x), to_dev(torch, res), ref))
    outs = []
    for rep in range(20):
        for w, xd, rd, ref in cases:
            outs.append((bn.dense_forward_packed_ternary(w, xd, residual=rd)[0], ref))
    torch.cuda.synchronize()
    for o, ref in outs:
        assert o.cpu().numpy().tobytes() == ref.tobytes()


@pytest.mark.parametrize("nt", ["1", "2"])
def test_small_m_swiglu_tiles_per_workgroup(orc, torch_dev, bn, tuning, nt):
    # gate|up with M = 48 and one or two tiles per workgroup
    tuning("LOOM_AMD_SKINNY_NT", nt)
    _swiglu_case(orc, torch_dev, bn, hidden=2560, inter=6912, M=48, seed=131, norm="strict",
                 with_norm_w=True)


def test_gemm_odd_stage_count_repeatable(orc, torch_dev, bn):
    # K = 6912 gives an odd number of K stages (a one-stage tail before the
    # epilogue reuses the stage buffers): many back-to-back launches must all
    # produce the oracle's bytes
    torch = torch_dev
    m = orc.random_matrix(2560, 6912, seed=41)
    x = orc.normal_f32(1024 * 6912, seed=42).reshape(1024, 6912)
    ref = orc.dense_forward(m, x, simd=True).pre
    w = gpu_matrix(bn, m)
    xd = to_dev(torch, x)
    outs = [bn.dense_forward_packed_ternary(w, xd)[0] for _ in range(40)]
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert o.cpu().numpy().tobytes() == ref.tobytes(), f"launch {i} differs"


def test_swiglu_split_k(orc, torch_dev, bn):
    # gate|up at the BitNet-2B shape with 100 tokens: two-matrix 64-token tiles
    # split over K
    _swiglu_case(orc, torch_dev, bn, hidden=2560, inter=6912, M=100, seed=99, norm="strict",
                 with_norm_w=True)


# ---------------------------------------------------------------- golden fixtures
def _golden(name):
    import os
    return np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name))


@pytest.mark.parametrize("name", ["config0", "tail_3x17", "odd_33x65", "down_m4"])
def test_golden_dense(orc, torch_dev, bn, name):
    # GPU Dense forward against the committed fixtures (written from the
    # oracle by tests/golden/make_golden.py), bit for bit.
    import json
    import os
    from tests.golden import make_golden as mg
    torch = torch_dev
    w, x = mg.dense_inputs(name)
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "manifest.json")) as f:
        m = json.load(f)["dense"][name]
    assert mg.sha(w.words, np.float32(w.scale), x) == m["inputs_sha256"]
    pre, _, taps = bn.dense_forward_packed_ternary(gpu_matrix(bn, w), to_dev(torch, x), taps=True)
    torch.cuda.synchronize()
    pre = pre.cpu().numpy()
    acc = taps.acc.cpu().numpy()
    assert mg.sha(pre) == m["pre_sha256"] and mg.sha(acc) == m["acc_sha256"]


def test_golden_ms_offline_kat(orc, torch_dev, bn):
    # TestMicrosoftOfflinePackedBitNetRowsDecode (poly/tests/bitnet_cpu_test.go:334-362)
    # through the GPU offline import: xq {2,-3} with amax 127 (x = xq exactly).
    import json
    import os
    torch = torch_dev
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_kats.json")) as f:
        k = json.load(f)["microsoft_offline_decode"]
    w = bn.TernaryMatrix.from_ms_offline(np.array(k["packed"], np.uint8), k["rows"], k["cols"], k["scale"])
    # the KAT fixes xq and amax: feed them to the quantized matvec directly
    xq = np.zeros((1, bn.padded_cols(k["cols"])), np.int8)
    xq[0, :k["cols"]] = k["xq"]
    q = bn.QuantizedRows(to_dev(torch, xq), to_dev(torch, np.array([k["amax"]], np.float32)),
                         to_dev(torch, np.array([sum(k["xq"])], np.int32)), k["cols"])
    out = bn.ternary_matvec_quantized(w, q)
    # scale 0.5 and amax 127 make the output scale exactly 0.5: every output
    # is an exact half-integer, so the KAT holds bit for bit
    assert np.array_equal(out.cpu().numpy()[0], np.array(k["out"], np.float32))


@pytest.mark.parametrize("rows,cols", [(8, 4), (64, 2560), (128, 6912), (7, 33), (2, 5)])
def test_ms_offline_import_matches_oracle(orc, torch_dev, bn, rows, cols):
    # packMicrosoftOfflineBitNetRowsToU32FromBytes (poly/bitnet_cpu.go:1078-1098)
    # on the device == the oracle's packer, seen through a Dense forward.
    torch = torch_dev
    rng = np.random.default_rng(rows * 1000 + cols)
    packed = rng.integers(0, 256, size=(rows // 4) * cols, dtype=np.uint8)
    ref = orc.pack_ms_offline_bytes(packed, rows, cols, scale=0.5)
    x = orc.normal_f32(3 * cols, rows + cols).reshape(3, cols)
    want = orc.dense_forward(ref, x, simd=False)
    w = bn.TernaryMatrix.from_ms_offline(packed, rows, cols, 0.5)
    pre, _, taps = bn.dense_forward_packed_ternary(w, to_dev(torch, x), taps=True)
    assert np.array_equal(taps.acc.cpu().numpy(), want.acc)
    assert np.array_equal(pre.cpu().numpy(), want.pre)


def test_golden_swiglu(orc, torch_dev, bn):
    from tests.golden import make_golden as mg
    torch = torch_dev
    g, u, d, wn, x = mg.swiglu_inputs()
    f = _golden("swiglu_small.npz")
    for act in (mg.ACT_SILU, mg.ACT_RELU2):
        h, out = bn.swiglu_forward_packed_ternary(gpu_matrix(bn, g), gpu_matrix(bn, u), gpu_matrix(bn, d),
                                                  to_dev(torch, x), inner_norm=to_dev(torch, wn),
                                                  eps=1e-5, activation=act)
        h = h.cpu().numpy()
        out = out.cpu().numpy()
        if act == mg.ACT_RELU2:  # no exp(): every stage bit-exact
            assert np.array_equal(h, f[f"h_{act}"]) and np.array_equal(out, f[f"out_{act}"])
        else:  # exp() last bits: h within 1 fp32 ulp
            assert ulp_diff_f32(h, f[f"h_{act}"]).max() <= 1
