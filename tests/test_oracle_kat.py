"""Pins the CPU oracle to loom's own known-answer tests and to closed forms.

Each test names the reference test (or the mathematical fact) it checks.
Citations are relative to the loom v0.83.0 tree.
"""
import math

import numpy as np
import pytest


# ---------------------------------------------------------------- weight quant
def test_absmean_quantizer_kat(orc):
    # TestBitNetTernaryQuantizerUsesAbsMean (poly/tests/bitnet_cpu_test.go:134-153)
    master = np.array([-0.2, -0.8, 0.1, 0.8], np.float32)
    scale = orc.ternary_scale(master)
    assert abs(scale - 0.475) <= 1e-6
    assert [orc.quant_value(v, scale) for v in master] == [0, -1, 0, 1]


def test_absmean_scale_closed_forms(orc):
    # bitNetTernaryScale: empty and all-zero masters give 1.0; absmean otherwise.
    assert orc.ternary_scale(np.zeros(0, np.float32)) == 1.0
    assert orc.ternary_scale(np.zeros(9, np.float32)) == 1.0
    w = np.array([3.0, -1.0, 0.0, 4.0], np.float32)
    assert orc.ternary_scale(w) == np.float32(2.0)


def test_quant_value_rounds_half_away(orc):
    # math.Round is half away from zero: v/scale = +-0.5 -> +-1 (ties-to-even gives 0).
    assert orc.quant_value(1.0, 2.0) == 1
    assert orc.quant_value(-1.0, 2.0) == -1
    assert orc.quant_value(0.999, 2.0) == 0
    assert orc.quant_value(100.0, 1.0) == 1
    assert orc.quant_value(-100.0, 1.0) == -1
    assert orc.quant_value(0.5, 0.0) == 1  # scale 0 -> 1


def test_already_ternary_master_packs_at_unit_scale(orc):
    # packFloat32AsBitNetTernaryMatrix alreadyTernary quirk (poly/bitnet_cpu.go:941-954)
    master = np.array([1, 0, -1, 1, 1, 0, 0, -1], np.float32)
    m = orc.pack_float32(master, 2, 4)
    assert m.scale == 1.0
    # codes: -1 -> 0, 0 -> 1, +1 -> 2 at bits 2*(c%16)
    assert m.words[0] == (2 | 1 << 2 | 0 << 4 | 2 << 6)
    assert m.words[1] == (2 | 1 << 2 | 1 << 4 | 0 << 6)
    # the same values times 0.02 use the absmean scale instead
    m2 = orc.pack_float32(master * np.float32(0.02), 2, 4)
    assert m2.scale != 1.0
    assert np.array_equal(m2.words, m.words)


# ---------------------------------------------------------------- packers
def test_microsoft_offline_decode_kat(orc):
    # TestMicrosoftOfflinePackedBitNetRowsDecode (poly/tests/bitnet_cpu_test.go:334-362)
    packed = np.array([0b10100001, 0b00011000, 0b10010000, 0b00001010], np.float32)
    m = orc.pack_ms_offline_float_slots(packed, 8, 2, scale=0.5)
    xq = np.array([2, -3], np.int8)
    out, _ = orc.matvec_scalar(m, xq, orc.output_scale(m.scale, 127.0))
    assert np.allclose(out, [1.5, -2.5, -2.5, -2.5, 1, 1.5, 2.5, 2.5], atol=1e-6, rtol=0)


def test_microsoft_bytes_match_float_slots(orc):
    # TestSetMicrosoftBitNetPackedMatrixBytesMatchesFloatU8Slots (:284-315)
    b = np.array([(i * 17) & 0xFF for i in range(8)], np.uint8)
    a = orc.pack_ms_offline_bytes(b, 8, 4)
    f = orc.pack_ms_offline_float_slots(b.astype(np.float32), 8, 4)
    assert np.array_equal(a.words, f.words)


def test_microsoft_offline_without_master(orc):
    # TestGetBitNetTernaryMatrixFindsOfflinePackedWithoutMasterSlab (:317-332)
    m = orc.pack_ms_offline_float_slots(np.array([0x01, 0x10], np.float32), 4, 2)
    assert (m.rows, m.cols, m.row_words, m.words.size) == (4, 2, 1, 4)
    # code 3 maps to code 1 (ternary 0): byte 0xFF decodes to zeros
    z = orc.pack_ms_offline_bytes(np.array([0xFF, 0xFF], np.uint8), 4, 2)
    assert np.all(z.words == (1 | 1 << 2))


# ---------------------------------------------------------------- matvec
def _decode(m):
    """Decode packed words to int ternary values by the documented bit layout."""
    w = np.zeros((m.rows, m.cols), np.int64)
    rw = m.row_words
    for r in range(m.rows):
        for c in range(m.cols):
            code = (int(m.words[r * rw + c // 16]) >> (2 * (c % 16))) & 3
            w[r, c] = code - 1
    return w


def test_tail_columns_brute_force(orc):
    # TestBitNetTernaryKernelHandlesTailColumns (:216-247): 3x17 against the
    # closed form sum over quantized weights.
    rows, cols = 3, 17
    weights = orc.deterministic_weights(rows * cols)
    m = orc.pack_float32(weights, rows, cols)
    xq, amax = orc.quant_act(orc.deterministic_weights(cols))
    os_ = orc.output_scale(m.scale, amax)
    got, acc = orc.matvec_scalar(m, xq, os_)
    for r in range(rows):
        s = 0
        for c in range(cols):
            q = orc.quant_value(float(weights[r * cols + c]), m.scale)
            s += int(xq[c]) * q
        assert acc[r] == s
        assert got[r] == float(s) * os_


@pytest.mark.parametrize("rows,cols", [(40, 70), (8, 64), (33, 65), (16, 128),
                                       (64, 2560), (128, 6912), (7, 191), (3, 17)])
def test_simd_matches_scalar_bit_identical(orc, rows, cols):
    # TestBitNetPackedMatVecMatchesScalar / TestBitNetTernaryDenseSimdMatchesScalar
    # (poly/tests/bitnet_packed_test.go:15-52; bitnet_simd_test.go:13-45)
    weights = orc.deterministic_weights(rows * cols)
    x = orc.deterministic_weights(2 * cols).reshape(2, cols)
    m = orc.pack_float32(weights, rows, cols)
    scalar = orc.dense_forward(m, x, simd=False)
    simd = orc.dense_forward(m, x, simd=True, workers=8)
    assert np.array_equal(scalar.pre.view(np.uint32), simd.pre.view(np.uint32))
    assert np.array_equal(scalar.acc, simd.acc)
    # and both equal the brute-force integer product over the decoded weights
    w = _decode(m)
    ref = scalar.xq.astype(np.int64) @ w.T
    assert np.array_equal(ref, scalar.acc.astype(np.int64))


@pytest.mark.parametrize("n_bytes", [32, 64, 96, 512, 1536, 4096])
def test_code_row_dot_avx2_matches_go(orc, n_bytes):
    # TestBitNetTernaryKernelMatchesGo (poly/simd/bitnet_ternary_test.go:11-36);
    # Go's math/rand stream (seed 42) cannot be reproduced, so numpy draws the
    # same distributions: codes in {0,1,2}, acts in [-128,127].
    if not orc.simd_available():
        pytest.skip("no AVX2")
    rng = np.random.default_rng(42)
    for _ in range(200):
        codes = rng.integers(0, 3, n_bytes).astype(np.uint8)
        acts = rng.integers(-128, 128, n_bytes).astype(np.int8)
        want = int(codes.astype(np.int64) @ acts.astype(np.int64))
        assert orc.code_row_dot(codes, acts, avx2=False) == want
        assert orc.code_row_dot(codes, acts, avx2=True) == want


def test_run_rows_plan(orc):
    # bitNetRunRows (poly/bitnet_cpu.go:780-808) chunking thresholds
    import ctypes as C
    n, c = C.c_int(), C.c_int()
    orc.lib().orc_run_rows_plan(6912, 2560, 8, C.byref(n), C.byref(c))
    assert (n.value, c.value) == (8, 864)
    orc.lib().orc_run_rows_plan(100, 2000, 8, C.byref(n), C.byref(c))  # work < 262144
    assert (n.value, c.value) == (1, 100)
    orc.lib().orc_run_rows_plan(3, 200000, 8, C.byref(n), C.byref(c))  # rows < 4
    assert (n.value, c.value) == (1, 3)
    orc.lib().orc_run_rows_plan(10, 100000, 4, C.byref(n), C.byref(c))
    assert (n.value, c.value) == (4, 3)


# ---------------------------------------------------------------- activation quant
def test_activation_quant_closed_forms(orc):
    # bitNetQuantizedActivation (poly/bitnet_cpu.go:73-95)
    q, amax = orc.quant_act(np.array([3.0, -3.0, 0.0, 1.5], np.float32))
    assert amax == 3.0
    assert q.tolist() == [127, -127, 0, 64]  # 1.5*127/3 = 63.5 -> 64 (half away)
    q, amax = orc.quant_act(np.array([-1.5, 0.5, -0.5, 127.0], np.float32))
    assert amax == 127.0  # scale 1.0: exercises the tie rule directly
    assert q.tolist() == [-2, 1, -1, 127]
    q, amax = orc.quant_act(np.zeros(5, np.float32))
    assert amax == np.float32(1e-5) and not q.any()
    q, amax = orc.quant_act(np.array([1e-6, -2e-6], np.float32))
    assert amax == np.float32(1e-5)
    # NaN never wins the max and converts through Go's amd64 int64 indefinite to -128
    q, amax = orc.quant_act(np.array([np.nan, 2.0, -1.0], np.float32))
    assert amax == 2.0 and q.tolist() == [-128, 127, -64]


def test_activation_quant_float64_rounds_abs_to_f32(orc):
    x = np.array([1.0000000001, -0.5], np.float64)
    q, amax = orc.quant_act(x)
    assert amax == np.float32(1.0000000001)
    assert q.tolist() == [127, -64]


def test_activation_quant_matches_numpy_restatement(orc):
    # property: per-element formula holds over a large random row
    x = orc.normal_f32(4096, 7)
    q, amax = orc.quant_act(x)
    assert amax == np.float32(np.max(np.abs(x)))
    v = x.astype(np.float64) * (127.0 / np.float64(amax))
    ref = np.clip(np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5)), -128, 127)
    assert np.array_equal(q.astype(np.int64), ref.astype(np.int64))


# ---------------------------------------------------------------- dense
def test_packed_dense_matches_dequantized(orc):
    # TestPackedTernaryDenseMatchesDequantizedPath (poly/tests/bitnet_cpu_test.go:184-214)
    weights = orc.deterministic_weights(15)
    scale = orc.ternary_scale(weights)
    deq = np.array([orc.quant_value(v, scale) for v in weights], np.float32) * np.float32(scale)
    x = np.array([0.1, -0.2, 0.3, -0.4, 0.5, 0.6, -0.7, 0.8, -0.9, 1.0], np.float32).reshape(2, 5)
    ref = x.astype(np.float64) @ deq.reshape(3, 5).T.astype(np.float64)
    got = orc.dense_forward(orc.pack_float32(weights, 3, 5), x, simd=True)
    assert np.max(np.abs(ref - got.post)) <= 5e-3


def test_dense_rows_are_independent(orc):
    # loom processes batch rows one by one (poly/dense.go:83-99): row b of an
    # M-row forward equals a 1-row forward of row b.
    m = orc.random_matrix(96, 200, seed=3)
    x = orc.normal_f32(4 * 200, 5).reshape(4, 200)
    full = orc.dense_forward(m, x)
    for b in range(4):
        one = orc.dense_forward(m, x[b:b + 1])
        assert np.array_equal(one.pre[0].view(np.uint32), full.pre[b].view(np.uint32))


def test_dense_activations(orc):
    m = orc.random_matrix(32, 64, seed=9)
    x = orc.normal_f32(64, 1).reshape(1, 64)
    lin = orc.dense_forward(m, x, activation=orc.ACT_LINEAR)
    relu = orc.dense_forward(m, x, activation=orc.ACT_RELU)
    relu2 = orc.dense_forward(m, x, activation=orc.ACT_RELU2)
    assert np.array_equal(relu.post, np.where(lin.pre < 0, np.float32(0), lin.pre))
    assert np.array_equal(relu2.post, np.where(lin.pre < 0, np.float32(0), lin.pre * lin.pre))
    assert np.array_equal(lin.post, lin.pre)


# ---------------------------------------------------------------- Activate, id by id
# loom's Activate for float32 (poly/poly.go:167-200; ids poly/poly.go:90-97).
# Each branch is pinned by IEEE closed forms at special points and, for the
# branches that call exp/tanh/pow, by an independent fp64 formulation
# (scipy's expit, tanh from expm1, x*x*x for the cube): where that value lies
# safely inside one fp32 rounding interval the fp32 result is fixed whatever
# the last fp64 bit of the library routine, so it is checked bit for bit;
# elsewhere within 1 fp32 ulp.

def _act(orc, v, act):
    return np.float32(orc.activate(float(np.float32(v)), act))


def _bits(v):
    return np.asarray(v, np.float32).view(np.uint32).item()


def _ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, np.int64(-2**31) - ia, ia)
    ib = np.where(ib < 0, np.int64(-2**31) - ib, ib)
    return int(np.abs(ia - ib))


def _fp32_fixed(y, rel):
    """fp32(y) if every value within rel of y rounds to the same fp32, else None."""
    if rel > 1e-6:
        return None
    lo, hi = np.float32(y * (1.0 - rel)), np.float32(y * (1.0 + rel))
    return lo if _bits(lo) == _bits(hi) else None


def _act_samples():
    rng = np.random.default_rng(20240501)
    v = (rng.standard_normal(3000) * 3.0).astype(np.float32)
    return np.concatenate([v, np.linspace(-6, 6, 241, dtype=np.float32)])


def _tanh64(z):
    # tanh(z) = -expm1(-2z) / (2 + expm1(-2z)); sign-symmetric form
    a = abs(z)
    e = math.expm1(-2.0 * a)
    t = -e / (2.0 + e)
    return math.copysign(t, z)


def _check_libm_branch(orc, act, value64, rel, min_exact, abs_err=None):
    # abs_err(v): an absolute error bound that replaces the 1-ulp fallback
    # where the reference's own fp64 arithmetic leaves fewer correct bits
    # than fp32 holds
    exact = 0
    for v in _act_samples():
        got = _act(orc, v, act)
        r = value64(float(v))
        y, post = r[0], r[1]
        want = _fp32_fixed(y, r[2] if len(r) > 2 else rel)
        if want is not None:
            want = post(want)
            assert _bits(got) == _bits(want), (act, float(v), float(got), float(want))
            exact += 1
        elif abs_err is not None and abs_err(float(v)) > 0:
            assert abs(float(got) - y) <= abs_err(float(v)), (act, float(v))
        else:
            assert _ulps(got, post(np.float32(y))) <= 1, (act, float(v))
    assert exact >= min_exact, (act, exact)


def test_activate_relu_and_relu2_closed_forms(orc):
    # ReLU (0): v < 0 -> 0, else v (so -0 and NaN pass through); ReLU2 (6): v*v in fp32.
    for v in _act_samples():
        assert _bits(_act(orc, v, orc.ACT_RELU)) == _bits(np.float32(0) if v < 0 else v)
        want = np.float32(0) if v < 0 else np.float32(v) * np.float32(v)
        assert _bits(_act(orc, v, orc.ACT_RELU2)) == _bits(want)
    assert _bits(_act(orc, -0.0, orc.ACT_RELU)) == 0x80000000
    assert _bits(_act(orc, -0.0, orc.ACT_RELU2)) == 0x00000000  # (-0)*(-0) = +0
    assert np.isnan(_act(orc, np.nan, orc.ACT_RELU))
    assert np.isnan(_act(orc, np.nan, orc.ACT_RELU2))
    assert _act(orc, -np.inf, orc.ACT_RELU) == 0 and _act(orc, np.inf, orc.ACT_RELU) == np.inf
    assert _act(orc, 3e19, orc.ACT_RELU2) == np.inf  # fp32 product overflows


def test_activate_linear_and_unknown_ids_are_identity(orc):
    # ActivationLinear (-1) and any id outside the enum take the default branch.
    for act in (orc.ACT_LINEAR, 7, 99, -5):
        for v in (-2.5, 0.0, -0.0, 1e-40, 3.0e38, np.inf, -np.inf):
            assert _bits(_act(orc, v, act)) == _bits(np.float32(v))
        assert np.isnan(_act(orc, np.nan, act))


def test_activate_leaky_relu_multiplies_in_fp64(orc):
    # LeakyReLU (5): T(float64(v) * 0.01) for v < 0 -- an fp64 product with the
    # fp64 constant 0.01, then one rounding to fp32.  The exact product is
    # formed with fractions and rounded to fp64 (float() of a Fraction is
    # correctly rounded), then to fp32.
    from fractions import Fraction
    c = Fraction(0.01)
    fp32_form_differs = 0
    for v in _act_samples():
        got = _act(orc, v, orc.ACT_LEAKY_RELU)
        if not v < 0:
            assert _bits(got) == _bits(v)
            continue
        want = np.float32(float(Fraction(float(v)) * c))
        assert _bits(got) == _bits(want), float(v)
        if _bits(np.float32(v) * np.float32(0.01)) != _bits(want):
            fp32_form_differs += 1
    # the samples separate loom's fp64 product from an fp32 one (v * 0.01f)
    assert fp32_form_differs > 10
    assert _bits(_act(orc, -0.0, orc.ACT_LEAKY_RELU)) == 0x80000000
    assert _act(orc, -np.inf, orc.ACT_LEAKY_RELU) == -np.inf
    assert np.isnan(_act(orc, np.nan, orc.ACT_LEAKY_RELU))
    # subnormal result: -1e-40 * 0.01 = -1e-42 (fp32 subnormal), not flushed
    assert _act(orc, -1e-40, orc.ACT_LEAKY_RELU) == np.float32(float(Fraction(float(np.float32(-1e-40))) * c))


def test_activate_sigmoid(orc):
    # Sigmoid (4): T(1 / (1 + exp(-v))), fp64 then one rounding.
    from scipy.special import expit
    _check_libm_branch(orc, orc.ACT_SIGMOID, lambda v: (float(expit(v)), lambda f: f),
                       rel=1e-12, min_exact=3000)
    assert _act(orc, 0.0, orc.ACT_SIGMOID) == np.float32(0.5)
    assert _act(orc, 30.0, orc.ACT_SIGMOID) == np.float32(1.0)  # 1 - 9.4e-14 rounds to 1
    assert _act(orc, -30.0, orc.ACT_SIGMOID) == np.float32(1.0 / (1.0 + math.exp(30.0)))
    assert _act(orc, np.inf, orc.ACT_SIGMOID) == 1.0
    assert _bits(_act(orc, -np.inf, orc.ACT_SIGMOID)) == 0  # 1/(1+inf) = +0
    assert np.isnan(_act(orc, np.nan, orc.ACT_SIGMOID))


def test_activate_silu_multiplies_in_fp32(orc):
    # SiLU (1): v * T(1/(1+exp(-v))) -- the sigmoid is rounded to fp32 first
    # and the product is an fp32 multiply (Go's T * T), not fp32(v64 * sig64).
    from scipy.special import expit
    _check_libm_branch(orc, orc.ACT_SILU,
                       lambda v: (float(expit(v)), lambda f, v=v: np.float32(v) * f),
                       rel=1e-12, min_exact=3000)
    fp64_form_differs = 0
    for v in _act_samples():
        sig = _fp32_fixed(float(expit(float(v))), 1e-12)
        if sig is None:
            continue
        if _bits(np.float32(float(v) * float(expit(float(v))))) != _bits(np.float32(v) * sig):
            fp64_form_differs += 1
    assert fp64_form_differs > 10  # the samples separate the two multiplications
    assert _bits(_act(orc, 0.0, orc.ACT_SILU)) == 0
    assert _act(orc, 30.0, orc.ACT_SILU) == np.float32(30.0)
    assert _act(orc, np.inf, orc.ACT_SILU) == np.inf
    assert np.isnan(_act(orc, -np.inf, orc.ACT_SILU))  # -inf * 0
    assert np.isnan(_act(orc, np.nan, orc.ACT_SILU))


def test_activate_tanh(orc):
    # Tanh (3): T(math.Tanh(float64(v))) -- tanh in fp64, then one rounding.
    _check_libm_branch(orc, orc.ACT_TANH, lambda v: (_tanh64(v), lambda f: f),
                       rel=1e-12, min_exact=3000)
    assert _bits(_act(orc, -0.0, orc.ACT_TANH)) == 0x80000000
    assert _act(orc, 30.0, orc.ACT_TANH) == 1.0 and _act(orc, -30.0, orc.ACT_TANH) == -1.0
    assert _act(orc, np.inf, orc.ACT_TANH) == 1.0 and _act(orc, -np.inf, orc.ACT_TANH) == -1.0
    assert np.isnan(_act(orc, np.nan, orc.ACT_TANH))
    # tiny v: tanh(v) = v to fp64 precision
    assert _act(orc, 1e-20, orc.ACT_TANH) == np.float32(1e-20)


def _gelu64(v):
    # tanh-form GELU with the cube as x*x*x and tanh from expm1; the margin
    # grows as 1 + tanh cancels (v < 0): a few fp64 ulps of tanh, relative
    # to 1 + tanh
    inner = math.sqrt(2.0 / math.pi) * (v + 0.044715 * (v * v * v))
    t = _tanh64(inner)
    one_t = 1.0 + t
    rel = 1e-13 / one_t if one_t > 0 else 1.0
    return 0.5 * v * one_t, (lambda f: f), min(rel, 1.0)


def test_activate_gelu_tanh_form(orc):
    # GELU (2): T(0.5*v64*(1 + tanh(sqrt(2/pi)*(v64 + 0.044715*pow(v64, 3))))).
    # (1 + tanh) cancels for v < 0, so the exact check asks for a margin that
    # grows with the cancellation.
    def cancelled(v):
        # 1 + tanh(z) for z < -17: fp64 tanh is within a few ulps of -1
        # (ulp 1.1e-16), so the reference keeps only its absolute error,
        # 0.5*|v|*(4 * 2^-53), plus the fp32 rounding of the result
        y = _gelu64(v)[0]
        return 0.5 * abs(v) * 4 * 2.0**-53 + abs(y) * 2.0**-23 if _gelu64(v)[2] > 1e-9 else 0.0
    _check_libm_branch(orc, orc.ACT_GELU, _gelu64, rel=None, min_exact=2500, abs_err=cancelled)
    # the tanh form, not the erf form: at v = 1 they are ~1.5e-4 apart (> 1000 ulps)
    erf_form = np.float32(0.5 * (1.0 + math.erf(1.0 / math.sqrt(2.0))))
    assert _ulps(_act(orc, 1.0, orc.ACT_GELU), erf_form) > 1000
    assert _bits(_act(orc, 0.0, orc.ACT_GELU)) == 0
    assert _act(orc, 30.0, orc.ACT_GELU) == np.float32(30.0)
    assert _bits(_act(orc, -30.0, orc.ACT_GELU)) == 0x80000000  # (0.5*-30)*(1 + -1) = -0
    assert _act(orc, np.inf, orc.ACT_GELU) == np.inf
    assert np.isnan(_act(orc, -np.inf, orc.ACT_GELU))  # -inf * 0
    assert np.isnan(_act(orc, np.nan, orc.ACT_GELU))


def test_dense_post_applies_activate_per_element(orc):
    # DenseForwardPackedTernaryCPU (poly/dense.go:94-98): post = Activate(pre) elementwise,
    # for every id, on the fp32 pre-activation.
    m = orc.random_matrix(48, 96, seed=19)
    x = orc.normal_f32(3 * 96, 2).reshape(3, 96) * np.float32(40.0)
    for act in (orc.ACT_LINEAR, 0, 1, 2, 3, 4, 5, 6):
        out = orc.dense_forward(m, x, activation=act)
        want = np.array([_act(orc, v, act) for v in out.pre.ravel()], np.float32).reshape(out.pre.shape)
        assert out.post.tobytes() == want.tobytes(), act


# ---------------------------------------------------------------- swiglu pieces
def test_gate_product_closed_forms(orc):
    assert orc.swiglu_gate_product(0.0, 5.0) == 0.0
    assert orc.swiglu_gate_product(3.0, 0.0) == 0.0
    assert orc.swiglu_gate_product(-2.0, 3.0, orc.ACT_RELU2) == 0.0
    assert orc.swiglu_gate_product(2.0, 3.0, orc.ACT_RELU2) == 12.0
    # sigma(40) rounds to 1 in fp64 -> product is g*u exactly
    assert orc.swiglu_gate_product(40.0, 0.5) == 20.0
    g = 0.75
    assert orc.swiglu_gate_product(g, 2.0) == (g * (1.0 / (1.0 + math.exp(-g)))) * 2.0


def test_inner_norm_closed_form(orc):
    # constant row c: scale = 1/sqrt(c^2 + eps); unit weights
    n, c, eps = 6912, 0.25, 1e-5
    h = orc.bitnet_rmsnorm_row(np.full(n, c, np.float32), None, eps)
    want = np.float32(np.float64(c) * (1.0 / math.sqrt(c * c + eps)))
    assert np.all(h == want)
    # weights multiply after the scale: w=2 doubles (exactly, power of two)
    h2 = orc.bitnet_rmsnorm_row(np.full(n, c, np.float32), np.full(n, 2.0, np.float32), eps)
    assert np.all(h2 == np.float32(2 * np.float64(want)))
    # eps <= 0 defaults to 1e-5
    h3 = orc.bitnet_rmsnorm_row(np.full(8, c, np.float32), None, 0.0)
    assert np.all(h3 == want)


def _seq_sum_sq(v64):
    # loom's sequential fp64 sum of squares (np.add.accumulate adds in order)
    return float(np.add.accumulate(v64 * v64)[-1])


def _differs(a, b):
    return not np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


def _association_probes():
    # probe elements found by tests/golden/find_association_probes.py: tiny
    # values appended to a seeded row, each with a weight for which the two
    # fp64 associations round to different fp32 values
    import json
    import os
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                           "association_probes.json")) as f:
        return json.load(f)


def test_inner_norm_f32_association(orc):
    # bitNetRMSNormTensorRowWeighted (poly/bitnet_cpu.go:893-913) writes
    # T(float64(v) * scale * w): Go evaluates left to right, (v*scale)*w.
    # On the probe elements the other association gives another fp32 value;
    # the oracle must give the reference's on every element.
    P = _association_probes()
    probes = P["inner_norm_f32"]
    base = orc.normal_f32(P["base_n"], P["base_seed"])
    x = np.concatenate([base, np.array([p["x"] for p in probes], np.float32)])
    w = np.concatenate([orc.uniform_f32(P["base_n"], 0.5, 1.5, 602),
                        np.array([p["w"] for p in probes], np.float32)])
    n, eps = x.size, P["eps"]
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    scale = 1.0 / math.sqrt(_seq_sum_sq(x64) / n + eps)
    ref = ((x64 * scale) * w64).astype(np.float32)
    alt = (x64 * (scale * w64)).astype(np.float32)
    tail = slice(P["base_n"], None)
    assert np.all(ref[tail].view(np.uint32) != alt[tail].view(np.uint32)), \
        "a probe no longer separates the associations"
    got = orc.bitnet_rmsnorm_row(x, w, eps)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_inner_norm_f64_association(orc):
    # bitNetRMSNormFloat64Weighted (poly/bitnet_cpu.go:868-887) writes
    # data[i] *= scale * w: the product scale*w is formed first, the opposite
    # association of the fp32-row helper above.
    import ctypes as C
    n, eps = 2560, 1e-5
    d = orc.normal_f32(n, 603).astype(np.float64) * (1.0 + 2.0 ** -30)
    w = orc.uniform_f32(n, 0.5, 1.5, 604)
    w64 = w.astype(np.float64)
    scale = 1.0 / math.sqrt(_seq_sum_sq(d) / n + eps)
    ref = d * (scale * w64)
    alt = (d * scale) * w64
    assert _differs(ref, alt), "inputs do not separate the associations"
    got = d.copy()
    orc.lib().orc_bitnet_rmsnorm_f64(got.ctypes.data_as(C.c_void_p), n,
                                     w.ctypes.data_as(C.c_void_p), eps)
    assert np.array_equal(got.view(np.uint64), ref.view(np.uint64))


def test_rmsnorm_divides_by_rms(orc):
    # RMSNormForwardPolymorphic (poly/norm.go:102-138): normed = x / rms, a
    # division, then T(normed * g); multiplying by 1/rms rounds the probe
    # elements to other fp32 values.
    P = _association_probes()
    probes = P["rmsnorm"]
    base = orc.normal_f32(P["base_n"], P["base_seed"])
    x = np.concatenate([base, np.array([p["x"] for p in probes], np.float32)])
    g = np.concatenate([orc.uniform_f32(P["base_n"], 0.5, 1.5, 606),
                        np.array([p["g"] for p in probes], np.float32)])
    n, eps = x.size, P["eps"]
    got = orc.rmsnorm_forward(np.stack([x, x[::-1].copy()]), g, eps)
    g64 = g.astype(np.float64)
    x64 = x.astype(np.float64)
    rms = math.sqrt(_seq_sum_sq(x64) / n + eps)
    ref = ((x64 / rms) * g64).astype(np.float32)
    alt = ((x64 * (1.0 / rms)) * g64).astype(np.float32)
    tail = slice(P["base_n"], None)
    assert np.all(ref[tail].view(np.uint32) != alt[tail].view(np.uint32)), \
        "a probe no longer separates division from the reciprocal"
    assert np.array_equal(got[0].view(np.uint32), ref.view(np.uint32))
    # second row (reversed: another sum order) still follows the formula
    xr = x64[::-1]
    rr = math.sqrt(_seq_sum_sq(xr) / n + eps)
    assert np.array_equal(got[1].view(np.uint32), ((xr / rr) * g64).astype(np.float32).view(np.uint32))


def test_norm_sums_are_sequential(orc):
    # every norm sums its squares in element order: a row whose pairwise and
    # sequential sums differ must follow the sequential one
    n = 4096
    x = orc.normal_f32(n, 607) * np.float32(1e3)
    x[::97] = np.float32(3e-4)
    x64 = x.astype(np.float64)
    seq = _seq_sum_sq(x64)
    assert seq != float(np.sum(x64 * x64)) or seq != math.fsum(x64 * x64)
    scale = 1.0 / math.sqrt(seq / n + 1e-5)
    want = (x64 * scale).astype(np.float32)
    got = orc.bitnet_rmsnorm_row(x, None, 1e-5)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rmsnorm_layer_closed_form(orc):
    x = np.full((2, 8), 3.0, np.float32)
    y = orc.rmsnorm_forward(x, np.ones(8, np.float32), eps=1e-6)
    assert np.all(y == np.float32(3.0 / math.sqrt(9.0 + 1e-6)))


def test_swiglu_stages_compose(orc):
    # the SwiGLU oracle is exactly: quant -> gate/up matvec -> gate product ->
    # inner norm -> quant -> down matvec, each stage checked against the
    # stand-alone oracle pieces pinned above.
    H, I = 64, 96
    g = orc.random_matrix(I, H, 11)
    u = orc.random_matrix(I, H, 12)
    d = orc.random_matrix(H, I, 13)
    x = orc.normal_f32(3 * H, 14).reshape(3, H)
    nw = orc.uniform_f32(I, 0.5, 1.5, 15)
    r = orc.swiglu_forward(g, u, d, x, inner_norm=nw, eps=1e-5)
    for s in range(3):
        xq, amax = orc.quant_act(x[s])
        assert np.array_equal(xq, r.xq[s]) and amax == r.amax[s]
        gv, ga = orc.matvec_scalar(g, xq, orc.output_scale(g.scale, amax))
        uv, ua = orc.matvec_scalar(u, xq, orc.output_scale(u.scale, amax))
        assert np.array_equal(ga, r.acc_gate[s]) and np.array_equal(ua, r.acc_up[s])
        h = np.array([orc.swiglu_gate_product(a, b) for a, b in zip(gv, uv)], np.float32)
        h = orc.bitnet_rmsnorm_row(h, nw, 1e-5)
        assert np.array_equal(h.view(np.uint32), r.h[s].view(np.uint32))
        hq, hamax = orc.quant_act(h)
        assert np.array_equal(hq, r.hq[s])
        dv, da = orc.matvec_scalar(d, hq, orc.output_scale(d.scale, hamax))
        assert np.array_equal(da, r.acc_down[s])
        assert np.array_equal(dv.astype(np.float32).view(np.uint32), r.out[s].view(np.uint32))


# ---------------------------------------------------------------- entity blob
def test_entity_blob_round_trip(orc):
    # TestEntityBitNetTernaryBlobRoundTrip (poly/tests/entity_test.go:331-348)
    words = np.array([0x49249249, 0x92492492, 0x24924924, 0x49249249, 0x92492492,
                      0x24924924, 0x49249249, 0x92492492], np.uint32)
    raw = orc.entity_encode(8, 4, 0, 0.05, 1, words)
    assert len(raw) == 24 + 32
    m, off = orc.entity_decode(raw)
    assert (m.rows, m.cols, off, m.row_words) == (8, 4, 0, 1)
    assert m.scale == np.float32(0.05)
    assert np.array_equal(m.words, words)
    # header layout: little endian u32 fields, scale as fp32 bits
    assert raw[:4] == (8).to_bytes(4, "little")
    assert raw[12:16] == np.float32(0.05).tobytes()
    with pytest.raises(ValueError):
        orc.entity_decode(raw[:20])
    with pytest.raises(ValueError):
        orc.entity_decode(raw[:40])


def test_entity_large_offset(orc):
    # TestEntityBitNetCollectLargeOffsetKeys (:352-412): offsets beyond 20000 survive
    raw = orc.entity_encode(4, 8, 6553600, 2.0, 1, np.array([9, 10, 11, 12], np.uint32))
    m, off = orc.entity_decode(raw)
    assert off == 6553600 and m.scale == 2.0
