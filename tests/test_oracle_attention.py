"""Pins the oracle's attention / block / LM-head restatements (CPU only).

Checks come from loom's own tests where they exist (DotTile order, LM head
SIMD-vs-scalar bar) and otherwise from what the mathematics fixes: closed
forms (one cached position, RoPE at position 0), an independent numpy
formulation (complex rotation for RoPE, matrix softmax attention with GQA
grouping), and invariants (incremental decode == full-sequence pass).
Citations are relative to the loom v0.83.0 tree.
"""
import math

import numpy as np
import pytest


# ---------------------------------------------------------------- DotTile / LM head
def avx2_order_reference(x, w, prev):
    """avx2OrderReference from poly/simd/dot_test.go:14-36 (loom's own spec of
    the amd64 kernel's order): two 4-lane accumulators over 8-wide blocks."""
    n = len(x)
    y0 = [0.0] * 4
    y1 = [0.0] * 4
    i = 0
    while i + 8 <= n:
        for j in range(4):
            y0[j] += float(x[i + j]) * float(w[i + j])
        for j in range(4):
            y1[j] += float(x[i + 4 + j]) * float(w[i + 4 + j])
        i += 8
    s = [y0[j] + y1[j] for j in range(4)]
    acc = (s[0] + s[2]) + (s[1] + s[3])
    acc += prev
    while i < n:
        acc += float(x[i]) * float(w[i])
        i += 1
    return acc


def test_dot_tile_matches_loom_avx2_order(orc):
    # TestDotTileMatchesAVX2Order (poly/simd/dot_test.go:38-60): bit-identical.
    rng = np.random.default_rng(1)
    for n in [0, 1, 2, 3, 7, 8, 9, 15, 16, 17, 31, 33, 64, 100, 257, 576, 1000, 1536]:
        for _ in range(20):
            x = rng.standard_normal(n).astype(np.float32)
            w = rng.standard_normal(n).astype(np.float32)
            prev = float(rng.standard_normal() * 3)
            got = orc.dot_tile(x, w, prev)
            want = avx2_order_reference(x, w, prev)
            assert np.float64(got).tobytes() == np.float64(want).tobytes(), (n, got, want)


def test_dot_tile_order_differs_from_sequential(orc):
    # A case where the tree and the sequential chain round differently, so a
    # plain sequential implementation cannot pass the test above by accident.
    x = np.array([1e16, 1, -1e16, 1, 1, 1, 1, 1] * 2, np.float32)
    w = np.ones(16, np.float32)
    seq = 0.0
    for a in x:
        seq += float(a)
    assert orc.dot_tile(x, w) != seq


def test_lm_head_simd_close_to_scalar(orc):
    # TestLMHeadFP32SimdMatchesScalar (poly/tests/lmhead_simd_test.go:16-57):
    # H=320, V=700, SIMD vs scalar within 1e-3; both within fp64 rounding of the exact sums.
    H, V = 320, 700
    table = orc.normal_f32(V * H, 3) * np.float32(0.05)
    hidden = orc.normal_f32(H, 4) * np.float32(0.1)
    a = orc.lm_head(hidden, table, simd=False)
    b = orc.lm_head(hidden, table, simd=True)
    assert np.abs(a - b).max() < 1e-3
    exact = np.array([math.fsum(float(h) * float(t) for h, t in zip(hidden, table[v * H:(v + 1) * H]))
                      for v in range(V)], np.float32)
    assert np.abs(a - exact).max() <= 1e-6 and np.abs(b - exact).max() <= 1e-6


def test_argmax_first_strict_max(orc):
    # SampleTopK greedy (poly/sampling.go:44-55): first strict maximum wins.
    assert orc.argmax_first(np.array([1, 3, 3, 2], np.float32)) == 1
    assert orc.argmax_first(np.array([5, 3, 5], np.float32)) == 0
    assert orc.argmax_first(np.array([np.nan, 3, 9], np.float32)) == 0  # NaN at 0 is never beaten
    assert orc.argmax_first(np.array([1, np.nan, 9], np.float32)) == 2  # NaN never wins
    assert orc.argmax_first(np.array([-np.inf, -3], np.float32)) == 1


# ---------------------------------------------------------------- MHA
HID, HEADS, KV, HD, MSL = 128, 4, 2, 32, 64


def make_mha(orc, seed=1, simd=True, msl=MSL):
    q = orc.random_matrix(HEADS * HD, HID, seed=seed)
    k = orc.random_matrix(KV * HD, HID, seed=seed + 1)
    v = orc.random_matrix(KV * HD, HID, seed=seed + 2)
    o = orc.random_matrix(HID, HEADS * HD, seed=seed + 3)
    wn = orc.uniform_f32(HEADS * HD, 0.5, 1.5, seed=seed + 4)
    return orc.MHA(q, k, v, o, HEADS, KV, HD, msl, theta=500000.0, eps=1e-5, inner_norm=wn,
                   simd=simd)


def test_mha_single_position_attention_is_v(orc):
    # One cached position: softmax weight exp(0)/exp(0) = 1 exactly, so the
    # attention output is float64(V) of that position, head by head (GQA).
    m = make_mha(orc)
    x = orc.normal_f32(HID, 7).reshape(1, HID)
    _, _, _, attn = m.forward(x)
    v_row = m.cache_v[: KV * HD].astype(np.float64)
    for h in range(HEADS):
        kvh = h // (HEADS // KV)
        assert np.array_equal(attn[0, h * HD:(h + 1) * HD], v_row[kvh * HD:(kvh + 1) * HD])


def test_mha_rope_identity_at_position_zero(orc):
    # angle 0 -> cos 1, sin 0: the cached K row at position 0 is the K
    # projection itself, i.e. loom's Dense packed path output.
    m = make_mha(orc)
    x = orc.normal_f32(HID, 8).reshape(1, HID)
    m.forward(x)
    kproj = orc.dense_forward(m.mats[1], x, simd=True).pre[0]
    assert np.array_equal(m.cache_k[: KV * HD], kproj)


def test_mha_rope_matches_complex_rotation(orc):
    # RoPE (poly/mha.go:292-313) is a rotation of the half-split pairs by
    # pos / theta^(2d/headDim): compare with numpy complex multiplication.
    m = make_mha(orc)
    S = 5
    x = orc.normal_f32(S * HID, 9).reshape(S, HID)
    m.forward(x)
    kproj = orc.dense_forward(m.mats[1], x, simd=True).pre  # before RoPE, fp32
    half = HD // 2
    for pos in range(S):
        got = m.cache_k[pos * KV * HD:(pos + 1) * KV * HD].reshape(KV, HD)
        raw = kproj[pos].reshape(KV, HD).astype(np.float64)
        d = np.arange(half)
        ang = pos / np.power(500000.0, 2 * d / HD)
        z = (raw[:, :half] + 1j * raw[:, half:]) * np.exp(1j * ang)
        want = np.concatenate([z.real, z.imag], axis=1).astype(np.float32)
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7)


def test_mha_attention_matches_numpy_softmax(orc):
    # Independent formulation: softmax(Q K^T / sqrt(hd)) V over the causal cache,
    # with GQA grouping h -> h // (heads / kv_heads).
    m = make_mha(orc, seed=11)
    S = 9
    x = orc.normal_f32(S * HID, 12).reshape(S, HID)
    _, _, q, attn = m.forward(x)
    K = m.cache_k[: S * KV * HD].reshape(S, KV, HD).astype(np.float64)
    V = m.cache_v[: S * KV * HD].reshape(S, KV, HD).astype(np.float64)
    for s in range(S):
        for h in range(HEADS):
            kvh = h // (HEADS // KV)
            qh = q[s, h * HD:(h + 1) * HD]
            sc = K[: s + 1, kvh] @ qh / math.sqrt(HD)
            p = np.exp(sc - sc.max())
            want = (p[:, None] * V[: s + 1, kvh]).sum(0) / p.sum()
            assert np.allclose(attn[s, h * HD:(h + 1) * HD], want, rtol=1e-12, atol=1e-14)


def test_mha_incremental_equals_full_pass(orc):
    # Decoding token by token through the warm KV cache gives the same bits as
    # one full-sequence pass (poly/mha_layout.go:62-70: seq 1 + warm cache is
    # incremental, anything else resets).
    S = 7
    x = orc.normal_f32(S * HID, 13).reshape(S, HID)
    full = make_mha(orc, seed=21)
    pre_f, post_f, _, _ = full.forward(x)
    inc = make_mha(orc, seed=21)
    inc.forward(x[:3])
    outs = []
    for s in range(3, S):
        pre_i, post_i, _, _ = inc.forward(x[s:s + 1])
        outs.append(post_i[0])
        assert inc.kv_offset == s + 1
    assert np.array_equal(np.stack(outs), post_f[3:])
    assert np.array_equal(inc.cache_k, full.cache_k)


def test_mha_prefill_resets_cache(orc):
    m = make_mha(orc, seed=31)
    x = orc.normal_f32(4 * HID, 32).reshape(4, HID)
    _, a, _, _ = m.forward(x)
    _, b, _, _ = m.forward(x)  # seq > 1 resets: same outputs again
    assert np.array_equal(a, b) and m.kv_offset == 4


# ---------------------------------------------------------------- block
def test_block_is_norm_mha_add_norm_swiglu_add(orc):
    # forwardOnCPUNormal (poly/transformer_forward.go:228-245) composed from
    # the separately pinned pieces: bit-identical.
    S, inter = 6, 256
    n1 = orc.uniform_f32(HID, 0.5, 1.5, 41)
    n2 = orc.uniform_f32(HID, 0.5, 1.5, 42)
    g = orc.random_matrix(inter, HID, 43)
    u = orc.random_matrix(inter, HID, 44)
    d = orc.random_matrix(HID, inter, 45)
    fn = orc.uniform_f32(inter, 0.5, 1.5, 46)
    blk = orc.Block(make_mha(orc, seed=51), n1, n2, g, u, d, fn)
    x = orc.normal_f32(S * HID, 47).reshape(S, HID)
    got = blk.forward(x)

    mha = make_mha(orc, seed=51)
    y = orc.rmsnorm_forward(x, n1, 1e-5)
    _, o, _, _ = mha.forward(y)
    h = (o + x).astype(np.float32)
    y2 = orc.rmsnorm_forward(h, n2, 1e-5)
    f = orc.swiglu_forward(g, u, d, y2, inner_norm=fn, eps=1e-5).out
    want = (f + h).astype(np.float32)
    assert np.array_equal(got, want)


def test_mha_stages_compose_to_forward(orc):
    # The stage entry points used by the GPU stage checks (attention, output
    # projection) reproduce MHA.forward bit for bit.
    m = make_mha(orc, seed=61)
    S = 6
    x = orc.normal_f32(S * HID, 62).reshape(S, HID)
    pre, post, q, attn = m.forward(x)
    a = orc.attention(q, m.cache_k.reshape(MSL, KV * HD), m.cache_v.reshape(MSL, KV * HD), 0, MSL,
                      HEADS, KV, HD)
    assert np.array_equal(a, attn)
    p2, o2 = orc.attn_out(m.mats[3], attn, inner_norm=m.inner_norm, eps=1e-5)
    assert np.array_equal(p2, pre) and np.array_equal(o2, post)


def test_mha_project_and_row_stages_compose(orc):
    # The finer stages of the GPU stage checks reproduce MHA.forward bit for
    # bit: project (Q and the K/V cache rows), attention of single rows at
    # their own positions, the fp64 inner norm + requantization, and the O
    # projection from the int8 rows (dense_quantized) with a bias.
    import ctypes as C
    m = make_mha(orc, seed=63)
    bo = orc.normal_f32(HID, 64) * np.float32(0.1)
    m._bo = bo
    m.c.bias_o = bo.ctypes.data_as(C.c_void_p)
    S = 7
    x = orc.normal_f32(S * HID, 65).reshape(S, HID)
    pre, post, q, attn = m.forward(x)
    m2 = make_mha(orc, seed=63)
    q2 = m2.project(x, 0)
    assert np.array_equal(q2, q)
    assert np.array_equal(m2.cache_k, m.cache_k) and np.array_equal(m2.cache_v, m.cache_v)
    ck, cv = m2.cache_k.reshape(MSL, KV * HD), m2.cache_v.reshape(MSL, KV * HD)
    for r in (0, 3, S - 1):
        a = orc.attention(q2[r:r + 1], ck, cv, r, MSL, HEADS, KV, HD)
        assert np.array_equal(a[0], attn[r])
    normed = attn.copy()
    for r in range(S):
        orc.lib().orc_bitnet_rmsnorm_f64(normed[r].ctypes.data_as(C.c_void_p), normed.shape[1],
                                         m.inner_norm.ctypes.data_as(C.c_void_p), 1e-5)
    assert np.array_equal(normed.astype(np.float32), pre)
    aq, aam = orc.quant_rows(normed)
    assert np.array_equal(orc.dense_quantized(m.mats[3], aq, aam, bias=bo), post)


def test_swiglu_row_stages_compose(orc):
    # swiglu_gate_rows + inner norm + requantization + dense_quantized (down)
    # reproduce swiglu_forward bit for bit, with biases, for both gates.
    H, I = 64, 96
    g = orc.random_matrix(I, H, 71)
    u = orc.random_matrix(I, H, 72)
    d = orc.random_matrix(H, I, 73)
    nw = orc.uniform_f32(I, 0.5, 1.5, 74)
    bias = orc.normal_f32(2 * I + H, 75) * np.float32(0.1)
    x = orc.normal_f32(4 * H, 76).reshape(4, H)
    for act in (orc.ACT_SILU, orc.ACT_RELU2):
        r = orc.swiglu_forward(g, u, d, x, inner_norm=nw, bias=bias, eps=1e-5, activation=act)
        xq, am = orc.quant_rows(x)
        assert np.array_equal(xq, r.xq) and np.array_equal(am, r.amax)
        h = orc.swiglu_gate_rows(g, u, xq, am, activation=act, bias=bias[:2 * I])
        hn = np.stack([orc.bitnet_rmsnorm_row(h[i], nw, 1e-5) for i in range(4)])
        assert np.array_equal(hn.view(np.uint32), r.h.view(np.uint32))
        hq, ham = orc.quant_rows(hn)
        assert np.array_equal(hq, r.hq) and np.array_equal(ham, r.hamax)
        out = orc.dense_quantized(d, hq, ham, bias=bias[2 * I:])
        assert np.array_equal(out.view(np.uint32), r.out.view(np.uint32))


def test_attention_threads_do_not_change_bits(orc):
    # the oracle splits (query, head) pairs over threads; each pair runs the
    # reference's loops, so 1 thread and many give the same bytes
    import os
    import subprocess
    import sys
    code = ("import numpy as np, sys; sys.path.insert(0, %r); from oracle import oracle as orc; "
            "q = orc.normal_f32(5*4*32, 1).astype(np.float64).reshape(5, 128); "
            "k = orc.normal_f32(40*64, 2).reshape(40, 64); v = orc.normal_f32(40*64, 3).reshape(40, 64); "
            "a = orc.attention(q, k, v, 30, 40, 4, 2, 32); sys.stdout.write(a.tobytes().hex())")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    outs = []
    for th in ("1", "6"):
        env = dict(os.environ, OMP_NUM_THREADS=th)
        outs.append(subprocess.run([sys.executable, "-c", code % root], env=env, check=True,
                                   capture_output=True, text=True).stdout)
    assert outs[0] == outs[1] and len(outs[0]) > 0


def test_lm_head_scalar_order_pinned(orc):
    # The scalar head (poly/transformer.go:681-687, dotTileGo in
    # poly/simd/dot.go:14-21) is one sequential fp64 sum per logit: equal bit
    # for bit to the same loop in Python floats (fp64), ragged widths included.
    for V, H in [(5, 1), (7, 13), (9, 37), (4, 300)]:
        table = orc.normal_f32(V * H, 40 + H) * np.float32(0.3)
        hidden = orc.normal_f32(H, 50 + H)
        got = orc.lm_head(hidden, table, simd=False)
        for v in range(V):
            s = 0.0
            for d in range(H):
                s += float(hidden[d]) * float(table[v * H + d])
            assert got[v] == np.float32(s), (V, H, v)
    # A row whose two orders differ: x = 2^30 everywhere, w = (1, 1, -1, 0...)
    # scaled so the products are 2^60, 1, -2^60.  In order the 1 is absorbed
    # (2^60 + 1 rounds to 2^60) and the sum is 0; DotTile keeps the three in
    # separate lanes and returns 1.
    H = 16
    hidden = np.full(H, 2.0 ** 30, np.float32)
    row = np.zeros(H, np.float32)
    row[0], row[1], row[2] = 2.0 ** 30, 2.0 ** -30, -(2.0 ** 30)
    assert orc.lm_head(hidden, row, simd=False)[0] == 0.0
    assert orc.lm_head(hidden, row, simd=True)[0] == 1.0


def test_attention_two_stages_compose_to_attention(orc):
    # orc_attention_args -> exp -> orc_attention_chains (the split used to
    # check a device's chains given the device's own exp) reproduces the
    # attention of poly/mha.go:316-354 bit for bit: GQA, a nonzero base,
    # listed rows in any subset, a ring shorter than the positions.
    rng = np.random.default_rng(81)
    for heads, kv, hd, S, base, msl in [(4, 2, 32, 5, 0, 40), (6, 3, 16, 4, 9, 20),
                                        (8, 1, 64, 3, 30, 33), (2, 2, 8, 6, 12, 10)]:
        q = rng.standard_normal((S, heads * hd)) * 2.0
        ck = rng.standard_normal((msl, kv * hd)).astype(np.float32)
        cv = rng.standard_normal((msl, kv * hd)).astype(np.float32)
        want = orc.attention(q, ck, cv, base, msl, heads, kv, hd)
        for rows in (None, [S - 1], [0, S - 1], list(range(0, S, 2))):
            r = np.arange(S) if rows is None else np.asarray(rows)
            args = orc.attention_args(q, ck, base, msl, heads, kv, hd, rows=r)
            assert args.size == sum(heads * (base + int(i) + 1) for i in r)
            assert np.all(args <= 0.0)  # score - max
            got = orc.attention_chains(orc.exp_rows(args), cv, base, msl, heads, kv, hd, r)
            assert got.tobytes() == want[r].tobytes(), (heads, kv, hd, base, rows)


def test_attention_args_are_dimension_order_chains(orc):
    # Each exp argument is (sum_d Q*K in dimension order) * scale - max: on a
    # row whose terms cancel, the dimension-order chain and a pairwise sum
    # give different scores, and the oracle takes the chain's.
    hd, heads, kv = 4, 1, 1
    q = np.array([[1e16, 1.0, -1e16, 1.0]])
    ck = np.array([[1, 1, 1, 1], [0, 0, 0, 0]], np.float32)
    args = orc.attention_args(q, ck, 1, 2, heads, kv, hd, rows=[0])
    chain = ((1e16 + 1.0) - 1e16) + 1.0          # = 1.0 in fp64 (1e16 + 1 rounds to 1e16)
    assert chain == 1.0 and (1e16 - 1e16) + (1.0 + 1.0) == 2.0
    score0 = chain * (1.0 / math.sqrt(hd))
    mx = max(score0, 0.0)
    assert args.tolist() == [score0 - mx, 0.0 - mx]
    # probabilities then expSum and the position-order value chain
    cv = np.array([[1e16, 0, 0, 0], [1.0, 0, 0, 0]], np.float32)
    p = np.array([1.0, 0.5])
    out = orc.attention_chains(p, cv, 1, 2, heads, kv, hd, [0])
    assert out[0, 0] == (1.0 * float(np.float32(1e16)) + 0.5 * 1.0) / 1.5


def test_attention_chains_detect_another_order(orc):
    # The bit-exact check of a device's strict attention against
    # attention_chains would catch a device that summed in another order:
    # the same probabilities summed in reverse position order (or by a
    # pairwise tree) give different bits for most outputs at these sizes.
    rng = np.random.default_rng(83)
    heads, kv, hd, base, msl = 4, 1, 64, 300, 301
    q = rng.standard_normal((1, heads * hd))
    ck = rng.standard_normal((msl, kv * hd)).astype(np.float32)
    cv = rng.standard_normal((msl, kv * hd)).astype(np.float32)
    args = orc.attention_args(q, ck, base, msl, heads, kv, hd, rows=[0])
    p = orc.exp_rows(args).reshape(heads, base + 1)
    got = orc.attention_chains(p.ravel(), cv, base, msl, heads, kv, hd, [0])[0].reshape(heads, hd)
    v = cv[:base + 1].astype(np.float64)
    rev = np.zeros((heads, hd))
    es = np.zeros(heads)
    for kp in range(base, -1, -1):
        rev += p[:, kp:kp + 1] * v[kp][None, :]
        es += p[:, kp]
    rev /= es[:, None]
    tree = (p @ v) / p.sum(axis=1, keepdims=True)   # BLAS / pairwise orders
    assert np.count_nonzero(rev != got) > got.size // 4
    assert np.count_nonzero(tree != got) > got.size // 4
    assert np.max(np.abs(rev - got)) < 1e-13  # same values, other roundings


# ---------------------------------------------------------------- per-head Q/K RMSNorm
def test_qk_norm_eps_rule(orc):
    # mhaQKNormEpsilon (poly/mha.go:19-24): RMSNormEps when set, else 1e-6
    assert orc.lib().orc_qk_norm_eps(0.0) == 1e-6
    assert orc.lib().orc_qk_norm_eps(-1.0) == 1e-6
    assert orc.lib().orc_qk_norm_eps(1e-5) == 1e-5


def test_per_head_rmsnorm_constant_head_closed_form(orc):
    # a constant head c (a power of two: every square and partial sum exact):
    # rms = sqrt(c^2 + eps), x = c * (1/rms) * g (poly/mha.go:584-614)
    heads, hd, c = 3, 64, 0.25
    for eps in (1e-5, 1e-6):
        x = np.full(heads * hd, c)
        got = orc.per_head_rmsnorm(x, None, heads, hd, eps)
        inv = 1.0 / math.sqrt((hd * (c * c)) / hd + eps)
        assert np.all(got == c * inv * 1.0)
    # eps <= 0 inside the helper -> 1e-6
    a = orc.per_head_rmsnorm(np.full(hd, c), None, 1, hd, 0.0)
    b = orc.per_head_rmsnorm(np.full(hd, c), None, 1, hd, 1e-6)
    assert np.array_equal(a, b)


def test_per_head_rmsnorm_gamma_lengths(orc):
    # gamma of length head_dim is shared by every head; of length
    # heads*head_dim, one block per head; any other length -> unit weights
    rng = np.random.default_rng(91)
    heads, hd = 4, 32
    x = rng.standard_normal(heads * hd)
    g1 = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    shared = orc.per_head_rmsnorm(x, g1, heads, hd, 1e-6)
    tiled = orc.per_head_rmsnorm(x, np.tile(g1, heads), heads, hd, 1e-6)
    assert np.array_equal(shared, tiled)
    gh = rng.uniform(0.5, 1.5, heads * hd).astype(np.float32)
    per = orc.per_head_rmsnorm(x, gh, heads, hd, 1e-6)
    unit = orc.per_head_rmsnorm(x, None, heads, hd, 1e-6)
    odd = orc.per_head_rmsnorm(x, gh[:hd + 1], heads, hd, 1e-6)
    assert np.array_equal(odd, unit)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        xs = x[sl]
        s = 0.0
        for v in xs:
            s += v * v
        inv = 1.0 / math.sqrt(s / hd + 1e-6)
        assert per[sl].tolist() == [float(a) * inv * float(g) for a, g in zip(xs, gh[sl])]
        assert unit[sl].tolist() == [float(a) * inv * 1.0 for a in xs]


def test_per_head_rmsnorm_order_and_association(orc):
    # the sum of squares is the dimension-order chain: 2^27 then 63 ones
    # (each 1 is lost against 2^54 in order; a pairwise sum keeps 64)
    hd = 64
    x = np.ones(hd)
    x[0] = 2.0**27
    got = orc.per_head_rmsnorm(x, None, 1, hd, 1e-6)
    inv_chain = 1.0 / math.sqrt(2.0**54 / hd + 1e-6)
    inv_pair = 1.0 / math.sqrt((2.0**54 + 64) / hd + 1e-6)
    assert inv_chain != inv_pair
    assert got[1] == 1.0 * inv_chain * 1.0
    # x * inv * g is (x * inv) * g: probes where x * (inv * g) rounds differently
    rng = np.random.default_rng(92)
    found = 0
    for _ in range(200):
        xs = rng.standard_normal(hd)
        g = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        out = orc.per_head_rmsnorm(xs, g, 1, hd, 1e-6)
        s = 0.0
        for v in xs:
            s += v * v
        inv = 1.0 / math.sqrt(s / hd + 1e-6)
        left = [(float(a) * inv) * float(b) for a, b in zip(xs, g)]
        right = [float(a) * (inv * float(b)) for a, b in zip(xs, g)]
        assert out.tolist() == left
        found += sum(1 for a, b in zip(left, right) if a != b)
    assert found > 50


def test_per_head_rmsnorm_f32_rounds_each_result(orc):
    # applyPerHeadRMSNormTensor[float32]: fp64 arithmetic on the widened
    # values, each result rounded to fp32
    rng = np.random.default_rng(93)
    heads, hd = 2, 16
    x = rng.standard_normal(heads * hd).astype(np.float32)
    g = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    got = orc.per_head_rmsnorm(x, g, heads, hd, 1e-6)
    assert got.dtype == np.float32
    for h in range(heads):
        xs = x[h * hd:(h + 1) * hd]
        s = 0.0
        for v in xs:
            s += float(v) * float(v)
        inv = 1.0 / math.sqrt(s / hd + 1e-6)
        want = np.array([float(a) * inv * float(b) for a, b in zip(xs, g)], np.float32)
        assert got[h * hd:(h + 1) * hd].tobytes() == want.tobytes()


def _make_mha_qk(orc, seed, q_norm, k_norm, eps=1e-5):
    q = orc.random_matrix(HEADS * HD, HID, seed=seed)
    k = orc.random_matrix(KV * HD, HID, seed=seed + 1)
    v = orc.random_matrix(KV * HD, HID, seed=seed + 2)
    o = orc.random_matrix(HID, HEADS * HD, seed=seed + 3)
    wn = orc.uniform_f32(HEADS * HD, 0.5, 1.5, seed=seed + 4)
    return orc.MHA(q, k, v, o, HEADS, KV, HD, MSL, theta=500000.0, eps=eps, inner_norm=wn,
                   q_norm=q_norm, k_norm=k_norm)


def test_mha_qk_norm_before_rope(orc):
    # MHAForwardPackedTernaryCPU (poly/mha.go:281-314): Q (fp64, after bias)
    # and the fp32 K cache row are normalized per head, then rotated.  At
    # position 0 the rotation is the identity, so Q and K equal the norms of
    # the plain projections bit for bit; at later positions they equal the
    # rotation (numpy complex multiply) of the normalized rows within 1e-12,
    # and differ from normalizing the rotated rows (gamma is per dimension).
    gq = orc.uniform_f32(HD, 0.5, 1.5, seed=94)
    gk = orc.uniform_f32(KV * HD, 0.5, 1.5, seed=95)
    for eps, qk_eps in ((1e-5, 1e-5), (0.0, 1e-6)):
        x = orc.normal_f32(HID, 96).reshape(1, HID)
        plain = _make_mha_qk(orc, 97, None, None, eps=eps)
        q_raw = plain.project(x, 0)[0]
        k_raw = plain.cache_k[:KV * HD].copy()
        m = _make_mha_qk(orc, 97, gq, gk, eps=eps)
        q0 = m.project(x, 0)[0]
        assert q0.tobytes() == orc.per_head_rmsnorm(q_raw, gq, HEADS, HD, qk_eps).tobytes()
        assert m.cache_k[:KV * HD].tobytes() == orc.per_head_rmsnorm(k_raw, gk, KV, HD, qk_eps).tobytes()
        assert np.array_equal(m.cache_v[:KV * HD], plain.cache_v[:KV * HD])  # V untouched
        pos, half = 37, HD // 2
        qp = m.project(x, pos)[0]
        qn = orc.per_head_rmsnorm(q_raw, gq, HEADS, HD, qk_eps)

        def rope(row):
            out = np.empty_like(row)
            for h in range(HEADS):
                d = np.arange(half)
                ang = pos / np.power(500000.0, 2 * d / HD)
                z = (row[h * HD:h * HD + half] + 1j * row[h * HD + half:(h + 1) * HD]) * np.exp(1j * ang)
                out[h * HD:h * HD + half], out[h * HD + half:(h + 1) * HD] = z.real, z.imag
            return out
        want = rope(qn)
        assert np.abs(qp - want).max() <= 1e-12 * np.abs(want).max()
        other = orc.per_head_rmsnorm(rope(q_raw), gq, HEADS, HD, qk_eps)
        assert np.abs(qp - other).max() > 1e-6 * np.abs(want).max()


def test_mha_qk_norm_forward_composes(orc):
    # a whole forward with Q/K norms equals its stages: project (with the
    # norms), attention over the caches, output stage
    gq = orc.uniform_f32(HEADS * HD, 0.5, 1.5, seed=98)
    gk = orc.uniform_f32(HD, 0.5, 1.5, seed=99)
    m = _make_mha_qk(orc, 101, gq, gk)
    S = 6
    x = orc.normal_f32(S * HID, 102).reshape(S, HID)
    pre, post, q, attn = m.forward(x)
    m2 = _make_mha_qk(orc, 101, gq, gk)
    q2 = m2.project(x, 0)
    assert np.array_equal(q2, q)
    ck, cv = m2.cache_k.reshape(MSL, KV * HD), m2.cache_v.reshape(MSL, KV * HD)
    assert np.array_equal(orc.attention(q2, ck, cv, 0, MSL, HEADS, KV, HD), attn)


def test_mha_batch_is_one_timeline(orc):
    # loom's [batch, seq, d_model] input (poly/mha.go:251-371): the batch's
    # sequences share one KV timeline from position 0, so the literal batch
    # loop equals one call on the batch's rows concatenated -- the mapping the
    # device block's shared-timeline call uses.  Both then continue the same
    # way with warm single-token steps, and a later batch call restarts.
    B, S = 3, 5
    x = orc.normal_f32(B * S * HID, 201).reshape(B, S, HID)
    mb, mf = make_mha(orc, seed=202), make_mha(orc, seed=202)
    pre_b, post_b = mb.forward_batch(x)
    pre_f, post_f, _, _ = mf.forward(x.reshape(B * S, HID))
    assert np.array_equal(pre_b.reshape(B * S, HID), pre_f)
    assert np.array_equal(post_b.reshape(B * S, HID), post_f)
    assert mb.kv_offset == mf.kv_offset == B * S
    assert np.array_equal(mb.cache_k, mf.cache_k) and np.array_equal(mb.cache_v, mf.cache_v)
    # the last sequence's first query attends to the earlier sequences' rows:
    # running that sequence alone (its own timeline from 0) gives other values
    alone = make_mha(orc, seed=202)
    _, post_alone, _, _ = alone.forward(x[B - 1])
    assert not np.array_equal(post_alone, post_b[B - 1])
    for step in range(3):
        x1 = orc.normal_f32(HID, 210 + step).reshape(1, 1, HID)
        _, pb = mb.forward_batch(x1)
        _, pf, _, _ = mf.forward(x1.reshape(1, HID))
        assert np.array_equal(pb.reshape(1, HID), pf)
    assert mb.kv_offset == B * S + 3
    pre_b2, post_b2 = mb.forward_batch(x)  # not a single-token step: restarts at 0
    assert mb.kv_offset == B * S
    assert np.array_equal(post_b2, post_b)
