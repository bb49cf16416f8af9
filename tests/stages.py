"""Stage-wise parity checks of the gfx950 decoder block against the CPU oracle
(loom's MHAForwardPackedTernaryCPU / forwardOnCPUNormal restated).  Shared by
the GPU test modules; not collected itself.

Every stage is compared with the oracle fed the GPU's own input to that stage,
so a difference is pinned to the stage that made it.  Bars:
  * int8 quantization of the GPU's normalized rows, and every projection from
    the GPU's int8 rows (O + bias + residual, gate/up, down + residual):
    bit-exact in both norm modes;
  * RMSNorm1/2 and the SwiGLU inner norm (fp32 rows): bit-exact in strict
    mode (the reference's sequential fp64 sums), within 1 fp32 ulp in fast
    mode (fixed-order tree sums);
  * the MHA inner norm (fp64 rows): bit-exact strict, within 1e-13 of the row
    scale fast;
  * Q after RoPE within 1e-12 of the row scale (pow/cos/sin last bits;
    bit-exact at position 0, where the rotation is the identity), the K cache
    within 1 fp32 ulp (V bit-exact), attention within 1e-12 of the row scale
    of the oracle (exp last bits; fast mode also sums in another fixed
    order); in strict mode the attention is also bit-exact against the
    oracle's exp-free chains (dimension-order scores, maximum, position-order
    expSum and value sums, division) evaluated around the device's own exp,
    which pins every summation order of poly/mha.go:316-354;
  * the SiLU gate product (exp) within 1 fp32 ulp; ReLU2 bit-exact.
Citations are relative to the loom v0.83.0 tree.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

ACT_SILU, ACT_RELU2 = 1, 6


class Shape:
    def __init__(self, hidden, heads, kv, hd, inter, msl, theta=500000.0):
        self.hidden, self.heads, self.kv, self.hd, self.inter, self.msl = hidden, heads, kv, hd, inter, msl
        self.theta = theta
        self.q_dim, self.kv_dim = heads * hd, kv * hd


SMALL = Shape(256, 4, 2, 64, 512, 64)
BITNET_2B = Shape(2560, 20, 5, 128, 6912, 640)  # BitNet-b1.58-2B block (config 2)


class Weights:
    """Oracle matrices + fp32 vectors of one block (seeded)."""

    def __init__(self, orc, sh: Shape, seed: int, act: int = ACT_RELU2, bias: bool = False,
                 qk: str | None = None, attn_eps: float = 1e-5):
        """qk: per-head Q/K norm weights (poly/mha.go:285-290): None, "shared"
        (length head_dim), "per_head" (heads*head_dim and kv_heads*head_dim),
        "odd" (a Q norm of another length: unit weights; no K norm).
        attn_eps: the MHA layer's RMSNormEps (0: inner 1e-5, Q/K 1e-6)."""
        self.sh, self.act = sh, act
        self.attn_eps = attn_eps
        self.q = orc.random_matrix(sh.q_dim, sh.hidden, seed)
        self.k = orc.random_matrix(sh.kv_dim, sh.hidden, seed + 1)
        self.v = orc.random_matrix(sh.kv_dim, sh.hidden, seed + 2)
        self.o = orc.random_matrix(sh.hidden, sh.q_dim, seed + 3)
        self.g = orc.random_matrix(sh.inter, sh.hidden, seed + 4)
        self.u = orc.random_matrix(sh.inter, sh.hidden, seed + 5)
        self.d = orc.random_matrix(sh.hidden, sh.inter, seed + 6)
        self.n1 = orc.uniform_f32(sh.hidden, 0.5, 1.5, seed + 7)
        self.n2 = orc.uniform_f32(sh.hidden, 0.5, 1.5, seed + 8)
        self.an = orc.uniform_f32(sh.q_dim, 0.5, 1.5, seed + 9)
        self.fn = orc.uniform_f32(sh.inter, 0.5, 1.5, seed + 10)
        self.bias = None
        if bias:
            self.bias = [orc.normal_f32(n, seed + 11 + i) * np.float32(0.1)
                         for i, n in enumerate([sh.q_dim, sh.kv_dim, sh.kv_dim, sh.hidden])]
        self.qn = self.kn = None
        if qk == "shared":
            self.qn = orc.uniform_f32(sh.hd, 0.5, 1.5, seed + 20)
            self.kn = orc.uniform_f32(sh.hd, 0.5, 1.5, seed + 21)
        elif qk == "per_head":
            self.qn = orc.uniform_f32(sh.q_dim, 0.5, 1.5, seed + 20)
            self.kn = orc.uniform_f32(sh.kv_dim, 0.5, 1.5, seed + 21)
        elif qk == "odd":
            self.qn = orc.uniform_f32(sh.hd + 3, 0.5, 1.5, seed + 20)
        elif qk is not None:
            raise ValueError(qk)

    def gpu(self, tf):
        from loom_amd.bitnet import TernaryMatrix

        def m(x):
            return TernaryMatrix.from_words(x.words, x.rows, x.cols, x.scale)

        b = self.bias or [None] * 4
        return tf.BlockWeights(m(self.q), m(self.k), m(self.v), m(self.o), m(self.g), m(self.u),
                               m(self.d), self.n1, self.n2, self.an, self.fn, *b,
                               q_norm=self.qn, k_norm=self.kn)

    def cfg(self, tf, norm="strict", max_batch=1):
        sh = self.sh
        return tf.BlockConfig(sh.hidden, sh.heads, sh.kv, sh.hd, sh.inter, max_seq_len=sh.msl,
                              max_batch=max_batch, rope_theta=sh.theta, norm_eps=1e-5,
                              attn_eps=self.attn_eps, ffn_eps=1e-5, ffn_activation=self.act,
                              norm=norm)

    def oracle_mha(self, orc):
        sh = self.sh
        m = orc.MHA(self.q, self.k, self.v, self.o, sh.heads, sh.kv, sh.hd, sh.msl,
                    theta=sh.theta, eps=self.attn_eps, inner_norm=self.an, q_norm=self.qn,
                    k_norm=self.kn)
        if self.bias:
            # the oracle MHA wrapper has no bias arguments: set them on its C struct
            self._bias_keep = [np.ascontiguousarray(b, np.float32) for b in self.bias]
            from oracle.oracle import _p
            m.c.bias_q, m.c.bias_k, m.c.bias_v, m.c.bias_o = (_p(b) for b in self._bias_keep)
        return m

    def oracle_block(self, orc):
        return orc.Block(self.oracle_mha(orc), self.n1, self.n2, self.g, self.u, self.d, self.fn,
                         norm_eps=1e-5, ffn_eps=1e-5, ffn_activation=self.act)


def ulp_diff_f32(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _f32_rows(got, want, strict, what):
    if strict:
        bad = np.count_nonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad == 0, f"{what}: {bad} elements not bit-exact"
    else:
        u = ulp_diff_f32(got, want).max()
        assert u <= 1, f"{what}: {u} fp32 ulps from the oracle (fast bar: 1)"


def _quant(orc, rows, xq, amax, what):
    # bitNetQuantizeActivationNumeric / ...Float64 (poly/bitnet_cpu.go:45-117)
    # of the GPU's own rows: bit-exact
    q_ref, a_ref = orc.quant_rows(rows)
    assert np.array_equal(xq, q_ref), f"{what}: {np.count_nonzero(xq != q_ref)} int8 values differ"
    assert amax.tobytes() == a_ref.tobytes(), f"{what}: amax differs"


def _rel_rows(got, want, tol, what):
    scale = np.abs(want).max(axis=1, keepdims=True)
    err = (np.abs(got - want) / np.where(scale > 0, scale, 1.0)).max()
    assert err <= tol, f"{what}: off by {err:.3e} of the row scale (bar {tol:g})"


def device_exp(a):
    """exp of fp64 values with the device exp the library's kernels call
    (loom_amd_exp_rows)."""
    import torch
    from loom_amd import _lib
    x = torch.from_numpy(np.ascontiguousarray(a, np.float64)).cuda()
    y = torch.empty_like(x)
    rc = _lib.lib().loom_amd_exp_rows(C.c_void_p(x.data_ptr()), x.numel(), C.c_void_p(y.data_ptr()),
                                      C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, _lib.lib().loom_amd_last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy()


def strict_attention_bit_exact(orc, sh, q, cache_k, cache_v, base, R, attn):
    """Strict attention rows R against the reference's chains around the
    device's exp (poly/mha.go:324-352): the exp arguments score - max from the
    GPU's Q and K cache (dimension-order dots, maximum from -1e9), the
    device's exp of them, then expSum and the value sums in position order
    and the division -- every value bit for bit."""
    args = orc.attention_args(q, cache_k, base, sh.msl, sh.heads, sh.kv, sh.hd, rows=R)
    ref = orc.attention_chains(device_exp(args), cache_v, base, sh.msl, sh.heads, sh.kv, sh.hd, R)
    bad = np.count_nonzero(attn.view(np.uint64) != ref.view(np.uint64))
    assert bad == 0, f"strict attention: {bad} of {attn.size} values differ from the reference chains"


def f64_inner_norm(orc, rows, w, eps=1e-5):
    """bitNetRMSNormFloat64Weighted (poly/bitnet_cpu.go:868-887) per row."""
    out = np.array(rows, np.float64, copy=True)
    wp = np.ascontiguousarray(w, np.float32)
    for r in range(out.shape[0]):
        orc.lib().orc_bitnet_rmsnorm_f64(out[r].ctypes.data_as(C.c_void_p), out.shape[1],
                                         wp.ctypes.data_as(C.c_void_p), eps)
    return out


def check_stages(orc, w: Weights, mha_ref, x_in, T, out, cache_k, cache_v, base, strict=True,
                 rows=None):
    """Stage-wise parity of one GPU block call over the seq token rows of one
    sequence at positions base..base+seq-1.

    T: the call's taps as numpy arrays (BlockTaps.numpy()); out: the block's
    output rows; cache_k/v: the GPU's ring caches of the sequence.  mha_ref:
    an oracle MHA whose caches hold the positions before base; this call's
    K/V rows are written into it.  rows: the row indices checked past the
    Q/K/V projection (None = all rows); every row's Q and K/V are checked."""
    sh = w.sh
    seq = x_in.shape[0]
    R = np.arange(seq) if rows is None else np.unique(np.asarray(rows))
    # RMSNorm1 (poly/norm.go:102-138) and its quantization
    y1 = T["y1"]
    _f32_rows(y1[R], orc.rmsnorm_forward(x_in[R], w.n1, 1e-5), strict, "rmsnorm1")
    _quant(orc, y1[R], T["xq1"][R], T["amax1"][R], "rmsnorm1 int8")
    # Q/K/V + bias + RoPE (poly/mha.go:262-314), the oracle fed the GPU's y1
    q_ref = mha_ref.project(y1, base)
    q = T["q"]
    _rel_rows(q, q_ref, 1e-12, "Q after RoPE")
    if base == 0:
        # position 0: cos = 1, sin = 0 exactly -> the rotation is the identity
        assert np.array_equal(q[0], q_ref[0])
    kd = sh.kv_dim
    ck_ref = mha_ref.cache_k.reshape(sh.msl, kd)
    cv_ref = mha_ref.cache_v.reshape(sh.msl, kd)
    span = slice(base, base + seq)
    assert np.array_equal(cache_v[span], cv_ref[span]), "V cache not bit-exact"
    assert ulp_diff_f32(cache_k[span], ck_ref[span]).max() <= 1, "K cache beyond 1 ulp"
    if base == 0:
        assert np.array_equal(cache_k[0], ck_ref[0])
    # attention (poly/mha.go:316-354), the oracle fed the GPU's Q and caches
    if rows is None:
        attn_ref = orc.attention(q, cache_k, cache_v, base, sh.msl, sh.heads, sh.kv, sh.hd)
    else:
        attn_ref = np.stack([orc.attention(q[r:r + 1], cache_k, cache_v, base + int(r), sh.msl,
                                           sh.heads, sh.kv, sh.hd)[0] for r in R])
    attn = T["attn"][R]
    _rel_rows(attn, attn_ref, 1e-12, "attention")
    if strict:
        strict_attention_bit_exact(orc, sh, q, cache_k, cache_v, base, R, attn)
    # MHA inner norm of the GPU's attention rows (poly/mha.go:356-360) and the
    # fp64 requantization
    an = T["attn_norm"][R]
    an_ref = f64_inner_norm(orc, attn, w.an)
    if strict:
        assert np.array_equal(an.view(np.uint64), an_ref.view(np.uint64)), "MHA inner norm not bit-exact"
    else:
        _rel_rows(an, an_ref, 1e-13, "MHA inner norm")
    _quant(orc, an, T["aq"][R], T["aamax"][R], "attention int8")
    # O projection + bias (poly/mha.go:362-368) + residual
    # (poly/transformer_forward.go:236), from the GPU's int8 rows
    bo = w.bias[3] if w.bias else None
    o = orc.dense_quantized(w.o, T["aq"][R], T["aamax"][R], bias=bo)
    mid = T["mid"]
    mid_ref = (o + x_in[R]).astype(np.float32)
    assert np.array_equal(mid[R].view(np.uint32), mid_ref.view(np.uint32)), \
        "O projection + residual not bit-exact"
    # RMSNorm2 of the GPU's mid and its quantization
    y2 = T["y2"][R]
    _f32_rows(y2, orc.rmsnorm_forward(mid[R], w.n2, 1e-5), strict, "rmsnorm2")
    _quant(orc, y2, T["xq2"][R], T["amax2"][R], "rmsnorm2 int8")
    # gate/up + gate product (poly/swiglu.go:303-312) from the GPU's int8 rows
    h = T["h"][R]
    h_ref = orc.swiglu_gate_rows(w.g, w.u, T["xq2"][R], T["amax2"][R], activation=w.act)
    if w.act == ACT_RELU2:
        assert np.array_equal(h.view(np.uint32), h_ref.view(np.uint32)), "ReLU2 gate product"
    else:  # SiLU: exp()'s last fp64 bit
        assert ulp_diff_f32(h, h_ref).max() <= 1, "SiLU gate product beyond 1 ulp"
    # SwiGLU inner norm of the GPU's h (poly/bitnet_cpu.go:893-913), requant
    hn = T["hn"][R]
    hn_ref = np.stack([orc.bitnet_rmsnorm_row(h[i], w.fn, 1e-5) for i in range(len(R))])
    _f32_rows(hn, hn_ref, strict, "ffn inner norm")
    _quant(orc, hn, T["hq"][R], T["hamax"][R], "ffn int8")
    # down (poly/swiglu.go:316-320) + residual (poly/transformer_forward.go:244)
    dn = orc.dense_quantized(w.d, T["hq"][R], T["hamax"][R])
    out_ref = (dn + mid[R]).astype(np.float32)
    assert np.array_equal(out[R].view(np.uint32), out_ref.view(np.uint32)), \
        "down + residual not bit-exact"


def run_block_case(orc, torch, tf, w: Weights, seqs, seed, strict=True, rows_for=None, blk=None):
    """Prefill seqs[0] tokens then further calls of seqs[1:] tokens, each
    checked stage by stage.  rows_for(seq) picks the rows checked past the
    projection (None = all)."""
    sh = w.sh
    own = blk is None
    if own:
        blk = tf.BitNetBlock(w.cfg(tf, "strict" if strict else "fast"), w.gpu(tf))
    mha_ref = w.oracle_mha(orc)
    base = 0
    for i, seq in enumerate(seqs):
        x_in = orc.normal_f32(seq * sh.hidden, seed + i).reshape(seq, sh.hidden)
        x = to_dev(torch, x_in)
        print(f"  block call {i}: seq={seq} base={base}", flush=True)
        _, taps = blk.forward(x, taps=True)
        torch.cuda.synchronize()
        assert blk.kv_offset == base + seq
        ck, cv = (t.cpu().numpy() for t in blk.kv_cache(0))
        rows = rows_for(seq) if rows_for else None
        check_stages(orc, w, mha_ref, x_in, taps.numpy(), x.cpu().numpy(), ck, cv, base, strict,
                     rows)
        base += seq
    if own:
        blk.release()
