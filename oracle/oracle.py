"""ctypes front end of the CPU oracle (oracle/bitnet_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package ``loom_amd``.

The C library restates loom's BitNet CPU path (poly/bitnet_cpu.go,
poly/dense.go, poly/swiglu.go, poly/norm.go, poly/entity_bitnet.go); each C
function cites the reference line it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libbitnet_oracle.so")

ACT_RELU, ACT_SILU, ACT_GELU, ACT_TANH, ACT_SIGMOID, ACT_LEAKY_RELU, ACT_RELU2 = range(7)
ACT_LINEAR = -1

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p


def _declare(L: C.CDLL) -> None:
    i, f, d, u8, sz = C.c_int, C.c_float, C.c_double, C.c_uint8, C.c_size_t
    sig = {
        "orc_act_maxabs_f32": (f, [P, i]),
        "orc_act_maxabs_f64": (f, [P, i]),
        "orc_quant_value_act": (C.c_int8, [d, f]),
        "orc_quant_act_f32": (f, [P, i, P]),
        "orc_quant_act_f64": (f, [P, i, P]),
        "orc_ternary_scale": (f, [P, C.c_long]),
        "orc_quant_value": (u8, [f, f]),
        "orc_storage_to_code": (u8, [u8]),
        "orc_pack_ternary_rows": (None, [P, i, i, P]),
        "orc_pack_float32": (f, [P, i, i, P]),
        "orc_pack_ms_offline_bytes": (None, [P, i, i, P]),
        "orc_pack_ms_offline_float_slots": (None, [P, i, i, P]),
        "orc_output_scale": (d, [f, f]),
        "orc_matvec_scalar": (None, [P, i, i, i, P, d, P, P]),
        "orc_codes_stride": (i, [i]),
        "orc_ensure_codes": (None, [P, i, i, i, P]),
        "orc_code_row_dot_go": (C.c_int32, [P, P, i]),
        "orc_code_row_dot_avx2": (C.c_int32, [P, P, i]),
        "orc_simd_available": (i, []),
        "orc_matvec_simd": (None, [P, i, i, P, d, P, P, i]),
        "orc_run_rows_plan": (None, [i, i, i, P, P]),
        "orc_dense_forward": (None, [P, P, i, i, i, i, P, P, P, P, P]),
        "orc_activate_f32": (f, [f, i]),
        "orc_swiglu_gate_product": (d, [d, d, i]),
        "orc_bitnet_rmsnorm_row_f32": (None, [P, i, P, d]),
        "orc_bitnet_rmsnorm_f64": (None, [P, i, P, d]),
        "orc_swiglu_forward": (None, [P, P, P, P, P, d, i, P, i, i, i,
                                      P, P, P, P, P, P, P, P, P]),
        "orc_rmsnorm_forward": (None, [P, i, i, P, d, P, P]),
        "orc_attention": (None, [P, P, P, i, i, i, i, i, i, P]),
        "orc_attention_span": (C.c_long, [P, i, i, i]),
        "orc_attention_args": (None, [P, P, P, i, i, i, i, i, i, P]),
        "orc_attention_chains": (None, [P, P, P, i, i, i, i, i, i, P]),
        "orc_exp_rows": (None, [P, C.c_long, P]),
        "orc_attn_out": (None, [P, P, P, d, P, i, i, i, i, P, P]),
        "orc_mha_forward": (None, [P, P, i, i, i, P, P, P, P]),
        "orc_mha_project": (None, [P, P, i, i, i, i, P]),
        "orc_per_head_rmsnorm_f64": (None, [P, P, i, i, i, d]),
        "orc_per_head_rmsnorm_f32": (None, [P, P, i, i, i, d]),
        "orc_qk_norm_eps": (d, [d]),
        "orc_dense_quantized": (None, [P, P, P, i, P, i, i, P]),
        "orc_swiglu_gate_rows": (None, [P, P, P, i, P, P, i, i, i, P]),
        "orc_block_forward": (None, [P, P, i, i, i]),
        "orc_lm_head_seq": (None, [P, P, i, i, P]),
        "orc_dot_tile": (d, [P, P, i, d]),
        "orc_lm_head_dottile": (None, [P, P, i, i, P]),
        "orc_argmax_first": (i, [P, i]),
        "orc_entity_blob_bytes": (sz, [i]),
        "orc_entity_encode": (sz, [i, i, i, f, i, P, i, P]),
        "orc_entity_decode_header": (i, [P, sz, P, P, P, P, P, P]),
        "orc_deterministic_weights": (None, [P, i]),
        "orc_fill_normal_f32": (None, [P, C.c_long, C.c_uint64]),
        "orc_fill_ternary_codes": (None, [P, C.c_long, C.c_uint64]),
        "orc_fill_uniform_f32": (None, [P, C.c_long, f, f, C.c_uint64]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(P)


# ---------------------------------------------------------------- inputs
def deterministic_weights(n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_deterministic_weights(_p(out), n)
    return out


def normal_f32(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal_f32(_p(out), n, seed)
    return out


def uniform_f32(n: int, lo: float, hi: float, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_uniform_f32(_p(out), n, lo, hi, seed)
    return out


def ternary_native(n: int, seed: int) -> np.ndarray:
    """uint8(int8) ternary storage values, P(0)=.5, P(+1)=P(-1)=.25."""
    out = np.empty(n, np.uint8)
    lib().orc_fill_ternary_codes(_p(out), n, seed)
    return out


# ---------------------------------------------------------------- matrix
@dataclass
class Matrix:
    """BitNetTernaryMatrix (poly/bitnet_cpu.go:14-43): row-major packed words."""
    rows: int
    cols: int
    scale: float
    words: np.ndarray  # uint32, rows*row_words
    codes: np.ndarray | None = None

    @property
    def row_words(self) -> int:
        return (self.cols + 15) // 16

    def ensure_codes(self) -> np.ndarray:
        if self.codes is None:
            stride = lib().orc_codes_stride(self.cols)
            self.codes = np.empty(self.rows * stride, np.uint8)
            lib().orc_ensure_codes(_p(self.words), self.rows, self.cols, self.row_words,
                                   _p(self.codes))
        return self.codes

    def _c(self, simd: bool):
        class _M(C.Structure):
            _fields_ = [("rows", C.c_int), ("cols", C.c_int), ("row_words", C.c_int),
                        ("scale", C.c_float), ("words", P), ("codes", P)]
        codes = self.ensure_codes() if simd else None
        return _M(self.rows, self.cols, self.row_words, self.scale, _p(self.words), _p(codes))

    def entity_blob(self, offset: int = 0) -> bytes:
        return entity_encode(self.rows, self.cols, offset, self.scale, self.row_words, self.words)


def pack_native(native: np.ndarray, rows: int, cols: int, scale: float) -> Matrix:
    """packNativeTernaryToBitNetMatrix (poly/bitnet_cpu.go:918-932)."""
    native = np.ascontiguousarray(native, np.uint8)
    words = np.empty(rows * ((cols + 15) // 16), np.uint32)
    lib().orc_pack_ternary_rows(_p(native), rows, cols, _p(words))
    return Matrix(rows, cols, float(np.float32(scale if scale != 0 else 1.0)), words)


def pack_float32(master: np.ndarray, rows: int, cols: int) -> Matrix:
    """packFloat32AsBitNetTernaryMatrix (poly/bitnet_cpu.go:934-962)."""
    master = np.ascontiguousarray(master, np.float32)
    words = np.empty(rows * ((cols + 15) // 16), np.uint32)
    scale = lib().orc_pack_float32(_p(master), rows, cols, _p(words))
    return Matrix(rows, cols, float(scale), words)


def pack_ms_offline_bytes(packed: np.ndarray, rows: int, cols: int, scale: float = 1.0) -> Matrix:
    packed = np.ascontiguousarray(packed, np.uint8)
    words = np.empty(rows * ((cols + 15) // 16), np.uint32)
    lib().orc_pack_ms_offline_bytes(_p(packed), rows, cols, _p(words))
    return Matrix(rows, cols, scale, words)


def pack_ms_offline_float_slots(packed: np.ndarray, rows: int, cols: int, scale: float = 1.0) -> Matrix:
    packed = np.ascontiguousarray(packed, np.float32)
    words = np.empty(rows * ((cols + 15) // 16), np.uint32)
    lib().orc_pack_ms_offline_float_slots(_p(packed), rows, cols, _p(words))
    return Matrix(rows, cols, scale, words)


def random_matrix(rows: int, cols: int, seed: int, alpha: float = 0.02) -> Matrix:
    """Synthetic BitNet weights: ternary codes times alpha, packed by loom's
    float32 packer so Scale is loom's absmean of the master."""
    native = ternary_native(rows * cols, seed)
    master = native.view(np.int8).astype(np.float32) * np.float32(alpha)
    return pack_float32(master, rows, cols)


# ---------------------------------------------------------------- quant
def act_maxabs(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x)
    if x.dtype == np.float64:
        return float(lib().orc_act_maxabs_f64(_p(x), x.size))
    x = x.astype(np.float32, copy=False)
    return float(lib().orc_act_maxabs_f32(_p(x), x.size))


def quant_act(x: np.ndarray) -> tuple[np.ndarray, float]:
    x = np.ascontiguousarray(x)
    q = np.empty(x.size, np.int8)
    if x.dtype == np.float64:
        amax = lib().orc_quant_act_f64(_p(x), x.size, _p(q))
    else:
        x = x.astype(np.float32, copy=False)
        amax = lib().orc_quant_act_f32(_p(x), x.size, _p(q))
    return q, float(amax)


def quant_act_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.int8)
    amax = np.empty(x.shape[0], np.float32)
    for r in range(x.shape[0]):
        amax[r] = lib().orc_quant_act_f32(_p(x[r]), x.shape[1], _p(q[r]))
    return q, amax


def ternary_scale(w: np.ndarray) -> float:
    w = np.ascontiguousarray(w, np.float32)
    return float(lib().orc_ternary_scale(_p(w), w.size))


def quant_value(v: float, scale: float) -> int:
    return int(np.uint8(lib().orc_quant_value(v, scale)).view(np.int8))


def output_scale(weight_scale: float, amax: float) -> float:
    return float(lib().orc_output_scale(weight_scale, amax))


# ---------------------------------------------------------------- matvec
def matvec_scalar(m: Matrix, xq: np.ndarray, output_scale_: float):
    xq = np.ascontiguousarray(xq, np.int8)
    out = np.empty(m.rows, np.float64)
    acc = np.empty(m.rows, np.int32)
    lib().orc_matvec_scalar(_p(m.words), m.rows, m.cols, m.row_words, _p(xq),
                            output_scale_, _p(out), _p(acc))
    return out, acc


def matvec_simd(m: Matrix, xq: np.ndarray, output_scale_: float, workers: int = 0):
    xq = np.ascontiguousarray(xq, np.int8)
    codes = m.ensure_codes()
    out = np.empty(m.rows, np.float64)
    acc = np.empty(m.rows, np.int32)
    lib().orc_matvec_simd(_p(codes), m.rows, m.cols, _p(xq), output_scale_, _p(out), _p(acc),
                          workers or (os.cpu_count() or 1))
    return out, acc


def code_row_dot(codes: np.ndarray, acts: np.ndarray, avx2: bool) -> int:
    codes = np.ascontiguousarray(codes, np.uint8)
    acts = np.ascontiguousarray(acts, np.int8)
    fn = lib().orc_code_row_dot_avx2 if avx2 else lib().orc_code_row_dot_go
    return int(fn(_p(codes), _p(acts), codes.size))


def simd_available() -> bool:
    return bool(lib().orc_simd_available())


# ---------------------------------------------------------------- layers
@dataclass
class DenseResult:
    pre: np.ndarray
    post: np.ndarray
    xq: np.ndarray
    amax: np.ndarray
    acc: np.ndarray


def dense_forward(m: Matrix, x: np.ndarray, activation: int = ACT_LINEAR, simd: bool = True,
                  workers: int = 0) -> DenseResult:
    """DenseForwardPackedTernaryCPU (poly/dense.go:66-101)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, m.cols)
    M = x.shape[0]
    pre = np.empty((M, m.rows), np.float32)
    post = np.empty((M, m.rows), np.float32)
    xq = np.empty((M, m.cols), np.int8)
    amax = np.empty(M, np.float32)
    acc = np.empty((M, m.rows), np.int32)
    cm = m._c(simd)
    lib().orc_dense_forward(C.byref(cm), _p(x), M, activation, int(simd),
                            workers or (os.cpu_count() or 1),
                            _p(pre), _p(post), _p(xq), _p(amax), _p(acc))
    return DenseResult(pre, post, xq, amax, acc)


@dataclass
class SwiGLUResult:
    out: np.ndarray
    h: np.ndarray
    xq: np.ndarray
    amax: np.ndarray
    hq: np.ndarray
    hamax: np.ndarray
    acc_gate: np.ndarray
    acc_up: np.ndarray
    acc_down: np.ndarray


def swiglu_forward(gate: Matrix, up: Matrix, down: Matrix, x: np.ndarray,
                   inner_norm: np.ndarray | None = None, bias: np.ndarray | None = None,
                   eps: float = 1e-5, activation: int = ACT_SILU, simd: bool = True,
                   workers: int = 0) -> SwiGLUResult:
    """SwiGLUForwardPackedTernaryCPU (poly/swiglu.go:270-322)."""
    hidden, inter = gate.cols, gate.rows
    x = np.ascontiguousarray(x, np.float32).reshape(-1, hidden)
    M = x.shape[0]
    out = np.empty((M, hidden), np.float32)
    h = np.empty((M, inter), np.float32)
    xq = np.empty((M, hidden), np.int8)
    amax = np.empty(M, np.float32)
    hq = np.empty((M, inter), np.int8)
    hamax = np.empty(M, np.float32)
    ag = np.empty((M, inter), np.int32)
    au = np.empty((M, inter), np.int32)
    ad = np.empty((M, hidden), np.int32)
    cg, cu, cd = gate._c(simd), up._c(simd), down._c(simd)
    nw = None if inner_norm is None else np.ascontiguousarray(inner_norm, np.float32)
    bs = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_swiglu_forward(C.byref(cg), C.byref(cu), C.byref(cd), _p(bs), _p(nw), eps,
                             activation, _p(x), M, int(simd), workers or (os.cpu_count() or 1),
                             _p(out), _p(h), _p(xq), _p(amax), _p(hq), _p(hamax),
                             _p(ag), _p(au), _p(ad))
    return SwiGLUResult(out, h, xq, amax, hq, hamax, ag, au, ad)


def dense_quantized(m: Matrix, xq: np.ndarray, amax: np.ndarray, bias: np.ndarray | None = None,
                    simd: bool = True, workers: int = 0) -> np.ndarray:
    """Output / down projection stage from given int8 rows (poly/mha.go:362-368,
    poly/swiglu.go:316-320): fp32(matvec + bias) per row."""
    xq = np.ascontiguousarray(xq, np.int8).reshape(-1, m.cols)
    amax = np.ascontiguousarray(amax, np.float32).reshape(-1)
    out = np.empty((xq.shape[0], m.rows), np.float32)
    cm = m._c(simd)
    bs = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_dense_quantized(C.byref(cm), _p(xq), _p(amax), xq.shape[0], _p(bs), int(simd),
                              workers or (os.cpu_count() or 1), _p(out))
    return out


def swiglu_gate_rows(gate: Matrix, up: Matrix, xq: np.ndarray, amax: np.ndarray,
                     activation: int = ACT_SILU, bias: np.ndarray | None = None,
                     simd: bool = True, workers: int = 0) -> np.ndarray:
    """Gate/up stage of SwiGLUForwardPackedTernaryCPU (poly/swiglu.go:303-312)
    from given int8 rows: h = fp32(gate product), before the inner norm."""
    xq = np.ascontiguousarray(xq, np.int8).reshape(-1, gate.cols)
    amax = np.ascontiguousarray(amax, np.float32).reshape(-1)
    h = np.empty((xq.shape[0], gate.rows), np.float32)
    cg, cu = gate._c(simd), up._c(simd)
    bs = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_swiglu_gate_rows(C.byref(cg), C.byref(cu), _p(bs), activation, _p(xq), _p(amax),
                               xq.shape[0], int(simd), workers or (os.cpu_count() or 1), _p(h))
    return h


def quant_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """bitNetQuantizeActivationNumeric / ...Float64 per row (fp32 or fp64 rows)."""
    x = np.ascontiguousarray(x)
    q = np.empty(x.shape, np.int8)
    amax = np.empty(x.shape[0], np.float32)
    for r in range(x.shape[0]):
        q[r], amax[r] = quant_act(x[r])
    return q, amax


def swiglu_gate_product(g: float, u: float, activation: int = ACT_SILU) -> float:
    return float(lib().orc_swiglu_gate_product(g, u, activation))


def bitnet_rmsnorm_row(h: np.ndarray, weight: np.ndarray | None, eps: float) -> np.ndarray:
    h = np.array(h, np.float32, copy=True)
    w = None if weight is None else np.ascontiguousarray(weight, np.float32)
    lib().orc_bitnet_rmsnorm_row_f32(_p(h), h.size, _p(w), eps)
    return h


def rmsnorm_forward(x: np.ndarray, gain: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    g = np.ascontiguousarray(gain, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm_forward(_p(x), rows, n, _p(g), eps, _p(y), None)
    return y


def activate(v: float, activation: int) -> float:
    return float(lib().orc_activate_f32(v, activation))


# ---------------------------------------------------------------- entity blob
def entity_encode(rows: int, cols: int, offset: int, scale: float, row_words: int,
                  words: np.ndarray) -> bytes:
    words = np.ascontiguousarray(words, np.uint32)
    n = int(lib().orc_entity_blob_bytes(words.size))
    raw = np.empty(n, np.uint8)
    lib().orc_entity_encode(rows, cols, offset, scale, row_words, _p(words), words.size, _p(raw))
    return raw.tobytes()


def entity_decode(raw: bytes) -> tuple[Matrix, int]:
    buf = np.frombuffer(raw, np.uint8)
    vals = [C.c_int() for _ in range(5)]
    scale = C.c_float()
    rc = lib().orc_entity_decode_header(_p(buf), buf.size, C.byref(vals[0]), C.byref(vals[1]),
                                        C.byref(vals[2]), C.byref(scale), C.byref(vals[3]),
                                        C.byref(vals[4]))
    if rc == -1:
        raise ValueError("bitnet ternary blob too short")
    if rc == -2:
        raise ValueError("bitnet ternary blob truncated")
    rows, cols, offset, row_words, n_words = (v.value for v in vals)
    words = np.frombuffer(raw, np.uint32, count=n_words, offset=24).copy()
    m = Matrix(rows, cols, scale.value, words)
    return m, offset


# ---------------------------------------------------------------- attention, block, LM head
class _CMatrix(C.Structure):
    _fields_ = [("rows", C.c_int), ("cols", C.c_int), ("row_words", C.c_int),
                ("scale", C.c_float), ("words", P), ("codes", P)]


class _CMHA(C.Structure):
    _fields_ = [("d_model", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("msl", C.c_int), ("theta", C.c_double),
                ("eps", C.c_double), ("q", P), ("k", P), ("v", P), ("o", P),
                ("bias_q", P), ("bias_k", P), ("bias_v", P), ("bias_o", P),
                ("inner_norm", P), ("cache_k", P), ("cache_v", P), ("kv_offset", C.c_int),
                ("q_norm", P), ("q_norm_len", C.c_int), ("k_norm", P), ("k_norm_len", C.c_int)]


class _CBlock(C.Structure):
    _fields_ = [("hidden", C.c_int), ("norm1", P), ("norm2", P), ("norm_eps", C.c_double),
                ("mha", _CMHA), ("gate", P), ("up", P), ("down", P), ("ffn_inner_norm", P),
                ("ffn_eps", C.c_double), ("ffn_activation", C.c_int)]


def _cmat(m: Matrix, simd: bool) -> _CMatrix:
    codes = m.ensure_codes() if simd else None
    return _CMatrix(m.rows, m.cols, m.row_words, m.scale, _p(m.words), _p(codes))


def attention(q: np.ndarray, cache_k: np.ndarray, cache_v: np.ndarray, seq_base: int, msl: int,
              num_heads: int, num_kv_heads: int, head_dim: int) -> np.ndarray:
    """Attention stage of MHAForwardPackedTernaryCPU (poly/mha.go:316-354):
    q [seq, q_dim] fp64 after RoPE, caches [msl, kv_dim] fp32; returns fp64."""
    q = np.ascontiguousarray(q, np.float64).reshape(-1, num_heads * head_dim)
    ck = np.ascontiguousarray(cache_k, np.float32)
    cv = np.ascontiguousarray(cache_v, np.float32)
    out = np.empty_like(q)
    lib().orc_attention(_p(q), _p(ck), _p(cv), q.shape[0], seq_base, msl, num_heads,
                        num_kv_heads, head_dim, _p(out))
    return out


def per_head_rmsnorm(x: np.ndarray, gamma: np.ndarray | None, heads: int, head_dim: int,
                     eps: float) -> np.ndarray:
    """applyPerHeadRMSNormFloat64 (fp64 rows) or applyPerHeadRMSNormTensor
    (fp32 rows) of poly/mha.go:584-646 on a copy of one row; gamma None or
    empty: unit weights (any other length than head_dim or heads*head_dim
    also means unit weights)."""
    g = np.zeros(0, np.float32) if gamma is None else np.ascontiguousarray(gamma, np.float32)
    out = np.array(x, copy=True)
    if out.dtype == np.float64:
        lib().orc_per_head_rmsnorm_f64(_p(out), _p(g), g.size, heads, head_dim, eps)
    else:
        out = np.ascontiguousarray(out, np.float32)
        lib().orc_per_head_rmsnorm_f32(_p(out), _p(g), g.size, heads, head_dim, eps)
    return out


def _attn_rows(q, rows):
    rows = np.arange(q.shape[0]) if rows is None else np.asarray(rows)
    return np.ascontiguousarray(rows, np.int32)


def attention_args(q: np.ndarray, cache_k: np.ndarray, seq_base: int, msl: int, num_heads: int,
                   num_kv_heads: int, head_dim: int, rows=None) -> np.ndarray:
    """Stage 1 of the attention (poly/mha.go:324-337) for rows `rows` of q
    (all by default): the exp arguments score - max, flat, per row, per head,
    positions 0..seq_base+row."""
    q = np.ascontiguousarray(q, np.float64).reshape(-1, num_heads * head_dim)
    r = _attn_rows(q, rows)
    n = lib().orc_attention_span(_p(r), r.size, seq_base, num_heads)
    out = np.empty(n, np.float64)
    lib().orc_attention_args(_p(q), _p(np.ascontiguousarray(cache_k, np.float32)), _p(r), r.size,
                             seq_base, msl, num_heads, num_kv_heads, head_dim, _p(out))
    return out


def attention_chains(probs: np.ndarray, cache_v: np.ndarray, seq_base: int, msl: int,
                     num_heads: int, num_kv_heads: int, head_dim: int, rows) -> np.ndarray:
    """Stage 2 of the attention (poly/mha.go:339-352) from probabilities in
    attention_args' layout: [len(rows), q_dim] fp64."""
    r = np.ascontiguousarray(rows, np.int32)
    p = np.ascontiguousarray(probs, np.float64)
    assert p.size == lib().orc_attention_span(_p(r), r.size, seq_base, num_heads)
    out = np.empty((r.size, num_heads * head_dim), np.float64)
    lib().orc_attention_chains(_p(p), _p(np.ascontiguousarray(cache_v, np.float32)), _p(r), r.size,
                               seq_base, msl, num_heads, num_kv_heads, head_dim, _p(out))
    return out


def exp_rows(x: np.ndarray) -> np.ndarray:
    """The C library's exp elementwise (the exp orc_attention uses)."""
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty_like(x)
    lib().orc_exp_rows(_p(x), x.size, _p(y))
    return y


def attn_out(o: Matrix, attn: np.ndarray, inner_norm: np.ndarray | None = None,
             eps: float = 1e-5, bias_o: np.ndarray | None = None, simd: bool = True):
    """Output stage of MHAForwardPackedTernaryCPU (poly/mha.go:356-368):
    returns (pre, post) fp32 for fp64 attention rows (before the inner norm)."""
    a = np.array(attn, np.float64, copy=True).reshape(-1, o.cols)
    seq = a.shape[0]
    pre = np.empty((seq, o.cols), np.float32)
    post = np.empty((seq, o.rows), np.float32)
    cm = _cmat(o, simd)
    wn = None if inner_norm is None else np.ascontiguousarray(inner_norm, np.float32)
    bo = None if bias_o is None else np.ascontiguousarray(bias_o, np.float32)
    lib().orc_attn_out(C.byref(cm), _p(bo), _p(wn), eps, _p(a), seq, o.cols, int(simd),
                       os.cpu_count() or 1, _p(pre), _p(post))
    return pre, post


class MHA:
    """MHAForwardPackedTernaryCPU (poly/mha.go:204-371) with its KV ring cache."""

    def __init__(self, q: Matrix, k: Matrix, v: Matrix, o: Matrix, num_heads: int,
                 num_kv_heads: int, head_dim: int, msl: int, theta: float = 500000.0,
                 eps: float = 1e-5, inner_norm: np.ndarray | None = None, simd: bool = True,
                 q_norm: np.ndarray | None = None, k_norm: np.ndarray | None = None):
        """eps is the layer's RMSNormEps (<= 0: the inner norm takes 1e-5 and
        the per-head Q/K norms 1e-6, poly/mha.go:19-24); q_norm / k_norm are
        QNormWeight / KNormWeight (None or empty: no per-head norm)."""
        self.mats = (q, k, v, o)
        self.simd = simd
        self.d_model = q.cols
        self.num_heads, self.num_kv_heads, self.head_dim, self.msl = (
            num_heads, num_kv_heads, head_dim, msl)
        kv_dim = num_kv_heads * head_dim
        self.cache_k = np.zeros(msl * kv_dim, np.float32)
        self.cache_v = np.zeros(msl * kv_dim, np.float32)
        self.inner_norm = None if inner_norm is None else np.ascontiguousarray(inner_norm, np.float32)
        self._cm = [_cmat(m, simd) for m in self.mats]
        self.q_norm = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
        self.k_norm = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
        self.c = _CMHA(self.d_model, num_heads, num_kv_heads, head_dim, msl, theta, eps,
                       *(C.cast(C.pointer(cm), P) for cm in self._cm),
                       None, None, None, None, _p(self.inner_norm), _p(self.cache_k),
                       _p(self.cache_v), 0,
                       _p(self.q_norm), 0 if self.q_norm is None else self.q_norm.size,
                       _p(self.k_norm), 0 if self.k_norm is None else self.k_norm.size)

    @property
    def kv_offset(self) -> int:
        return self.c.kv_offset

    def project(self, x: np.ndarray, base: int, workers: int = 0) -> np.ndarray:
        """Projection stage only (poly/mha.go:262-314): Q/K/V of the rows at
        positions base.., the K/V rows written into this MHA's caches; returns
        Q after bias and RoPE (fp64).  kv_offset is left unchanged."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.d_model)
        q = np.empty((x.shape[0], self.num_heads * self.head_dim), np.float64)
        lib().orc_mha_project(C.byref(self.c), _p(x), x.shape[0], base, int(self.simd),
                              workers or (os.cpu_count() or 1), _p(q))
        return q

    def forward_batch(self, x: np.ndarray, workers: int = 0):
        """loom's 3-D input [batch, seq, d_model], its batch loop restated
        literally (poly/mha.go:251-371 with mhaPrepareKVForForward,
        poly/mha_layout.go:62-70): unless the call is a warm single-token step
        (batch 1, seq 1, kv_offset > 0) the caches are zeroed and kv_offset
        restarts at 0; sequence b's rows take positions kv_start + b*seq + s,
        its K/V rows are written, then each of its queries attends to every
        position up to its own -- those of the sequences before it included;
        kv_offset ends at kv_start + batch*seq.  Returns (pre, post) as
        [batch, seq, d_model] fp32."""
        x = np.ascontiguousarray(x, np.float32)
        batch, seq = x.shape[0], x.shape[1]
        x = x.reshape(batch, seq, self.d_model)
        if not (batch == 1 and seq == 1 and self.c.kv_offset > 0):
            self.cache_k[:] = 0.0
            self.cache_v[:] = 0.0
            self.c.kv_offset = 0
        kv_start = self.c.kv_offset
        pre = np.empty((batch, seq, self.d_model), np.float32)
        post = np.empty((batch, seq, self.mats[3].rows), np.float32)
        for b in range(batch):
            seq_base = kv_start + b * seq
            q = self.project(x[b], seq_base, workers)
            attn = attention(q, self.cache_k, self.cache_v, seq_base, self.msl, self.num_heads,
                             self.num_kv_heads, self.head_dim)
            pre[b], post[b] = attn_out(self.mats[3], attn, self.inner_norm, self.c.eps, simd=self.simd)
        self.c.kv_offset = kv_start + batch * seq
        return pre, post

    def forward(self, x: np.ndarray, workers: int = 0):
        """Returns (pre, post, q_after_rope, attn_before_norm)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.d_model)
        seq = x.shape[0]
        q_dim = self.num_heads * self.head_dim
        pre = np.empty((seq, self.d_model), np.float32)
        post = np.empty((seq, self.d_model), np.float32)
        q = np.empty((seq, q_dim), np.float64)
        attn = np.empty((seq, q_dim), np.float64)
        lib().orc_mha_forward(C.byref(self.c), _p(x), seq, int(self.simd),
                              workers or (os.cpu_count() or 1), _p(pre), _p(post), _p(q), _p(attn))
        return pre, post, q, attn


class Block:
    """One decoder block (poly/transformer_forward.go:228-245)."""

    def __init__(self, mha: MHA, norm1: np.ndarray, norm2: np.ndarray, gate: Matrix, up: Matrix,
                 down: Matrix, ffn_inner_norm: np.ndarray | None = None, norm_eps: float = 1e-5,
                 ffn_eps: float = 1e-5, ffn_activation: int = ACT_SILU):
        self.mha = mha
        self.norm1 = np.ascontiguousarray(norm1, np.float32)
        self.norm2 = np.ascontiguousarray(norm2, np.float32)
        self.ffn = (gate, up, down)
        self._fm = [_cmat(m, mha.simd) for m in self.ffn]
        self.ffn_inner_norm = (None if ffn_inner_norm is None
                               else np.ascontiguousarray(ffn_inner_norm, np.float32))
        self.c = _CBlock(mha.d_model, _p(self.norm1), _p(self.norm2), norm_eps, mha.c,
                         *(C.cast(C.pointer(cm), P) for cm in self._fm),
                         _p(self.ffn_inner_norm), ffn_eps, ffn_activation)

    def forward(self, x: np.ndarray, workers: int = 0) -> np.ndarray:
        x = np.array(x, np.float32, copy=True).reshape(-1, self.mha.d_model)
        lib().orc_block_forward(C.byref(self.c), _p(x), x.shape[0], int(self.mha.simd),
                                workers or (os.cpu_count() or 1))
        self.mha.c.kv_offset = self.c.mha.kv_offset
        return x


def dot_tile(x: np.ndarray, w: np.ndarray, prev: float = 0.0) -> float:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    return float(lib().orc_dot_tile(_p(x), _p(w), x.size, prev))


def lm_head(hidden: np.ndarray, table: np.ndarray, simd: bool = True) -> np.ndarray:
    """applyFP32LMHeadRows (poly/transformer.go:664-719): DotTile order with SIMD on."""
    hidden = np.ascontiguousarray(hidden, np.float32)
    table = np.ascontiguousarray(table, np.float32)
    vocab = table.size // hidden.size
    out = np.empty(vocab, np.float32)
    fn = lib().orc_lm_head_dottile if simd else lib().orc_lm_head_seq
    fn(_p(hidden), _p(table), vocab, hidden.size, _p(out))
    return out


def argmax_first(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_argmax_first(_p(logits), logits.size))
