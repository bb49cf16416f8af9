"""BitNet b1.58 ternary layers on gfx950: the host-side mirror of loom's packed
ternary CPU entry points, running on libloom_accel_amd.so.

Names and argument meaning follow loom:

=====================================  =============================================
loom (poly/)                           here
=====================================  =============================================
BitNetTernaryMatrix (bitnet_cpu.go:14) ``TernaryMatrix`` (device-resident, repacked)
bitNetQuantizeActivationNumeric (:97)  ``quantize_activation``
bitNetTernaryMatVecQuantized (:536)    ``ternary_matvec_quantized`` (all rows at once)
DenseForwardPackedTernaryCPU           ``dense_forward_packed_ternary``
  (dense.go:66-101)                      returns (preAct, postAct)
SwiGLUForwardPackedTernaryCPU          ``swiglu_forward_packed_ternary``
  (swiglu.go:270-322)                    returns (preAct = normalized h, postAct)
bitNetRMSNormTensorRowWeighted         ``norm_quant_rows`` (with the requantization)
  (bitnet_cpu.go:893-913)
=====================================  =============================================

Tensors are torch CUDA (HIP) tensors; torch only provides device memory and the
stream.  All compute runs in the HIP kernels of the library; there is no CPU or
PyTorch fallback -- a missing library raises.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check

ACT_RELU, ACT_SILU, ACT_GELU, ACT_TANH, ACT_SIGMOID, ACT_LEAKY_RELU, ACT_RELU2 = range(7)
ACT_LINEAR = -1

NORM_STRICT = 1
NORM_FAST = 0
TILE_COLS = 256


def _torch():
    import torch
    return torch


def padded_cols(k: int) -> int:
    return (k + TILE_COLS - 1) // TILE_COLS * TILE_COLS


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(device: int):
    torch = _torch()
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _norm_mode(norm) -> int:
    if norm in (NORM_STRICT, "strict"):
        return NORM_STRICT
    if norm in (NORM_FAST, "fast"):
        return NORM_FAST
    raise ValueError(f"norm must be 'strict' or 'fast', got {norm!r}")


class TernaryMatrix:
    """A loom BitNetTernaryMatrix repacked once into the gfx950 tile layout."""

    def __init__(self, handle: int, device: int):
        self._h = C.c_void_p(handle)
        self.device = device
        rows, cols, scale, nbytes = C.c_int(), C.c_int(), C.c_float(), C.c_size_t()
        check(_lib.lib().loom_amd_matrix_shape(self._h, C.byref(rows), C.byref(cols),
                                                C.byref(scale), C.byref(nbytes)), "matrix_shape")
        self.rows, self.cols = rows.value, cols.value
        self.scale = scale.value
        self.device_bytes = nbytes.value

    @classmethod
    def from_words(cls, words: np.ndarray, rows: int, cols: int, scale: float,
                   row_words: int | None = None, device: int = 0) -> "TernaryMatrix":
        words = np.ascontiguousarray(words, np.uint32)
        rw = row_words or (cols + 15) // 16
        out = C.c_void_p()
        check(_lib.lib().loom_amd_matrix_create(device, words.ctypes.data_as(C.c_void_p),
                                                words.size, rows, cols, rw, scale,
                                                C.byref(out)), "matrix_create")
        return cls(out.value, device)

    @classmethod
    def from_entity_blob(cls, blob: bytes, device: int = 0) -> "TernaryMatrix":
        buf = (C.c_char * len(blob)).from_buffer_copy(blob)
        out = C.c_void_p()
        used = C.c_size_t()
        check(_lib.lib().loom_amd_matrix_from_entity_blob(device, C.addressof(buf), len(blob),
                                                          C.byref(out), C.byref(used)),
              "matrix_from_entity_blob")
        return cls(out.value, device)

    @classmethod
    def from_ms_offline(cls, packed: np.ndarray, rows: int, cols: int, scale: float,
                        device: int = 0) -> "TernaryMatrix":
        """Microsoft offline U8 layout ((rows/4) x cols bytes) with the
        checkpoint's weight_scale (packMicrosoftOfflineBitNetRowsToU32FromBytes)."""
        packed = np.ascontiguousarray(packed, np.uint8)
        if packed.size < (rows // 4) * cols:
            raise ValueError("packed holds fewer than (rows/4)*cols bytes")
        out = C.c_void_p()
        check(_lib.lib().loom_amd_matrix_from_ms_offline(device, packed.ctypes.data_as(C.c_void_p),
                                                         rows, cols, scale, C.byref(out)),
              "matrix_from_ms_offline")
        return cls(out.value, device)

    @classmethod
    def from_float32(cls, master: np.ndarray, rows: int, cols: int,
                     device: int = 0) -> "TernaryMatrix":
        """Pack an fp32 master as loom's packFloat32AsBitNetTernaryMatrix
        (poly/bitnet_cpu.go:934-962): absmean scale, codes round(w/scale)
        clamped to [-1, 1], scale 1 for an already-ternary master."""
        master = np.ascontiguousarray(master, np.float32)
        if master.size < rows * cols:
            raise ValueError("master holds fewer than rows*cols weights")
        out = C.c_void_p()
        scale = C.c_float()
        check(_lib.lib().loom_amd_matrix_from_float32(device, master.ctypes.data_as(C.c_void_p),
                                                      rows, cols, C.byref(out), C.byref(scale)),
              "matrix_from_float32")
        return cls(out.value, device)

    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise _lib.AMDError("matrix released")
        return self._h

    def release(self) -> None:
        if self._h is not None:
            _lib.lib().loom_amd_matrix_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


@dataclass
class QuantizedRows:
    xq: object    # int8 [M, Kp] (zero padded past K)
    amax: object  # fp32 [M]
    xsum: object  # int32 [M]
    k: int

    def unpadded(self):
        return self.xq[:, : self.k]


def quantize_activation(x) -> QuantizedRows:
    """Per-row absmax int8 quantization (poly/bitnet_cpu.go:45-117); fp32 or fp64 rows."""
    torch = _torch()
    if x.dim() == 1:
        x = x.unsqueeze(0)
    x = x.contiguous()
    m, k = x.shape
    dev = x.device.index or 0
    xq = torch.empty((m, padded_cols(k)), dtype=torch.int8, device=x.device)
    amax = torch.empty(m, dtype=torch.float32, device=x.device)
    xsum = torch.empty(m, dtype=torch.int32, device=x.device)
    if x.dtype == torch.float64:
        fn = _lib.lib().loom_amd_quantize_rows_f64
    elif x.dtype == torch.float32:
        fn = _lib.lib().loom_amd_quantize_rows
    else:
        raise TypeError("activations must be float32 or float64")
    check(fn(_ptr(x), m, k, _ptr(xq), xq.shape[1], _ptr(amax), _ptr(xsum), _stream(dev)),
          "quantize_rows")
    return QuantizedRows(xq, amax, xsum, k)


def ternary_matvec_quantized(w: TernaryMatrix, q: QuantizedRows, want_acc: bool = False):
    """bitNetTernaryMatVecQuantized over all rows: returns fp32 out [M, N] (loom's
    fp64 result cast to fp32 as the Dense caller does) and optionally int32 acc."""
    torch = _torch()
    if q.k != w.cols:
        raise ValueError(f"activation width {q.k} != matrix cols {w.cols}")
    if q.xq.shape[1] < padded_cols(w.cols):
        raise ValueError("quantized rows are not padded to the tile width")
    m = q.xq.shape[0]
    out = torch.empty((m, w.rows), dtype=torch.float32, device=q.xq.device)
    acc = torch.empty((m, w.rows), dtype=torch.int32, device=q.xq.device) if want_acc else None
    check(_lib.lib().loom_amd_ternary_matmul(w.handle, _ptr(q.xq), q.xq.shape[1], _ptr(q.amax),
                                             _ptr(q.xsum), m, _ptr(out), _ptr(acc),
                                             _stream(w.device)), "ternary_matmul")
    return (out, acc) if want_acc else out


@dataclass
class DenseTaps:
    xq: object
    amax: object
    acc: object


def dense_forward_packed_ternary(w: TernaryMatrix, x, activation: int = ACT_LINEAR,
                                 residual=None, taps: bool = False, out=None):
    """DenseForwardPackedTernaryCPU (poly/dense.go:66-101) for every row of x.

    Returns (preAct, postAct[, DenseTaps]).  With ``residual`` the fp32 sum
    pre + residual (loom's Tensor.Add, poly/poly.go:481-494) is returned as preAct.
    """
    torch = _torch()
    if x.dim() == 1:
        x = x.unsqueeze(0)
    x = x.contiguous()
    if x.dtype != torch.float32 or x.shape[1] != w.cols:
        raise ValueError(f"x must be float32 [M, {w.cols}]")
    m = x.shape[0]
    pre = out if out is not None else torch.empty((m, w.rows), dtype=torch.float32, device=x.device)
    post = None
    if activation != ACT_LINEAR:
        post = torch.empty_like(pre)
    t = None
    ct = None
    if taps:
        t = DenseTaps(torch.empty((m, w.cols), dtype=torch.int8, device=x.device),
                      torch.empty(m, dtype=torch.float32, device=x.device),
                      torch.empty((m, w.rows), dtype=torch.int32, device=x.device))
        ct = _lib.DenseTaps(t.xq.data_ptr(), t.amax.data_ptr(), t.acc.data_ptr())
    if residual is not None:
        residual = residual.contiguous()
        if residual.shape != pre.shape:
            raise ValueError("residual shape must be [M, N]")
    check(_lib.lib().loom_amd_dense_forward(w.handle, _ptr(x), m, activation, _ptr(pre), _ptr(post),
                                            _ptr(residual), C.byref(ct) if ct else None,
                                            _stream(w.device)), "dense_forward")
    post = pre if post is None else post
    return (pre, post, t) if taps else (pre, post)


@dataclass
class SwiGLUTaps:
    xq: object
    amax: object
    acc_gate: object
    acc_up: object
    hq: object
    hamax: object
    acc_down: object


def swiglu_forward_packed_ternary(gate: TernaryMatrix, up: TernaryMatrix, down: TernaryMatrix,
                                  x, inner_norm=None, eps: float = 1e-5,
                                  activation: int = ACT_SILU, norm="strict", bias=None,
                                  residual=None, taps: bool = False):
    """SwiGLUForwardPackedTernaryCPU (poly/swiglu.go:270-322) for every row of x.

    Returns (preAct, postAct[, SwiGLUTaps]): preAct is the normalized gate
    product h [M, inter] (loom's preAct), postAct the FFN output [M, hidden]
    (plus ``residual`` in fp32 when given).  ``norm='strict'`` sums the inner
    RMSNorm in loom's sequential order (bit-exact); ``'fast'`` uses a parallel
    fixed-order sum (normalized values within 1 fp32 ulp).
    """
    torch = _torch()
    if x.dim() == 1:
        x = x.unsqueeze(0)
    x = x.contiguous()
    hidden, inter = gate.cols, gate.rows
    if x.dtype != torch.float32 or x.shape[1] != hidden:
        raise ValueError(f"x must be float32 [M, {hidden}]")
    m = x.shape[0]
    h = torch.empty((m, inter), dtype=torch.float32, device=x.device)
    out = torch.empty((m, hidden), dtype=torch.float32, device=x.device)
    t = None
    ct = None
    if taps:
        i8, f, i = torch.int8, torch.float32, torch.int32
        t = SwiGLUTaps(torch.empty((m, hidden), dtype=i8, device=x.device),
                       torch.empty(m, dtype=f, device=x.device),
                       torch.empty((m, inter), dtype=i, device=x.device),
                       torch.empty((m, inter), dtype=i, device=x.device),
                       torch.empty((m, inter), dtype=i8, device=x.device),
                       torch.empty(m, dtype=f, device=x.device),
                       torch.empty((m, hidden), dtype=i, device=x.device))
        ct = _lib.SwiGLUTaps(*(v.data_ptr() for v in (t.xq, t.amax, t.acc_gate, t.acc_up, t.hq,
                                                      t.hamax, t.acc_down)))
    if inner_norm is not None:
        inner_norm = inner_norm.contiguous()
        if inner_norm.numel() != inter:
            raise ValueError("inner_norm must hold `inter` weights")
    if bias is not None:
        bias = bias.contiguous()
        if bias.numel() != 2 * inter + hidden:
            raise ValueError("bias must hold gate|up|down biases (2*inter + hidden)")
    if residual is not None:
        residual = residual.contiguous()
        if residual.shape != out.shape:
            raise ValueError("residual shape must be [M, hidden]")
    check(_lib.lib().loom_amd_swiglu_forward(
        gate.handle, up.handle, down.handle, _ptr(bias), _ptr(inner_norm), float(eps), activation,
        _norm_mode(norm), _ptr(x), m, _ptr(out), _ptr(residual), _ptr(h),
        C.byref(ct) if ct else None, _stream(gate.device)), "swiglu_forward")
    return (h, out, t) if taps else (h, out)


def norm_quant_rows(h, weight=None, eps: float = 1e-5, norm="strict") -> QuantizedRows:
    """Inner RMSNorm in place on h [M, n] fp32, then requantization."""
    torch = _torch()
    if h.dtype != torch.float32 or not h.is_contiguous() or h.dim() != 2:
        raise ValueError("h must be a contiguous float32 [M, n] tensor")
    m, n = h.shape
    dev = h.device.index or 0
    hq = torch.empty((m, padded_cols(n)), dtype=torch.int8, device=h.device)
    amax = torch.empty(m, dtype=torch.float32, device=h.device)
    xsum = torch.empty(m, dtype=torch.int32, device=h.device)
    if weight is not None:
        weight = weight.contiguous()
    check(_lib.lib().loom_amd_norm_quant_rows(_ptr(h), m, n, _ptr(weight), float(eps),
                                              _norm_mode(norm), _ptr(hq), hq.shape[1],
                                              _ptr(amax), _ptr(xsum), _stream(dev)),
          "norm_quant_rows")
    return QuantizedRows(hq, amax, xsum, n)
