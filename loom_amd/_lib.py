"""ctypes binding of libloom_accel_amd.so (the C-ABI of include/loom_accel.h and
include/loom_accel_amd.h).

The shared library is built in-tree by loom_amd.build (hipcc, gfx950).  There is
no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

from . import build as _build

LIB_PATH = _build.LIB_PATH

_lib: C.CDLL | None = None

P = C.c_void_p
i32 = C.c_int
f32 = C.c_float
f64 = C.c_double
sz = C.c_size_t
cstr = C.c_char_p


class LibraryMissing(RuntimeError):
    pass


class LayerDesc(C.Structure):
    """loom_accel_layer_desc (poly/accel/include/loom_accel.h:16-20)."""
    _fields_ = [("layer_name", cstr), ("dtype", cstr), ("size_label", cstr)]


class DenseTaps(C.Structure):
    _fields_ = [("xq", P), ("amax", P), ("acc", P)]


class SwiGLUTaps(C.Structure):
    _fields_ = [("xq", P), ("amax", P), ("acc_gate", P), ("acc_up", P), ("hq", P),
                ("hamax", P), ("acc_down", P)]


class BlockDesc(C.Structure):
    """loom_amd_block_desc."""
    _fields_ = [("hidden", i32), ("num_heads", i32), ("num_kv_heads", i32), ("head_dim", i32),
                ("intermediate", i32), ("max_seq_len", i32), ("max_batch", i32),
                ("rope_theta", f64), ("norm_eps", f64), ("attn_eps", f64), ("ffn_eps", f64),
                ("ffn_activation", i32), ("norm_mode", i32)]


class BlockWeights(C.Structure):
    """loom_amd_block_weights (matrix handles + host fp32 arrays)."""
    _fields_ = [("q", P), ("k", P), ("v", P), ("o", P), ("gate", P), ("up", P), ("down", P),
                ("norm1", P), ("norm2", P), ("attn_inner_norm", P), ("ffn_inner_norm", P),
                ("bias_q", P), ("bias_k", P), ("bias_v", P), ("bias_o", P),
                ("q_norm", P), ("q_norm_len", i32), ("k_norm", P), ("k_norm_len", i32)]


class BlockTaps(C.Structure):
    """loom_amd_block_taps."""
    _fields_ = [("y1", P), ("q", P), ("attn", P), ("mid", P), ("xq1", P), ("amax1", P),
                ("attn_norm", P), ("aq", P), ("aamax", P), ("y2", P), ("xq2", P), ("amax2", P),
                ("h", P), ("hn", P), ("hq", P), ("hamax", P)]


class ModelDesc(C.Structure):
    """loom_amd_model_desc."""
    _fields_ = [("block", BlockDesc), ("num_layers", i32), ("vocab", i32),
                ("final_norm_eps", f64), ("max_tokens", i32), ("max_prefill", i32),
                ("lm_head_order", i32)]


# name -> (restype, argtypes); every symbol declared in include/*.h.
SIGNATURES = {
    # loom_accel.h (v2 plugin ABI)
    "loom_accel_api_version": (i32, []),
    "loom_accel_vendor_id": (cstr, []),
    "loom_accel_npu_available": (i32, []),
    "loom_accel_plugin_open": (P, [cstr]),
    "loom_accel_plugin_close": (None, [P]),
    "loom_accel_weight_bytes": (sz, [C.POINTER(LayerDesc)]),
    "loom_accel_compile_layer": (i32, [P, C.POINTER(LayerDesc), P, sz, C.POINTER(P),
                                       C.POINTER(f64), C.c_char_p, sz]),
    "loom_accel_release_layer": (None, [P]),
    "loom_accel_layer_io_bytes": (i32, [P, C.POINTER(sz), C.POINTER(sz), C.c_char_p, sz]),
    "loom_accel_first_infer": (i32, [P, C.POINTER(f64), C.c_char_p, sz]),
    "loom_accel_infer": (i32, [P, P, sz, P, sz, C.POINTER(f64), C.c_char_p, sz]),
    "loom_accel_last_error": (cstr, [P]),
    # loom_accel_amd.h (device-resident extension)
    "loom_amd_last_error": (cstr, []),
    "loom_amd_device_count": (i32, []),
    "loom_amd_kernel_variant": (cstr, [i32]),
    "loom_amd_matrix_create": (i32, [i32, P, sz, i32, i32, i32, f32, C.POINTER(P)]),
    "loom_amd_matrix_from_entity_blob": (i32, [i32, P, sz, C.POINTER(P), C.POINTER(sz)]),
    "loom_amd_matrix_from_ms_offline": (i32, [i32, P, i32, i32, f32, C.POINTER(P)]),
    "loom_amd_matrix_from_float32": (i32, [i32, P, i32, i32, C.POINTER(P), C.POINTER(f32)]),
    "loom_amd_matrix_release": (None, [P]),
    "loom_amd_matrix_shape": (i32, [P, C.POINTER(i32), C.POINTER(i32), C.POINTER(f32),
                                    C.POINTER(sz)]),
    "loom_amd_matrix_tiles": (P, [P]),
    "loom_amd_quantize_rows": (i32, [P, i32, i32, P, i32, P, P, P]),
    "loom_amd_quantize_rows_f64": (i32, [P, i32, i32, P, i32, P, P, P]),
    "loom_amd_ternary_matmul": (i32, [P, P, i32, P, P, i32, P, P, P]),
    "loom_amd_norm_quant_rows": (i32, [P, i32, i32, P, f64, i32, P, i32, P, P, P]),
    "loom_amd_ordered_sum_rows": (i32, [P, i32, i32, f64, P, i32, P]),
    "loom_amd_exp_rows": (i32, [P, C.c_long, P, P]),
    "loom_amd_reload_tuning": (i32, []),
    "loom_amd_dense_forward": (i32, [P, P, i32, i32, P, P, P, C.POINTER(DenseTaps), P]),
    "loom_amd_dense_forward_noalloc": (i32, [P, P, i32, i32, P, P, P, P]),
    "loom_amd_swiglu_forward": (i32, [P, P, P, P, P, f64, i32, i32, P, i32, P, P, P,
                                      C.POINTER(SwiGLUTaps), P]),
    "loom_amd_block_create": (i32, [i32, C.POINTER(BlockDesc), C.POINTER(BlockWeights),
                                    C.POINTER(P)]),
    "loom_amd_block_release": (None, [P]),
    "loom_amd_block_forward": (i32, [P, P, i32, i32, C.POINTER(BlockTaps), P]),
    "loom_amd_block_kv_offset": (i32, [P]),
    "loom_amd_block_kv_cache": (i32, [P, i32, C.POINTER(P), C.POINTER(P)]),
    "loom_amd_lm_head": (i32, [P, i32, i32, P, i32, P, P]),
    "loom_amd_lm_head_sequential": (i32, [P, i32, i32, P, i32, P, P]),
    "loom_amd_greedy_sample": (i32, [P, i32, i32, P, P]),
    "loom_amd_model_create": (i32, [i32, C.POINTER(ModelDesc), C.POINTER(BlockWeights), P, P, P,
                                    C.POINTER(P)]),
    "loom_amd_model_release": (None, [P]),
    "loom_amd_model_prefill": (i32, [P, P, i32, i32, P, P]),
    "loom_amd_model_decode": (i32, [P, i32, i32, P, P]),
    "loom_amd_model_tokens": (i32, [P, P, i32, P]),
    "loom_amd_model_position": (i32, [P]),
    "loom_amd_model_last_hidden": (P, [P]),
}


def lib() -> C.CDLL:
    """Load the in-tree library (raises LibraryMissing if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m loom_amd.build` "
                "(hipcc, gfx950); loom_amd has no CPU fallback")
        handle = C.CDLL(LIB_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


class AMDError(RuntimeError):
    pass


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().loom_amd_last_error().decode(errors="replace")
        raise AMDError(f"{what}: {msg}" if what else msg)
