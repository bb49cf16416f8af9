"""Host-side mirror of loom's ``poly/accel`` package for the AMD plugin.

loom loads vendor plugins through cgo: ``dlopen(RTLD_NOW|RTLD_LOCAL)``, a
``dlsym`` for each of the 12 v2 symbols, an API-version check, then
``loom_accel_plugin_open`` (poly/accel/plugin_linux.go:45-92, 184-212).  This
module performs the same sequence over ctypes and exposes the same surface,
``Plugin`` / ``CompiledLayer`` / ``CompileResult`` / ``InferResult`` /
``LayerBinding`` (poly/accel/accel.go:11-47, poly/accel/binding.go:4-41), with
the same error behaviour, so a Python test reads like loom's own plugin tests.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

from . import _lib

API_VERSION = 2  # LOOM_ACCEL_API_VERSION (poly/accel/include/loom_accel.h:11)
ERR_BUF = 512    # loom passes 512-byte error buffers (poly/accel/plugin_linux.go:243)

V2_SYMBOLS = (
    "loom_accel_api_version", "loom_accel_vendor_id", "loom_accel_npu_available",
    "loom_accel_plugin_open", "loom_accel_plugin_close", "loom_accel_weight_bytes",
    "loom_accel_compile_layer", "loom_accel_release_layer", "loom_accel_layer_io_bytes",
    "loom_accel_first_infer", "loom_accel_infer", "loom_accel_last_error",
)


class AccelError(RuntimeError):
    """An error string as loom's Go glue would format it."""


class ErrUnavailable(AccelError):
    """poly/accel/accel.go:9 -- the plugin could not be loaded."""


@dataclass(frozen=True)
class LayerDesc:
    """poly/accel/accel.go:11-16."""
    layer_name: str
    dtype: str
    size_label: str

    def _c(self) -> _lib.LayerDesc:
        return _lib.LayerDesc(self.layer_name.encode(), self.dtype.encode(),
                              self.size_label.encode())


@dataclass
class InferResult:
    infer_ms: float


@dataclass
class CompileResult:
    layer: "CompiledLayer"
    compile_ms: float
    first_infer_ms: float
    in_bytes: int
    out_bytes: int


def default_amd_path() -> str:
    """Plugin path, overridable by LOOM_ACCEL_AMD_SO (as LOOM_ACCEL_INTEL_SO is,
    poly/accel/paths_linux.go:14-27)."""
    return os.environ.get("LOOM_ACCEL_AMD_SO", _lib.LIB_PATH)


def _load(path: str) -> C.CDLL:
    if not os.path.exists(path):
        raise ErrUnavailable(f"accel: load {path}: no such file")
    try:
        h = C.CDLL(path, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    except OSError as e:
        raise ErrUnavailable(f"accel: load {path}: {e}") from e
    for name in V2_SYMBOLS:
        try:
            fn = getattr(h, name)
        except AttributeError as e:
            raise ErrUnavailable(f"accel: load {path}: missing symbol {name}") from e
        res, args = _lib.SIGNATURES[name]
        fn.restype, fn.argtypes = res, args
    return h


def npu_available(path: str | None = None) -> bool:
    """NPUAvailable analogue: 1 when a gfx950 GPU is visible."""
    try:
        return bool(_load(path or default_amd_path()).loom_accel_npu_available())
    except ErrUnavailable:
        return False


class CompiledLayer:
    """poly/accel/accel.go:41-47 (init once, infer many)."""

    def __init__(self, api: C.CDLL, handle: int, in_b: int, out_b: int):
        self._api = api
        self._h = handle
        self._in = in_b
        self._out = out_b

    def in_bytes(self) -> int:
        return self._in

    def out_bytes(self) -> int:
        return self._out

    def infer(self, inp, out) -> InferResult:
        """inp: bytes-like of in_bytes(); out: writable buffer of out_bytes()."""
        if self._h is None:
            raise ErrUnavailable("accel: layer released")
        inv = memoryview(inp).cast("B")
        outv = memoryview(out).cast("B")
        if inv.nbytes != self._in or outv.nbytes != self._out:
            raise AccelError(f"accel: buffer size mismatch in={inv.nbytes} want={self._in} "
                             f"out={outv.nbytes} want={self._out}")
        in_buf = (C.c_char * inv.nbytes).from_buffer_copy(inv)
        out_buf = (C.c_char * outv.nbytes).from_buffer(outv) if not outv.readonly else None
        if out_buf is None:
            raise AccelError("accel: output buffer is read-only")
        ms = C.c_double()
        err = C.create_string_buffer(ERR_BUF)
        rc = self._api.loom_accel_infer(self._h, C.addressof(in_buf), inv.nbytes,
                                        C.addressof(out_buf), outv.nbytes, C.byref(ms), err,
                                        ERR_BUF)
        if rc != 0:
            raise AccelError(f"accel: infer: {err.value.decode(errors='replace')}")
        return InferResult(ms.value)

    def release(self) -> None:
        if self._h is not None:
            self._api.loom_accel_release_layer(self._h)
            self._h = None


class Plugin:
    """poly/accel/accel.go:33-39 over libloom_accel_amd.so."""

    def __init__(self, api: C.CDLL, handle: int, device: str):
        self._api = api
        self._h = handle
        self._device = device

    def vendor_id(self) -> str:
        return self._api.loom_accel_vendor_id().decode()

    def device(self) -> str:
        return self._device

    def weight_bytes(self, desc: LayerDesc) -> int:
        d = desc._c()
        return int(self._api.loom_accel_weight_bytes(C.byref(d)))

    def compile_layer(self, desc: LayerDesc, weight_bytes: bytes) -> CompileResult:
        """Compile, then io_bytes, then first_infer with its error ignored
        (poly/accel/plugin_linux.go:227-273)."""
        d = desc._c()
        wbuf = (C.c_char * len(weight_bytes)).from_buffer_copy(weight_bytes) if weight_bytes else None
        out = C.c_void_p()
        ms = C.c_double()
        err = C.create_string_buffer(ERR_BUF)
        rc = self._api.loom_accel_compile_layer(
            self._h, C.byref(d), C.addressof(wbuf) if wbuf is not None else None,
            len(weight_bytes), C.byref(out), C.byref(ms), err, ERR_BUF)
        if rc != 0:
            raise AccelError(f"accel: compile {desc.layer_name}/{desc.dtype}/{desc.size_label}: "
                             f"{err.value.decode(errors='replace')}")
        in_b, out_b = C.c_size_t(), C.c_size_t()
        if self._api.loom_accel_layer_io_bytes(out, C.byref(in_b), C.byref(out_b), None, 0) != 0:
            self._api.loom_accel_release_layer(out)
            raise AccelError("accel: io_bytes failed")
        first = C.c_double()
        self._api.loom_accel_first_infer(out, C.byref(first), None, 0)
        layer = CompiledLayer(self._api, out.value, in_b.value, out_b.value)
        return CompileResult(layer, ms.value, first.value, in_b.value, out_b.value)

    def last_error(self) -> str:
        return self._api.loom_accel_last_error(self._h).decode(errors="replace")

    def close(self) -> None:
        if self._h is not None:
            self._api.loom_accel_plugin_close(self._h)
            self._h = None


def open_amd(path: str | None = None, device: str = "GPU") -> Plugin:
    """OpenIntel/OpenApple analogue (poly/accel/plugin_linux.go:184-212)."""
    path = path or default_amd_path()
    api = _load(path)
    if api.loom_accel_api_version() != API_VERSION:
        raise AccelError("accel: API version mismatch")
    h = api.loom_accel_plugin_open(device.encode())
    if not h:
        msg = api.loom_accel_last_error(None).decode(errors="replace")
        raise AccelError(f"accel: open device {device}: {msg}")
    return Plugin(api, h, device)


@dataclass
class LayerBinding:
    """poly/accel/binding.go:4-41."""
    desc: LayerDesc
    compiled: CompiledLayer | None
    compile_ms: float = 0.0
    first_infer_ms: float = 0.0
    target: str = field(default="AMDGPU")

    def infer(self, inp, out) -> InferResult:
        if self.compiled is None:
            raise ErrUnavailable("accel: plugin unavailable")
        return self.compiled.infer(inp, out)

    def in_bytes(self) -> int:
        return 0 if self.compiled is None else self.compiled.in_bytes()

    def out_bytes(self) -> int:
        return 0 if self.compiled is None else self.compiled.out_bytes()

    def release(self) -> None:
        if self.compiled is not None:
            self.compiled.release()
            self.compiled = None
