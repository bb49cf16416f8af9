"""loom_amd -- MI355X (gfx950) implementation of loom's BitNet b1.58 ternary
hot path, behind loom's v2 vendor plugin ABI.

    loom_amd.accel   mirror of poly/accel (Plugin / CompiledLayer over the C ABI)
    loom_amd.bitnet  device-resident ternary layers (Dense, SwiGLU FFN, stages)
    loom_amd.build   hipcc build of libloom_accel_amd.so

The compute is in loom_amd/csrc (HIP, gfx950 only); Python is the host.
"""
from . import build  # noqa: F401

__all__ = ["accel", "bitnet", "build"]
