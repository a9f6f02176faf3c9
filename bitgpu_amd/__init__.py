"""bitgpu_amd -- MI355X (gfx950) attention hot path of bitgpu, behind a C ABI.

The HIP kernels and the C ABI live in ``csrc/`` (built into ``lib/libbitgpu_attn.so``);
``engine`` mirrors the reference engine's per-layer attention dispatch on top of it.
"""
from ._lib import BitgpuError, GpuOutOfMemoryError, LIB_PATH  # noqa: F401

__version__ = "0.1.0"
