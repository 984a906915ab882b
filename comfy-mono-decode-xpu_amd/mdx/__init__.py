"""mdx: MI355X-native kernels of the Qwen3.5-style W4A8 hybrid decode step.

`mdx._C` mirrors the reference's operator surface (comfy_mono_decode_xpu._C); `mdx.layout`
prepares weights; libmdx.so (built by ../build.py) holds every kernel.
"""
from . import _lib, layout  # noqa: F401
from . import _C  # noqa: F401

__all__ = ["_C", "_lib", "layout"]
