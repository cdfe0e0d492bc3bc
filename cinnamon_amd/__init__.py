"""MI355X-native (gfx950) FP8 hot path of shyampathak22/cinnamon.

``cinnamon_amd.kernels`` is the drop-in for the reference's ``kernels`` module;
``cinnamon_amd.layers`` holds the FP8 grouped-expert layer.  The native code is
libcinnamon_fp8.so (C ABI: include/cinnamon_fp8.h), built by ``cinnamon_amd._build``.
"""
from . import _lib  # noqa: F401

__all__ = ["kernels", "layers"]
