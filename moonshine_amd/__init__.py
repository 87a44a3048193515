"""moonshine_amd: MI355X (gfx950) routed-MoE layer for Moonshine's K3 engine.

The product is libk3moe.so (HIP kernels + C ABI, include/*.h). This package
holds its ctypes binding (_lib), the seeded synthetic inputs of the
benchmark configurations (synth) and the layer drivers (layer, native;
imported lazily because they need torch).
"""
from . import synth  # noqa: F401
from ._lib import LIB_PATH, lib  # noqa: F401
