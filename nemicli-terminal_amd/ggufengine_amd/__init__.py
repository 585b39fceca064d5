"""MI355X (gfx950) GGUF quantized mat-vec path: drop-in replacements for the reference's
ggufengine/mmvq.py, ggufengine/cudakern.py and ggufengine/qlinear.py (same names, arguments, return
shapes and error behaviour), backed by hand-written HIP kernels in libnmq.so (C ABI: include/nmq.h)
loaded with ctypes.  There is no CPU or torch fallback: if libnmq.so is missing or the device is not
gfx950, the availability probes return False and direct calls raise.
"""
from . import gguf_types, encode  # noqa: F401
from ._native import available, lib  # noqa: F401
