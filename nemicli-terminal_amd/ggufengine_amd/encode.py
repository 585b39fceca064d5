"""GGUF block encoders (host C++ in libnmq.so, nmq_encode): fp32 weights -> block bytes.

The reference ships no quantiser for Q4_K, Q6_K or IQ2_XXS (only Q8_0 and ternary packers in its
tests); these are this library's own.  Results are checked against the dequantisation of the
encoded bytes, so the encoder decides only how realistic the weights are.
"""
from __future__ import annotations

import numpy as np

from . import _native
from .gguf_types import block_info


def encode(fmt, w: np.ndarray, threads: int = 0) -> np.ndarray:
    """w: fp32 array (any shape, size a multiple of the block) -> flat uint8 blocks."""
    t, _, bv, bb = block_info(fmt)
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    if w.size % bv:
        raise ValueError(f"{w.size} values are not a multiple of the block size {bv}")
    out = np.empty(w.size // bv * bb, dtype=np.uint8)
    n = _native.lib().nmq_encode(t, w.ctypes.data, w.size, out.ctypes.data, int(threads))
    if n < 0:
        _native.check(int(n))
    return out


def pack_ternary(codes: np.ndarray, d16: np.ndarray) -> np.ndarray:
    """TQ2_0 blocks from codes in {0, 1, 2} (value = (code - 1) * d) and per-block fp16 scales,
    written in the layout of the reference's dequantiser (quant.py:417-421)."""
    codes = np.asarray(codes, dtype=np.uint8).reshape(-1, 2, 4, 32)   # (block, half, shift, m)
    nb = codes.shape[0]
    out = np.zeros((nb, 66), dtype=np.uint8)
    qs = np.zeros((nb, 2, 32), dtype=np.uint8)
    for l in range(4):
        qs |= (codes[:, :, l, :] & 3) << (2 * l)
    out[:, :64] = qs.reshape(nb, 64)
    out[:, 64:66] = np.asarray(d16, dtype=np.float16).reshape(nb, 1).view(np.uint8)
    return out.ravel()
