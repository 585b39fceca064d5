"""
Drop-in for the reference's ggufengine/qlinear.py ("QLinear forward") on gfx950.

Same public surface (qlinear.py:42-52, 195-276): `kernel_available`, `quantizable`,
`build_quant_linear(raw, ggml_type, n_out, n_in, bias)` and `QuantLinear` with `n_out`, `n_in`, `b`,
`w = None`, `dtype`, `type_name` and `__call__(x)`.  The reference repacks GGUF blocks into torch's
int4 "tinygemm" groups; here the GGUF bytes stay as they are and every call runs the int8 mat-vec
kernels of libnmq (up to UNPACK_FROM rows) or unpacks to bf16 once per call for long inputs
(UNPACK_FROM rows and more, like the reference, then torch's GEMM).  Output dtype is bf16 like the
reference; `forward_f32` returns the fp32 result of the kernels.

Not reproduced: the reference's `mats` attribute (tinygemm-packed int4 tensors read directly by
models/moe.py `_StapelTeil`) -- experts in this library go through cudakern.mv / linear.PackedExperts.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native
from .gguf_types import GGML_TYPES, GGUFError
from .mmvq import Eingang, _starten

G = 32                 # sub-block size of the GGUF formats (the reference's tinygemm group size)
UNPACK_FROM = 256      # from this many rows: unpack to bf16 + GEMM instead of the mat-vec kernels
_FORMATS = ("Q4_0", "Q8_0", "Q4_K", "Q6_K")


def kernel_available(device: torch.device) -> bool:
    device = torch.device(device)
    return device.type == "cuda" and _native.available(device)


def quantizable(ggml_type: int, n_out: int, n_in: int, min_elements: int = 1 << 20) -> bool:
    """Kernel-capable; matrices smaller than `min_elements` stay dense in the reference's loader
    (qlinear.py:46-52)."""
    if ggml_type not in GGML_TYPES:
        return False
    name, bv, _ = GGML_TYPES[ggml_type]
    if name not in _FORMATS:
        return False
    return n_out > 0 and n_in > 0 and n_in % bv == 0 and n_out * n_in >= min_elements


class QuantLinear:
    """y = x @ W^T (+ b), W kept in its GGUF block format on the device."""

    def __init__(self, raw: torch.Tensor, ggml_type: int, n_out: int, n_in: int,
                 bias: Optional[torch.Tensor] = None, type_name: str = ""):
        self.raw = raw.reshape(-1)
        self.ggml_type = ggml_type
        self.n_out, self.n_in = n_out, n_in
        self.b = None if bias is None else bias.to(torch.bfloat16)
        self.type_name = type_name or GGML_TYPES[ggml_type][0]
        self.w = None   # duck typing with Linear (dtype queries)

    @property
    def dtype(self):
        return torch.bfloat16

    def bf16_weight(self) -> torch.Tensor:
        """The matrix as (n_out, n_in) bf16."""
        _, bv, _ = GGML_TYPES[self.ggml_type]
        out = torch.empty(self.n_out, self.n_in, dtype=torch.bfloat16, device=self.raw.device)
        L = _native.lib()
        _starten("entpacken", L.nmq_dequant_bf16, self.ggml_type, self.raw.data_ptr(), out.data_ptr(),
                 self.n_out * self.n_in // bv, _native.stream_ptr(self.raw.device))
        return out

    def forward_f32(self, x: torch.Tensor) -> torch.Tensor:
        """(..., n_in) -> (M, n_out) float32 through the int8 mat-vec kernels (no bias)."""
        x2 = x.reshape(-1, self.n_in)
        e = Eingang(x2)
        M = x2.shape[0]
        y = torch.empty(M, self.n_out, dtype=torch.float32, device=self.raw.device)
        L = _native.lib()
        _starten("mv", L.nmq_mv, self.ggml_type, self.raw.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
                 e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), self.n_out, self.n_in, M,
                 _native.stream_ptr(self.raw.device))
        return y

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        x2 = x.reshape(-1, self.n_in).to(torch.bfloat16)
        if x2.shape[0] >= UNPACK_FROM:
            y = x2 @ self.bf16_weight().t()
        else:
            y = self.forward_f32(x2).to(torch.bfloat16)
        if self.b is not None:
            y = y + self.b
        return y.reshape(*x.shape[:-1], self.n_out)


def build_quant_linear(raw: torch.Tensor, ggml_type: int, n_out: int, n_in: int,
                       bias: Optional[torch.Tensor] = None) -> QuantLinear:
    """raw: uint8 block bytes of an (n_out, n_in) GGUF matrix already on the device
    (reference qlinear.py:242-276)."""
    if ggml_type not in GGML_TYPES:
        raise GGUFError(f"tensor type {ggml_type} has no kernel here")
    name, block_size, type_size = GGML_TYPES[ggml_type]
    if raw.numel() != n_out * n_in // block_size * type_size or n_in % block_size:
        raise GGUFError("byte count mismatch in build_quant_linear")
    return QuantLinear(raw, ggml_type, n_out, n_in, bias, name)
