"""
Drop-in for the reference's ggufengine/qlinear.py ("QLinear forward") on gfx950.

Same public surface (qlinear.py:42-52, 195-276): `kernel_available`, `quantizable`, `G`, `UNPACK_FROM`,
`build_quant_linear(raw, ggml_type, n_out, n_in, bias)` and `QuantLinear` with `n_out`, `n_in`, `b`,
`w = None`, `dtype` (bf16), `type_name`, `bf16_weight()` and `__call__(x)`.  The reference repacks the GGUF
blocks into torch's int4 "tinygemm" groups and multiplies with `torch._weight_int4pack_mm`; here the GGUF
bytes stay as they are and a call is routed by its row count exactly like `packed.PackedLinear` (the int8
mat-vec kernels, the matrix-core kernels, or an unpack to bf16 + GEMM for long inputs), so W is read once
per call.  As in the reference, x is cast to bf16 first, the result is bf16 and the bias is added in bf16.

`mats` (the reference's list of tinygemm-packed tensors, which models/moe.py `_StapelTeil` stacks and
feeds to torch's int4 kernel) does not exist for these weights: reading it raises TypeError.  Expert
tensors of this library's formats never become QuantLinear lists in the reference's loader, because
`cudakern.IMMER_GEPACKT` names every format here, so `WeightLoader.experts` builds `PackedExperts` (the
gathered kernel) for them; `experts.PackedExperts.aus_quantlinear` turns a list of QuantLinear experts
made by other code into one.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native, packed
from .mmvq import Eingang, _starten
from .gguf_types import GGML_TYPES, GGUFError

G = 32                 # sub-block size of the GGUF formats (the reference's tinygemm group size)
UNPACK_FROM = 256      # the reference's row count from which it unpacks to bf16 (here: past the kernels)
_FORMATS = ("Q4_0", "Q8_0", "Q4_K", "Q6_K")


def kernel_available(device: torch.device) -> bool:
    device = torch.device(device)
    return device.type == "cuda" and _native.available(device)


def quantizable(ggml_type: int, n_out: int, n_in: int, min_elements: int = 1 << 20) -> bool:
    """A format this class serves and a whole number of blocks per row; matrices with fewer than
    `min_elements` values stay dense in the reference's loader (qlinear.py:46-52)."""
    spec = GGML_TYPES.get(ggml_type)
    if spec is None or spec[0] not in _FORMATS:
        return False
    return n_out > 0 and n_in > 0 and n_in % spec[1] == 0 and n_out * n_in >= min_elements


class QuantLinear:
    """y = x @ W^T (+ b) in bf16, W kept in its GGUF block format on the device."""

    def __init__(self, raw: torch.Tensor, ggml_type: int, n_out: int, n_in: int,
                 bias: Optional[torch.Tensor] = None, type_name: str = ""):
        self._layer = packed.PackedLinear(raw.reshape(-1), ggml_type, n_out, n_in, None, torch.bfloat16)
        self.raw = self._layer.raw.view(-1)
        self.ggml_type = ggml_type
        self.n_out, self.n_in = n_out, n_in
        self.b = None if bias is None else bias.to(torch.bfloat16)
        self.type_name = type_name or GGML_TYPES[ggml_type][0]
        self.w = None   # duck typing with the dense Linear (dtype queries)

    @property
    def dtype(self):
        return torch.bfloat16

    @property
    def mats(self):
        raise TypeError(
            "QuantLinear of libnmq keeps GGUF block bytes and has no tinygemm int4 planes; stack expert "
            "layers with experts.PackedExperts.aus_quantlinear() (the gathered expert kernel) instead")

    def route(self, m: int) -> str:
        """Kernel a call with m input rows runs (see packed.PackedLinear.route)."""
        return self._layer.route(m)

    def bf16_weight(self) -> torch.Tensor:
        """The matrix as (n_out, n_in) bf16: the exact dequantised values rounded to nearest even."""
        return packed.unpack(self.ggml_type, self.raw, self.n_out, self.n_in)

    def forward_f32(self, x: torch.Tensor) -> torch.Tensor:
        """(..., n_in) -> (M, n_out) float32 from the int8 mat-vec kernels on x as given (its two-stage
        input, not rounded to bf16 first), no bias; M of any size in launches of up to 16 rows."""
        rows = x.reshape(-1, self.n_in)
        e = Eingang(rows)
        y = torch.empty(rows.shape[0], self.n_out, dtype=torch.float32, device=self.raw.device)
        _starten("mv", _native.lib().nmq_mv, self.ggml_type, self.raw.data_ptr(), e.xq.data_ptr(),
                 e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), self.n_out, self.n_in,
                 rows.shape[0], _native.stream_ptr(self.raw.device))
        return y

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.reshape(-1, self.n_in).to(torch.bfloat16)
        y = self._layer.forward_raw(rows, self._layer.raw)
        if self.b is not None:
            y = y + self.b
        return y.reshape(*x.shape[:-1], self.n_out)


def build_quant_linear(raw: torch.Tensor, ggml_type: int, n_out: int, n_in: int,
                       bias: Optional[torch.Tensor] = None) -> QuantLinear:
    """raw: uint8 block bytes of an (n_out, n_in) GGUF matrix already on the device
    (reference qlinear.py:242-276)."""
    spec = GGML_TYPES.get(ggml_type)
    if spec is None:
        raise GGUFError(f"tensor type {ggml_type} has no kernel here")
    name, block_size, type_size = spec
    if n_in % block_size or raw.numel() != n_out * n_in // block_size * type_size:
        raise GGUFError("byte count mismatch in build_quant_linear")
    return QuantLinear(raw, ggml_type, n_out, n_in, bias, name)
