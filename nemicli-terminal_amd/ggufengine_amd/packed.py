"""
The reference's block-format linear layer, `PackedLinear` (models/common.py:364-431), for the formats
of this library: W (n_out, n_in) stays in its GGUF block bytes and each call is dispatched by the
number of input rows M exactly as `PackedLinear._rechnen` does (common.py:400-431):

  - M <= mmvq.MMVQ_BIS (Q4_K/Q6_K): mmvq.mv, the int8 mat-vec kernels;
  - M <= mmvq.MMQ_BIS (Q4_K/Q6_K): mmvq.mm;
  - M == 1 (other formats): cudakern.mv with expert id 0 (W itself);
  - M <= mm_bis (other formats): cudakern.mm;
  - else: W unpacked to the compute dtype piecewise (ZEILEN_JE_STUECK values at a time) and multiplied.

Every branch runs on libnmq's HIP kernels (the unpack too); without the library the constructor
raises instead of falling back.  Weights in pinned RAM (`hostmem`): `im_ram` is set and the kernels
read them over PCIe, or, with a `band` (band.Fliessband) and the layer's number `nr` on it, each call
computes on the matrix copied whole into a VRAM slot a few layers ahead (reference common.py:387-399).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native, cudakern, hostmem, mmvq
from .band import Fliessband
from .gguf_types import GGML_TYPES, GGUFError
from .mmvq import _starten


def unpack(fmt_type: int, raw: torch.Tensor, n_rows: int, n_in: int) -> torch.Tensor:
    """Rows of W in block format -> (n_rows, n_in) bf16, exact values rounded to nearest-even."""
    name, bs, _ = GGML_TYPES[fmt_type]
    out = torch.empty(n_rows, n_in, dtype=torch.bfloat16, device=raw.device)
    _starten("entpacken", _native.lib().nmq_dequant_bf16, fmt_type, raw.data_ptr(), out.data_ptr(),
             n_rows * n_in // bs, _native.stream_ptr(raw.device))
    return out


class PackedLinear:
    """y = x @ W^T (+ b) with W kept in block format (reference models/common.py:364-431)."""

    KERNEL_BIS = cudakern.MM_ZEILEN
    ZEILEN_JE_STUECK = 32 * 1024 * 1024          # values unpacked at once

    def __init__(self, raw: torch.Tensor, ggml_type: int, n_out: int, n_in: int,
                 bias: Optional[torch.Tensor] = None, dtype: torch.dtype = torch.bfloat16):
        if ggml_type not in GGML_TYPES:
            raise GGUFError(f"PackedLinear: type {ggml_type} is not one of this library's formats")
        name, bs, ts = GGML_TYPES[ggml_type]
        if n_in % bs or raw.numel() != n_out * (n_in // bs) * ts:
            raise GGUFError(f"PackedLinear: {raw.numel()} bytes do not hold {n_out}x{n_in} {name}")
        if not raw.is_cuda or not _native.available(raw.device):
            raise RuntimeError("PackedLinear: libnmq.so is not loaded or the device is not gfx950")
        self.raw = raw.view(1, -1)
        self.ggml_type = ggml_type
        self.n_out, self.n_in = n_out, n_in
        self.b = None if bias is None else bias.to(dtype)
        self.dtype = dtype
        self.w = None                            # duck-typing with Linear (as in the reference)
        self.name = name
        self.zeilen_bytes = n_in // bs * ts
        self.kernel = cudakern.verfuegbar(raw.device, name, n_in)
        self.mmvq = name in mmvq.FORMATE and mmvq.verfuegbar(raw.device, name, n_in)
        self.mm_bis = min(self.KERNEL_BIS, cudakern.mm_bis(raw.device)) if self.kernel else 1
        self.im_ram = hostmem.abgebildet(raw)    # pinned RAM, read over PCIe
        self.band: Optional[Fliessband] = None   # with it: whole copies a few matrices ahead
        self.nr = -1
        self._nullen: dict = {}

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if self.band is None:
            return self._rechnen(x, self.raw)
        roh = self.band.holen(self.nr).view(1, -1)
        try:
            return self._rechnen(x, roh)
        finally:
            self.band.fertig(self.nr)

    def _rechnen(self, x: torch.Tensor, raw: torch.Tensor) -> torch.Tensor:
        x2 = x.reshape(-1, self.n_in)
        M = x2.shape[0]
        if self.mmvq and M <= mmvq.MMVQ_BIS[self.name]:
            y = mmvq.mv(self.name, raw, x2, self.n_out, self.n_in).to(self.dtype)
        elif self.mmvq and M <= mmvq.MMQ_BIS[self.name]:
            y = mmvq.mm(self.name, raw, x2, self.n_out, self.n_in).to(self.dtype)
        elif self.kernel and M == 1:
            if M not in self._nullen:            # the row uses "expert" 0, i.e. W itself
                self._nullen[M] = torch.zeros(M, dtype=torch.long, device=raw.device)
            y = cudakern.mv(self.name, raw, self._nullen[M], x2, self.n_out, self.n_in).to(self.dtype)
        elif self.kernel and M <= self.mm_bis:
            y = cudakern.mm(self.name, raw, x2, self.n_out, self.n_in).to(self.dtype)
        else:
            xd = x2.to(self.dtype)
            y = torch.empty(M, self.n_out, dtype=self.dtype, device=x2.device)
            stueck = max(1, self.ZEILEN_JE_STUECK // self.n_in)
            for r0 in range(0, self.n_out, stueck):
                r1 = min(r0 + stueck, self.n_out)
                w = unpack(self.ggml_type, raw[0, r0 * self.zeilen_bytes:r1 * self.zeilen_bytes], r1 - r0,
                           self.n_in).to(self.dtype)
                y[:, r0:r1] = xd @ w.t()
                del w
        if self.b is not None:
            y = y + self.b
        return y.reshape(*x.shape[:-1], self.n_out)
