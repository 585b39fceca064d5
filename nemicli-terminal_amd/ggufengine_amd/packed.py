"""
`PackedLinear`, the reference's block-format linear layer (models/common.py:364-431), and the routing of
a call by its number of input rows, which `qlinear.QuantLinear` shares.

The weights W (n_out, n_in) stay in their GGUF block bytes.  At construction a layer builds its route
table: an ordered list of (most input rows, kernel) pairs from what the device offers for its format
and row length; a call takes the first route whose bound covers its row count M and otherwise unpacks
W to the compute dtype and multiplies.  The bounds are the reference's (`_rechnen`, common.py:400-431):

  Q4_K, Q6_K (mmvq formats)          M <= mmvq.mv_bis     the int8 mat-vec kernels (mmvq.mv; MMVQ_BIS,
                                                          or MMVQ_BIS_LANG for rows beyond 4096 values)
                                     M <= mmvq.MMQ_BIS    the fp16 matrix-core kernel (mmvq.mm)
  Q4_0, Q8_0, TQ2_0, IQ2_XXS         M == 1               the gathered kernel with expert id 0 (cudakern.mv)
                                     M <= mm_bis          the several-token kernels (cudakern.mm)
  any                                larger M             unpack (bf16, exact values) + matmul, in
                                                          column blocks of ZEILEN_JE_STUECK values

Weights in pinned RAM (`hostmem`) are read by the same kernels over PCIe (`im_ram`); with a `band`
(band.Fliessband) and the layer's number `nr` on it, every call computes on the copy of W that the band
has placed in a VRAM slot.  Everything runs on libnmq's HIP kernels: without the library, or on a CPU
tensor, the constructor raises.
"""
from __future__ import annotations

import contextlib
from typing import Callable, Dict, List, Optional, Tuple

import torch

from . import _native, cudakern, hostmem, mmvq
from .gguf_types import GGML_TYPES, GGUFError
from .mmvq import _starten

Route = Tuple[int, str]     # (most input rows, kernel name)


def unpack(fmt_type: int, raw: torch.Tensor, n_rows: int, n_in: int) -> torch.Tensor:
    """Rows of W in block format -> (n_rows, n_in) bf16: the exact dequantised values, rounded to nearest
    even (one device launch, `nmq_dequant_bf16`)."""
    _, bv, _ = GGML_TYPES[fmt_type]
    out = torch.empty(n_rows, n_in, dtype=torch.bfloat16, device=raw.device)
    _starten("entpacken", _native.lib().nmq_dequant_bf16, fmt_type, raw.data_ptr(), out.data_ptr(),
             n_rows * n_in // bv, _native.stream_ptr(raw.device))
    return out


def routes(name: str, device, n_in: int, mm_limit: int) -> List[Route]:
    """The kernels a layer of format `name` and row length n_in can use on `device`, by input rows."""
    if name in mmvq.FORMATE and mmvq.verfuegbar(device, name, n_in):
        return [(mmvq.mv_bis(name, n_in), "mmvq.mv"), (mmvq.MMQ_BIS[name], "mmvq.mm")]
    if cudakern.verfuegbar(device, name, n_in):
        return [(1, "cudakern.mv"), (mm_limit, "cudakern.mm")]
    return []


class PackedLinear:
    """y = x @ W^T (+ b) with W kept in a GGUF block format (reference models/common.py:364-431).
    Output in `dtype`; the bias is added in that dtype."""

    KERNEL_BIS = cudakern.MM_ZEILEN
    ZEILEN_JE_STUECK = 32 * 1024 * 1024          # values of W unpacked per block of output columns

    def __init__(self, raw: torch.Tensor, ggml_type: int, n_out: int, n_in: int,
                 bias: Optional[torch.Tensor] = None, dtype: torch.dtype = torch.bfloat16):
        spec = GGML_TYPES.get(ggml_type)
        if spec is None:
            raise GGUFError(f"PackedLinear: type {ggml_type} is not one of this library's formats")
        name, bv, bb = spec
        if n_out <= 0 or n_in <= 0 or n_in % bv or raw.numel() != n_out * (n_in // bv) * bb:
            raise GGUFError(f"PackedLinear: {raw.numel()} bytes are not {n_out}x{n_in} {name}")
        if not raw.is_cuda or not _native.available(raw.device):
            raise RuntimeError("PackedLinear: libnmq.so is not loaded or the device is not gfx950")
        self.name, self.ggml_type = name, ggml_type
        self.n_out, self.n_in = n_out, n_in
        self.raw = raw.view(1, -1)
        self.zeilen_bytes = n_in // bv * bb
        self.dtype = dtype
        self.b = None if bias is None else bias.to(dtype)
        self.w = None                            # duck typing with the dense Linear
        self.mmvq = name in mmvq.FORMATE and mmvq.verfuegbar(raw.device, name, n_in)
        self.kernel = cudakern.verfuegbar(raw.device, name, n_in)
        self.mm_bis = min(self.KERNEL_BIS, cudakern.mm_bis(raw.device)) if self.kernel else 1
        self.im_ram = hostmem.abgebildet(raw)    # pinned host memory read over PCIe
        self.band = None                         # band.Fliessband: W copied into a VRAM slot per use
        self.nr = -1
        self._routes = routes(name, raw.device, n_in, self.mm_bis)
        self._id0: Optional[torch.Tensor] = None

    # -- routing -------------------------------------------------------------------------------------
    def route(self, m: int) -> str:
        """Kernel name for m input rows ("unpack" past every bound)."""
        for upto, kind in self._routes:
            if m <= upto:
                return kind
        return "unpack"

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.reshape(-1, self.n_in)
        with self._weights() as raw:
            y = self.forward_raw(rows, raw)
        if self.b is not None:
            y = y + self.b
        return y.reshape(*x.shape[:-1], self.n_out)

    @contextlib.contextmanager
    def _weights(self):
        """W's bytes for one call: the layer's own, or the band's VRAM slot for the duration of the call."""
        if self.band is None:
            yield self.raw
            return
        slot = self.band.holen(self.nr)
        try:
            yield slot.view(1, -1)
        finally:
            self.band.fertig(self.nr)

    def forward_raw(self, rows: torch.Tensor, raw: torch.Tensor, dtype: Optional[torch.dtype] = None
                    ) -> torch.Tensor:
        """(M, n_in) -> (M, n_out) in `dtype` (default: the layer's), no bias, W read from `raw`."""
        dtype = dtype or self.dtype
        kind = self.route(rows.shape[0])
        if kind == "unpack":
            return self._by_unpacking(rows, raw, dtype)
        return _KERNELS[kind](self, rows, raw).to(dtype)

    # -- the kernels ---------------------------------------------------------------------------------
    def _mmvq_mv(self, rows, raw):
        return mmvq.mv(self.name, raw, rows, self.n_out, self.n_in)

    def _mmvq_mm(self, rows, raw):
        return mmvq.mm(self.name, raw, rows, self.n_out, self.n_in)

    def _cudakern_mv(self, rows, raw):
        if self._id0 is None or self._id0.device != raw.device:
            self._id0 = torch.zeros(1, dtype=torch.int64, device=raw.device)   # expert 0 = W itself
        return cudakern.mv(self.name, raw, self._id0, rows, self.n_out, self.n_in)

    def _cudakern_mm(self, rows, raw):
        return cudakern.mm(self.name, raw, rows, self.n_out, self.n_in)

    def _by_unpacking(self, rows: torch.Tensor, raw: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """W unpacked to bf16 in blocks of output columns (at most ZEILEN_JE_STUECK values at a time) and
        multiplied in `dtype`."""
        xs = rows.to(dtype)
        step = max(1, self.ZEILEN_JE_STUECK // self.n_in)
        flat = raw.reshape(-1)
        parts = []
        for r0 in range(0, self.n_out, step):
            n = min(step, self.n_out - r0)
            w = unpack(self.ggml_type, flat[r0 * self.zeilen_bytes:(r0 + n) * self.zeilen_bytes], n, self.n_in)
            parts.append(xs @ w.to(dtype).t())
            del w
        return parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)


_KERNELS: Dict[str, Callable] = {
    "mmvq.mv": PackedLinear._mmvq_mv,
    "mmvq.mm": PackedLinear._mmvq_mm,
    "cudakern.mv": PackedLinear._cudakern_mv,
    "cudakern.mm": PackedLinear._cudakern_mm,
}
