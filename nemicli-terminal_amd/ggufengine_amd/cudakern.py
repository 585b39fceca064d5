"""
Drop-in for the reference's ggufengine/cudakern.py, for the block formats of this path
(Q4_0, Q8_0, Q4_K, Q6_K, TQ2_0, IQ2_XXS), on gfx950.

Same names, arguments and return shapes as the reference (cudakern.py:31-54, 733-790):
`FORMATE`, `IMMER_GEPACKT`, `MM_ZEILEN`, `MM_GROESSEN`, `verfuegbar`, `mm_bis`, `mv`, `mm`.  As in
the reference, x is first rounded to bf16; the kernels then quantise it in two int8 stages and use
v_dot4_i32_i8 (the reference's cudakern kernels compute in fp32 on the bf16 values; both are checked
against the dequantised weights times the same bf16 x).  The expert gather reads `ids` on the device
(graph-capturable) and accepts the per-expert stride of `raw` or an address table (`adressen`).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native
from .gguf_types import TYPE_ID
from .mmvq import _starten, _werte, eingang_bf16

THREADS = 256
FORMATE = {"Q4_0": (32, 18), "Q8_0": (32, 34), "Q4_K": (256, 144), "Q6_K": (256, 210), "IQ2_XXS": (256, 66), "TQ2_0": (256, 66)}
# formats that always stay in their block bytes.  In the reference these are the formats without an int4
# repack in qlinear; this library repacks nothing, so every format it serves is one (the reference's
# loader then builds PackedExperts, the gathered kernel, for their expert tensors, models/common.py:215)
IMMER_GEPACKT = frozenset(FORMATE)
MM_ZEILEN = 16
MM_GROESSEN = tuple(range(2, MM_ZEILEN + 1))
MAX_N_IN = 1 << 20


def verfuegbar(device, fmt: str, n_in: int) -> bool:
    """Kernel for this format and row length on this device (reference cudakern.py:733-739)."""
    if fmt not in FORMATE or n_in <= 0 or n_in % FORMATE[fmt][0] or n_in > MAX_N_IN:
        return False
    return _native.available(device)


def mm_bis(device) -> int:
    """Most input rows of one `mm` call on this device (1: none) (reference cudakern.py:742-745)."""
    return MM_ZEILEN if _native.available(device) else 1


def mv(fmt: str, raw: torch.Tensor, ids: torch.Tensor, x: torch.Tensor, n_out: int, n_in: int,
       adressen: Optional[torch.Tensor] = None) -> torch.Tensor:
    """raw (n_exp, bytes per expert) on the GPU, ids (k,): expert ids.  x (n_in,) is shared by all
    experts, x (k, n_in) is each expert's own input.  adressen (n_exp,) int64 on the GPU: where each
    expert's bytes lie (then raw is not read).  -> (k, n_out) float32 (reference cudakern.py:756-774)."""
    if fmt not in FORMATE:
        raise ValueError(f"cudakern.mv: format {fmt}")
    geraet = x.device
    ids = ids.to(geraet, torch.int64).contiguous()
    k = ids.numel()
    y = torch.empty(k, n_out, dtype=torch.float32, device=geraet)
    if adressen is None:
        quelle, per = raw, raw.shape[1] if raw.dim() == 2 else raw.numel()
    else:
        quelle, per = adressen.to(geraet, torch.int64).contiguous(), -1
    x_group = 1 if x.dim() == 2 else k
    L = _native.lib()
    w = _werte(x, n_in, bf16=True)
    if w is not None:   # the launch rounds x to bf16 and quantises it (no quantisation launch)
        _starten("mv_experts", L.nmq_mv_experts_x, TYPE_ID[fmt], quelle.data_ptr(), None, ids.data_ptr(), k, per,
                 w[0].data_ptr(), w[1], None, x_group, y.data_ptr(), n_out, n_in, _native.stream_ptr(geraet))
        return y
    e = eingang_bf16(x)
    _starten("mv_experts", L.nmq_mv_experts, TYPE_ID[fmt], quelle.data_ptr(), ids.data_ptr(), k, per,
             e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), x_group, y.data_ptr(),
             n_out, n_in, _native.stream_ptr(geraet))
    return y


def mm(fmt: str, raw: torch.Tensor, x: torch.Tensor, n_out: int, n_in: int) -> torch.Tensor:
    """raw: one matrix (n_out rows) in block format on the GPU, x (M, n_in) with
    2 <= M <= mm_bis(device) -> (M, n_out) float32; every weight is read once per SPALTEN rows
    (reference cudakern.py:777-790)."""
    if fmt not in FORMATE:
        raise ValueError(f"cudakern.mm: format {fmt}")
    geraet = x.device
    M = x.shape[0]
    grenze = mm_bis(geraet)
    if not 2 <= M <= grenze:
        raise ValueError(f"mm: {M} rows (2..{grenze})")
    e = eingang_bf16(x)
    y = torch.empty(M, n_out, dtype=torch.float32, device=geraet)
    L = _native.lib()
    _starten("mv", L.nmq_mv, TYPE_ID[fmt], raw.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(),
             e.xs.data_ptr(), y.data_ptr(), n_out, n_in, M, _native.stream_ptr(geraet))
    return y
