"""
The reference's expert path around the gathered mat-vec, on this library's kernels:

  - `PackedExperts` (models/common.py:434-480): an expert tensor (n_exp, n_out, n_in) in GGUF block
    format; `matvec(ids, x)` applies the experts `ids` to one shared input, `matvec_je(ids, a)` each
    to its own input, both through `cudakern.mv` (the expert-id-gathered kernel, ids read on the GPU).
  - `auswahl(logits, k)`: the softmax router of `_Schicht._auswahl` (models/baukasten.py:171-190)
    without the grouped and sigmoid variants: p = softmax(logits), the k largest, their p optionally
    renormalised to sum 1 (+1e-20), times the weights scale.
  - `ExpertenLager` (models/moe.py:133-192): VRAM slots for the most used experts of a layer kept in
    pinned RAM (`hostmem`), read by the kernels through per-part address tables.
  - `Experten` (models/moe.py:252-321): y = sum_j w_j * down_j(silu(gate_j(x)) * up_j(x)).  Every
    (token, slot) pair on its own, in (token, slot) order (the reference's one-token and graph paths),
    the weighted sum per token in slot order.  Three launches: gate and up in one gathered launch
    reading each token's input through its k slots (x_group = k), the input rounded to bf16 (as
    cudakern.mv does) and quantised inside the launch; down on each slot's own activation
    bf16(silu(gate) * up), also formed and quantised inside its launch; the combine.

Every expert product runs on libnmq's HIP kernels; without the library the constructor raises.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import _native, cudakern
from .gguf_types import GGML_TYPES, GGUFError, TYPE_ID
from .mmvq import WERTE_BIS, Eingang, _starten, _werte, eingang_bf16


class PackedExperts:
    """Expert tensor (n_exp, n_out, n_in) kept in its GGUF block format (reference common.py:434-480)."""

    def __init__(self, raw: torch.Tensor, ggml_type: int, n_exp: int, n_out: int, n_in: int,
                 dtype: torch.dtype = torch.bfloat16):
        if ggml_type not in GGML_TYPES:
            raise GGUFError(f"PackedExperts: type {ggml_type} is not one of this library's formats")
        name, bs, ts = GGML_TYPES[ggml_type]
        if n_in % bs or raw.numel() != n_exp * n_out * (n_in // bs) * ts:
            raise GGUFError(f"PackedExperts: {raw.numel()} bytes do not hold {n_exp}x{n_out}x{n_in} {name}")
        if not raw.is_cuda or not cudakern.verfuegbar(raw.device, name, n_in):
            raise RuntimeError("PackedExperts: libnmq.so is not loaded or the device is not gfx950")
        self.raw = raw.view(n_exp, -1)
        self.geraet = raw.device
        self.ggml_type = ggml_type
        self.n_exp, self.n_out, self.n_in = n_exp, n_out, n_in
        self.dtype = dtype
        self.name = name
        self.kernel = True
        self.adressen: Optional[torch.Tensor] = None   # optional address table (n_exp,) int64 on the GPU

    def __len__(self) -> int:
        return self.n_exp

    def matvec(self, ids: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """The experts `ids` (k,) applied to one shared input x (n_in,) -> (k, n_out) float32."""
        return cudakern.mv(self.name, self.raw, ids, x.reshape(-1), self.n_out, self.n_in, self.adressen)

    def matvec_je(self, ids: torch.Tensor, a: torch.Tensor) -> torch.Tensor:
        """Expert ids[j] applied to its own input a[j]: (k, n_in) -> (k, n_out) float32."""
        return cudakern.mv(self.name, self.raw, ids, a.reshape(ids.numel(), -1), self.n_out, self.n_in,
                           self.adressen)

    def _quelle(self, dev):
        if self.adressen is None:
            return self.raw, self.raw.shape[1]
        return self.adressen.to(dev, torch.int64).contiguous(), -1

    def matvec_tokens(self, ids: torch.Tensor, x) -> torch.Tensor:
        """ids (L, k), x (L, n_in) or its Eingang: expert ids[t, j] applied to token t's input ->
        (L*k, n_out) float32, rows in (token, slot) order (each token's input read by its k slots).  A
        tensor x is rounded to bf16 first, as cudakern.mv does (in the launch itself for rows of up to
        WERTE_BIS values)."""
        L_, k = ids.shape
        dev = x.xq.device if isinstance(x, Eingang) else x.device
        flat = ids.reshape(-1).to(dev, torch.int64).contiguous()
        y = torch.empty(L_ * k, self.n_out, dtype=torch.float32, device=dev)
        quelle, per = self._quelle(dev)
        L = _native.lib()
        if not isinstance(x, Eingang):
            if x.numel() != L_ * self.n_in:
                raise ValueError(f"matvec_tokens: input of {x.numel()} values for {L_} tokens of {self.n_in}")
            w = _werte(x.reshape(L_, self.n_in), self.n_in, bf16=True)
            if w is not None:
                _starten("mv_experts", L.nmq_mv_experts_x, TYPE_ID[self.name], quelle.data_ptr(), None,
                         flat.data_ptr(), L_ * k, per, w[0].data_ptr(), w[1], None, k, y.data_ptr(), self.n_out,
                         self.n_in, _native.stream_ptr(dev))
                return y
        e = x if isinstance(x, Eingang) else eingang_bf16(x.reshape(L_, self.n_in))
        if e.n != L_ * self.n_in:
            raise ValueError(f"matvec_tokens: input of {e.n} values for {L_} tokens of {self.n_in}")
        _starten("mv_experts", L.nmq_mv_experts, TYPE_ID[self.name], quelle.data_ptr(), flat.data_ptr(),
                 L_ * k, per, e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), k, y.data_ptr(),
                 self.n_out, self.n_in, _native.stream_ptr(dev))
        return y


class ExpertenLager:
    """VRAM slots for the most used experts of one layer whose tensors live in pinned RAM (reference
    models/moe.py:133-192; the RAM side from `hostmem.empty` / `hostmem.abbilden`).

    Every part (gate, up, down ...) gets an address table on the GPU with one entry per expert: its
    slot in VRAM or its bytes in RAM.  The gathered kernels read through the table, so a HIP graph
    keeps working when experts move.  `zaehlen(ids)` counts on the GPU how often each expert is
    chosen (also inside a graph); `umsortieren()` (between steps, never inside a graph) moves the
    most used ones into the slots, after which the counts fade by half."""

    def __init__(self, teile, plaetze: int, device):
        self.teile = list(teile)
        self.n_exp = self.teile[0].n_exp
        self.plaetze = min(int(plaetze), self.n_exp)
        self.device = torch.device(device)
        self.zaehler = torch.zeros(self.n_exp, dtype=torch.float32, device=self.device)
        self.belegt = list(range(self.plaetze))           # expert held by each slot
        self.cache = [torch.empty(self.plaetze, t.raw.shape[1], dtype=torch.uint8, device=self.device)
                      for t in self.teile]
        for c, t in zip(self.cache, self.teile):
            c.copy_(t.raw[:self.plaetze], non_blocking=True)
            t.adressen = torch.empty(self.n_exp, dtype=torch.int64, device=self.device)
        self.verankern()

    def _tabelle(self, t: PackedExperts, c: torch.Tensor) -> torch.Tensor:
        per = t.raw.shape[1]
        table = torch.arange(self.n_exp, dtype=torch.int64) * per + t.raw.data_ptr()
        if self.plaetze:
            table[torch.tensor(self.belegt)] = torch.arange(self.plaetze, dtype=torch.int64) * per + c.data_ptr()
        return table

    def verankern(self) -> None:
        """Write the address tables from the current slots (again after the slots moved)."""
        for t, c in zip(self.teile, self.cache):
            t.adressen.copy_(self._tabelle(t, c))

    def zaehlen(self, ids: torch.Tensor) -> None:
        """Count the chosen experts (any shape, on the GPU)."""
        ids = ids.reshape(-1)
        self.zaehler.index_add_(0, ids, torch.ones(ids.numel(), dtype=torch.float32, device=ids.device))

    def treffer(self) -> float:
        """Share of the counted choices that the slots hold now."""
        total = float(self.zaehler.sum())
        return float(self.zaehler[self.belegt].sum()) / total if total and self.plaetze else 0.0

    def umsortieren(self) -> int:
        """The most used experts into the slots; returns how many moved in."""
        if not self.plaetze:
            return 0
        top = self.zaehler.topk(self.plaetze).indices.tolist()
        held = set(self.belegt)
        wanted = set(top)
        free = [p for p, e in enumerate(self.belegt) if e not in wanted]
        incoming = [e for e in top if e not in held]
        for p, e in zip(free, incoming):
            for t, c in zip(self.teile, self.cache):
                c[p].copy_(t.raw[e], non_blocking=True)
            self.belegt[p] = e
        if incoming:
            self.verankern()
        self.zaehler.mul_(0.5)
        return len(incoming)


def auswahl(logits: torch.Tensor, k: int, normieren: bool = True, scale: float = 1.0
            ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax router (reference baukasten.py:171-190, softmax gating, no groups):
    logits (L, n_exp) -> (ids (L, k) int64, weights (L, k) float32)."""
    p = torch.softmax(logits.float(), dim=-1)
    idx = p.topk(k, dim=-1)[1]
    w = p.gather(-1, idx)
    if normieren:
        w = w / (w.sum(-1, keepdim=True) + 1e-20)
    return idx, w * scale


class Experten:
    """Expert MLP of a MoE layer, gate/up/down in block format (reference moe.py:252-321, silu gate)."""

    def __init__(self, gate: PackedExperts, up: PackedExperts, down: PackedExperts):
        if not (gate.n_exp == up.n_exp == down.n_exp and gate.n_out == up.n_out == down.n_in
                and gate.n_in == up.n_in == down.n_out):
            raise GGUFError("Experten: gate/up/down shapes do not fit together")
        self.gate, self.up, self.down = gate, up, down
        self.n_exp = gate.n_exp

    @staticmethod
    def _gu(h_gate: torch.Tensor, h_up: torch.Tensor) -> torch.Tensor:
        return F.silu(h_gate) * h_up

    def _fused(self) -> bool:
        g, u = self.gate, self.up
        return (g.ggml_type == u.ggml_type and g.raw.shape == u.raw.shape and (g.adressen is None) == (u.adressen is None))

    def __call__(self, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """x (L, E) -> (L, E) float32; idx (L, k) expert ids, w (L, k) their weights.
        Three launches: gate and up together on every (token, slot), each token's input rounded to bf16
        and quantised in the launch; down on every slot, its input bf16(silu(gate) * up) formed and
        quantised in the launch; the weighted combine.  (Rows longer than WERTE_BIS values, or a gate
        and up of different layout: the input quantisations as launches of their own.)"""
        L_, E = x.shape
        k = idx.shape[1]
        dev = x.device
        if not self._fused() or max(E, self.gate.n_out) > WERTE_BIS or x.dtype != torch.float32:
            return self._aufgeteilt(x, idx, w)
        L = _native.lib()
        st = _native.stream_ptr(dev)
        n = L_ * k
        FF = self.gate.n_out
        xc = x.contiguous()
        flat = idx.reshape(-1).to(dev, torch.int64).contiguous()
        gu = torch.empty(2 * n, FF, dtype=torch.float32, device=dev)
        (wa, per), (wb, _) = self.gate._quelle(dev), self.up._quelle(dev)
        _starten("mv_experts2", L.nmq_mv_experts_x, TYPE_ID[self.gate.name], wa.data_ptr(), wb.data_ptr(),
                 flat.data_ptr(), n, per, xc.data_ptr(), _native.X_F32_BF16, None, k, gu.data_ptr(), FF, E, st)
        y = torch.empty(n, E, dtype=torch.float32, device=dev)
        wd, perd = self.down._quelle(dev)
        _starten("mv_experts", L.nmq_mv_experts_x, TYPE_ID[self.down.name], wd.data_ptr(), None, flat.data_ptr(), n,
                 perd, gu.data_ptr(), _native.X_SILU_MUL_BF16, gu[n:].data_ptr(), 1, y.data_ptr(), E, FF, st)
        out = torch.empty(L_, E, dtype=torch.float32, device=dev)
        wf = w.to(dev, torch.float32).contiguous()
        _starten("moe_combine", L.nmq_moe_combine, y.data_ptr(), wf.data_ptr(), L_, k, E, out.data_ptr(), st)
        return out

    def _aufgeteilt(self, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """The same layer with the inputs quantised by launches of their own (five launches when gate
        and up share a layout, else the per-tensor path)."""
        L_, E = x.shape
        k = idx.shape[1]
        if not self._fused():
            e = eingang_bf16(x)
            g = self.gate.matvec_tokens(idx, e)
            u = self.up.matvec_tokens(idx, e)
            y = self.down.matvec_je(idx.reshape(-1), self._gu(g, u))
            return (y.view(L_, -1, E) * w.float().unsqueeze(-1)).sum(1)
        L = _native.lib()
        dev = x.device
        st = _native.stream_ptr(dev)
        n = L_ * k
        FF = self.gate.n_out
        e = eingang_bf16(x)
        flat = idx.reshape(-1).to(dev, torch.int64).contiguous()
        gu = torch.empty(2 * n, FF, dtype=torch.float32, device=dev)
        (wa, per), (wb, _) = self.gate._quelle(dev), self.up._quelle(dev)
        _starten("mv_experts2", L.nmq_mv_experts2, TYPE_ID[self.gate.name], wa.data_ptr(), wb.data_ptr(),
                 flat.data_ptr(), n, per, e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), k,
                 gu.data_ptr(), FF, E, st)
        a = Eingang(n=n * FF, device=dev)
        _starten("silu_mul_quant", L.nmq_silu_mul_quant, gu.data_ptr(), gu[n:].data_ptr(), a.xq.data_ptr(),
                 a.xq2.data_ptr(), a.xd.data_ptr(), a.xs.data_ptr(), n * FF, st)
        y = torch.empty(n, E, dtype=torch.float32, device=dev)
        wd, perd = self.down._quelle(dev)
        _starten("mv_experts", L.nmq_mv_experts, TYPE_ID[self.down.name], wd.data_ptr(), flat.data_ptr(), n, perd,
                 a.xq.data_ptr(), a.xq2.data_ptr(), a.xd.data_ptr(), a.xs.data_ptr(), 1, y.data_ptr(), E, FF, st)
        out = torch.empty(L_, E, dtype=torch.float32, device=dev)
        wf = w.to(dev, torch.float32).contiguous()
        _starten("moe_combine", L.nmq_moe_combine, y.data_ptr(), wf.data_ptr(), L_, k, E, out.data_ptr(), st)
        return out
