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
    the weighted sum per token in slot order.  Two launches: gate and up in one gathered launch
    reading each token's input through its k slots (x_group = k), the input rounded to bf16 (as
    cudakern.mv does) and quantised inside the launch; down on each slot's own activation
    bf16(silu(gate) * up), also formed and quantised inside its launch, whose last workgroup per
    (token, row block) adds the slots' results in slot order (nmq_moe_down).

Every expert product runs on libnmq's HIP kernels; without the library the constructor raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import _native, cudakern, hostmem, packed
from .gguf_types import GGML_TYPES, GGUFError, TYPE_ID
from .mmvq import WERTE_BIS, Eingang, _starten, _werte, eingang_bf16

# (token, slot) pairs per expert (on average) from which Experten sorts them by expert and multiplies every
# used expert's rows at once (one host read per layer, so not inside a graph capture)
SORTIERT_AB = 4


class PackedExperts:
    """All experts of one tensor (n_exp, n_out, n_in) in their GGUF block bytes, multiplied on the device
    by the expert-id-gathered kernel (the reference's PackedExperts, models/common.py:434-480).  The ids
    stay on the device, so a captured graph follows new routings.  `adressen` (int64 (n_exp,) on the
    device), when set, gives each expert's address instead of the `per_expert` stride of `raw`."""

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
        self.im_ram = hostmem.abgebildet(raw)          # the bytes sit in pinned host memory
        self.adressen: Optional[torch.Tensor] = None

    @classmethod
    def aus_quantlinear(cls, experten, dtype: torch.dtype = torch.bfloat16) -> "PackedExperts":
        """One expert tensor from a list of qlinear.QuantLinear layers of one format and shape (no bias).
        Their bytes are used in place when they lie back to back in one allocation (the reference's
        loader cuts experts out of one tensor that way), else copied together once."""
        if not experten:
            raise GGUFError("aus_quantlinear: no experts")
        first = experten[0]
        if any(e.ggml_type != first.ggml_type or (e.n_out, e.n_in) != (first.n_out, first.n_in) or e.b is not None
               for e in experten):
            raise GGUFError("aus_quantlinear: experts differ in format or shape, or carry a bias")
        per, n = first.raw.numel(), len(experten)
        store, off = first.raw.untyped_storage(), first.raw.storage_offset()
        back_to_back = all(e.raw.untyped_storage().data_ptr() == store.data_ptr() and e.raw.is_contiguous()
                           and e.raw.storage_offset() == off + i * per for i, e in enumerate(experten))
        if back_to_back and off + per * n <= store.nbytes():
            whole = torch.empty(0, dtype=torch.uint8, device=first.raw.device).set_(store, off, (per * n,), (1,))
        else:
            whole = torch.cat([e.raw.reshape(-1) for e in experten])
        return cls(whole, first.ggml_type, len(experten), first.n_out, first.n_in, dtype)

    def __len__(self) -> int:
        return self.n_exp

    def _quelle(self, dev):
        """(tensor, per_expert) for the kernels: the stride of raw, or the address table (per = -1)."""
        if self.adressen is None:
            return self.raw, self.raw.shape[1]
        return self.adressen.to(dev, torch.int64).contiguous(), -1

    def matvec(self, ids: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """ids (k,) on one input x (n_in,) -> float32 (k, n_out), row j from expert ids[j]."""
        return cudakern.mv(self.name, self.raw, ids, x.reshape(-1), self.n_out, self.n_in, self.adressen)

    def matvec_je(self, ids: torch.Tensor, a: torch.Tensor) -> torch.Tensor:
        """ids (k,) with one input row each, a (k, n_in) -> float32 (k, n_out): expert ids[j] on a[j]."""
        return cudakern.mv(self.name, self.raw, ids, a.reshape(ids.numel(), -1), self.n_out, self.n_in,
                           self.adressen)

    def weights(self, ids: torch.Tensor) -> torch.Tensor:
        """The experts ids (k,) unpacked on the device: (k, n_out, n_in) in the compute dtype (exact values
        rounded to bf16 first)."""
        from .packed import unpack
        ids = ids.to(self.raw.device, torch.int64).reshape(-1)
        blocks = self.raw.index_select(0, ids).reshape(-1)
        w = unpack(self.ggml_type, blocks, ids.numel() * self.n_out, self.n_in)
        return w.view(-1, self.n_out, self.n_in).to(self.dtype)

    def __getitem__(self, e: int) -> "_OneExpert":
        if not 0 <= e < self.n_exp:
            raise IndexError(e)
        return _OneExpert(self, e)

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


class _OneExpert:
    """Expert e of a PackedExperts as a linear layer: x (..., n_in) -> (..., n_out) in the compute dtype,
    through the gathered kernel for one row and the unpacked weights for more."""

    def __init__(self, owner: PackedExperts, e: int):
        self.owner, self.e = owner, e
        self.n_out, self.n_in = owner.n_out, owner.n_in

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.reshape(-1, self.n_in)
        ids = torch.full((rows.shape[0],), self.e, dtype=torch.int64, device=self.owner.geraet)
        if rows.shape[0] == 1:
            y = self.owner.matvec_je(ids, rows).to(self.owner.dtype)
        else:
            w = self.owner.weights(ids[:1])[0]
            y = rows.to(w.dtype) @ w.t()
        return y.reshape(*x.shape[:-1], self.n_out)


class ExpertenLager:
    """The most chosen experts of one MoE layer, whose tensors live in pinned host memory, held in `plaetze`
    VRAM slots (the reference's ExpertenLager, models/moe.py:133-192).

    State: `zaehler` (device, fp32) counts how often each expert was chosen, decaying by half at every
    re-sort; `_slot` (host, int64) maps each expert to its slot or -1.  Each part (gate, up, down ...) owns
    a slot array `cache[i]` (plaetze x bytes per expert) and an address table `adressen` (device, int64,
    one entry per expert: its slot or its host bytes) that the gathered kernels read, so captured graphs
    stay valid while experts move.  Counting (`zaehlen`) is graph-safe; re-sorting (`umsortieren`) copies
    between steps, never inside a capture."""

    def __init__(self, teile, plaetze: int, device):
        self.teile = list(teile)
        n = self.teile[0].n_exp
        self.n_exp = n
        self.plaetze = max(0, min(int(plaetze), n))
        self.device = torch.device(device)
        self.zaehler = torch.zeros(n, dtype=torch.float32, device=self.device)
        self._eins = torch.ones(0, dtype=torch.float32, device=self.device)
        self._slot = torch.full((n,), -1, dtype=torch.int64)
        first = torch.arange(self.plaetze, dtype=torch.int64)
        self._slot[first] = first                       # experts 0 .. plaetze-1 start in the slots
        self.cache = [torch.empty(self.plaetze, t.raw.shape[1], dtype=torch.uint8, device=self.device)
                      for t in self.teile]
        for t in self.teile:
            t.adressen = torch.empty(n, dtype=torch.int64, device=self.device)
        self._einlagern(first, first)
        self.verankern()

    @property
    def belegt(self) -> list:
        """Expert held by each slot."""
        held = torch.nonzero(self._slot >= 0).flatten()
        out = [-1] * self.plaetze
        for e, s in zip(held.tolist(), self._slot[held].tolist()):
            out[s] = e
        return out

    def _einlagern(self, slots: torch.Tensor, experten: torch.Tensor) -> None:
        """cache[slot] <- the expert's bytes, for every part, one gather + scatter each."""
        if slots.numel() == 0:
            return
        s = slots.to(self.device)
        for t, c in zip(self.teile, self.cache):
            c.index_copy_(0, s, t.raw.index_select(0, experten.to(t.raw.device)).to(self.device, non_blocking=True))

    def verankern(self) -> None:
        """Rewrite every part's address table from the current slot map (also after the slots were
        re-filled from elsewhere)."""
        held = self._slot >= 0
        for t, c in zip(self.teile, self.cache):
            per = t.raw.shape[1]
            host = t.raw.data_ptr() + torch.arange(self.n_exp, dtype=torch.int64) * per
            if self.plaetze:
                host = torch.where(held, c.data_ptr() + self._slot.clamp(min=0) * per, host)
            t.adressen.copy_(host)

    def zaehlen(self, ids: torch.Tensor) -> None:
        """Add one to the count of every chosen expert (ids of any shape, on the device; graph-safe)."""
        flat = ids.reshape(-1).to(self.device, torch.int64)
        if self._eins.numel() < flat.numel():
            self._eins = torch.ones(flat.numel(), dtype=torch.float32, device=self.device)
        self.zaehler.scatter_add_(0, flat, self._eins[:flat.numel()])

    def treffer(self) -> float:
        """Fraction of the (decayed) counted choices that fall on experts in the slots."""
        c = self.zaehler.cpu()
        total = float(c.sum())
        if not self.plaetze or total == 0.0:
            return 0.0
        return float(c[self._slot >= 0].sum()) / total

    def umsortieren(self) -> int:
        """Move the `plaetze` most counted experts into the slots (each evicted expert's slot goes to one
        newcomer); halve the counts.  Returns the number of experts copied in."""
        if not self.plaetze:
            return 0
        want = torch.topk(self.zaehler.cpu(), self.plaetze).indices
        wanted = torch.zeros(self.n_exp, dtype=torch.bool)
        wanted[want] = True
        resident = self._slot >= 0
        leaving = torch.nonzero(resident & ~wanted).flatten()
        coming = want[~resident[want]]
        if coming.numel():
            slots = self._slot[leaving]
            self._slot[leaving] = -1
            self._slot[coming] = slots
            self._einlagern(slots, coming)
            self.verankern()
        self.zaehler.mul_(0.5)
        return int(coming.numel())


def auswahl(logits: torch.Tensor, k: int, normieren: bool = True, scale: float = 1.0, sigmoid: bool = False,
            wahl_bias: Optional[torch.Tensor] = None, n_group: int = 1, group_used: int = 1,
            nach_auswahl: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Router of a MoE layer (reference baukasten.py:156-190): logits (L, n_exp) -> (ids (L, k) int64,
    weights (L, k) float32).
    - nach_auswahl: the k largest logits, their softmax as the weights (softmax after the selection).
    - otherwise p = softmax(logits) (or sigmoid(logits) with `sigmoid`); the choice is made on
      p + wahl_bias (a per-expert selection correction that the weights do not see); with n_group > 1 the
      experts form n_group equal groups, and only the group_used groups with the best score (the group's
      largest choice value; with sigmoid the sum of its two largest) stay eligible.  The weights are p at
      the chosen experts, divided by their sum when `normieren`, then times `scale`."""
    x = logits.float()
    if nach_auswahl:
        top, idx = x.topk(k, dim=-1)
        return idx, torch.softmax(top, dim=-1)
    p = torch.sigmoid(x) if sigmoid else torch.softmax(x, dim=-1)
    wahl = p if wahl_bias is None else p + wahl_bias.to(p.device, torch.float32)
    if n_group > 1:
        L_, n = wahl.shape
        je = n // n_group
        gruppen = wahl.view(L_, n_group, je)
        wert = gruppen.topk(min(2, je), dim=-1)[0].sum(-1) if sigmoid else gruppen.amax(-1)
        offen = torch.zeros(L_, n_group, dtype=torch.bool, device=wahl.device)
        offen.scatter_(1, wert.topk(group_used, dim=-1)[1], True)
        wahl = wahl.masked_fill(~offen.repeat_interleave(je, dim=1), float("-inf"))
    idx = wahl.topk(k, dim=-1)[1]
    w = p.gather(-1, idx)
    if normieren:
        w = w / (w.sum(-1, keepdim=True) + 1e-20)
    return idx, w * scale


class Experten:
    """Expert MLP of a MoE layer in block format (reference moe.py:205-321): gate and up as two tensors or
    fused as one [gate | up] tensor of 2*FF rows per expert, or up alone (act(up), no gate); down; an
    optional bias per expert for each part ({"gate", "up", "gate_up", "down"}: (n_exp, width) fp32); the
    activation `akt` ("silu", "gelu" for the tanh form, or a callable on fp32 tensors) or `glu(gate, up)`
    combining both projections.  The silu-gated form without biases runs as nmq_moe_layer (two launches);
    every other form through the gathered launches with the bias, activation and combine in torch."""

    def __init__(self, gate: Optional[PackedExperts], up: Optional[PackedExperts], down: PackedExperts,
                 gate_up: Optional[PackedExperts] = None, bias: Optional[dict] = None, akt="silu", glu=None):
        if gate_up is not None:
            if gate is not None or up is not None:
                raise GGUFError("Experten: either gate_up or gate/up")
            ff = gate_up.n_out // 2
            teile, n_in = [gate_up], gate_up.n_in
            if gate_up.n_out != 2 * ff or ff != down.n_in:
                raise GGUFError("Experten: the fused [gate | up] tensor needs 2 x the down projection's inputs")
        else:
            if up is None:
                raise GGUFError("Experten: up (or gate_up) is required")
            teile = [t for t in (gate, up) if t is not None]
            ff, n_in = up.n_out, up.n_in
            if any(t.n_out != ff or t.n_in != n_in for t in teile) or ff != down.n_in:
                raise GGUFError("Experten: gate/up/down shapes do not fit together")
        if down.n_out != n_in or any(t.n_exp != down.n_exp for t in teile):
            raise GGUFError("Experten: gate/up/down shapes do not fit together")
        self.gate, self.up, self.down, self.gate_up = gate, up, down, gate_up
        self.n_exp, self.ff = down.n_exp, ff
        breite = {"gate": ff, "up": ff, "gate_up": 2 * ff, "down": down.n_out}
        self.bias = {}
        for name, b in (bias or {}).items():
            if name not in breite or tuple(b.shape) != (self.n_exp, breite[name]):
                raise GGUFError(f"Experten: bias {name!r} of shape {tuple(b.shape)}")
            self.bias[name] = b.float()
        if isinstance(akt, str) and akt not in ("silu", "gelu"):
            raise ValueError(f"Experten: activation {akt!r} (silu, gelu or a callable)")
        self.akt, self.glu = akt, glu
        self._work: dict = {}
        self._matrizen: dict = {}

    def _gate_up_quellen(self, dev):
        """(format, gate pointer, up pointer, per_expert) for the fused launches, or None where they do not
        apply (no gate, or a fused [gate | up] tensor read through an address table)."""
        if self.gate_up is not None:
            if self.gate_up.adressen is not None:
                return None
            gu = self.gate_up
            raw, per = gu._quelle(dev)
            _, bs, ts = GGML_TYPES[gu.ggml_type]
            return gu.name, raw.data_ptr(), raw.data_ptr() + self.ff * (gu.n_in // bs) * ts, per
        if self.gate is None or not self._fused():
            return None
        (wa, per), (wb, _) = self.gate._quelle(dev), self.up._quelle(dev)
        return self.gate.name, wa.data_ptr(), wb.data_ptr(), per

    @staticmethod
    def _gu(h_gate: torch.Tensor, h_up: torch.Tensor) -> torch.Tensor:
        return F.silu(h_gate) * h_up

    def _fused(self) -> bool:
        g, u = self.gate, self.up
        return (g.ggml_type == u.ggml_type and g.raw.shape == u.raw.shape and (g.adressen is None) == (u.adressen is None))

    def __call__(self, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """x (L, E) -> (L, E) float32; idx (L, k) expert ids, w (L, k) their weights (reference
        models/moe.py:264-277).  The silu-gated form without biases is one call of nmq_moe_layer, two
        launches: gate|up with the activation quantised in the same workgroups, then the down launch with the
        weighted combine on that input; for more tokens the gathered gate|up launch into fp32, then the down
        launch forming the activation in its staging.  (Rows longer than WERTE_BIS values, or a gate and up
        of different layout: the input quantisations as launches of their own.)  Other forms: _allgemein."""
        if idx.numel() >= SORTIERT_AB * self.n_exp:
            return self._sortiert(x, idx, w)
        if self.bias or self.glu is not None or self.akt != "silu" or (self.gate is None and self.gate_up is None):
            return self._allgemein(x, idx, w)
        L_, E = x.shape
        k = idx.shape[1]
        dev = x.device
        q = self._gate_up_quellen(dev)
        FF = self.ff
        if q is None or max(E, FF) > WERTE_BIS or x.dtype != torch.float32 or FF % 32:
            return self._aufgeteilt(x, idx, w)
        name, wa, wb, per = q
        flat = idx.reshape(-1).to(dev, torch.int64).contiguous()
        wd, perd = self.down._quelle(dev)
        out = torch.empty(L_, E, dtype=torch.float32, device=dev)
        wf = w.to(dev, torch.float32).contiguous()
        work = self._arbeitsplatz(L_, k, E, FF, dev)
        _starten("moe_layer", _native.lib().nmq_moe_layer, TYPE_ID[name], wa, wb, per, TYPE_ID[self.down.name],
                 wd.data_ptr(), perd, flat.data_ptr(), wf.data_ptr(), L_, k, x.contiguous().data_ptr(),
                 _native.X_F32_BF16, out.data_ptr(), E, FF, work.data_ptr(), work.numel(), _native.stream_ptr(dev))
        return out

    def _aktiviert(self, g: Optional[torch.Tensor], u: torch.Tensor) -> torch.Tensor:
        """glu(gate, up), act(gate) * up, or act(up) without a gate (reference moe.py:252-255)."""
        if self.glu is not None:
            return self.glu(g, u)
        akt = self.akt
        f = F.silu if akt == "silu" else ((lambda t: F.gelu(t, approximate="tanh")) if akt == "gelu" else akt)
        return f(u) if g is None else f(g) * u

    def _matrix(self, teil: str, e: int) -> packed.PackedLinear:
        """Expert e of part `teil` as a matrix (its block bytes in place), kept for later calls."""
        key = (teil, e)
        m = self._matrizen.get(key)
        if m is None:
            t = getattr(self, teil)
            m = packed.PackedLinear(t.raw[e], t.ggml_type, t.n_out, t.n_in, dtype=torch.float32)
            self._matrizen[key] = m
        return m

    def _sortiert(self, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """Many tokens (reference moe.py:290-321): the (token, slot) pairs sorted by expert, every used expert's
        rows multiplied at once as a matrix (PackedLinear's dispatch by row count: the int8 mat-vec kernels,
        the matrix cores, or unpacked weights), one host read of the per-expert counts, the results put back
        in (token, slot) order and summed there in a fixed order."""
        L_, E = x.shape
        k = idx.shape[1]
        flat = idx.reshape(-1).to(x.device, torch.int64)
        folge = flat.sort(stable=True)[1]
        xs = x.to(torch.bfloat16).float()[folge // k]   # the gathered launches' bf16 input
        anzahl = torch.bincount(flat, minlength=self.n_exp).tolist()
        ys = torch.empty(L_ * k, E, dtype=torch.float32, device=x.device)
        a = 0
        for e, c in enumerate(anzahl):
            if not c:
                continue
            sl = slice(a, a + c)
            a += c
            xe = xs[sl]

            def mit_bias(name, y):
                b = self.bias.get(name)
                return y if b is None else y + b[e].to(y.device)
            if self.gate_up is not None:
                gu = mit_bias("gate_up", self._matrix("gate_up", e)(xe))
                g, u = gu[:, :self.ff], gu[:, self.ff:]
            else:
                g = mit_bias("gate", self._matrix("gate", e)(xe)) if self.gate is not None else None
                u = mit_bias("up", self._matrix("up", e)(xe))
            act = self._aktiviert(g, u).to(torch.bfloat16).float()
            ys[sl] = mit_bias("down", self._matrix("down", e)(act))
        back = torch.empty_like(ys)
        back[folge] = ys
        return (back.view(L_, k, E) * w.float().to(x.device).unsqueeze(-1)).sum(1)

    def _allgemein(self, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """Every form of the layer: the gathered launches on each token's bf16 input (gate and up, or the
        fused [gate | up] tensor, or up alone), each part's bias per expert added, the activation in torch,
        the gathered down launch on each slot's activation (rounded to bf16 in the launch) plus its bias, and
        the weighted sum over the slots (reference moe.py:264-277)."""
        L_, E = x.shape
        e = eingang_bf16(x)
        flat = idx.reshape(-1).to(x.device, torch.int64).contiguous()

        def mit_bias(name, y):
            b = self.bias.get(name)
            return y if b is None else y + b.to(y.device).index_select(0, flat)
        if self.gate_up is not None:
            gu = mit_bias("gate_up", self.gate_up.matvec_tokens(idx, e))
            g, u = gu[:, :self.ff], gu[:, self.ff:]
        else:
            g = mit_bias("gate", self.gate.matvec_tokens(idx, e)) if self.gate is not None else None
            u = mit_bias("up", self.up.matvec_tokens(idx, e))
        y = mit_bias("down", self.down.matvec_je(flat, self._aktiviert(g, u).contiguous()))
        return (y.view(L_, -1, E) * w.float().unsqueeze(-1)).sum(1)

    def _arbeitsplatz(self, L_: int, k: int, E: int, FF: int, dev) -> torch.Tensor:
        """nmq_moe_layer's workspace for L_ tokens of k slots: kept per layer and device, grown when needed."""
        need = ctypes.c_int64(0)
        _native.check(_native.lib().nmq_moe_layer_work_bytes(L_, k, E, FF, ctypes.byref(need)))
        have = self._work.get(dev)
        if have is None or have.numel() < need.value:
            have = torch.zeros(max(need.value, 256), dtype=torch.uint8, device=dev)
            self._work[dev] = have
        return have

    def _aufgeteilt(self, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """The silu-gated layer with the inputs quantised by launches of their own (five launches when gate
        and up share a layout or come fused, else _allgemein)."""
        L_, E = x.shape
        k = idx.shape[1]
        dev = x.device
        q = self._gate_up_quellen(dev)
        if q is None:
            return self._allgemein(x, idx, w)
        name, wa, wb, per = q
        L = _native.lib()
        st = _native.stream_ptr(dev)
        n = L_ * k
        FF = self.ff
        e = eingang_bf16(x)
        flat = idx.reshape(-1).to(dev, torch.int64).contiguous()
        gu = torch.empty(2 * n, FF, dtype=torch.float32, device=dev)
        _starten("mv_experts2", L.nmq_mv_experts2, TYPE_ID[name], wa, wb, flat.data_ptr(), n, per, e.xq.data_ptr(),
                 e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(), k, gu.data_ptr(), FF, E, st)
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
