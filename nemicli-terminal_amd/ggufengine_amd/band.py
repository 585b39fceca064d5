"""
Whole matrices streamed from pinned RAM into a ring of VRAM slots (the contract of the reference's
`Fliessband`, models/common.py:295-361), used by `PackedLinear` for weights kept in RAM (`hostmem`).

Contract.  Sources are registered in their order of use in a forward pass and numbered from 0.
`holen(nr)` returns matrix nr's bytes in VRAM and queues the copies of the next matrices (up to PLAETZE
slots ahead) on a copy stream of default priority; `fertig(nr)` says the computation on nr is queued.
A number not above the previous one starts a new pass.  Ordering uses events only (no host waits):

  - a copy into a slot waits for the last computation of this pass that read the slot;
  - the computation on nr waits for nr's copy;
  - a new pass makes the copy stream wait for everything the compute stream queued before, so the
    previous pass's slots are not overwritten while still being read.

A matrix handed out by `holen` stays lent until `fertig`: a copy that would overwrite it raises
RuntimeError instead of racing with a computation that may not be queued yet.

HIP graphs: a capture must cover whole passes (a decode step), as in the reference.  The copies a pass
queues ahead belong to the stream state of that pass, so a pass cannot be split between captures, or
between a capture and eager calls: `holen` raises RuntimeError when a pass started outside the current
capture continues inside it, or the other way round.  A capture that ends inside a pass leaves copies
on the copy stream that were never joined, which the capture's end reports as an error.

Slots are PLAETZE equal views of one allocation whose stride is the largest source rounded up to 256
bytes, so every slot starts aligned for the kernels' 16-byte weight reads.
"""
from __future__ import annotations

from typing import List, Optional

import torch

PLAETZE = 4          # VRAM slots of the ring (the reference's schichten.BAND_PLAETZE)
SLOT_ALIGN = 256     # bytes


class _Slot:
    """One ring position: its bytes and what was last done to it."""

    __slots__ = ("data", "holds", "landed", "freed", "read", "lent")

    def __init__(self, data: torch.Tensor):
        self.data = data
        self.holds = -1                  # matrix copied (or being copied) into it this pass
        self.landed = torch.cuda.Event()     # that copy has finished (copy stream)
        self.freed = torch.cuda.Event()      # its last reader this pass has finished (compute stream)
        self.read = False                # `freed` was recorded this pass
        self.lent = -1                   # matrix handed out by holen() and not yet released

    def forget(self) -> None:
        self.holds, self.read = -1, False


class Fliessband:
    """Ring of PLAETZE VRAM slots fed from registered sources on a copy stream."""

    PLAETZE = PLAETZE

    def __init__(self, device):
        self.device = torch.device(device)
        self.quellen: List[torch.Tensor] = []
        self._slots: List[_Slot] = []
        self._copy: Optional[torch.cuda.Stream] = None
        self._last = None                # number handed out last (None: no pass started)
        self._pass_captured = False      # the current pass began inside a graph capture

    def anmelden(self, quelle: torch.Tensor) -> int:
        """Register a source (pinned RAM, its GPU view, or device memory); returns its number."""
        if self._slots:
            raise RuntimeError("Fliessband: sources are registered before the first holen()")
        self.quellen.append(quelle.reshape(-1).view(torch.uint8))
        return len(self.quellen) - 1

    # -- internals -------------------------------------------------------------------------------
    def _ring(self) -> List[_Slot]:
        if not self._slots:
            if not self.quellen:
                raise RuntimeError("Fliessband: no sources registered")
            stride = -(-max(q.numel() for q in self.quellen) // SLOT_ALIGN) * SLOT_ALIGN
            block = torch.empty(self.PLAETZE * stride, dtype=torch.uint8, device=self.device)
            self._slots = [_Slot(block[i * stride:(i + 1) * stride]) for i in range(self.PLAETZE)]
            self._copy = torch.cuda.Stream(self.device)
        return self._slots

    def _new_pass(self, compute: torch.cuda.Stream) -> None:
        lent = [s.lent for s in self._slots if s.lent >= 0]
        if lent:
            raise RuntimeError(f"Fliessband: a new pass starts while matrices {lent} are handed out and not "
                               f"released by fertig()")
        self._copy.wait_stream(compute)
        for s in self._slots:
            s.forget()

    def _queue_copy(self, nr: int) -> None:
        slot = self._slots[nr % self.PLAETZE]
        if slot.holds == nr:
            return
        if slot.lent >= 0:
            raise RuntimeError(f"Fliessband: matrix {nr} would overwrite matrix {slot.lent}, which holen() "
                               f"handed out and fertig() has not released")
        if slot.read:
            self._copy.wait_event(slot.freed)
        src = self.quellen[nr]
        with torch.cuda.stream(self._copy):
            slot.data[:src.numel()].copy_(src, non_blocking=True)
            slot.landed.record(self._copy)
        slot.holds, slot.read = nr, False

    # -- API -------------------------------------------------------------------------------------
    def holen(self, nr: int) -> torch.Tensor:
        """Matrix nr's bytes in its VRAM slot; the current stream waits for their copy, and the copies of
        the following matrices are queued behind it."""
        if not 0 <= nr < len(self.quellen):
            raise IndexError(f"Fliessband: matrix {nr} of {len(self.quellen)}")
        slots = self._ring()
        compute = torch.cuda.current_stream(self.device)
        capturing = torch.cuda.is_current_stream_capturing()
        if self._last is None or nr <= self._last:
            self._new_pass(compute)
            self._pass_captured = capturing
        elif capturing != self._pass_captured:
            raise RuntimeError("Fliessband: a pass is split between a graph capture and eager calls; a "
                               "capture must cover whole passes")
        for k in range(nr, min(nr + self.PLAETZE, len(self.quellen))):
            self._queue_copy(k)
        self._last = nr                  # set after the copies: a refused call can be retried
        slot = slots[nr % self.PLAETZE]
        compute.wait_event(slot.landed)
        slot.lent = nr
        return slot.data[:self.quellen[nr].numel()]

    def fertig(self, nr: int) -> None:
        """The computation on matrix nr is queued on the current stream: its slot may be refilled after it."""
        slot = self._slots[nr % self.PLAETZE]
        slot.freed.record(torch.cuda.current_stream(self.device))
        slot.read = True
        if slot.lent == nr:
            slot.lent = -1
