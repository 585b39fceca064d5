"""
Whole matrices streamed from pinned RAM into a ring of VRAM slots: the reference's `Fliessband`
(models/common.py:295-361), used by `PackedLinear` for weights kept in RAM (`hostmem`).

Each matrix is copied whole, on a copy stream of its own (default priority), a few matrices ahead
of its use, so a matrix read more than once (several tokens, prefill) is read from VRAM.  On MI355X
a lone copy from pinned RAM runs at 54 GB/s and a pass over 8 Q4_K 4096x4096 layers through the ring
at 44.6 GB/s; kernels reading RAM directly reach 52 GB/s.  Matrices are numbered in the order they are registered, which is their
order of use in a forward pass; a number not above the previous one starts a new pass.  Ordering is
by events only (no host synchronisation), so the band also runs inside a HIP graph capture:

  - a copy into a slot waits for the last computation that read the slot (`fertig` records it);
  - the computation waits for its matrix's copy (`holen` makes the current stream wait);
  - at the start of a pass the copy stream waits for everything the compute stream has queued, so
    slots from the previous pass are not overwritten while still being read.
"""
from __future__ import annotations

from typing import List, Optional

import torch

PLAETZE = 4  # VRAM slots of the ring (reference schichten.BAND_PLAETZE)


class Fliessband:
    """Ring of `PLAETZE` VRAM slots fed from registered sources (reference common.py:295-361)."""

    PLAETZE = PLAETZE

    def __init__(self, device):
        self.device = torch.device(device)
        self.quellen: List[torch.Tensor] = []    # flat uint8 sources, in order of use
        self._ring: Optional[torch.Tensor] = None
        self._strom: Optional[torch.cuda.Stream] = None
        self._inhalt: List[int] = []             # matrix held (or being copied) per slot, -1: none
        self._gelesen: List[bool] = []           # the slot's "done" event belongs to this pass
        self._ausgegeben: List[int] = []         # matrix handed out by holen() and not yet fertig(), -1: none
        self._fertig: list = []                  # per slot: the last computation that read it
        self._bereit: list = []                  # per slot: its copy has landed
        self._zuletzt = 1 << 62                  # number of the last matrix handed out

    def anmelden(self, quelle: torch.Tensor) -> int:
        """Register a source (any tensor the copy engine can read: pinned RAM or its GPU view); returns
        its number.  Registration order is the order of use."""
        if self._ring is not None:
            raise RuntimeError("Fliessband: sources are registered before the first holen()")
        self.quellen.append(quelle.reshape(-1).view(torch.uint8))
        return len(self.quellen) - 1

    def _anlegen(self) -> None:
        n = len(self.quellen)
        if n == 0:
            raise RuntimeError("Fliessband: no sources registered")
        groesste = max(q.numel() for q in self.quellen)
        self._ring = torch.empty(self.PLAETZE, groesste, dtype=torch.uint8, device=self.device)
        self._strom = torch.cuda.Stream(self.device)
        self._inhalt = [-1] * self.PLAETZE
        self._gelesen = [False] * self.PLAETZE
        self._ausgegeben = [-1] * self.PLAETZE
        self._fertig = [torch.cuda.Event() for _ in range(self.PLAETZE)]
        self._bereit = [torch.cuda.Event() for _ in range(self.PLAETZE)]

    def _laden(self, nr: int) -> None:
        platz = nr % self.PLAETZE
        if self._inhalt[platz] == nr:
            return
        if self._ausgegeben[platz] >= 0:         # its computation may not even be queued yet
            raise RuntimeError(f"Fliessband: matrix {nr} would overwrite matrix {self._ausgegeben[platz]}, "
                               f"which holen() handed out and fertig() has not released")
        if self._gelesen[platz]:                 # its reader in this pass must be done first
            self._strom.wait_event(self._fertig[platz])
        q = self.quellen[nr]
        with torch.cuda.stream(self._strom):
            self._ring[platz, :q.numel()].copy_(q, non_blocking=True)
            self._bereit[platz].record(self._strom)
        self._inhalt[platz] = nr
        self._gelesen[platz] = False

    def holen(self, nr: int) -> torch.Tensor:
        """The bytes of matrix `nr` in VRAM (the current stream waits for their copy); the copies of the
        next PLAETZE - 1 matrices are queued behind it.  Every matrix handed out is released with
        `fertig(nr)` once its computation is queued; a copy that would overwrite a matrix not yet
        released raises RuntimeError (the band's state is unchanged for that slot)."""
        if not 0 <= nr < len(self.quellen):
            raise IndexError(f"Fliessband: matrix {nr} of {len(self.quellen)}")
        if self._ring is None:
            self._anlegen()
        rechnen = torch.cuda.current_stream(self.device)
        if nr <= self._zuletzt:                  # a new pass: nothing queued before may be overwritten early
            offen = [a for a in self._ausgegeben if a >= 0]
            if offen:
                raise RuntimeError(f"Fliessband: a new pass starts at matrix {nr} while matrices {offen} are "
                                   f"handed out and not released by fertig()")
            self._strom.wait_stream(rechnen)
            self._inhalt = [-1] * self.PLAETZE
            self._gelesen = [False] * self.PLAETZE
        for k in range(nr, min(nr + self.PLAETZE, len(self.quellen))):
            self._laden(k)
        self._zuletzt = nr                       # after the copies: a refused holen() can be retried in its pass
        platz = nr % self.PLAETZE
        rechnen.wait_event(self._bereit[platz])
        self._ausgegeben[platz] = nr
        return self._ring[platz, :self.quellen[nr].numel()]

    def fertig(self, nr: int) -> None:
        """The computation on matrix `nr` is queued: its slot may be refilled after it."""
        platz = nr % self.PLAETZE
        self._fertig[platz].record(torch.cuda.current_stream(self.device))
        self._gelesen[platz] = True
        if self._ausgegeben[platz] == nr:
            self._ausgegeben[platz] = -1
