"""
Pinned host memory of exactly the requested size, mapped into the GPU's address space: the contract of
the reference's ggufengine/hostmem.py (`empty`, `abbilden`, `abgebildet`, `flush`, `pending`,
`ram_reicht`, `RAM_REST`), built on HIP for MI355X.

Why not torch's pinned allocator: it rounds every block up to a power of two (300 MB -> 512 MB) and keeps
freed blocks cached.  Weights that stay in RAM (MoE experts that do not fit in VRAM, offloaded layers)
come from `hipHostMalloc(portable | mapped)` instead.  On MI355X the GPU sees such a block at its host
address; `empty()` checks that with `hipHostGetDevicePointer` and refuses the block otherwise, so a
kernel is never handed an address the GPU cannot use.  The gathered mat-vec kernels then read experts
over PCIe through their address tables (cudakern.mv `adressen`).

Lifetime: the block's memory is the buffer of a ctypes array; every CPU tensor and every GPU view made
from it holds that array through torch's buffer reference.  When the last view dies, a finalizer puts the
address on a retirement queue (no lock, no runtime call: finalizers run at arbitrary points).  Retired
blocks are freed only by `flush()`, after a device synchronisation and never during a graph capture, so
a copy or kernel still queued on the device never loses its memory.
"""
from __future__ import annotations

import bisect
import collections
import ctypes
import os
import threading
import types
import weakref

import torch

RAM_REST = 8 << 30        # RAM that must stay free after pinning (else the caller keeps ordinary RAM)

_FLAG_PORTABLE = 0x1      # hipHostMallocPortable: pinned for every device
_FLAG_MAPPED = 0x2        # hipHostMallocMapped: visible to kernels


class _Runtime:
    """The three HIP host-memory calls, bound on first use from the runtime torch loaded."""

    def __init__(self):
        here = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
        lib = ctypes.CDLL(here if os.path.exists(here) else "libamdhip64.so.7")
        vpp = ctypes.POINTER(ctypes.c_void_p)
        self.malloc = lib.hipHostMalloc
        self.malloc.argtypes, self.malloc.restype = [vpp, ctypes.c_size_t, ctypes.c_uint], ctypes.c_int
        self.device_pointer = lib.hipHostGetDevicePointer
        self.device_pointer.argtypes = [vpp, ctypes.c_void_p, ctypes.c_uint]
        self.device_pointer.restype = ctypes.c_int
        self.free = lib.hipHostFree
        self.free.argtypes, self.free.restype = [ctypes.c_void_p], ctypes.c_int


class PinnedHeap:
    """Live pinned blocks (sorted start addresses for lookups) and the queue of retired ones."""

    def __init__(self):
        self._starts: list = []
        self._end: dict = {}
        self._retired: collections.deque = collections.deque()
        self._lock = threading.Lock()
        self._rt = None

    def runtime(self) -> _Runtime:
        if self._rt is None:
            self._rt = _Runtime()
        return self._rt

    def allocate(self, n_bytes: int, device) -> torch.Tensor:
        self.release()
        if not ram_reicht(n_bytes):
            raise RuntimeError(f"pinning {n_bytes} bytes would leave less than {RAM_REST >> 30} GB of RAM free")
        torch.zeros(1, device=torch.device(device))        # makes the device's context current
        rt = self.runtime()
        size = max(1, int(n_bytes))
        host = ctypes.c_void_p()
        err = rt.malloc(ctypes.byref(host), size, _FLAG_PORTABLE | _FLAG_MAPPED)
        if err or not host.value:
            raise RuntimeError(f"hipHostMalloc({n_bytes}): HIP error {err}")
        seen = ctypes.c_void_p()
        err = rt.device_pointer(ctypes.byref(seen), host, 0)
        if err or seen.value != host.value:
            rt.free(host)
            raise RuntimeError(f"the GPU does not see pinned RAM at its host address (error {err}, "
                               f"{seen.value!r} against {host.value:#x})")
        start = host.value
        with self._lock:
            bisect.insort(self._starts, start)
            self._end[start] = start + size
        buf = (ctypes.c_ubyte * int(n_bytes)).from_address(start) if n_bytes else (ctypes.c_ubyte * 1).from_address(start)
        weakref.finalize(buf, self._retired.append, start)
        t = torch.frombuffer(buf, dtype=torch.uint8)
        return t[:0] if not n_bytes else t

    def owns(self, addr: int) -> bool:
        with self._lock:
            i = bisect.bisect_right(self._starts, addr) - 1
            return i >= 0 and addr < self._end[self._starts[i]]

    def release(self) -> None:
        if not self._retired or torch.cuda.is_current_stream_capturing():
            return
        torch.cuda.synchronize()
        rt = self.runtime()
        while True:
            try:
                start = self._retired.popleft()
            except IndexError:
                break
            with self._lock:
                i = bisect.bisect_left(self._starts, start)
                if i < len(self._starts) and self._starts[i] == start:
                    del self._starts[i]
                self._end.pop(start, None)
            rt.free(ctypes.c_void_p(start))

    def waiting(self) -> int:
        return len(self._retired)


_heap = PinnedHeap()


def ram_reicht(n_bytes: int) -> bool:
    """True when RAM_REST would stay free after pinning n_bytes (True when psutil is missing)."""
    try:
        import psutil
    except ImportError:
        return True
    return psutil.virtual_memory().available - int(n_bytes) >= RAM_REST


def empty(n_bytes: int, device) -> torch.Tensor:
    """uint8 CPU tensor of exactly n_bytes in pinned RAM that the GPU sees at the same address.
    RuntimeError when the runtime cannot pin that much, when less than RAM_REST would stay free, or
    when the GPU would see the block elsewhere."""
    return _heap.allocate(n_bytes, device)


def abbilden(host: torch.Tensor, device) -> torch.Tensor:
    """The GPU tensor at the address of a block from `empty()` (or a part of one): kernels, copies and
    graphs read it over PCIe; nothing is held in VRAM.  The view keeps the block alive."""
    if not abgebildet(host):
        raise ValueError("only memory from hostmem.empty() can be mapped")
    flat = host.reshape(-1)
    holder = types.SimpleNamespace(host=flat, __cuda_array_interface__={
        "shape": (flat.numel(),), "typestr": "|u1", "strides": None, "data": (flat.data_ptr(), False),
        "version": 3})
    gpu = torch.as_tensor(holder, device=torch.device(device))
    if gpu.data_ptr() != flat.data_ptr():
        raise RuntimeError("no unified addressing: the GPU sees the block at another address")
    return gpu


def abgebildet(t: torch.Tensor) -> bool:
    """t starts inside a live block from `empty()` (as the CPU tensor or as its GPU view)."""
    return _heap.owns(t.data_ptr())


def flush() -> None:
    """Free the retired blocks (no tensor uses them any more) once the device has finished its work;
    nothing happens during a graph capture."""
    _heap.release()


def pending() -> int:
    """Retired blocks waiting for `flush()`."""
    return _heap.waiting()
