"""
Pinned host memory of exactly the requested size, mapped for the GPU: the reference's hostmem.py
(ggufengine/hostmem.py:1-125) on HIP.  Weights that stay in RAM (MoE experts that do not fit, offloaded
layers) are allocated with hipHostMalloc(portable | mapped) instead of torch's caching host allocator
(which rounds every pinned block up to a power of two and keeps freed blocks).  On MI355X the GPU sees
such a block at the same address (checked with hipHostGetDevicePointer; a different address is an
error, no kernel is handed the pointer then), so the gathered mat-vec kernels read experts from RAM
over PCIe through their address table (cudakern.mv `adressen`).

A block is freed only in `flush()`, never by the garbage collector: freeing waits for the device and
must neither disturb a graph capture nor pull the memory from under a copy still queued.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Dict, List

import numpy as np
import torch

_PORTABLE = 0x1      # hipHostMallocPortable: pinned for every device context
_MAPPED = 0x2        # hipHostMallocMapped: kernels read it over PCIe

RAM_REST = 8 << 30              # RAM left free after pinning (else the caller keeps ordinary RAM)

_pending: List[int] = []        # pointers of dead blocks, freed in flush()
_ranges: Dict[int, int] = {}    # start -> end of the live blocks (the same addresses on the GPU)
_lock = threading.Lock()
_hip_lib = None


def _hip() -> ctypes.CDLL:
    """The HIP runtime torch has loaded (the one libnmq.so binds to as well)."""
    global _hip_lib
    if _hip_lib is None:
        path = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
        L = ctypes.CDLL(path if os.path.exists(path) else "libamdhip64.so.7")
        pp, p, sz, u = ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint
        L.hipHostMalloc.argtypes, L.hipHostMalloc.restype = [pp, sz, u], ctypes.c_int
        L.hipHostGetDevicePointer.argtypes, L.hipHostGetDevicePointer.restype = [pp, p, u], ctypes.c_int
        L.hipHostFree.argtypes, L.hipHostFree.restype = [p], ctypes.c_int
        _hip_lib = L
    return _hip_lib


class _Block:
    """Owns one hipHostMalloc allocation; numpy (and through it every torch view) keeps it alive."""

    def __init__(self, ptr: int, n: int):
        self.ptr = ptr
        self.__array_interface__ = {"shape": (n,), "typestr": "|u1", "data": (ptr, False), "version": 3}

    def __del__(self):
        try:
            _pending.append(self.ptr)        # atomic under the GIL; no lock in a finaliser
        except Exception:                    # interpreter shutdown: the process frees it
            pass


def ram_reicht(n_bytes: int) -> bool:
    """Would RAM_REST stay free after pinning n_bytes?  Without psutil: yes."""
    try:
        import psutil
        return psutil.virtual_memory().available - int(n_bytes) >= RAM_REST
    except Exception:
        return True


def empty(n_bytes: int, device) -> torch.Tensor:
    """uint8 CPU tensor of n_bytes in pinned RAM, mapped for the GPU at the same address.
    RuntimeError if the runtime cannot pin that much, if less than RAM_REST would stay free, or if the
    GPU would see the block at another address."""
    flush()
    if not ram_reicht(n_bytes):
        raise RuntimeError(f"pinning {n_bytes} bytes would leave less than {RAM_REST >> 30} GB of RAM free")
    device = torch.device(device)
    torch.zeros(1, device=device)            # a current device context for the runtime calls
    L = _hip()
    n = max(1, int(n_bytes))
    ptr = ctypes.c_void_p()
    err = L.hipHostMalloc(ctypes.byref(ptr), n, _PORTABLE | _MAPPED)
    if err or not ptr.value:
        raise RuntimeError(f"hipHostMalloc({n_bytes}): HIP error {err}")
    dptr = ctypes.c_void_p()
    err = L.hipHostGetDevicePointer(ctypes.byref(dptr), ptr, 0)
    if err or dptr.value != ptr.value:
        L.hipHostFree(ptr)
        raise RuntimeError(f"the GPU does not see pinned RAM at the host address (error {err}, "
                           f"{dptr.value!r} vs {ptr.value:#x})")
    with _lock:
        _ranges[ptr.value] = ptr.value + n
    return torch.from_numpy(np.asarray(_Block(ptr.value, int(n_bytes))))


class _GpuView:
    """__cuda_array_interface__ of a host block; torch keeps this object (and through it the block)
    alive as long as the GPU tensor lives."""

    def __init__(self, host: torch.Tensor):
        self.host = host
        self.__cuda_array_interface__ = {"shape": (host.numel(),), "typestr": "|u1", "strides": None,
                                         "data": (host.data_ptr(), False), "version": 3}


def abbilden(host: torch.Tensor, device) -> torch.Tensor:
    """A block from `empty()` as a GPU tensor at the same address: kernels, copies and graphs read it
    over PCIe, nothing is held in VRAM."""
    if not abgebildet(host):
        raise ValueError("only blocks from hostmem.empty() can be mapped")
    view = torch.as_tensor(_GpuView(host.view(-1)), device=torch.device(device))
    if view.data_ptr() != host.data_ptr():
        raise RuntimeError("no unified addressing: the GPU sees the block at another address")
    return view


def abgebildet(t: torch.Tensor) -> bool:
    """t lies in a live block from `empty()` (also as the GPU tensor from `abbilden`)."""
    p = t.data_ptr()
    with _lock:
        return any(a <= p < e for a, e in _ranges.items())


def flush() -> None:
    """Free the blocks no tensor uses any more, once the device has finished all work."""
    if not _pending or torch.cuda.is_current_stream_capturing():
        return
    torch.cuda.synchronize()
    L = _hip()
    while _pending:
        try:
            ptr = _pending.pop()
        except IndexError:                   # emptied by another thread
            break
        with _lock:
            _ranges.pop(ptr, None)
        L.hipHostFree(ctypes.c_void_p(ptr))


def pending() -> int:
    """Dead blocks waiting for `flush()`."""
    return len(_pending)
