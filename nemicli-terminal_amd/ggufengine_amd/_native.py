"""ctypes binding of libnmq.so (C ABI in include/nmq.h).

torch is imported first so that libnmq.so binds to the HIP runtime torch already loaded (same
soname), and torch's streams and allocations are valid in the library.  Nothing here falls back
to another implementation: a missing library or a non-gfx950 device makes `available()` False and
every launch wrapper raise.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from typing import Optional

import torch  # noqa: F401  (loads the HIP runtime first)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.abspath(os.path.join(HERE, "..", "libnmq.so"))

NMQ_OK, NMQ_ERR_FORMAT, NMQ_ERR_SHAPE, NMQ_ERR_ARG, NMQ_ERR_DEVICE = 0, -1, -2, -3, -4
X_BF16, X_F32, X_F32_BF16, X_SILU_MUL_BF16 = 0, 1, 2, 3   # include/nmq.h NMQ_X_*
ACT_SILU, ACT_GELU, ACT_BF16 = 0, 1, 2                    # include/nmq.h NMQ_ACT_*
X_MAX_N_IN = 16384
ABI_VERSION = 2
MAX_COLS = 8

_lock = threading.Lock()
_lib = None
_load_error = None
_device_ok: dict = {}


class NativeError(RuntimeError):
    """A launch failed on the device (the reference raises RuntimeError on cuLaunchKernel errors,
    mmvq.py:817-818, cudakern.py:751-753)."""


def _bind(L: ctypes.CDLL) -> ctypes.CDLL:
    p, i, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    L.nmq_abi_version.restype = i
    L.nmq_strerror.argtypes, L.nmq_strerror.restype = [i], ctypes.c_char_p
    L.nmq_format_info.argtypes, L.nmq_format_info.restype = [i, p, p], i
    L.nmq_device_arch.argtypes, L.nmq_device_arch.restype = [ctypes.c_char_p, i], i
    L.nmq_quant_q8.argtypes, L.nmq_quant_q8.restype = [p, i, p, p, p, p, i64, p], i
    L.nmq_mv.argtypes, L.nmq_mv.restype = [i, p, p, p, p, p, p, i, i, i, p], i
    L.nmq_mm_input.argtypes, L.nmq_mm_input.restype = [p, i, p, p, p, p, i, i, p], i
    L.nmq_mm.argtypes, L.nmq_mm.restype = [i, p, p, p, p, p, p, i, i, i, p], i
    L.nmq_mv_experts.argtypes = [i, p, p, i, i64, p, p, p, p, i, p, i, i, p]
    L.nmq_mv_experts.restype = i
    L.nmq_mv_experts2.argtypes = [i, p, p, p, i, i64, p, p, p, p, i, p, i, i, p]
    L.nmq_mv_experts2.restype = i
    L.nmq_silu_mul_quant.argtypes, L.nmq_silu_mul_quant.restype = [p, p, p, p, p, p, i64, p], i
    L.nmq_moe_combine.argtypes, L.nmq_moe_combine.restype = [p, p, i, i, i, p, p], i
    L.nmq_mv_multi.argtypes = [i, i, p, p, p, p, p, p, p, i, p]
    L.nmq_mv_multi.restype = i
    L.nmq_mv_x.argtypes, L.nmq_mv_x.restype = [i, i, p, p, p, p, i, p, i, p], i
    L.nmq_mv_experts_x.argtypes = [i, p, p, p, i, i64, p, i, p, i, p, i, i, p]
    L.nmq_mv_experts_x.restype = i
    f = ctypes.c_float
    L.nmq_norm_q8.argtypes, L.nmq_norm_q8.restype = [p, p, f, p, p, f, p, p, p, p, p, i64, p], i
    L.nmq_akt_q8.argtypes, L.nmq_akt_q8.restype = [p, p, i, p, p, p, p, p, i64, p], i
    L.nmq_block_sums.argtypes, L.nmq_block_sums.restype = [i, p, p, p, p, p, i, i, p], i
    L.nmq_dequant_bf16.argtypes, L.nmq_dequant_bf16.restype = [i, p, p, i64, p], i
    L.nmq_encode.argtypes, L.nmq_encode.restype = [i, p, i64, p, i], i64
    L.nmq_moe_down_work_bytes.argtypes, L.nmq_moe_down_work_bytes.restype = [i, i, i, i, i, p], i
    L.nmq_moe_down.argtypes = [i, p, p, i, i, i64, p, i, p, p, p, i, i, p, i64, p]
    L.nmq_moe_down.restype = i
    L.nmq_moe_down_static.argtypes = [i, p, p, i, i, i64, p, i, p, p, p, i, i, p]
    L.nmq_moe_down_static.restype = i
    L.nmq_moe_gate_up.argtypes = [i, p, p, p, i, i, i64, p, i, p, p, p, p, i, i, p]
    L.nmq_moe_gate_up.restype = i
    L.nmq_moe_down_q8.argtypes = [i, p, p, i, i, i64, p, p, p, p, p, p, i, i, p, i64, p]
    L.nmq_moe_down_q8.restype = i
    L.nmq_moe_layer_work_bytes.argtypes, L.nmq_moe_layer_work_bytes.restype = [i, i, i, i, p], i
    L.nmq_moe_layer.argtypes = [i, p, p, i64, i, p, i64, p, p, i, i, p, i, p, i, i, p, i64, p]
    L.nmq_moe_layer.restype = i
    L.nmq_mv_gate_up_act.argtypes = [i, p, p, p, i, i, p, p, p, p, i, i, p]
    L.nmq_mv_gate_up_act.restype = i
    L.nmq_stream_read.argtypes, L.nmq_stream_read.restype = [p, i64, p, i, i, i, p], i
    L.nmq_set_tuning.argtypes, L.nmq_set_tuning.restype = [ctypes.c_char_p, i], i
    L.nmq_get_tuning.argtypes, L.nmq_get_tuning.restype = [ctypes.c_char_p, p], i
    return L


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it is missing (build it with `make -C nemicli-terminal_amd/csrc`)."""
    global _lib, _load_error
    if _lib is None:
        with _lock:
            if _lib is None and _load_error is None:
                try:
                    _lib = _bind(ctypes.CDLL(LIB_PATH))
                except OSError as exc:
                    _load_error = exc
    if _lib is None:
        raise NativeError(f"libnmq.so not loadable ({LIB_PATH}): {_load_error}")
    return _lib


def strerror(code: int) -> str:
    return lib().nmq_strerror(code).decode()


def check(code: int) -> None:
    if code == NMQ_OK:
        return
    if code in (NMQ_ERR_SHAPE, NMQ_ERR_ARG, NMQ_ERR_FORMAT):
        raise ValueError(strerror(code))
    raise NativeError(strerror(code))


def available(device=None) -> bool:
    """True when libnmq.so loads and `device` is a gfx950 GPU (the only target of the kernels)."""
    try:
        L = lib()
    except NativeError:
        return False
    dev = torch.device(device) if device is not None else torch.device("cuda")
    if dev.type != "cuda" or not torch.cuda.is_available():
        return False
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _device_ok:
        with _lock:
            if idx not in _device_ok:
                buf = ctypes.create_string_buffer(64)
                with torch.cuda.device(idx):
                    _device_ok[idx] = L.nmq_device_arch(buf, 64) == NMQ_OK
    return _device_ok[idx]


def stream_ptr(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


TUNE_DEFAULT = -(1 << 31)


def set_tuning(name: str, value: Optional[int]) -> None:
    """Override a knob of the launch planner (None: back to its measured default)."""
    rc = lib().nmq_set_tuning(name.encode(), TUNE_DEFAULT if value is None else int(value))
    if rc:
        raise ValueError(f"unknown tuning knob {name!r}")


def get_tuning(name: str) -> Optional[int]:
    v = ctypes.c_int(0)
    if lib().nmq_get_tuning(name.encode(), ctypes.byref(v)):
        raise ValueError(f"unknown tuning knob {name!r}")
    return None if v.value == TUNE_DEFAULT else v.value


@contextlib.contextmanager
def tuning(**knobs):
    """Launch-plan overrides for the duration of a with-block (timing runs and tests), restored after:
    `with tuning(MVM=2, MVT_MAX=1): ...`."""
    before = {k: get_tuning(k) for k in knobs}
    try:
        for k, v in knobs.items():
            set_tuning(k, v)
        yield
    finally:
        for k, v in before.items():
            set_tuning(k, v)
