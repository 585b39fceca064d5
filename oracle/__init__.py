"""CPU oracle for the GGUF quantized mat-vec path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only
as the checker (or as the timed CPU baseline).  The product path (nemicli-terminal_amd/) never
imports it and fails loudly when its own HIP library is missing.

numpy wrappers over liboracle.so (built from nmq_oracle.c and nmq_cpu_baseline.c by the Makefile
beside this file).  Each wrapped C function cites the reference lines it restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q4_0, Q8_0, Q4_K, Q6_K, IQ2_XXS, TQ2_0 = 2, 8, 12, 14, 16, 35
FORMATS = {"Q4_0": (Q4_0, 32, 18), "Q8_0": (Q8_0, 32, 34), "Q4_K": (Q4_K, 256, 144), "Q6_K": (Q6_K, 256, 210),
           "IQ2_XXS": (IQ2_XXS, 256, 66), "TQ2_0": (TQ2_0, 256, 66)}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        p, i, i64, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.or_half_to_float.argtypes, L.or_half_to_float.restype = [ctypes.c_uint16], f
        L.or_round_bf16.argtypes, L.or_round_bf16.restype = [f], f
        L.or_dequant.argtypes, L.or_dequant.restype = [i, p, i64, p], i
        L.or_quant_q8.argtypes, L.or_quant_q8.restype = [p, i64, p, p, p, p], None
        L.or_block_sums.argtypes, L.or_block_sums.restype = [i, p, i, i, p, p, p, p], i
        L.or_mv_int.argtypes, L.or_mv_int.restype = [i, p, i, i, p, p, p, p, i, p], i
        L.or_mv_deq.argtypes, L.or_mv_deq.restype = [i, p, i, i, p, i, p], i
        L.or_gemv_f32.argtypes, L.or_gemv_f32.restype = [p, i, i, p, p, i], None
        L.or_deq_gemv_f32.argtypes, L.or_deq_gemv_f32.restype = [i, p, i, i, p, p, i], i
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def fmt_id(fmt) -> int:
    return FORMATS[fmt][0] if isinstance(fmt, str) else int(fmt)


def fmt_info(fmt):
    for name, (t, bv, bb) in FORMATS.items():
        if t == fmt_id(fmt):
            return name, bv, bb
    raise KeyError(fmt)


def half_to_float(bits: np.ndarray) -> np.ndarray:
    f = lib().or_half_to_float
    return np.array([f(int(b)) for b in np.asarray(bits, dtype=np.uint16).ravel()], dtype=np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """RNE rounding of fp32 to bf16 (returned as fp32): torch's .to(torch.bfloat16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(nan, u.astype(np.uint32), r)
    return r.view(np.float32).reshape(np.shape(x))


def dequant(fmt, raw: np.ndarray) -> np.ndarray:
    """quant.py:484-503 `dequantize` -> flat fp32."""
    _, bv, bb = fmt_info(fmt)
    raw = np.ascontiguousarray(raw, dtype=np.uint8).ravel()
    assert raw.size % bb == 0
    nb = raw.size // bb
    out = np.empty(nb * bv, dtype=np.float32)
    assert lib().or_dequant(fmt_id(fmt), _ptr(raw), nb, _ptr(out)) == 0
    return out


def quant_q8(x: np.ndarray):
    """mmvq.py:62-83 quant_q8 on fp32 values (flattened) -> (xq, xq2, xd, xs)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    n = x.size
    assert n % 32 == 0
    xq = np.empty(n, np.int8)
    xq2 = np.empty(n, np.int8)
    xd = np.empty(n // 32, np.float32)
    xs = np.empty(n // 32, np.float32)
    lib().or_quant_q8(_ptr(x), n, _ptr(xq), _ptr(xq2), _ptr(xd), _ptr(xs))
    return xq, xq2, xd, xs


def norm_row(h: np.ndarray, w: np.ndarray, eps: float, r=None, rs: float = 1.0):
    """mmvq.py:102-120 norm_q8 without its quantisation: v = h + rs*r in fp32 (product and sum each
    rounded, numpy float32 semantics), then the RMS norm in fp64, xn = v / sqrt(mean(v^2) + eps) * w.
    -> (v float32, xn float64).  Pinned by closed forms in tests/test_oracle.py."""
    h = np.ascontiguousarray(h, dtype=np.float32).ravel()
    v = h if r is None else h + np.float32(rs) * np.ascontiguousarray(r, dtype=np.float32).ravel()
    v64 = v.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(v64 * v64) + float(eps))
    return v, v64 * inv * np.asarray(w, np.float64).ravel()


GELU_C = 0.7978845608      # sqrt(2/pi) as written in mmvq.py:127
GELU_A = 0.044715


def akt(g: np.ndarray, u=None, gelu: bool = False) -> np.ndarray:
    """mmvq.py:122-133 akt_q8 without its quantisation, in fp64: silu(g) = g / (1 + exp(-g)) or the tanh
    form of gelu, 0.5 g (1 + tanh(GELU_C (g + GELU_A g^3))), times u if given.  Pinned by the odd-part
    identities act(x) - act(-x) = x, by silu = x * expit(x) and by the erf form of gelu
    (tests/test_oracle.py)."""
    x = np.asarray(g, np.float64).ravel()
    if gelu:
        a = 0.5 * x * (1.0 + np.tanh(GELU_C * (x + GELU_A * x * x * x)))
    else:
        with np.errstate(over="ignore"):
            a = x / (1.0 + np.exp(-x))
    return a if u is None else a * np.asarray(u, np.float64).ravel()


def block_sums(fmt, raw: np.ndarray, n_out: int, n_in: int, xq: np.ndarray, xq2: np.ndarray):
    """int32 sums per 16 weights: (s1, s2), each (n_out, n_in/16)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).ravel()
    xq = np.ascontiguousarray(xq, dtype=np.int8).ravel()
    xq2 = np.ascontiguousarray(xq2, dtype=np.int8).ravel()
    s1 = np.empty((n_out, n_in // 16), np.int32)
    s2 = np.empty((n_out, n_in // 16), np.int32)
    assert lib().or_block_sums(fmt_id(fmt), _ptr(raw), n_out, n_in, _ptr(xq), _ptr(xq2), _ptr(s1), _ptr(s2)) == 0
    return s1, s2


def mv_int(fmt, raw, n_out, n_in, xq, xq2, xd, xs, ncols=1) -> np.ndarray:
    """Integer-decomposition mat-vec, fp64 combine -> (ncols, n_out) float64."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).ravel()
    a = [np.ascontiguousarray(v) for v in (xq, xq2, xd, xs)]
    y = np.empty((ncols, n_out), np.float64)
    assert lib().or_mv_int(fmt_id(fmt), _ptr(raw), n_out, n_in, *[_ptr(v) for v in a], ncols, _ptr(y)) == 0
    return y


def mv_deq(fmt, raw, n_out, n_in, x) -> np.ndarray:
    """Dequantise + matmul, fp64 accumulation: x (ncols, n_in) fp32 -> (ncols, n_out) float64."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).ravel()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n_in)
    y = np.empty((x.shape[0], n_out), np.float64)
    assert lib().or_mv_deq(fmt_id(fmt), _ptr(raw), n_out, n_in, _ptr(x), x.shape[0], _ptr(y)) == 0
    return y


def mm_input(x: np.ndarray):
    """Two-stage fp16 input of the several-token path, per token row (the per-token scaling of
    mmvq.py:617-641 with a power-of-two scale and a second stage): xs = 2^(e - 8) for
    max|x| = f 2^e (f in [0.5, 1), e >= -100), v = x / xs, xh = fp16(v), xl = fp16(v - xh), both
    rounded to nearest even, and per 32 values the fp32 sum of xh + xl (each run of 8 added in order,
    then the 4 runs pairwise) -> (xh, xl float16 (M, n), xsum float32 (M, n/32), xs float32 (M,))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x = x.reshape(-1, x.shape[-1])
    m = np.abs(x).max(axis=1).astype(np.float64)
    _, e = np.frexp(m)
    e = np.maximum(e, -100)
    v = (x.astype(np.float64) * np.ldexp(1.0, 8 - e)[:, None]).astype(np.float32)   # exact
    xh = v.astype(np.float16)
    xl = (v - xh.astype(np.float32)).astype(np.float16)                              # v - xh exact
    w = (xh.astype(np.float32) + xl.astype(np.float32)).reshape(x.shape[0], -1, 4, 8)
    run = w[..., 0]
    for j in range(1, 8):
        run = run + w[..., j]                                                         # float32 adds
    xsum = (run[..., 0] + run[..., 1]) + (run[..., 2] + run[..., 3])
    return xh, xl, xsum.astype(np.float32), np.ldexp(1.0, e - 8).astype(np.float32)


def mm_x(x: np.ndarray) -> np.ndarray:
    """The input the several-token path multiplies with: xs * (xh + xl) in float64 (M, n)."""
    xh, xl, _, xs = mm_input(x)
    return (xh.astype(np.float64) + xl.astype(np.float64)) * xs.astype(np.float64)[:, None]

def gemv_f32(w: np.ndarray, x: np.ndarray, threads: int) -> np.ndarray:
    """CPU baseline GEMV (F.linear of the Linear path, models/common.py:526-527)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty(w.shape[0], np.float32)
    lib().or_gemv_f32(_ptr(w), w.shape[0], w.shape[1], _ptr(x), _ptr(y), threads)
    return y


def deq_gemv_f32(fmt, raw, n_out, n_in, x, threads: int) -> np.ndarray:
    """CPU baseline of the PackedLinear fallback: dequantise per call + GEMV (common.py:414-428)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).ravel()
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty(n_out, np.float32)
    assert lib().or_deq_gemv_f32(fmt_id(fmt), _ptr(raw), n_out, n_in, _ptr(x), _ptr(y), threads) == 0
    return y


def rel_err_rows(y: np.ndarray, ref: np.ndarray) -> np.ndarray:
    """Per output row-vector: max_i |y - ref| / max_i |ref| (test_gguf_iq.py:215 convention)."""
    y = np.asarray(y, np.float64).reshape(-1, np.shape(ref)[-1])
    ref = np.asarray(ref, np.float64).reshape(y.shape)
    return np.abs(y - ref).max(axis=1) / np.maximum(np.abs(ref).max(axis=1), 1e-30)
