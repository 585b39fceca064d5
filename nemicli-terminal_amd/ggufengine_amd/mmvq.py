"""
Drop-in for the reference's ggufengine/mmvq.py (int8 mat-vec on Q4_K / Q6_K blocks), on gfx950.

Same names, arguments and return shapes as the reference module (mmvq.py:25-37, 808-938):
`FORMATE`, `SPALTEN`, `MMVQ_BIS`, `MMQ_BIS`, `ZEILEN_JE_WARP`, `verfuegbar`, `Eingang`, `mv`,
`eingang_teilen`, `mm`, `entpacken`, `norm_q8`, `akt_q8`, `schritt_moeglich`.  The arithmetic is the reference's: the
input is quantised per 32 values in two int8 stages (about 15 bits, fp32 scale and sum), every
weight byte is read once and multiplied with v_dot4_i32_i8, and the per-sub-block scales are applied
in fp32.  Launches go through libnmq.so (include/nmq.h) on torch's current stream, so they can be
captured in a HIP graph.  No torch or CPU fallback: `verfuegbar` is False without the library or a
gfx950 device, and calls raise.

Differences from the reference (documented, same results within the parity tolerance):
  - up to 16 tokens per launch on the int8 matrix cores, SPALTEN = 8 on the dot4 kernels (the
    reference compiles 1..9 per launch); MMVQ_BIS (where callers switch to `mm`) is 8 for rows of up to
    4096 values or a multiple of 2048 up to 32768 and, for other rows, MMVQ_BIS_LANG: 1 for Q4_K and 4 for
    Q6_K, measured on MI355X (the reference: 16 for both); `mv_bis(fmt, n_in)` picks between them;
  - `mm` (the reference's fp16 tensor-core MMQ tiles for 17..112 tokens) runs on the fp16 matrix
    cores with exact integer weights and a two-stage fp16 input (about 22 bits against the
    reference's fp16 weights and input), 64 tokens per launch;
  - of the fused one-token steps, norm_q8 and akt_q8 are provided; rope_kv and attention1 are not,
    so `schritt_moeglich` returns False and callers take their unfused layer path
    (models/baukasten.py:205).
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from typing import Optional

import torch

from . import _native
from .gguf_types import TYPE_ID

FORMATE = {"Q4_K": (256, 144), "Q6_K": (256, 210)}
WARPS = 4                     # waves per workgroup (at most; fewer for short matrices)
SPALTEN = _native.MAX_COLS    # tokens (input rows) per launch, weights read once for all of them
# weight rows per team of lanes by token count (the kernels are compiled for these)
ZEILEN_JE_WARP = {"Q4_K": lambda nc: 1 if nc == 1 else 2, "Q6_K": lambda nc: 1 if nc == 1 else 2}
# Most tokens per call for the int8 mat-vec kernels; from one more token on, callers take `mm` (the fp16
# matrix cores); the reference's 16 / 16 (mmvq.py:32).  Measured on MI355X, each call with its input
# launch (mv / mm, us):
#   rows of up to 4096 values (the dense-read matrix-core kernel up to 8 tokens): Q4_K 14336x4096 at 8
#   tokens 13.3 / 25.0, at 9 19.7 / 25.0, at 12 26.0 / 25.1; Q6_K 14336x4096 at 8 22.5 / 32.8, at 9
#   31.8 / 32.8, at 12 41.0 / 33.0; 4096x4096 at 9 11.0 / 11.0 (Q4_K), 13.8 / 13.3 (Q6_K);
#   longer rows of a multiple of 2048 values (the dense kernel over K ranges in one launch): Q4_K
#   4096x14336 at 2 / 4 / 8 tokens 14.9 / 15.6 / 17.4 against 25.2 / 25.6 / 25.9; Q6_K 4096x14336 at
#   2-4 tokens 20.6-26.7 / 35.6-35.8 (the few-token long-row kernel), at 5 / 8 25.0 / 26.0 against
#   35.9 / 36.1;
#   other long rows (MMVQ_BIS_LANG): Q4_K 4096x14336 on the other kernels at 2 tokens 27.9 / 25.0, at 4
#   39.0 / 25.5; Q6_K at 5 tokens 51.2 / 36.6.
MMVQ_BIS = {"Q4_K": 8, "Q6_K": 8}
MMVQ_BIS_LANG = {"Q4_K": 1, "Q6_K": 4}
MMQ_BIS = {"Q4_K": 112, "Q6_K": 112}


def mv_bis(fmt: str, n_in: int) -> int:
    """Most tokens per call that go to `mv` for rows of n_in values (more go to `mm`)."""
    dense = n_in <= 4096 or (n_in % 2048 == 0 and n_in <= 32768)
    return MMVQ_BIS[fmt] if dense else MMVQ_BIS_LANG[fmt]


def verfuegbar(device, fmt: str, n_in: int) -> bool:
    """Kernel for this format and row length on this device (reference mmvq.py:808-810)."""
    return fmt in FORMATE and n_in % 256 == 0 and n_in > 0 and _native.available(device)


def _starten(name: str, fn, *args) -> None:
    """Every launch of this module goes through here (name of the kernel family, C function,
    arguments); a nonzero return raises like the reference's _starten (mmvq.py:813-818)."""
    _native.check(fn(*args))


def _z(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


class Eingang:
    """The two-stage int8 input of a vector (or of M token rows back to back): xq, xq2 int8 (n),
    xd = scale and xs = sum per 32 values (float32, n/32).  Built once per input, shared by every
    matrix that reads it.  Without x only the buffers (reference mmvq.py:821-849)."""

    def __init__(self, x: Optional[torch.Tensor] = None, n: int = 0, device=None):
        if x is not None:
            x = x.reshape(-1)
            if x.dtype != torch.float32:
                x = x.to(torch.bfloat16)
            x = x.contiguous()
            n, device = x.numel(), x.device
        if n % 32:
            raise ValueError(f"Eingang: {n} values are not a multiple of 32")
        self.n = n
        self.xq = torch.empty(n, dtype=torch.int8, device=device)
        self.xq2 = torch.empty(n, dtype=torch.int8, device=device)          # rest, scale xd / 254
        self.xd = torch.empty(n // 32, dtype=torch.float32, device=device)
        self.xs = torch.empty(n // 32, dtype=torch.float32, device=device)
        if x is not None:
            L = _native.lib()
            _starten("quant_q8", L.nmq_quant_q8, x.data_ptr(), int(x.dtype == torch.float32),
                     *[t.data_ptr() for t in (self.xq, self.xq2, self.xd, self.xs)], n,
                     _native.stream_ptr(x.device))

    def zeiger(self, ab: int = 0) -> list:
        """Pointers to xq, xq2, xd, xs from value `ab` on (the start of a token row)."""
        if not ab:
            return [_z(self.xq), _z(self.xq2), _z(self.xd), _z(self.xs)]
        return [_z(self.xq[ab:]), _z(self.xq2[ab:]), _z(self.xd[ab // 32:]), _z(self.xs[ab // 32:])]


def eingang_bf16(x: torch.Tensor) -> Eingang:
    """The Eingang of x rounded to bf16 first (the input convention of the cudakern entry points,
    reference cudakern.py:764), in one launch: fp32 x is rounded inside the quantisation kernel."""
    x = x.reshape(-1)
    if x.dtype == torch.bfloat16:
        return Eingang(x)
    xf = x.float().contiguous()
    e = Eingang(n=xf.numel(), device=xf.device)
    _starten("quant_q8", _native.lib().nmq_quant_q8, xf.data_ptr(), 2,
             *[t.data_ptr() for t in (e.xq, e.xq2, e.xd, e.xs)], e.n, _native.stream_ptr(xf.device))
    return e


_TEILEN = threading.local()


@contextlib.contextmanager
def eingang_teilen():
    """Matrices with the same input (q/k/v, gate/up): inside, the int8 input of a tensor is built
    once (keyed by data pointer, shape and dtype, as the reference keys its MMQ input,
    mmvq.py:868-899) and reused by `mv` and `mm`."""
    alt = getattr(_TEILEN, "werte", None)
    _TEILEN.werte = {}
    try:
        yield
    finally:
        _TEILEN.werte = alt


def _eingang(x: torch.Tensor) -> Eingang:
    geteilt = getattr(_TEILEN, "werte", None)
    if geteilt is None:
        return Eingang(x)
    key = (x.data_ptr(), tuple(x.shape), x.dtype)
    e = geteilt.get(key)
    if e is None:
        e = geteilt[key] = Eingang(x)
    return e


# Longest input a one-token launch quantises itself (measured on MI355X: past this, staging the values
# in every workgroup costs more than one quantisation launch).
WERTE_BIS = 8192


def _werte(x: torch.Tensor, n_in: int, bf16: bool):
    """(values tensor, x_mode) for a launch that quantises one token's input itself, or None where the
    quantisation launch is used (long rows, views that are not 16-byte aligned).  fp32 stays fp32
    (bf16: rounded to bf16 in the launch, the cudakern convention), other types go to bf16 first as
    in Eingang."""
    if n_in > WERTE_BIS or x.numel() % n_in or not x.is_contiguous():
        return None
    if x.dtype == torch.float32:
        t, mode = x, (_native.X_F32_BF16 if bf16 else _native.X_F32)
    else:
        t, mode = (x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16).contiguous()), _native.X_BF16
    if t.data_ptr() % 16:
        return None
    return t, mode


def _mv_werte(fmt: str, raws, t: torch.Tensor, mode: int, n_outs, n_in: int) -> list:
    """One launch (per MAX_MATRIZEN matrices) on one token given as values -> [(n_out,) float32]."""
    dev = raws[0].device
    ys = [torch.empty(n, dtype=torch.float32, device=dev) for n in n_outs]
    L = _native.lib()
    for a in range(0, len(raws), MAX_MATRIZEN):
        part = range(a, min(a + MAX_MATRIZEN, len(raws)))
        k = len(part)
        _starten("mv", L.nmq_mv_x, TYPE_ID[fmt], k, (ctypes.c_void_p * k)(*[raws[i].data_ptr() for i in part]),
                 (ctypes.c_int * k)(*[int(n_outs[i]) for i in part]),
                 (ctypes.c_void_p * k)(*[ys[i].data_ptr() for i in part]), t.data_ptr(), mode, None, n_in,
                 _native.stream_ptr(dev))
    return ys


def _mv(fmt: str, raw: torch.Tensor, e: Eingang, n_out: int, n_in: int) -> torch.Tensor:
    if e.n % n_in:
        raise ValueError(f"mv: input of {e.n} values is not a multiple of n_in={n_in}")
    M = e.n // n_in
    y = torch.empty(M, n_out, dtype=torch.float32, device=raw.device)
    L = _native.lib()
    _starten("mv", L.nmq_mv, TYPE_ID[fmt], raw.data_ptr(), e.xq.data_ptr(), e.xq2.data_ptr(),
             e.xd.data_ptr(), e.xs.data_ptr(), y.data_ptr(), n_out, n_in, M, _native.stream_ptr(raw.device))
    return y


def mv(fmt: str, raw: torch.Tensor, x, n_out: int, n_in: int) -> torch.Tensor:
    """raw: (n_out, n_in) in block format on the GPU; x: (M, n_in) or (n_in,) bf16/float32, or an
    Eingang of M rows -> (M, n_out) float32, or (n_out,) for a vector (reference mmvq.py:852-865)."""
    if fmt not in FORMATE:
        raise ValueError(f"mmvq.mv: format {fmt} (this module serves {tuple(FORMATE)})")
    if not isinstance(x, Eingang) and x.numel() == n_in:
        w = _werte(x.reshape(-1), n_in, bf16=False)
        if w is not None:   # one token: the launch quantises it (no separate quantisation launch)
            y = _mv_werte(fmt, [raw], w[0], w[1], [n_out], n_in)[0]
            return y if x.dim() == 1 else y.view(1, n_out)
    e = x if isinstance(x, Eingang) else _eingang(x)
    y = _mv(fmt, raw, e, n_out, n_in)
    vektor = y.shape[0] == 1 if isinstance(x, Eingang) else x.dim() == 1
    return y[0] if vektor else y


MAX_MATRIZEN = 4   # matrices per mv_mehrere launch (include/nmq.h NMQ_MAX_MATS)


def mv_mehrere(fmt: str, raws, x, n_outs, n_in: int) -> list:
    """Several matrices of one format on one token's input in one launch (q/k/v or gate/up sharing an
    Eingang): raws[i] (n_outs[i], n_in) in block format, x (n_in,) or an Eingang of one row ->
    [(n_outs[i],) float32].  Each result equals `mv(fmt, raws[i], x, n_outs[i], n_in)`; the rows of all
    matrices share the launch.  More than MAX_MATRIZEN matrices go in several launches."""
    if fmt not in FORMATE:
        raise ValueError(f"mmvq.mv_mehrere: format {fmt} (this module serves {tuple(FORMATE)})")
    if len(raws) != len(n_outs) or not raws:
        raise ValueError("mv_mehrere: one n_out per matrix")
    if not isinstance(x, Eingang):
        if x.numel() != n_in:
            raise ValueError(f"mv_mehrere: one token of {n_in} values expected, the input holds {x.numel()}")
        w = _werte(x.reshape(-1), n_in, bf16=False)
        if w is not None:
            return _mv_werte(fmt, raws, w[0], w[1], n_outs, n_in)
    e = x if isinstance(x, Eingang) else _eingang(x.reshape(-1))
    if e.n != n_in:
        raise ValueError(f"mv_mehrere: one token of {n_in} values expected, the input holds {e.n}")
    dev = raws[0].device
    ys = [torch.empty(n, dtype=torch.float32, device=dev) for n in n_outs]
    L = _native.lib()
    for a in range(0, len(raws), MAX_MATRIZEN):
        part = range(a, min(a + MAX_MATRIZEN, len(raws)))
        k = len(part)
        ws = (ctypes.c_void_p * k)(*[raws[i].data_ptr() for i in part])
        ns = (ctypes.c_int * k)(*[int(n_outs[i]) for i in part])
        yp = (ctypes.c_void_p * k)(*[ys[i].data_ptr() for i in part])
        _starten("mv", L.nmq_mv_multi, TYPE_ID[fmt], k, ws, ns, yp, e.xq.data_ptr(), e.xq2.data_ptr(),
                 e.xd.data_ptr(), e.xs.data_ptr(), n_in, _native.stream_ptr(dev))
    return ys


def _mmq_eingang(x2: torch.Tensor) -> tuple:
    """(xh, xl float16, xsum, xs float32) for x2 (M, n): the two-stage fp16 input of `mm` in one launch
    (reference mmvq.py:882-899); inside eingang_teilen() built once per input."""
    geteilt = getattr(_TEILEN, "werte", None)
    key = ("mm", x2.data_ptr(), tuple(x2.shape), x2.dtype)
    if geteilt is not None and key in geteilt:
        return geteilt[key]
    if x2.dtype not in (torch.float32, torch.bfloat16):
        x2 = x2.to(torch.bfloat16)
    x2 = x2.contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    M, n = x2.shape
    # in the matrix cores' operand order, rows padded to a multiple of 16 (include/nmq.h)
    xh = torch.empty((M + 15) // 16 * 16, n, dtype=torch.float16, device=x2.device)
    xl = torch.empty_like(xh)
    xsum = torch.empty(xh.shape[0], n // 32, dtype=torch.float32, device=x2.device)
    xs = torch.empty(M, dtype=torch.float32, device=x2.device)
    _starten("mmq_eingang", _native.lib().nmq_mm_input, x2.data_ptr(), int(x2.dtype == torch.float32),
             xh.data_ptr(), xl.data_ptr(), xsum.data_ptr(), xs.data_ptr(), n, M, _native.stream_ptr(x2.device))
    if geteilt is not None:
        geteilt[key] = (xh, xl, xsum, xs)
    return xh, xl, xsum, xs


def mm(fmt: str, raw: torch.Tensor, x: torch.Tensor, n_out: int, n_in: int) -> torch.Tensor:
    """Several tokens on the matrix cores: x (M, n_in) bf16/float32 -> (M, n_out) float32 (reference
    mmvq.py:902-920).  The weights are unpacked once per launch of up to 64 tokens as exact fp16
    integer products, the input goes in as two fp16 stages (about 22 bits), d and the min term are
    applied in fp32 per block."""
    if fmt not in FORMATE:
        raise ValueError(f"mmvq.mm: format {fmt}")
    x2 = x.reshape(-1, n_in)
    xh, xl, xsum, xs = _mmq_eingang(x2)
    M = x2.shape[0]
    y = torch.empty(M, n_out, dtype=torch.float32, device=raw.device)
    _starten("mmq", _native.lib().nmq_mm, TYPE_ID[fmt], raw.data_ptr(), xh.data_ptr(), xl.data_ptr(),
             xsum.data_ptr(), xs.data_ptr(), y.data_ptr(), n_out, n_in, M, _native.stream_ptr(raw.device))
    return y


def entpacken(fmt: str, raw: torch.Tensor, n_out: int, n_in: int) -> torch.Tensor:
    """raw: (n_out, n_in) in block format -> (n_out, n_in) bf16 (reference mmvq.py:923-931): the
    exact fp32 value of quant.py rounded to nearest-even bf16."""
    bs, _ = FORMATE[fmt]
    out = torch.empty(n_out, n_in, dtype=torch.bfloat16, device=raw.device)
    L = _native.lib()
    _starten("entpacken", L.nmq_dequant_bf16, TYPE_ID[fmt], raw.data_ptr(), out.data_ptr(), n_out * n_in // bs,
             _native.stream_ptr(raw.device))
    return out


def _f32(t: torch.Tensor) -> torch.Tensor:
    """t as a contiguous float32 vector (t itself when it already is one)."""
    if t.dim() == 1 and t.dtype == torch.float32 and t.is_contiguous():
        return t
    return t.reshape(-1).to(torch.float32).contiguous()


def norm_q8(h: torch.Tensor, w: torch.Tensor, eps: float, rest: Optional[torch.Tensor] = None,
            rs: float = 1.0):
    """RMS norm of one row, fused with its Eingang (reference mmvq.py:951-961).  With `rest`, first
    h = h + rs * rest.  -> (normalised float32, Eingang, new h) in one launch."""
    h = _f32(h)
    n = h.numel()
    w = _f32(w)
    if w.numel() != n:
        raise ValueError(f"norm_q8: weight of {w.numel()} values for a row of {n}")
    e = Eingang(n=n, device=h.device)
    xn = torch.empty(n, dtype=torch.float32, device=h.device)
    hn = None
    if rest is not None:
        rest = _f32(rest)
        if rest.numel() != n:
            raise ValueError(f"norm_q8: rest of {rest.numel()} values for a row of {n}")
        hn = torch.empty(n, dtype=torch.float32, device=h.device)
    _starten("norm_q8", _native.lib().nmq_norm_q8, h.data_ptr(), None if rest is None else rest.data_ptr(),
             float(rs), None if hn is None else hn.data_ptr(), w.data_ptr(), float(eps), xn.data_ptr(),
             *[t.data_ptr() for t in (e.xq, e.xq2, e.xd, e.xs)], n, _native.stream_ptr(h.device))
    return xn, e, (h if hn is None else hn)


def akt_q8(g: torch.Tensor, u: Optional[torch.Tensor], gelu: bool):
    """act(g) * u (without u: act(g)), act = silu or tanh-gelu -> (float32, Eingang) in one launch
    (reference mmvq.py:964-971)."""
    g = _f32(g)
    n = g.numel()
    if u is not None:
        u = _f32(u)
        if u.numel() != n:
            raise ValueError(f"akt_q8: up of {u.numel()} values for a gate of {n}")
    e = Eingang(n=n, device=g.device)
    a = torch.empty(n, dtype=torch.float32, device=g.device)
    _starten("akt_q8", _native.lib().nmq_akt_q8, g.data_ptr(), None if u is None else u.data_ptr(), int(bool(gelu)),
             a.data_ptr(), *[t.data_ptr() for t in (e.xq, e.xq2, e.xd, e.xs)], n, _native.stream_ptr(g.device))
    return a, e


def gate_up_akt(fmt: str, raw_gate: torch.Tensor, raw_up: torch.Tensor, x: torch.Tensor, n_out: int, n_in: int,
                gelu: bool = False) -> Eingang:
    """The FFN's gate and up mat-vecs on one token and act(gate) * up as the down projection's Eingang
    (reference models/baukasten.py:217-241: mv on gate and up, then akt_q8): one launch where the library
    takes the shape (nmq_mv_gate_up_act: Q4_K, TQ2_0, IQ2_XXS, rows of at most 4096 values, n_out % 32 == 0,
    an fp32 input), bit for bit mv_mehrere + akt_q8; otherwise those two calls."""
    dev = raw_gate.device
    xf = _f32(x)
    if xf.numel() != n_in:
        raise ValueError(f"gate_up_akt: one token of {n_in} values expected, the input holds {xf.numel()}")
    e = Eingang(n=n_out, device=dev)
    rc = _native.lib().nmq_mv_gate_up_act(TYPE_ID[fmt], raw_gate.data_ptr(), raw_up.data_ptr(), xf.data_ptr(),
                                          _native.X_F32, _native.ACT_GELU if gelu else _native.ACT_SILU,
                                          e.xq.data_ptr(), e.xq2.data_ptr(), e.xd.data_ptr(), e.xs.data_ptr(),
                                          n_out, n_in, _native.stream_ptr(dev))
    if rc != _native.NMQ_ERR_SHAPE:
        _native.check(rc)
        return e
    g, u = mv_mehrere(fmt, [raw_gate, raw_up], xf, [n_out, n_out], n_in)
    return akt_q8(g, u, gelu)[1]


def schritt_moeglich(device, H: int, Hkv: int, D: int) -> bool:
    """The whole fused one-token step also needs rope_kv and attention1, which are not part of this
    library: always False, so callers run their general layer path (reference mmvq.py:1009-1014,
    models/baukasten.py:205).  norm_q8 and akt_q8 are available on their own."""
    return False
