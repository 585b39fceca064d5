"""Writes the golden fixtures of tests/golden/ (committed; tests only read them).

Run in the build container:  python tests/golden/gen_golden.py
It reads the reference's IQ2_XXS grid as text (ggufengine/iqtabellen.py:11-77, hex literals only).
Nothing here imports or executes reference code; every expected value below comes from one of:

  known_<FMT>   Q4_0 / Q8_0 / Q4_K / Q6_K blocks built value by value following the *kernel* indexing
                of the reference's cudakern.py (dot_Q4_0 :315-321, dot_Q8_0 :307-313, dot_Q4_K with
                skala_k4 :360-377, dot_Q6_K :394-407) with scales chosen as powers of two, so that every expected
                value d*sc*q - dmin*m is exact.  The oracle follows quant.py (the vectorised
                dequantiser); agreement pins both readings of the layout against each other.
  iq2_xxs       random blocks (the reference's `zufallsbloecke`, tests/test_gguf_iq.py:81-101) and
                values from a restatement of its pure-Python `ref_iq2_xxs` (:43-54).
  tq2_0         random blocks and values from a restatement of `ref_tq2_0`
                (tests/test_gguf_ternaer.py:62-69); plus ternary weights and their encoding by a
                restatement of `pack_tq2_0` (:143-154), whose dequantisation must be lossless (:239-245).
"""
from __future__ import annotations

import os
import re
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_TABLES = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/ggufengine/iqtabellen.py"


def grid_from_text(path: str) -> list:
    text = open(path, encoding="utf-8").read()
    m = re.search(r"IQ2XXS_GRID\s*=\s*\((.*?)\)", text, re.S)
    return [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", m.group(1))]


def f16(b: bytes, o: int) -> float:
    return struct.unpack_from("<e", b, o)[0]


# ---- known-answer blocks (cudakern.py kernel indexing, exact values) --------------------------------

def known_q8_0(rng, nb):
    raw, vals = bytearray(), []
    for _ in range(nb):
        d = 2.0 ** int(rng.integers(-12, -4))
        q = rng.integers(-128, 128, 32)
        raw += struct.pack("<e", d) + bytes(int(v) & 255 for v in q)
        vals += [d * int(v) for v in q]                     # dot_Q8_0: h2f(d) * (float)qs[j]
    return np.frombuffer(bytes(raw), np.uint8), np.array(vals, np.float32)


def known_q4_0(rng, nb):
    raw, vals = bytearray(), []
    for _ in range(nb):
        d = 2.0 ** int(rng.integers(-12, -4))
        q = rng.integers(0, 16, 32)                     # nibble of value j
        qs = bytes(int(q[j]) | (int(q[j + 16]) << 4) for j in range(16))
        raw += struct.pack("<e", d) + qs
        vals += [d * (int(v) - 8) for v in q]           # dot_Q4_0: (q[j] & 15) - 8 at j, (q[j] >> 4) - 8 at j + 16
    return np.frombuffer(bytes(raw), np.uint8), np.array(vals, np.float32)


def pack_scales_k4(sc, m):
    """12 bytes such that cudakern skala_k4 (== ggml get_scale_min_k4) returns sc[j], m[j]."""
    out = [0] * 12
    for j in range(4):
        out[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return bytes(out)


def skala_k4(sc12, s):
    if s < 4:
        return sc12[s] & 63, sc12[s + 4] & 63
    return (sc12[s + 4] & 15) | ((sc12[s - 4] >> 6) << 4), (sc12[s + 4] >> 4) | ((sc12[s] >> 6) << 4)


def known_q4_k(rng, nb):
    raw, vals = bytearray(), []
    for _ in range(nb):
        d = 2.0 ** int(rng.integers(-14, -6))
        dmin = 2.0 ** int(rng.integers(-14, -6))
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        mn = [int(v) for v in rng.integers(0, 64, 8)]
        sc12 = pack_scales_k4(sc, mn)
        assert all(skala_k4(sc12, s) == (sc[s], mn[s]) for s in range(8))
        q = rng.integers(0, 16, 256)                     # value 32 s + t of sub-block s
        qs = [0] * 128
        for s in range(8):                               # dot_Q4_K: byte 16 + 32 (s >> 1) + t, shift 4 (s & 1)
            for t in range(32):
                qs[32 * (s >> 1) + t] |= int(q[32 * s + t]) << (4 * (s & 1))
        raw += struct.pack("<ee", d, dmin) + sc12 + bytes(qs)
        for s in range(8):
            for t in range(32):
                vals.append(d * sc[s] * int(q[32 * s + t]) - dmin * mn[s])
    return np.frombuffer(bytes(raw), np.uint8), np.array(vals, np.float64).astype(np.float32)


def known_q6_k(rng, nb):
    raw, vals = bytearray(), []
    for _ in range(nb):
        d = 2.0 ** int(rng.integers(-14, -6))
        sc = [int(v) for v in rng.integers(-128, 128, 16)]
        q = rng.integers(0, 64, 256)
        ql, qh = [0] * 128, [0] * 64
        for s in range(8):                               # dot_Q6_K: n = s >> 2, g = s & 3
            n, g = s >> 2, s & 3
            for t in range(32):
                v = int(q[32 * s + t])
                ql[64 * n + 32 * (g & 1) + t] |= (v & 15) << (4 * (g >> 1))
                qh[32 * n + t] |= (v >> 4) << (2 * g)
        raw += bytes(ql) + bytes(qh) + bytes(v & 255 for v in sc) + struct.pack("<e", d)
        for s in range(8):
            n, g = s >> 2, s & 3
            for t in range(32):                          # sc[8n + 2g + (t >= 16)]
                vals.append(d * sc[8 * n + 2 * g + (t >= 16)] * (int(q[32 * s + t]) - 32))
    return np.frombuffer(bytes(raw), np.uint8), np.array(vals, np.float64).astype(np.float32)


# ---- reference-test restatements ---------------------------------------------------------------------

def random_blocks(size, scale_offsets, nb, seed):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nb, size), dtype=np.uint8)
    for o in scale_offsets:
        s = (rng.random(nb) * 0.01 + 0.001).astype(np.float16)
        raw[:, o:o + 2] = s.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def ksign(i):
    return i | ((bin(i).count("1") & 1) << 7)


def ref_iq2_xxs(b: bytes, grid) -> list:
    out = []
    for o in range(0, len(b), 66):
        d = f16(b, o)
        for ib in range(8):
            q = b[o + 2 + 8 * ib:o + 10 + 8 * ib]
            aux1 = struct.unpack_from("<I", q, 4)[0]
            db = d * (0.5 + (aux1 >> 28)) * 0.25
            for l in range(4):
                g = [(grid[q[l]] >> (8 * j)) & 0xFF for j in range(8)]
                s = ksign((aux1 >> (7 * l)) & 127)
                out += [db * g[j] * (-1 if s & (1 << j) else 1) for j in range(8)]
    return out


def ref_tq2_0(b: bytes) -> list:
    out = []
    for o in range(0, len(b), 66):
        d = f16(b, o + 64)
        for j in (0, 32):
            for l in range(4):
                out += [(((b[o + j + m] >> (2 * l)) & 3) - 1) * d for m in range(32)]
    return out


def rund(v):  # roundf / lroundf: halves away from zero
    return int(v + 0.5) if v >= 0 else -int(-v + 0.5)


def pack_tq2_0(x) -> bytes:
    out = bytearray()
    for i in range(0, len(x), 256):
        blk = x[i:i + 256]
        d = max(abs(v) for v in blk)
        idv = 1.0 / d if d else 0.0
        qs = bytearray(64)
        for j in (0, 32):
            for m in range(32):
                for n in range(4):
                    qs[j + m] |= ((rund(blk[4 * j + m + 32 * n] * idv) + 1) & 3) << (2 * n)
        out += qs + struct.pack("<e", d)
    return bytes(out)


def ternary(rows, cols, group, seed):
    """d * {-1, 0, +1} with fp16 d per group, first value of every group +d (the reference's
    `ternaer`, tests/test_gguf_ternaer.py:195-203)."""
    rng = np.random.default_rng(seed)
    t = rng.integers(-1, 2, size=(rows, cols)).astype(np.float32)
    t.reshape(rows, -1, group)[:, :, 0] = 1
    d = (rng.random((rows, cols // group, 1)) * 0.08 + 0.02).astype(np.float16).astype(np.float32)
    return (t.reshape(rows, -1, group) * d).reshape(rows, cols)


def main() -> None:
    grid = grid_from_text(REF_TABLES)
    rng = np.random.default_rng(20261201)
    out = {}
    for name, fn, nb in (("q8_0", known_q8_0, 24), ("q4_k", known_q4_k, 6), ("q6_k", known_q6_k, 6)):
        raw, vals = fn(rng, nb)
        out[f"known_{name}_raw"], out[f"known_{name}_vals"] = raw, vals
    raw = random_blocks(66, (0,), 6, seed=0)
    out["iq2_xxs_raw"] = raw
    out["iq2_xxs_vals"] = np.array(ref_iq2_xxs(raw.tobytes(), grid), np.float64).astype(np.float32)
    raw = random_blocks(66, (64,), 7, seed=0)
    out["tq2_0_raw"] = raw
    out["tq2_0_vals"] = np.array(ref_tq2_0(raw.tobytes()), np.float64).astype(np.float32)
    w = ternary(3, 512, 256, seed=1)
    out["tq2_0_ternary_w"] = w.reshape(-1)
    out["tq2_0_ternary_raw"] = np.frombuffer(pack_tq2_0(w.reshape(-1).tolist()), np.uint8)
    out["iq2xxs_grid"] = np.array(grid, dtype=np.uint64)
    # added later with a generator of its own, so the fixtures above stay as they were
    raw, vals = known_q4_0(np.random.default_rng(20261202), 24)
    out["known_q4_0_raw"], out["known_q4_0_vals"] = raw, vals
    path = os.path.join(HERE, "formats.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
