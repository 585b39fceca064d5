"""The GGUF reader and writer on the CPU (ggufengine_amd.gguf): files built by the writer read back
exactly; malformed and hostile files raise GGUFError and nothing else (the reference's hardening
tests, tests/test_gguf_haertung.py, restated: unaligned, overlapping and truncated tensors, metadata
budgets, alignment, random corruption)."""
import os
import random
import struct

import numpy as np
import pytest

from ggufengine_amd import gguf as G
from ggufengine_amd.gguf_types import GGUFError


def _meta():
    return {
        "general.architecture": (G.T_STRING, "llama"),
        "general.name": (G.T_STRING, "probe ü"),
        "llama.block_count": (G.T_UINT32, 32),
        "a.u8": (G.T_UINT8, 255), "a.i8": (G.T_INT8, -128), "a.u16": (G.T_UINT16, 65535),
        "a.i16": (G.T_INT16, -32768), "a.i32": (G.T_INT32, -5), "a.f32": (G.T_FLOAT32, 0.5),
        "a.bool": (G.T_BOOL, True), "a.u64": (G.T_UINT64, 1 << 63), "a.i64": (G.T_INT64, -(1 << 40)),
        "a.f64": (G.T_FLOAT64, 1.25),
        "a.tokens": (G.T_ARRAY, (G.T_STRING, ["<s>", "</s>", "x"])),
        "a.scores": (G.T_ARRAY, (G.T_FLOAT32, [0.0, -1.5, 2.0])),
        "a.nested": (G.T_ARRAY, (G.T_ARRAY, [(G.T_UINT8, [1, 2]), (G.T_UINT8, [])])),
    }


def _tensors():
    rng = np.random.default_rng(5)
    return [
        ("blk.0.attn_norm.weight", (64,), 0, rng.standard_normal(64).astype(np.float32).tobytes()),
        ("blk.0.ffn_gate.weight", (512, 3), 12, rng.integers(0, 256, 3 * 2 * 144, dtype=np.uint8).tobytes()),
        ("blk.0.ffn_down.weight", (256, 2), 14, rng.integers(0, 256, 2 * 210, dtype=np.uint8).tobytes()),
        ("blk.0.attn_q.weight", (64, 2), 8, rng.integers(0, 256, 2 * 2 * 34, dtype=np.uint8).tobytes()),
    ]


@pytest.mark.parametrize("alignment", [32, 64, 8])
def test_round_trip(tmp_path, alignment):
    p = tmp_path / "m.gguf"
    meta = _meta()
    if alignment != G.DEFAULT_ALIGNMENT:
        meta["general.alignment"] = (G.T_UINT32, alignment)
    G.write_gguf(p, meta, _tensors(), alignment=alignment)
    with G.GGUFFile(p) as gf:
        assert gf.version == 3 and gf.alignment == alignment and gf.data_offset % alignment == 0
        assert gf.architecture == "llama" and gf.get("general.name") == "probe ü"
        assert gf.require("llama.block_count") == 32 and gf.get("missing", 7) == 7
        assert gf.metadata["a.i8"] == -128 and gf.metadata["a.u64"] == 1 << 63 and gf.metadata["a.bool"] is True
        assert gf.metadata["a.f32"] == 0.5 and gf.metadata["a.f64"] == 1.25
        assert gf.metadata["a.tokens"] == ["<s>", "</s>", "x"] and gf.metadata["a.scores"] == [0.0, -1.5, 2.0]
        assert gf.metadata["a.nested"] == [[1, 2], []]
        with pytest.raises(GGUFError):
            gf.require("missing")
        assert [t.name for t in gf.tensor_list] == [t[0] for t in _tensors()]
        for name, dims, typ, data in _tensors():
            ti = gf.tensors[name]
            assert ti.dims == dims and ti.shape == tuple(reversed(dims)) and ti.ggml_type == typ
            assert ti.n_bytes == len(data) and ti.offset % alignment == 0
            assert bytes(gf.tensor_bytes(ti)) == data
            buf = bytearray(100)
            got = b""
            for start in range(0, ti.n_bytes, 100):
                n = gf.read_into(ti, buf, start)
                got += bytes(buf[:n])
            assert got == data
        assert gf.tensors["blk.0.ffn_gate.weight"].type_name == "Q4_K"
        assert gf.tensors["blk.0.ffn_gate.weight"].n_elements == 1536


def _raw(tensors, meta=None, align=32, version=3, magic=b"GGUF"):
    """Byte-level GGUF (no checks, for malformed files): tensors = [(name, dims, type, offset, bytes)]."""
    meta = {"general.architecture": ("s", "t")} if meta is None else meta
    text = lambda s: struct.pack("<Q", len(s.encode())) + s.encode()
    h = magic + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, (kind, v) in (meta.items() if isinstance(meta, dict) else meta):
        h += text(k)
        if kind == "s":
            h += struct.pack("<I", G.T_STRING) + text(v)
        elif kind == "u32":
            h += struct.pack("<II", G.T_UINT32, v)
        elif kind == "arr_u8":
            h += struct.pack("<IIQ", G.T_ARRAY, G.T_UINT8, len(v)) + bytes(v)
        elif kind == "raw":
            h += v
    for name, dims, typ, off, _ in tensors:
        h += text(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        h += struct.pack("<IQ", typ, off)
    h += b"\0" * (-len(h) % align)
    data = bytearray(max((off + len(b) for *_, off, b in tensors), default=0))
    for *_, off, b in tensors:
        data[off:off + len(b)] = b
    return h + bytes(data)


def _open(tmp_path, content):
    p = tmp_path / "x.gguf"
    p.write_bytes(content)
    G.GGUFFile(p).close()


def test_valid_minimal(tmp_path):
    _open(tmp_path, _raw([("a", (8,), 0, 0, b"\1" * 32), ("b", (8,), 0, 32, b"\2" * 32)]))


T1 = [("a", (8,), 0, 0, b"\1" * 32)]
ARCH = ("general.architecture", ("s", "t"))
REJECTED = {   # case: (file bytes, words of the expected message)
    "magic": (lambda: _raw(T1, magic=b"GGUX"), "magic"),
    "version": (lambda: _raw(T1, version=1), "version"),
    "small": (lambda: b"GGUF" + b"\0" * 10, "too small"),
    "unaligned": (lambda: _raw([("a", (8,), 0, 4, b"\1" * 32)]), "multiple"),
    "overlap": (lambda: _raw([("a", (16,), 0, 0, b"\1" * 64), ("b", (8,), 0, 32, b"\2" * 32)]), "overlaps"),
    "past_end": (lambda: _raw(T1)[:-8], "past the end"),
    "align_24": (lambda: _raw(T1, [ARCH, ("general.alignment", ("u32", 24))], align=24), "power of two"),
    "align_4": (lambda: _raw(T1, [ARCH, ("general.alignment", ("u32", 4))], align=4), "power of two"),
    "dup_key": (lambda: _raw(T1, [ARCH, ("k", ("s", "a")), ("k", ("s", "b"))]), "twice"),
    "dup_tensor": (lambda: _raw([("a", (8,), 0, 0, b"\1" * 32), ("a", (8,), 0, 32, b"\2" * 32)]), "twice"),
    "unknown_type": (lambda: _raw([("a", (8,), 4, 0, b"\1" * 32)]), "unknown ggml type"),
    "ne0_blocks": (lambda: _raw([("a", (100,), 12, 0, b"\1" * 144)]), "whole number"),
    "dims_0": (lambda: _raw([("a", (), 0, 0, b"")]), "0 dimensions"),
    "dims_6": (lambda: _raw([("a", (1, 1, 1, 1, 1, 8), 0, 0, b"\1" * 32)]), "6 dimensions"),
    "zero_dim": (lambda: _raw([("a", (8, 0), 0, 0, b"")]), "dimension 0"),
    "nested_3": (lambda: _raw(T1, [ARCH, ("n", ("raw", struct.pack("<IIQ", G.T_ARRAY, G.T_ARRAY, 1)
                                               + struct.pack("<IQ", G.T_ARRAY, 1)
                                               + struct.pack("<IQ", G.T_UINT8, 0)))]), "nested"),
    "bad_utf8": (lambda: _raw(T1, [ARCH, ("s", ("raw", struct.pack("<IQ", G.T_STRING, 2) + b"\xff\xfe"))]), "UTF-8"),
    "unknown_vtype": (lambda: _raw(T1, [ARCH, ("s", ("raw", struct.pack("<I", 13)))]), "value type"),
    "empty_key": (lambda: _raw(T1, [ARCH, ("", ("s", "x"))]), "empty metadata key"),
    "empty_name": (lambda: _raw([("", (8,), 0, 0, b"\1" * 32)]), "empty tensor name"),
    "string_limit": (lambda: _raw(T1, [ARCH, ("s", ("raw", struct.pack("<IQ", G.T_STRING, G.MAX_STRING + 1)))]),
                     "at most"),
    "array_limit": (lambda: _raw(T1, [ARCH, ("s", ("raw", struct.pack("<IIQ", G.T_ARRAY, G.T_UINT8,
                                                                       G.MAX_ARRAY + 1)))]), "at most"),
}


@pytest.mark.parametrize("case", sorted(REJECTED))
def test_rejected(tmp_path, case):
    make, words = REJECTED[case]
    with pytest.raises(GGUFError, match=words):
        _open(tmp_path, make())


def test_metadata_budget(tmp_path, monkeypatch):
    monkeypatch.setattr(G, "MAX_META_ELEMENTS", 100)
    meta = {f"x.{i}": ("arr_u8", [1] * 40) for i in range(3)}     # 120 elements > 100
    meta["general.architecture"] = ("s", "t")
    with pytest.raises(GGUFError):
        _open(tmp_path, _raw([("a", (8,), 0, 0, b"\1" * 32)], meta))


def test_missing_architecture(tmp_path):
    p = tmp_path / "m.gguf"
    G.write_gguf(p, {"general.name": (G.T_STRING, "x")}, [("a", (8,), 0, b"\0" * 32)])
    with G.GGUFFile(p) as gf, pytest.raises(GGUFError):
        gf.architecture


def test_every_truncation_and_random_corruption(tmp_path):
    """Cut at every header position, and 300 seeded corruptions (bytes, truncation, huge counts):
    the reader accepts or raises GGUFError, nothing else."""
    base = _raw([("a", (32,), 0, 0, b"\1" * 128), ("b", (8, 4), 0, 128, b"\2" * 128)],
                {"general.name": ("s", "probe"), "x.n": ("u32", 3), "x.l": ("arr_u8", list(range(40))),
                 "general.architecture": ("s", "t")})
    _open(tmp_path, base)
    p = tmp_path / "f.gguf"
    for cut in range(0, len(base) - 256):
        p.write_bytes(base[:cut])
        with pytest.raises(GGUFError):
            G.GGUFFile(p).close()
    rng = random.Random(7)
    big = (0xFFFFFFFF, 0xFFFFFFFFFFFFFFFF, 1 << 40, 1 << 31, 0, 7)
    for _ in range(300):
        b = bytearray(base)
        kind = rng.randrange(4)
        if kind == 0:
            for _k in range(rng.randint(1, 8)):
                b[rng.randrange(len(b))] = rng.randrange(256)
        elif kind == 1:
            del b[rng.randrange(len(b)):]
        else:
            width = 8 if kind == 2 else 4
            i = rng.randrange(4, len(b) - width)
            b[i:i + width] = struct.pack("<Q" if width == 8 else "<I", rng.choice(big) & ((1 << 8 * width) - 1))
        p.write_bytes(bytes(b))
        try:
            G.GGUFFile(p).close()
        except GGUFError:
            pass


def test_wide_q2_0(tmp_path):
    """A Q2_0 tensor that only fits at 128 values per block (before the next tensor) is read as PQ2_0."""
    a = ("a", (512,), G.Q2_0, 0, b"\1" * 136)     # 64-value blocks: 144 bytes; 128-value: 136
    b = ("b", (8,), 0, 136, b"\2" * 32)
    p = tmp_path / "q.gguf"
    p.write_bytes(_raw([a, b], {"general.alignment": ("u32", 8), "general.architecture": ("s", "t")}, align=8))
    with G.GGUFFile(p) as gf:
        assert gf.tensors["a"].ggml_type == G.PQ2_0 and gf.tensors["a"].n_bytes == 136


def test_writer_checks(tmp_path):
    with pytest.raises(GGUFError):
        G.write_gguf(tmp_path / "w.gguf", {}, [("a", (8,), 0, b"\0" * 31)])      # wrong byte count
    with pytest.raises(GGUFError):
        G.write_gguf(tmp_path / "w.gguf", {}, [("a", (100,), 12, b"\0" * 144)])  # not whole blocks
