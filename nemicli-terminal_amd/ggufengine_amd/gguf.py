"""
GGUF files for this library: a checked reader with the reference's API (`GGUFFile`, `TensorInfo`,
`GGUFError`, the value-type ids and limits; contract of ggufengine/gguf.py:171-369), the upload of a
tensor's raw block bytes to the GPU (the reference's weight loader, models/common.py:83-116: large file
reads into a ring of pinned buffers, copies on a copy stream), and a writer (the tests and synthetic
models build their files with it).

Every byte of the file is untrusted.  Reading happens in two stages: `_scan` walks the header through one
bounds-checked cursor (every length and count bounded before use, metadata budgets counted), then
`_place` turns the tensor records into TensorInfos and checks them in one sweep in offset order
(aligned, inside the data section, no overlap).  Any violation raises GGUFError and nothing else, and no
allocation is sized from an unchecked number.  Tensor bytes are read-only views of a memory map or
positional reads into a caller's buffer.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from typing import Any, Dict, List, NamedTuple, Optional, Sequence, Tuple

from .gguf_types import GGML_ALL_TYPES, GGUFError

GGUF_MAGIC = b"GGUF"
SUPPORTED_VERSIONS = (2, 3)

# limits on what a header may declare (the reference's, gguf.py:35-44)
MAX_TENSORS = 1 << 18
MAX_KV = 1 << 16
MAX_STRING = 16 << 20
MAX_ARRAY = 1 << 24
MAX_NAME = 512
MAX_DIMS = 5
MAX_ELEMENTS = 1 << 40
MAX_META_ELEMENTS = 1 << 23     # all array elements of all metadata values together
MAX_META_BYTES = 512 << 20      # all string bytes of all metadata values together
DEFAULT_ALIGNMENT = 32
MIN_ALIGNMENT, MAX_ALIGNMENT = 8, 1 << 16

# metadata value types (GGUF specification)
(T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL,
 T_STRING, T_ARRAY, T_UINT64, T_INT64, T_FLOAT64) = range(13)
_FIXED = {T_UINT8: "B", T_INT8: "b", T_UINT16: "H", T_INT16: "h", T_UINT32: "I", T_INT32: "i",
          T_FLOAT32: "f", T_BOOL: "?", T_UINT64: "Q", T_INT64: "q", T_FLOAT64: "d"}

GGML_TYPES = GGML_ALL_TYPES
Q2_0, PQ2_0 = 42, 142


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dims: Tuple[int, ...]      # GGUF order: dims[0] (ne0) varies fastest
    ggml_type: int
    offset: int                # from the start of the data section
    n_elements: int
    n_bytes: int

    @property
    def type_name(self) -> str:
        return GGML_TYPES[self.ggml_type][0]

    @property
    def shape(self) -> Tuple[int, ...]:
        """Row-major shape (numpy / torch order)."""
        return tuple(reversed(self.dims))


def tensor_info(name: str, dims: Sequence[int], ggml_type: int, offset: int) -> TensorInfo:
    """A checked TensorInfo: known type, 1..MAX_DIMS positive dims, element count bounded, ne0 whole
    blocks."""
    spec = GGML_TYPES.get(ggml_type)
    if spec is None:
        raise GGUFError(f"tensor {name!r}: unknown ggml type {ggml_type}")
    dims = tuple(int(d) for d in dims)
    if not 1 <= len(dims) <= MAX_DIMS:
        raise GGUFError(f"tensor {name!r}: {len(dims)} dimensions")
    count = 1
    for d in dims:
        if d < 1:
            raise GGUFError(f"tensor {name!r}: dimension {d} in {dims}")
        count *= d
        if count > MAX_ELEMENTS:
            raise GGUFError(f"tensor {name!r}: more than {MAX_ELEMENTS} elements")
    _, block, size = spec
    if dims[0] % block:
        raise GGUFError(f"tensor {name!r}: ne0 = {dims[0]} is not a whole number of {block}-value blocks")
    return TensorInfo(name, dims, ggml_type, int(offset), count, count // block * size)


class _Header:
    """Little-endian reads from the file's header region; every read checks the remaining length, and
    the metadata budgets (array elements, string bytes) are counted here."""

    def __init__(self, buf, end: int):
        self.buf, self.pos, self.end = buf, 0, end
        self.elements = 0
        self.text_bytes = 0

    def take(self, n: int) -> int:
        """Advance over n bytes, returning where they start."""
        if n < 0 or n > self.end - self.pos:
            raise GGUFError(f"truncated file: {n} bytes needed at offset {self.pos}, {self.end - self.pos} left")
        at = self.pos
        self.pos += n
        return at

    def fixed(self, code: str):
        return struct.unpack_from("<" + code, self.buf, self.take(struct.calcsize("<" + code)))[0]

    def text(self, limit: int) -> str:
        n = self.fixed("Q")
        if n > limit:
            raise GGUFError(f"string of {n} bytes (at most {limit})")
        self.text_bytes += n
        if self.text_bytes > MAX_META_BYTES:
            raise GGUFError("metadata strings exceed their total budget")
        at = self.take(n)
        try:
            return bytes(self.buf[at:at + n]).decode("utf-8")
        except UnicodeDecodeError as exc:
            raise GGUFError(f"string at offset {at} is not UTF-8: {exc}") from None

    def value(self, vtype: int, level: int = 0):
        if vtype in _FIXED:
            return self.fixed(_FIXED[vtype])
        if vtype == T_STRING:
            return self.text(MAX_STRING)
        if vtype != T_ARRAY:
            raise GGUFError(f"unknown metadata value type {vtype}")
        if level > 1:
            raise GGUFError("arrays nested more than one level deep")
        etype, n = self.fixed("I"), self.fixed("Q")
        if n > MAX_ARRAY:
            raise GGUFError(f"array of {n} elements (at most {MAX_ARRAY})")
        self.elements += n
        if self.elements > MAX_META_ELEMENTS:
            raise GGUFError("metadata arrays exceed their total budget")
        if etype in _FIXED:
            code = _FIXED[etype]
            at = self.take(n * struct.calcsize("<" + code))
            return list(struct.unpack_from(f"<{n}{code}", self.buf, at))
        if etype in (T_STRING, T_ARRAY):
            return [self.value(etype, level + 1) for _ in range(n)]
        raise GGUFError(f"unknown array element type {etype}")


class _Scan(NamedTuple):
    version: int
    metadata: Dict[str, Any]
    records: List[Tuple[str, Tuple[int, ...], int, int]]   # name, dims, ggml type, offset
    end: int                                                 # first byte after the tensor records


def _scan(buf, size: int) -> _Scan:
    """The header: magic, version, counts, metadata, tensor records, every read bounded."""
    h = _Header(buf, size)
    at = h.take(4)
    if bytes(buf[at:at + 4]) != GGUF_MAGIC:
        raise GGUFError("bad magic (not a GGUF file)")
    version = h.fixed("I")
    if version not in SUPPORTED_VERSIONS:
        raise GGUFError(f"GGUF version {version} (supported: {SUPPORTED_VERSIONS})")
    n_tensors, n_kv = h.fixed("Q"), h.fixed("Q")
    if n_tensors > MAX_TENSORS or n_kv > MAX_KV:
        raise GGUFError(f"{n_tensors} tensors / {n_kv} metadata entries exceed the limits")
    meta: Dict[str, Any] = {}
    for _ in range(n_kv):
        key = h.text(MAX_NAME)
        if not key:
            raise GGUFError("empty metadata key")
        if key in meta:
            raise GGUFError(f"metadata key {key!r} appears twice")
        meta[key] = h.value(h.fixed("I"))
    records = []
    for _ in range(n_tensors):
        name = h.text(MAX_NAME)
        if not name:
            raise GGUFError("empty tensor name")
        n_dims = h.fixed("I")
        if not 1 <= n_dims <= MAX_DIMS:
            raise GGUFError(f"tensor {name!r}: {n_dims} dimensions")
        dims = tuple(h.fixed("Q") for _ in range(n_dims))
        records.append((name, dims, h.fixed("I"), h.fixed("Q")))
    return _Scan(version, meta, records, h.pos)


def _alignment(meta: Dict[str, Any]) -> int:
    a = meta.get("general.alignment", DEFAULT_ALIGNMENT)
    if type(a) is not int or not MIN_ALIGNMENT <= a <= MAX_ALIGNMENT or a & (a - 1):
        raise GGUFError(f"general.alignment {a!r} is not a power of two in [{MIN_ALIGNMENT}, {MAX_ALIGNMENT}]")
    return a


def _place(records, align: int, data_size: int) -> List[TensorInfo]:
    """TensorInfos in file order, after one sweep in offset order that checks alignment, extent and
    overlap and reads a 64-value Q2_0 tensor that only fits the room before the next tensor with
    128-value blocks as PQ2_0 (a fork's older files)."""
    infos = [tensor_info(*r) for r in records]
    seen = set()
    for ti in infos:
        if ti.name in seen:
            raise GGUFError(f"tensor name {ti.name!r} appears twice")
        seen.add(ti.name)
    order = sorted(range(len(infos)), key=lambda i: infos[i].offset)
    end_prev = 0
    for pos, i in enumerate(order):
        ti = infos[i]
        room = (infos[order[pos + 1]].offset if pos + 1 < len(order) else data_size) - ti.offset
        if ti.ggml_type == Q2_0 and ti.n_bytes > room:
            wide = tensor_info(ti.name, ti.dims, PQ2_0, ti.offset)
            if wide.n_bytes <= room:
                ti = infos[i] = wide
        if ti.offset % align:
            raise GGUFError(f"tensor {ti.name!r}: offset {ti.offset} not a multiple of {align}")
        if ti.offset > data_size or ti.n_bytes > data_size - ti.offset:
            raise GGUFError(f"tensor {ti.name!r} ({ti.n_bytes} bytes at {ti.offset}) runs past the end of "
                            f"the data section ({data_size} bytes)")
        if ti.offset < end_prev:
            raise GGUFError(f"tensor {ti.name!r} overlaps the tensor before it")
        end_prev = ti.offset + ti.n_bytes
    return infos


class GGUFFile:
    """A checked, read-only GGUF file (version 2 or 3): `version`, `alignment`, `metadata`, `tensors`
    (by name), `tensor_list` (file order), `data_offset`, `file_size`.  Tensor bytes come as read-only
    views of a memory map (`tensor_bytes`) or as positional reads into a caller's buffer (`read_into`,
    safe from several threads: no shared file position)."""

    def __init__(self, path):
        self.path = os.fspath(path)
        self._mm = None
        self._fd = os.open(self.path, os.O_RDONLY | getattr(os, "O_CLOEXEC", 0))
        try:
            self.file_size = os.fstat(self._fd).st_size
            if self.file_size < 24:
                raise GGUFError("file too small to be GGUF")
            self._mm = mmap.mmap(self._fd, 0, access=mmap.ACCESS_READ)
            head = _scan(self._mm, self.file_size)
            self.version, self.metadata = head.version, head.metadata
            self.alignment = _alignment(self.metadata)
            self.data_offset = -(-head.end // self.alignment) * self.alignment
            if self.data_offset > self.file_size:
                raise GGUFError("data section starts past the end of the file")
            self.tensor_list = _place(head.records, self.alignment, self.file_size - self.data_offset)
            self.tensors: Dict[str, TensorInfo] = {ti.name: ti for ti in self.tensor_list}
        except BaseException:
            self.close()
            raise

    # ---- metadata ------------------------------------------------------------------------------
    def get(self, key: str, default=None):
        return self.metadata.get(key, default)

    def require(self, key: str):
        try:
            return self.metadata[key]
        except KeyError:
            raise GGUFError(f"required metadata key {key!r} missing") from None

    @property
    def architecture(self) -> str:
        arch = self.metadata.get("general.architecture")
        if isinstance(arch, str):
            return arch
        raise GGUFError("general.architecture missing or not a string")

    # ---- tensor bytes --------------------------------------------------------------------------
    def _span(self, ti: TensorInfo, start: int, n: int) -> int:
        pos = self.data_offset + ti.offset + start
        if pos + n > self.file_size:
            raise GGUFError("tensor out of bounds")
        return pos

    def tensor_bytes(self, ti: TensorInfo) -> memoryview:
        """Read-only view of the tensor's bytes in the memory map (no copy)."""
        pos = self._span(ti, 0, ti.n_bytes)
        return memoryview(self._mm)[pos:pos + ti.n_bytes]

    def read_into(self, ti: TensorInfo, out, start: int = 0) -> int:
        """Read tensor bytes [start, start + len(out)) into the writable buffer `out` with positional
        reads (large sequential requests instead of page faults on the map), stopping at the tensor's
        end; returns the number of bytes read."""
        if not 0 <= start <= ti.n_bytes:
            raise GGUFError("read outside the tensor")
        dst = memoryview(out).cast("B")
        n = min(dst.nbytes, ti.n_bytes - start)
        pos = self._span(ti, start, n)
        done = 0
        while done < n:
            got = os.preadv(self._fd, [dst[done:n]], pos + done)
            if got <= 0:
                raise GGUFError("unexpected end of file")
            done += got
        return n

    def close(self) -> None:
        mm, self._mm = self._mm, None
        if mm is not None:
            try:
                mm.close()
            except BufferError:        # a tensor still views the map; it is unmapped with the last view
                pass
        fd, self._fd = self._fd, -1
        if fd >= 0:
            os.close(fd)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ---- upload to the GPU --------------------------------------------------------------------------

class Uploader:
    """Raw tensor bytes onto a device (models/common.py:83-116 `_roh`): to the GPU as reads of up to
    CHUNK bytes into a ring of BUFFERS pinned host buffers, each copied on a copy stream while the
    next is read, so file reads overlap the transfers; on the CPU a zero-copy view of the map.  The
    compute stream waits for the copies before the returned tensor is used there."""

    CHUNK = 32 << 20
    BUFFERS = 4

    def __init__(self, device):
        import torch
        self.device = torch.device(device)
        self._ring = None
        self._pos = 0
        self._stream = None

    def __call__(self, gf: GGUFFile, ti: TensorInfo):
        import torch
        if self.device.type != "cuda":
            import warnings
            with warnings.catch_warnings():    # the map is read-only; torch warns about that
                warnings.simplefilter("ignore")
                return torch.frombuffer(gf.tensor_bytes(ti), dtype=torch.uint8)
        if self._ring is None:
            self._ring = [[torch.empty(self.CHUNK, dtype=torch.uint8, pin_memory=True), None]
                          for _ in range(self.BUFFERS)]
            self._stream = torch.cuda.Stream(self.device)
        out = torch.empty(ti.n_bytes, dtype=torch.uint8, device=self.device)
        # `out` may reuse memory that work queued on the compute stream still reads
        self._stream.wait_stream(torch.cuda.current_stream(self.device))
        for start in range(0, ti.n_bytes, self.CHUNK):
            slot = self._ring[self._pos]
            self._pos = (self._pos + 1) % len(self._ring)
            if slot[1] is not None:
                slot[1].synchronize()          # its previous copy must be done before it is refilled
            n = gf.read_into(ti, slot[0].numpy(), start)
            with torch.cuda.stream(self._stream):
                out[start:start + n].copy_(slot[0][:n], non_blocking=True)
                slot[1] = torch.cuda.Event()
                slot[1].record(self._stream)
        out.record_stream(self._stream)
        torch.cuda.current_stream(self.device).wait_stream(self._stream)
        return out


def load_raw(gf: GGUFFile, name: str, device, uploader: Optional[Uploader] = None):
    """The named tensor's block bytes on `device` as uint8 (one Uploader per device is reused when
    given)."""
    ti = gf.tensors.get(name)
    if ti is None:
        raise GGUFError(f"no tensor {name!r} in {gf.path}")
    return (uploader or Uploader(device))(gf, ti)


# ---- writer -------------------------------------------------------------------------------------

def _enc_text(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _enc_value(vtype: int, value) -> bytes:
    if vtype in _FIXED:
        return struct.pack("<" + _FIXED[vtype], value)
    if vtype == T_STRING:
        return _enc_text(value)
    if vtype == T_ARRAY:
        etype, items = value
        body = b"".join(_enc_value(etype, v) for v in items)
        return struct.pack("<IQ", etype, len(items)) + body
    raise GGUFError(f"unknown metadata value type {vtype}")


def write_gguf(path, metadata: Dict[str, Tuple[int, Any]], tensors: Sequence[Tuple[str, Sequence[int], int, bytes]],
               alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """Write a GGUF file.  metadata: key -> (value type, value); an array value is
    (T_ARRAY, (element type, [elements])).  tensors: (name, dims in GGUF order (ne0 first), ggml
    type, block bytes), placed back to back at `alignment`.  A `general.alignment` entry other than
    `alignment` is the caller's to keep consistent."""
    head = GGUF_MAGIC + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, (vtype, value) in metadata.items():
        head += _enc_text(key) + struct.pack("<I", vtype) + _enc_value(vtype, value)
    offset, placed = 0, []
    for name, dims, ggml_type, data in tensors:
        ti = tensor_info(name, dims, ggml_type, offset)
        if len(data) != ti.n_bytes:
            raise GGUFError(f"tensor {name!r}: {len(data)} bytes given, {ti.n_bytes} expected")
        head += _enc_text(name) + struct.pack("<I", len(ti.dims))
        head += b"".join(struct.pack("<Q", d) for d in ti.dims) + struct.pack("<IQ", ggml_type, offset)
        placed.append((offset, data))
        offset = -(-(offset + ti.n_bytes) // alignment) * alignment
    head += b"\0" * (-len(head) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for off, data in placed:
            f.write(b"\0" * (off - pos))
            f.write(data)
            pos = off + len(data)
