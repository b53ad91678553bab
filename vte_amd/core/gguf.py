"""GGUF model files: reader (memory-mapped, zero-copy tensor views) and a
small writer.

Reference behaviour followed:
* header, metadata skipping and tensor-info parsing of
  vte/compiler/gguf_parser.py:15-86 and vte/compiler/sanitizer.py:110-200
  (magic ``GGUF``, version, tensor count, metadata count; 64-bit string
  lengths with a 64 KiB cap; value types 0..12 with arrays; dims stored
  innermost-first and reported reversed as (rows, cols));
* tensor data starts at the first multiple of the alignment after the tensor
  infos (gguf_parser.py:54-57; the alignment is ``general.alignment`` when
  the file sets it, else 32) and every tensor must lie inside the file
  (gguf_parser.py:107-122);
* tied embeddings: ``output.weight`` absent, or at the same offset as
  ``token_embd.weight`` (gguf_parser.py:124-133);
* block sizes of the GGML types (the table ggml_types.block_size_bytes reads
  from the ``gguf`` package, gguf_parser.py:87-105), restated here from the
  published GGML format (that package is not installed).

The reader never copies tensor bytes: ``tensor(name)`` is a numpy view of the
memory map, so uploading a weight is one host-to-device copy from the page
cache.  Errors raise ``HIPSafetyError`` as the reference does.
"""
from __future__ import annotations

import math
import mmap
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from ..bridge.hip_runtime import HIPSafetyError

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32
MAX_STRING = 65536

# GGML tensor types: id -> (name, elements per block, bytes per block)
GGML_TYPES = {
    0: ("f32", 1, 4),
    1: ("f16", 1, 2),
    2: ("q4_0", 32, 18),
    3: ("q4_1", 32, 20),
    6: ("q5_0", 32, 22),
    7: ("q5_1", 32, 24),
    8: ("q8_0", 32, 34),
    9: ("q8_1", 32, 36),
    10: ("q2_k", 256, 84),
    11: ("q3_k", 256, 110),
    12: ("q4_k", 256, 144),
    13: ("q5_k", 256, 176),
    14: ("q6_k", 256, 210),
    15: ("q8_k", 256, 292),
    30: ("bf16", 1, 2),
}
GGML_TYPE_ID = {v[0]: k for k, v in GGML_TYPES.items()}

# metadata value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


def tensor_nbytes(type_id: int, n_elements: int) -> int:
    """Bytes of a tensor of ``n_elements`` of a GGML type (whole blocks only)."""
    if type_id not in GGML_TYPES:
        raise HIPSafetyError(f"GGUF: unknown tensor type {type_id}")
    _, blk, nb = GGML_TYPES[type_id]
    if n_elements % blk:
        raise HIPSafetyError(f"GGUF: {n_elements} elements is not a whole number of {blk}-element blocks")
    return n_elements // blk * nb


@dataclass
class TensorInfo:
    name: str
    shape: tuple          # reversed GGML dims: (rows, cols) for a matrix
    type_id: int
    offset: int           # absolute file offset of the first byte
    nbytes: int
    is_tied: bool = False
    tied_to: str = ""

    @property
    def type_name(self) -> str:
        return GGML_TYPES[self.type_id][0]

    @property
    def n_elements(self) -> int:
        return math.prod(self.shape)


@dataclass
class GGUFHeader:
    version: int
    tensor_count: int
    kv_count: int
    metadata: dict = field(default_factory=dict)


class _Cursor:
    """Bounds-checked little-endian reads over the mapped file."""

    def __init__(self, buf, size: int):
        self.buf, self.size, self.pos = buf, size, 0

    def take(self, n: int) -> bytes:
        if n < 0 or self.pos + n > self.size:
            raise HIPSafetyError(f"GGUF: unexpected end of file at byte {self.pos} (need {n})")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.unpack("<Q")
        if n > MAX_STRING:
            raise HIPSafetyError(f"GGUF: string of {n} bytes exceeds {MAX_STRING}")
        return self.take(n).decode("utf-8", errors="replace")

    def value(self, vtype: int):
        if vtype in _SCALAR:
            return self.unpack(_SCALAR[vtype])
        if vtype == T_STR:
            return self.string()
        if vtype == T_ARR:
            atype, n = self.unpack("<I"), self.unpack("<Q")
            if atype in _SCALAR and atype != T_BOOL:
                fmt = _SCALAR[atype]
                arr = np.frombuffer(self.take(n * struct.calcsize(fmt)), dtype=np.dtype(fmt))
                return arr.copy()
            return [self.value(atype) for _ in range(n)]
        raise HIPSafetyError(f"GGUF: unsupported metadata value type {vtype}")


class GGUFReader:
    """Parses a GGUF file and exposes its metadata and tensor views."""

    def __init__(self, path):
        self.path = Path(path)
        self._f = open(self.path, "rb")
        self.file_size = self.path.stat().st_size
        if self.file_size < 24:
            self._f.close()
            raise HIPSafetyError(f"GGUF: {self.path} is too small ({self.file_size} bytes)")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    def _parse(self) -> None:
        c = _Cursor(self._mm, self.file_size)
        if c.take(4) != GGUF_MAGIC:
            raise HIPSafetyError(f"GGUF: bad magic in {self.path}")
        version = c.unpack("<I")
        if version not in (2, 3):
            raise HIPSafetyError(f"GGUF: unsupported version {version}")
        n_tensors, n_kv = c.unpack("<Q"), c.unpack("<Q")
        meta = {}
        for _ in range(n_kv):
            key = c.string()
            meta[key] = c.value(c.unpack("<I"))
        self.header = GGUFHeader(version, n_tensors, n_kv, meta)
        raw = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.unpack("<I")
            if nd < 1 or nd > 4:
                raise HIPSafetyError(f"GGUF: tensor {name} has {nd} dimensions")
            dims = [c.unpack("<Q") for _ in range(nd)]
            type_id, rel = c.unpack("<I"), c.unpack("<Q")
            raw.append((name, tuple(reversed(dims)), type_id, rel))
        align = int(meta.get("general.alignment", DEFAULT_ALIGNMENT))
        if align <= 0 or align & (align - 1):
            raise HIPSafetyError(f"GGUF: alignment {align} is not a power of two")
        self.alignment = align
        self.data_offset = -(-c.pos // align) * align
        self.tensors: dict[str, TensorInfo] = {}
        for name, shape, type_id, rel in raw:
            if name in self.tensors:
                raise HIPSafetyError(f"GGUF: duplicate tensor {name}")
            nbytes = tensor_nbytes(type_id, math.prod(shape))
            off = self.data_offset + rel
            if rel % align:
                raise HIPSafetyError(f"GGUF: tensor {name} offset {rel} is not {align}-aligned")
            if off + nbytes > self.file_size:
                raise HIPSafetyError(f"GGUF: tensor {name} (offset {off}, {nbytes} B) runs past the end of the file "
                                     f"({self.file_size} B)")
            self.tensors[name] = TensorInfo(name, shape, type_id, off, nbytes)
        emb, out = self.tensors.get("token_embd.weight"), self.tensors.get("output.weight")
        if emb is not None and out is not None and emb.offset == out.offset:
            out.is_tied, out.tied_to = True, emb.name

    @property
    def metadata(self) -> dict:
        return self.header.metadata

    def tensor(self, name: str) -> np.ndarray:
        """Zero-copy view of a tensor: uint8 [rows, row_bytes] for block types,
        float32 / float16 / uint16 (bf16) [shape] for plain types."""
        if name not in self.tensors:
            raise KeyError(name)
        t = self.tensors[name]
        buf = np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset)
        if t.type_id == 0:
            return buf.view(np.float32).reshape(t.shape)
        if t.type_id == 1:
            return buf.view(np.float16).reshape(t.shape)
        if t.type_id == 30:
            return buf.view(np.uint16).reshape(t.shape)
        rows = math.prod(t.shape[:-1]) if len(t.shape) > 1 else 1
        return buf.reshape(rows, t.nbytes // rows)

    def close(self) -> None:
        mm, self._mm = getattr(self, "_mm", None), None
        if mm is not None:
            try:
                mm.close()
            except BufferError:  # views still alive: the map closes when they are released
                pass
        if getattr(self, "_f", None) is not None:
            self._f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(v) -> tuple[int, bytes]:
    if isinstance(v, bool):
        return T_BOOL, struct.pack("<?", v)
    if isinstance(v, int):
        return (T_U32, struct.pack("<I", v)) if 0 <= v < 2 ** 32 else (T_I64, struct.pack("<q", v))
    if isinstance(v, float):
        return T_F32, struct.pack("<f", v)
    if isinstance(v, str):
        return T_STR, _pack_string(v)
    if isinstance(v, np.ndarray):
        codes = {np.dtype("<i4"): T_I32, np.dtype("<f4"): T_F32, np.dtype("<u4"): T_U32, np.dtype("<u1"): T_U8,
                 np.dtype("<i8"): T_I64, np.dtype("<f8"): T_F64}
        at = codes[v.dtype]
        return T_ARR, struct.pack("<IQ", at, v.size) + np.ascontiguousarray(v).tobytes()
    if isinstance(v, (list, tuple)):
        if not v:
            return T_ARR, struct.pack("<IQ", T_STR, 0)
        items = [_pack_value(x) for x in v]
        if len({t for t, _ in items}) != 1:
            raise ValueError("GGUF arrays hold one value type")
        return T_ARR, struct.pack("<IQ", items[0][0], len(items)) + b"".join(b for _, b in items)
    raise TypeError(f"cannot store {type(v).__name__} in GGUF metadata")


def write_gguf(path, metadata: dict, tensors: list, alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file.  ``tensors``: (name, type_name, shape, data) with
    shape in (rows, cols) order and data the raw bytes (uint8 array or bytes)
    or a float32 / float16 array for those types."""
    meta = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        meta["general.alignment"] = alignment
    head = bytearray(GGUF_MAGIC + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for k, v in meta.items():
        t, b = _pack_value(v)
        head += _pack_string(k) + struct.pack("<I", t) + b
    blobs, rel = [], 0
    for name, tname, shape, data in tensors:
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes() if isinstance(data, np.ndarray) \
            else bytes(data)
        tid = GGML_TYPE_ID[tname]
        if len(raw) != tensor_nbytes(tid, math.prod(shape)):
            raise ValueError(f"{name}: {len(raw)} bytes for {tname} {shape}")
        dims = list(reversed(shape))
        head += _pack_string(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", tid, rel)
        blobs.append((rel, raw))
        rel = -(-(rel + len(raw)) // alignment) * alignment
    data_off = -(-len(head) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_off - len(head)))
        for r, raw in blobs:
            f.seek(data_off + r)
            f.write(raw)
        f.truncate(data_off + rel)
