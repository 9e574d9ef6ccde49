"""Minimal GGUF v2/v3 reader: header, metadata, tensor table, zero-copy tensor
bytes and per-expert slices.

Follows the container rules of gguf.zig's `Gguf.parse` (gguf.zig:587-657),
`tensorBytes` (gguf.zig:425-436) and `expertBytes` (gguf.zig:482-488): little-
endian, `general.alignment` (default 32, power of two) aligns the data section,
the expert axis of a stacked `*_exps` tensor is the slowest one.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass

from . import workloads as W

MAGIC = 0x46554747  # "GGUF"


class GgufError(Exception):
    """Carries the reference's error name (NotGgufFile, TruncatedFile, ...)."""


@dataclass
class Tensor:
    name: str
    dims: tuple
    ttype: int
    offset: int

    def elem_count(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def byte_size(self):
        if self.ttype not in W.BLOCK:
            return None
        epb, bpb = W.BLOCK[self.ttype]
        n = self.elem_count()
        return None if n % epb else n // epb * bpb


_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class _Cursor:
    def __init__(self, data):
        self.d, self.p = data, 0

    def take(self, fmt):
        n = struct.calcsize(fmt)
        if self.p + n > len(self.d):
            raise GgufError("TruncatedFile")
        v = struct.unpack_from(fmt, self.d, self.p)[0]
        self.p += n
        return v

    def string(self):
        n = self.take("<Q")
        if self.p + n > len(self.d):
            raise GgufError("TruncatedFile")
        s = bytes(self.d[self.p:self.p + n]).decode("utf-8", "replace")
        self.p += n
        return s

    def value(self, vt):
        if vt in _SCALAR:
            return self.take(_SCALAR[vt])
        if vt == 8:
            return self.string()
        if vt == 9:
            et = self.take("<I")
            n = self.take("<Q")
            if n > len(self.d) - self.p + 1:
                raise GgufError("TruncatedFile")
            return [self.value(et) for _ in range(n)]
        raise GgufError("InvalidMetadata")


class Gguf:
    def __init__(self, data):
        self.data = data
        c = _Cursor(data)
        if c.take("<I") != MAGIC:
            raise GgufError("NotGgufFile")
        self.version = c.take("<I")
        if self.version not in (2, 3):
            raise GgufError("UnsupportedVersion")
        n_tensors, n_kv = c.take("<Q"), c.take("<Q")
        if n_tensors > len(data) or n_kv > len(data):
            raise GgufError("TooManyTensors")
        self.kv = {}
        for _ in range(n_kv):
            key = c.string()
            vt = c.take("<I")
            val = c.value(vt)
            self.kv.setdefault(key, val)  # first occurrence wins
        self.alignment = 32
        if "general.alignment" in self.kv:
            a = self.kv["general.alignment"]
            if not isinstance(a, int) or a <= 0 or a > (1 << 24) or a & (a - 1):
                raise GgufError("InvalidMetadata")
            self.alignment = a
        self.tensors = {}
        self.order = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.take("<I")
            if nd == 0 or nd > 8:
                raise GgufError("InvalidTensorShape")
            dims = tuple(c.take("<Q") for _ in range(nd))
            tt = c.take("<I")
            off = c.take("<Q")
            t = Tensor(name, dims, tt, off)
            self.tensors.setdefault(name, t)
            self.order.append(t)
        self.data_offset = (c.p + self.alignment - 1) // self.alignment * self.alignment
        if self.data_offset > len(data):
            raise GgufError("TruncatedFile")

    @classmethod
    def load(cls, path: str) -> "Gguf":
        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        return cls(memoryview(mm))

    @classmethod
    def from_bytes(cls, b: bytes) -> "Gguf":
        return cls(memoryview(bytes(b)))

    def arch(self):
        return self.kv.get("general.architecture")

    def tensor(self, name: str) -> Tensor | None:
        return self.tensors.get(name)

    def tensor_bytes(self, t: Tensor) -> memoryview:
        if t.ttype not in W.BLOCK:
            raise GgufError("UnsupportedType")
        n = t.byte_size()
        if n is None:
            raise GgufError("InvalidTensorShape")
        start = self.data_offset + t.offset
        if start + n > len(self.data):
            raise GgufError("TensorDataOutOfRange")
        return self.data[start:start + n]

    def expert_bytes(self, name: str, expert: int, n_experts: int) -> memoryview:
        if n_experts == 0 or expert >= n_experts:
            raise GgufError("InvalidTensorShape")
        t = self.tensor(name)
        if t is None:
            raise GgufError("TensorNotFound")
        allb = self.tensor_bytes(t)
        if len(allb) % n_experts:
            raise GgufError("InvalidTensorShape")
        per = len(allb) // n_experts
        return allb[expert * per:(expert + 1) * per]


# ------------------------------------------------------------------ writing

# metadata value types (gguf.zig ValueType)
U8, I8, U16, I16, U32, I32, F32V, BOOL, STR, ARR, U64, I64, F64V = range(13)


def _pack_value(vt: int, v) -> bytes:
    if vt in _SCALAR:
        return struct.pack(_SCALAR[vt], v)
    if vt == STR:
        b = v.encode()
        return struct.pack("<Q", len(b)) + b
    raise GgufError("InvalidMetadata")


def _typed(v):
    """(value type, value) of a metadata entry: explicit (type, value) pairs pass
    through; Python ints are u32 (u64 when larger), floats f32, strings and bools
    as themselves, lists arrays of the first element's type."""
    if isinstance(v, tuple) and len(v) == 2 and isinstance(v[0], int) and not isinstance(v[0], bool):
        return v
    if isinstance(v, bool):
        return BOOL, v
    if isinstance(v, int):
        return (U32, v) if 0 <= v < 2 ** 32 else (U64 if v >= 0 else I64, v)
    if isinstance(v, float):
        return F32V, v
    if isinstance(v, str):
        return STR, v
    if isinstance(v, list):
        return ARR, v
    raise GgufError("InvalidMetadata")


def write(metadata: dict, tensors: list, alignment: int = 32, version: int = 3) -> bytes:
    """A GGUF v2/v3 image (the layout Gguf.parse reads, gguf.zig:587-657): metadata
    in dict order, then `tensors` = [(name, dims fastest-first, ggml type, payload
    bytes)], each payload at an `alignment`-aligned offset of the data section."""
    out = [struct.pack("<IIQQ", MAGIC, version, len(tensors), len(metadata))]
    for key, v in metadata.items():
        vt, val = _typed(v)
        kb = key.encode()
        out.append(struct.pack("<Q", len(kb)) + kb + struct.pack("<I", vt))
        if vt == ARR:
            et, _ = _typed(val[0]) if val else (U32, 0)
            out.append(struct.pack("<IQ", et, len(val)) + b"".join(_pack_value(et, x) for x in val))
        else:
            out.append(_pack_value(vt, val))
    offs, off = [], 0
    for name, dims, tt, payload in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(payload)
    for (name, dims, tt, payload), o in zip(tensors, offs):
        nb = name.encode()
        out.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)))
        out.append(b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", tt, o))
    head = b"".join(out)
    data_off = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(off)
    for (_, _, _, payload), o in zip(tensors, offs):
        body[o:o + len(payload)] = bytes(payload)
    return head + b"\0" * (data_off - len(head)) + bytes(body)
