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
