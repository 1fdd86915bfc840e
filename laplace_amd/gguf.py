"""GGUF v2/v3 reader and device residency for its weights.

Parses a GGUF file as the reference's ``GGUFContext::open`` does
(src/gguf.cpp:209-389): magic "GGUF", version 2 or 3, tensor and key/value
counts, the typed metadata values (scalars, strings and one level of arrays,
src/gguf.cpp:73-190), the tensor infos (name, up to 4 dims, type, offset),
``general.alignment`` (u32 or u64, default 32) and the data section at the
next multiple of it; every tensor's bytes (``Tensor::nbytes``,
src/tensor.h:141-157) must lie inside the file. The file is memory-mapped;
tensors are zero-copy numpy views into the mapping.

:meth:`GGUFFile.register` copies the data section to the GPU once
(``lp_register_weights``, the counterpart of ``matmul_register_weights`` /
``metal_register_weights``, src/matmul.cpp:446-448, src/metal.mm:552-621):
afterwards the host-pointer entries (``lp_gemm`` ...) resolve any weight
pointer inside the mapping to its device copy instead of uploading it.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib
from .matmul import Tensor, bytes_per_block, elements_per_block

GGUF_MAGIC = 0x46554747          # "GGUF" little-endian

# value types (src/gguf.cpp:12-26)
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}
_BOOL, _STRING, _ARRAY = 7, 8, 9


class GGUFError(ValueError):
    pass


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> memoryview:
        if n < 0 or self.pos + n > len(self.buf):
            raise GGUFError(f"read past EOF at {self.pos} (+{n})")
        v = memoryview(self.buf)[self.pos:self.pos + n]
        self.pos += n
        return v

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar("<Q")
        return bytes(self.take(n)).decode("utf-8", errors="replace")

    def value(self, vt: int):
        if vt in _SCALAR:
            return self.scalar(_SCALAR[vt])
        if vt == _BOOL:
            return self.scalar("<B") != 0
        if vt == _STRING:
            return self.string()
        if vt == _ARRAY:
            et, n = self.scalar("<I"), self.scalar("<Q")
            if et == _ARRAY:
                raise GGUFError("nested arrays are not supported")
            if et == _STRING:
                return [self.string() for _ in range(n)]
            if et == _BOOL:
                return [int(b) for b in self.take(n)]
            if et not in _SCALAR:
                raise GGUFError(f"bad array element type {et}")
            dt = np.dtype(_SCALAR[et])
            return np.frombuffer(self.take(n * dt.itemsize), dtype=dt).copy()
        raise GGUFError(f"bad value type {vt}")


@dataclass
class GGUFTensor:
    name: str
    type: int
    dims: tuple          # dims[0] innermost (GGUF order)
    offset: int          # relative to the data section
    nbytes: int
    data: np.ndarray     # uint8 view into the mapping

    def as_tensor(self) -> Tensor:
        return Tensor(self.type, self.dims, self.data, name=self.name)


def tensor_nbytes(t: int, dims) -> int:
    """Tensor::nbytes (src/tensor.h:150-157): whole blocks of the element count."""
    bpb, epb = bytes_per_block(t), elements_per_block(t)
    if bpb == 0 or epb == 0:
        return 0
    n = 1
    for d in dims:
        if d == 0:
            return 0
        n *= int(d)
    return (n + epb - 1) // epb * bpb


class GGUFFile:
    """A parsed, memory-mapped GGUF file."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        try:
            self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError as e:          # empty file
            self._f.close()
            raise GGUFError(f"cannot map {path}: {e}") from None
        self._registered = False
        try:
            self._parse()
        except GGUFError:
            self.close()
            raise

    def _parse(self) -> None:
        r = _Reader(self._mm)
        if r.scalar("<I") != GGUF_MAGIC:
            raise GGUFError("bad magic")
        self.version = r.scalar("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"unsupported version {self.version} (need 2 or 3)")
        n_tensors, n_kv = r.scalar("<Q"), r.scalar("<Q")
        self.metadata = {}
        for _ in range(n_kv):
            key = r.string()
            self.metadata[key] = r.value(r.scalar("<I"))
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.scalar("<I")
            if nd > 4:
                raise GGUFError(f"bad n_dims {nd} for tensor '{name}'")
            dims = tuple(r.scalar("<Q") for _ in range(nd))
            infos.append((name, dims, r.scalar("<I"), r.scalar("<Q")))
        a = self.metadata.get("general.alignment", 32)
        self.alignment = int(a) if isinstance(a, (int, np.integer)) and not isinstance(a, bool) else 32
        if self.alignment and r.pos % self.alignment:
            r.take(self.alignment - r.pos % self.alignment)
        self.data_offset = r.pos
        size = len(self._mm)
        buf = np.frombuffer(self._mm, dtype=np.uint8)
        self.tensors = {}
        for name, dims, t, off in infos:
            nb = tensor_nbytes(t, dims)
            start = self.data_offset + off
            if start > size or nb > size - start:
                raise GGUFError(f"tensor '{name}' data [{start}, +{nb}) past EOF ({size})")
            self.tensors[name] = GGUFTensor(name, t, dims, off, nb, buf[start:start + nb])
        self._buf = buf

    def find_tensor(self, name: str):
        t = self.tensors.get(name)
        return t.as_tensor() if t is not None else None

    def register(self) -> None:
        """Copy the data section to the GPU once; host pointers into it then
        resolve to the device copy in the host-pointer entries."""
        region = self._buf[self.data_offset:]
        if region.size:
            check(lib().lp_register_weights(region.ctypes.data, region.nbytes), "lp_register_weights")
            self._registered = region.ctypes.data

    def close(self) -> None:
        if getattr(self, "_registered", False):
            # only this file's region: other registered files stay resident
            lib().lp_release_region(self._registered)
            self._registered = False
        self.tensors = {}
        self._buf = None
        if getattr(self, "_mm", None) is not None:
            try:
                self._mm.close()
            except BufferError:
                pass                     # a view still refers to the mapping
            self._mm = None
        if getattr(self, "_f", None) is not None:
            self._f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def write_gguf(path: str, tensors, metadata=None, alignment: int = 32, version: int = 3) -> None:
    """Write a GGUF file (the layout GGUFFile reads): ``tensors`` is a list of
    (name, type, dims, uint8 bytes). Used to build test files; metadata values
    may be int (u32/u64), float (f32), bool, str, or a list of str / a numpy
    array of a scalar type."""
    meta = dict(metadata or {})
    if alignment != 32:
        meta["general.alignment"] = np.uint32(alignment)

    def s(x: str) -> bytes:
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    codes = {np.dtype("<u1"): 0, np.dtype("<i1"): 1, np.dtype("<u2"): 2, np.dtype("<i2"): 3,
             np.dtype("<u4"): 4, np.dtype("<i4"): 5, np.dtype("<f4"): 6, np.dtype("<u8"): 10,
             np.dtype("<i8"): 11, np.dtype("<f8"): 12}

    def val(v) -> bytes:
        if isinstance(v, bool):
            return struct.pack("<IB", _BOOL, int(v))
        if isinstance(v, str):
            return struct.pack("<I", _STRING) + s(v)
        if isinstance(v, np.generic):
            dt = v.dtype.newbyteorder("<")
            return struct.pack("<I", codes[dt]) + np.asarray(v, dtype=dt).tobytes()
        if isinstance(v, int):
            return struct.pack("<IQ", 10, v) if v >= 2 ** 32 or v < 0 else struct.pack("<II", 4, v)
        if isinstance(v, float):
            return struct.pack("<If", 6, v)
        if isinstance(v, (list, tuple)) and all(isinstance(e, str) for e in v):
            return struct.pack("<IIQ", _ARRAY, _STRING, len(v)) + b"".join(s(e) for e in v)
        if isinstance(v, np.ndarray):
            dt = v.dtype.newbyteorder("<")
            return struct.pack("<IIQ", _ARRAY, codes[dt], v.size) + v.astype(dt).tobytes()
        raise TypeError(f"unsupported metadata value {v!r}")

    head = struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(meta))
    head += b"".join(s(k) + val(v) for k, v in meta.items())
    offs, off = [], 0
    for name, t, dims, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(data)
    for (name, t, dims, data), o in zip(tensors, offs):
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        pos = 0
        for (name, t, dims, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            f.write(np.asarray(data, dtype=np.uint8).tobytes())
            pos = o + len(data)


__all__ = ["GGUFFile", "GGUFTensor", "GGUFError", "write_gguf", "tensor_nbytes"]
