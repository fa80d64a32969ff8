"""GGUF v3 reader and writer for the decode path's host side.

The reference's loader (model/loader.zig:2525-2785, the GGUF rules in
gguf.zig:147-234,393-424) stays the caller of the backend; this module plays
that caller's role for the tests and the benchmark: it lays out GGUF images the
reference loader accepts (magic, version 3, general.alignment 32, data section
aligned, tensor offsets multiples of the alignment, dims[0] = row length) and
reads their tensor tables back.  Tensor bytes live in one numpy uint8 array so
an 8B-parameter image is filled in place without copies.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

# GGUF metadata value types (model/loader.zig:98-113)
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)

# tensor type ids (model/loader.zig:119-153)
F32, F16, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS = 0, 1, 8, 11, 12, 13, 14, 23
TYPE_NAMES = {F32: "f32", F16: "f16", Q8_0: "q8_0", Q3_K: "q3_k", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k",
              IQ4_XS: "iq4_xs"}
# (values per block, bytes per block): gguf.zig:531-567
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210), IQ4_XS: (256, 136)}


def row_bytes(ttype: int, cols: int) -> int:
    nv, nb = BLOCK[ttype]
    if cols % nv:
        raise ValueError(f"row length {cols} is not a multiple of {nv} for {TYPE_NAMES[ttype]}")
    return cols // nv * nb


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == T_STR:
        return _str(v)
    if vtype == T_ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        if etype == T_STR:
            return out + b"".join(_str(s) for s in items)
        fmt = {T_U32: "I", T_I32: "i", T_F32: "f", T_U8: "B", T_I8: "b", T_U64: "Q", T_F64: "d"}[etype]
        return out + np.asarray(items, dtype=np.dtype("<" + fmt)).tobytes()
    fmt = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}[vtype]
    return struct.pack(fmt, v)


@dataclass
class TensorInfo:
    name: str
    ttype: int
    dims: tuple  # dims[0] = row length (reduction dim)
    offset: int = 0  # relative to the data section

    @property
    def row_len(self) -> int:
        return int(self.dims[0])

    @property
    def rows(self) -> int:
        r = 1
        for d in self.dims[1:]:
            r *= int(d)
        return r

    @property
    def nbytes(self) -> int:
        return row_bytes(self.ttype, self.row_len) * self.rows


@dataclass
class GGUFImage:
    """A laid-out GGUF image: `buf` holds the whole file; tensor data is filled in place."""
    buf: np.ndarray
    data_offset: int
    tensors: dict = field(default_factory=dict)  # name -> TensorInfo
    metadata: dict = field(default_factory=dict)

    def tensor_view(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        start = self.data_offset + t.offset
        return self.buf[start:start + t.nbytes]

    def tensor_file_offset(self, name: str) -> int:
        return self.data_offset + self.tensors[name].offset

    def save(self, path: str) -> None:
        self.buf.tofile(path)


def layout(metadata: list, tensors: list, alignment: int = 32) -> GGUFImage:
    """Builds the header and an image buffer; metadata is [(key, vtype, value)]."""
    head = bytearray(b"GGUF")
    head += struct.pack("<IQQ", 3, len(tensors), len(metadata))
    md = {}
    for key, vtype, value in metadata:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
        md[key] = value
    off = 0
    tmap = {}
    for t in tensors:
        off = (off + alignment - 1) // alignment * alignment
        t.offset = off
        off += t.nbytes
        tmap[t.name] = t
    for t in tensors:
        head += _str(t.name) + struct.pack("<I", len(t.dims))
        head += b"".join(struct.pack("<Q", int(d)) for d in t.dims)
        head += struct.pack("<IQ", t.ttype, t.offset)
    data_offset = (len(head) + alignment - 1) // alignment * alignment
    total = data_offset + ((off + alignment - 1) // alignment * alignment)
    buf = np.zeros(total, dtype=np.uint8)
    buf[:len(head)] = np.frombuffer(bytes(head), dtype=np.uint8)
    return GGUFImage(buf=buf, data_offset=data_offset, tensors=tmap, metadata=md)


class _Reader:
    def __init__(self, b):
        self.b, self.p = b, 0

    def u(self, fmt):
        v = struct.unpack_from(fmt, self.b, self.p)[0]
        self.p += struct.calcsize(fmt)
        return v

    def s(self):
        n = self.u("<Q")
        v = bytes(self.b[self.p:self.p + n]).decode(errors="replace")
        self.p += n
        return v

    def value(self, vt):
        if vt == T_STR:
            return self.s()
        if vt == T_ARR:
            et, n = self.u("<I"), self.u("<Q")
            return [self.value(et) for _ in range(n)]
        fmt = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
               T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}[vt]
        return self.u(fmt)


def read(buf: np.ndarray, keep_arrays: bool = False) -> GGUFImage:
    """Parses the header of a GGUF image (reference rules: model/loader.zig:2541-2600)."""
    mv = memoryview(buf)
    r = _Reader(mv)
    if bytes(mv[:4]) != b"GGUF":
        raise ValueError("invalid magic")
    r.p = 4
    version = r.u("<I")
    if version not in (2, 3):
        raise ValueError(f"unsupported GGUF version {version}")
    nt, nkv = r.u("<Q"), r.u("<Q")
    md = {}
    for _ in range(nkv):
        k = r.s()
        vt = r.u("<I")
        if vt == T_ARR and not keep_arrays:
            et, n = r.u("<I"), r.u("<Q")
            if et == T_STR:
                for _ in range(n):
                    r.s()
            else:
                r.p += n * struct.calcsize({T_U32: "I", T_I32: "i", T_F32: "f", T_U8: "B", T_I8: "b",
                                            T_U64: "Q", T_F64: "d", T_U16: "H", T_I16: "h", T_BOOL: "?",
                                            T_I64: "q"}[et])
            md[k] = ("array", n)
        else:
            md[k] = r.value(vt)
    align = int(md.get("general.alignment", 32))
    tensors = {}
    for _ in range(nt):
        name = r.s()
        nd = r.u("<I")
        dims = tuple(r.u("<Q") for _ in range(nd))
        tt = r.u("<I")
        off = r.u("<Q")
        if off % align:
            raise ValueError(f"tensor {name} offset {off} not aligned to {align}")
        tensors[name] = TensorInfo(name, tt, dims, off)
    data_offset = (r.p + align - 1) // align * align
    img = GGUFImage(buf=buf, data_offset=data_offset, tensors=tensors, metadata=md)
    for t in tensors.values():
        if data_offset + t.offset + t.nbytes > len(buf):
            raise ValueError(f"truncated: tensor {t.name}")
    return img
