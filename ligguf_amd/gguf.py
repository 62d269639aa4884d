"""GGUF v3 writer and reader for the tensors the decode path needs.

The reader follows what the reference loader accepts (fast/lil_gguf.cpp:
328-499): magic "GGUF", version 3, metadata key/value pairs, tensor infos,
data aligned to 32 bytes (the reference ignores general.alignment,
:377-378), dims[0] = row length.  The writer emits exactly that, with the
llama keys as uint32/float32 (kvrd32 reads 4 bytes, :96-104) and a
tokenizer.ggml.tokens array of vocab strings (:264-289).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from .lib import BLOCK, row_size

ALIGN = 32
# gguf value types (fast/lil_gguf.h:45-49)
GUINT8, GINT8, GUINT16, GINT16, GUINT32, GINT32, GFLOAT32, GBOOL, GSTRING, GARRAY, GUINT64, GINT64, GFLOAT64 = range(13)


@dataclass
class GGUFTensor:
    name: str
    type: int
    dims: list          # dims[0] = row length
    offset: int         # relative to the data section
    data: np.ndarray = None

    @property
    def rows(self) -> int:
        r = 1
        for d in self.dims[1:]:
            r *= d
        return r

    @property
    def nbytes(self) -> int:
        return self.rows * row_size(self.type, self.dims[0])


@dataclass
class GGUFFile:
    kv: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(tag: int, v) -> bytes:
    if tag == GUINT32:
        return struct.pack("<I", v)
    if tag == GINT32:
        return struct.pack("<i", v)
    if tag == GFLOAT32:
        return struct.pack("<f", v)
    if tag == GUINT64:
        return struct.pack("<Q", v)
    if tag == GBOOL:
        return struct.pack("<B", 1 if v else 0)
    if tag == GSTRING:
        return _str(v)
    if tag == GARRAY:
        etag, items = v
        out = [struct.pack("<IQ", etag, len(items))]
        if etag == GSTRING:
            out.extend(_str(s) for s in items)
        elif etag == GFLOAT32:
            out.append(np.asarray(items, dtype="<f4").tobytes())
        elif etag == GINT32:
            out.append(np.asarray(items, dtype="<i4").tobytes())
        else:
            raise ValueError(f"array of tag {etag} not supported")
        return b"".join(out)
    raise ValueError(f"tag {tag} not supported")


def write_gguf(path: str, kv: list, tensors: list) -> None:
    """kv: [(key, tag, value)], tensors: [(name, type, dims, bytes ndarray)]"""
    head = [b"GGUF", struct.pack("<IQQ", 3, len(tensors), len(kv))]
    for key, tag, val in kv:
        head.append(_str(key) + struct.pack("<I", tag) + _value(tag, val))
    off = 0
    offsets = []
    for name, t, dims, data in tensors:
        need = row_size(t, dims[0]) * int(np.prod(dims[1:], dtype=np.int64))
        assert data.nbytes == need, (name, data.nbytes, need)
        offsets.append(off)
        head.append(_str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) +
                    struct.pack("<IQ", t, off))
        off += (need + ALIGN - 1) // ALIGN * ALIGN
    blob = b"".join(head)
    pad = (ALIGN - len(blob) % ALIGN) % ALIGN
    with open(path, "wb") as f:
        f.write(blob)
        f.write(b"\0" * pad)
        pos = 0
        for (name, t, dims, data), o in zip(tensors, offsets):
            if o > pos:
                f.write(b"\0" * (o - pos))
                pos = o
            raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            f.write(raw.tobytes())
            pos += raw.nbytes


class _Reader:
    def __init__(self, mm: np.ndarray):
        self.mm = mm
        self.p = 0

    def u32(self):
        v = int(np.frombuffer(self.mm, "<u4", 1, self.p)[0]); self.p += 4; return v

    def u64(self):
        v = int(np.frombuffer(self.mm, "<u8", 1, self.p)[0]); self.p += 8; return v

    def string(self):
        n = self.u64()
        s = bytes(self.mm[self.p:self.p + n]).decode("utf-8", "replace"); self.p += n; return s

    def value(self, tag):
        sizes = {GUINT8: "<u1", GINT8: "<i1", GUINT16: "<u2", GINT16: "<i2", GUINT32: "<u4", GINT32: "<i4",
                 GFLOAT32: "<f4", GBOOL: "<u1", GUINT64: "<u8", GINT64: "<i8", GFLOAT64: "<f8"}
        if tag in sizes:
            dt = np.dtype(sizes[tag])
            v = np.frombuffer(self.mm, dt, 1, self.p)[0]
            self.p += dt.itemsize
            return v.item()
        if tag == GSTRING:
            return self.string()
        if tag == GARRAY:
            et = self.u32()
            n = self.u64()
            if et == GSTRING:
                return [self.string() for _ in range(n)]
            if et in sizes:
                dt = np.dtype(sizes[et])
                a = np.frombuffer(self.mm, dt, n, self.p).copy()
                self.p += dt.itemsize * n
                return a
            raise ValueError(f"array of tag {et}")
        raise ValueError(f"tag {tag}")


def read_gguf(path: str) -> GGUFFile:
    """Memory-map a GGUF v3 file; tensor .data are views into the map."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    r = _Reader(mm)
    if bytes(mm[:4]) != b"GGUF":
        raise ValueError("wrong magic")
    r.p = 4
    if r.u32() != 3:
        raise ValueError("GGUF version must be 3")
    nt, nkv = r.u64(), r.u64()
    g = GGUFFile()
    for _ in range(nkv):
        key = r.string()
        tag = r.u32()
        g.kv[key] = r.value(tag)
    infos = []
    for _ in range(nt):
        name = r.string()
        nd = r.u32()
        dims = [r.u64() for _ in range(nd)]
        t = r.u32()
        off = r.u64()
        infos.append(GGUFTensor(name, t, dims, off))
    base = (r.p + ALIGN - 1) // ALIGN * ALIGN
    for t in infos:
        if t.type not in BLOCK:
            raise ValueError(f"tensor {t.name} has unsupported type {t.type}")
        t.data = mm[base + t.offset: base + t.offset + t.nbytes]
        g.tensors[t.name] = t
    return g
