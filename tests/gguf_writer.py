"""A minimal GGUF v3 writer -- test-only.

Layout (little endian): magic "GGUF", u32 version, u64 tensor count, u64
metadata count; metadata as (string key, u32 kind, value); tensor infos as
(string name, u32 n_dims, u64 ne[n_dims], u32 type, u64 offset); padding to
the alignment; then the tensor data, each tensor at an aligned offset from
the start of the data section.  Strings are u64 length + bytes.
"""
import struct

import numpy as np

K_U8, K_I8, K_U16, K_I16, K_U32, K_I32, K_F32, K_BOOL, K_STRING, K_ARRAY, K_U64, K_I64, K_F64 = range(13)
_FMT = {K_U8: "<B", K_I8: "<b", K_U16: "<H", K_I16: "<h", K_U32: "<I", K_I32: "<i", K_F32: "<f", K_BOOL: "<B",
        K_U64: "<Q", K_I64: "<q", K_F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _scalar(kind, v):
    if kind == K_STRING:
        return _str(v)
    return struct.pack(_FMT[kind], v)


class Writer:
    def __init__(self, alignment=32, version=3):
        self.kv = []          # (key, kind, value, arr_kind)
        self.tensors = []     # (name, ne, type, bytes)
        self.alignment = alignment
        self.version = version

    def add_kv(self, key, kind, value, arr_kind=None):
        self.kv.append((key, kind, value, arr_kind))

    def add_tensor(self, name, ne, type_, data):
        self.tensors.append((name, list(ne), int(type_), np.ascontiguousarray(data).view(np.uint8).reshape(-1)))

    def header(self, offsets):
        out = [b"GGUF", struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv))]
        for key, kind, value, ak in self.kv:
            out.append(_str(key) + struct.pack("<I", kind))
            if kind == K_ARRAY:
                out.append(struct.pack("<IQ", ak, len(value)))
                out += [_scalar(ak, e) for e in value]
            else:
                out.append(_scalar(kind, value))
        for (name, ne, t, _), off in zip(self.tensors, offsets):
            out.append(_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne) +
                       struct.pack("<IQ", t, off))
        return b"".join(out)

    def offsets(self):
        offs, cur = [], 0
        for _, _, _, b in self.tensors:
            offs.append(cur)
            cur += (len(b) + self.alignment - 1) // self.alignment * self.alignment
        return offs

    def write(self, path):
        offs = self.offsets()
        h = self.header(offs)
        pad = (-len(h)) % self.alignment
        with open(path, "wb") as f:
            f.write(h + b"\0" * pad)
            for (_, _, _, b), off in zip(self.tensors, offs):
                f.write(b.tobytes())
                f.write(b"\0" * ((-len(b)) % self.alignment))
        return len(h) + pad, offs
