"""Minimal GGUF writer for tests (file format v1-v3: header, typed metadata, tensor infos,
aligned data section).  Independent of the library's reader."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


class Writer:
    def __init__(self, version=3, alignment=None):
        self.version = version
        self.alignment = alignment
        self.kv = []
        self.tensors = []  # (name, dims (ggml order), type, bytes or None, size for the info)
        if alignment is not None:
            self.kv.append(("general.alignment", U32, alignment))

    def _count(self, n):
        return struct.pack("<I" if self.version == 1 else "<Q", n)

    def _str(self, s):
        b = s.encode() if isinstance(s, str) else s
        return self._count(len(b)) + b

    def _val(self, t, v):
        if t == STR:
            return self._str(v)
        if t == ARR:
            et, items = v
            out = struct.pack("<I", et) + self._count(len(items))
            return out + b"".join(self._val(et, x) for x in items)
        return struct.pack(_FMT[t], v)

    def add(self, key, t, value):
        self.kv.append((key, t, value))

    def add_tensor(self, name, dims, ggml_type, data):
        self.tensors.append((name, list(dims), ggml_type, bytes(data)))

    def to_bytes(self, declared_offsets=None):
        align = self.alignment or 32
        out = bytearray(struct.pack("<II", 0x46554747, self.version))
        out += self._count(len(self.tensors)) + self._count(len(self.kv))
        for k, t, v in self.kv:
            out += self._str(k) + struct.pack("<I", t) + self._val(t, v)
        offs, cur = [], 0
        for _, _, _, data in self.tensors:
            offs.append(cur)
            cur += len(data)
            cur = (cur + align - 1) // align * align
        if declared_offsets is not None:
            offs = declared_offsets
        for (name, dims, gt, _), off in zip(self.tensors, offs):
            out += self._str(name) + struct.pack("<I", len(dims))
            out += b"".join(self._count(d) for d in dims)
            out += struct.pack("<IQ", gt, off)
        data_start = (len(out) + align - 1) // align * align
        out += b"\0" * (data_start - len(out))
        for (_, _, _, data), off in zip(self.tensors, offs):
            if data_start + off > len(out):
                out += b"\0" * (data_start + off - len(out))
            out += data
        return bytes(out), data_start


def tensor_data_f32(arr):
    return np.ascontiguousarray(arr, dtype=np.float32).tobytes()
