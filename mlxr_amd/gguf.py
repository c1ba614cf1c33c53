"""GGUF files for the quantized matmul: ctypes over the reader in libmlxr_qgemm.so.

Mirrors the reference's ``mlxr::registry::GGUFFile`` (daemon/registry/gguf_parser.h:122-202:
``parse``, ``header``, ``metadata``, ``tensors``, ``data_offset``, ``find_tensor``,
``get_tensor_names``, the ``get_arch`` / ``get_context_length`` / ... getters with the
same defaults, gguf_parser.cpp:493-550) and the zero-copy tensor view of
``MMapWeightLoader::map_tensor`` (core/runtime/mmap_loader.cpp:102-150).  Block sizes
follow GGUF (Q6_K 210 B, Q2_K 84 B, Q3_K 110 B) and the data section honours
``general.alignment``.  ``upload`` feeds a quantized weight to the packed device layout,
the step the reference's loader skips (daemon/server/model_loader.cpp:236-245).
"""
import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import qgemm

GGUF_MAGIC = 0x46554747


class GGMLType:
    F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 0, 1, 2, 3, 6, 7, 8, 9
    Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 10, 11, 12, 13, 14, 15
    I8, I16, I32, I64, F64, BF16 = 24, 25, 26, 27, 28, 30


class MetaType:
    UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL = 0, 1, 2, 3, 4, 5, 6, 7
    STRING, ARRAY, UINT64, INT64, FLOAT64 = 8, 9, 10, 11, 12


_SCALAR_NP = {MetaType.UINT8: np.uint8, MetaType.INT8: np.int8, MetaType.UINT16: np.uint16,
              MetaType.INT16: np.int16, MetaType.UINT32: np.uint32, MetaType.INT32: np.int32,
              MetaType.FLOAT32: np.float32, MetaType.BOOL: np.uint8, MetaType.UINT64: np.uint64,
              MetaType.INT64: np.int64, MetaType.FLOAT64: np.float64}
_SIGNED = {MetaType.INT8, MetaType.INT16, MetaType.INT32, MetaType.INT64}


class _Header(ctypes.Structure):
    _fields_ = [("magic", ctypes.c_uint32), ("version", ctypes.c_uint32), ("tensor_count", ctypes.c_uint64),
                ("metadata_kv_count", ctypes.c_uint64), ("alignment", ctypes.c_uint64),
                ("data_offset", ctypes.c_uint64), ("file_size", ctypes.c_uint64)]


class _TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 4),
                ("type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("file_offset", ctypes.c_uint64),
                ("size", ctypes.c_uint64), ("data", ctypes.c_void_p)]


class _ValueU(ctypes.Union):
    _fields_ = [("u64", ctypes.c_uint64), ("i64", ctypes.c_int64), ("f64", ctypes.c_double)]


class _Value(ctypes.Structure):
    _fields_ = [("type", ctypes.c_uint32), ("v", _ValueU), ("str", ctypes.c_void_p), ("len", ctypes.c_uint64),
                ("elem_type", ctypes.c_uint32), ("data", ctypes.c_void_p)]


_P = ctypes.c_void_p
_SIGS = {
    "mlxr_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "mlxr_gguf_open_memory": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.POINTER(_P)]),
    "mlxr_gguf_close": (None, [_P]),
    "mlxr_gguf_get_header": (ctypes.c_int, [_P, ctypes.POINTER(_Header)]),
    "mlxr_gguf_get_tensor": (ctypes.c_int, [_P, ctypes.c_uint64, ctypes.POINTER(_TensorInfo)]),
    "mlxr_gguf_find_tensor": (ctypes.c_int64, [_P, ctypes.c_char_p]),
    "mlxr_gguf_get_key": (ctypes.c_int, [_P, ctypes.c_uint64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_Value)]),
    "mlxr_gguf_get_value": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(_Value)]),
    "mlxr_gguf_get_array_string": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(_P),
                                                  ctypes.POINTER(ctypes.c_uint64)]),
    "mlxr_gguf_type_bytes": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]),
    "mlxr_gguf_block_size": (ctypes.c_int, [ctypes.c_uint32]),
    "mlxr_gguf_type_name": (ctypes.c_char_p, [ctypes.c_uint32]),
    "mlxr_gguf_quant_type": (ctypes.c_int, [ctypes.c_uint32]),
    "mlxr_gguf_upload": (ctypes.c_int, [_P, ctypes.c_uint64, _P, _P]),
}
_bound = None


def _lib():
    global _bound
    l = qgemm.lib()
    if _bound is not l:
        for name, (res, args) in _SIGS.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _bound = l
    return l


# ------------------------------------------------------------------ type helpers
# (reference gguf_parser.cpp: gguf_type_name, gguf_block_size :103-132,
#  calculate_tensor_size :179-241 with GGUF block sizes)

def gguf_type_name(t):
    return _lib().mlxr_gguf_type_name(int(t)).decode()


def gguf_block_size(t):
    return _lib().mlxr_gguf_block_size(int(t))


def type_bytes(t, n_elements):
    out = ctypes.c_uint64(0)
    qgemm._check(_lib().mlxr_gguf_type_bytes(int(t), int(n_elements), ctypes.byref(out)))
    return out.value


def calculate_tensor_size(dims, t):
    n = 1
    for d in dims:
        n *= int(d)
    return type_bytes(t, n)


def quant_type(t):
    """The QuantType the matmul uses for ggml type t (raises for types it does not run)."""
    rc = _lib().mlxr_gguf_quant_type(int(t))
    qgemm._check(rc if rc < 0 else 0)
    return qgemm.QuantType(rc)


@dataclass
class GGUFHeader:
    magic: int
    version: int
    tensor_count: int
    metadata_kv_count: int


@dataclass
class GGUFTensorInfo:
    """reference gguf_parser.h:110-117, plus the absolute file offset."""
    name: str
    n_dimensions: int
    dimensions: list
    type: int
    offset: int
    size: int
    file_offset: int = 0
    index: int = field(default=-1, repr=False)


class GGUFFile:
    """A parsed .gguf file kept open as a read-only map (call ``close`` or use ``with``)."""

    def __init__(self, path=None):
        self._h = None
        self._mem = None
        self._error = ""
        if path is not None and not self.parse(path):
            raise qgemm.QGemmError(-1, self._error)

    # ---- parse (reference gguf_parser.cpp:278-316) -------------------------
    def parse(self, path):
        """Parse ``path``; False with ``error()`` set on failure (the reference's contract)."""
        self.close()
        h = _P()
        rc = _lib().mlxr_gguf_open(str(path).encode(), ctypes.byref(h))
        return self._opened(rc, h)

    def parse_bytes(self, data):
        """Parse an in-memory file (kept referenced by this object)."""
        self.close()
        self._mem = np.frombuffer(bytes(data), dtype=np.uint8)
        h = _P()
        rc = _lib().mlxr_gguf_open_memory(self._mem.ctypes.data, self._mem.size, ctypes.byref(h))
        return self._opened(rc, h)

    def _opened(self, rc, h):
        if rc != 0:
            self._error = _lib().mlxr_qgemm_last_error().decode()
            self._mem = None
            return False
        self._h = h
        self._error = ""
        hd = _Header()
        qgemm._check(_lib().mlxr_gguf_get_header(self._h, ctypes.byref(hd)))
        self._hdr = hd
        self._tensors = None
        self._meta = None
        return True

    def close(self):
        if self._h is not None:
            _lib().mlxr_gguf_close(self._h)
            self._h = None
        self._mem = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def error(self):
        return self._error

    def has_error(self):
        return bool(self._error)

    def _need(self):
        if self._h is None:
            raise RuntimeError("GGUF file is not open")

    # ---- header / layout ----------------------------------------------------
    def header(self):
        self._need()
        h = self._hdr
        return GGUFHeader(h.magic, h.version, h.tensor_count, h.metadata_kv_count)

    def data_offset(self):
        self._need()
        return self._hdr.data_offset

    def alignment(self):
        self._need()
        return self._hdr.alignment

    def file_size(self):
        self._need()
        return self._hdr.file_size

    # ---- metadata -----------------------------------------------------------
    def _value(self, key, v):
        t = v.type
        if t == MetaType.STRING:
            return ctypes.string_at(v.str, v.len).decode("utf-8", errors="replace")
        if t in (MetaType.FLOAT32, MetaType.FLOAT64):
            return v.v.f64
        if t == MetaType.BOOL:
            return bool(v.v.u64)
        if t in _SIGNED:
            return v.v.i64
        if t == MetaType.ARRAY:
            if v.elem_type in _SCALAR_NP:
                dt = np.dtype(_SCALAR_NP[v.elem_type])
                if v.len == 0:
                    return np.zeros(0, dtype=dt)
                raw = ctypes.string_at(v.data, int(v.len) * dt.itemsize)
                arr = np.frombuffer(raw, dtype=dt).copy()
                return arr.astype(bool) if v.elem_type == MetaType.BOOL else arr
            if v.elem_type == MetaType.STRING:
                out = []
                s, n = _P(), ctypes.c_uint64()
                for j in range(v.len):
                    qgemm._check(_lib().mlxr_gguf_get_array_string(self._h, key.encode(), j, ctypes.byref(s),
                                                                   ctypes.byref(n)))
                    out.append(ctypes.string_at(s, n.value).decode("utf-8", errors="replace"))
                return out
            return None  # arrays of arrays are walked but not exposed
        return v.v.u64

    def metadata(self):
        """{key: value} in file order (strings, ints, floats, bools, numpy arrays, lists)."""
        self._need()
        if self._meta is None:
            meta = {}
            k, v = ctypes.c_char_p(), _Value()
            for i in range(self._hdr.metadata_kv_count):
                qgemm._check(_lib().mlxr_gguf_get_key(self._h, i, ctypes.byref(k), ctypes.byref(v)))
                key = k.value.decode("utf-8", errors="replace")
                meta[key] = (v.type, self._value(key, v))
            self._meta = meta
        return {k: val for k, (_, val) in self._meta.items()}

    def metadata_type(self, key):
        self.metadata()
        return self._meta[key][0] if key in self._meta else None

    def has_metadata(self, key):
        return key in self.metadata()

    def get_metadata(self, key):
        return self.metadata().get(key)

    def get_arch(self):
        return self.get_metadata("general.architecture") or ""

    def _arch_u32(self, suffix, default):
        v = self.get_metadata(self.get_arch() + suffix)
        return int(v) if v is not None else default

    def get_context_length(self):
        return self._arch_u32(".context_length", 2048)

    def get_embedding_length(self):
        return self._arch_u32(".embedding_length", 0)

    def get_block_count(self):
        return self._arch_u32(".block_count", 0)

    def get_feed_forward_length(self):
        return self._arch_u32(".feed_forward_length", 0)

    def get_attention_head_count(self):
        return self._arch_u32(".attention.head_count", 0)

    def get_attention_head_count_kv(self):
        return self._arch_u32(".attention.head_count_kv", self.get_attention_head_count())

    def get_rope_freq_base(self):
        v = self.get_metadata(self.get_arch() + ".rope.freq_base")
        return float(v) if v is not None else 10000.0

    def get_tokenizer_model(self):
        return self.get_metadata("tokenizer.ggml.model") or ""

    # ---- tensors ------------------------------------------------------------
    def _info(self, i):
        t = _TensorInfo()
        qgemm._check(_lib().mlxr_gguf_get_tensor(self._h, i, ctypes.byref(t)))
        return t

    def tensors(self):
        self._need()
        if self._tensors is None:
            out = []
            for i in range(self._hdr.tensor_count):
                t = self._info(i)
                out.append(GGUFTensorInfo(t.name.decode("utf-8", errors="replace"), t.n_dims,
                                          [int(t.dims[d]) for d in range(t.n_dims)], t.type, t.offset, t.size,
                                          t.file_offset, i))
            self._tensors = out
        return self._tensors

    def find_tensor(self, name):
        self._need()
        i = _lib().mlxr_gguf_find_tensor(self._h, name.encode())
        return None if i < 0 else self.tensors()[i]

    def get_tensor_names(self):
        return [t.name for t in self.tensors()]

    def tensor_bytes(self, name):
        """Zero-copy uint8 view of a tensor's bytes in the map (MMapWeightLoader::map_tensor).
        Raises if the tensor's data range is not inside the file.  Valid while the file is open."""
        info = self._lookup(name)
        t = self._info(info.index)
        if not t.data:
            raise qgemm.QGemmError(-1, f"tensor {info.name}: data range [{t.file_offset}, +{t.size}) is outside "
                                       f"the {self._hdr.file_size}-byte file")
        buf = (ctypes.c_uint8 * t.size).from_address(t.data)
        return np.frombuffer(buf, dtype=np.uint8)

    def _lookup(self, name):
        info = self.find_tensor(name) if isinstance(name, str) else self.tensors()[int(name)]
        if info is None:
            raise KeyError(name)
        return info

    def upload(self, name, device="cuda", stream=None):
        """Pack a 2-D quantized weight [N = dims[1], K = dims[0]] into device memory and return
        a PackedWeight for q_gemm_dequant."""
        torch = qgemm._torch()
        info = self._lookup(name)
        qt = quant_type(info.type)
        if info.n_dimensions != 2:
            raise qgemm.QGemmError(-3, f"tensor {info.name} is not 2-D")
        K, N = info.dimensions
        buf = torch.empty(qgemm.packed_size(qt, N, K), dtype=torch.uint8, device=device)
        qgemm._check(_lib().mlxr_gguf_upload(self._h, info.index, buf.data_ptr(), qgemm._stream_ptr(stream)))
        return qgemm.PackedWeight(buf, qt, N, K)
