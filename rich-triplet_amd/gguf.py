"""GGUF reader and weight loader: Python face of include/rt_gguf.h.

Mirrors the reference's `GgufFile` (src/gguf_loader.rs:156-744) and
`load_linear_from_gguf` (src/transformer4.rs:1177-1256) with the same names and
meanings: `open`, `tensor_info` (name, shape in GGUF order, gguf_type,
data_offset), `find_tensor`, `read_tensor_bytes`, the `decode_*` family and a
`metadata` dict.  Every call goes through librt_hip.so; errors raise `RtError`
(the reference returns io::Error or panics).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import RT_OK, RtError, check, lib

# ggml type ids (GgufType, gguf_loader.rs:41-72)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 30
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4K", Q5_K: "Q5K", Q6_K: "Q6K",
              BF16: "Bf16"}
# metadata value types (GgufMetaValue, gguf_loader.rs:828-905)
META_U8, META_I8, META_U16, META_I16, META_U32, META_I32, META_F32, META_BOOL, META_STR, META_ARRAY, \
    META_U64, META_I64, META_F64 = range(13)

LINEAR_Q4K, LINEAR_BF16, LINEAR_F32, LINEAR_Q6K, LINEAR_Q8_0 = 1, 2, 3, 4, 5
LOAD_KEEP_PACKED = 1


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_int32), ("dims", C.c_int64 * 4), ("type", C.c_int32),
                ("offset", C.c_uint64), ("n_bytes", C.c_uint64)]


class _Linear(C.Structure):
    _fields_ = [("format", C.c_int32), ("src_type", C.c_int32), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("bytes", C.c_uint64)]


@dataclass
class GgufTensorInfo:
    """GgufTensorInfo (gguf_loader.rs:139-154)."""
    name: str
    shape: list[int]        # GGUF order: shape[0] varies fastest ([in, out] for a weight)
    gguf_type: int
    data_offset: int
    n_bytes: int

    def n_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


class GgufFile:
    """GgufFile::open (gguf_loader.rs:167-230); the handle closes on `close()`."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().rt_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h
        self.file_path = str(path)
        L = lib()
        self.tensor_info: list[GgufTensorInfo] = []
        for i in range(L.rt_gguf_n_tensors(h)):
            t = _Tensor()
            check(L.rt_gguf_tensor_info(h, i, C.byref(t)))
            self.tensor_info.append(GgufTensorInfo(t.name.decode(), [int(t.dims[d]) for d in range(t.n_dims)],
                                                   int(t.type), int(t.offset), int(t.n_bytes)))
        self.data_start = int(L.rt_gguf_data_start(h))
        self.metadata = {k: self._meta_value(k) for k in self._meta_keys()}

    @classmethod
    def open(cls, path: str) -> "GgufFile":
        return cls(path)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().rt_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- metadata ---------------------------------------------------------
    def _meta_keys(self) -> list[str]:
        L = lib()
        out = []
        for i in range(L.rt_gguf_n_metadata(self._h)):
            k = C.c_char_p()
            check(L.rt_gguf_meta_key(self._h, i, C.byref(k)))
            out.append(k.value.decode())
        return out

    def _meta_value(self, key: str):
        """Scalars, strings and string arrays as Python values; numeric arrays as their count
        (the decode path reads none of them)."""
        L = lib()
        kb = key.encode()
        t, et, n = C.c_int32(), C.c_int32(), C.c_uint64()
        check(L.rt_gguf_meta_type(self._h, kb, C.byref(t), C.byref(et), C.byref(n)))
        t = t.value
        if t == META_STR:
            s = C.c_char_p()
            check(L.rt_gguf_meta_str(self._h, kb, C.byref(s)))
            return s.value.decode(errors="replace")
        if t in (META_F32, META_F64):
            f = C.c_float()
            check(L.rt_gguf_meta_f32(self._h, kb, C.byref(f)))
            return f.value
        if t in (META_U8, META_U16, META_U32, META_U64, META_I32, META_I64):
            u = C.c_uint64()
            check(L.rt_gguf_meta_u64(self._h, kb, C.byref(u)))
            v = u.value
            return v - (1 << 64) if t in (META_I32, META_I64) and v >= 1 << 63 else v
        if t == META_ARRAY and et.value == META_STR:
            out = []
            for i in range(n.value):
                s = C.c_char_p()
                check(L.rt_gguf_meta_array_str(self._h, kb, i, C.byref(s)))
                out.append(s.value.decode(errors="replace"))
            return out
        if t == META_ARRAY:
            return ("array", et.value, n.value)
        return ("type", t)  # bool, i8, i16: not read by the reference's loaders

    def meta_u64(self, key: str) -> int | None:
        """GgufMetaValue::as_u64 (gguf_loader.rs:880-890)."""
        u = C.c_uint64()
        return u.value if lib().rt_gguf_meta_u64(self._h, key.encode(), C.byref(u)) == RT_OK else None

    def meta_f32(self, key: str) -> float | None:
        """GgufMetaValue::as_f32 (gguf_loader.rs:899-905)."""
        f = C.c_float()
        return f.value if lib().rt_gguf_meta_f32(self._h, key.encode(), C.byref(f)) == RT_OK else None

    # ---- tensors ----------------------------------------------------------
    def find_tensor(self, name: str) -> int | None:
        """gguf_loader.rs:248-250"""
        i = lib().rt_gguf_find_tensor(self._h, name.encode())
        return None if i < 0 else int(i)

    def read_tensor_bytes(self, idx: int) -> np.ndarray:
        """gguf_loader.rs:233-246"""
        info = self.tensor_info[idx]
        if info.n_bytes == 0:
            raise RtError(1, f"unsupported gguf type {info.gguf_type} for tensor {info.name}")
        out = np.empty(info.n_bytes, np.uint8)
        check(lib().rt_gguf_read_tensor(self._h, idx, out.ctypes.data, out.size))
        return out

    def tensor_to_f32(self, idx: int) -> np.ndarray:
        """tensor_to_f32 (gguf_loader.rs:745-760): flat f32 in GGUF element order."""
        n = self.tensor_info[idx].n_elements()
        out = np.empty(n, np.float32)
        check(lib().rt_gguf_tensor_to_f32(self._h, idx, out.ctypes.data, n))
        return out

    # the reference's per-type names (gguf_loader.rs:384-743)
    decode_f32 = decode_f16_to_f32 = decode_q4_0_to_f32 = decode_q6k_to_f32 = tensor_to_f32
    decode_q4k_to_f32 = decode_q8_0_to_f32 = decode_q5k_to_f32 = tensor_to_f32

    def decode_bf16(self, idx: int) -> np.ndarray:
        """gguf_loader.rs:395-403"""
        return self.read_tensor_bytes(idx).view(np.uint16)

    def decode_q4k_to_q4kmat(self, idx: int) -> tuple[np.ndarray, int, int]:
        """gguf_loader.rs:360-381: (blocks, rows, cols) with the [in, out] shape flipped."""
        info = self.tensor_info[idx]
        if info.gguf_type != Q4_K:
            raise RtError(1, f"decode_q4k_to_q4kmat called on non-Q4K tensor {info.name}")
        rows, cols = (info.shape[1], info.shape[0]) if len(info.shape) >= 2 else (1, info.shape[0])
        return self.read_tensor_bytes(idx), rows, cols


class Linear:
    """A weight resident in device memory, as load_linear_from_gguf leaves it:
    format is LINEAR_Q4K (packed 144-B blocks), LINEAR_BF16, LINEAR_F32, or
    with keep_packed LINEAR_Q6K / LINEAR_Q8_0 (planar layout), row-major
    [rows=out_features, cols=in_features]."""

    def __init__(self, raw: _Linear):
        self._raw = raw
        self.format, self.src_type = int(raw.format), int(raw.src_type)
        self.rows, self.cols, self.bytes = int(raw.rows), int(raw.cols), int(raw.bytes)

    @property
    def ptr(self) -> int:
        return int(self._raw.data or 0)

    def free(self) -> None:
        if self._raw.data:
            check(lib().rt_linear_free(C.byref(self._raw)))

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def load_linear_from_gguf(gguf: GgufFile, idx: int, keep_packed: bool = False) -> Linear:
    """transformer4.rs:1177-1256, then the device upload (metal_decode.rs:1259-1277).
    keep_packed: Q6_K and Q8_0 stay packed for the native GEMVs instead of
    widening to BF16."""
    raw = _Linear()
    check(lib().rt_gguf_load_linear_ex(gguf._h, idx, LOAD_KEEP_PACKED if keep_packed else 0, C.byref(raw)))
    return Linear(raw)


def q4k_quantize_bf16(m: np.ndarray) -> np.ndarray:
    """Q4KMat::quantize_from_bf16 (autograd2.rs:1252-1289): bf16 bits
    [rows, cols] -> Q4_K blocks, row by row."""
    m = np.ascontiguousarray(m, np.uint16)
    rows, cols = m.shape
    out = np.zeros(max(1, rows * (cols // 256) * 144), np.uint8)
    check(lib().rt_q4k_quantize_bf16(m.ctypes.data, rows, cols, out.ctypes.data))
    return out[: rows * (cols // 256) * 144]


def q4k_quantize(m: np.ndarray) -> np.ndarray:
    """Q4KMat::quantize (autograd2.rs:1138-1168): f32 [rows, cols] -> Q4_K blocks."""
    m = np.ascontiguousarray(m, np.float32)
    rows, cols = m.shape
    out = np.zeros(max(1, rows * (cols // 256) * 144), np.uint8)  # the library reports a bad cols itself
    check(lib().rt_q4k_quantize(m.ctypes.data, rows, cols, out.ctypes.data))
    return out[: rows * (cols // 256) * 144]
