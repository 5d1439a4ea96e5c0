"""rich_triplet_amd -- Python binding of librt_hip.so (the MI355X Q4_K / BF16
decode hot path of rich-triplet) over its C ABI, include/rt_hip.h.

The directory name carries a hyphen, so it is loaded by path:

    import importlib.util, pathlib, sys
    d = pathlib.Path("rich-triplet_amd")
    spec = importlib.util.spec_from_file_location("rich_triplet_amd", d / "__init__.py",
                                                  submodule_search_locations=[str(d)])
    rt = importlib.util.module_from_spec(spec); sys.modules["rich_triplet_amd"] = rt
    spec.loader.exec_module(rt)

There is no CPU fallback: every call goes to the HIP library, and a missing
library or a failed call raises RtError.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

PKG_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "librt_hip.so"

RT_OK, RT_EINVAL, RT_EHIP, RT_ENOMEM, RT_ESTATE = 0, 1, 2, 3, 4


class RtError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"rt status {code}: {msg}")
        self.code = code


def build(jobs: int = 8) -> None:
    """Compile librt_hip.so for gfx950 in-tree (hipcc cross-compiles without a GPU)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", str(PKG_DIR)], check=True)


_lib = None

_vp, _i64, _sz, _u32, _i32 = C.c_void_p, C.c_int64, C.c_size_t, C.c_uint32, C.c_int32

_SIGNATURES = {
    "rt_last_error": (C.c_char_p, []),
    "rt_abi_version": (C.c_int32, []),
    "rt_q4k_dequant_f32": (_i32, [_vp, _sz, _vp, _vp]),
    "rt_q4k_dequant_bf16": (_i32, [_vp, _sz, _vp, _vp]),
    "rt_q4k_gemv": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "rt_bf16_gemv": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "rt_gemv_q4k_t": (_i32, [_vp, _sz, _vp, _sz, _vp]),
    "rt_gemv_bf16_t": (_i32, [_vp, _sz, _vp, _sz, _vp]),
    "rt_weight_cache_clear": (_i32, []),
}


def lib() -> C.CDLL:
    """Load librt_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RtError(RT_ESTATE, f"{LIB_PATH} is missing: run __graft_entry__.build() or make -C rich-triplet_amd")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int) -> None:
    if status != RT_OK:
        raise RtError(status, lib().rt_last_error().decode(errors="replace"))


def _p(t) -> int | None:
    """Device pointer of a torch tensor (or an int address, or None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream


# ---------------------------------------------------------------------------
# device-pointer API (torch tensors on cuda:N)
# ---------------------------------------------------------------------------
def q4k_dequant_f32(blocks, out, n_blocks: int | None = None, stream=None) -> None:
    n = blocks.numel() // 144 if n_blocks is None else n_blocks
    check(lib().rt_q4k_dequant_f32(_p(blocks), n, _p(out), _stream(stream)))


def q4k_dequant_bf16(blocks, out, n_blocks: int | None = None, stream=None) -> None:
    n = blocks.numel() // 144 if n_blocks is None else n_blocks
    check(lib().rt_q4k_dequant_bf16(_p(blocks), n, _p(out), _stream(stream)))


def q4k_gemv(w, x, y, n: int, k: int, stream=None) -> None:
    check(lib().rt_q4k_gemv(_p(w), _p(x), _p(y), n, k, _stream(stream)))


def bf16_gemv(w, x, y, n: int, k: int, stream=None) -> None:
    check(lib().rt_bf16_gemv(_p(w), _p(x), _p(y), n, k, _stream(stream)))


# ---------------------------------------------------------------------------
# host-pointer API (numpy arrays), mirrors metal_ops::metal_gemv_*_t
# ---------------------------------------------------------------------------
def gemv_q4k_t(a, blocks, rows: int):
    import numpy as np
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty(rows, np.float32)
    check(lib().rt_gemv_q4k_t(a.ctypes.data, a.size, blocks.ctypes.data, rows, out.ctypes.data))
    return out


def gemv_bf16_t(a, w, rows: int):
    import numpy as np
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    w = np.ascontiguousarray(w, np.uint16)
    out = np.empty(rows, np.float32)
    check(lib().rt_gemv_bf16_t(a.ctypes.data, a.size, w.ctypes.data, rows, out.ctypes.data))
    return out


def weight_cache_clear() -> None:
    check(lib().rt_weight_cache_clear())
