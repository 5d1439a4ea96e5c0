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
import os
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
# RT_HIP_LIB selects another build of the library (e.g. the host-AddressSanitizer
# one, `make -C rich-triplet_amd asan`); by default the in-tree librt_hip.so.
LIB_PATH = pathlib.Path(os.environ["RT_HIP_LIB"]).resolve() if os.environ.get("RT_HIP_LIB") else PKG_DIR / "librt_hip.so"

RT_OK, RT_EINVAL, RT_EHIP, RT_ENOMEM, RT_ESTATE = 0, 1, 2, 3, 4


LINEAR_Q4K, LINEAR_BF16, LINEAR_F32, LINEAR_Q6K, LINEAR_Q8_0 = 1, 2, 3, 4, 5  # RT_LINEAR_* (rt_hip.h)


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
    "rt_gemm_workspace_release": (_i32, [_vp]),
    "rt_gemm_workspace_held": (_sz, [_vp]),
    "rt_q4k_gemv_batch": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "rt_q4k_gemv_batch_noalloc": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "rt_qlinear_forward": (_i32, [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "rt_decode_memory": (_i32, [_vp, _vp]),
    "rt_decode_verify_batched": (_i32, [_vp, _vp]),
    "rt_linear_gemv_batch": (_i32, [_i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "rt_gelu_tanh": (_i32, [_vp, _vp, _sz, _vp]),
    "rt_stream_read": (_i32, [_vp, _sz, _vp, _vp]),
    "rt_stream_read_cfg": (_i32, [_vp, _sz, _vp, _vp, _i32, _i32]),
    "rt_empty_launch": (_i32, [_i32, _i32, _vp]),
    "rt_trace_read": (_i32, [_vp, _sz, C.POINTER(_i32), C.POINTER(_i32)]),
    "rt_qlinear_forward_host": (_i32, [_i32, _vp, _sz, _vp, _vp, _vp, _i64, _i64, _i64]),
    "rt_noalloc_scratch_bytes": (_sz, []),
    "rt_q6k_repack": (_i32, [_vp, _sz, _vp]),
    "rt_q8_0_repack": (_i32, [_vp, _sz, _vp]),
    "rt_q6k_dequant_f32": (_i32, [_vp, _sz, _vp, _vp]),
    "rt_q8_0_dequant_f32": (_i32, [_vp, _sz, _vp, _vp]),
    "rt_q6k_gemv": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "rt_q8_0_gemv": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "rt_linear_gemm_f32": (_i32, [_i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "rt_q4k_gemv_multi": (_i32, [_vp, _vp, _vp, _i32, _vp, _i64, _vp]),
    "rt_q4k_gemm_bf16": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "rt_q4k_gemm_f32": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "rt_matmul_q4k_t": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp]),
    "rt_decode_create": (_i32, [_vp, C.POINTER(_vp)]),
    "rt_decode_destroy": (_i32, [_vp]),
    "rt_decode_set_layer": (_i32, [_vp, _i32, _vp, _i32]),
    "rt_decode_set_layer_formats": (_i32, [_vp, _i32, _vp, _vp, _i32]),
    "rt_decode_set_embed": (_i32, [_vp, _vp, _vp, _i32]),
    "rt_decode_sync_kv": (_i32, [_vp, _i32, _vp, _vp, _i32, _i32]),
    "rt_decode_step": (_i32, [_vp, _i32, _i32, _vp]),
    "rt_decode_step_async": (_i32, [_vp, _i32, _i32]),
    "rt_decode_synchronize": (_i32, [_vp]),
    "rt_decode_set_graph": (_i32, [_vp, _i32]),
    "rt_decode_logits": (_i32, [_vp, C.POINTER(_vp)]),
    "rt_decode_kv": (_i32, [_vp, _i32, C.POINTER(_vp), C.POINTER(_vp)]),
    "rt_decode_hidden": (_i32, [_vp, C.POINTER(_vp), C.POINTER(_vp)]),
    "rt_decode_get_stream": (_i32, [_vp, C.POINTER(_vp)]),
    "rt_decode_step_batch": (_i32, [_vp, _vp, _i32, _i32, _vp]),
    "rt_decode_step_batch_async": (_i32, [_vp, _vp, _i32, _i32]),
    "rt_decode_logits_batch": (_i32, [_vp, C.POINTER(_vp)]),
    "rt_decode_prefill": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp]),
    "rt_decode_set_prefill_chunk": (_i32, [_vp, _i32]),
    # GGUF reader and loader (include/rt_gguf.h)
    "rt_gguf_open": (_i32, [C.c_char_p, C.POINTER(_vp)]),
    "rt_gguf_close": (_i32, [_vp]),
    "rt_gguf_n_tensors": (_i64, [_vp]),
    "rt_gguf_n_metadata": (_i64, [_vp]),
    "rt_gguf_data_start": (C.c_uint64, [_vp]),
    "rt_gguf_tensor_info": (_i32, [_vp, _i64, _vp]),
    "rt_gguf_find_tensor": (_i64, [_vp, C.c_char_p]),
    "rt_gguf_meta_key": (_i32, [_vp, _i64, C.POINTER(C.c_char_p)]),
    "rt_gguf_meta_type": (_i32, [_vp, C.c_char_p, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(C.c_uint64)]),
    "rt_gguf_meta_u64": (_i32, [_vp, C.c_char_p, C.POINTER(C.c_uint64)]),
    "rt_gguf_meta_f32": (_i32, [_vp, C.c_char_p, C.POINTER(C.c_float)]),
    "rt_gguf_meta_str": (_i32, [_vp, C.c_char_p, C.POINTER(C.c_char_p)]),
    "rt_gguf_meta_array_str": (_i32, [_vp, C.c_char_p, C.c_uint64, C.POINTER(C.c_char_p)]),
    "rt_gguf_read_tensor": (_i32, [_vp, _i64, _vp, C.c_uint64]),
    "rt_gguf_tensor_to_f32": (_i32, [_vp, _i64, _vp, C.c_uint64]),
    "rt_q4k_quantize": (_i32, [_vp, _sz, _sz, _vp]),
    "rt_q4k_quantize_bf16": (_i32, [_vp, _sz, _sz, _vp]),
    "rt_decode_set_lm_head": (_i32, [_vp, _i32, _vp, _i32]),
    "rt_gguf_load_linear": (_i32, [_vp, _i64, _vp]),
    "rt_gguf_load_linear_ex": (_i32, [_vp, _i64, _i32, _vp]),
    "rt_linear_free": (_i32, [_vp]),
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


def linear_gemv_batch(fmt: int, w, a, c, m: int, n: int, k: int, stream=None) -> None:
    """c[m][n] = a[m][k] . W[n][k] for m <= 8 rows and a weight in Q4_K, Q6_K,
    Q8_0 (planar) or BF16 (gemv_bf16_t_batch for BF16)."""
    check(lib().rt_linear_gemv_batch(fmt, _p(w), _p(a), _p(c), m, n, k, _stream(stream)))


def q4k_gemv_batch(w, a, c, m: int, n: int, k: int, stream=None) -> None:
    """c[m][n] = a[m][k] . W[n][k] for m <= 8 rows (gemv_q4k_t_batch)."""
    check(lib().rt_q4k_gemv_batch(_p(w), _p(a), _p(c), m, n, k, _stream(stream)))


def trace_read():
    """The decode-step timeline of a library built with RT_TRACE=1, as a uint64
    array [kernels][slots][4] (see rt_trace_read); raises RtError(RT_ESTATE)
    for a library built without it."""
    import numpy as np
    k, s = C.c_int32(0), C.c_int32(0)
    check(lib().rt_trace_read(None, 0, C.byref(k), C.byref(s)))
    buf = np.zeros((k.value, s.value, 4), dtype=np.uint64)
    check(lib().rt_trace_read(buf.ctypes.data_as(C.c_void_p), buf.nbytes, None, None))
    return buf


def stream_read(buf, nbytes: int, sink, stream=None, kind: int = 0, grid: int = 0) -> None:
    """Read nbytes of buf with 16-byte loads and discard them (a bandwidth
    floor); kind 0 strided, 1 one slice per workgroup, 2 and 3 the same with
    nontemporal loads; grid 0 by size."""
    check(lib().rt_stream_read_cfg(_p(buf), nbytes, _p(sink), _stream(stream), kind, grid))


def empty_launch(grid: int = 1, threads: int = 64, stream=None) -> None:
    """A kernel with no body (the cost of a launch)."""
    check(lib().rt_empty_launch(grid, threads, _stream(stream)))


def gelu_tanh(x, y, stream=None) -> None:
    """y = gelu_tanh(x) on the device, as the decode and prefill kernels compute it."""
    check(lib().rt_gelu_tanh(_p(x), _p(y), x.numel(), _stream(stream)))


def q4k_gemv_batch_noalloc(w, a, c, m: int, n: int, k: int, stream=None) -> None:
    """q4k_gemv_batch on a fixed per-GPU workspace: no device allocation.
    Calls that overlap on one GPU share that workspace and race."""
    check(lib().rt_q4k_gemv_batch_noalloc(_p(w), _p(a), _p(c), m, n, k, _stream(stream)))


def q6k_gemv(w, x, y, n: int, k: int, stream=None) -> None:
    """y = W x on planar Q6_K weights (q6k_repack)."""
    check(lib().rt_q6k_gemv(_p(w), _p(x), _p(y), n, k, _stream(stream)))


def q8_0_gemv(w, x, y, n: int, k: int, stream=None) -> None:
    """y = W x on planar Q8_0 weights (q8_0_repack)."""
    check(lib().rt_q8_0_gemv(_p(w), _p(x), _p(y), n, k, _stream(stream)))


def q4k_gemv_multi(ws, ys, ns, x, k: int, stream=None) -> None:
    """y_i = W_i x for up to 4 Q4_K matrices sharing x, one launch (q|k|v, gate|up)."""
    cnt = len(ws)
    if not (len(ys) == cnt == len(ns)):
        raise ValueError("ws, ys and ns must have the same length")
    wa = (C.c_void_p * max(cnt, 1))(*[_p(w) for w in ws])
    ya = (C.c_void_p * max(cnt, 1))(*[_p(y) for y in ys])
    na = (C.c_int64 * max(cnt, 1))(*[int(n) for n in ns])
    check(lib().rt_q4k_gemv_multi(wa, ya, na, cnt, _p(x), k, _stream(stream)))


def linear_gemm_f32(fmt: int, w, a, c, m: int, n: int, k: int, stream=None) -> None:
    """c[m][n] = a[m][k] . W[n][k] for a weight in format fmt (LINEAR_Q4K,
    LINEAR_BF16, LINEAR_Q6K or LINEAR_Q8_0, the last two planar)."""
    check(lib().rt_linear_gemm_f32(fmt, _p(w), _p(a), _p(c), m, n, k, _stream(stream)))


def qlinear_forward(fmt: int, w, x, out, m: int, n: int, k: int, bias=None, stream=None) -> None:
    """QLinear::forward: out[m][n] = x[m][k] . W[n][k] (+ bias[n]) for a weight of
    format fmt (LINEAR_Q4K, LINEAR_BF16, LINEAR_F32, LINEAR_Q6K or LINEAR_Q8_0)."""
    check(lib().rt_qlinear_forward(fmt, _p(w), None if bias is None else _p(bias), _p(x), _p(out), m, n, k,
                                   _stream(stream)))


def qlinear_forward_host(fmt: int, w, x, bias=None):
    """QLinear::forward on host numpy arrays: w (Q4_K blocks, BF16 bits or f32
    [n, k]), x [m, k] f32, bias [n] or None -> [m, n] f32 (weights cached)."""
    import numpy as np
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w)
    m, k = x.shape
    n = {LINEAR_Q4K: w.size // (k // 256 * 144) if k % 256 == 0 else 0, LINEAR_BF16: w.size // k,
         LINEAR_F32: w.size // k}.get(fmt, 0)
    out = np.empty((m, max(n, 1)), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    check(lib().rt_qlinear_forward_host(fmt, w.ctypes.data, w.nbytes, None if b is None else b.ctypes.data,
                                        x.ctypes.data, out.ctypes.data, m, n, k))
    return out


def q6k_dequant_f32(w, out, n_blocks: int, stream=None) -> None:
    check(lib().rt_q6k_dequant_f32(_p(w), n_blocks, _p(out), _stream(stream)))


def q8_0_dequant_f32(w, out, n_elem: int, stream=None) -> None:
    check(lib().rt_q8_0_dequant_f32(_p(w), n_elem, _p(out), _stream(stream)))


def q6k_repack(gguf_bytes):
    """GGUF Q6_K block bytes (numpy uint8) -> the planar device layout (numpy)."""
    import numpy as np
    src = np.ascontiguousarray(gguf_bytes, np.uint8)
    if src.size % 210:
        raise RtError(RT_EINVAL, f"Q6_K data of {src.size} bytes is not whole 210-byte blocks")
    out = np.empty_like(src)
    check(lib().rt_q6k_repack(src.ctypes.data, src.size // 210, out.ctypes.data))
    return out


def q8_0_repack(gguf_bytes):
    """GGUF Q8_0 block bytes (numpy uint8) -> the planar device layout (numpy)."""
    import numpy as np
    src = np.ascontiguousarray(gguf_bytes, np.uint8)
    if src.size % 34:
        raise RtError(RT_EINVAL, f"Q8_0 data of {src.size} bytes is not whole 34-byte blocks")
    out = np.empty_like(src)
    check(lib().rt_q8_0_repack(src.ctypes.data, src.size // 34, out.ctypes.data))
    return out


def q4k_gemm(a, w, c, m: int, n: int, k: int, stream=None) -> None:
    """C[m,n] = A[m,k] . W[n,k]^T on device; A is a bf16 or f32 tensor (bf16 may be
    passed as int16/uint16 bits), W packed Q4_K bytes, C f32."""
    import torch
    if a.dtype in (torch.bfloat16, torch.int16, getattr(torch, "uint16", torch.int16)):
        check(lib().rt_q4k_gemm_bf16(_p(a), _p(w), _p(c), m, n, k, _stream(stream)))
    elif a.dtype == torch.float32:
        check(lib().rt_q4k_gemm_f32(_p(a), _p(w), _p(c), m, n, k, _stream(stream)))
    else:
        raise TypeError(f"q4k_gemm: activations must be bfloat16 or float32, got {a.dtype}")


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


def matmul_q4k_t(a, blocks, rows: int):
    """Q4KMat::matmul_q4k_t_exact: a [m, k] f32 (numpy) -> [m, rows] f32."""
    import numpy as np
    a = np.ascontiguousarray(a, np.float32)
    if a.ndim == 1:
        a = a.reshape(1, -1)
    blocks = np.ascontiguousarray(blocks, np.uint8)
    m, k = a.shape
    out = np.empty((m, rows), np.float32)
    check(lib().rt_matmul_q4k_t(a.ctypes.data, m, k, blocks.ctypes.data, rows, out.ctypes.data))
    return out


def weight_cache_clear() -> None:
    check(lib().rt_weight_cache_clear())


def gemm_workspace_release(stream=None) -> None:
    """Free this thread's GEMM / batched-GEMV workspace for `stream` (torch
    stream or None for the null stream) on the current device."""
    check(lib().rt_gemm_workspace_release(_stream(stream)))


def gemm_workspace_held(stream=None) -> int:
    return int(lib().rt_gemm_workspace_held(_stream(stream)))


# ---------------------------------------------------------------------------
# Gemma-3 decode engine (rt_decode_*), mirrors MetalDecodeContext
# ---------------------------------------------------------------------------
class Gemma3Config(C.Structure):
    """rt_gemma3_config (Config4, transformer4.rs:112-131)."""
    _fields_ = [(n, C.c_int32) for n in ("hidden", "ffn", "n_q_heads", "n_kv_heads", "head_dim", "n_layers",
                                         "vocab", "sliding_window", "global_every", "max_seq")] + \
               [(n, C.c_float) for n in ("rope_theta_local", "rope_theta_global", "rope_fs_local",
                                         "rope_fs_global", "eps", "attn_scale")]


class Gemma3Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "in_norm", "post_attn_norm",
                                          "pre_ffn_norm", "post_ffn_norm", "q_norm", "k_norm")]


GEMMA3_4B = dict(hidden=2560, ffn=10240, n_q_heads=8, n_kv_heads=4, head_dim=256, n_layers=34, vocab=262144,
                 sliding_window=1024, global_every=6, rope_theta_local=10000.0, rope_theta_global=1000000.0,
                 rope_fs_local=1.0, rope_fs_global=0.125, eps=1e-6, attn_scale=1.0 / 16.0)
"""Config4::gemma3_4b (transformer4.rs:112-131) with vocab 262144 (the GGUF
embedding table size, metal_decode.rs lm_head_vocab)."""


def _addr(x) -> int:
    if isinstance(x, int):
        return x
    if hasattr(x, "ptr") and hasattr(x, "format"):  # a Linear loaded from GGUF (device memory)
        return x.ptr
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    import numpy as np
    assert isinstance(x, np.ndarray) and x.flags["C_CONTIGUOUS"]
    return x.ctypes.data


class DecodeMemory(C.Structure):
    _fields_ = [(k, C.c_uint64) for k in ("weights", "kv_cache", "activation", "batch", "prefill", "total")]


class HipDecodeContext:
    """One Gemma-3 decode context on the current HIP device.

    new / set_layer / set_embed / sync_kv_from_cpu / decode_step mirror
    MetalDecodeContext::{new, sync_kv_from_cpu, decode_step}
    (metal_decode.rs:971, 1366, 2028).  Arrays may be numpy (host, copied) or
    torch cuda tensors (device, borrowed: keep them alive)."""

    def __init__(self, cfg: dict, max_seq: int):
        fields = {k: cfg[k] for k, _ in Gemma3Config._fields_ if k != "max_seq"}
        self.cfg = dict(cfg, max_seq=max_seq)
        self._c = Gemma3Config(max_seq=max_seq, **fields)
        h = C.c_void_p()
        check(lib().rt_decode_create(C.byref(self._c), C.byref(h)))
        self._h = h
        self._keep = []

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().rt_decode_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _on_device(x) -> int:
        return int((hasattr(x, "is_cuda") and x.is_cuda) or (hasattr(x, "ptr") and hasattr(x, "format")))

    PROJECTIONS = ("q", "k", "v", "o", "gate", "up", "down")

    def set_layer(self, i: int, w: dict, formats=None) -> None:
        """w: the 7 projections and 6 norm vectors (Gemma3Layer fields); all
        host arrays, or all device memory (torch cuda tensors or GGUF-loaded
        `Linear`s).  formats: RT_LINEAR_* per projection (q, k, v, o, gate, up,
        down); by default a `Linear`'s own format, else Q4_K."""
        if formats is None:
            formats = [getattr(w[k], "format", LINEAR_Q4K) for k in self.PROJECTIONS]
        elif isinstance(formats, dict):
            formats = [formats.get(k, LINEAR_Q4K) for k in self.PROJECTIONS]
        dev = self._on_device(w["q"])
        L = Gemma3Layer(**{k: _addr(w[k]) for k, _ in Gemma3Layer._fields_})
        if dev:
            self._keep.append(w)
        f = (C.c_int32 * 7)(*formats)
        check(lib().rt_decode_set_layer_formats(self._h, i, C.byref(L), f, dev))

    def set_embed(self, embed, final_norm) -> None:
        dev = self._on_device(embed)
        if dev:
            self._keep.append((embed, final_norm))
        check(lib().rt_decode_set_embed(self._h, _addr(embed), _addr(final_norm), dev))

    def set_lm_head(self, fmt: int = 0, w=None) -> None:
        """An lm_head apart from the embedding: LINEAR_Q4K blocks [vocab][hidden/256]
        or LINEAR_BF16 [vocab, hidden]; w None restores the tied embedding."""
        dev = self._on_device(w) if w is not None else 0
        if dev:
            self._keep.append(w)
        check(lib().rt_decode_set_lm_head(self._h, fmt, _addr(w) if w is not None else None, dev))

    def sync_kv_from_cpu(self, layer: int, k, v, seq_len: int) -> None:
        check(lib().rt_decode_sync_kv(self._h, layer, _addr(k), _addr(v), seq_len, self._on_device(k)))

    def decode_step(self, token: int, position: int):
        import numpy as np
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().rt_decode_step(self._h, token, position, out.ctypes.data))
        return out

    def decode_step_batch(self, tokens, start_position: int):
        """decode_step_batch (metal_decode.rs:2079-2179): logits [m, vocab] for
        m <= 8 tokens at start_position, start_position+1, ..."""
        import numpy as np
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        out = np.empty((t.size, self.cfg["vocab"]), np.float32)
        check(lib().rt_decode_step_batch(self._h, t.ctypes.data, t.size, start_position, out.ctypes.data))
        return out

    def decode_step_batch_async(self, tokens, start_position: int) -> None:
        import numpy as np
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        check(lib().rt_decode_step_batch_async(self._h, t.ctypes.data, t.size, start_position))

    PREFILL_REFERENCE, PREFILL_SLIDING = 0, 1

    def prefill(self, tokens, start_position: int = 0, mode: int = 0):
        """GPU prefill (replaces the CPU prefill of generate_cached_streaming,
        transformer4.rs:2103-2139, and sync_kv_from_cpu): fills KV rows
        start_position .. start_position+len(tokens)-1 and returns the last
        token's logits.  mode PREFILL_REFERENCE (0) keeps the reference's
        prefill window rule (start_position 0); PREFILL_SLIDING (1) windows every
        row like a decode step."""
        import numpy as np
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().rt_decode_prefill(self._h, t.ctypes.data, t.size, start_position, mode, out.ctypes.data))
        return out

    def set_prefill_chunk(self, rows: int) -> None:
        check(lib().rt_decode_set_prefill_chunk(self._h, rows))

    def decode_step_async(self, token: int, position: int) -> None:
        check(lib().rt_decode_step_async(self._h, token, position))

    def synchronize(self) -> None:
        check(lib().rt_decode_synchronize(self._h))

    def set_graph(self, enabled: bool) -> None:
        check(lib().rt_decode_set_graph(self._h, int(enabled)))

    @property
    def verify_batched(self) -> bool:
        """True when decode_step_batch runs the M tokens through each layer
        together (batched GEMVs, one pass over the weights)."""
        v = C.c_int32(0)
        check(lib().rt_decode_verify_batched(self._h, C.byref(v)))
        return bool(v.value)

    def memory(self) -> dict:
        """Device bytes by what they hold (print_metal_memory, metal_decode.rs:1285-1354)."""
        m = DecodeMemory()
        check(lib().rt_decode_memory(self._h, C.byref(m)))
        return {k: int(getattr(m, k)) for k, _ in DecodeMemory._fields_}

    def print_memory(self) -> None:
        """The reference's one-line report, in MB."""
        m = self.memory()
        print("[ HIP ] GPU buffer memory: " + "  ".join(
            f"{k}={m[k] / 1048576.0:.1f} MB" for k in ("weights", "kv_cache", "activation", "batch", "prefill", "total")),
            file=sys.stderr)

    def logits_ptr(self) -> int:
        p = C.c_void_p()
        check(lib().rt_decode_logits(self._h, C.byref(p)))
        return p.value

    def kv_ptrs(self, layer: int) -> tuple[int, int]:
        k, v = C.c_void_p(), C.c_void_p()
        check(lib().rt_decode_kv(self._h, layer, C.byref(k), C.byref(v)))
        return k.value, v.value

    def stream_ptr(self) -> int:
        s = C.c_void_p()
        check(lib().rt_decode_get_stream(self._h, C.byref(s)))
        return s.value


from .gguf import GgufFile, GgufTensorInfo, Linear, load_linear_from_gguf, q4k_quantize, q4k_quantize_bf16  # noqa: E402,F401
from . import generate  # noqa: E402,F401
from .generate import GEMMA3_EOS, NgramDraftEngine, generate_greedy, greedy_token  # noqa: E402,F401
