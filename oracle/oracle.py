"""ctypes binding of liboracle.so -- the CPU restatement of rich-triplet's
portable x86 decode path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing that is
measured or shipped.  Each wrapper names the reference file:line it follows
(paths relative to the rich-triplet checkout, src/...).
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build() -> None:
    """Compile liboracle.so from oracle/rt_oracle.c (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None
_lib_path = None


def use_native_build(out_dir: str) -> str:
    """Compile rt_oracle.c for this host's CPU (gcc -O3 -march=native, still
    -ffp-contract=off: no fused multiply-adds, no reassociation, so the
    results equal liboracle.so's) into out_dir, and bind that library
    instead.  For the CPU baseline, which is timed on the GPU box's host."""
    global _lib, _lib_path
    so = os.path.join(out_dir, "liboracle_native.so")
    subprocess.run(["gcc", "-O3", "-march=native", "-std=c11", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
                    "-pthread", "-shared", "-o", so, str(HERE / "rt_oracle.c"), "-lm"], check=True)
    _lib, _lib_path = None, so
    lib()
    return so


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if _lib_path is None and not LIB_PATH.exists():
            build()
        L = C.CDLL(str(_lib_path or LIB_PATH))
        sig = {
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16_rne": (C.c_uint16, [C.c_float]),
            "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "orc_q4k_scale_min": (None, [_u8p, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
            "orc_q4k_pack_scales": (None, [_u8p, _u8p, _u8p]),
            "orc_q4k_dequant_row": (None, [_u8p, _sz, _sz, _f32p]),
            "orc_q4k_dequant_gguf": (None, [_u8p, _sz, _f32p]),
            "orc_f32_to_f16_trunc": (C.c_uint16, [C.c_float]),
            "orc_q4k_quantize_block": (None, [_f32p, _u8p]),
            "orc_q4k_quantize": (None, [_f32p, _sz, _sz, _u8p]),
            "orc_q4_0_dequant": (None, [_u8p, _sz, _f32p]),
            "orc_q4_0_to_q4k": (None, [_u8p, _sz, _sz, _u8p]),
            "orc_q6k_dequant": (None, [_u8p, _sz, _f32p]),
            "orc_q5k_dequant": (None, [_u8p, _sz, _f32p]),
            "orc_q8_0_dequant": (None, [_u8p, _sz, _f32p]),
            "orc_q4k_dot_row": (C.c_float, [_u8p, _sz, _sz, _f32p]),
            "orc_q4k_gemv_mt": (None, [_u8p, _sz, _sz, _f32p, _f32p, C.c_int]),
            "orc_q4k_gemv_f64": (None, [_u8p, _sz, _sz, _f32p, _f64p]),
            "orc_bf16_dot_row": (C.c_float, [_u16p, _sz, _sz, _f32p]),
            "orc_bf16_gemv_mt": (None, [_u16p, _sz, _sz, _f32p, _f32p, C.c_int]),
            "orc_bf16_gemv_f64": (None, [_u16p, _sz, _sz, _f32p, _f64p]),
            "orc_q4k_matmul": (None, [_f32p, _sz, _u8p, _sz, _sz, _f32p, C.c_int]),
            "orc_q4k_matmul_f64": (None, [_f32p, _sz, _u8p, _sz, _sz, _f64p, C.c_int]),
            "orc_rms_norm_gemma3": (None, [_f32p, _f32p, _sz, C.c_float, _f32p]),
            "orc_per_head_norm": (None, [_f32p, _f32p, _sz, _sz, C.c_float, _f32p]),
            "orc_rope_neox": (None, [_f32p, _sz, _sz, C.c_float, _sz, C.c_float]),
            "orc_gelu_tanh": (C.c_float, [C.c_float]),
            "orc_gqa_attention_decode": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz, C.c_float, _f32p]),
            "orc_rng_u64": (C.c_uint64, [C.c_uint64, C.c_uint64]),
            "orc_synth_normal_f32": (None, [C.c_uint64, _sz, C.c_float, C.c_float, _f32p]),
            "orc_synth_bf16": (None, [C.c_uint64, _sz, C.c_float, _u16p]),
            "orc_synth_q4k": (None, [C.c_uint64, _sz, C.c_float, _u8p]),
            "orc_hw_threads": (C.c_int, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        L.orc_gemma3_decode_step.restype = None
        L.orc_gemma3_layer.restype = None
        _lib = L
    return _lib


# ---------------------------------------------------------------------------
# scalar conversions
# ---------------------------------------------------------------------------
def f16_to_f32(bits: int) -> float:
    """autograd2.rs:1048-1070"""
    return lib().orc_f16_to_f32(bits)


def f32_to_f16_rne(v: float) -> int:
    return lib().orc_f32_to_f16_rne(v)


def bf16_to_f32(bits: int) -> float:
    """autograd2.rs:700-703"""
    return lib().orc_bf16_to_f32(bits)


def f32_to_bf16(v: float) -> int:
    """autograd2.rs:709-719"""
    return lib().orc_f32_to_bf16(v)


# ---------------------------------------------------------------------------
# Q4_K
# ---------------------------------------------------------------------------
def scale_min(sc: np.ndarray, j: int) -> tuple[float, float]:
    """autograd2.rs:1075-1085"""
    sv, mv = C.c_float(), C.c_float()
    lib().orc_q4k_scale_min(np.ascontiguousarray(sc, np.uint8), j, C.byref(sv), C.byref(mv))
    return sv.value, mv.value


def pack_scales(sv, mv) -> np.ndarray:
    """autograd2.rs:1119-1132"""
    out = np.zeros(12, np.uint8)
    lib().orc_q4k_pack_scales(np.asarray(sv, np.uint8), np.asarray(mv, np.uint8), out)
    return out


def q4k_dequant(blocks: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Q4KMat::dequantize_row_into for every row: autograd2.rs:1326-1366."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty((rows, cols), np.float32)
    L = lib()
    for r in range(rows):
        row = np.empty(cols, np.float32)
        L.orc_q4k_dequant_row(blocks, cols, r, row)
        out[r] = row
    return out


def q4k_dequant_gguf(blocks: np.ndarray, n_elem: int) -> np.ndarray:
    """gguf_loader.rs:551-621"""
    out = np.empty(n_elem, np.float32)
    lib().orc_q4k_dequant_gguf(np.ascontiguousarray(blocks, np.uint8), n_elem, out)
    return out


def f32_to_f16_trunc(v: float) -> int:
    """Q4KMat::f32_to_f16 (autograd2.rs:1090-1117): mantissa truncated."""
    return int(lib().orc_f32_to_f16_trunc(float(v)))


def q4k_quantize(m: np.ndarray) -> np.ndarray:
    """Q4KMat::quantize (autograd2.rs:1138-1168, quantize_block 1171-1245); m is [rows, cols]."""
    m = np.ascontiguousarray(m, np.float32)
    rows, cols = m.shape
    out = np.zeros(rows * (cols // 256) * 144, np.uint8)
    lib().orc_q4k_quantize(m, rows, cols, out)
    return out


def _dequant(fn: str, nbytes_per_block: int, elems_per_block: int):
    def run(data: np.ndarray, n_elem: int) -> np.ndarray:
        data = np.ascontiguousarray(data, np.uint8)
        assert data.size >= (n_elem + elems_per_block - 1) // elems_per_block * nbytes_per_block
        out = np.empty(n_elem, np.float32)
        getattr(lib(), fn)(data, n_elem, out)
        return out
    return run


q4_0_dequant = _dequant("orc_q4_0_dequant", 18, 32)    # gguf_loader.rs:425-480
q6k_dequant = _dequant("orc_q6k_dequant", 210, 256)    # gguf_loader.rs:482-549
q5k_dequant = _dequant("orc_q5k_dequant", 176, 256)    # gguf_loader.rs:664-743
q8_0_dequant = _dequant("orc_q8_0_dequant", 34, 32)    # gguf_loader.rs:628-650


def q4_0_to_q4k(data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """load_linear_from_gguf's Q4_0 branch (transformer4.rs:1198-1207): Q4_0 bytes
    of a [cols, rows] GGUF tensor -> Q4_K blocks of the [rows, cols] matrix."""
    out = np.zeros(rows * (cols // 256) * 144, np.uint8)
    lib().orc_q4_0_to_q4k(np.ascontiguousarray(data, np.uint8), rows, cols, out)
    return out


def q4k_gemv(blocks: np.ndarray, rows: int, cols: int, a: np.ndarray, threads: int = 0) -> np.ndarray:
    """Q4KMat::gemv_mt / dot_row (x86): autograd2.rs:1953-2035, 1654-1701."""
    y = np.empty(rows, np.float32)
    lib().orc_q4k_gemv_mt(np.ascontiguousarray(blocks, np.uint8), rows, cols,
                          np.ascontiguousarray(a, np.float32), y, threads)
    return y


def q4k_gemv_f64(blocks: np.ndarray, rows: int, cols: int, a: np.ndarray) -> np.ndarray:
    y = np.empty(rows, np.float64)
    lib().orc_q4k_gemv_f64(np.ascontiguousarray(blocks, np.uint8), rows, cols,
                           np.ascontiguousarray(a, np.float32), y)
    return y


def bf16_gemv(w: np.ndarray, rows: int, cols: int, a: np.ndarray, threads: int = 0) -> np.ndarray:
    """MatBf16::gemv_mt / dot_row (x86): autograd2.rs:954-1000, 879-887."""
    y = np.empty(rows, np.float32)
    lib().orc_bf16_gemv_mt(np.ascontiguousarray(w, np.uint16), rows, cols,
                           np.ascontiguousarray(a, np.float32), y, threads)
    return y


def bf16_gemv_f64(w: np.ndarray, rows: int, cols: int, a: np.ndarray) -> np.ndarray:
    y = np.empty(rows, np.float64)
    lib().orc_bf16_gemv_f64(np.ascontiguousarray(w, np.uint16), rows, cols,
                            np.ascontiguousarray(a, np.float32), y)
    return y


def q4k_matmul(a: np.ndarray, blocks: np.ndarray, n: int, k: int, threads: int = 0) -> np.ndarray:
    """matmul_q4k_t M>1 (scalar order): autograd2.rs:1437-1457."""
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    c = np.empty((m, n), np.float32)
    lib().orc_q4k_matmul(a, m, np.ascontiguousarray(blocks, np.uint8), n, k, c, threads)
    return c


def q4k_matmul_f64(a: np.ndarray, blocks: np.ndarray, n: int, k: int, threads: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    c = np.empty((m, n), np.float64)
    lib().orc_q4k_matmul_f64(a, m, np.ascontiguousarray(blocks, np.uint8), n, k, c, threads)
    return c


# ---------------------------------------------------------------------------
# decode-step math
# ---------------------------------------------------------------------------
def rms_norm_gemma3(x: np.ndarray, gamma: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """autograd2.rs:3477-3496"""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rms_norm_gemma3(x, np.ascontiguousarray(gamma, np.float32), x.size, eps, out)
    return out


def per_head_norm(x, gamma, n_heads, head_dim, eps=1e-6):
    """transformer4.rs:2485-2508"""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_per_head_norm(x, np.ascontiguousarray(gamma, np.float32), n_heads, head_dim, eps, out)
    return out


def rope_neox(x, n_heads, head_dim, theta, pos, freq_scale):
    """transformer4.rs:2742-2772 (returns a rotated copy)."""
    y = np.array(x, np.float32, copy=True)
    lib().orc_rope_neox(y, n_heads, head_dim, theta, pos, freq_scale)
    return y


def gelu_tanh(v: float) -> float:
    """autograd2.rs:3082-3091"""
    return lib().orc_gelu_tanh(v)


def gqa_attention_decode(q, k_cache, v_cache, k_start, k_end, n_q_heads, n_kv_heads, d_head, scale):
    """transformer4.rs:2806-2879 (t_q == 1, non-BLAS loops)."""
    out = np.empty(n_q_heads * d_head, np.float32)
    lib().orc_gqa_attention_decode(np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k_cache, np.float32),
                                   np.ascontiguousarray(v_cache, np.float32), k_start, k_end, n_q_heads,
                                   n_kv_heads, d_head, scale, out)
    return out


# ---------------------------------------------------------------------------
# Gemma-3 decode step
# ---------------------------------------------------------------------------
class Gemma3Cfg(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("hidden", "ffn", "n_q_heads", "n_kv_heads", "head_dim", "n_layers",
                                         "vocab", "sliding_window", "global_every")] + \
               [(n, C.c_float) for n in ("rope_theta_local", "rope_theta_global", "rope_fs_local",
                                         "rope_fs_global", "eps", "attn_scale")]


class Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "in_norm", "post_attn_norm",
                                          "pre_ffn_norm", "post_ffn_norm", "q_norm", "k_norm", "k_cache",
                                          "v_cache")] + [("fmt", C.c_int32 * 7)]


PROJECTIONS = ("q", "k", "v", "o", "gate", "up", "down")


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def make_cfg(d: dict) -> Gemma3Cfg:
    return Gemma3Cfg(**{k: d[k] for k, _ in Gemma3Cfg._fields_})


def make_layers(layers: list[dict]) -> C.Array:
    """Layer dicts -> orc_layer array.  An optional L["fmt"] maps projection
    names to formats (1 Q4_K, 2 BF16, 4 Q6_K and 5 Q8_0 in GGUF block bytes)."""
    arr = (Layer * len(layers))()
    for i, L in enumerate(layers):
        for name, _ in Layer._fields_:
            if name != "fmt":
                setattr(arr[i], name, _ptr(L[name]))
        fmt = L.get("fmt", {})
        arr[i].fmt = (C.c_int32 * 7)(*[fmt.get(p, 1) for p in PROJECTIONS])
    return arr


def gemma3_decode_step(cfg: dict, layers: list[dict], embed: np.ndarray, final_norm: np.ndarray,
                       token: int, pos: int, threads: int = 0, want_hidden: bool = False):
    """transformer4.rs:2358-2385 + Gemma3Block::forward_cached (1954-1964).

    Mutates every layer's k_cache / v_cache (row `pos`), like the reference's
    cache.append."""
    c = make_cfg(cfg)
    arr = make_layers(layers)
    logits = np.empty(cfg["vocab"], np.float32)
    hidden = np.empty(cfg["hidden"], np.float32)
    lib().orc_gemma3_decode_step(C.byref(c), arr, C.c_void_p(_ptr(embed)), C.c_void_p(_ptr(final_norm)),
                                 C.c_uint32(token), C.c_uint32(pos), C.c_void_p(_ptr(logits)),
                                 C.c_void_p(_ptr(hidden)), C.c_int(threads))
    return (logits, hidden) if want_hidden else logits


def proj_gemv(fmt: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """orc_proj_gemv: y = W x for a projection of format fmt."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    lib().orc_proj_gemv(C.c_int(fmt), C.c_void_p(_ptr(np.ascontiguousarray(w))), C.c_size_t(rows),
                        C.c_size_t(cols), C.c_void_p(_ptr(x)), C.c_void_p(_ptr(y)), C.c_int(threads))
    return y


def proj_matmul(fmt: int, a: np.ndarray, w: np.ndarray, n: int, k: int, threads: int = 0) -> np.ndarray:
    """orc_proj_matmul: C = A W^T for a projection of format fmt."""
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    c = np.empty((m, n), np.float32)
    lib().orc_proj_matmul(C.c_int(fmt), C.c_void_p(_ptr(a)), C.c_size_t(m), C.c_void_p(_ptr(np.ascontiguousarray(w))),
                          C.c_size_t(n), C.c_size_t(k), C.c_void_p(_ptr(c)), C.c_int(threads))
    return c


def qlinear_forward(fmt: int, a: np.ndarray, w: np.ndarray, n: int, k: int, bias=None, threads: int = 0) -> np.ndarray:
    """orc_qlinear_forward: QLinear::forward, C = A W^T (+ bias) for a weight of
    format fmt (1 Q4_K, 2 BF16, 3 F32 [n, k], 4 Q6_K, 5 Q8_0 GGUF blocks)."""
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    c = np.empty((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_qlinear_forward(C.c_int(fmt), C.c_void_p(_ptr(a)), C.c_size_t(m),
                              C.c_void_p(_ptr(np.ascontiguousarray(w))), C.c_void_p(None if b is None else _ptr(b)),
                              C.c_size_t(n), C.c_size_t(k), C.c_void_p(_ptr(c)), C.c_int(threads))
    return c


def gqa_attention_prefill(q, k_cache, v_cache, p0, T, lo_fixed, window, n_q_heads, n_kv_heads, d_head, scale):
    """orc_gqa_attention_prefill: rows p0 .. p0+T-1, keys [lo(r), r]."""
    q = np.ascontiguousarray(q, np.float32)
    k_cache = np.ascontiguousarray(k_cache, np.float32)
    v_cache = np.ascontiguousarray(v_cache, np.float32)
    out = np.empty((T, n_q_heads * d_head), np.float32)
    lib().orc_gqa_attention_prefill(C.c_void_p(_ptr(q)), C.c_void_p(_ptr(k_cache)), C.c_void_p(_ptr(v_cache)),
                                    C.c_size_t(p0), C.c_size_t(T), C.c_size_t(lo_fixed), C.c_size_t(window),
                                    C.c_size_t(n_q_heads), C.c_size_t(n_kv_heads), C.c_size_t(d_head),
                                    C.c_float(scale), C.c_void_p(_ptr(out)))
    return out


def gemma3_prefill(cfg: dict, layers: list[dict], embed: np.ndarray, final_norm: np.ndarray, tokens,
                   start: int = 0, mode: int = 0, threads: int = 0) -> np.ndarray:
    """Prefill of `tokens` at positions start.. (forward_cached over the prompt,
    transformer4.rs:1900-1964 and 2103-2139); mode 0 = the reference's prefill
    window rule, 1 = per-row sliding window.  Mutates the layers' caches."""
    c = make_cfg(cfg)
    arr = make_layers(layers)
    t = np.ascontiguousarray(np.asarray(tokens, np.uint32))
    logits = np.empty(cfg["vocab"], np.float32)
    lib().orc_gemma3_prefill(C.byref(c), arr, C.c_void_p(_ptr(embed)), C.c_void_p(_ptr(final_norm)),
                             C.c_void_p(_ptr(t)), C.c_size_t(t.size), C.c_size_t(start), C.c_int(mode),
                             C.c_void_p(_ptr(logits)), C.c_int(threads))
    return logits


# ---------------------------------------------------------------------------
# seeded synthetic data
# ---------------------------------------------------------------------------
def synth_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_normal_f32(seed, n, mean, std, out)
    return out


def synth_bf16(seed: int, n: int, std: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().orc_synth_bf16(seed, n, std, out)
    return out


def synth_q4k(seed: int, rows: int, cols: int, d_std: float = 0.02) -> np.ndarray:
    """Random Q4_K blocks as specified for the benchmark configs: f16 d, dmin =
    |N(0, d_std)|, 6-bit scales/mins uniform 0..63, nibbles uniform 0..15."""
    assert cols % 256 == 0
    nb = rows * cols // 256
    out = np.empty(nb * 144, np.uint8)
    lib().orc_synth_q4k(seed, nb, d_std, out)
    return out


def hw_threads() -> int:
    return lib().orc_hw_threads()


GEMMA3_4B = dict(hidden=2560, ffn=10240, n_q_heads=8, n_kv_heads=4, head_dim=256, n_layers=34, vocab=262144,
                 sliding_window=1024, global_every=6, rope_theta_local=10000.0, rope_theta_global=1000000.0,
                 rope_fs_local=1.0, rope_fs_global=0.125, eps=1e-6, attn_scale=1.0 / 16.0)
"""Config4::gemma3_4b (transformer4.rs:112-131) with BASELINE's vocab 262144."""

if os.environ.get("RT_ORACLE_BUILD_ON_IMPORT") == "1":
    build()
