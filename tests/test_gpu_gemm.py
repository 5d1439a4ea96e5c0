"""GPU parity of the Q4_K GEMM (matrix-core path) against the CPU oracle, called
through the C ABI (rt_q4k_gemm_bf16 / rt_q4k_gemm_f32 / rt_matmul_q4k_t).

The reference result is the oracle's Q4_K dequantisation (bit-exact with
autograd2.rs:1326-1366 and gguf_loader.rs:551-621, pinned in test_oracle.py)
multiplied by A in float64, and, at small sizes, the oracle's scalar f32
restatement of matmul_q4k_t itself (autograd2.rs:1437-1457)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3  # rel-L2 bound for fp32 accumulation against the reference CPU path


def _sync():
    import torch
    torch.cuda.synchronize()


def _bf16_activations(seed: int, m: int, k: int, orc):
    """N(0,1) activations rounded to bf16: (bits as int16 tensor on CPU, exact f64 values)."""
    import torch
    a = torch.from_numpy(orc.synth_normal(seed, m * k).reshape(m, k)).to(torch.bfloat16)
    return a.view(torch.int16), a.to(torch.float64).numpy()


def _reference(orc, a64, blocks, n, k):
    w = orc.q4k_dequant_gguf(blocks, n * k).reshape(n, k).astype(np.float64)
    return a64 @ w.T


def _run_bf16(rt, dev, a_bits, blocks, m, n, k):
    import torch
    c = torch.empty(m, n, dtype=torch.float32, device=dev)
    rt.q4k_gemm(a_bits.to(dev), to_dev(blocks, dev), c, m, n, k)
    _sync()
    return c.cpu().numpy()


@pytest.mark.parametrize("m,n,k,seed", [
    (2, 256, 256, 1),        # smaller than one tile
    (17, 300, 512, 2),       # ragged M and N (N not a multiple of 16)
    (130, 260, 768, 3),      # ragged, more than one tile each way
    (64, 2048, 2560, 4),     # Gemma q-projection shape, short prompt
    (512, 10240, 2560, 5),   # prefill, gate/up shape
    (512, 2560, 10240, 6),   # prefill, down-projection shape
    (1100, 1024, 2560, 7),   # above 1024 rows: half-block kernel, K split 4 ways, ragged M
    (2100, 2560, 10240, 8),  # half-block kernel, K split 3 ways (long-prompt down shape)
    (1024, 2560, 2048, 9),   # the kernel switch: eight-wave kernel up to 1024 rows (K split 2 ways) ...
    (1025, 2560, 2048, 10),  # ... half-block kernel from 1025 (K split 2 ways), one ragged row
    (1000, 16384, 512, 11),  # under 1024 rows with 512 tiles: half-block kernel, ragged M
])
def test_gemm_bf16_vs_oracle(rt, orc, dev, m, n, k, seed):
    blocks = orc.synth_q4k(100 + seed, n, k)
    a_bits, a64 = _bf16_activations(seed, m, k, orc)
    got = _run_bf16(rt, dev, a_bits, blocks, m, n, k)
    ref = _reference(orc, a64, blocks, n, k)
    err = rel_l2(got, ref)
    print(f"gemm bf16 m={m} n={n} k={k}: rel-L2 vs f64 {err:.3e}")
    assert np.all(np.isfinite(got))
    assert err < GEMM_TOL


@pytest.mark.parametrize("m,n,k", [
    (4608, 9216, 3072),    # FLUX-12B QKV: half-block kernel (648 tiles of 256 x 256)
    (4608, 12288, 3072),   # FLUX-12B MLP up: half-block kernel
    (4608, 3072, 12288),   # FLUX-12B MLP down: 256 x 256 kernel (216 tiles), one round
    (4096, 2560, 10240),   # 4096-row prefill down: 256 x 256 kernel, K split 3 ways
    (4096, 2560, 2048),    # 4096-row prefill o: 256 x 256 kernel (160 tiles)
    (1500, 5632, 8192),    # 256 x 256 kernel, K split 3 ways, ragged M
    (1300, 9000, 2560),    # 256 x 256 kernel, ragged M and N
])
def test_gemm_flux_shapes(rt, orc, dev, m, n, k):
    """FLUX-12B shapes (QKV, MLP-up, MLP-down) and the shapes that take the
    256 x 256-tile kernel; reference on the GPU in f32 from the oracle's
    dequantised weights (a library GEMM, not this library's kernels)."""
    import torch
    blocks = orc.synth_q4k(7 + n, n, k)
    a = torch.from_numpy(orc.synth_normal(11 + k, m * k).reshape(m, k)).to(torch.bfloat16)
    w = torch.from_numpy(orc.q4k_dequant_gguf(blocks, n * k).reshape(n, k)).to(dev)
    c = torch.empty(m, n, dtype=torch.float32, device=dev)
    ad = a.to(dev)
    rt.q4k_gemm(ad.view(torch.int16), to_dev(blocks, dev), c, m, n, k)
    ref = ad.float() @ w.T
    _sync()
    err = float((c.double() - ref.double()).norm() / ref.double().norm())
    print(f"gemm bf16 m={m} n={n} k={k}: rel-L2 vs f32 library GEMM {err:.3e}")
    assert torch.isfinite(c).all()
    assert err < GEMM_TOL


def test_gemm_vs_scalar_oracle(rt, orc, dev):
    """Against the literal restatement of matmul_q4k_t (f32, sequential k)."""
    import torch
    m, n, k = 48, 1024, 2560
    blocks = orc.synth_q4k(21, n, k)
    a = orc.synth_normal(22, m * k).reshape(m, k)
    ref = orc.q4k_matmul(a, blocks, n, k)
    c = torch.empty(m, n, dtype=torch.float32, device=dev)
    rt.q4k_gemm(to_dev(a, dev), to_dev(blocks, dev), c, m, n, k)
    _sync()
    err = rel_l2(c.cpu().numpy(), ref)
    print(f"gemm f32 vs scalar oracle rel-L2 {err:.3e}")
    assert err < GEMM_TOL


def test_gemm_extreme_row_scales(rt, orc, dev):
    """Per-row power-of-two scaling: rows of A at 2^100, 2^-100, zero, one-hot;
    W rows with huge d (|w| far beyond f16's 65504) and subnormal d.

    Criterion per element: |C - ref| <= 2e-3 * ||a_i * w_j||_2, the error scale
    of rounding both operands to an 11-bit significand (unit roundoff 2^-11)
    with exact products and f32 sums.  It is independent of cancellation in
    the result, and it fails if a row or column lost its scale: A at 2^-100 or
    d = 2^-24 underflows f16 without one, and d = 1000 overflows it."""
    import torch
    m, n, k = 8, 64, 512
    blocks = orc.synth_q4k(31, n, k).reshape(n, k // 256, 144)
    blocks[3, :, 0:2] = np.array([0x63D0], np.uint16).view(np.uint8)   # d = 1000.0
    blocks[3, :, 2:4] = np.array([0x5A40], np.uint16).view(np.uint8)   # dmin = 200.0
    blocks[5, :, 0:2] = np.array([0x0001], np.uint16).view(np.uint8)   # d = dmin = 2^-24 (subnormal)
    blocks[5, :, 2:4] = np.array([0x0001], np.uint16).view(np.uint8)
    blocks = blocks.reshape(-1)
    a = orc.synth_normal(32, m * k).reshape(m, k).astype(np.float64)
    a[1] *= 2.0 ** 100
    a[2] *= 2.0 ** -100
    a[3] = 0.0
    a[4] = 0.0
    a[4, 77] = 3.0
    a32 = a.astype(np.float32)
    c = torch.empty(m, n, dtype=torch.float32, device=dev)
    rt.q4k_gemm(to_dev(a32, dev), to_dev(blocks, dev), c, m, n, k)
    _sync()
    got = c.cpu().numpy().astype(np.float64)
    a64 = a32.astype(np.float64)
    w64 = orc.q4k_dequant_gguf(blocks, n * k).reshape(n, k).astype(np.float64)
    ref = a64 @ w64.T
    scale = np.sqrt((a64 ** 2) @ (w64 ** 2).T)
    assert np.all(np.isfinite(got))
    assert np.all(got[3] == 0.0)
    bound = 2e-3 * scale
    bad = np.argwhere(np.abs(got - ref) > bound)
    assert bad.size == 0, f"elements outside the f16 rounding bound: {bad[:8].tolist()}"
    # away from the planted columns the usual rel-L2 bar holds row by row
    keep = np.setdiff1d(np.arange(n), [3, 5])
    for r in (0, 1, 2, 4):
        assert rel_l2(got[r, keep], ref[r, keep]) < GEMM_TOL, r


def test_gemm_nan_row_propagates(rt, orc, dev):
    import torch
    m, n, k = 4, 128, 256
    blocks = orc.synth_q4k(41, n, k)
    a = orc.synth_normal(42, m * k).reshape(m, k)
    a[2, 5] = np.nan
    c = torch.empty(m, n, dtype=torch.float32, device=dev)
    rt.q4k_gemm(to_dev(a, dev), to_dev(blocks, dev), c, m, n, k)
    _sync()
    got = c.cpu().numpy()
    assert np.all(np.isnan(got[2]))
    assert np.all(np.isfinite(np.delete(got, 2, axis=0)))


def test_gemm_deterministic(rt, orc, dev):
    import torch
    m, n, k = 256, 1024, 2560
    blocks = to_dev(orc.synth_q4k(51, n, k), dev)
    a_bits, _ = _bf16_activations(52, m, k, orc)
    ad = a_bits.to(dev)
    c1 = torch.empty(m, n, dtype=torch.float32, device=dev)
    c2 = torch.empty_like(c1)
    rt.q4k_gemm(ad, blocks, c1, m, n, k)
    rt.q4k_gemm(ad, blocks, c2, m, n, k)
    _sync()
    assert torch.equal(c1, c2)


def test_matmul_q4k_t_host(rt, orc):
    """Host drop-in (Q4KMat::matmul_q4k_t_exact): M>1 through the GEMM, M=1
    through the GEMV exactly like rt_gemv_q4k_t (autograd2.rs:1440-1443)."""
    n, k = 512, 1024
    blocks = orc.synth_q4k(61, n, k)
    a = orc.synth_normal(62, 3 * k).reshape(3, k)
    got = rt.matmul_q4k_t(a, blocks, n)
    ref = orc.q4k_matmul(a, blocks, n, k)
    assert got.shape == (3, n)
    assert rel_l2(got, ref) < GEMM_TOL
    one = rt.matmul_q4k_t(a[:1], blocks, n)
    assert np.array_equal(one[0], rt.gemv_q4k_t(a[0], blocks, n))
    rt.weight_cache_clear()


def test_gemm_workspace_under_graph_capture(rt, orc, dev):
    """A stream's workspace does not grow during a capture: the call returns
    RT_ESTATE before launching anything.  After one uncaptured call of that
    size the same call captures, and every replay (with eager work on the
    stream between replays) equals the eager result."""
    import ctypes as C
    import torch
    hip = C.CDLL("libamdhip64.so")
    m, n, k = 300, 1024, 2560
    blocks = to_dev(orc.synth_q4k(55, n, k), dev)
    a_bits, _ = _bf16_activations(56, m, k, orc)
    a = a_bits.to(dev)
    s = torch.cuda.Stream()
    c = torch.zeros(m, n, dtype=torch.float32, device=dev)
    assert hip.hipStreamBeginCapture(C.c_void_p(s.cuda_stream), 2) == 0  # hipStreamCaptureModeRelaxed
    with pytest.raises(rt.RtError) as err:
        rt.q4k_gemm(a, blocks, c, m, n, k, stream=s)
    graph = C.c_void_p()
    assert hip.hipStreamEndCapture(C.c_void_p(s.cuda_stream), C.byref(graph)) == 0
    if graph.value:
        hip.hipGraphDestroy(graph)
    assert err.value.code == rt.RT_ESTATE
    rt.q4k_gemm(a, blocks, c, m, n, k, stream=s)  # uncaptured: the workspace grows
    s.synchronize()
    eager = c.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rt.q4k_gemm(a, blocks, c, m, n, k, stream=s)
    for _ in range(3):
        c.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, eager)
