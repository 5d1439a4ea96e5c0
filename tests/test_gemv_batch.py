"""Batched Q4_K GEMV (rt_q4k_gemv_batch, gemv_q4k_t_batch of
metal_decode.rs:459-521): every row of the batch against the float64 GEMV
of the oracle's dequantisation."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import rel_l2, to_dev


def test_batch_gemv_rejects_bad_calls(rt):
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    L = rt.lib()
    assert L.rt_q4k_gemv_batch(addr, addr, addr, 0, 64, 256, None) == rt.RT_EINVAL
    assert L.rt_q4k_gemv_batch(addr, addr, addr, 9, 64, 256, None) == rt.RT_EINVAL
    assert "outside [1, 8]" in L.rt_last_error().decode()
    assert L.rt_q4k_gemv_batch(addr, addr, addr, 2, 64, 300, None) == rt.RT_EINVAL


# decode shapes (K split into one-super-block slices), ragged row counts that
# end inside a 64-row workgroup and a 16-row wave, one super-block (no split)
SHAPES = [(10240, 2560), (2560, 10240), (2560, 2048), (2048, 2560), (1024, 2560), (100, 512), (37, 256)]


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("n,k", SHAPES)
def test_batch_gemv_matches_float64(rt, orc, dev, n, k, m):
    import torch
    blocks = orc.synth_q4k(900 + n + k, n, k)
    a = np.stack([orc.synth_normal(1000 + 7 * i + k, k) for i in range(m)])
    a[m // 2] *= 1e-3  # a row of another magnitude (per-row, per-chunk scales)
    c = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    rt.q4k_gemv_batch(to_dev(blocks, dev), to_dev(a, dev), c, m, n, k)
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    # 15-bit activation digits per 64-element chunk: ~3e-5 on long rows; rows
    # of one or two super-blocks average fewer rounding errors (up to ~1e-4)
    tol = 1e-4 if k >= 2048 else 3e-4
    for i in range(m):
        ref = orc.q4k_gemv_f64(blocks, n, k, a[i])
        assert rel_l2(got[i], ref) < tol, (i, rel_l2(got[i], ref))


@pytest.mark.gpu
def test_batch_gemv_is_deterministic_and_row_independent(rt, orc, dev):
    """Same rows give the same bits in any batch position and call; a row's
    result does not depend on the other rows of the batch."""
    import torch
    n, k = 2560, 10240
    blocks = to_dev(orc.synth_q4k(77, n, k), dev)
    a = np.stack([orc.synth_normal(78 + i, k) for i in range(8)])
    c8 = torch.empty((8, n), dtype=torch.float32, device=dev)
    c1 = torch.empty((1, n), dtype=torch.float32, device=dev)
    rt.q4k_gemv_batch(blocks, to_dev(a, dev), c8, 8, n, k)
    first = c8.clone()
    rt.q4k_gemv_batch(blocks, to_dev(a, dev), c8, 8, n, k)
    rt.q4k_gemv_batch(blocks, to_dev(a[5:6], dev), c1, 1, n, k)
    torch.cuda.synchronize()
    assert torch.equal(first, c8)
    assert torch.equal(c1[0], c8[5])


# ---------------------------------------------------------------------------
# Q6_K, Q8_0 and BF16 (rt_linear_gemv_batch: gemv_bf16_t_batch,
# metal_decode.rs:527-558, and the same batch for the k-quants kept packed)
# ---------------------------------------------------------------------------
Q6K, Q8_0, BF16 = 4, 5, 2
# decode shapes (one-super-block and four-super-block K slices), ragged row
# counts, and rows of whole 64-element chunks that are not whole super-blocks
# (Q8_0 / BF16 only: K slices of two chunks and of one)
LIN_SHAPES = [(fmt, n, k) for fmt in (Q6K, Q8_0, BF16)
              for n, k in ((1024, 2560), (2560, 10240), (2560, 2048), (10240, 2560), (100, 512))] + \
             [(Q8_0, 130, 1152), (BF16, 130, 1152), (Q8_0, 70, 576), (BF16, 70, 64), (Q6K, 37, 768)]


def linear_weights(rt, orc, fmt, n, k, seed):
    """(device bytes, float64 dequantised [n, k]) of a synthetic weight."""
    from test_kquant import synth_q6k, synth_q8_0
    rng = np.random.default_rng(seed)
    if fmt == Q6K:
        src = synth_q6k(rng, n * k // 256)
        return rt.q6k_repack(src), orc.q6k_dequant(src, n * k).reshape(n, k).astype(np.float64)
    if fmt == Q8_0:
        src = synth_q8_0(rng, n * k // 32)
        return rt.q8_0_repack(src), orc.q8_0_dequant(src, n * k).reshape(n, k).astype(np.float64)
    w = orc.synth_bf16(seed, n * k)
    return w, (w.astype(np.uint32) << 16).view(np.float32).reshape(n, k).astype(np.float64)


def test_linear_gemv_batch_rejects_bad_calls(rt):
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    L = rt.lib()
    assert L.rt_linear_gemv_batch(Q6K, addr, addr, addr, 2, 64, 320, None) == rt.RT_EINVAL  # Q6_K: whole super-blocks
    assert "multiple of 256" in L.rt_last_error().decode()
    assert L.rt_linear_gemv_batch(Q8_0, addr, addr, addr, 2, 64, 96, None) == rt.RT_EINVAL  # 64-element chunks
    assert L.rt_linear_gemv_batch(BF16, addr, addr, addr, 9, 64, 256, None) == rt.RT_EINVAL
    assert L.rt_linear_gemv_batch(3, addr, addr, addr, 2, 64, 256, None) == rt.RT_EINVAL  # F32 has none
    assert "no batched GEMV" in L.rt_last_error().decode()
    assert L.rt_linear_gemv_batch(BF16, addr + 4, addr, addr, 2, 64, 256, None) == rt.RT_EINVAL


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("fmt,n,k", LIN_SHAPES)
def test_linear_gemv_batch_matches_float64(rt, orc, dev, fmt, n, k, m):
    import torch
    w, W = linear_weights(rt, orc, fmt, n, k, 4000 + fmt * 100 + n + k)
    a = np.stack([orc.synth_normal(5000 + 7 * i + k, k) for i in range(m)])
    a[m // 2] *= 1e-3  # a row of another magnitude
    c = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    rt.linear_gemv_batch(fmt, to_dev(w, dev), to_dev(a, dev), c, m, n, k)
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    ref = a.astype(np.float64) @ W.T
    # Q6_K / Q8_0: 16-bit activation digits per 64-element chunk (~3e-5 on
    # long rows, more on rows of a few chunks); BF16: x split into bf16
    # hi + lo (2^-17) with the weights exact, f32 accumulation
    tol = 2e-5 if fmt == BF16 else (1e-4 if k >= 2048 else 3e-4)
    for i in range(m):
        assert rel_l2(got[i], ref[i]) < tol, (i, rel_l2(got[i], ref[i]))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", [Q6K, Q8_0, BF16])
def test_linear_gemv_batch_is_row_independent(rt, orc, dev, fmt):
    """A row gives the same bits alone and in any batch position; x*4 scales
    the result exactly for the digit-staged formats."""
    import torch
    n, k = 2560, 2560
    w, _ = linear_weights(rt, orc, fmt, n, k, 77 + fmt)
    wd = to_dev(w, dev)
    a = np.stack([orc.synth_normal(78 + i, k) for i in range(8)])
    c8 = torch.empty((8, n), dtype=torch.float32, device=dev)
    c1 = torch.empty((1, n), dtype=torch.float32, device=dev)
    c4 = torch.empty((1, n), dtype=torch.float32, device=dev)
    rt.linear_gemv_batch(fmt, wd, to_dev(a, dev), c8, 8, n, k)
    rt.linear_gemv_batch(fmt, wd, to_dev(a[5:6], dev), c1, 1, n, k)
    rt.linear_gemv_batch(fmt, wd, to_dev(4 * a[5:6], dev), c4, 1, n, k)
    torch.cuda.synchronize()
    assert torch.equal(c1[0], c8[5])
    if fmt != BF16:
        assert torch.equal(c4[0], 4 * c1[0])


@pytest.mark.gpu
def test_gemm_workspace_release_frees_and_regrows(rt, orc, dev):
    """rt_gemm_workspace_release frees the stream's workspace (held bytes
    drop to 0) and the next call allocates it again with the same result."""
    import torch
    n, k = 1024, 2560
    blocks = to_dev(orc.synth_q4k(55, n, k), dev)
    a = to_dev(np.stack([orc.synth_normal(56 + i, k) for i in range(4)]), dev)
    c0 = torch.empty((4, n), dtype=torch.float32, device=dev)
    c1 = torch.empty_like(c0)
    rt.q4k_gemv_batch(blocks, a, c0, 4, n, k)
    assert rt.gemm_workspace_held() > 0
    rt.gemm_workspace_release()
    assert rt.gemm_workspace_held() == 0
    rt.gemm_workspace_release()  # nothing held: a no-op
    rt.q4k_gemv_batch(blocks, a, c1, 4, n, k)
    torch.cuda.synchronize()
    assert rt.gemm_workspace_held() > 0
    assert torch.equal(c0, c1)
