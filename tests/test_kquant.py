"""Q6_K / Q8_0 kept packed on the device (kquant.hip): the planar repack, the
dequantisation (bit-exact with the oracle's restatements of
decode_q6k_to_f32 / decode_q8_0_to_f32, gguf_loader.rs:482-549 and 628-650)
and the native GEMVs (vs float64 products of those dequantised weights)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2, to_dev


def synth_q6k(rng, n_blocks: int) -> np.ndarray:
    """GGUF Q6_K blocks: random ql/qh bytes, int8 scales, d = f16 of |N(0, 0.02)|."""
    b = rng.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.02, n_blocks)).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return b.reshape(-1)


def synth_q8_0(rng, n_blocks: int) -> np.ndarray:
    b = rng.integers(0, 256, size=(n_blocks, 34), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.02, n_blocks)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    return b.reshape(-1)


# ---------------------------------------------------------------------------
# CPU: the planar layout
# ---------------------------------------------------------------------------
def test_q6k_repack_planes(rt):
    rng = np.random.default_rng(1)
    n = 7
    src = synth_q6k(rng, n)
    out = rt.q6k_repack(src)
    blk = src.reshape(n, 210)
    assert np.array_equal(out[:n * 128].reshape(n, 128), blk[:, :128])
    assert np.array_equal(out[n * 128:n * 192].reshape(n, 64), blk[:, 128:192])
    assert np.array_equal(out[n * 192:n * 208].reshape(n, 16), blk[:, 192:208])
    assert np.array_equal(out[n * 208:].reshape(n, 2), blk[:, 208:])


def test_q8_0_repack_planes(rt):
    rng = np.random.default_rng(2)
    n = 9
    src = synth_q8_0(rng, n)
    out = rt.q8_0_repack(src)
    blk = src.reshape(n, 34)
    assert np.array_equal(out[:n * 32].reshape(n, 32), blk[:, 2:])
    assert np.array_equal(out[n * 32:].reshape(n, 2), blk[:, :2])


def test_repack_rejects_partial_blocks(rt):
    with pytest.raises(rt.RtError):
        rt.q6k_repack(np.zeros(211, np.uint8))
    with pytest.raises(rt.RtError):
        rt.q8_0_repack(np.zeros(35, np.uint8))


def test_gemv_entry_points_validate_shapes(rt):
    import ctypes as C
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    L = rt.lib()
    assert L.rt_q6k_gemv(addr, addr, addr, 4, 300, None) == rt.RT_EINVAL
    assert "multiple of 256" in L.rt_last_error().decode()
    assert L.rt_q8_0_gemv(addr, addr, addr, 4, 48, None) == rt.RT_EINVAL
    assert L.rt_q8_0_gemv(addr + 4, addr, addr, 4, 64, None) == rt.RT_EINVAL
    assert L.rt_q8_0_dequant_f32(addr, 33, addr, None) == rt.RT_EINVAL


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
@pytest.mark.gpu
def test_q6k_dequant_bit_exact(rt, orc, dev):
    import torch
    rng = np.random.default_rng(3)
    n_blocks = 1000
    src = synth_q6k(rng, n_blocks)
    src[:210 * 4].reshape(4, 210)[:, 192:208] = np.array([-128, 127, 0, 1, -1, 64, -64, 5] * 2,
                                                         np.int8).view(np.uint8)  # extreme scales
    w = to_dev(rt.q6k_repack(src), dev)
    out = torch.empty(n_blocks * 256, dtype=torch.float32, device=dev)
    rt.q6k_dequant_f32(w, out, n_blocks)
    torch.cuda.synchronize()
    ref = orc.q6k_dequant(src, n_blocks * 256)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
def test_q8_0_dequant_bit_exact(rt, orc, dev):
    import torch
    rng = np.random.default_rng(4)
    n_blocks = 2000
    src = synth_q8_0(rng, n_blocks)
    w = to_dev(rt.q8_0_repack(src), dev)
    out = torch.empty(n_blocks * 32, dtype=torch.float32, device=dev)
    rt.q8_0_dequant_f32(w, out, n_blocks * 32)
    torch.cuda.synchronize()
    ref = orc.q8_0_dequant(src, n_blocks * 32)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


# Shapes: the decode projections (v 1024x2560, down 2560x10240, o 2560x2048),
# the two-iteration tile (N >= 4096), ragged row counts, and K without a
# specialised tile (generic kernel).
Q6K_SHAPES = [(1024, 2560), (2560, 10240), (2560, 2048), (4096, 2560), (1001, 2560), (37, 768), (5, 256)]
Q8_SHAPES = [(1024, 2560), (2560, 10240), (2560, 2048), (4100, 2560), (1001, 2560), (37, 96), (3, 32)]


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", Q6K_SHAPES)
def test_q6k_gemv_matches_float64(rt, orc, dev, n, k):
    import torch
    rng = np.random.default_rng(n + k)
    src = synth_q6k(rng, n * k // 256)
    x = rng.standard_normal(k).astype(np.float32)
    w = to_dev(rt.q6k_repack(src), dev)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    rt.q6k_gemv(w, to_dev(x, dev), y, n, k)
    torch.cuda.synchronize()
    W = orc.q6k_dequant(src, n * k).reshape(n, k).astype(np.float64)
    ref = W @ x.astype(np.float64)
    # digit-staged activations: ~3e-5 rel-L2 (16-bit integer digits per 64-chunk)
    assert rel_l2(y.cpu().numpy(), ref) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", Q8_SHAPES)
def test_q8_0_gemv_matches_float64(rt, orc, dev, n, k):
    import torch
    rng = np.random.default_rng(n * 3 + k)
    src = synth_q8_0(rng, n * k // 32)
    x = rng.standard_normal(k).astype(np.float32)
    w = to_dev(rt.q8_0_repack(src), dev)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    rt.q8_0_gemv(w, to_dev(x, dev), y, n, k)
    torch.cuda.synchronize()
    W = orc.q8_0_dequant(src, n * k).reshape(n, k).astype(np.float64)
    ref = W @ x.astype(np.float64)
    assert rel_l2(y.cpu().numpy(), ref) < 1e-4


@pytest.mark.gpu
def test_q6k_gemv_scaled_and_onehot_inputs(rt, orc, dev):
    """x*4 scales y exactly (power-of-two digits); a one-hot x returns the
    dequantised column up to the 2^-15 digit step."""
    import torch
    n, k = 512, 2560
    rng = np.random.default_rng(9)
    src = synth_q6k(rng, n * k // 256)
    w = to_dev(rt.q6k_repack(src), dev)
    x = rng.standard_normal(k).astype(np.float32)
    y1 = torch.empty(n, dtype=torch.float32, device=dev)
    y4 = torch.empty(n, dtype=torch.float32, device=dev)
    rt.q6k_gemv(w, to_dev(x, dev), y1, n, k)
    rt.q6k_gemv(w, to_dev(4 * x, dev), y4, n, k)
    e = np.zeros(k, np.float32)
    e[1234] = 1.0
    ye = torch.empty(n, dtype=torch.float32, device=dev)
    rt.q6k_gemv(w, to_dev(e, dev), ye, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(y4.cpu().numpy(), 4 * y1.cpu().numpy())
    col = orc.q6k_dequant(src, n * k).reshape(n, k)[:, 1234]
    assert np.allclose(ye.cpu().numpy(), col, rtol=1e-6, atol=0)
