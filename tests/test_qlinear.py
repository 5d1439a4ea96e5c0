"""QLinear::forward (qlinear.rs:82-111) through rt_qlinear_forward: the
matmul of the weight's format (Q4_K, BF16, F32, and the Q6_K / Q8_0 the
reference widens to BF16) plus add_bias_rows (qlinear.rs:49-60).

The oracle's orc_qlinear_forward is pinned by the reference's own QLinear
tests (qlinear.rs:161-202, restated with their fixture formula) and by a
float64 product; the GPU path is held to the oracle."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import rel_l2, to_dev
from test_kquant import synth_q6k, synth_q8_0

F_Q4K, F_BF16, F_F32, F_Q6K, F_Q80 = 1, 2, 3, 4, 5


def spread(rows: int, cols: int, scale: float, salt: int) -> np.ndarray:
    """The reference's test fixture (qlinear.rs:144-149): element (r, c) from
    i = (r*131 + c*37 + salt*7919) % 251, (sin(0.41 i)*0.7 + cos(0.13 i)*0.3)*scale."""
    r, c = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    i = ((r * 131 + c * 37 + salt * 7919) % 251).astype(np.float32)
    return ((np.sin(i * np.float32(0.41)) * np.float32(0.7) + np.cos(i * np.float32(0.13)) * np.float32(0.3))
            * np.float32(scale)).astype(np.float32)


def spread_vec(n: int, scale: float, salt: int) -> np.ndarray:
    """qlinear.rs:151-158: k = (i*53 + salt*6151) % 241, (sin(0.29 k)*0.6 + cos(0.17 k)*0.4)*scale."""
    k = ((np.arange(n) * 53 + salt * 6151) % 241).astype(np.float32)
    return ((np.sin(k * np.float32(0.29)) * np.float32(0.6) + np.cos(k * np.float32(0.17)) * np.float32(0.4))
            * np.float32(scale)).astype(np.float32)


def to_bf16_bits(w: np.ndarray, orc) -> np.ndarray:
    return np.array([orc.f32_to_bf16(float(v)) for v in w.reshape(-1)], np.uint16)


# ---------------------------------------------------------------------------
# oracle pins (CPU)
# ---------------------------------------------------------------------------
def test_oracle_agrees_across_weight_formats(orc):
    """qlinear.rs:161-179: f32 and bf16 weights give the same output to 0.05."""
    w, b, x = spread(6, 8, 1.0, 5), spread_vec(6, 0.5, 6), spread(4, 8, 1.0, 7)
    rf = orc.qlinear_forward(F_F32, x, w, 6, 8, b)
    rh = orc.qlinear_forward(F_BF16, x, to_bf16_bits(w, orc), 6, 8, b)
    assert rf.shape == (4, 6)
    assert np.all(np.abs(rf - rh) < 0.05)


def test_oracle_applies_bias_once_per_row(orc):
    """qlinear.rs:181-193: biased = plain + b, element by element."""
    w, x = spread(3, 5, 1.0, 8), spread(4, 5, 1.0, 9)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    plain = orc.qlinear_forward(F_F32, x, w, 3, 5)
    biased = orc.qlinear_forward(F_F32, x, w, 3, 5, b)
    assert np.array_equal(biased, plain + b)  # one f32 add per element: exact


def test_oracle_f32_matmul_vs_float64(orc):
    rng = np.random.default_rng(3)
    x, w = rng.standard_normal((5, 300)).astype(np.float32), rng.standard_normal((17, 300)).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert rel_l2(orc.qlinear_forward(F_F32, x, w, 17, 300), ref) < 2e-6  # sequential f32 sum of 300 terms


def test_qlinear_rejects_before_launch(rt):
    """Bad calls fail on the host (the pointers here are never dereferenced)."""
    L = rt.lib()
    buf = (C.c_uint8 * 64)()
    p = (C.addressof(buf) + 15) & ~15
    assert L.rt_qlinear_forward(7, p, None, p, p, 1, 4, 256, None) == rt.RT_EINVAL  # no such format
    assert L.rt_qlinear_forward(F_F32, p, None, p, p, 1, 4, 6, None) == rt.RT_EINVAL  # f32 rows in 16-byte loads
    assert L.rt_qlinear_forward(F_F32, p, p + 2, p, p, 1, 4, 8, None) == rt.RT_EINVAL  # bias not 4-byte aligned
    assert L.rt_qlinear_forward(F_BF16, p, None, p, p, 2, 4, 12, None) == rt.RT_EINVAL  # eight weights per load
    assert L.rt_qlinear_forward(F_BF16, p, None, p, p, 9, 4, 12, None) == rt.RT_EINVAL
    assert L.rt_qlinear_forward(F_F32, p, None, p, p, 0, 4, 8, None) == rt.RT_EINVAL
    assert L.rt_qlinear_forward(F_F32, None, None, p, p, 1, 4, 8, None) == rt.RT_EINVAL


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
def _weights(orc, fmt: int, n: int, k: int, seed: int):
    """(device-layout weight bytes, oracle-layout weight bytes, dequantised f32 [n, k])."""
    rng = np.random.default_rng(seed)
    if fmt == F_F32:
        w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        return w, w, w
    if fmt == F_BF16:
        w = orc.synth_bf16(seed, n * k)
        return w, w, (w.astype(np.uint32) << 16).view(np.float32).reshape(n, k)
    if fmt == F_Q6K:
        src = synth_q6k(rng, n * k // 256)
        return None, src, orc.q6k_dequant(src, n * k).reshape(n, k)
    if fmt == F_Q80:
        src = synth_q8_0(rng, n * k // 32)
        return None, src, orc.q8_0_dequant(src, n * k).reshape(n, k)
    w = orc.synth_q4k(seed, n, k)
    return w, w, orc.q4k_dequant(w, n, k).reshape(n, k)


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k", [(1, 2560, 2560), (3, 257, 264), (8, 1024, 2048), (11, 300, 264), (40, 520, 512),
                                   (300, 2560, 1024), (1, 6, 8)])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("fmt", [F_F32, F_BF16])
def test_qlinear_f32_bf16_weights_vs_oracle(rt, orc, dev, m, n, k, with_bias, fmt):
    """F32 and BF16 weights: up to 8 rows per group on the f32-arithmetic GEMV
    (also any m when k is not a multiple of 64), else the matrix cores on f16
    operands."""
    import torch
    w, _, _ = _weights(orc, fmt, n, k, 10 + m + n)
    x = np.random.default_rng(20 + k).standard_normal((m, k)).astype(np.float32)
    b = np.random.default_rng(30 + n).standard_normal(n).astype(np.float32) if with_bias else None
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    rt.qlinear_forward(fmt, to_dev(w, dev), to_dev(x, dev), out, m, n, k,
                       bias=None if b is None else to_dev(b, dev))
    torch.cuda.synchronize()
    ref = orc.qlinear_forward(fmt, x, w, n, k, b)
    f32_path = m <= 8 or k % 64 != 0
    assert rel_l2(out.cpu().numpy(), ref) < (1e-5 if f32_path else 1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", [F_Q4K, F_BF16, F_Q6K, F_Q80, F_F32])
def test_qlinear_bias_every_format(rt, orc, dev, fmt):
    """With a bias the output is the unbiased output plus the bias, exactly
    (one f32 add, as add_bias_rows), and both agree with the oracle."""
    import torch
    m, n, k = 37, 384, 512
    w_dev, w_orc, _ = _weights(orc, fmt, n, k, 40 + fmt)
    if fmt == F_Q6K:
        w_dev = rt.q6k_repack(w_orc)
    elif fmt == F_Q80:
        w_dev = rt.q8_0_repack(w_orc)
    x = np.random.default_rng(41).standard_normal((m, k)).astype(np.float32)
    b = np.random.default_rng(42).standard_normal(n).astype(np.float32)
    wd, xd = to_dev(w_dev, dev), to_dev(x, dev)
    plain = torch.empty((m, n), dtype=torch.float32, device=dev)
    biased = torch.empty((m, n), dtype=torch.float32, device=dev)
    rt.qlinear_forward(fmt, wd, xd, plain, m, n, k)
    rt.qlinear_forward(fmt, wd, xd, biased, m, n, k, bias=to_dev(b, dev))
    torch.cuda.synchronize()
    p, q = plain.cpu().numpy(), biased.cpu().numpy()
    assert np.array_equal(q, p + b)
    ref = orc.qlinear_forward(fmt, x, w_orc, n, k, b)
    assert rel_l2(q, ref) < 1e-3


@pytest.mark.gpu
def test_qlinear_reference_fixture_on_gpu(rt, orc, dev):
    """qlinear.rs:161-179 on the device: f32 and bf16 weights agree to 0.05."""
    import torch
    w, b, x = spread(6, 8, 1.0, 5), spread_vec(6, 0.5, 6), spread(4, 8, 1.0, 7)
    outs = []
    for fmt, wb in ((F_F32, w), (F_BF16, to_bf16_bits(w, orc))):
        o = torch.empty((4, 6), dtype=torch.float32, device=dev)
        rt.qlinear_forward(fmt, to_dev(wb, dev), to_dev(x, dev), o, 4, 6, 8, bias=to_dev(b, dev))
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
    assert np.all(np.abs(outs[0] - outs[1]) < 0.05)
    assert rel_l2(outs[0], orc.qlinear_forward(F_F32, x, w, 6, 8, b)) < 1e-5


def test_qlinear_host_rejects_before_upload(rt):
    """Weight sizes that do not match the shape, and formats a QLinear never
    holds, fail before anything is uploaded."""
    import numpy as np
    x = np.zeros((2, 256), np.float32)
    with pytest.raises(rt.RtError, match="needs"):
        rt.qlinear_forward_host(F_F32, np.zeros(255 * 3, np.float32), x)
    with pytest.raises(rt.RtError, match="QLinear holds"):
        rt.qlinear_forward_host(F_Q6K, np.zeros(210, np.uint8), x)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", [F_Q4K, F_BF16, F_F32])
def test_qlinear_host_drop_in(rt, orc, dev, fmt):
    """The host drop-in (cached weight, staged x / bias / out) equals the device
    entry point's result on the same inputs, and the oracle within tolerance."""
    import torch
    m, n, k = 5, 300, 512
    w, w_orc, _ = _weights(orc, fmt, n, k, 70 + fmt)
    x = np.random.default_rng(71).standard_normal((m, k)).astype(np.float32)
    b = np.random.default_rng(72).standard_normal(n).astype(np.float32)
    got = rt.qlinear_forward_host(fmt, w, x, b)
    again = rt.qlinear_forward_host(fmt, w, x, b)  # second call: cached weight
    o = torch.empty((m, n), dtype=torch.float32, device=dev)
    rt.qlinear_forward(fmt, to_dev(w, dev), to_dev(x, dev), o, m, n, k, bias=to_dev(b, dev))
    torch.cuda.synchronize()
    assert np.array_equal(got, again) and np.array_equal(got, o.cpu().numpy())
    assert rel_l2(got, orc.qlinear_forward(fmt, x, w_orc, n, k, b)) < 1e-3
    rt.weight_cache_clear()
