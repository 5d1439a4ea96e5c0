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
