"""rt_q4k_gemv_batch_noalloc: the batched Q4_K GEMV on a fixed per-GPU
workspace.  It has no counterpart in the reference; its results must equal
rt_q4k_gemv_batch's (same kernels) bit for bit, also when a call follows
another one of a different size on the same workspace."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import rel_l2, to_dev


def test_noalloc_rejects_oversize_and_bad_calls(rt):
    """Shapes whose workspace exceeds the fixed array fail before any launch."""
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    L = rt.lib()
    cap = L.rt_noalloc_scratch_bytes()
    assert cap == 8 << 20
    # k = 2560: 10 K slices x 8 rows x 4 bytes = 320 bytes of partials per output row
    n_big = cap // 320 + 1
    assert L.rt_q4k_gemv_batch_noalloc(addr, addr, addr, 2, n_big, 2560, None) == rt.RT_EINVAL
    assert "workspace" in L.rt_last_error().decode()
    assert L.rt_q4k_gemv_batch_noalloc(addr, addr, addr, 9, 64, 256, None) == rt.RT_EINVAL
    assert L.rt_q4k_gemv_batch_noalloc(addr, addr, addr, 2, 64, 300, None) == rt.RT_EINVAL
    assert L.rt_q4k_gemv_batch_noalloc(None, addr, addr, 2, 64, 256, None) == rt.RT_EINVAL


@pytest.mark.gpu
def test_noalloc_equals_batch_entry_point(rt, orc, dev):
    """Three calls in a row on the shared workspace, each smaller than the one
    before (rows, batch and K split all change), against rt_q4k_gemv_batch."""
    import torch
    cases = [(8, 10240, 2560), (3, 2560, 10240), (1, 1024, 2560)]
    for i, (m, n, k) in enumerate(cases):
        print(f"noalloc case {i}: m={m} n={n} k={k}", flush=True)
        blocks = orc.synth_q4k(4000 + i, n, k)
        a = np.stack([orc.synth_normal(4100 + 10 * i + r, k) for r in range(m)])
        w_d, a_d = to_dev(blocks, dev), to_dev(a, dev)
        c_ref = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        c_na = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        rt.q4k_gemv_batch(w_d, a_d, c_ref, m, n, k)
        rt.q4k_gemv_batch_noalloc(w_d, a_d, c_na, m, n, k)
        torch.cuda.synchronize()
        assert torch.equal(c_na, c_ref), i
        got = c_na.cpu().numpy()
        for r in range(m):
            assert rel_l2(got[r], orc.q4k_gemv_f64(blocks, n, k, a[r])) < 1e-4, (i, r)
