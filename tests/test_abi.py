"""The C-ABI library loads, exports every symbol include/*.h declares, and
rejects bad shapes on the host before any GPU work (no GPU needed)."""
from __future__ import annotations

import ctypes as C
import pathlib
import re

import pytest

from conftest import REPO


def declared_symbols() -> set[str]:
    names = set()
    for h in (REPO / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(rt_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    assert {"rt_q4k_gemv", "rt_bf16_gemv", "rt_q4k_dequant_f32", "rt_last_error"} <= names


def test_library_exports_every_declared_symbol(rt):
    lib = rt.lib()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(rt.exported_symbols()) <= declared_symbols()
    assert lib.rt_abi_version() >= 1


@pytest.mark.parametrize("n,k,what", [(16, 100, "multiple of 256"), (0, 256, "positive"), (16, -256, "positive")])
def test_q4k_gemv_rejects_bad_shapes_before_launch(rt, n, k, what):
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    st = rt.lib().rt_q4k_gemv(addr, addr, addr, n, k, None)
    assert st == rt.RT_EINVAL
    assert what in rt.lib().rt_last_error().decode()


def test_null_and_misaligned_pointers_are_rejected(rt):
    L = rt.lib()
    assert L.rt_q4k_gemv(None, None, None, 16, 256, None) == rt.RT_EINVAL
    buf = (C.c_uint8 * 64)()
    addr = ((C.addressof(buf) + 15) & ~15) + 4
    assert L.rt_bf16_gemv(addr, addr, addr, 16, 256, None) == rt.RT_EINVAL
    assert "aligned" in L.rt_last_error().decode()
    assert L.rt_bf16_gemv(addr - 4, addr - 4, addr - 4, 16, 12, None) == rt.RT_EINVAL
    assert L.rt_gemv_q4k_t(None, 256, None, 4, None) == rt.RT_EINVAL
    with pytest.raises(rt.RtError):
        rt.check(L.rt_gemv_bf16_t(addr, 7, addr, 4, addr))


@pytest.mark.parametrize("m,n,k,what", [(0, 16, 256, "positive"), (4, 16, 300, "multiple of 256"),
                                        (4, -1, 256, "positive"), (2 ** 31, 16, 256, "int32")])
def test_q4k_gemm_rejects_bad_shapes_before_launch(rt, m, n, k, what):
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    for fn in (rt.lib().rt_q4k_gemm_bf16, rt.lib().rt_q4k_gemm_f32):
        assert fn(addr, addr, addr, m, n, k, None) == rt.RT_EINVAL
        assert what in rt.lib().rt_last_error().decode()


def test_q4k_gemm_rejects_null_and_misaligned(rt):
    L = rt.lib()
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    assert L.rt_q4k_gemm_bf16(None, addr, addr, 4, 16, 256, None) == rt.RT_EINVAL
    assert L.rt_q4k_gemm_f32(addr + 4, addr, addr, 4, 16, 256, None) == rt.RT_EINVAL
    assert "aligned" in L.rt_last_error().decode()
    assert L.rt_q4k_gemm_f32(addr, addr, addr + 2, 4, 16, 256, None) == rt.RT_EINVAL
    assert L.rt_matmul_q4k_t(None, 2, 256, None, 4, None) == rt.RT_EINVAL
    assert L.rt_matmul_q4k_t(addr, 2, 100, addr, 4, addr) == rt.RT_EINVAL


def test_measurement_probes_reject_bad_arguments_before_launch(rt):
    """rt_stream_read_cfg (kinds 0..3: strided or sliced, plain or nontemporal
    loads) and rt_empty_launch check their arguments before any HIP call."""
    L = rt.lib()
    buf = (C.c_uint8 * 64)()
    addr = (C.addressof(buf) + 15) & ~15
    assert L.rt_stream_read_cfg(addr, 16, addr, None, 4, 0) == rt.RT_EINVAL
    assert "kind" in L.rt_last_error().decode()
    assert L.rt_stream_read_cfg(addr, 16, addr, None, -1, 0) == rt.RT_EINVAL
    assert L.rt_stream_read_cfg(addr, 16, addr, None, 2, 70000) == rt.RT_EINVAL
    assert L.rt_stream_read_cfg(addr + 4, 16, addr, None, 3, 0) == rt.RT_EINVAL
    assert L.rt_stream_read_cfg(None, 16, addr, None, 0, 0) == rt.RT_EINVAL
    assert L.rt_stream_read_cfg(addr, 0, addr, None, 3, 0) == rt.RT_OK  # nothing to read
    assert L.rt_empty_launch(0, 64, None) == rt.RT_EINVAL
    assert L.rt_empty_launch(1, 2048, None) == rt.RT_EINVAL


def test_zero_block_dequant_is_a_no_op(rt):
    assert rt.lib().rt_q4k_dequant_f32(None, 0, None, None) == rt.RT_OK


def test_trace_read_refused_without_traced_build(rt):
    """rt_trace_read belongs to the RT_TRACE build (librt_hip_trace.so); the
    product library refuses it with RT_ESTATE and a message naming the build,
    before any HIP call."""
    if "trace" in str(rt.LIB_PATH):
        pytest.skip("the traced build is loaded")
    L = rt.lib()
    k, s = C.c_int32(-1), C.c_int32(-1)
    assert L.rt_trace_read(None, 0, C.byref(k), C.byref(s)) == rt.RT_ESTATE
    assert "RT_TRACE" in L.rt_last_error().decode()
    assert k.value == -1 and s.value == -1
