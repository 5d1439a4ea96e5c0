"""GGUF reader and loader (include/rt_gguf.h, rich-triplet_amd/gguf.py) against
files written by tests/gguf_writer.py from the published layout, and the
oracle's restatements of the reference decoders (gguf_loader.rs) and of the
Q4_K quantiser (autograd2.rs:1090-1320).

The oracle functions used here are pinned in this file by closed forms
(Q4_0, Q8_0), by numpy restatements with independent index arithmetic (Q5_K,
Q6_K), by the reference's own tests (Q4KMat quantise round trips, f16 round
trip) and by the truncation property of Q4KMat::f32_to_f16.  Everything except
`test_load_linear_*` runs without a GPU.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from gguf_writer import ARRAY, BOOL, F32 as MF32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64, write_gguf

GG_F32, GG_F16, GG_Q4_0, GG_Q8_0, GG_Q4_K, GG_Q5_K, GG_Q6_K, GG_BF16 = 0, 1, 2, 8, 12, 13, 14, 30
BLOCK = {GG_Q4_0: (18, 32), GG_Q8_0: (34, 32), GG_Q4_K: (144, 256), GG_Q5_K: (176, 256), GG_Q6_K: (210, 256)}


# ---------------------------------------------------------------------------
# synthetic tensors
# ---------------------------------------------------------------------------
def _f16_bits(orc, vals):
    return np.array([orc.lib().orc_f32_to_f16_rne(float(v)) for v in vals], np.uint16)


def synth_blocks(orc, ggtype: int, n_elem: int, seed: int) -> np.ndarray:
    """Random quant bytes with finite f16 scale fields (N(0, 0.05) magnitudes)."""
    rng = np.random.default_rng(seed)
    bpb, epb = BLOCK[ggtype]
    nb = (n_elem + epb - 1) // epb
    raw = rng.integers(0, 256, size=(nb, bpb), dtype=np.uint8)
    scale_at = {GG_Q4_0: [0], GG_Q8_0: [0], GG_Q4_K: [0, 2], GG_Q5_K: [0, 2], GG_Q6_K: [208]}[ggtype]
    for off in scale_at:
        h = _f16_bits(orc, np.abs(rng.normal(0.0, 0.05, nb)).astype(np.float32))
        raw[:, off] = (h & 0xFF).astype(np.uint8)
        raw[:, off + 1] = (h >> 8).astype(np.uint8)
    return raw.reshape(-1)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------------------
# oracle pins (independent statements of the reference's formats)
# ---------------------------------------------------------------------------
def test_oracle_q8_0_and_q4_0_closed_forms(orc):
    n = 32 * 7 - 5  # ragged tail
    q8 = synth_blocks(orc, GG_Q8_0, n, 1).reshape(-1, 34)
    d = np.array([orc.f16_to_f32(int(b[0]) | (int(b[1]) << 8)) for b in q8], np.float32)
    want = (d[:, None] * q8[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)[:n]
    assert np.array_equal(_bits(orc.q8_0_dequant(q8.reshape(-1), n)), _bits(want))
    q4 = synth_blocks(orc, GG_Q4_0, n, 2).reshape(-1, 18)
    s = np.array([orc.f16_to_f32(int(b[0]) | (int(b[1]) << 8)) for b in q4], np.float32)
    nib = np.concatenate([q4[:, 2:] & 15, q4[:, 2:] >> 4], axis=1).astype(np.float32) - 8.0  # elements k, k+16
    want = (nib * s[:, None]).reshape(-1)[:n]
    assert np.array_equal(_bits(orc.q4_0_dequant(q4.reshape(-1), n)), _bits(want))


def test_oracle_q6k_against_index_formula(orc):
    """Element e of a block: half h = e//128, r = e%128, quarter k = r//32,
    l = r%32; low bits from ql[64h + l + 32(k&1)] (high nibble when k >= 2),
    two high bits (qh[32h + l] >> 2k) & 3, scale int8 sc[8h + l//16 + 2k]:
    value = (d*sc) * (q - 32)."""
    n = 256 * 3
    raw = synth_blocks(orc, GG_Q6_K, n, 3).reshape(-1, 210)
    e = np.arange(256)
    h, r = e // 128, e % 128
    k, l = r // 32, r % 32
    want = []
    for b in raw:
        ql, qh, sc = b[:128], b[128:192], b[192:208].view(np.int8)
        d = np.float32(orc.f16_to_f32(int(b[208]) | (int(b[209]) << 8)))
        byte = ql[64 * h + l + 32 * (k & 1)]
        lo = np.where(k >= 2, byte >> 4, byte & 15).astype(np.int32)
        hi = ((qh[32 * h + l] >> (2 * k)) & 3).astype(np.int32)
        s = (d * sc[8 * h + l // 16 + 2 * k].astype(np.float32)).astype(np.float32)
        want.append((s * ((lo | (hi << 4)) - 32).astype(np.float32)).astype(np.float32))
    assert np.array_equal(_bits(orc.q6k_dequant(raw.reshape(-1), n)), _bits(np.concatenate(want)))


def test_oracle_q5k_against_index_formula(orc):
    """Element e: chunk c = e//64, half = (e%64)//32, l = e%32; low nibble of
    qs[32c + l] (high nibble for half 1), fifth bit (qh[l] >> (2c + half)) & 1,
    scale/min pair 2c + half of the Q4_K packing."""
    n = 256 * 2 + 100
    raw = synth_blocks(orc, GG_Q5_K, n, 4).reshape(-1, 176)
    e = np.arange(256)
    c, half, l = e // 64, (e % 64) // 32, e % 32
    want = []
    for b in raw:
        d = np.float32(orc.f16_to_f32(int(b[0]) | (int(b[1]) << 8)))
        dm = np.float32(orc.f16_to_f32(int(b[2]) | (int(b[3]) << 8)))
        sc, qh, qs = b[4:16], b[16:48], b[48:176]
        j = 2 * c + half
        sm = np.array([orc.scale_min(sc, int(x)) for x in range(8)], np.float32)
        byte = qs[32 * c + l]
        q = np.where(half == 1, byte >> 4, byte & 15) | (((qh[l] >> j) & 1) << 4)
        want.append(((d * sm[j, 0]).astype(np.float32) * q.astype(np.float32)
                     - (dm * sm[j, 1]).astype(np.float32)).astype(np.float32))
    want = np.concatenate(want)[:n]
    assert np.array_equal(_bits(orc.q5k_dequant(raw.reshape(-1), n)), _bits(want))


def test_oracle_f16_trunc(orc):
    """Q4KMat::f32_to_f16 truncates toward zero: the result is the f16 value of
    largest magnitude not above |v| (numpy's RNE value, stepped one ulp toward
    zero when it rounded away), flushing to zero below 2^-24; an exponent past
    f16's range (|v| >= 2^16) gives Inf, while [65504, 2^16) truncates to 65504;
    plus the reference's own round-trip values (autograd2.rs:5725-5737)."""
    rng = np.random.default_rng(5)
    vals = np.concatenate([rng.normal(0, 1, 3000), rng.normal(0, 1e-5, 1000), rng.normal(0, 3e4, 500),
                           [0.0, -0.0, 1.0, -1.0, 0.5, 65504.0, -65504.0, 0.001, 100.0, 65519.0, 65535.9,
                            65536.0, -1e5, 1e-8]]).astype(np.float32)
    for v in vals:
        got = orc.f32_to_f16_trunc(float(v))
        if abs(float(v)) >= 65536.0:
            want = 0xFC00 if v < 0 else 0x7C00
        else:
            with np.errstate(over="ignore"):
                r = np.float16(v)
            if not np.isfinite(r):  # RNE overflowed in [65520, 2^16): truncation keeps 65504
                r = np.float16(np.sign(v) * 65504.0)
            elif abs(float(r)) > abs(float(v)):
                r = np.nextafter(r, np.float16(0.0))
            want = int(r.view(np.uint16))
        assert got == want, (v, got, want)
    for v in (0.0, 1.0, -1.0, 0.5, 65504.0, -65504.0, 0.001, 100.0):
        back = orc.f16_to_f32(orc.f32_to_f16_trunc(v))
        assert abs(back - v) < abs(v) * 0.002 + 1e-6


def test_oracle_q4k_quantize_reference_cases(orc):
    """The reference's Q4KMat tests: round trip < 0.15 (autograd2.rs:5658-5687,
    5706-5745), zeros stay zero (5689-5704); and every element lies within one
    quantisation step of its sub-block's grid."""
    m = np.array([[((r * 256 + c) / 1024.0) * 2.0 - 1.0 for c in range(256)] for r in range(4)], np.float32)
    q = orc.q4k_quantize(m)
    assert q.size == 4 * 144
    assert np.abs(orc.q4k_dequant(q, 4, 256) - m).max() < 0.15
    z = orc.q4k_quantize(np.zeros((2, 256), np.float32))
    assert np.abs(orc.q4k_dequant(z, 2, 256)).max() < 1e-6
    big = np.sin(np.arange(16 * 512, dtype=np.float32) * np.float32(0.001)).reshape(16, 512).astype(np.float32)
    assert np.abs(orc.q4k_dequant(orc.q4k_quantize(big), 16, 512) - big).max() < 0.15
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (8, 512)).astype(np.float32)
    x[1, :256] = np.abs(x[1, :256])          # a non-negative block (mins stay 0)
    x[2, 256:] = 0.25                        # a constant block
    blocks = orc.q4k_quantize(x)
    dq = orc.q4k_dequant(blocks, 8, 512)
    for r in range(8):
        for b in range(2):
            bp = blocks[(r * 2 + b) * 144:(r * 2 + b + 1) * 144]
            d = orc.f16_to_f32(int(bp[0]) | (int(bp[1]) << 8))
            for j in range(8):
                sv, _ = orc.scale_min(bp[4:16], j)
                seg = slice(256 * b + 32 * j, 256 * b + 32 * j + 32)
                step = d * sv
                lo, hi = x[r, seg].min(), x[r, seg].max()
                # a step of 0 only when the sub-block has no spread
                assert step > 0 or hi - min(lo, 0.0) <= 63 * d + 1e-6
                # within half a step inside the representable span, or clamped at an end
                err = np.abs(dq[r, seg] - x[r, seg])
                assert np.all(err <= max(step, 1e-7) * 0.5 + (hi - min(lo, 0.0)) / 15.0 + 1e-5)


def test_oracle_q4_0_to_q4k_is_quantise_of_decode(orc):
    """The requantisation path equals Q4KMat::quantize applied to the Q4_0
    values (the signed-nibble remap of gguf_loader.rs:282-357 is value-preserving)."""
    rows, cols = 6, 512
    raw = synth_blocks(orc, GG_Q4_0, rows * cols, 7)
    vals = orc.q4_0_dequant(raw, rows * cols).reshape(rows, cols)
    assert np.array_equal(orc.q4_0_to_q4k(raw, rows, cols), orc.q4k_quantize(vals))


# ---------------------------------------------------------------------------
# the reader (CPU)
# ---------------------------------------------------------------------------
def _sample_file(tmp_path, orc, alignment=64):
    tensors = [
        ("blk.0.attn_q.weight", [512, 3], GG_Q4_K, synth_blocks(orc, GG_Q4_K, 512 * 3, 11)),
        ("token_embd.weight", [64, 5], GG_F32, np.arange(320, dtype=np.float32).view(np.uint8)),
        ("norm.half", [40], GG_F16, _f16_bits(orc, np.linspace(-2, 2, 40)).view(np.uint8)),
        ("lin.bf16", [32, 4], GG_BF16, np.array([orc.f32_to_bf16(float(v)) for v in np.linspace(-1, 1, 128)],
                                                 np.uint16).view(np.uint8)),
        ("q40", [512, 2], GG_Q4_0, synth_blocks(orc, GG_Q4_0, 1024, 12)),
        ("q80", [64, 3], GG_Q8_0, synth_blocks(orc, GG_Q8_0, 192, 13)),
        ("q5k", [256, 2], GG_Q5_K, synth_blocks(orc, GG_Q5_K, 512, 14)),
        ("q6k", [256, 3, 1], GG_Q6_K, synth_blocks(orc, GG_Q6_K, 768, 15)),
        ("iq2", [256], 16, np.zeros(66, np.uint8)),  # a type with no block size in the reader
    ]
    meta = [("general.architecture", STR, "gemma3"), ("gemma3.block_count", U32, 34),
            ("gemma3.rope.freq_base", MF32, 1e6), ("u8", U8, 7), ("i8", I8, -3), ("u16", U16, 65000),
            ("i16", I16, -30000), ("i32", I32, -5), ("u64", U64, 1 << 40), ("i64", I64, -(1 << 40)),
            ("f64", F64, 0.125), ("flag", BOOL, True),
            ("tokenizer.ggml.tokens", ARRAY, ["<pad>", "<eos>", "hello", ""], STR),
            ("nums", ARRAY, [1, 2, 3], U32)]
    path = tmp_path / "sample.gguf"
    layout = write_gguf(path, meta, tensors, alignment=alignment)
    return path, tensors, layout


def test_reader_header_metadata_directory(rt, orc, tmp_path):
    path, tensors, layout = _sample_file(tmp_path, orc)
    g = rt.GgufFile(str(path))
    assert len(g.tensor_info) == len(tensors)
    for info, (name, dims, ttype, data) in zip(g.tensor_info, tensors):
        assert (info.name, info.shape, info.gguf_type) == (name, dims, ttype)
        assert info.data_offset == layout["offsets"][name]
        if ttype != 16:
            assert info.n_bytes == len(data)
        else:
            assert info.n_bytes == 0
    assert g.data_start == layout["data_start"]
    md = g.metadata
    assert md["general.architecture"] == "gemma3" and md["gemma3.block_count"] == 34
    assert md["general.alignment"] == 64
    assert abs(md["gemma3.rope.freq_base"] - 1e6) < 1 and md["f64"] == 0.125
    assert md["u8"] == 7 and md["u16"] == 65000 and md["u64"] == 1 << 40
    assert md["i32"] == -5 and md["i64"] == -(1 << 40)
    assert md["tokenizer.ggml.tokens"] == ["<pad>", "<eos>", "hello", ""]
    assert md["nums"] == ("array", U32, 3)
    assert g.meta_u64("i8") is None and g.meta_f32("u8") is None  # as_u64 / as_f32 reject these types
    assert g.find_tensor("q40") == 4 and g.find_tensor("missing") is None
    for i, (name, dims, ttype, data) in enumerate(tensors):
        if ttype != 16:
            assert np.array_equal(g.read_tensor_bytes(i), np.asarray(data, np.uint8).view(np.uint8))
    blocks, rows, cols = g.decode_q4k_to_q4kmat(0)
    assert (rows, cols) == (3, 512) and np.array_equal(blocks, tensors[0][3])
    g.close()


@pytest.mark.parametrize("alignment", [None, 32, 256])
def test_reader_alignment(rt, orc, tmp_path, alignment):
    path = tmp_path / "a.gguf"
    data = synth_blocks(orc, GG_Q8_0, 64, 20)
    layout = write_gguf(path, [("x", U32, 1)], [("t0", [32], GG_F32, np.ones(32, np.float32).view(np.uint8)),
                                               ("t1", [64], GG_Q8_0, data)], alignment=alignment)
    g = rt.GgufFile(str(path))
    assert g.data_start == layout["data_start"] and g.data_start % (alignment or 32) == 0
    assert np.array_equal(g.read_tensor_bytes(1), data)
    g.close()


def test_decoders_match_oracle(rt, orc, tmp_path):
    """tensor_to_f32 for every supported type, bit for bit against the oracle."""
    path, tensors, _ = _sample_file(tmp_path, orc)
    g = rt.GgufFile(str(path))
    ref = {GG_Q4_K: lambda d, n: orc.q4k_dequant_gguf(d, n), GG_Q4_0: orc.q4_0_dequant, GG_Q8_0: orc.q8_0_dequant,
           GG_Q5_K: orc.q5k_dequant, GG_Q6_K: orc.q6k_dequant,
           GG_F32: lambda d, n: np.asarray(d, np.uint8).view(np.float32)[:n],
           GG_F16: lambda d, n: np.array([orc.f16_to_f32(int(b)) for b in np.asarray(d, np.uint8).view(np.uint16)],
                                         np.float32)}
    for i, (name, dims, ttype, data) in enumerate(tensors):
        if ttype in ref:
            n = int(np.prod(dims))
            got = g.tensor_to_f32(i)
            assert np.array_equal(_bits(got), _bits(ref[ttype](np.asarray(data, np.uint8), n))), name
    with pytest.raises(rt.RtError):
        g.tensor_to_f32(3)  # BF16 has no f32 decoding in tensor_to_f32, as in the reference
    with pytest.raises(rt.RtError):
        g.tensor_to_f32(8)
    g.close()


def test_quantize_matches_oracle(rt, orc):
    rng = np.random.default_rng(21)
    x = rng.normal(0, 1, (16, 768)).astype(np.float32)
    x[3] = np.abs(x[3])
    x[4, :256] = 0.0
    x[5, 256:512] = -2.5
    x[6] *= 1e-6
    x[7] *= 3e4
    assert np.array_equal(rt.q4k_quantize(x), orc.q4k_quantize(x))
    m = np.array([[((r * 256 + c) / 1024.0) * 2.0 - 1.0 for c in range(256)] for r in range(4)], np.float32)
    assert np.abs(orc.q4k_dequant(rt.q4k_quantize(m), 4, 256) - m).max() < 0.15
    with pytest.raises(rt.RtError):
        rt.q4k_quantize(np.zeros((2, 100), np.float32))


def test_quantize_bf16_matches_oracle_on_widened_rows(rt, orc):
    """quantize_from_bf16 (the q4k-lm-head requantisation): the blocks of
    the f32-widened rows, as the oracle's quantiser makes them, on an
    embedding-like bf16 matrix with a zero row and a row of one value."""
    w = orc.synth_bf16(31, 37 * 512).reshape(37, 512)
    w[5] = 0
    w[9] = 0x3F80  # 1.0
    widened = (w.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(rt.q4k_quantize_bf16(w), orc.q4k_quantize(widened))
    with pytest.raises(rt.RtError):
        rt.q4k_quantize_bf16(np.zeros((2, 100), np.uint16))


def test_requant_path_matches_oracle_on_cpu(rt, orc, tmp_path):
    """The library's decode + quantise of a Q4_0 tensor equals the oracle's
    Q4_0 -> Q4_K requantisation (the device upload itself is a GPU test)."""
    rows, cols = 5, 768
    raw = synth_blocks(orc, GG_Q4_0, rows * cols, 22)
    path = tmp_path / "q40.gguf"
    write_gguf(path, [], [("w", [cols, rows], GG_Q4_0, raw)])
    g = rt.GgufFile(str(path))
    vals = g.tensor_to_f32(0).reshape(rows, cols)
    assert np.array_equal(rt.q4k_quantize(vals), orc.q4_0_to_q4k(raw, rows, cols))
    g.close()


def test_reader_rejects_bad_files(rt, orc, tmp_path):
    p = tmp_path / "bad"
    p.write_bytes(b"GGML" + b"\0" * 60)
    with pytest.raises(rt.RtError, match="not a GGUF"):
        rt.GgufFile(str(p))
    path, _, _ = _sample_file(tmp_path, orc)
    blob = path.read_bytes()
    v1 = tmp_path / "v1.gguf"
    v1.write_bytes(blob[:4] + (1).to_bytes(4, "little") + blob[8:])
    with pytest.raises(rt.RtError, match="version"):
        rt.GgufFile(str(v1))
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(blob[:200])
    with pytest.raises(rt.RtError):
        rt.GgufFile(str(cut))
    short = tmp_path / "short.gguf"
    short.write_bytes(blob[:-100])  # directory intact, last tensor runs past the end
    g = rt.GgufFile(str(short))
    with pytest.raises(rt.RtError, match="outside the file"):
        g.read_tensor_bytes(7)
    g.close()
    with pytest.raises(rt.RtError):
        rt.GgufFile(str(tmp_path / "does-not-exist.gguf"))


def test_reader_rejects_oversized_and_wrapping_tensors(rt, orc, tmp_path):
    """A tensor whose byte size exceeds the file fails at open; a data offset
    near 2^64 (offset + size would wrap) fails the read instead of passing a
    wrapped bounds check."""
    import struct
    big = tmp_path / "big.gguf"
    write_gguf(big, [], [("huge", [1 << 60], GG_F32, np.zeros(64, np.uint8))])
    with pytest.raises(rt.RtError, match="larger than the file"):
        rt.GgufFile(str(big))
    wrap = tmp_path / "wrap.gguf"
    write_gguf(wrap, [], [("w", [16], GG_F32, np.zeros(64, np.uint8))])
    blob = bytearray(wrap.read_bytes())
    name = b"w"
    at = blob.index(struct.pack("<Q", len(name)) + name) + 8 + len(name)
    at += 4 + 8 + 4  # n_dims, one dimension, type -> the offset field
    blob[at:at + 8] = struct.pack("<Q", (1 << 64) - 32)
    wrap.write_bytes(bytes(blob))
    g = rt.GgufFile(str(wrap))
    with pytest.raises(rt.RtError, match="outside the file"):
        g.read_tensor_bytes(0)
    g.close()


def test_load_linear_rejects_before_upload(rt, orc, tmp_path):
    """Shape and type errors are reported on the host, before any device call."""
    path = tmp_path / "w.gguf"
    write_gguf(path, [], [("q40", [96, 4], GG_Q4_0, synth_blocks(orc, GG_Q4_0, 384, 30)),
                          ("iq", [256], 16, np.zeros(66, np.uint8))])
    g = rt.GgufFile(str(path))
    with pytest.raises(rt.RtError, match="multiple of 256"):
        rt.load_linear_from_gguf(g, 0)
    with pytest.raises(rt.RtError, match="unsupported"):
        rt.load_linear_from_gguf(g, 1)
    g.close()


# ---------------------------------------------------------------------------
# device upload (GPU)
# ---------------------------------------------------------------------------
def _download(ptr: int, n: int) -> np.ndarray:
    hip = C.CDLL("libamdhip64.so")
    out = np.empty(n, np.uint8)
    assert hip.hipMemcpy(C.c_void_p(out.ctypes.data), C.c_void_p(ptr), C.c_size_t(n), 2) == 0  # DeviceToHost
    return out


@pytest.mark.gpu
def test_load_linear_formats_on_device(rt, orc, tmp_path):
    rows, cols = 48, 512
    q4k = synth_blocks(orc, GG_Q4_K, rows * cols, 40)
    q40 = synth_blocks(orc, GG_Q4_0, rows * cols, 41)
    q6k = synth_blocks(orc, GG_Q6_K, rows * cols, 42)
    q80 = synth_blocks(orc, GG_Q8_0, rows * cols, 43)
    f16 = _f16_bits(orc, np.random.default_rng(44).normal(0, 1, rows * cols)).view(np.uint8)
    f32 = np.random.default_rng(45).normal(0, 1, rows * cols).astype(np.float32)
    path = tmp_path / "model.gguf"
    write_gguf(path, [("general.architecture", STR, "gemma3")],
               [("q4k", [cols, rows], GG_Q4_K, q4k), ("q40", [cols, rows], GG_Q4_0, q40),
                ("q6k", [cols, rows], GG_Q6_K, q6k), ("q80", [cols, rows], GG_Q8_0, q80),
                ("f16", [cols, rows], GG_F16, f16), ("f32", [cols, rows], GG_F32, f32.view(np.uint8))])
    g = rt.GgufFile(str(path))
    bf = lambda v: np.array([orc.f32_to_bf16(float(x)) for x in v], np.uint16)  # noqa: E731
    want = {"q4k": (1, q4k), "q40": (1, orc.q4_0_to_q4k(q40, rows, cols)),
            "q6k": (2, bf(orc.q6k_dequant(q6k, rows * cols)).view(np.uint8)),
            "q80": (2, bf(orc.q8_0_dequant(q80, rows * cols)).view(np.uint8)),
            "f16": (2, bf([orc.f16_to_f32(int(b)) for b in f16.view(np.uint16)]).view(np.uint8)),
            "f32": (3, f32.view(np.uint8))}
    for name, (fmt, data) in want.items():
        lin = rt.load_linear_from_gguf(g, g.find_tensor(name))
        assert (lin.format, lin.rows, lin.cols) == (fmt, rows, cols), name
        assert np.array_equal(_download(lin.ptr, lin.bytes), data), name
        lin.free()
    g.close()


@pytest.mark.gpu
def test_gemv_on_loaded_weights(rt, orc, tmp_path, dev):
    """A Q4_K and a requantised Q4_0 weight straight from the file feed the GEMV."""
    import torch
    rows, cols = 1024, 2560
    q4k = orc.synth_q4k(50, rows, cols)
    q40 = synth_blocks(orc, GG_Q4_0, rows * cols, 51)
    path = tmp_path / "proj.gguf"
    write_gguf(path, [], [("q4k", [cols, rows], GG_Q4_K, q4k), ("q40", [cols, rows], GG_Q4_0, q40)])
    g = rt.GgufFile(str(path))
    a = orc.synth_normal(52, cols)
    x = torch.from_numpy(a).to(dev)
    for name, blocks in (("q4k", q4k), ("q40", orc.q4_0_to_q4k(q40, rows, cols))):
        lin = rt.load_linear_from_gguf(g, g.find_tensor(name))
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        rt.check(rt.lib().rt_q4k_gemv(lin.ptr, x.data_ptr(), y.data_ptr(), rows, cols, None))
        torch.cuda.synchronize()
        ref = orc.q4k_gemv_f64(blocks, rows, cols, a)
        got = y.cpu().numpy().astype(np.float64)
        assert np.sqrt(((got - ref) ** 2).sum() / (ref ** 2).sum()) < 1e-4, name
        lin.free()
    g.close()


@pytest.mark.gpu
def test_load_linear_keep_packed_feeds_native_gemvs(rt, orc, tmp_path, dev):
    """keep_packed: Q6_K and Q8_0 tensors land in the planar device layout
    (byte-equal to rt.q6k_repack / q8_0_repack of the file bytes) and feed the
    native GEMVs; other types load as without the flag."""
    import torch
    rows, cols = 640, 2560
    q6k = synth_blocks(orc, GG_Q6_K, rows * cols, 60)
    q80 = synth_blocks(orc, GG_Q8_0, rows * cols, 61)
    q4k = orc.synth_q4k(62, rows, cols)
    path = tmp_path / "packed.gguf"
    write_gguf(path, [], [("q6k", [cols, rows], GG_Q6_K, q6k), ("q80", [cols, rows], GG_Q8_0, q80),
                          ("q4k", [cols, rows], GG_Q4_K, q4k)])
    g = rt.GgufFile(str(path))
    a = orc.synth_normal(63, cols)
    x = torch.from_numpy(a).to(dev)
    cases = (("q6k", 4, rt.q6k_repack(q6k), orc.q6k_dequant(q6k, rows * cols), rt.q6k_gemv),
             ("q80", 5, rt.q8_0_repack(q80), orc.q8_0_dequant(q80, rows * cols), rt.q8_0_gemv))
    for name, fmt, planar, deq, gemv in cases:
        lin = rt.load_linear_from_gguf(g, g.find_tensor(name), keep_packed=True)
        assert (lin.format, lin.rows, lin.cols, lin.bytes) == (fmt, rows, cols, planar.size), name
        assert np.array_equal(_download(lin.ptr, lin.bytes), planar), name
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        gemv(lin.ptr, x.data_ptr(), y.data_ptr(), rows, cols)
        torch.cuda.synchronize()
        ref = deq.reshape(rows, cols).astype(np.float64) @ a.astype(np.float64)
        got = y.cpu().numpy().astype(np.float64)
        assert np.sqrt(((got - ref) ** 2).sum() / (ref ** 2).sum()) < 1e-4, name
        lin.free()
    lin = rt.load_linear_from_gguf(g, g.find_tensor("q4k"), keep_packed=True)
    assert lin.format == 1 and np.array_equal(_download(lin.ptr, lin.bytes), q4k)
    lin.free()
    g.close()
