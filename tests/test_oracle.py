"""Pins the CPU oracle (oracle/rt_oracle.c) before anything is compared with it.

Each check is chosen so that a plausible restatement mistake -- a dropped term,
a swapped nibble half, a wrong scale/min index, a transposed operand -- fails:
closed forms from the reference's own tests, library routines (numpy float16,
torch bfloat16, float64 math), invariants and float64 brute force.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import rel_l2


# --------------------------------------------------------------------------
# f16 / bf16 conversions
# --------------------------------------------------------------------------
def test_f16_to_f32_all_patterns_match_ieee(orc):
    """autograd2.rs:1048-1070 vs numpy's IEEE half for all 65536 bit patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # (NaN payloads are not compared: any arithmetic on d quiets them, and the
    # ctypes float return path already widens through double.)


def test_f16_round_trip_known_values(orc):
    """Values of the reference's f16 round-trip test (autograd2.rs:5657-5745)."""
    for v in (0.0, 1.0, -1.0, 0.5, 65504.0, -65504.0, 0.001, 100.0, 6.1e-5, 1e-7):
        h = orc.f32_to_f16_rne(v)
        assert h == int(np.float16(v).view(np.uint16)), v
        assert orc.f16_to_f32(h) == float(np.float16(v))


def test_f16_rne_matches_numpy_on_random_floats(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.normal(0, 0.02, 4000), rng.normal(0, 1e-4, 2000), rng.normal(0, 3e4, 500)])
    for v in vals.astype(np.float32):
        assert orc.f32_to_f16_rne(float(v)) == int(np.float16(v).view(np.uint16)), v


def test_bf16_conversions_match_torch(orc):
    """autograd2.rs:700-719 (RNE, ties to even) vs torch's bfloat16 cast."""
    import torch
    rng = np.random.default_rng(2)
    vals = np.concatenate([rng.normal(0, 1, 3000), rng.normal(0, 0.02, 3000),
                           [0.0, -0.0, 1.0, 3.0e38, -3.0e38, 1e-40, 1.00390625, 1.01171875]]).astype(np.float32)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([orc.f32_to_bf16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)
    for b in (0x0000, 0x3F80, 0xBF80, 0x7F7F, 0x0001):
        assert orc.bf16_to_f32(b) == float(np.array([b << 16], np.uint32).view(np.float32)[0])


# --------------------------------------------------------------------------
# Q4_K block format
# --------------------------------------------------------------------------
def test_scale_min_inverts_pack_scales_for_every_value(orc):
    """scale_min (autograd2.rs:1075-1085) must invert pack_scales (1119-1132)
    for all 64 values in every one of the 8 slots."""
    for v in range(64):
        for j in range(8):
            sv = np.full(8, (v + 7 * j) % 64, np.uint8)
            mv = np.full(8, (63 - v + 3 * j) % 64, np.uint8)
            sv[j], mv[j] = v, 63 - v
            sc = orc.pack_scales(sv, mv)
            for jj in range(8):
                assert orc.scale_min(sc, jj) == (float(sv[jj]), float(mv[jj]))


def test_scale_min_matches_llama_cpp_bit_layout(orc):
    """Independent statement of the 12-byte layout (llama.cpp get_scale_min_k4,
    named at gguf_loader.rs:547-550): 6-bit fields at fixed bit offsets."""
    rng = np.random.default_rng(3)
    for _ in range(500):
        sc = rng.integers(0, 256, 12, dtype=np.uint8)
        bits = np.unpackbits(sc, bitorder="little")  # bit i of byte k at 8k+i

        def field(byte, lo_bit, n):
            return sum(int(bits[8 * byte + lo_bit + t]) << t for t in range(n))

        for j in range(8):
            if j < 4:
                sv, mv = field(j, 0, 6), field(j + 4, 0, 6)
            else:
                sv = field(j + 4, 0, 4) | (field(j - 4, 6, 2) << 4)
                mv = field(j + 4, 4, 4) | (field(j, 6, 2) << 4)
            assert orc.scale_min(sc, j) == (float(sv), float(mv))


def _make_test_q4k(n_rows: int, k: int) -> np.ndarray:
    """The reference's make_test_q4k fixture (metal_ops.rs:1121-1152): every
    block d=f16trunc(0.1)=0x2E66, dmin=f16trunc(0.05)=0x2A66, scale bytes
    [2,2,2,2,1,1,1,1,0,0,0,0], nibble bytes 0x55."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0x2E66], np.uint16).view(np.uint8)
    blk[2:4] = np.array([0x2A66], np.uint16).view(np.uint8)
    blk[4:8] = 2
    blk[8:12] = 1
    blk[16:] = 0x55
    return np.tile(blk, n_rows * (k // 256))


MAKE_TEST_Q4K_FIRST_HALF = 15561.0 / 16384.0
"""Closed form for elements 0..127 of make_test_q4k: d=1638/16384,
dmin=819/16384, sv=2, mv=1, q=5 -> (d*2)*5 - dmin = 15561/16384 (exact in f32).
Elements 128..255 have sv=mv=0 -> 0."""


def test_f16_trunc_constants_of_make_test_q4k(orc):
    assert orc.f16_to_f32(0x2E66) == 1638.0 / 16384.0
    assert orc.f16_to_f32(0x2A66) == 819.0 / 16384.0


def test_dequant_make_test_q4k_closed_form(orc):
    blocks = _make_test_q4k(4, 512)
    w = orc.q4k_dequant(blocks, 4, 512)
    expect = np.tile(np.r_[np.full(128, MAKE_TEST_Q4K_FIRST_HALF), np.zeros(128)], 2)
    assert np.array_equal(w, np.tile(expect.astype(np.float32), (4, 1)))


def _numpy_dequant(blocks: np.ndarray) -> np.ndarray:
    """Vectorised float32 restatement written from the format description
    (not from the oracle's loops): chunk c owns nibble bytes 32c..32c+31."""
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dm = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc = b[:, 4:16].astype(np.uint32)
    sv = np.empty((b.shape[0], 8), np.uint32)
    mv = np.empty_like(sv)
    sv[:, :4] = sc[:, 0:4] & 63
    mv[:, :4] = sc[:, 4:8] & 63
    sv[:, 4:] = (sc[:, 8:12] & 15) | ((sc[:, 0:4] >> 6) << 4)
    mv[:, 4:] = (sc[:, 8:12] >> 4) | ((sc[:, 4:8] >> 6) << 4)
    q = b[:, 16:].reshape(-1, 4, 32)
    nib = np.stack([q & 15, q >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)  # sub-block 2c lo, 2c+1 hi
    scale = (d[:, None] * sv.astype(np.float32))[:, :, None]
    mn = (dm[:, None] * mv.astype(np.float32))[:, :, None]
    return (scale * nib - mn).astype(np.float32).reshape(-1)


def test_dequant_random_blocks_two_restatements_and_numpy_agree(orc):
    rows, cols = 24, 1024
    blocks = orc.synth_q4k(11, rows, cols)
    w_row = orc.q4k_dequant(blocks, rows, cols).reshape(-1)
    w_gguf = orc.q4k_dequant_gguf(blocks, rows * cols)
    w_np = _numpy_dequant(blocks)
    assert np.array_equal(w_row.view(np.uint32), w_gguf.view(np.uint32))
    assert np.array_equal(w_row.view(np.uint32), w_np.view(np.uint32))


def test_dequant_subnormal_and_special_d(orc):
    """f16-subnormal d/dmin (0.24% of |N(0,0.02)| draws) and large d decode exactly."""
    blocks = orc.synth_q4k(5, 8, 256)
    b = blocks.reshape(8, 144)
    for i, (dbits, mbits) in enumerate([(0x0001, 0x0003), (0x03FF, 0x0200), (0x0400, 0x0001), (0x7BFF, 0x3C00),
                                        (0x8001, 0x83FF), (0x0000, 0x0000), (0x3555, 0x1234), (0x0010, 0x7000)]):
        b[i, 0:2] = np.array([dbits], np.uint16).view(np.uint8)
        b[i, 2:4] = np.array([mbits], np.uint16).view(np.uint8)
    w = orc.q4k_dequant(blocks, 8, 256).reshape(-1)
    assert np.array_equal(w.view(np.uint32), _numpy_dequant(blocks).view(np.uint32))
    assert np.all(w[5 * 256:6 * 256] == 0)


def test_gguf_restatement_clips_a_ragged_tail(orc):
    blocks = orc.synth_q4k(6, 1, 512)
    full = orc.q4k_dequant_gguf(blocks, 512)
    part = orc.q4k_dequant_gguf(blocks, 300)
    assert np.array_equal(part, full[:300])


# --------------------------------------------------------------------------
# GEMV
# --------------------------------------------------------------------------
def test_q4k_gemv_make_test_q4k_like_reference(orc):
    """metal_ops.rs:1154-1235: a = (c+1)*0.01 and ((c%7)-3)*0.1 vs dequant-then-dot."""
    for n, k, fn in ((4, 256, lambda c: (c + 1) * 0.01), (64, 512, lambda c: ((c % 7) - 3.0) * 0.1)):
        blocks = _make_test_q4k(n, k)
        a = np.array([fn(c) for c in range(k)], np.float32)
        y = orc.q4k_gemv(blocks, n, k, a)
        # closed form: every row is the same; first 128 of each 256 carry the constant weight
        cols = np.arange(k)
        ref = sum(MAKE_TEST_Q4K_FIRST_HALF * float(a[c]) for c in cols if c % 256 < 128)
        assert np.allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_q4k_gemv_vs_f64_brute_force(orc):
    rows, cols = 300, 2560
    blocks = orc.synth_q4k(21, rows, cols)
    a = orc.synth_normal(22, cols)
    y = orc.q4k_gemv(blocks, rows, cols, a)
    w = _numpy_dequant(blocks).reshape(rows, cols).astype(np.float64)
    ref = w @ a.astype(np.float64)
    assert rel_l2(y, ref) < 2e-6
    assert rel_l2(orc.q4k_gemv_f64(blocks, rows, cols, a), ref) < 1e-12


def test_q4k_gemv_invariants(orc):
    rows, cols = 64, 1024
    blocks = orc.synth_q4k(31, rows, cols)
    a = orc.synth_normal(32, cols)
    y = orc.q4k_gemv(blocks, rows, cols, a)
    # scaling x by a power of two scales y exactly
    assert np.array_equal(orc.q4k_gemv(blocks, rows, cols, 4.0 * a), 4.0 * y)
    # one-hot x picks a dequantised column exactly (integer trick reduces to scale*q - min)
    w = orc.q4k_dequant(blocks, rows, cols)
    for col in (0, 31, 32, 63, 64, 200, 255, 256, 700, 1023):
        e = np.zeros(cols, np.float32)
        e[col] = 1.0
        assert np.array_equal(orc.q4k_gemv(blocks, rows, cols, e), w[:, col])
    # zero d and dmin make a block contribute nothing
    z = blocks.copy().reshape(rows, cols // 256, 144)
    z[:, 1, 0:4] = 0
    ref = orc.q4k_gemv_f64(blocks, rows, cols, a) - (w[:, 256:512].astype(np.float64) @ a[256:512])
    assert rel_l2(orc.q4k_gemv(z.reshape(-1), rows, cols, a), ref) < 1e-5


def test_q4k_gemv_thread_count_does_not_change_results(orc):
    rows, cols = 1024, 512
    blocks = orc.synth_q4k(41, rows, cols)
    a = orc.synth_normal(42, cols)
    assert np.array_equal(orc.q4k_gemv(blocks, rows, cols, a, 1), orc.q4k_gemv(blocks, rows, cols, a, 8))


def test_bf16_gemv_exact_on_small_integers_and_vs_f64(orc):
    """metal_ops.rs:1239-1305 style inputs; small integers make every product
    and partial sum exact in f32."""
    rng = np.random.default_rng(4)
    n, k = 128, 256
    wf = rng.integers(-8, 9, (n, k)).astype(np.float32)
    w = np.array([orc.f32_to_bf16(float(v)) for v in wf.reshape(-1)], np.uint16)
    a = rng.integers(-4, 5, k).astype(np.float32)
    assert np.array_equal(orc.bf16_gemv(w, n, k, a), (wf.astype(np.float64) @ a).astype(np.float32))
    w2 = orc.synth_bf16(5, 512 * 2560)
    a2 = orc.synth_normal(6, 2560)
    ref = (w2.astype(np.uint32) << 16).view(np.float32).reshape(512, 2560).astype(np.float64) @ a2
    assert rel_l2(orc.bf16_gemv(w2, 512, 2560, a2), ref) < 1e-6


def test_q4k_matmul_vs_f64(orc):
    m, n, k = 5, 40, 512
    blocks = orc.synth_q4k(51, n, k)
    a = orc.synth_normal(52, m * k).reshape(m, k)
    ref = a.astype(np.float64) @ _numpy_dequant(blocks).reshape(n, k).astype(np.float64).T
    assert rel_l2(orc.q4k_matmul(a, blocks, n, k), ref) < 2e-6
    assert rel_l2(orc.q4k_matmul_f64(a, blocks, n, k), ref) < 1e-12


# --------------------------------------------------------------------------
# decode-step math (cases of metal_decode.rs:2697-3157)
# --------------------------------------------------------------------------
def test_rms_norm_gemma3(orc):
    x = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)
    g = np.array([0.1, 0.2, 0.0, -0.1, 0.05, 0.0, 0.0, 0.15], np.float32)
    rms = math.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
    assert np.allclose(orc.rms_norm_gemma3(x, g), x / rms * (1.0 + g.astype(np.float64)), rtol=0, atol=1e-6)
    # scale invariance (up to eps) and gamma = 0 gives unit RMS
    y = orc.rms_norm_gemma3(1000.0 * x, np.zeros(8, np.float32))
    assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-6


def test_per_head_norm_shares_gamma(orc):
    x = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)
    g = np.array([0.1, 0.2, 0.0, -0.1], np.float32)
    out = orc.per_head_norm(x, g, 2, 4)
    for h in range(2):
        xs = x[4 * h:4 * h + 4].astype(np.float64)
        assert np.allclose(out[4 * h:4 * h + 4], xs / math.sqrt(np.mean(xs ** 2) + 1e-6) * (1 + g), atol=1e-6)


def test_rope_neox(orc):
    """NeoX pairs (i, i+d/2), angle = pos*fs/theta^(2i/d)."""
    x = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)
    assert np.array_equal(orc.rope_neox(x, 2, 4, 10000.0, 0, 1.0), x)  # position 0 is the identity
    y = orc.rope_neox(x, 2, 4, 10000.0, 3, 1.0)
    for h in range(2):
        for i in range(2):
            ang = 3.0 / 10000.0 ** (2 * i / 4)
            x0, x1 = float(x[4 * h + i]), float(x[4 * h + i + 2])
            assert abs(y[4 * h + i] - (x0 * math.cos(ang) - x1 * math.sin(ang))) < 1e-5
            assert abs(y[4 * h + i + 2] - (x0 * math.sin(ang) + x1 * math.cos(ang))) < 1e-5
    # rotation preserves each pair's norm; freq_scale scales the position
    rng = np.random.default_rng(7)
    v = rng.normal(size=8 * 256).astype(np.float32)
    r = orc.rope_neox(v, 8, 256, 1e6, 4096, 0.125)
    assert np.allclose(np.linalg.norm(r), np.linalg.norm(v), rtol=1e-5)
    assert np.allclose(r, orc.rope_neox(v, 8, 256, 1e6, 512, 1.0), atol=1e-5)


def test_gelu_tanh_including_saturation(orc):
    xs = [-2.0, -1.0, 0.0, 0.5, 1.0, 2.0, 3.0, 4.0, 10.0, 12.655, -15.0, 20.0, -25.0, 100.0]
    for v in xs:
        ref = 0.5 * v * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))
        got = orc.gelu_tanh(v)
        assert math.isfinite(got)
        assert abs(got - ref) <= 1e-6 * max(1.0, abs(ref)), v
    assert orc.gelu_tanh(100.0) == 100.0 and orc.gelu_tanh(-25.0) == 0.0


def test_gqa_attention_reference_case(orc):
    """metal_decode.rs test_attention_decode: 2 q heads, 1 kv head, d=4, 3 keys."""
    q = np.array([1, 0, 1, 0, 0, 1, 0, 1], np.float32)
    k = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]], np.float32)
    v = np.array([[10, 20, 30, 40], [50, 60, 70, 80], [90, 100, 110, 120]], np.float32)
    out = orc.gqa_attention_decode(q, k, v, 0, 3, 2, 1, 4, 0.5)
    for h in range(2):
        s = np.array([q[4 * h:4 * h + 4] @ k[c] for c in range(3)], np.float64) * 0.5
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(out[4 * h:4 * h + 4], p @ v.astype(np.float64), atol=1e-4)


def test_gqa_attention_window_and_groups(orc):
    rng = np.random.default_rng(8)
    nq, nkv, d, T = 8, 4, 64, 50
    q = rng.normal(size=nq * d).astype(np.float32)
    kc = rng.normal(size=(T, nkv * d)).astype(np.float32)
    vc = rng.normal(size=(T, nkv * d)).astype(np.float32)
    out = orc.gqa_attention_decode(q, kc, vc, 20, 50, nq, nkv, d, 1 / 8)
    for h in range(nq):
        kv = h // (nq // nkv)
        K = kc[20:50, kv * d:(kv + 1) * d].astype(np.float64)
        V = vc[20:50, kv * d:(kv + 1) * d].astype(np.float64)
        s = K @ q[h * d:(h + 1) * d] / 8
        p = np.exp(s - s.max())
        assert np.allclose(out[h * d:(h + 1) * d], (p / p.sum()) @ V, atol=1e-5)


# --------------------------------------------------------------------------
# full decode step against a float64 numpy restatement (tiny shape)
# --------------------------------------------------------------------------
def tiny_cfg():
    return dict(hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=64, n_layers=6, vocab=300,
                sliding_window=8, global_every=6, rope_theta_local=10000.0, rope_theta_global=1000000.0,
                rope_fs_local=1.0, rope_fs_global=0.125, eps=1e-6, attn_scale=1.0 / 8.0)


def make_model(orc, cfg, max_seq, ctx, seed=100, gamma_std=0.1):
    H, F, D = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QD, KVD = cfg["n_q_heads"] * D, cfg["n_kv_heads"] * D
    layers = []
    s = seed
    for _ in range(cfg["n_layers"]):
        L = {}
        for name, (rows, cols) in dict(q=(QD, H), k=(KVD, H), v=(KVD, H), o=(H, QD), gate=(F, H), up=(F, H),
                                       down=(H, F)).items():
            s += 1
            L[name] = orc.synth_q4k(s, rows, cols)
        for name, n in dict(in_norm=H, post_attn_norm=H, pre_ffn_norm=H, post_ffn_norm=H, q_norm=D,
                            k_norm=D).items():
            s += 1
            L[name] = orc.synth_normal(s, n, 0.0, gamma_std)
        s += 1
        kc = np.zeros((max_seq, KVD), np.float32)
        kc[:ctx] = orc.synth_normal(s, ctx * KVD).reshape(ctx, KVD)
        s += 1
        vc = np.zeros((max_seq, KVD), np.float32)
        vc[:ctx] = orc.synth_normal(s, ctx * KVD).reshape(ctx, KVD)
        L["k_cache"], L["v_cache"] = kc, vc
        layers.append(L)
    embed = orc.synth_bf16(seed + 9999, cfg["vocab"] * H)
    final_norm = orc.synth_normal(seed + 9998, H, 0.0, gamma_std)
    return layers, embed, final_norm


def np_decode_step(cfg, layers, embed, final_norm, token, pos):
    """float64 restatement of transformer4.rs:1900-1964 / 2358-2385 (independent of the C oracle)."""
    H, D = cfg["hidden"], cfg["head_dim"]
    NQ, NKV = cfg["n_q_heads"], cfg["n_kv_heads"]
    eps = cfg["eps"]

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x) + eps) * (1.0 + g.astype(np.float64))

    def deq(b, rows, cols):
        return _numpy_dequant(b).reshape(rows, cols).astype(np.float64)

    def rope(x, nh, theta, fs):
        x = x.reshape(nh, D).copy()
        half = D // 2
        i = np.arange(half)
        ang = pos * fs / theta ** (2 * i / D)
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half] = x0 * c - x1 * s
        x[:, half:] = x0 * s + x1 * c
        return x.reshape(-1)

    x = (embed[token * H:(token + 1) * H].astype(np.uint32) << 16).view(np.float32).astype(np.float64) * math.sqrt(H)
    for li, L in enumerate(layers):
        glob = li % cfg["global_every"] == cfg["global_every"] - 1
        theta = cfg["rope_theta_global"] if glob else cfg["rope_theta_local"]
        fs = cfg["rope_fs_global"] if glob else cfg["rope_fs_local"]
        n = rms(x, L["in_norm"])
        q = deq(L["q"], NQ * D, H) @ n
        k = deq(L["k"], NKV * D, H) @ n
        v = deq(L["v"], NKV * D, H) @ n
        q = np.concatenate([rms(q[h * D:(h + 1) * D], L["q_norm"]) for h in range(NQ)])
        k = np.concatenate([rms(k[h * D:(h + 1) * D], L["k_norm"]) for h in range(NKV)])
        q, k = rope(q, NQ, theta, fs), rope(k, NKV, theta, fs)
        K = L["k_cache"].astype(np.float64)
        V = L["v_cache"].astype(np.float64)
        K[pos], V[pos] = k, v
        k_end = pos + 1
        k_start = 0 if glob else max(0, k_end - cfg["sliding_window"])
        attn = np.empty(NQ * D)
        for h in range(NQ):
            kv = h // (NQ // NKV)
            s = K[k_start:k_end, kv * D:(kv + 1) * D] @ q[h * D:(h + 1) * D] * cfg["attn_scale"]
            p = np.exp(s - s.max())
            attn[h * D:(h + 1) * D] = (p / p.sum()) @ V[k_start:k_end, kv * D:(kv + 1) * D]
        o = deq(L["o"], H, NQ * D) @ attn
        x2 = x + rms(o, L["post_attn_norm"])
        n2 = rms(x2, L["pre_ffn_norm"])
        g = deq(L["gate"], cfg["ffn"], H) @ n2
        u = deq(L["up"], cfg["ffn"], H) @ n2
        hmid = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3))) * u
        m = deq(L["down"], H, cfg["ffn"]) @ hmid
        x = x2 + rms(m, L["post_ffn_norm"])
    xn = rms(x, final_norm)
    W = (embed.astype(np.uint32) << 16).view(np.float32).reshape(cfg["vocab"], H).astype(np.float64)
    return W @ xn


@pytest.mark.parametrize("pos", [3, 20])
def test_decode_step_vs_float64_restatement(orc, pos):
    """Tiny Gemma-3 (5 local + 1 global layer, window 8): position 3 sits inside
    the window, 20 slides it (local layers see 8 keys, the global layer 21)."""
    cfg = tiny_cfg()
    layers, embed, fnorm = make_model(orc, cfg, max_seq=32, ctx=pos)
    ref = np_decode_step(cfg, layers, embed, fnorm, token=7, pos=pos)
    got = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=7, pos=pos)
    assert rel_l2(got, ref) < 1e-4
    # the step appended row `pos` to every layer's cache and left others alone
    assert np.any(layers[0]["k_cache"][pos] != 0) and np.all(layers[0]["k_cache"][pos + 1:] == 0)
