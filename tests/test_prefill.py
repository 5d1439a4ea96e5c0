"""Prefill: the oracle's restatement of the reference prefill (forward_cached
over the whole prompt, transformer4.rs:1900-1964 and 2103-2139; attention
2882-2940 / 2661-2700) pinned on the CPU, then the GPU prefill
(rt_decode_prefill) against it."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from test_oracle import make_model

LOGITS_TOL = 1e-3  # rel-L2 of logits vs the oracle's f32 CPU order
# KV rows, per row (rel-L2 of each cache row), against the float64
# restatement of the arithmetic the GPU ran (assert_kv_rows): prompts or
# chunks of up to 8 rows run their projections on the batched GEMVs (16-bit
# activation digits, ~3e-5 per projection), so against the oracle; longer
# ones on the GEMM with f16-rounded operands (~3e-4 per projection), so
# against np_prefill(gpu_ops), which rounds every projection operand as the
# GEMM does and forms the attention's products from bf16 hi + lo parts as
# the prefill attention does (~2^-16 per product).  Against the oracle
# itself a later layer's rows inherit that rounding through the residual
# stream, and on the rare row whose sublayer
# output nearly cancels before a post-norm rescales it (the synthetic
# weights share a large positive mean, so the rounding errors of a row add
# coherently) it grows by 10-1000x: up to 2e-1 on one row of an 1100-row
# 4B-width prompt, ~3e-3 on a layer's aggregate of a tiny one, while the
# logits stay near 3e-5.  The restatement with the GPU's operand rounding
# reproduces those rows to ~1e-4, so the gap is that rounding and nothing
# else.
#   The bar of a row is KV_TOL plus c times the oracle's own deviation from
# float64 on that row, which measures how much the row amplifies rounding:
# about 5e-7 on an ordinary row (the bar stays ~KV_TOL) and 25-160x that on
# the rows of the mixed-format models (Q6_K / Q8_0 weights ~30x larger than
# Q4_K ones) that nearly cancel.  c is the ratio of the unit of the GPU
# arithmetic the comparison leaves unmodelled to f32's (2^-24): the batched
# GEMVs' digits, 2^-15 (c = 512); on the GEMM path the attention's bf16
# hi + lo products, 2^-16 (c = 256), which the restatement reproduces only
# approximately (the GPU splits the probabilities scaled by each 32-key
# stage's running maximum, the restatement by the row's final one).
KV_TOL = 2e-3         # per row
KV_C_DIGITS, KV_C_GEMM = 512.0, 256.0
KV_ORACLE_TOL = 5e-3  # per layer (aggregate), against the oracle


def row_err(a, b):
    return np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-30)


def assert_kv_rows(d, cfg, layers, embed, fnorm, toks, mode, gemm, ref_layers=None, agg_layers=None):
    """Every KV row of every layer of the GPU context d after a prefill of
    toks from position 0, against np_prefill(gpu_ops) (gemm True: the GEMM
    path) or the oracle (gemm False: the batched-GEMV path) within the row's
    bar (KV_TOL + c x the oracle's deviation from float64 on the row), and
    every layer within KV_ORACLE_TOL of agg_layers (default: the oracle).
    ref_layers: the oracle's caches after this prefill (computed if None)."""
    T = len(toks)
    if ref_layers is None:
        ref_layers = fresh_caches(layers)
        orc_mod().gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    with np.errstate(invalid="ignore", divide="ignore"):
        _, kv64, _ = np_prefill(cfg, layers, embed, fnorm, toks, mode)
        kv16 = np_prefill(cfg, layers, embed, fnorm, toks, mode, gpu_ops=True)[1] if gemm else None
    agg_layers = agg_layers or ref_layers
    for li in range(cfg["n_layers"]):
        k, v = read_kv(d, cfg, li, T)
        for i, c in enumerate(("k_cache", "v_cache")):
            g, o = (k, v)[i], ref_layers[li][c][:T]
            model = kv16[li][i] if gemm else o
            bar = KV_TOL + (KV_C_GEMM if gemm else KV_C_DIGITS) * row_err(o, kv64[li][i])
            er = row_err(g, model)
            agg = rel_l2(g, agg_layers[li][c][:T])
            r = int(np.argmax(er / bar))
            print(f"  layer {li} {'kv'[i]}: per-row max {er.max():.2e} vs "
                  f"{'GPU-operand float64' if gemm else 'the oracle'} (worst row {r}: {er[r]:.2e} of bar "
                  f"{bar[r]:.2e}); aggregate {agg:.2e}", flush=True)
            assert np.all(er <= bar), (li, "kv"[i], r, er[r], bar[r])
            assert agg < KV_ORACLE_TOL, (li, "kv"[i], agg)


def orc_mod():
    from oracle import oracle as o
    return o


def tiny(group: int = 2, **kw):
    base = dict(hidden=512, ffn=1024, n_q_heads=2, n_kv_heads=1, head_dim=256, n_layers=3, vocab=1000,
                sliding_window=8, global_every=3, rope_theta_local=10000.0, rope_theta_global=1000000.0,
                rope_fs_local=1.0, rope_fs_global=0.125, eps=1e-6, attn_scale=1.0 / 16.0)
    if group == 4:
        base.update(n_q_heads=4, n_kv_heads=1, head_dim=128, attn_scale=1.0 / np.sqrt(128.0))
    elif group == 1:
        base.update(n_q_heads=2, n_kv_heads=2, head_dim=256)
    base.update(kw)
    return base


def fresh_caches(layers, rows=None):
    """Copies of the model with zeroed caches (a prefill fills them itself)."""
    out = []
    for L in layers:
        M = dict(L)
        M["k_cache"] = np.zeros_like(L["k_cache"])
        M["v_cache"] = np.zeros_like(L["v_cache"])
        out.append(M)
    return out




def r16(x):
    """x rounded to f16's 11 significant bits, round-to-nearest-even, at any
    exponent: the prefill GEMM rounds each operand row to f16 after a
    power-of-two scale, so its rounding does not depend on the row's range."""
    m, e = np.frexp(x)
    return np.ldexp(np.round(m * 2048.0) / 2048.0, e)


def q4k_gemm_weights(blocks, rows, cols):
    """The f16 weights the prefill GEMM multiplies, as float64 [rows, cols].
    A Q4_K weight is w = s q - m (s = d sc, m = dmin mn of its sub-block);
    the GEMM forms it from the f16 half 1024 + q (low nibbles) or 1024 + 16 q
    (high nibbles) with one v_fma_mix: s (1024 + q) - fl32(m + 1024 s),
    resp. (s/16)(1024 + 16 q) - fl32(m + 64 s), rounded once to f16.  The
    f32 rounding of the constant moves some weights by one f16 ulp, all in
    the same direction within a sub-block."""
    s, m, nib, hi = _q4k_fields(blocks)
    c32 = np.where(hi, m + 64.0 * s, m + 1024.0 * s).astype(np.float32).astype(np.float64)
    pre = np.where(hi, (s / 16.0) * (1024.0 + 16.0 * nib), s * (1024.0 + nib)) - c32
    return r16(pre).reshape(rows, cols)


def _q4k_fields(blocks):
    """Per weight of Q4_K blocks (float64, [blocks, 8, 32]): the sub-block
    scale s = d sc and min m = dmin mn, the nibble q, and whether q is a
    high nibble (odd sub-block)."""
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dm = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    sc = b[:, 4:16].astype(np.uint32)
    sv = np.empty((b.shape[0], 8), np.uint32)
    mv = np.empty_like(sv)
    sv[:, :4], mv[:, :4] = sc[:, 0:4] & 63, sc[:, 4:8] & 63
    sv[:, 4:] = (sc[:, 8:12] & 15) | ((sc[:, 0:4] >> 6) << 4)
    mv[:, 4:] = (sc[:, 8:12] >> 4) | ((sc[:, 4:8] >> 6) << 4)
    q = b[:, 16:].reshape(-1, 4, 32)
    nib = np.stack([q & 15, q >> 4], axis=2).reshape(-1, 8, 32).astype(np.float64)
    return (d[:, None] * sv)[:, :, None], (dm[:, None] * mv)[:, :, None], nib, (np.arange(8) % 2 == 1)[None, :, None]


def bf16_split(x):
    """x (as f32) = hi + lo + O(2^-16 |x|): hi = bf16(x), lo = bf16(x - hi),
    both round-to-nearest-even (v_cvt_pk_bf16_f32), as float64."""
    def bf16(a):
        u = a.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    x32 = np.ascontiguousarray(x, np.float32)
    hi = bf16(x32)
    lo = bf16(np.ascontiguousarray(x32 - hi, np.float32))
    return hi.astype(np.float64), lo.astype(np.float64)


def split_matmul(a, b):
    """a @ b as the prefill attention's matrix cores form it from bf16 parts:
    hi*hi + hi*lo + lo*hi (lo*lo dropped), summed in float64."""
    ah, al = bf16_split(a)
    bh, bl = bf16_split(b)
    return ah @ bh + ah @ bl + al @ bh


def np_prefill(cfg, layers, embed, final_norm, tokens, mode, gpu_ops=False):
    """float64 restatement of a whole-prompt prefill (forward_cached over the
    prompt, transformer4.rs:1900-1964, attention 2882-2940 / 2661-2700),
    vectorised over rows and independent of the C oracle.  Returns the last
    row's logits, each layer's K and V rows, and each layer's conditioning per
    row as the fraction of a projection's magnitude that survives cancellation,
    |W x| / | |W| |x| |: (K, the smallest over heads, before the per-head norm
    divides it out; V; o and down, before their post-norms do; o counts as 1 on
    rows with no visible keys, whose attention is exactly 0).

    gpu_ops: the same in float64 with the GPU prefill's operand rounding:
    every projection operand rounded to f16 as the GEMM rounds it
    (activation rows by r16, Q4_K weights by q4k_gemm_weights), and the
    attention's scores and output products formed from bf16 hi + lo parts
    as its matrix cores form them (split_matmul); norms, RoPE, softmax and
    GELU stay float64."""
    mm = split_matmul if gpu_ops else (lambda a, b: a @ b)
    rnd = r16 if gpu_ops else (lambda a: a)
    from test_oracle import _numpy_dequant
    H, D, F = cfg["hidden"], cfg["head_dim"], cfg["ffn"]
    NQ, NKV = cfg["n_q_heads"], cfg["n_kv_heads"]
    eps, T, W_ = cfg["eps"], len(tokens), cfg["sliding_window"]
    pos = np.arange(T)

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * (1.0 + g.astype(np.float64))

    def deq(L, p, rows, cols):
        b, fmt = L[p], L.get("fmt", {}).get(p, 1)
        if fmt == 1:  # Q4_K
            if gpu_ops:
                return q4k_gemm_weights(b, rows, cols)
            return _numpy_dequant(b).reshape(rows, cols).astype(np.float64)
        # Q6_K / Q8_0 (GGUF blocks) and BF16: the f32 value, which the GEMM
        # rounds to f16 once (proj_gemm)
        from oracle import oracle as o
        if fmt == 4:
            w = o.q6k_dequant(b, rows * cols)
        elif fmt == 5:
            w = o.q8_0_dequant(b, rows * cols)
        else:
            w = (np.asarray(b).astype(np.uint32) << 16).view(np.float32)
        return rnd(w.reshape(rows, cols).astype(np.float64))

    def rope(x, nh, theta, fs):
        x = x.reshape(T, nh, D).copy()
        half = D // 2
        ang = np.outer(pos * fs, 1.0 / theta ** (2 * np.arange(half) / D))[:, None, :]
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = x[..., :half].copy(), x[..., half:].copy()
        x[..., :half] = x0 * c - x1 * s
        x[..., half:] = x0 * s + x1 * c
        return x.reshape(T, nh * D)

    E = (embed.astype(np.uint32) << 16).view(np.float32).reshape(cfg["vocab"], H).astype(np.float64)
    x = E[np.asarray(tokens)] * np.sqrt(H)
    out_kv, cond = [], []
    for li, L in enumerate(layers):
        glob = cfg["global_every"] > 0 and li % cfg["global_every"] == cfg["global_every"] - 1
        theta = cfg["rope_theta_global"] if glob else cfg["rope_theta_local"]
        fs = cfg["rope_fs_global"] if glob else cfg["rope_fs_local"]
        n = rnd(rms(x, L["in_norm"]))
        Wk, Wv = deq(L, "k", NKV * D, H), deq(L, "v", NKV * D, H)
        q, k, v = n @ deq(L, "q", NQ * D, H).T, n @ Wk.T, n @ Wv.T
        mag_k = (np.abs(n) @ np.abs(Wk).T).reshape(T, NKV, D)
        kc = np.linalg.norm(k.reshape(T, NKV, D), axis=2) / np.linalg.norm(mag_k, axis=2)
        vc = np.linalg.norm(v, axis=1) / np.linalg.norm(np.abs(n) @ np.abs(Wv).T, axis=1)
        cond.append((kc.min(axis=1), vc))
        q = rms(q.reshape(T, NQ, D), L["q_norm"]).reshape(T, NQ * D)
        k = rms(k.reshape(T, NKV, D), L["k_norm"]).reshape(T, NKV * D)
        q, k = rope(q, NQ, theta, fs), rope(k, NKV, theta, fs)
        out_kv.append((k, v))
        attn = np.zeros((T, NQ * D))
        for h in range(NQ):
            kv = h // (NQ // NKV)
            S = mm(q[:, h * D:(h + 1) * D], k[:, kv * D:(kv + 1) * D].T) * cfg["attn_scale"]
            r, c = np.meshgrid(pos, pos, indexing="ij")
            if glob or W_ == 0:
                vis = c <= r
            elif mode == 0:  # the reference's prefill rule: one window for the whole prompt
                lo = max(0, T - W_)
                vis = (r >= lo) & (c >= lo) & (c <= r)
            else:
                vis = (c <= r) & (c >= r + 1 - W_)
            S = np.where(vis, S, -np.inf)
            m = S.max(axis=1, keepdims=True)
            P = np.where(vis, np.exp(S - np.where(np.isfinite(m), m, 0)), 0.0)
            den = P.sum(axis=1, keepdims=True)
            attn[:, h * D:(h + 1) * D] = np.where(den > 0, mm(P, v[:, kv * D:(kv + 1) * D]) / np.where(den > 0, den, 1), 0)
        Wo, Wd = deq(L, "o", H, NQ * D), deq(L, "down", H, F)
        o = rnd(attn) @ Wo.T
        x2 = x + rms(o, L["post_attn_norm"])
        n2 = rnd(rms(x2, L["pre_ffn_norm"]))
        g, u = n2 @ deq(L, "gate", F, H).T, n2 @ deq(L, "up", F, H).T
        hm = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * u
        dn = rnd(hm) @ Wd.T
        x = x2 + rms(dn, L["post_ffn_norm"])
        # the post-norms rescale each sublayer output to unit RMS: a row whose
        # o or down output mostly cancels carries its rounding error, so
        # enlarged, into the residual stream of every later layer
        with np.errstate(invalid="ignore", divide="ignore"):
            co = np.linalg.norm(o, axis=1) / np.linalg.norm(np.abs(attn) @ np.abs(Wo).T, axis=1)
        cd = np.linalg.norm(dn, axis=1) / np.linalg.norm(np.abs(hm) @ np.abs(Wd).T, axis=1)
        cond[-1] = cond[-1] + (np.where(np.isfinite(co), co, 1.0), cd)
    return E @ rms(x[-1], final_norm), out_kv, cond


# ---------------------------------------------------------------------------
# oracle pins (CPU)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("mixed", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
def test_np_prefill_restates_the_oracle(orc, mode, mixed):
    """np_prefill (float64, the KV bar's restatement) agrees with the oracle's
    f32 prefill on the logits and on every KV row, with Q4_K layers and with
    Q6_K / Q8_0 / BF16 projections mixed in, under both window rules (20 rows
    pass the window of 8)."""
    from test_kquant import MIXED_PLAN, apply_formats
    cfg = tiny(2)
    T = 20
    layers, embed, fnorm = make_model(orc, cfg, max_seq=T, ctx=0, seed=8100 + mode + 2 * mixed)
    if mixed:
        apply_formats(orc, cfg, layers, MIXED_PLAN, seed=8110 + mode)
    toks = [(7 * i + 1) % cfg["vocab"] for i in range(T)]
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    lg, kv, _ = np_prefill(cfg, layers, embed, fnorm, toks, mode)
    assert rel_l2(ref, lg) < 1e-5
    for li in range(cfg["n_layers"]):
        assert row_err(ref_layers[li]["k_cache"][:T], kv[li][0]).max() < 1e-4
        assert row_err(ref_layers[li]["v_cache"][:T], kv[li][1]).max() < 1e-4


def test_q4k_gemm_weights_round_the_dequantised_weight(orc):
    """The GEMM's f16 weights are within one f16 ulp of the exact Q4_K
    weight plus the f32 rounding of the constant m + 1024 s (which dominates
    only where s q nearly cancels m), equal to its plain f16 rounding on
    most weights, and exact where the weight needs at most 11 bits (d = 1,
    dmin = 0)."""
    from test_oracle import _numpy_dequant
    blocks = orc.synth_q4k(21, 64, 1024)
    exact = _numpy_dequant(blocks).astype(np.float64).reshape(64, 1024)
    got = q4k_gemm_weights(blocks, 64, 1024)
    s, m, _, _ = _q4k_fields(blocks)
    c_ulp = np.broadcast_to(2.0 ** -23 * (m + 1024.0 * s), (blocks.size // 144, 8, 32)).reshape(64, 1024)
    ulp = np.ldexp(1.0, np.frexp(exact)[1] - 11)
    assert np.all(np.abs(got - exact) <= ulp + c_ulp)
    assert np.mean(np.abs(got - exact) > ulp) < 0.01
    assert np.mean(got == r16(exact)) > 0.9
    b = blocks.reshape(-1, 144).copy()
    b[:, 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)  # d = 1
    b[:, 2:4] = 0                                              # dmin = 0
    assert np.array_equal(q4k_gemm_weights(b, 64, 1024), _numpy_dequant(b).astype(np.float64).reshape(64, 1024))


def test_r16_is_float16_rounding_at_any_scale():
    """r16 (the f16 operand rounding of np_prefill) is numpy's own float16
    round-to-nearest-even wherever float16 is normal, and commutes with
    power-of-two scales (ties included: x.5 ulp cases)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(200000) * 100
    x = x[np.abs(x) > 1e-3]
    ties = (1024 + np.arange(1, 200, 2) / 2.0) * 2.0 ** -10  # exactly half an f16 ulp above a grid point
    for v in (x, ties, -ties):
        assert np.array_equal(r16(v), v.astype(np.float16).astype(np.float64))
        assert np.array_equal(r16(v * 2.0 ** -60), r16(v) * 2.0 ** -60)


def np_attention_reference(q, kc, vc, T, k_start, nq, nkv, d, scale):
    """float64 brute force of gqa_attention_cached's prefill branch written
    from its own conditions (transformer4.rs:2909-2937): query row r attends
    window index c (key k_start + c) iff r >= k_start and c <= r - k_start."""
    out = np.zeros((T, nq * d))
    t_kv = T - k_start
    for qh in range(nq):
        kvh = qh // (nq // nkv)
        K = kc[k_start:T, kvh * d:(kvh + 1) * d].astype(np.float64)
        V = vc[k_start:T, kvh * d:(kvh + 1) * d].astype(np.float64)
        S = q[:, qh * d:(qh + 1) * d].astype(np.float64) @ K.T * scale
        for r in range(T):
            if r < k_start:
                continue
            max_kv = min(r - k_start, t_kv - 1)
            e = np.exp(S[r, :max_kv + 1] - S[r, :max_kv + 1].max())
            out[r, qh * d:(qh + 1) * d] = (e / e.sum()) @ V[:max_kv + 1]
    return out


def np_attention_windowed(q, k, v, T, window, nq, nkv, d, scale):
    """float64 brute force of gqa_attention_windowed's mask (transformer4.rs:
    2686-2695): causal_ok = c <= r, window_ok = r < window || c >= r + 1 - window."""
    out = np.zeros((T, nq * d))
    for qh in range(nq):
        kvh = qh // (nq // nkv)
        S = q[:, qh * d:(qh + 1) * d].astype(np.float64) @ k[:T, kvh * d:(kvh + 1) * d].astype(np.float64).T * scale
        for r in range(T):
            ok = np.array([c <= r and (r < window or c >= r + 1 - window) for c in range(T)])
            s = np.where(ok, S[r], -np.inf)
            e = np.exp(s - s.max())
            out[r, qh * d:(qh + 1) * d] = (e / e.sum()) @ v[:T, kvh * d:(kvh + 1) * d].astype(np.float64)
    return out


@pytest.mark.parametrize("nq,nkv", [(2, 1), (4, 2), (2, 2)])
@pytest.mark.parametrize("T,window", [(20, 8), (7, 8), (33, 1)])
def test_oracle_prefill_attention_vs_bruteforce(orc, nq, nkv, T, window):
    rng = np.random.default_rng(T * 10 + nq + nkv)
    d = 16
    q = rng.standard_normal((T, nq * d)).astype(np.float32)
    kc = rng.standard_normal((T, nkv * d)).astype(np.float32)
    vc = rng.standard_normal((T, nkv * d)).astype(np.float32)
    scale = 0.25
    k_start = max(0, T - window)
    got = orc.gqa_attention_prefill(q, kc, vc, 0, T, k_start, 0, nq, nkv, d, scale)
    ref = np_attention_reference(q, kc, vc, T, k_start, nq, nkv, d, scale)
    assert np.abs(got - ref).max() < 1e-5
    if k_start > 0:  # rows before the window start attend to nothing
        assert not np.any(got[:k_start])
    got = orc.gqa_attention_prefill(q, kc, vc, 0, T, 0, window, nq, nkv, d, scale)
    ref = np_attention_windowed(q, kc, vc, T, window, nq, nkv, d, scale)
    assert np.abs(got - ref).max() < 1e-5


def test_oracle_prefill_attention_offset_rows(orc):
    """Rows at p0 > 0 see the cache rows before the chunk: the last rows of a
    full-prompt attention equal a chunk's rows at the same positions."""
    rng = np.random.default_rng(5)
    T, p0, d, nq, nkv = 30, 12, 16, 4, 2
    q = rng.standard_normal((T, nq * d)).astype(np.float32)
    kc = rng.standard_normal((T, nkv * d)).astype(np.float32)
    vc = rng.standard_normal((T, nkv * d)).astype(np.float32)
    for lo_fixed, window in [(0, 0), (0, 7), (10, 0)]:
        full = orc.gqa_attention_prefill(q, kc, vc, 0, T, lo_fixed, window, nq, nkv, d, 0.3)
        part = orc.gqa_attention_prefill(q[p0:], kc, vc, p0, T - p0, lo_fixed, window, nq, nkv, d, 0.3)
        assert np.array_equal(full[p0:], part)


@pytest.mark.parametrize("group", [2, 4])
def test_oracle_sliding_prefill_equals_decode_steps(orc, group):
    """Per-row sliding window: a prefill of T tokens is T decode steps (the
    decode-step oracle, pinned separately, restates the t_q == 1 branch)."""
    cfg = tiny(group)
    T, max_seq = 14, 16
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=4100 + group)
    toks = [(7 * i + 3) % cfg["vocab"] for i in range(T)]
    a = fresh_caches(layers)
    got = orc.gemma3_prefill(cfg, a, embed, fnorm, toks, 0, mode=1)
    b = fresh_caches(layers)
    for i, t in enumerate(toks):
        ref = orc.gemma3_decode_step(cfg, b, embed, fnorm, token=t, pos=i)
    assert rel_l2(got, ref) < 2e-5
    for La, Lb in zip(a, b):
        assert rel_l2(La["k_cache"][:T], Lb["k_cache"][:T]) < 2e-5
        assert rel_l2(La["v_cache"][:T], Lb["v_cache"][:T]) < 2e-5


def test_oracle_reference_prefill_short_prompt_equals_sliding(orc):
    """With T <= window both window rules select the same keys."""
    cfg = tiny(2)
    layers, embed, fnorm = make_model(orc, cfg, max_seq=8, ctx=0, seed=4200)
    toks = [1, 2, 3, 4, 5, 6, 7, 8]
    a, b = fresh_caches(layers), fresh_caches(layers)
    la = orc.gemma3_prefill(cfg, a, embed, fnorm, toks, 0, mode=0)
    lb = orc.gemma3_prefill(cfg, b, embed, fnorm, toks, 0, mode=1)
    assert np.array_equal(la, lb)


def test_oracle_reference_prefill_long_prompt_differs(orc):
    """T > window: the reference rule zeroes the attention of early rows, so
    the result differs from the sliding rule (a dropped lo_fixed would not)."""
    cfg = tiny(2)
    T = 14
    layers, embed, fnorm = make_model(orc, cfg, max_seq=T, ctx=0, seed=4300)
    toks = list(range(3, 3 + T))
    a, b = fresh_caches(layers), fresh_caches(layers)
    la = orc.gemma3_prefill(cfg, a, embed, fnorm, toks, 0, mode=0)
    lb = orc.gemma3_prefill(cfg, b, embed, fnorm, toks, 0, mode=1)
    assert rel_l2(la, lb) > 1e-6
    # layer 0's K/V rows come before any attention, so they agree; layer 1's
    # rows before the window start see a residual stream without attention
    assert np.array_equal(a[0]["k_cache"], b[0]["k_cache"])
    early = T - cfg["sliding_window"]
    assert rel_l2(a[1]["k_cache"][:early], b[1]["k_cache"][:early]) > 1e-2


# ---------------------------------------------------------------------------
# GPU prefill vs the oracle
# ---------------------------------------------------------------------------
def gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq):
    d = rt.HipDecodeContext(cfg, max_seq)
    for i, L in enumerate(layers):
        d.set_layer(i, L)
    d.set_embed(embed, fnorm)
    return d


def read_kv(d, cfg, layer, rows):
    from test_gpu_decode import d2h
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    kp, vp = d.kv_ptrs(layer)
    return d2h(kp, rows * kvd).reshape(rows, kvd), d2h(vp, rows * kvd).reshape(rows, kvd)


@pytest.mark.gpu
@pytest.mark.parametrize("group", [2, 4, 1])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("T", [1, 5, 20, 77])
def test_gpu_prefill_matches_oracle(rt, orc, group, mode, T):
    """T = 1 and 5 (inside the window of 8), 20 and 77 (window passed: the
    reference rule zeroes early rows' attention; 77 rows span several 64-column
    attention workgroups and 32-key stages)."""
    cfg = tiny(group)
    max_seq = 96
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=5000 + 10 * group + T)
    toks = [(13 * i + 5) % cfg["vocab"] for i in range(T)]
    d = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    got = d.prefill(toks, 0, mode)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    assert_kv_rows(d, cfg, layers, embed, fnorm, toks, mode, T > 8, ref_layers)
    d.close()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("T", [6, 77])
def test_gpu_generic_shape_prefill_matches_oracle(rt, orc, mode, T):
    """A shape outside the fused decode kernels (hidden 768, 4 heads x 128,
    ffn 1536): prefill (batched GEMV at 6 rows, the GEMM at 77) and the
    following decode step against the oracle."""
    from test_gpu_decode import generic_cfg
    import copy
    cfg = generic_cfg()
    max_seq = 96
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=7000 + T + mode)
    toks = [(13 * i + 5) % cfg["vocab"] for i in range(T)]
    d = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    got = d.prefill(toks, 0, mode)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    assert_kv_rows(d, cfg, layers, embed, fnorm, toks, mode, T > 8, ref_layers)
    if mode == 1:  # the step after a sliding-rule prefill sees the prefilled cache
        step = d.decode_step(11, T)
        rstep = orc.gemma3_decode_step(cfg, copy.deepcopy(ref_layers), embed, fnorm, token=11, pos=T)
        assert rel_l2(step, rstep) < LOGITS_TOL
    d.close()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
def test_gpu_long_prompt_prefill_matches_oracle(rt, orc, mode):
    """1100 rows: the projections run on the half-block GEMM with K split
    (the consumers add the partial tiles while reading them), attention on
    eight-wave workgroups of 128 columns; logits and KV rows vs the oracle."""
    cfg = tiny(2, sliding_window=300)
    T, max_seq = 1100, 1104
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=6400 + mode)
    toks = [(29 * i + 7) % cfg["vocab"] for i in range(T)]
    d = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    got = d.prefill(toks, 0, mode)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    assert_kv_rows(d, cfg, layers, embed, fnorm, toks, mode, True, ref_layers)
    d.close()


@pytest.mark.gpu
def test_gpu_prefill_chunks_and_continuation(rt, orc):
    """Chunked prefill (7 rows per chunk: chunks of up to 8 rows run their
    projections on the batched GEMV, larger ones on the GEMM) and a prefill
    continued at start_position > 0 give the single-call result (sliding
    rule), and the next decode step sees the prefilled cache."""
    cfg = tiny(2)
    T, max_seq = 30, 40
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=6100)
    toks = [(11 * i + 2) % cfg["vocab"] for i in range(T)]
    d1 = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    full = d1.prefill(toks, 0, 1)
    d2 = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    d2.set_prefill_chunk(7)
    chunked = d2.prefill(toks, 0, 1)
    d3 = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    d3.prefill(toks[:17], 0, 1)
    cont = d3.prefill(toks[17:], 17, 1)
    assert rel_l2(chunked, full) < LOGITS_TOL  # batched GEMV (16-bit digits) vs GEMM (f16 operands)
    assert rel_l2(cont, full) < 1e-5           # both halves on the GEMM
    for li in range(cfg["n_layers"]):
        k1, v1 = read_kv(d1, cfg, li, T)
        k3, v3 = read_kv(d3, cfg, li, T)
        assert rel_l2(k3, k1) < 1e-5 and rel_l2(v3, v1) < 1e-5
    ref_layers = fresh_caches(layers)
    orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, 1)
    nxt = d1.decode_step(9, T)
    ref = orc.gemma3_decode_step(cfg, ref_layers, embed, fnorm, token=9, pos=T)
    assert rel_l2(nxt, ref) < LOGITS_TOL
    for d in (d1, d2, d3):
        d.close()


@pytest.mark.gpu
def test_gpu_prefill_wide_window_key_split_continuation(rt, orc):
    """GQA group 1 (one q head per KV head), window 512, a continuation at
    start_position 30 of 640 rows under the sliding rule: the attention runs
    on eight-wave workgroups of 128 rows with the keys split, and a row
    block's keys start 32-aligned below the window of its first row, so its
    range is window + 128 + 30 keys here.  The prompt's last row is the last
    row of a full block, so the logits see whether it attended to its own and
    the 29 keys before it; every KV row against the oracle too."""
    cfg = tiny(1, sliding_window=512)
    p0, T = 30, 640
    max_seq = p0 + T + 8
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=6700)
    toks = [(17 * i + 4) % cfg["vocab"] for i in range(p0 + T)]
    d = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    d.prefill(toks[:p0], 0, 1)
    got = d.prefill(toks[p0:], p0, 1)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, 1)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    # both calls run on the GEMM (30 and 640 rows), whose rounding is per row
    assert_kv_rows(d, cfg, layers, embed, fnorm, toks, 1, True, ref_layers)
    d.close()


@pytest.mark.gpu
def test_gpu_prefill_rejects_bad_calls(rt, orc):
    cfg = tiny(2)
    layers, embed, fnorm = make_model(orc, cfg, max_seq=16, ctx=0, seed=6200)
    d = gpu_ctx(rt, cfg, layers, embed, fnorm, 16)
    with pytest.raises(rt.RtError):
        d.prefill([], 0, 0)
    with pytest.raises(rt.RtError):
        d.prefill([1, 2], 3, 0)  # the reference rule starts at position 0
    with pytest.raises(rt.RtError):
        d.prefill([1] * 10, 10, 1)  # past max_seq
    with pytest.raises(rt.RtError):
        d.prefill([1, cfg["vocab"]], 0, 1)  # token out of range
    with pytest.raises(rt.RtError):
        d.prefill([1, 2], 0, 2)  # unknown mode
    with pytest.raises(rt.RtError):
        d.set_prefill_chunk(0)
    d.close()


@pytest.mark.gpu
def test_gemma3_4b_shape_prefill_equals_decode_steps(rt, orc):
    """Gemma-3-4B layer shapes (2 layers, one local one global, vocab 4096):
    a 300-token sliding-rule prefill on the matrix cores equals 300 GPU decode
    steps (GEMV path, pinned to the oracle elsewhere) in logits and KV rows
    (the prefill's rows also per row against np_prefill(gpu_ops))."""
    cfg = dict(rt.GEMMA3_4B, n_layers=2, global_every=2, vocab=4096)
    T, max_seq = 300, 320
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=6300)
    toks = [(97 * i + 1) % cfg["vocab"] for i in range(T)]
    d1 = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    got = d1.prefill(toks, 0, 1)
    d2 = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    for i, t in enumerate(toks):
        d2.decode_step_async(t, i)
    d2.synchronize()
    from test_gpu_decode import d2h
    ref = d2h(d2.logits_ptr(), cfg["vocab"])
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    steps = [dict(zip(("k_cache", "v_cache"), read_kv(d2, cfg, li, T))) for li in range(2)]
    assert_kv_rows(d1, cfg, layers, embed, fnorm, toks, 1, True, agg_layers=steps)
    d1.close()
    d2.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T,mode", [(1100, 0), (1100, 1), (960, 1)])
def test_gemma3_4b_width_long_prefill_matches_oracle(rt, orc, T, mode):
    """The benchmarked prefill path at Gemma-3-4B widths: 2 layers (one local
    with window 1024, one global) and 1100 rows, so each projection set
    (q|k|v, gate|up) runs as one launch of the half-block GEMM, K is split
    where tiles are few and the consumers add the partial tiles; both window
    rules.  At 960 rows the gate|up set (640 tiles) still runs as one
    half-block launch while q|k|v, o and down take the eight-wave kernel.
    Logits against the oracle at the north-star bar.  KV rows: the oracle
    on every row against a float64 restatement (np_prefill), and the GPU on
    every row within KV_TOL of the same restatement with the GPU's operand
    rounding (np_prefill gpu_ops).

    Layer 0's KV rows carry only the f16-operand rounding of their own
    projections (~3e-4 from the oracle on every row).  Later layers inherit
    the rounding of the whole residual stream: on most rows less (the
    synthetic weights have a large positive mean, ~3.3, so activations are
    large), but on the few rows whose sublayer outputs the post-norms scale
    up from near-cancellation the error adds coherently across the row and
    reaches 1e-2 to 2e-1 from the oracle on under 1% of rows.  With zero-mean
    weights the same prompt shows no such rows (every row 3e-4 to 8e-4).
    The restatement with the GPU's operand rounding reproduces those rows to
    within 1e-3 (5e-5
    on layer 0), so the gap to the oracle is the operand rounding; the
    oracle's own per-row median (1e-3) and 99th percentile (1e-2) are held
    as well."""
    cfg = dict(rt.GEMMA3_4B, n_layers=2, global_every=2, vocab=4096)
    max_seq = T + 4
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=6500 + mode)
    toks = [(31 * i + 3) % cfg["vocab"] for i in range(T)]
    d = gpu_ctx(rt, cfg, layers, embed, fnorm, max_seq)
    got = d.prefill(toks, 0, mode)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    with np.errstate(invalid="ignore", divide="ignore"):
        lg64, kv64, _ = np_prefill(cfg, layers, embed, fnorm, toks, mode)
        _, kv16, _ = np_prefill(cfg, layers, embed, fnorm, toks, mode, gpu_ops=True)
    assert rel_l2(ref, lg64) < 1e-5
    err = rel_l2(got, ref)
    print(f"4B-width prefill T={T} mode={mode}: logits rel-L2 {err:.2e}", flush=True)
    assert np.all(np.isfinite(got)) and err < LOGITS_TOL
    for li in range(2):
        k, v = read_kv(d, cfg, li, T)
        for g, o, e64, e16 in ((k, ref_layers[li]["k_cache"][:T], kv64[li][0], kv16[li][0]),
                               (v, ref_layers[li]["v_cache"][:T], kv64[li][1], kv16[li][1])):
            assert row_err(o, e64).max() < 1e-4  # the oracle on every row, against float64
            er, e_ops = row_err(g, o), row_err(g, e16)
            print(f"  layer {li}: per-row median {np.median(er):.2e} p99 {np.percentile(er, 99):.2e} "
                  f"max {er.max():.2e} vs the oracle; max {e_ops.max():.2e} vs GPU-operand float64", flush=True)
            assert e_ops.max() < KV_TOL, (li, int(np.argmax(e_ops)), e_ops.max())
            assert np.median(er) < 1e-3 and np.percentile(er, 99) < 1e-2
            if li == 0:
                assert er.max() < 1e-3
    d.close()
