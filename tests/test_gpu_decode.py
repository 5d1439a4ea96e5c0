"""GPU decode step (librt_hip.so rt_decode_*) against the CPU oracle's
restatement of the reference decode step (transformer4.rs:1900-1964,
2358-2385), on seeded synthetic weights."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from test_oracle import make_model

pytestmark = pytest.mark.gpu

LOGITS_TOL = 1e-3  # rel-L2 of the logits vs the oracle's f32 CPU order


def tiny(group: int = 2, **kw):
    base = dict(hidden=512, ffn=1024, n_q_heads=2, n_kv_heads=1, head_dim=256, n_layers=6, vocab=1000,
                sliding_window=8, global_every=6, rope_theta_local=10000.0, rope_theta_global=1000000.0,
                rope_fs_local=1.0, rope_fs_global=0.125, eps=1e-6, attn_scale=1.0 / 16.0)
    if group == 4:
        base.update(n_q_heads=4, n_kv_heads=1, head_dim=128, attn_scale=1.0 / np.sqrt(128.0))
    elif group == 1:
        base.update(n_q_heads=2, n_kv_heads=2, head_dim=256)
    base.update(kw)
    return base


def build_ctx(rt, cfg, layers, embed, fnorm, ctx_len, max_seq):
    d = rt.HipDecodeContext(cfg, max_seq)
    for i, L in enumerate(layers):
        d.set_layer(i, L)
        d.sync_kv_from_cpu(i, np.ascontiguousarray(L["k_cache"][:ctx_len]),
                           np.ascontiguousarray(L["v_cache"][:ctx_len]), ctx_len)
    d.set_embed(embed, fnorm)
    return d


@pytest.mark.parametrize("group", [2, 4, 1])
@pytest.mark.parametrize("pos", [0, 3, 20])
def test_tiny_decode_step_matches_oracle(rt, orc, group, pos):
    """Position 0 (first token, no history), 3 (inside the window of 8) and 20
    (window slid; the global layer sees 21 keys)."""
    cfg = tiny(group)
    max_seq = 48
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=pos, seed=500 + group)
    d = build_ctx(rt, cfg, layers, embed, fnorm, pos, max_seq)
    got = d.decode_step(17, pos)
    ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=17, pos=pos)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < LOGITS_TOL
    d.close()


@pytest.mark.parametrize("group", [2, 4])
@pytest.mark.parametrize("window,max_seq,pos", [(40, 300, 250), (37, 200, 63), (0, 130, 129)])
def test_tiny_decode_ragged_chunks(rt, orc, group, window, max_seq, pos):
    """Key spans that split into several chunks whose last wave's keys are
    partly filled (global: 251 keys over 10 chunks of 26, waves of 7; window
    40 over 3 chunks of 14, waves of 4), a window that does not divide into
    16, and global_every 0 with the new row the last of max_seq."""
    cfg = tiny(group, sliding_window=window, global_every=0 if window == 0 else 6)
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=pos, seed=900 + pos + group)
    d = build_ctx(rt, cfg, layers, embed, fnorm, pos, max_seq)
    got = d.decode_step(5, pos)
    ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=5, pos=pos)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < LOGITS_TOL
    d.close()


@pytest.mark.parametrize("group", [2, 4])
def test_tiny_decode_long_context(rt, orc, group):
    """A context of 19,990 rows in a max_seq of 20,000: the global layer's
    keys split into 625 chunks, so the chunk merge folds its partials in
    several batches, and an 8-token verify batch splits the same keys for its
    row attention; both against the oracle (the batch against 8 sequential
    oracle steps)."""
    import copy
    cfg = tiny(group, n_layers=3, global_every=3)
    max_seq, ctx = 20000, 19990
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=2000 + group)
    d = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    olayers = copy.deepcopy(layers)
    got = d.decode_step(11, ctx)
    ref = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=11, pos=ctx)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < LOGITS_TOL
    toks = [(13 * i + 5) % cfg["vocab"] for i in range(8)]
    gb = d.decode_step_batch(toks, ctx + 1)
    for i, t in enumerate(toks):
        r = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=t, pos=ctx + 1 + i)
        assert rel_l2(gb[i], r) < LOGITS_TOL, i
    d.close()


def test_tiny_multi_step_kv_append_and_graph_replay(rt, orc):
    """Several consecutive steps replay one captured graph; K/V rows appended
    by the GPU match the oracle's cache.append rows."""
    cfg = tiny(2)
    max_seq, ctx = 40, 5
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=77)
    d = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    tokens = [3, 999, 0, 512, 41, 7, 8, 9, 10, 11]
    for i, tok in enumerate(tokens):
        pos = ctx + i
        got = d.decode_step(tok, pos)
        ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=tok, pos=pos)
        assert rel_l2(got, ref) < LOGITS_TOL, (i, rel_l2(got, ref))
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    rows = ctx + len(tokens)
    for li in (0, 5):
        kp, vp = d.kv_ptrs(li)
        k, v = d2h(kp, rows * kvd), d2h(vp, rows * kvd)
        kr = layers[li]["k_cache"][:rows].reshape(-1)
        vr = layers[li]["v_cache"][:rows].reshape(-1)
        assert np.array_equal(k[:ctx * kvd], kr[:ctx * kvd])   # prefilled rows untouched
        assert np.array_equal(v[:ctx * kvd], vr[:ctx * kvd])
        assert rel_l2(k, kr) < 1e-4 and rel_l2(v, vr) < 1e-4  # appended rows
    d.close()


def d2h(ptr: int, n: int) -> np.ndarray:
    """Copy n floats from a device pointer owned by the library."""
    import ctypes
    out = np.empty(n, np.float32)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipDeviceSynchronize()
    st = hip.hipMemcpy(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(ptr), ctypes.c_size_t(n * 4), 2)
    assert st == 0
    return out


def test_eager_and_graph_paths_agree(rt, orc):
    cfg = tiny(2)
    layers, embed, fnorm = make_model(orc, cfg, max_seq=32, ctx=12, seed=91)
    d1 = build_ctx(rt, cfg, layers, embed, fnorm, 12, 32)
    d2 = build_ctx(rt, cfg, layers, embed, fnorm, 12, 32)
    d2.set_graph(False)
    a = d1.decode_step(5, 12)
    b = d2.decode_step(5, 12)
    assert np.array_equal(a, b)
    d1.close()
    d2.close()


def test_decode_rejects_bad_calls(rt, orc):
    cfg = tiny(2)
    d = rt.HipDecodeContext(cfg, 16)
    with pytest.raises(rt.RtError) as e:
        d.decode_step(1, 0)  # weights not set
    assert e.value.code == rt.RT_ESTATE
    layers, embed, fnorm = make_model(orc, cfg, max_seq=16, ctx=0, seed=3)
    for i, L in enumerate(layers):
        d.set_layer(i, L)
    d.set_embed(embed, fnorm)
    with pytest.raises(rt.RtError):
        d.decode_step(cfg["vocab"], 0)   # token out of range
    with pytest.raises(rt.RtError):
        d.decode_step(0, 16)             # position beyond max_seq
    d.close()
    with pytest.raises(rt.RtError):
        rt.HipDecodeContext(dict(cfg, hidden=700), 16)  # unsupported shape (not whole Q4_K blocks)


def test_gemma3_4b_shape_decode_step_matches_oracle(rt, orc, dev):
    """34 layers, hidden 2560, FFN 10240, 8/4 heads of 256,
    5 local (window 1024) : 1 global, vocab 262144, 4096 prefilled tokens of
    N(0,1) K/V, f32 cache; decode at position 4096."""
    cfg = dict(rt.GEMMA3_4B)
    ctx = 4096
    max_seq = ctx + 8
    H, F, D = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QD, KVD = cfg["n_q_heads"] * D, cfg["n_kv_heads"] * D
    layers = []
    s = 9000
    for _ in range(cfg["n_layers"]):
        L = {}
        for name, (rows, cols) in dict(q=(QD, H), k=(KVD, H), v=(KVD, H), o=(H, QD), gate=(F, H), up=(F, H),
                                       down=(H, F)).items():
            s += 1
            L[name] = orc.synth_q4k(s, rows, cols)
        for name, n in dict(in_norm=H, post_attn_norm=H, pre_ffn_norm=H, post_ffn_norm=H, q_norm=D,
                            k_norm=D).items():
            s += 1
            L[name] = orc.synth_normal(s, n, 0.0, 0.1)
        s += 1
        kc = np.zeros((max_seq, KVD), np.float32)
        kc[:ctx] = orc.synth_normal(s, ctx * KVD).reshape(ctx, KVD)
        s += 1
        vc = np.zeros((max_seq, KVD), np.float32)
        vc[:ctx] = orc.synth_normal(s, ctx * KVD).reshape(ctx, KVD)
        L["k_cache"], L["v_cache"] = kc, vc
        layers.append(L)
    embed = orc.synth_bf16(8888, cfg["vocab"] * H, 0.02)
    fnorm = orc.synth_normal(8887, H, 0.0, 0.1)
    d = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    got = d.decode_step(12345, ctx)
    ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=12345, pos=ctx)
    err = rel_l2(got, ref)
    print(f"gemma3-4b shape logits rel-L2 {err:.3e}")
    assert np.all(np.isfinite(got))
    assert err < LOGITS_TOL
    assert int(np.argmax(got)) == int(np.argmax(ref))
    # next token continues from the appended row
    got2 = d.decode_step(int(np.argmax(got)), ctx + 1)
    ref2 = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=int(np.argmax(ref)), pos=ctx + 1)
    assert rel_l2(got2, ref2) < LOGITS_TOL
    d.close()


# ---------------------------------------------------------------------------
# decode_step_batch (metal_decode.rs:2079-2179)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("m", [1, 3, 8])
def test_batch_matches_sequential_and_oracle(rt, orc, m):
    """M tokens at consecutive positions: the window of 8 slides inside the
    batch and the global layer sees every earlier batch token.  The batch
    runs every layer for all M rows at once (batched GEMVs on the int8
    matrix cores, the causal row attention, a batched lm_head), so it agrees
    with M single steps to the digit rounding of the two GEMV paths."""
    import copy
    cfg = tiny(2)
    max_seq, ctx = 48, 9
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=300 + m)
    toks = [(7 * i + 3) % cfg["vocab"] for i in range(m)]
    d_batch = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    d_seq = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    got = d_batch.decode_step_batch(toks, ctx)
    assert got.shape == (m, cfg["vocab"])
    seq = np.stack([d_seq.decode_step(t, ctx + i) for i, t in enumerate(toks)])
    olayers = copy.deepcopy(layers)
    ref = np.stack([orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=t, pos=ctx + i)
                    for i, t in enumerate(toks)])
    for i in range(m):
        assert rel_l2(got[i], seq[i]) < 2e-4, (i, rel_l2(got[i], seq[i]))
        assert rel_l2(got[i], ref[i]) < LOGITS_TOL, i
    for li in range(cfg["n_layers"]):
        kb, vb = d_batch.kv_ptrs(li)
        ks, vs = d_seq.kv_ptrs(li)
        kvd = cfg["n_kv_heads"] * cfg["head_dim"]
        n = (ctx + m) * kvd * 4
        hb, hs = _read_dev(kb, n).view(np.float32), _read_dev(ks, n).view(np.float32)
        assert np.array_equal(hb[:ctx * kvd], hs[:ctx * kvd]), li  # rows before the batch untouched
        assert rel_l2(hb, hs) < 2e-4, li
        assert rel_l2(_read_dev(vb, n).view(np.float32), _read_dev(vs, n).view(np.float32)) < 2e-4, li
    d_batch.close()
    d_seq.close()


def _read_dev(ptr: int, nbytes: int) -> np.ndarray:
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    out = np.empty(nbytes, np.uint8)
    assert hip.hipMemcpy(C.c_void_p(out.ctypes.data), C.c_void_p(ptr), C.c_size_t(nbytes), 2) == 0
    return out


def test_batch_graph_replay_and_eager(rt, orc):
    """Two batches in a row reuse the captured graph for their M; the eager
    launch order gives the same logits bit for bit."""
    cfg = tiny(4)
    max_seq, ctx = 40, 6
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=444)
    d_g = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    d_e = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    d_e.set_graph(False)
    a1 = d_g.decode_step_batch([1, 2, 3], ctx)
    a2 = d_g.decode_step_batch([4, 5, 6], ctx + 3)
    b1 = d_e.decode_step_batch([1, 2, 3], ctx)
    b2 = d_e.decode_step_batch([4, 5, 6], ctx + 3)
    assert np.array_equal(a1, b1) and np.array_equal(a2, b2)
    # a single step after the batches continues the same cache
    s1 = d_g.decode_step(9, ctx + 6)
    s2 = d_e.decode_step(9, ctx + 6)
    assert np.array_equal(s1, s2)
    d_g.close()
    d_e.close()


def test_batch_rejects_bad_calls(rt, orc):
    cfg = tiny(2)
    layers, embed, fnorm = make_model(orc, cfg, max_seq=16, ctx=4, seed=5)
    d = build_ctx(rt, cfg, layers, embed, fnorm, 4, 16)
    for toks, start in (([], 4), ([1] * 9, 4), ([1, 2], 15), ([1, cfg["vocab"]], 4), ([1], -1)):
        with pytest.raises(rt.RtError):
            d.decode_step_batch(toks, start)
    d.close()


def test_gemma3_4b_shape_batch_matches_sequential(rt, orc, dev):
    """The batched path at the full Gemma-3-4B shape (34 layers, vocab
    262144, ctx 1024): three tokens against three single steps (whose path
    the oracle test above checks); the two GEMV paths differ only in their
    activation digits."""
    cfg = dict(rt.GEMMA3_4B)
    ctx = 1024
    max_seq = ctx + 8
    H, F, D = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QD, KVD = cfg["n_q_heads"] * D, cfg["n_kv_heads"] * D
    layers = []
    s = 12000
    for _ in range(cfg["n_layers"]):
        L = {}
        for name, (rows, cols) in dict(q=(QD, H), k=(KVD, H), v=(KVD, H), o=(H, QD), gate=(F, H), up=(F, H),
                                       down=(H, F)).items():
            s += 1
            L[name] = orc.synth_q4k(s, rows, cols)
        for name, n in dict(in_norm=H, post_attn_norm=H, pre_ffn_norm=H, post_ffn_norm=H, q_norm=D,
                            k_norm=D).items():
            s += 1
            L[name] = orc.synth_normal(s, n, 0.0, 0.1)
        s += 1
        kc = np.zeros((max_seq, KVD), np.float32)
        kc[:ctx] = orc.synth_normal(s, ctx * KVD).reshape(ctx, KVD)
        s += 1
        vc = np.zeros((max_seq, KVD), np.float32)
        vc[:ctx] = orc.synth_normal(s, ctx * KVD).reshape(ctx, KVD)
        L["k_cache"], L["v_cache"] = kc, vc
        layers.append(L)
    embed = orc.synth_bf16(9888, cfg["vocab"] * H, 0.02)
    fnorm = orc.synth_normal(9887, H, 0.0, 0.1)
    toks = [11, 222, 3333]
    d_b = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    got = d_b.decode_step_batch(toks, ctx)
    d_b.close()
    d_s = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    for i, t in enumerate(toks):
        ref = d_s.decode_step(t, ctx + i)
        err = rel_l2(got[i], ref)
        print(f"gemma3-4b batch token {i}: rel-L2 vs single step {err:.2e}")
        assert err < 1e-3
        assert int(np.argmax(got[i])) == int(np.argmax(ref))
    d_s.close()


def test_failed_set_unsets_layer_and_embed(rt, orc):
    """A re-set that fails (a null norm pointer, a null final norm) is refused
    before anything is uploaded and leaves that layer (embedding) unset: the
    next step answers RT_ESTATE instead of running a graph over freed
    weights.  Setting it again restores the step bit for bit."""
    import ctypes as C
    cfg = tiny(2)
    max_seq, pos = 32, 6
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=pos, seed=31)
    d = build_ctx(rt, cfg, layers, embed, fnorm, pos, max_seq)
    first = d.decode_step(9, pos)
    L = rt.lib()
    out = np.empty(cfg["vocab"], np.float32)
    fields = {k: (0 if k == "q_norm" else rt._addr(layers[1][k])) for k, _ in rt.Gemma3Layer._fields_}
    bad = rt.Gemma3Layer(**fields)
    fmts = (C.c_int32 * 7)(*([rt.LINEAR_Q4K] * 7))
    assert L.rt_decode_set_layer_formats(d._h, 1, C.byref(bad), fmts, 0) == rt.RT_EINVAL
    assert "q_norm is null" in L.rt_last_error().decode()
    assert L.rt_decode_step(d._h, 9, pos, out.ctypes.data) == rt.RT_ESTATE
    d.set_layer(1, layers[1])
    assert np.array_equal(d.decode_step(9, pos), first)
    assert L.rt_decode_set_embed(d._h, rt._addr(embed), None, 0) == rt.RT_EINVAL
    assert L.rt_decode_step(d._h, 9, pos, out.ctypes.data) == rt.RT_ESTATE
    d.set_embed(embed, fnorm)
    assert np.array_equal(d.decode_step(9, pos), first)
    d.close()


# ---------------------------------------------------------------------------
# Shapes outside the fused kernels' templates: every step runs as a one-row
# pass of the rows kernels (batched GEMV, row attention, batched lm_head).
# ---------------------------------------------------------------------------
def generic_cfg(**kw):
    """hidden 768, 4 heads x 128 over 2 KV heads, ffn 1536: no fused template."""
    base = dict(hidden=768, ffn=1536, n_q_heads=4, n_kv_heads=2, head_dim=128, attn_scale=1.0 / np.sqrt(128.0))
    base.update(kw)
    return tiny(2, **base)


@pytest.mark.parametrize("pos", [0, 3, 20])
def test_generic_shape_decode_step_matches_oracle(rt, orc, pos):
    cfg = generic_cfg()
    max_seq = 48
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=pos, seed=1500 + pos)
    d = build_ctx(rt, cfg, layers, embed, fnorm, pos, max_seq)
    got = d.decode_step(17, pos)
    ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=17, pos=pos)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    d.close()


def test_generic_shape_steps_batch_and_graph(rt, orc):
    """Consecutive steps replay one captured graph and append K/V rows as the
    oracle does; a verify batch matches single steps; eager equals graph."""
    import copy
    cfg = generic_cfg(n_layers=3, global_every=3)
    max_seq, ctx = 40, 5
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=1600)
    d = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    d_e = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    d_e.set_graph(False)
    olayers = copy.deepcopy(layers)
    for i, tok in enumerate([3, 999, 41, 7]):
        got = d.decode_step(tok, ctx + i)
        assert np.array_equal(got, d_e.decode_step(tok, ctx + i)), i
        ref = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=tok, pos=ctx + i)
        assert rel_l2(got, ref) < LOGITS_TOL, i
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    for li in range(cfg["n_layers"]):
        kp, _ = d.kv_ptrs(li)
        k = _read_dev(kp, (ctx + 4) * kvd * 4).view(np.float32).reshape(ctx + 4, kvd)
        assert rel_l2(k[ctx:], olayers[li]["k_cache"][ctx:ctx + 4]) < 1e-3, li
    toks = [5, 6, 7]
    got = d.decode_step_batch(toks, ctx + 4)
    seq = np.stack([d_e.decode_step(t, ctx + 4 + i) for i, t in enumerate(toks)])
    for i in range(len(toks)):
        assert rel_l2(got[i], seq[i]) < 2e-4, i
    d.close()
    d_e.close()


def test_generic_shape_refusals(rt, orc):
    """A projection format a decode layer cannot hold (F32) is refused; a
    shape that neither kernel set serves is refused at create with both
    reasons."""
    cfg = generic_cfg(n_layers=1, global_every=0)
    layers, embed, fnorm = make_model(orc, cfg, max_seq=16, ctx=0, seed=1700)
    d = rt.HipDecodeContext(cfg, 16)
    H, F = cfg["hidden"], cfg["ffn"]
    w = dict(layers[0], down=np.zeros(H * F, np.float32))
    with pytest.raises(rt.RtError, match="unsupported format"):
        d.set_layer(0, w, formats=[rt.LINEAR_Q4K] * 6 + [rt.LINEAR_F32])
    d.close()
    with pytest.raises(rt.RtError, match="rows kernels"):
        rt.HipDecodeContext(generic_cfg(hidden=5120), 16)


@pytest.mark.gpu
def test_generic_shape_mixed_formats_match_oracle(rt, orc):
    """A rows-kernel shape (hidden 768) with projections in Q6_K, Q8_0 and
    BF16 beside Q4_K (layer 0's q|k|v set in three formats): single steps
    and a verify batch run on the batched GEMV of each format, a 20-row
    prefill on the f16 GEMM of each; all against the oracle.

    The synthetic Q6_K / Q8_0 weights are about 30x larger than the Q4_K
    ones, and some draws of such mixed models amplify rounding a hundredfold
    (a 3e-5 change of the norm gammas moves the oracle's own logits by
    1.7e-3).  This plan and seed keep that response under 1e-4, so the bar
    measures the kernels and not the model's conditioning."""
    import copy
    from test_kquant import apply_formats
    from test_prefill import assert_kv_rows, fresh_caches
    cfg = generic_cfg(n_layers=3, global_every=3)
    max_seq, ctx = 48, 6
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=1810)
    plan = {0: dict(q=5, v=2, down=4), 1: dict(gate=2, o=5, k=4), 2: dict(up=5, down=2, v=4)}
    dev_layers, fmts = apply_formats(orc, cfg, layers, plan, seed=1811)
    d = rt.HipDecodeContext(cfg, max_seq)
    for i, (D, f) in enumerate(zip(dev_layers, fmts)):
        d.set_layer(i, D, formats=f)
        d.sync_kv_from_cpu(i, np.ascontiguousarray(layers[i]["k_cache"][:ctx]),
                           np.ascontiguousarray(layers[i]["v_cache"][:ctx]), ctx)
    d.set_embed(embed, fnorm)
    assert d.verify_batched
    olayers = copy.deepcopy(layers)
    for i, tok in enumerate([3, 999]):
        got = d.decode_step(tok, ctx + i)
        ref = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=tok, pos=ctx + i)
        assert rel_l2(got, ref) < LOGITS_TOL, (i, rel_l2(got, ref))
    toks = [5, 6, 7]
    got = d.decode_step_batch(toks, ctx + 2)
    for i, t in enumerate(toks):
        ref = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=t, pos=ctx + 2 + i)
        assert rel_l2(got[i], ref) < LOGITS_TOL, (i, rel_l2(got[i], ref))
    d.close()
    # prefill of 20 rows (GEMM) in chunks of 7 (batched GEMVs), sliding rule
    T = 20
    d = rt.HipDecodeContext(cfg, max_seq)
    for i, (D, f) in enumerate(zip(dev_layers, fmts)):
        d.set_layer(i, D, formats=f)
    d.set_embed(embed, fnorm)
    d.set_prefill_chunk(7)
    ptoks = [(13 * i + 5) % cfg["vocab"] for i in range(T)]
    got = d.prefill(ptoks, 0, 1)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, ptoks, 0, 1)
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    assert_kv_rows(d, cfg, layers, embed, fnorm, ptoks, 1, False, ref_layers)
    d.close()


def gemma3_1b_cfg(**kw):
    """The reference's gemma3_1b preset widths (transformer4.rs:84-104):
    hidden 1152 (18 chunks of 64, not whole Q4_K super-blocks), 4 q heads
    and 1 KV head of 256, FFN 6912, sliding window 512; few layers, a small
    vocabulary."""
    base = dict(hidden=1152, ffn=6912, n_q_heads=4, n_kv_heads=1, head_dim=256, n_layers=3, vocab=1024,
                sliding_window=512, global_every=3, rope_theta_local=10000.0, rope_theta_global=1000000.0,
                rope_fs_local=1.0, rope_fs_global=0.125, eps=1e-6, attn_scale=1.0 / 16.0)
    base.update(kw)
    return base


def gemma3_1b_model(rt, orc, cfg, max_seq, ctx, seed):
    """A model at those widths: the projections that read the hidden width
    (q, k, v, gate, up) in Q8_0 or BF16 per layer, o in Q4_K, down in Q6_K;
    returns the oracle's layers, the device layers and their formats."""
    from test_kquant import synth_q6k, synth_q8_0
    H, F, D = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QD, KVD = cfg["n_q_heads"] * D, cfg["n_kv_heads"] * D
    rng = np.random.default_rng(seed)
    shapes = dict(q=(QD, H), k=(KVD, H), v=(KVD, H), o=(H, QD), gate=(F, H), up=(F, H), down=(H, F))
    layers, dev_layers, fmts = [], [], []
    s = seed
    for li in range(cfg["n_layers"]):
        L, Dl, fmt = {}, {}, {}
        wide = 5 if li % 2 == 0 else 2  # Q8_0 / BF16 for the hidden-width rows
        for name, (rows, cols) in shapes.items():
            s += 1
            f = 1 if name == "o" else 4 if name == "down" else wide
            if name == "k" and li == 1:
                f = 5  # a k in Q8_0 beside BF16 q and v: one set, two formats
            fmt[name] = f
            if f == 1:
                L[name] = Dl[name] = orc.synth_q4k(s, rows, cols)
            elif f == 4:
                L[name] = synth_q6k(rng, rows * cols // 256)
                Dl[name] = rt.q6k_repack(L[name])
            elif f == 5:
                L[name] = synth_q8_0(rng, rows * cols // 32)
                Dl[name] = rt.q8_0_repack(L[name])
            else:
                L[name] = Dl[name] = orc.synth_bf16(s, rows * cols)
        for name, n in dict(in_norm=H, post_attn_norm=H, pre_ffn_norm=H, post_ffn_norm=H, q_norm=D,
                            k_norm=D).items():
            s += 1
            L[name] = Dl[name] = orc.synth_normal(s, n, 0.0, 0.1)
        kc = np.zeros((max_seq, KVD), np.float32)
        vc = np.zeros((max_seq, KVD), np.float32)
        kc[:ctx] = orc.synth_normal(s + 1, ctx * KVD).reshape(ctx, KVD)
        vc[:ctx] = orc.synth_normal(s + 2, ctx * KVD).reshape(ctx, KVD)
        s += 2
        L["k_cache"], L["v_cache"], L["fmt"] = kc, vc, fmt
        layers.append(L)
        dev_layers.append(Dl)
        fmts.append([fmt[p] for p in ("q", "k", "v", "o", "gate", "up", "down")])
    embed = orc.synth_bf16(seed + 9999, cfg["vocab"] * H)
    final_norm = orc.synth_normal(seed + 9998, H, 0.0, 0.1)
    return layers, dev_layers, fmts, embed, final_norm


def gemma3_1b_ctx(rt, cfg, layers, dev_layers, fmts, embed, fnorm, ctx, max_seq):
    d = rt.HipDecodeContext(cfg, max_seq)
    for i, (D, f) in enumerate(zip(dev_layers, fmts)):
        d.set_layer(i, D, formats=f)
        if ctx:
            d.sync_kv_from_cpu(i, np.ascontiguousarray(layers[i]["k_cache"][:ctx]),
                               np.ascontiguousarray(layers[i]["v_cache"][:ctx]), ctx)
    d.set_embed(embed, fnorm)
    return d


@pytest.mark.parametrize("pos", [0, 3, 20])
def test_gemma3_1b_shape_decode_matches_oracle(rt, orc, pos):
    """The gemma3_1b preset's widths on the rows kernels (MetalDecodeContext::
    new takes any Config4, metal_decode.rs:971-1277): a decode step, the next
    step, and a verify batch of 3 against the oracle."""
    import copy
    cfg = gemma3_1b_cfg()
    max_seq = 40
    layers, dev_layers, fmts, embed, fnorm = gemma3_1b_model(rt, orc, cfg, max_seq, pos, seed=1900 + pos)
    d = gemma3_1b_ctx(rt, cfg, layers, dev_layers, fmts, embed, fnorm, pos, max_seq)
    assert d.verify_batched
    olayers = copy.deepcopy(layers)
    for i, tok in enumerate((17, 250)):
        got = d.decode_step(tok, pos + i)
        ref = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=tok, pos=pos + i)
        assert np.all(np.isfinite(got))
        assert rel_l2(got, ref) < LOGITS_TOL, (i, rel_l2(got, ref))
    toks = [5, 6, 700]
    got = d.decode_step_batch(toks, pos + 2)
    for i, t in enumerate(toks):
        ref = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=t, pos=pos + 2 + i)
        assert rel_l2(got[i], ref) < LOGITS_TOL, (i, rel_l2(got[i], ref))
    d.close()


@pytest.mark.parametrize("T,mode,chunk", [(20, 1, 0), (20, 0, 0), (13, 1, 5)])
def test_gemma3_1b_shape_prefill_matches_oracle(rt, orc, T, mode, chunk):
    """Prefill at the gemma3_1b widths (the f16 GEMM of each format; chunks of
    5 rows on the batched GEMVs) against the oracle, and the next step."""
    from test_prefill import assert_kv_rows, fresh_caches
    cfg = gemma3_1b_cfg(sliding_window=8)
    max_seq = 32
    layers, dev_layers, fmts, embed, fnorm = gemma3_1b_model(rt, orc, cfg, max_seq, 0, seed=1950 + T)
    d = gemma3_1b_ctx(rt, cfg, layers, dev_layers, fmts, embed, fnorm, 0, max_seq)
    if chunk:
        d.set_prefill_chunk(chunk)
    toks = [(31 * i + 2) % cfg["vocab"] for i in range(T)]
    got = d.prefill(toks, 0, mode)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    assert_kv_rows(d, cfg, layers, embed, fnorm, toks, mode, (chunk or T) > 8, ref_layers)
    if mode == 1:
        nxt = d.decode_step(9, T)
        rstep = orc.gemma3_decode_step(cfg, ref_layers, embed, fnorm, token=9, pos=T)
        assert rel_l2(nxt, rstep) < LOGITS_TOL
    d.close()


def test_gemma3_1b_shape_refuses_q4k_at_hidden_width(rt, orc):
    """Q4_K rows are whole super-blocks: a q projection of 1152 columns in
    Q4_K is refused (real gemma-3-1b files quantise those tensors with other
    types)."""
    cfg = gemma3_1b_cfg(n_layers=1, global_every=0)
    layers, dev_layers, fmts, embed, fnorm = gemma3_1b_model(rt, orc, cfg, 8, 0, seed=1990)
    d = rt.HipDecodeContext(cfg, 8)
    with pytest.raises(rt.RtError, match="unsupported format"):
        d.set_layer(0, dev_layers[0], formats=[1] + fmts[0][1:])
    d.close()


# ---------------------------------------------------------------------------
# An lm_head apart from the embedding (metal_decode.rs:1079-1107): Q4_K (the
# model's own or the BF16 one requantised, feature q4k-lm-head) or untied BF16
# ---------------------------------------------------------------------------
def lm_head_ref(orc, cfg, fmt, w, hidden, fnorm):
    """Logits of the final-normed hidden state (final_norm, transformer4.rs:
    2370-2380, in float64) through the head: Q4_K dot_row in float64
    (orc_q4k_gemv_f64) or the BF16 GEMV in float64."""
    h = hidden.astype(np.float64)
    xn = h / np.sqrt(np.mean(h * h) + cfg["eps"]) * (1.0 + fnorm.astype(np.float64))
    if fmt == 1:
        return orc.q4k_gemv_f64(w, cfg["vocab"], cfg["hidden"], xn.astype(np.float32))
    W = (w.astype(np.uint32) << 16).view(np.float32).reshape(cfg["vocab"], cfg["hidden"])
    return W.astype(np.float64) @ xn


def check_head(rt, orc, cfg, fmt, head, d, layers, embed, fnorm, ctx, m):
    """Steps at ctx, ctx+1 and a verify batch of m at ctx+2 through the head,
    against the oracle's hidden state times the head."""
    import copy
    olayers = copy.deepcopy(layers)
    for i, t in enumerate([7, 9]):
        got = d.decode_step(t, ctx + i)
        _, hid = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=t, pos=ctx + i, want_hidden=True)
        ref = lm_head_ref(orc, cfg, fmt, head, hid, fnorm)
        assert rel_l2(got, ref) < LOGITS_TOL, (i, rel_l2(got, ref))
        assert int(np.argmax(got)) == int(np.argmax(ref))
    toks = [(37 * i + 5) % cfg["vocab"] for i in range(m)]
    got = d.decode_step_batch(toks, ctx + 2)
    for i, t in enumerate(toks):
        _, hid = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=t, pos=ctx + 2 + i, want_hidden=True)
        ref = lm_head_ref(orc, cfg, fmt, head, hid, fnorm)
        assert rel_l2(got[i], ref) < LOGITS_TOL, (i, rel_l2(got[i], ref))
        assert int(np.argmax(got[i])) == int(np.argmax(ref))


@pytest.mark.parametrize("fmt", [1, 2])
def test_lm_head_apart_from_embedding(rt, orc, fmt):
    """A Q4_K lm_head (the embedding requantised by quantize_from_bf16, as
    the q4k-lm-head feature does) or an untied BF16 one: two decode steps, a
    verify batch of 3 and a prefill's last row against the oracle's final
    hidden state times the head; w = None restores the tied logits bit for
    bit."""
    from test_prefill import fresh_caches
    cfg = tiny(2)
    max_seq, ctx = 40, 6
    H, V = cfg["hidden"], cfg["vocab"]
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=2100 + fmt)
    head = rt.q4k_quantize_bf16(embed.reshape(V, H)) if fmt == 1 else orc.synth_bf16(2200, V * H)
    d = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    tied = d.decode_step(7, ctx)
    d.set_lm_head(fmt, head)
    check_head(rt, orc, cfg, fmt, head, d, layers, embed, fnorm, ctx, 3)
    d.set_lm_head(0, None)
    assert np.array_equal(d.decode_step(7, ctx), tied)
    d.close()
    # prefill (12 rows: the GEMM path) and its last row's logits
    d = build_ctx(rt, cfg, layers, embed, fnorm, 0, max_seq)
    d.set_lm_head(fmt, head)
    toks = [(13 * i + 2) % V for i in range(12)]
    got = d.prefill(toks, 0, 1)
    olayers = fresh_caches(layers)
    for i, t in enumerate(toks):
        _, hid = orc.gemma3_decode_step(cfg, olayers, embed, fnorm, token=t, pos=i, want_hidden=True)
    ref = lm_head_ref(orc, cfg, fmt, head, hid, fnorm)
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    d.close()


def test_gemma3_4b_shape_q4k_lm_head(rt, orc):
    """The Q4_K lm_head at Gemma-3-4B widths (K = 2560: the single-token
    GEMV and the one-slice batched GEMV over the vocabulary rows), 2 layers,
    vocab 4096: steps and a verify batch of 8 against the oracle; a head
    bound by device pointer gives the same logits."""
    import torch
    cfg = dict(rt.GEMMA3_4B, n_layers=2, global_every=2, vocab=4096)
    H, V = cfg["hidden"], cfg["vocab"]
    max_seq, ctx = 64, 40
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=2300)
    head = rt.q4k_quantize_bf16(embed.reshape(V, H))
    d = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    d.set_lm_head(1, head)
    check_head(rt, orc, cfg, 1, head, d, layers, embed, fnorm, ctx, 8)
    first = d.decode_step(7, ctx)
    d.set_lm_head(1, torch.from_numpy(head).to("cuda:0"))
    assert np.array_equal(d.decode_step(7, ctx), first)
    d.close()


def test_generic_shape_q4k_lm_head(rt, orc):
    """A Q4_K lm_head at hidden 768 (three super-blocks per row: the batched
    head splits K and adds the partials; the rows path serves even the
    single token): steps and a verify batch of 5 against the oracle."""
    cfg = generic_cfg()
    H, V = cfg["hidden"], cfg["vocab"]
    max_seq, ctx = 32, 6
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=2500)
    head = rt.q4k_quantize_bf16(embed.reshape(V, H))
    d = build_ctx(rt, cfg, layers, embed, fnorm, ctx, max_seq)
    d.set_lm_head(1, head)
    check_head(rt, orc, cfg, 1, head, d, layers, embed, fnorm, ctx, 5)
    d.close()


def test_lm_head_rejects_bad_calls(rt, orc):
    import ctypes as C
    cfg = gemma3_1b_cfg(n_layers=1, global_every=0)  # hidden 1152: no Q4_K head
    layers, dev_layers, fmts, embed, fnorm = gemma3_1b_model(rt, orc, cfg, 8, 0, seed=2400)
    d = gemma3_1b_ctx(rt, cfg, layers, dev_layers, fmts, embed, fnorm, 0, 8)
    first = d.decode_step(3, 0)
    L = rt.lib()
    blocks = (C.c_uint8 * 144)()
    assert L.rt_decode_set_lm_head(d._h, rt.LINEAR_Q4K, C.addressof(blocks), 0) == rt.RT_EINVAL
    assert "unsupported" in L.rt_last_error().decode()
    assert L.rt_decode_set_lm_head(d._h, 3, C.addressof(blocks), 0) == rt.RT_EINVAL  # F32
    assert np.array_equal(d.decode_step(3, 0), first)  # the tied head serves on
    d.close()


def test_memory_report(rt, orc):
    """rt_decode_memory (print_metal_memory, metal_decode.rs:1285-1354): the
    weights and KV cache of a context add up to what its shapes hold, for
    uploaded and for device-bound weights; prefill scratch appears after a
    prefill."""
    import torch
    cfg = tiny(2)
    max_seq, pos = 40, 4
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=pos, seed=61)
    H, F, D = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QD, KVD = cfg["n_q_heads"] * D, cfg["n_kv_heads"] * D
    proj = sum(r * (c // 256) * 144 for r, c in ((QD, H), (KVD, H), (KVD, H), (H, QD), (F, H), (F, H), (H, F)))
    # per Q4_K projection also its GEMM row exponents (4 bytes per output row)
    exps = (QD + 2 * KVD + H + 2 * F + H) * 4
    weights = cfg["n_layers"] * (proj + exps + (4 * H + 2 * D) * 4) + cfg["vocab"] * H * 2 + H * 4
    kv = cfg["n_layers"] * 2 * max_seq * KVD * 4
    d = build_ctx(rt, cfg, layers, embed, fnorm, pos, max_seq)
    m = d.memory()
    assert m["weights"] == weights and m["kv_cache"] == kv and m["prefill"] == 0
    assert m["activation"] > 0 and m["batch"] > 0
    assert m["total"] == sum(m[k] for k in ("weights", "kv_cache", "activation", "batch", "prefill"))
    d.prefill([1, 2, 3], 0, 1)
    assert d.memory()["prefill"] > 0
    d.print_memory()
    d.close()
    # the same weights bound by device pointer
    dev = torch.device("cuda:0")
    dl = [{k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in L.items() if k not in ("k_cache", "v_cache")}
          for L in layers]
    d2 = rt.HipDecodeContext(cfg, max_seq)
    for i, L in enumerate(dl):
        d2.set_layer(i, L)
    d2.set_embed(torch.from_numpy(embed).to(dev), torch.from_numpy(fnorm).to(dev))
    assert d2.memory()["weights"] == weights
    d2.close()


def test_gelu_tanh_matches_oracle(rt, orc):
    """The device gelu_tanh against the oracle's (glibc tanhf, as Rust's f32
    tanh): identical wherever tanh saturates (|x| >= 6, where the FFN of the
    synthetic models sends most gate values), and elsewhere within the two
    ulps of tanh that separate two libm's, |dy| <= |x| 2^-23 + |y| 2^-23."""
    import torch
    x = np.concatenate([np.linspace(-40, 40, 160_001, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 1e30, -1e30], np.float32)])
    ref = np.array([orc.gelu_tanh(float(v)) for v in x], np.float32)
    y = torch.empty(len(x), device="cuda")
    rt.gelu_tanh(torch.from_numpy(x).cuda(), y)
    got = y.cpu().numpy()
    sat = np.abs(x) >= 6
    assert np.array_equal(got[sat].view(np.int32), ref[sat].view(np.int32))
    tol = (np.abs(x) + np.abs(ref)) * 2.0 ** -23
    assert np.all(np.abs(got - ref) <= tol)
