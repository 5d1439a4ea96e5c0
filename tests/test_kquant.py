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


# ---------------------------------------------------------------------------
# oracle: per-format projections (CPU)
# ---------------------------------------------------------------------------
def test_oracle_proj_gemv_formats(orc):
    """orc_proj_gemv against float64 products of the pinned dequantisers."""
    rng = np.random.default_rng(11)
    rows, cols = 24, 512
    x = rng.standard_normal(cols).astype(np.float32)
    q6 = synth_q6k(rng, rows * cols // 256)
    q8 = synth_q8_0(rng, rows * cols // 32)
    bf = orc.synth_bf16(12, rows * cols)
    q4 = orc.synth_q4k(13, rows, cols)
    cases = [(4, q6, orc.q6k_dequant(q6, rows * cols)), (5, q8, orc.q8_0_dequant(q8, rows * cols)),
             (2, bf, (bf.astype(np.uint32) << 16).view(np.float32)),
             (1, q4, orc.q4k_dequant(q4, rows, cols).reshape(-1))]
    for fmt, w, deq in cases:
        y = orc.proj_gemv(fmt, w, rows, cols, x)
        ref = deq.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
        assert rel_l2(y, ref) < 1e-6, fmt


def test_oracle_proj_matmul_formats(orc):
    """orc_proj_matmul (the prefill GEMM of each format) against float64
    products of the pinned dequantisers; row by row it equals orc_proj_gemv
    (Q4_K: orc_q4k_matmul, the GEMV keeps the reference's blocked order)."""
    rng = np.random.default_rng(12)
    m, rows, cols = 3, 20, 512
    a = rng.standard_normal((m, cols)).astype(np.float32)
    q6 = synth_q6k(rng, rows * cols // 256)
    q8 = synth_q8_0(rng, rows * cols // 32)
    bf = orc.synth_bf16(14, rows * cols)
    q4 = orc.synth_q4k(15, rows, cols)
    cases = [(4, q6, orc.q6k_dequant(q6, rows * cols)), (5, q8, orc.q8_0_dequant(q8, rows * cols)),
             (2, bf, (bf.astype(np.uint32) << 16).view(np.float32)),
             (1, q4, orc.q4k_dequant(q4, rows, cols).reshape(-1))]
    for fmt, w, deq in cases:
        c = orc.proj_matmul(fmt, a, w, rows, cols)
        ref = a.astype(np.float64) @ deq.reshape(rows, cols).astype(np.float64).T
        assert rel_l2(c, ref) < 1e-6, fmt
        if fmt == 1:
            assert np.array_equal(c, orc.q4k_matmul(a, w, rows, cols))
            continue
        for i in range(m):
            assert np.array_equal(c[i], orc.proj_gemv(fmt, w, rows, cols, a[i])), fmt


# ---------------------------------------------------------------------------
# decode step with per-projection formats (GPU)
# ---------------------------------------------------------------------------
SHAPES = lambda cfg: dict(  # noqa: E731
    q=(cfg["n_q_heads"] * cfg["head_dim"], cfg["hidden"]), k=(cfg["n_kv_heads"] * cfg["head_dim"], cfg["hidden"]),
    v=(cfg["n_kv_heads"] * cfg["head_dim"], cfg["hidden"]), o=(cfg["hidden"], cfg["n_q_heads"] * cfg["head_dim"]),
    gate=(cfg["ffn"], cfg["hidden"]), up=(cfg["ffn"], cfg["hidden"]), down=(cfg["hidden"], cfg["ffn"]))


def apply_formats(orc, cfg, layers, plan, seed):
    """Replace projections by Q6_K / Q8_0 (GGUF block bytes) or BF16 weights;
    returns the device-side dicts (planar layouts) and their format lists."""
    rng = np.random.default_rng(seed)
    shapes = SHAPES(cfg)
    dev_layers, fmts = [], []
    for li, L in enumerate(layers):
        plan_l = plan.get(li, {})
        L["fmt"] = dict(plan_l)
        D = dict(L)
        for p, fmt in plan_l.items():
            rows, cols = shapes[p]
            if fmt == 4:
                L[p] = synth_q6k(rng, rows * cols // 256)
                D[p] = __import__("conftest").load_pkg().q6k_repack(L[p])
            elif fmt == 5:
                L[p] = synth_q8_0(rng, rows * cols // 32)
                D[p] = __import__("conftest").load_pkg().q8_0_repack(L[p])
            else:
                L[p] = orc.synth_bf16(seed + li * 10 + len(p), rows * cols)
                D[p] = L[p]
        dev_layers.append(D)
        fmts.append([plan_l.get(p, 1) for p in ("q", "k", "v", "o", "gate", "up", "down")])
    return dev_layers, fmts


MIXED_PLAN = {0: dict(v=4, down=4), 2: dict(q=5, o=4, gate=2), 3: dict(k=4, up=5), 4: dict(v=2, down=5),
              5: dict(q=4, k=4, v=4, o=5, gate=4, up=4, down=2)}


def mixed_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, ctx, max_seq, layers):
    d = rt.HipDecodeContext(cfg, max_seq)
    for i, (D, f) in enumerate(zip(dev_layers, fmts)):
        d.set_layer(i, D, formats=f)
        d.sync_kv_from_cpu(i, np.ascontiguousarray(layers[i]["k_cache"][:ctx]),
                           np.ascontiguousarray(layers[i]["v_cache"][:ctx]), ctx)
    d.set_embed(embed, fnorm)
    return d


@pytest.mark.gpu
@pytest.mark.parametrize("pos", [0, 3, 20])
def test_mixed_format_decode_matches_oracle(rt, orc, pos):
    """Q4_K_M-like layers (v, down in Q6_K), a q in Q8_0 (split q/k/v set), a
    gate in BF16 (split gate/up), and a global layer with every projection
    outside Q4_K, against the oracle's exact dequantisation."""
    from test_gpu_decode import tiny
    from test_oracle import make_model
    cfg = tiny(2)
    max_seq = 32
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=pos, seed=7000 + pos)
    dev_layers, fmts = apply_formats(orc, cfg, layers, MIXED_PLAN, seed=7100 + pos)
    d = mixed_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, pos, max_seq, layers)
    got = d.decode_step(11, pos)
    ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=11, pos=pos)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < 1e-3, rel_l2(got, ref)
    # the next steps replay the captured graph; the batch path runs the same layers
    for i, tok in enumerate((3, 900)):
        got = d.decode_step(tok, pos + 1 + i)
        ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=tok, pos=pos + 1 + i)
        assert rel_l2(got, ref) < 1e-3
    batch = d.decode_step_batch([5, 6, 7], pos + 3)
    for i, tok in enumerate((5, 6, 7)):
        ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=tok, pos=pos + 3 + i)
        assert rel_l2(batch[i], ref) < 1e-3, (i, rel_l2(batch[i], ref))
    d.close()


@pytest.mark.gpu
def test_q4_k_m_layout_at_gemma3_4b_shape(rt, orc):
    """Gemma-3-4B layer shapes with v and down in Q6_K (the Q4_K_M recipe):
    the specialised Q6_K tiles (K = 2560, 10240) inside the decode graph.  The
    native result is closer to the exact product than the reference's way of
    running Q6_K (widened to BF16 at load, transformer4.rs:1233-1242)."""
    from test_oracle import make_model
    cfg = dict(rt.GEMMA3_4B, n_layers=2, global_every=2, vocab=4096)
    ctx, max_seq = 40, 64
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=7300)
    plan = {0: dict(v=4, down=4), 1: dict(v=4, down=4)}
    dev_layers, fmts = apply_formats(orc, cfg, layers, plan, seed=7301)
    d = mixed_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, ctx, max_seq, layers)
    got = d.decode_step(17, ctx)
    import copy
    widened = copy.deepcopy(layers)
    shapes = SHAPES(cfg)
    for L in widened:
        for p in ("v", "down"):
            rows, cols = shapes[p]
            bits = orc.q6k_dequant(L[p], rows * cols).view(np.uint32).astype(np.uint64)
            L[p] = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)  # f32 -> bf16, RNE
            L["fmt"][p] = 2
    ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=17, pos=ctx)
    ref_bf16 = orc.gemma3_decode_step(cfg, widened, embed, fnorm, token=17, pos=ctx)
    assert rel_l2(got, ref) < 1e-3, rel_l2(got, ref)
    assert rel_l2(got, ref) < rel_l2(ref_bf16, ref)
    d.close()


@pytest.mark.gpu
@pytest.mark.parametrize("m", [3, 8])
def test_q4_k_m_layout_verify_batch_at_gemma3_4b_shape(rt, orc, m):
    """decode_step_batch (metal_decode.rs:2079-2179) at Gemma-3-4B layer shapes
    with v and down in Q6_K and one layer's q in Q8_0 and gate in BF16: the M
    tokens go through each layer together on the batched GEMV of each format
    (encode_layer_batch sends BF16 projections to gemv_bf16_t_batch,
    2225-2239), against M consecutive oracle decode steps."""
    import copy
    from test_oracle import make_model
    cfg = dict(rt.GEMMA3_4B, n_layers=2, global_every=2, vocab=4096)
    ctx, max_seq = 40, 64
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=7310 + m)
    plan = {0: dict(v=4, down=4, q=5), 1: dict(v=4, down=4, gate=2)}
    dev_layers, fmts = apply_formats(orc, cfg, layers, plan, seed=7311 + m)
    d = mixed_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, ctx, max_seq, layers)
    assert d.verify_batched
    toks = [(311 * i + 7) % cfg["vocab"] for i in range(m)]
    got = d.decode_step_batch(toks, ctx)
    ref_layers = copy.deepcopy(layers)
    for i, t in enumerate(toks):
        ref = orc.gemma3_decode_step(cfg, ref_layers, embed, fnorm, token=t, pos=ctx + i)
        err = rel_l2(got[i], ref)
        print(f"Q4_K_M verify batch m={m} token {i}: logits rel-L2 {err:.2e}", flush=True)
        assert err < 1e-3, (i, err)
    d.close()


# ---------------------------------------------------------------------------
# prefill with per-projection formats
# ---------------------------------------------------------------------------
PROJS = ("q", "k", "v", "o", "gate", "up", "down")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", [5, 2])
@pytest.mark.parametrize("shape", ["tiny", "gemma3_4b"])
def test_uniform_format_model_fused_decode_matches_oracle(rt, orc, shape, fmt):
    """Every projection in Q8_0 (a Q8_0 file) or in BF16 (a BF16 file): q|k|v
    and gate|up run as the fused launches of that format beside their
    prologues (k_qkv8 / k_gateup8, k_qkv16 / k_gateup16; the tiny and the
    Gemma-3-4B widths), o and down as GEMVs of the format.  Steps at three
    positions (the first eager, the others graph replays) and a verify batch
    against the oracle's exact dequantisation."""
    from test_gpu_decode import tiny
    from test_oracle import make_model
    if shape == "tiny":
        cfg, ctx, max_seq = tiny(2), 6, 32
    else:
        cfg, ctx, max_seq = dict(rt.GEMMA3_4B, n_layers=2, global_every=2, vocab=4096), 40, 64
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=ctx, seed=7700 + ctx + fmt)
    plan = {li: {p: fmt for p in PROJS} for li in range(cfg["n_layers"])}
    dev_layers, fmts = apply_formats(orc, cfg, layers, plan, seed=7701 + ctx + fmt)
    d = mixed_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, ctx, max_seq, layers)
    for i, tok in enumerate((11, 3, 900)):
        got = d.decode_step(tok, ctx + i)
        ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=tok, pos=ctx + i)
        assert np.all(np.isfinite(got))
        assert rel_l2(got, ref) < 1e-3, (i, rel_l2(got, ref))
    batch = d.decode_step_batch([5, 6, 7], ctx + 3)
    for i, tok in enumerate((5, 6, 7)):
        ref = orc.gemma3_decode_step(cfg, layers, embed, fnorm, token=tok, pos=ctx + 3 + i)
        assert rel_l2(batch[i], ref) < 1e-3, (i, rel_l2(batch[i], ref))
    d.close()


def test_oracle_mixed_prefill_equals_decode_steps(orc):
    """Per-row sliding window: the oracle prefill of a model with projections
    in every format is T decode steps of the decode-step oracle (whose
    per-format GEMV is pinned above)."""
    from test_gpu_decode import tiny
    from test_oracle import make_model
    from test_prefill import fresh_caches
    cfg = tiny(2)
    T = 12
    layers, embed, fnorm = make_model(orc, cfg, max_seq=T, ctx=0, seed=7350)
    apply_formats(orc, cfg, layers, MIXED_PLAN, seed=7351)
    toks = [(5 * i + 1) % cfg["vocab"] for i in range(T)]
    a = fresh_caches(layers)
    got = orc.gemma3_prefill(cfg, a, embed, fnorm, toks, 0, mode=1)
    b = fresh_caches(layers)
    for i, t in enumerate(toks):
        ref = orc.gemma3_decode_step(cfg, b, embed, fnorm, token=t, pos=i)
    assert rel_l2(got, ref) < 2e-5
    for La, Lb in zip(a, b):
        assert rel_l2(La["k_cache"], Lb["k_cache"]) < 2e-5
        assert rel_l2(La["v_cache"], Lb["v_cache"]) < 2e-5


# partial 256-row/column tiles, K of one to five stages of 64 and long K, and
# tile grids with a multiple of 8 tiles (the per-XCD tile order) and without
GEMM_CASES = [(4, 1, 256, 512), (4, 77, 300, 2560), (5, 130, 200, 192), (5, 8, 1000, 1024), (2, 5, 129, 64),
              (2, 200, 384, 2048), (1, 33, 256, 512), (2, 512, 1024, 256), (5, 1100, 520, 320),
              (4, 600, 2048, 1024), (2, 300, 260, 128),
              (2, 300, 512, 4096), (4, 64, 2560, 10240)]  # split-K (8 and 20 slices)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,m,n,k", GEMM_CASES)
def test_linear_gemm_matches_float64(rt, orc, dev, fmt, m, n, k):
    """rt_linear_gemm_f32 against the float64 product of the exactly
    dequantised weights; shapes with partial 128-row and 128-column tiles."""
    import torch
    rng = np.random.default_rng(100 + fmt * 7 + m)
    a = rng.standard_normal((m, k)).astype(np.float32)
    if fmt == 4:
        src = synth_q6k(rng, n * k // 256)
        w, deq = rt.q6k_repack(src), orc.q6k_dequant(src, n * k)
    elif fmt == 5:
        src = synth_q8_0(rng, n * k // 32)
        w, deq = rt.q8_0_repack(src), orc.q8_0_dequant(src, n * k)
    elif fmt == 2:
        w = orc.synth_bf16(200 + m, n * k)
        deq = (w.astype(np.uint32) << 16).view(np.float32)
    else:
        w = orc.synth_q4k(300 + m, n, k)
        deq = orc.q4k_dequant(w, n, k).reshape(-1)
    c = torch.empty((m, n), dtype=torch.float32, device=dev)
    rt.linear_gemm_f32(fmt, to_dev(w, dev), to_dev(a, dev), c, m, n, k)
    torch.cuda.synchronize()
    ref = a.astype(np.float64) @ deq.reshape(n, k).astype(np.float64).T
    got = c.cpu().numpy()
    assert np.all(np.isfinite(got))
    # f16 operands (11-bit significands) with f32 accumulation: ~2e-4
    assert rel_l2(got, ref) < 1e-3, rel_l2(got, ref)


def test_linear_gemm_rejects_bad_shapes(rt):
    with pytest.raises(rt.RtError):
        rt.linear_gemm_f32(3, 16, 16, 16, 1, 1, 258)  # f32 rows are read as 16-byte vectors
    with pytest.raises(rt.RtError):
        rt.linear_gemm_f32(6, 16, 16, 16, 1, 1, 256)  # no such format
    with pytest.raises(rt.RtError):
        rt.linear_gemm_f32(4, 16, 16, 16, 1, 1, 96)  # Q6_K rows are 256-element blocks
    with pytest.raises(rt.RtError):
        rt.linear_gemm_f32(5, 16, 16, 16, 0, 1, 64)
    with pytest.raises(rt.RtError):
        rt.linear_gemm_f32(2, 16, 16, 16, 9, 1, 96)  # above 8 rows K moves in stages of 64
    with pytest.raises(rt.RtError):
        rt.linear_gemm_f32(2, 16, 16, 16, 1, 1, 100)  # eight bf16 weights per load


def plain_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, max_seq):
    d = rt.HipDecodeContext(cfg, max_seq)
    for i, (D, f) in enumerate(zip(dev_layers, fmts)):
        d.set_layer(i, D, formats=f)
    d.set_embed(embed, fnorm)
    return d


@pytest.mark.gpu
@pytest.mark.parametrize("T,mode,chunk", [(3, 1, 0), (20, 0, 0), (30, 1, 7)])
def test_mixed_format_prefill_matches_oracle(rt, orc, T, mode, chunk):
    """Prefill of a model with projections in Q6_K, Q8_0 and BF16 (the GEMM
    on f16-widened rows) against the oracle's prefill; chunks of 7 rows take
    the batched GEMV of each format.  The next decode step reads the
    prefilled cache."""
    from test_gpu_decode import tiny
    from test_oracle import make_model
    from test_prefill import LOGITS_TOL, assert_kv_rows, fresh_caches
    cfg = tiny(2)
    max_seq = 40
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=7400 + T)
    dev_layers, fmts = apply_formats(orc, cfg, layers, MIXED_PLAN, seed=7401 + T)
    d = plain_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, max_seq)
    if chunk:
        d.set_prefill_chunk(chunk)
    toks = [(17 * i + 4) % cfg["vocab"] for i in range(T)]
    got = d.prefill(toks, 0, mode)
    ref_layers = fresh_caches(layers)
    ref = orc.gemma3_prefill(cfg, ref_layers, embed, fnorm, toks, 0, mode)
    assert np.all(np.isfinite(got))
    print(f"mixed-format prefill T={T} mode={mode} chunk={chunk}: logits rel-L2 {rel_l2(got, ref):.2e}", flush=True)
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    assert_kv_rows(d, cfg, layers, embed, fnorm, toks, mode, (chunk or T) > 8, ref_layers)
    if mode == 1:
        nxt = d.decode_step(9, T)
        ref = orc.gemma3_decode_step(cfg, ref_layers, embed, fnorm, token=9, pos=T)
        assert rel_l2(nxt, ref) < LOGITS_TOL
    d.close()


@pytest.mark.gpu
def test_q4_k_m_layout_prefill_at_gemma3_4b_shape(rt, orc):
    """Gemma-3-4B layer shapes with v and down in Q6_K: a 200-token prefill
    equals 200 GPU decode steps (native Q6_K GEMV, pinned to the oracle
    above) in logits and KV rows, and its KV rows match np_prefill(gpu_ops)
    (Q6_K widened to f16 for the GEMM) on every row."""
    from test_gpu_decode import d2h
    from test_oracle import make_model
    from test_prefill import LOGITS_TOL, assert_kv_rows, read_kv
    cfg = dict(rt.GEMMA3_4B, n_layers=2, global_every=2, vocab=4096)
    T, max_seq = 200, 224
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=7500)
    plan = {0: dict(v=4, down=4), 1: dict(v=4, down=4)}
    dev_layers, fmts = apply_formats(orc, cfg, layers, plan, seed=7501)
    toks = [(89 * i + 3) % cfg["vocab"] for i in range(T)]
    d1 = plain_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, max_seq)
    got = d1.prefill(toks, 0, 1)
    d2 = plain_ctx(rt, cfg, dev_layers, fmts, embed, fnorm, max_seq)
    for i, t in enumerate(toks):
        d2.decode_step_async(t, i)
    d2.synchronize()
    ref = d2h(d2.logits_ptr(), cfg["vocab"])
    assert rel_l2(got, ref) < LOGITS_TOL, rel_l2(got, ref)
    steps = [dict(zip(("k_cache", "v_cache"), read_kv(d2, cfg, li, T))) for li in range(2)]
    assert_kv_rows(d1, cfg, layers, embed, fnorm, toks, 1, True, agg_layers=steps)
    d1.close()
    d2.close()


def test_gemv_multi_rejects_bad_calls(rt):
    with pytest.raises(rt.RtError):
        rt.q4k_gemv_multi([], [], [], 16, 2560)  # no matrix
    with pytest.raises(rt.RtError):
        rt.q4k_gemv_multi([16] * 5, [16] * 5, [256] * 5, 16, 2560)  # more than four
    with pytest.raises(rt.RtError):
        rt.q4k_gemv_multi([16, 16], [16, 16], [256, 256], 16, 2000)  # K not whole blocks
    with pytest.raises(rt.RtError):
        rt.q4k_gemv_multi([16, 16], [16, 16], [256, 0], 16, 2560)  # empty matrix
