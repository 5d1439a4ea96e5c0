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
    with pytest.raises(rt.RtError):
        d.prefill([1, 2, 3], 0, 0)  # prefill runs Q4_K projections only
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
