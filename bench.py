#!/usr/bin/env python3
"""bench.py -- rich-triplet's Q4_K / BF16 decode hot path on one MI355X.

Step (the `value` workload): every projection GEMV of one
Gemma-3-4B decode token -- 34 layers x {q 2560->2048, k 2560->1024,
v 2560->1024, o 2048->2560, gate/up 2560->10240, down 10240->2560} Q4_K
GEMVs, each layer with its own weights, plus the BF16 lm_head 2560->262144 --
captured in one hipGraph.  3.148 GB of weights per step, far beyond the 256 MB
MALL, so every step streams from HBM.  value = algorithmic bytes / time.

Also measured in the same run and reported next to it:
  decode   -- BASELINE config 3: the full decode step (rt_decode_*) at
              context 4096 with an f32 KV cache, tok/s;
  roofline -- the dominant kernel (the 10240x2560 Q4_K GEMV of gate/up):
              algorithmic bytes per launch / average launch time from HIP
              events around a graph of back-to-back launches;
  gemm     -- BASELINE configs 2 and 4: the Q4_K GEMM (bf16 activations,
              f32 output) on the matrix cores, TFLOP/s and the fraction of
              the 2.5 PFLOP/s dense f16 peak, with a plain f16 library GEMM
              of the same shape timed beside it for reference;
  cpu_baseline -- the C restatement of the reference's x86 CPU path
              (oracle/, "port") on a bounded sample, on this host's cores.

Synthetic data (torch RNG on the GPU): Q4_K blocks with f16 d, dmin =
|N(0,0.02)|, 6-bit scales/mins uniform 0..63, nibbles uniform; BF16 weights
N(0,0.02); activations N(0,1); KV N(0,1).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-decode] [--skip-gemm] [--skip-cpu]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import pathlib
import sys
import time

REPO = pathlib.Path(__file__).resolve().parent
PEAK_HBM_GBS = 8000.0  # MI355X published HBM3E bandwidth
PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16/bf16 matrix peak
# configs 2 (prefill, Gemma-3-4B shapes) and 4 (FLUX-12B transformer shapes): (label, M, N, K)
GEMM_SHAPES = [("config2_gate_up", 512, 10240, 2560), ("config2_down", 512, 2560, 10240),
               ("config4_qkv", 4608, 9216, 3072), ("config4_mlp_up", 4608, 12288, 3072),
               ("config4_mlp_down", 4608, 3072, 12288)]

H, F, QD, KVD, L, V = 2560, 10240, 2048, 1024, 34, 262144
# streaming-read floor candidates (rt_stream_read_cfg kind, grid; grid 0 = by size;
# kinds 2 and 3 load with the nontemporal hint)
READ_CFGS = [(0, 0), (0, 512), (0, 1024), (1, 512), (1, 1024), (1, 2048), (2, 0), (2, 768), (2, 1024), (3, 1024)]
Q4K_SHAPES = [("q", QD, H), ("k", KVD, H), ("v", KVD, H), ("o", H, QD), ("gate", F, H), ("up", F, H),
              ("down", H, F)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_pkg():
    d = REPO / "rich-triplet_amd"
    spec = importlib.util.spec_from_file_location("rich_triplet_amd", d / "__init__.py",
                                                  submodule_search_locations=[str(d)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["rich_triplet_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def prefill_flops(T: int, mode: int, window: int = 1024, global_every: int = 6, nq: int = 8, d: int = 256):
    """Flops a T-token prefill needs: the 7 projections (2*N*K per row) and
    attention (2 flops per q.k product term and per p*v term: 4*d*nq per
    visible key) of every row, except where a row's result cannot reach the
    KV cache or the last row's logits: in mode 0 (the reference's prefill
    window) a local layer's rows r < T - window see no key, so their o
    projection is zero; and the last layer's attention, o projection and FFN
    only feed the last row's logits.  mode 0: local rows r >= T - window see
    r - (T - window) + 1 keys; mode 1: min(r + 1, window) keys."""
    shp = {name: (n, k) for name, n, k in Q4K_SHAPES}
    per_row = {name: 2 * n * k for name, (n, k) in shp.items()}
    qkv = per_row["q"] + per_row["k"] + per_row["v"]
    rest = per_row["gate"] + per_row["up"] + per_row["down"]
    w = min(window, T)
    is_glob = [i % global_every == global_every - 1 for i in range(L)]
    gemm = 0
    for i in range(L - 1):
        o_rows = T if (is_glob[i] or mode == 1) else w
        gemm += T * (qkv + rest) + o_rows * per_row["o"]
    gemm += T * qkv + per_row["o"] + rest  # last layer: K/V rows for every row, the rest for the last row
    glob_keys = T * (T + 1) // 2
    loc_keys = w * (w + 1) // 2 if mode == 0 else sum(min(r + 1, window) for r in range(T))
    attn_keys = sum(glob_keys if is_glob[i] else loc_keys for i in range(L - 1))
    attn_keys += T if is_glob[L - 1] else w  # the last row's keys in the last layer
    return gemm, 4 * d * nq * attn_keys


def q4k_bytes(n: int, k: int) -> int:
    return n * (k // 256) * 144


def gemv_bytes(n: int, k: int, w_bytes: int) -> int:
    """Algorithmic bytes of one GEMV: weights + x (f32) + y (f32)."""
    return w_bytes + 4 * k + 4 * n


def synth_q4k(torch, n: int, k: int, gen) -> "torch.Tensor":
    """Random Q4_K blocks on the GPU, packed like pack_scales (autograd2.rs:1119-1132)."""
    nb = n * k // 256
    dev = "cuda"
    blk = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device=dev, generator=gen)
    dd = (torch.randn(nb, 2, device=dev, generator=gen).abs() * 0.02).half()
    blk[:, 0:4] = dd.view(torch.uint8).view(nb, 4)
    sv = torch.randint(0, 64, (nb, 8), dtype=torch.int32, device=dev, generator=gen)
    mv = torch.randint(0, 64, (nb, 8), dtype=torch.int32, device=dev, generator=gen)
    sc = torch.empty(nb, 12, dtype=torch.int32, device=dev)
    sc[:, 0:4] = (sv[:, 0:4] & 63) | ((sv[:, 4:8] & 0x30) << 2)
    sc[:, 4:8] = (mv[:, 0:4] & 63) | ((mv[:, 4:8] & 0x30) << 2)
    sc[:, 8:12] = (sv[:, 4:8] & 15) | ((mv[:, 4:8] & 15) << 4)
    blk[:, 4:16] = sc.to(torch.uint8)
    return blk.reshape(-1)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-gemm", action="store_true")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the PMC probe: a 256 MiB copy (calibration) and 20 launches of the dominant "
                         "kernel on distinct weights; meant to run under rocprofv3 --pmc")
    ap.add_argument("--decode-profile", action="store_true",
                    help="only run the config-3 decode step (a 256 MiB copy first, as the counter calibration), "
                         "--warmup then --steps tokens; meant to run under rocprofv3")
    ap.add_argument("--prefill-profile", action="store_true",
                    help="only run the 4096-token GPU prefill of the config-3 context, --warmup then --steps "
                         "times; meant to run under rocprofv3")
    ap.add_argument("--gemm-tiles", action="store_true",
                    help="only time the M=512 Q4_K GEMM at 128, 160 and 256 tiles of 128x256 (one per CU): how "
                         "the time per K-chunk grows with the tiles in flight")
    ap.add_argument("--launch-probe", action="store_true",
                    help="only measure the launch floor inside a graph: empty dependent launches, and streaming "
                         "reads of 4-118 MB fitted to a fixed cost per launch plus a rate")
    ap.add_argument("--q4-k-m", action="store_true",
                    help="with --decode-profile: the Q4_K_M layout (v and down in Q6_K)")
    ap.add_argument("--q8-0", action="store_true",
                    help="with --decode-profile: every projection in Q8_0 (planar)")
    ap.add_argument("--bf16-model", action="store_true",
                    help="with --decode-profile: every projection in BF16")
    ap.add_argument("--q4k-lm-head", action="store_true",
                    help="with --decode-profile: a Q4_K lm_head (random blocks) instead of the BF16 tied one")
    ap.add_argument("--decode-timeline", action="store_true",
                    help="per-wave timeline of the last layer of a config-3 decode step and of the lm_head: needs "
                         "the traced library (make -C rich-triplet_amd trace; RT_HIP_LIB=rich-triplet_amd/"
                         "librt_hip_trace.so)")
    ap.add_argument("--shared-weights", action="store_true",
                    help="with --decode-profile: bind every layer to layer 0's projections and norms (53 MB, "
                         "which stays in the 256 MB last-level cache between layers), to see how much of each "
                         "layer kernel's time is HBM traffic")
    ap.add_argument("--verify-rows", type=int, default=0,
                    help="with --decode-profile: run decode_step_batch calls of this many rows (1..8) instead "
                         "of single-token steps")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the hot path is benchmarked on a single "
                                   "MI355X (see DESIGN.md for how it would shard); run with --gpus 1"}))
        return 2

    import torch
    rt = load_pkg()
    rt.lib()  # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    t0 = time.time()

    if args.launch_probe:
        print(json.dumps(launch_probe(rt, torch, dev)))
        return 0
    if args.gemm_tiles:
        print(json.dumps(gemm_tiles_probe(rt, torch, dev, torch.Generator(device=dev).manual_seed(args.seed))))
        return 0

    if args.traffic_probe:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        a.fill_(1)
        torch.cuda.synchronize()
        b.copy_(a)  # calibration: reads and writes exactly 256 MiB
        torch.cuda.synchronize()
        # the dominant kernel: gate|up of 20 distinct layers, one launch each
        ws = [(synth_q4k(torch, F, H, gen), synth_q4k(torch, F, H, gen)) for _ in range(20)]
        x = torch.randn(H, device=dev, generator=gen)
        ys = [torch.empty(F, device=dev), torch.empty(F, device=dev)]
        for wg, wu in ws:
            rt.q4k_gemv_multi([wg, wu], ys, [F, F], x, H)
        torch.cuda.synchronize()
        print(json.dumps({"traffic_probe": "done", "copy_bytes": 256 << 20, "gemv_launches": len(ws)}))
        return 0

    # ---------------- weights: 34 distinct layers + tied BF16 embedding --------
    layers = []
    for li in range(L):
        w = {name: synth_q4k(torch, n, k, gen) for name, n, k in Q4K_SHAPES}
        for name in ("in_norm", "post_attn_norm", "pre_ffn_norm", "post_ffn_norm"):
            w[name] = torch.randn(H, device=dev, generator=gen) * 0.1
        w["q_norm"] = torch.randn(256, device=dev, generator=gen) * 0.1
        w["k_norm"] = torch.randn(256, device=dev, generator=gen) * 0.1
        layers.append(w)
    embed = (torch.randn(V * H, device=dev, generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16)
    final_norm = torch.randn(H, device=dev, generator=gen) * 0.1
    if args.prefill_profile:
        d, pos = build_decode(rt, torch, dev, gen, layers, embed, final_norm, args)
        toks = [(7 * i + 3) % V for i in range(pos)]
        for _ in range(args.warmup):
            d.prefill(toks, 0, 0)
        t1 = time.perf_counter()
        for _ in range(args.steps):
            d.prefill(toks, 0, 0)
        dt = (time.perf_counter() - t1) / args.steps
        print(json.dumps({"prefill_profile": "done", "tokens": pos, "steps": args.steps,
                          "ms_per_prefill": round(dt * 1e3, 3)}))
        d.close()
        return 0
    if args.decode_timeline:
        try:
            rt.trace_read()
        except rt.RtError as e:
            print(json.dumps({"error": f"--decode-timeline needs the traced library: {e}"}))
            return 2
        d, pos = build_decode(rt, torch, dev, gen, layers, embed, final_norm, args)
        for _ in range(args.warmup + args.steps):
            d.decode_step_async(pos % V, pos)
            pos += 1
        d.synchronize()
        out = decode_timeline(rt.trace_read())
        for row in out["kernels"]:
            log(f"{row['kernel']:7s} waves {row['waves']:5d}  gap before {row['gap_before_us']:5.2f} us | last wave "
                f"starts {row['start_max']:.2f} | staged p50 {row['staged_p50']:.2f} max {row['staged_max']:.2f} | "
                f"loads landed p50 {row['landed_p50']:.2f} max {row['landed_max']:.2f} | end p50 "
                f"{row['end_p50']:.2f} p90 {row['end_p90']:.2f} p99 {row['end_p99']:.2f} max {row['end_max']:.2f} us")
        log(f"layer span (q|k|v start to down end): {out['layer_span_us']:.2f} us")
        print(json.dumps({"decode_timeline": out, "steps": args.steps, "warmup": args.warmup}))
        d.close()
        return 0
    if args.decode_profile:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        a.fill_(1)
        torch.cuda.synchronize()
        b.copy_(a)  # counter calibration: reads and writes exactly 256 MiB
        torch.cuda.synchronize()
        del a, b
        fmts = None
        if args.q4_k_m:
            layers = [dict(w, v=synth_q6k_planar(torch, KVD, H, gen), down=synth_q6k_planar(torch, H, F, gen))
                      for w in layers]
            fmts = [1, 1, 4, 1, 1, 1, 4]
        elif args.q8_0:
            layers = [dict(w, **{name: synth_q8_0_planar(torch, n, k, gen) for name, n, k in Q4K_SHAPES})
                      for w in layers]
            fmts = [5] * 7
        elif args.bf16_model:
            layers = [dict(w, **{name: (torch.randn(n * k, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
                                 .view(torch.int16) for name, n, k in Q4K_SHAPES}) for w in layers]
            fmts = [2] * 7
        if args.shared_weights:
            layers = [layers[0]] * L
        d, pos = build_decode(rt, torch, dev, gen, layers, embed, final_norm, args, formats=fmts)
        if args.q4k_lm_head:
            head = synth_q4k(torch, V, H, gen)
            d.set_lm_head(1, head)
        bm = args.verify_rows

        def one(pos):
            if bm:
                d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
                return pos + bm
            d.decode_step_async(pos % V, pos)
            return pos + 1

        for _ in range(args.warmup):
            pos = one(pos)
        d.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.steps):
            pos = one(pos)
        d.synchronize()
        dt = (time.perf_counter() - t1) / args.steps
        print(json.dumps({"decode_profile": "done", "steps": args.steps, "verify_rows": bm,
                          "q4k_lm_head": args.q4k_lm_head, "q4_k_m": args.q4_k_m, "q8_0": args.q8_0,
                          "bf16_model": args.bf16_model, "shared_weights": args.shared_weights,
                          "ms_per_call": round(dt * 1e3, 4)}))
        d.close()
        return 0
    x_h = torch.randn(H, device=dev, generator=gen)
    x_q = torch.randn(QD, device=dev, generator=gen)
    x_f = torch.randn(F, device=dev, generator=gen)
    outs = {name: torch.empty(n, device=dev) for name, n, _ in Q4K_SHAPES}
    logits = torch.empty(V, device=dev)
    torch.cuda.synchronize()
    log(f"synthetic weights ready ({time.time() - t0:.1f}s)")

    # The step launches the projections as the decode step does: q|k|v and
    # gate|up share their input and run as one multi-matrix GEMV each.
    shape = {name: (n, k) for name, n, k in Q4K_SHAPES}
    step_launches = [("qkv", ("q", "k", "v"), x_h), ("o", ("o",), x_q), ("gateup", ("gate", "up"), x_h),
                     ("down", ("down",), x_f)]

    def launch_bytes(names):
        k = shape[names[0]][1]
        return sum(q4k_bytes(*shape[nm]) + 4 * shape[nm][0] for nm in names) + 4 * k

    step_bytes = L * sum(launch_bytes(names) for _, names, _ in step_launches)
    q4k_step_bytes = step_bytes
    step_bytes += gemv_bytes(V, H, V * H * 2)

    def enqueue_layer(w, names, x, stream):
        k = shape[names[0]][1]
        if len(names) == 1:
            rt.q4k_gemv(w[names[0]], x, outs[names[0]], shape[names[0]][0], k, stream=stream)
        else:
            rt.q4k_gemv_multi([w[nm] for nm in names], [outs[nm] for nm in names], [shape[nm][0] for nm in names],
                              x, k, stream=stream)

    # ---------------- the config-1 step as one graph ---------------------------
    def enqueue_step(stream):
        for w in layers:
            for _, names, x in step_launches:
                enqueue_layer(w, names, x, stream)
        rt.bf16_gemv(embed, x_h, logits, V, H, stream=stream)

    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        enqueue_step(cap)  # eager warm-up on the capture stream
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        enqueue_step(torch.cuda.current_stream())
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (step_ms * 1e-3) / 1e9
    log(f"config-1 step {step_ms:.3f} ms -> {value:.0f} GB/s ({step_bytes / 1e9:.3f} GB per step)")

    def time_graph(enqueue, reps):
        """Average ms of one replay of a graph of enqueue(stream) (one eager warm-up run first)."""
        with torch.cuda.stream(cap):
            enqueue(cap)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            enqueue(torch.cuda.current_stream())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        del g
        return a.elapsed_time(b) / reps

    # the same step without the BF16 lm_head: the Q4_K GEMVs alone
    def enqueue_q4k_only(stream):
        for w in layers:
            for _, names, x in step_launches:
                enqueue_layer(w, names, x, stream)

    q4k_ms = time_graph(enqueue_q4k_only, max(5, args.steps // 2))
    q4k_only = {"ms": round(q4k_ms, 4), "bytes": q4k_step_bytes,
                "GBps": round(q4k_step_bytes / (q4k_ms * 1e-3) / 1e9, 1),
                "frac_of_hbm_peak": round(q4k_step_bytes / (q4k_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    log(f"config-1 Q4_K GEMVs alone: {q4k_ms:.3f} ms -> {q4k_only['GBps']} GB/s")

    # ---------------- per-shape kernel timings (dominant kernel = gate/up) ------
    per_shape = {}
    reps = 10
    for name, n, k in Q4K_SHAPES + [("lm_head", V, H)]:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            s = torch.cuda.current_stream()
            if name == "lm_head":
                rt.bf16_gemv(embed, x_h, logits, V, H, stream=s)
            else:
                x = x_q if name == "o" else (x_f if name == "down" else x_h)
                for w in layers:
                    rt.q4k_gemv(w[name], x, outs[name], n, k, stream=s)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        launches = reps * (1 if name == "lm_head" else L)
        us = a.elapsed_time(b) * 1e3 / launches
        wb = V * H * 2 if name == "lm_head" else q4k_bytes(n, k)
        byts = gemv_bytes(n, k, wb)
        per_shape[name] = {"n": n, "k": k, "us_per_launch": round(us, 3), "GBps": round(byts / us / 1e3, 1),
                           "bytes_per_launch": byts}
        del g
    for fused, names, x in step_launches:
        if len(names) == 1:
            continue
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            s = torch.cuda.current_stream()
            for w in layers:
                enqueue_layer(w, names, x, s)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / (reps * L)
        byts = launch_bytes(names)
        per_shape[fused + "_fused"] = {"n": [shape[nm][0] for nm in names], "k": shape[names[0]][1],
                                       "us_per_launch": round(us, 3), "GBps": round(byts / us / 1e3, 1),
                                       "bytes_per_launch": byts}
        del g
    # ---------------- Q6_K / Q8_0 kept packed vs widened to BF16 ---------------
    # Q4_K_M files hold attn_v and ffn_down in Q6_K; the reference widens them
    # (and Q8_0) to BF16 at load (transformer4.rs:1233-1242).
    kquant = {}
    for name, n, k in (("v", KVD, H), ("down", H, F)):
        x = x_f if name == "down" else x_h
        y = torch.empty(n, device=dev)
        nb6, nb8 = n * k // 256, n * k // 32
        ws = {"q6k": [], "q8_0": [], "bf16": []}
        for _ in range(L):
            w6 = torch.randint(0, 256, (nb6 * 210,), dtype=torch.uint8, device=dev, generator=gen)
            w6[nb6 * 208:].view(torch.float16).copy_((torch.randn(nb6, device=dev, generator=gen) * 0.02).abs())
            w8 = torch.randint(0, 256, (nb8 * 34,), dtype=torch.uint8, device=dev, generator=gen)
            w8[n * k:].view(torch.float16).copy_((torch.randn(nb8, device=dev, generator=gen) * 0.02).abs())
            ws["q6k"].append(w6)
            ws["q8_0"].append(w8)
            ws["bf16"].append((torch.randn(n * k, device=dev, generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16))
        for fmt, fn, wbytes in (("q6k", rt.q6k_gemv, nb6 * 210), ("q8_0", rt.q8_0_gemv, nb8 * 34),
                                ("bf16", rt.bf16_gemv, n * k * 2)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                s = torch.cuda.current_stream()
                for w in ws[fmt]:
                    fn(w, x, y, n, k, stream=s)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                g.replay()
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / (reps * L)
            byts = gemv_bytes(n, k, wbytes)
            kquant[f"{fmt}_{name}"] = {"n": n, "k": k, "us_per_launch": round(us, 3),
                                       "GBps": round(byts / us / 1e3, 1), "bytes_per_launch": byts}
            del g
        del ws
        log(f"{name} {n}x{k}: Q6_K {kquant['q6k_' + name]['us_per_launch']} us, "
            f"Q8_0 {kquant['q8_0_' + name]['us_per_launch']} us, BF16 (reference widening) "
            f"{kquant['bf16_' + name]['us_per_launch']} us")
    # Streaming-read floor: a kernel that only reads, with 16-byte loads, the
    # same bytes per launch as the GEMV, from 34 distinct buffers in one graph
    # (the lm_head's from the 1.34 GB embedding itself); the fastest of a few
    # access patterns and grids.
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    floor = {}
    for label, nbytes in (("gateup_fused", per_shape["gateup_fused"]["bytes_per_launch"]),
                          ("gate", per_shape["gate"]["bytes_per_launch"]),
                          ("lm_head", per_shape["lm_head"]["bytes_per_launch"])):
        nb16 = (nbytes + 15) // 16 * 16
        if label == "lm_head":
            nb16 = embed.numel() * 2 // 16 * 16
            srcs, nrep = [embed] * 4, 4
        else:
            bufs = torch.empty(L, nb16, dtype=torch.uint8, device=dev)
            bufs.fill_(7)
            srcs, nrep = [bufs[i] for i in range(L)], L
        best = None
        for kind, grid in READ_CFGS:
            def enqueue_reads(stream, srcs=srcs, nb16=nb16, kind=kind, grid=grid):
                for b in srcs:
                    rt.stream_read(b, nb16, sink, stream=stream, kind=kind, grid=grid)

            us = time_graph(enqueue_reads, max(2, reps // 4) if label == "lm_head" else reps) * 1e3 / nrep
            if best is None or us < best[0]:
                best = (us, kind, grid)
        us = best[0]
        gbps = nb16 / us / 1e3
        floor[label] = {"bytes_per_launch": nb16, "us_per_launch": round(us, 3), "GBps": round(gbps, 1),
                        "frac_of_hbm_peak": round(gbps / PEAK_HBM_GBS, 4),
                        "read_kind_grid": [best[1], best[2]],
                        "gemv_frac_of_floor": round(per_shape[label]["GBps"] / (nbytes / us / 1e3), 4)}
        log(f"streaming-read floor, {nb16 / 1e6:.1f} MB per launch: {us:.2f} us, {gbps:.0f} GB/s "
            f"(kind {best[1]}, grid {best[2]}); the GEMV reaches {floor[label]['gemv_frac_of_floor']:.2f} of it")
        if label != "lm_head":
            del bufs
    # dominant kernel of the step (largest share of its time): the gate|up GEMV
    dom = per_shape["gateup_fused"]
    roofline = {"bound": "hbm", "achieved": dom["GBps"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(dom["GBps"] / PEAK_HBM_GBS, 4), "traffic": measured_traffic(),
                "kernel": "k_q4k_gemv_dig_multi<NB=10,T=320,ITERS=2> (Q4_K GEMV, gate|up 2 x 10240x2560 in one "
                          "launch)",
                "bytes_per_launch": dom["bytes_per_launch"], "us_per_launch": dom["us_per_launch"],
                "copy_floor": floor["gateup_fused"],
                "single_matrix": {"kernel": "k_q4k_gemv_dig<NB=10,T=960,ITERS=2> (10240x2560)",
                                  "us_per_launch": per_shape["gate"]["us_per_launch"],
                                  "GBps": per_shape["gate"]["GBps"],
                                  "frac": round(per_shape["gate"]["GBps"] / PEAK_HBM_GBS, 4),
                                  "copy_floor": floor["gate"]}}
    per_shape["lm_head"]["copy_floor"] = floor["lm_head"]
    log(f"dominant kernel gate|up 2x10240x2560: {dom['us_per_launch']} us/launch, {dom['GBps']} GB/s "
        f"(one 10240x2560 matrix alone: {per_shape['gate']['us_per_launch']} us)")

    # ---------------- config 3: full decode step -------------------------------
    decode = None
    if not args.skip_decode:
        ctx = 4096
        d, pos = build_decode(rt, torch, dev, gen, layers, embed, final_norm, args)
        for _ in range(args.warmup):
            d.decode_step_async(pos % V, pos)
            pos += 1
        d.synchronize()
        t_start = time.perf_counter()
        for _ in range(args.steps):
            d.decode_step_async(pos % V, pos)
            pos += 1
        d.synchronize()
        dt = (time.perf_counter() - t_start) / args.steps
        kv_read = (29 * 1024 + 5 * (ctx + 1)) * KVD * 4 * 2
        q4k_weights = L * sum(q4k_bytes(n, k) for _, n, k in Q4K_SHAPES)
        dec_bytes = q4k_weights + gemv_bytes(V, H, V * H * 2) + kv_read + H * 2 + L * 2 * KVD * 4
        decode = {"workload": "config 3: Gemma-3-4B decode step, ctx 4096, f32 KV, 34 layers, vocab 262144",
                  "tok_per_s": round(1.0 / dt, 1), "ms_per_token": round(dt * 1e3, 4),
                  "bytes_per_token": dec_bytes, "GBps": round(dec_bytes / dt / 1e9, 1),
                  "frac_of_hbm_peak": round(dec_bytes / dt / 1e9 / PEAK_HBM_GBS, 4),
                  "launches_per_token": 6 * L + 1}
        log(f"decode step {dt * 1e3:.3f} ms -> {1 / dt:.1f} tok/s")
        # batched verify (decode_step_batch, M = 8 draft tokens per call)
        bm = 8
        reps = max(2, args.steps // 4)
        for _ in range(2):
            d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
            pos += bm
        d.synchronize()
        t_start = time.perf_counter()
        for _ in range(reps):
            d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
            pos += bm
        d.synchronize()
        dtb = (time.perf_counter() - t_start) / reps
        decode["batch_verify"] = {"m": bm, "ms_per_call": round(dtb * 1e3, 4), "tok_per_s": round(bm / dtb, 1),
                                  "note": "every layer runs the 8 rows at once: batched Q4_K GEMV (int8 MFMA, one "
                                          "pass over the weights), key-split causal attention, batched lm_head"}
        log(f"decode_step_batch M={bm}: {dtb * 1e3:.3f} ms per call -> {bm / dtb:.1f} tok/s")
        decode["q4k_lm_head"] = q4k_lm_head_decode(rt, torch, gen, d, ctx, dec_bytes, args)
        decode["q4_k_m_layout"] = q4_k_m_layout_decode(rt, torch, dev, gen, layers, embed, final_norm, args)
        decode["q8_0_model"] = q8_0_model_decode(rt, torch, dev, gen, layers, embed, final_norm, args)
        # GPU prefill of a config-3-length prompt (4096 tokens) on the same weights
        toks = [(7 * i + 3) % V for i in range(ctx)]
        pf = {"tokens": ctx}
        for mode, name in ((0, "reference_window"), (1, "sliding_window")):
            d.prefill(toks, 0, mode)  # first call allocates the chunk scratch
            reps_p = 3
            t_start = time.perf_counter()
            for _ in range(reps_p):
                d.prefill(toks, 0, mode)
            dtp = (time.perf_counter() - t_start) / reps_p
            gf, af = prefill_flops(ctx, mode)
            pf[name] = {"ms": round(dtp * 1e3, 2), "tok_per_s": round(ctx / dtp, 1),
                        "gemm_TFLOP": round(gf / 1e12, 2), "attn_TFLOP": round(af / 1e12, 3),
                        "TFLOPs": round((gf + af) / dtp / 1e12, 1)}
            log(f"prefill {ctx} tokens ({name}): {dtp * 1e3:.1f} ms -> {ctx / dtp:.0f} tok/s, "
                f"{(gf + af) / dtp / 1e12:.0f} TFLOP/s")
        decode["prefill"] = pf
        d.close()

    # ---------------- configs 2 and 4: Q4_K GEMM on the matrix cores ------------
    gemm = None
    if not args.skip_gemm:
        gemm = {}
        for label, m, n, k in GEMM_SHAPES:
            w = synth_q4k(torch, n, k, gen)
            a = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
            c = torch.empty(m, n, device=dev)
            ab = a.view(torch.int16)
            for _ in range(2):
                rt.q4k_gemm(ab, w, c, m, n, k)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps_g = 10
            e0.record()
            for _ in range(reps_g):
                rt.q4k_gemm(ab, w, c, m, n, k)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps_g
            tf = 2.0 * m * n * k / us / 1e6
            # a plain f16 library GEMM of the same shape (weights already dequantised), for reference
            af, wf = a.to(torch.float16), torch.randn(n, k, device=dev, generator=gen).to(torch.float16)
            for _ in range(2):
                cf = af @ wf.T
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps_g):
                cf = af @ wf.T
            e1.record()
            torch.cuda.synchronize()
            us_lib = e0.elapsed_time(e1) * 1e3 / reps_g
            gemm[label] = {"m": m, "n": n, "k": k, "us": round(us, 1), "TFLOPs": round(tf, 1),
                           "frac_of_mfma_peak": round(tf / PEAK_F16_TFLOPS, 4),
                           "library_f16_gemm_us": round(us_lib, 1)}
            log(f"gemm {label} {m}x{n}x{k}: {us:.1f} us, {tf:.1f} TFLOP/s "
                f"({tf / PEAK_F16_TFLOPS * 100:.1f}% of peak); library f16 GEMM {us_lib:.1f} us")
            del w, a, c, ab, af, wf, cf

    # ---------------- CPU baseline (oracle = C port of the reference path) -----
    cpu = None
    if not args.skip_cpu:
        sys.path.insert(0, str(REPO))
        import tempfile
        from oracle import oracle as orc
        native_dir = tempfile.mkdtemp(prefix="rt_oracle_native_")
        orc.use_native_build(native_dir)  # gcc -O3 -march=native on this host
        nproc = os.cpu_count() or 1
        threads = min(nproc, 16)  # gemv_mt's hardware count, capped at the box's 16-CPU share
        host = [(name, n, k, orc.synth_q4k(77 + i, n, k)) for i, (name, n, k) in enumerate(Q4K_SHAPES)]
        xs = {H: orc.synth_normal(5, H), QD: orc.synth_normal(6, QD), F: orc.synth_normal(7, F)}
        lm_rows = 16384
        lm = orc.synth_bf16(8, lm_rows * H)
        sample_bytes = sum(gemv_bytes(n, k, q4k_bytes(n, k)) for _, n, k, _ in host) + \
            gemv_bytes(lm_rows, H, lm_rows * H * 2)
        reps_done, t_cpu = 0, 0.0
        while t_cpu < 10.0 or reps_done < 2:
            t1 = time.perf_counter()
            for name, n, k, blk in host:
                orc.q4k_gemv(blk, n, k, xs[k], threads)
            orc.bf16_gemv(lm, lm_rows, H, xs[H], threads)
            t_cpu += time.perf_counter() - t1
            reps_done += 1
        cpu_gbs = sample_bytes * reps_done / t_cpu / 1e9
        cpu = {"value": round(cpu_gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
               "nproc": nproc,
               "threads_rule": "gemv_mt (autograd2.rs:1961-1968): min(hw, N/128) threads per GEMV, hw = "
                               f"min(nproc={nproc}, 16); 16 is the CPU share of one GPU on this box",
               "build": "gcc -O3 -march=native -ffp-contract=off -fno-fast-math (oracle/rt_oracle.c, built on "
                        "this host at bench time)",
               "sample": f"one layer's 7 Q4_K projection GEMVs + {lm_rows} lm_head rows, "
                         f"{reps_done} reps in {t_cpu:.1f}s; oracle/rt_oracle.c dot_row/gemv_mt "
                         f"(scalar x86 branch of autograd2.rs)",
               "cpu_model": cpu_model()}
        log(f"cpu baseline {cpu_gbs:.2f} GB/s on {threads} threads")

    out = {
        "metric": "Q4_K GEMV HBM GB/s (% of peak); decode tok/s at Gemma-3-4B shape",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, f32 accumulate; GEMV activations staged as 16-bit fixed point per 64-element "
                 "chunk (3e-5 rel-L2)",
        "data": "synthetic",
        "frac_of_hbm_peak": round(value / PEAK_HBM_GBS, 4),
        "config": {"workload": "config 1: Gemma-3-4B projection set of one decode token, 34 distinct layers x "
                               "{q,k,v,o,gate,up,down} Q4_K GEMV (q|k|v and gate|up, which share their input, "
                               "one launch each) + BF16 lm_head 2560->262144, one hipGraph",
                   "bytes_per_step": step_bytes, "parallelism": "single GPU"},
        "q4k_only": q4k_only,
        "roofline": roofline,
        "per_shape": per_shape,
        "kquant_gemv": kquant,
        "decode": decode,
        "gemm": gemm,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def gemm_tiles_probe(rt, torch, dev, gen) -> dict:
    """Whole rt_q4k_gemm_bf16 calls at M = 512, K = 2560 with 128, 160 and 256
    output tiles (N = 8192, 10240, 16384), and config 2's down shape: with
    one tile per CU, how the time of a tile's 40 K-chunks grows with the
    number of tiles in flight (what a balanced split of config 2 could gain)."""
    out = []
    for m, n, k in ((512, 8192, 2560), (512, 10240, 2560), (512, 16384, 2560), (512, 2560, 10240)):
        w = synth_q4k(torch, n, k, gen)
        a = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16).view(torch.int16)
        c = torch.empty(m, n, device=dev)
        for _ in range(3):
            rt.q4k_gemm(a, w, c, m, n, k)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            rt.q4k_gemm(a, w, c, m, n, k)
        e1.record()
        torch.cuda.synchronize()
        out.append({"m": m, "n": n, "k": k, "tiles": (m // 128) * (n // 256), "us": round(e0.elapsed_time(e1) * 1e3 / 20, 1)})
        del w, a, c
    return {"gemm_tiles": out}


def launch_probe(rt, torch, dev) -> dict:
    """The launch floor of this GPU inside a graph, the figures that set the
    decode step's launch structure: (1) µs per launch of a graph of 100
    dependent empty kernels (one wave, and 256 / 1024 workgroups), (2) µs per
    launch of streaming reads (the fastest of READ_CFGS) of 4-118 MB from
    distinct buffers (>= 600 MB per replay, beyond the 256 MB MALL), fitted by
    least squares to t = fixed + bytes / rate."""
    cap = torch.cuda.Stream()

    def per_launch_us(enqueue, n, reps):
        with torch.cuda.stream(cap):
            enqueue(cap)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            enqueue(torch.cuda.current_stream())
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        del g
        return a.elapsed_time(b) * 1e3 / (reps * n)

    out = {"empty_launch_us": {}, "stream_read": []}
    for grid, thr in ((1, 64), (256, 256), (1024, 256)):
        us = per_launch_us(lambda st, grid=grid, thr=thr: [rt.empty_launch(grid, thr, st) for _ in range(100)], 100, 20)
        out["empty_launch_us"][f"{grid}x{thr}"] = round(us, 3)
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    xs, ys = [], []
    for nbytes in (4 << 20, 8 << 20, 14796800, 29583360, 59166720, 118333440):
        nbuf = min(160, -(-(600 << 20) // nbytes))
        bufs = torch.empty(nbuf, nbytes, dtype=torch.uint8, device=dev)
        bufs.fill_(3)
        best = None
        for kind, grid in READ_CFGS:
            us = per_launch_us(lambda st, kind=kind, grid=grid: [rt.stream_read(bufs[i], nbytes, sink, stream=st,
                                                                                kind=kind, grid=grid)
                                                                 for i in range(nbuf)], nbuf, 10)
            best = us if best is None else min(best, us)
        out["stream_read"].append({"bytes": nbytes, "us": round(best, 3), "GBps": round(nbytes / best / 1e3, 1)})
        xs.append(nbytes)
        ys.append(best)
        del bufs
    n = len(xs)
    mx, my = sum(xs) / n, sum(ys) / n
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    out["fit"] = {"fixed_us": round(my - slope * mx, 3), "rate_GBps": round(1e-3 / slope, 1)}
    return out


def decode_timeline(tr) -> dict:
    """Per-kernel statistics of a traced decode step (rt_trace_read's record:
    [kernel][slot][entry, staged, landed, exit] in 10 ns ticks).  Slots hold
    the last launch of each kernel: the last layer's six and the lm_head.
    Slots not rewritten by that launch (a smaller grid than an earlier layer's)
    carry older stamps and are dropped: only stamps from the last q|k|v launch
    on count.  Times are us from each kernel's first wave; the gap is from the
    previous kernel's last wave end to this kernel's first wave start."""
    import numpy as np
    names = ["q|k|v", "attn", "merge", "o", "gate|up", "down", "lm_head"]
    live = [tr[k][tr[k][:, 0] > 0].astype(np.int64) for k in range(len(names))]
    t0 = int(live[0][:, 0].min())
    rows, prev_end = [], None
    for k, name in enumerate(names):
        a = live[k][live[k][:, 0] >= t0]
        s0, end = int(a[:, 0].min()), int(a[:, 3].max())
        rel = (a - s0) * 0.01
        p50 = lambda c: round(float(np.percentile(rel[:, c], 50)), 3)
        rows.append({"kernel": name, "waves": int(len(a)),
                     "gap_before_us": round((s0 - prev_end) * 0.01, 3) if prev_end is not None else 0.0,
                     "start_max": round(float(rel[:, 0].max()), 3), "staged_p50": p50(1),
                     "staged_max": round(float(rel[:, 1].max()), 3), "landed_p50": p50(2),
                     "landed_max": round(float(rel[:, 2].max()), 3), "end_p50": p50(3),
                     "end_p90": round(float(np.percentile(rel[:, 3], 90)), 3),
                     "end_p99": round(float(np.percentile(rel[:, 3], 99)), 3),
                     "end_max": round(float(rel[:, 3].max()), 3)})
        prev_end = end
    span = (int(live[5][live[5][:, 0] >= t0][:, 3].max()) - t0) * 0.01
    return {"kernels": rows, "layer_span_us": round(span, 3)}


def build_decode(rt, torch, dev, gen, layers, embed, final_norm, args, ctx: int = 4096, formats=None):
    """The config-3 decode context: the 34 synthetic layers, N(0,1) K/V rows
    0..ctx-1 in every layer, the BF16 tied embedding; returns it and the
    first position to decode (ctx)."""
    d = rt.HipDecodeContext(dict(rt.GEMMA3_4B), ctx + 8 * (args.warmup + args.steps) + 8 * (2 + max(2, args.steps // 4)) + 8)
    for li, w in enumerate(layers):
        if formats:
            d.set_layer(li, w, formats=formats)
        else:
            d.set_layer(li, w)
        kv = torch.randn(2, ctx, KVD, device=dev, generator=gen)
        d.sync_kv_from_cpu(li, kv[0], kv[1], ctx)
        del kv
    d.set_embed(embed, final_norm)
    torch.cuda.synchronize()
    return d, ctx


def q4k_lm_head_decode(rt, torch, gen, d, ctx: int, dec_bytes: int, args) -> dict:
    """The config-3 step and M = 8 verify with a Q4_K lm_head (the reference's
    q4k-lm-head feature, metal_decode.rs:1082-1094): the same context and
    positions from ctx, the 262144x2560 head as random Q4_K blocks (the same
    bytes as a requantised embedding; parity is in the tests); the tied BF16
    head is restored afterwards."""
    head = synth_q4k(torch, V, H, gen)
    d.set_lm_head(1, head)
    pos = ctx
    for _ in range(args.warmup):
        d.decode_step_async(pos % V, pos)
        pos += 1
    d.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        d.decode_step_async(pos % V, pos)
        pos += 1
    d.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    bm, reps = 8, max(2, args.steps // 4)
    d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
    d.synchronize()
    t0 = time.perf_counter()
    for r in range(reps):
        d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
    d.synchronize()
    dtb = (time.perf_counter() - t0) / reps
    d.set_lm_head(0, None)
    del head
    nbytes = dec_bytes - V * H * 2 + q4k_bytes(V, H)
    out = {"workload": "config 3 with a Q4_K lm_head (feature q4k-lm-head) instead of the BF16 tied one",
           "tok_per_s": round(1.0 / dt, 1), "ms_per_token": round(dt * 1e3, 4), "bytes_per_token": nbytes,
           "GBps": round(nbytes / dt / 1e9, 1), "frac_of_hbm_peak": round(nbytes / dt / 1e9 / PEAK_HBM_GBS, 4),
           "verify_m": bm, "verify_ms_per_call": round(dtb * 1e3, 4), "verify_tok_per_s": round(bm / dtb, 1)}
    log(f"Q4_K lm_head: decode step {dt * 1e3:.3f} ms -> {1 / dt:.1f} tok/s; verify M={bm} {dtb * 1e3:.3f} ms")
    return out


def q8_0_model_decode(rt, torch, dev, gen, layers, embed, final_norm, args) -> dict:
    """The config-3 step and the M = 8 verify with every projection in Q8_0
    (a Q8_0 file; planar layout, random codes and scales): q|k|v and gate|up
    run as the fused Q8_0 launches."""
    ctx = 4096
    q8 = [{name: synth_q8_0_planar(torch, n, k, gen) for name, n, k in Q4K_SHAPES} for _ in range(L)]
    d = rt.HipDecodeContext(dict(rt.GEMMA3_4B), ctx + 8 * (args.warmup + args.steps) + 8 * 12 + 8)
    for li, w in enumerate(layers):
        d.set_layer(li, dict(w, **q8[li]), formats=[5] * 7)
        kv = torch.randn(2, ctx, KVD, device=dev, generator=gen)
        d.sync_kv_from_cpu(li, kv[0], kv[1], ctx)
        del kv
    d.set_embed(embed, final_norm)
    torch.cuda.synchronize()
    pos = ctx
    for _ in range(args.warmup):
        d.decode_step_async(pos % V, pos)
        pos += 1
    d.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        d.decode_step_async(pos % V, pos)
        pos += 1
    d.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    bm, reps = 8, max(4, args.steps // 2)
    for _ in range(2):
        d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
        pos += bm
    d.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
        pos += bm
    d.synchronize()
    dtb = (time.perf_counter() - t0) / reps
    wbytes = L * sum(n * k // 32 * 34 for _, n, k in Q4K_SHAPES) + V * H * 2
    out = {"formats": "every projection Q8_0 (planar); BF16 tied lm_head", "decode_ms_per_token": round(dt * 1e3, 4),
           "decode_tok_per_s": round(1.0 / dt, 1), "weight_bytes_per_token": wbytes,
           "GBps": round(wbytes / dt / 1e9, 1), "verify_m": bm, "verify_ms_per_call": round(dtb * 1e3, 4)}
    log(f"Q8_0 model: decode step {dt * 1e3:.3f} ms ({wbytes / dt / 1e9:.0f} GB/s of weights); "
        f"verify M={bm} {dtb * 1e3:.3f} ms per call")
    d.close()
    del q8
    return out


def synth_q8_0_planar(torch, n: int, k: int, gen) -> "torch.Tensor":
    """Random planar Q8_0 (rt_q8_0_repack layout: int8 q [n][k] | f16 d [n*k/32]),
    d = f16 of |N(0, 0.02)|."""
    nq = n * k
    w = torch.randint(0, 256, (nq + nq // 32 * 2,), dtype=torch.uint8, device="cuda", generator=gen)
    d = (torch.randn(nq // 32, device="cuda", generator=gen).abs() * 0.02).half()
    w[nq:] = d.view(torch.uint8)
    return w


def synth_q6k_planar(torch, n: int, k: int, gen) -> "torch.Tensor":
    """Random planar Q6_K (rt_q6k_repack layout: ql | qh | int8 scales | f16 d),
    d = f16 of |N(0, 0.02)|."""
    nbt = n * k // 256
    w = torch.randint(0, 256, (nbt * 210,), dtype=torch.uint8, device="cuda", generator=gen)
    d = (torch.randn(nbt, device="cuda", generator=gen).abs() * 0.02).half()
    w[nbt * 208:] = d.view(torch.uint8)
    return w


def q4_k_m_layout_decode(rt, torch, dev, gen, layers, embed, final_norm, args) -> dict:
    """The config-3 step and the M = 8 verify batch with the Q4_K_M recipe's
    layout: v and down in Q6_K (kept packed), the other projections Q4_K.
    The verify reads every weight once per call (batched GEMV of each
    format); weight bytes per call = the layers' projections + the lm_head."""
    q6 = [{"v": synth_q6k_planar(torch, KVD, H, gen), "down": synth_q6k_planar(torch, H, F, gen)} for _ in range(L)]
    ctx = 4096
    d = rt.HipDecodeContext(dict(rt.GEMMA3_4B), ctx + 8 * (args.warmup + args.steps) + 8 * 12 + 8)
    fmts = [1, 1, 4, 1, 1, 1, 4]
    for li, w in enumerate(layers):
        d.set_layer(li, dict(w, **q6[li]), formats=fmts)
        kv = torch.randn(2, ctx, KVD, device=dev, generator=gen)
        d.sync_kv_from_cpu(li, kv[0], kv[1], ctx)
        del kv
    d.set_embed(embed, final_norm)
    torch.cuda.synchronize()
    pos = ctx
    for _ in range(args.warmup):
        d.decode_step_async(pos % V, pos)
        pos += 1
    d.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        d.decode_step_async(pos % V, pos)
        pos += 1
    d.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    bm, reps = 8, max(4, args.steps // 2)
    for _ in range(2):
        d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
        pos += bm
    d.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        d.decode_step_batch_async([(pos + i) % V for i in range(bm)], pos)
        pos += bm
    d.synchronize()
    dtb = (time.perf_counter() - t0) / reps
    q6b = lambda n, k: n * k // 256 * 210  # noqa: E731
    layer_bytes = sum(q4k_bytes(n, k) for name, n, k in Q4K_SHAPES if name not in ("v", "down")) + q6b(KVD, H) + q6b(H, F)
    wbytes = L * layer_bytes + V * H * 2
    out = {"formats": "q, k, o, gate, up Q4_K; v, down Q6_K (planar); BF16 tied lm_head",
           "verify_batched": d.verify_batched, "decode_ms_per_token": round(dt * 1e3, 4),
           "verify_m": bm, "verify_ms_per_call": round(dtb * 1e3, 4), "verify_tok_per_s": round(bm / dtb, 1),
           "weight_bytes_per_call": wbytes, "weight_GBps": round(wbytes / dtb / 1e9, 1)}
    log(f"Q4_K_M layout: decode step {dt * 1e3:.3f} ms; verify M={bm} {dtb * 1e3:.3f} ms per call "
        f"({'batched' if d.verify_batched else 'per-token'}), weights {wbytes / dtb / 1e9:.0f} GB/s")
    d.close()
    del q6
    return out


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration),
    or None when the summary is absent."""
    f = REPO / "profiles" / "q4k_gemv_gateup_2x10240x2560_traffic.txt"
    try:
        for line in f.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch="):
                return int(float(line.split("=", 1)[1]))
    except OSError:
        pass
    return None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
