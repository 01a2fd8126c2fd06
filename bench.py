#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matvec hot path (one GPU).

Headline workload: GGUF Q4_0 fused dequant+GEMV at the LLaMA-7B gate_proj
shape, W = 11008 x 4096 (Q4_0 blocks: fp16 d ~ U(0.005, 0.02), uniform 4-bit
codes), x fp16 [1, 4096] ~ N(0, 1), y fp16 [1, 11008], fp32 accumulation.
One step = one fused GEMV launch through the C ABI.  Weights rotate over
`--copies` distinct HBM-resident copies (16 x 25.4 MB = 406 MB, more than the
256 MB Infinity Cache), so every step streams its weights from HBM.  The K
timed steps are replayed from HIP graphs of `--chunk` launches, bracketed by
HIP events on the launch stream.

Also reported (same JSON line): the LLaMA-7B Q4_0 decode weight sweep, all 32
layers resident (7 projection GEMVs per layer + lm_head 32000 x 4096, one HIP
graph per token) as tokens/s, fused (q/k/v grouped, gate+up+SiLU in one
launch: 129 launches) and unfused (225 launches), and the CPU baseline (torch
restatement of dequant -> F.linear in fp32 on the host cores).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "Q4_0 GEMV µs + HBM GB/s (% peak) at 11008x4096 b=1; 7B decode tok/s"
HBM_PEAK_GBS = 8000.0

M0, K0 = 11008, 4096
Q4_0_ROW_BYTES = K0 // 32 * 18
# algorithmic bytes of one call: packed weights + scales, x, y
ALGO_BYTES_CFG0 = M0 * Q4_0_ROW_BYTES + K0 * 2 + M0 * 2  # 25,392,640

# LLaMA-7B: hidden 4096, ffn 11008, vocab 32000, 32 layers
LAYER_SHAPES = [(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008)]  # q k v o gate up down
LM_HEAD = (32000, 4096)
N_LAYERS = 32


def q4_bytes(m: int, k: int) -> int:
    return m * (k // 32) * 18


def sweep_bytes() -> int:
    per_layer = sum(q4_bytes(m, k) + 2 * k + 2 * m for m, k in LAYER_SHAPES)
    m, k = LM_HEAD
    return N_LAYERS * per_layer + q4_bytes(m, k) + 2 * k + 2 * m


PROFILE = os.path.join(ROOT, "profiles", "q4_0_gemv_11008x4096_b1.txt")


def measured_traffic():
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (None when absent)."""
    try:
        with open(PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _ensure_built() -> None:
    from gdsllm_amd import build as b

    if not (b.LIB.exists() and b.EXT.exists()):
        b.build_all()


class Q4Gemv:
    """Launches gdsllm_fused_q4_0_gemv on torch's current stream."""

    def __init__(self):
        from gdsllm_amd import capi, check

        self.lib = capi()
        self.check = check

    def __call__(self, w, x, y, m: int, k: int) -> None:
        import torch

        s = torch.cuda.current_stream().cuda_stream
        self.check(self.lib.gdsllm_fused_q4_0_gemv(w.data_ptr(), x.data_ptr(), y.data_ptr(), m, k, 1, k, m, s))


def bench_gemv(args, dev):
    import torch

    from gdsllm_amd import synthetic as syn

    gemv = Q4Gemv()
    copies = [syn.q4_0_weights(M0, K0, torch.Generator(device=dev).manual_seed(1000 + i)) for i in range(args.copies)]
    x = syn.activations(1, K0, torch.Generator(device=dev).manual_seed(999))
    ys = torch.empty(args.copies, M0, dtype=torch.float16, device=dev)
    n = args.copies

    for i in range(max(args.warmup, n)):
        gemv(copies[i % n], x, ys[i % n], M0, K0)
    torch.cuda.synchronize()

    chunk = args.chunk
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(chunk):
            gemv(copies[i % n], x, ys[i % n], M0, K0)
    graph.replay()
    torch.cuda.synchronize()

    K = args.steps
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(K // chunk):
        graph.replay()
    for i in range(K % chunk):
        gemv(copies[i % n], x, ys[i % n], M0, K0)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    return {"ms": ms, "weights0": copies[0], "x": x, "y0": ys[0].clone()}


def bench_decode_sweep(args, dev):
    """LLaMA-7B Q4_0 decode weight sweep, one HIP graph per token, timed two ways.

    unfused: 225 single GEMV launches (7 per layer + lm_head), every GEMV
    reading a synthetic x of its in_dim.
    fused: 129 launches with the reference layer's data flow (llama.py:212-256):
    q/k/v in one grouped launch on x_attn, o on x_o, gate+up+SiLU in one launch
    on x_mlp writing h, down on that h; lm_head last.  Same weights, same
    224 + 1 projections.  Returns (ms fused, ms unfused, weights)."""
    import ctypes

    import torch

    from gdsllm_amd import capi, check
    from gdsllm_amd import synthetic as syn

    gemv = Q4Gemv()
    lib = capi()
    gen = torch.Generator(device=dev).manual_seed(2004)
    layers = [[syn.q4_0_weights(m, k, gen) for m, k in LAYER_SHAPES] for _ in range(N_LAYERS)]
    lm_head = syn.q4_0_weights(*LM_HEAD, gen)
    xs = {k: syn.activations(1, k, gen) for k in (4096, 11008)}
    ys = {m: torch.empty(1, m, dtype=torch.float16, device=dev) for m in (4096, 11008, 32000)}
    x_attn, x_o, x_mlp = (syn.activations(1, 4096, gen) for _ in range(3))
    y_qkv = [torch.empty(1, 4096, dtype=torch.float16, device=dev) for _ in range(3)]
    y_o, y_down = torch.empty(1, 4096, dtype=torch.float16, device=dev), torch.empty(1, 4096, dtype=torch.float16, device=dev)
    h = torch.empty(1, 11008, dtype=torch.float16, device=dev)
    qkv_w = [(ctypes.c_void_p * 3)(*[w.data_ptr() for w in lw[:3]]) for lw in layers]
    qkv_y = (ctypes.c_void_p * 3)(*[y.data_ptr() for y in y_qkv])
    qkv_m = (ctypes.c_int64 * 3)(4096, 4096, 4096)

    def token_unfused():
        for lw in layers:
            for w, (m, k) in zip(lw, LAYER_SHAPES):
                gemv(w, xs[k], ys[m], m, k)
        gemv(lm_head, xs[LM_HEAD[1]], ys[LM_HEAD[0]], *LM_HEAD)

    def token_fused():
        st = torch.cuda.current_stream().cuda_stream
        for li, lw in enumerate(layers):
            check(lib.gdsllm_fused_q4_0_gemv_group(3, qkv_w[li], qkv_y, qkv_m, x_attn.data_ptr(), 4096, 1, 4096, st))
            gemv(lw[3], x_o, y_o, 4096, 4096)
            check(lib.gdsllm_fused_q4_0_gate_up_silu(lw[4].data_ptr(), lw[5].data_ptr(), x_mlp.data_ptr(),
                                                     h.data_ptr(), 11008, 4096, 1, 4096, 11008, st))
            gemv(lw[6], h, y_down, 4096, 11008)
        gemv(lm_head, x_attn, ys[LM_HEAD[0]], *LM_HEAD)

    ms_unfused = _replay_ms(token_unfused, args.sweep_tokens)
    ms_fused = _replay_ms(token_fused, args.sweep_tokens)
    return ms_fused, ms_unfused, (layers, lm_head)


def _replay_ms(capture, reps: int, warm: int = 3) -> float:
    """Captures `capture()` (launches on the current stream) into a HIP graph
    once, replays it `warm` times untimed, then `reps` times between HIP
    events on the launch stream; returns ms per replay."""
    import torch

    capture()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capture()
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def _gemv_call(fmt: str, w, x, y, m: int, k: int, b: int) -> None:
    import torch

    from gdsllm_amd import capi, check

    fn = capi().gdsllm_fused_q4_0_gemv if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv
    check(fn(w.data_ptr(), x.data_ptr(), y.data_ptr(), m, k, b, k, m, torch.cuda.current_stream().cuda_stream))


def bench_q8_layer(dev, layers_rotated: int = 3, reps: int = 50):
    """Q8_0 LLaMA-7B decoder layer at batch 1: 7 GEMVs per layer, rotating over
    `layers_rotated` distinct layers (3 x 215 MB > the 256 MB Infinity Cache)."""
    import torch

    from gdsllm_amd import synthetic as syn

    gen = torch.Generator(device=dev).manual_seed(1001)
    layers = [[syn.q8_0_weights(m, k, gen) for m, k in LAYER_SHAPES] for _ in range(layers_rotated)]
    xs = {k: syn.activations(1, k, gen) for k in (4096, 11008)}
    ys = {m: torch.empty(1, m, dtype=torch.float16, device=dev) for m in (4096, 11008)}

    def run():
        for lw in layers:
            for w, (m, k) in zip(lw, LAYER_SHAPES):
                _gemv_call("q8_0", w, xs[k], ys[m], m, k, 1)

    ms = _replay_ms(run, reps) / layers_rotated
    nbytes = sum(m * (k // 32) * 34 + 2 * k + 2 * m for m, k in LAYER_SHAPES)
    return {"us_per_layer": round(ms * 1e3, 3), "bytes_per_layer": nbytes,
            "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1), "pct_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / 80, 1),
            "layers_rotated": layers_rotated}


def bench_int8_layer(dev, layers_rotated: int = 2, reps: int = 50, ref_reps: int = 5):
    """Per-column int8 LLaMA-7B decoder layer at batch 1 (the converter's int8
    format): 7 fused GEMVs per layer over `layers_rotated` distinct layers
    (2 x 202 MB > the 256 MB Infinity Cache).  Beside it, the reference's
    expression for the same layer on the same GPU,
    F.linear(x, (w.float() * scale).half()) per projection (runtime/llama.py:162-165)."""
    import torch
    import torch.nn.functional as F

    from gdsllm_amd import capi, check
    from gdsllm_amd import synthetic as syn

    gen = torch.Generator(device=dev).manual_seed(1007)
    layers = [[syn.int8_weights(m, k, gen) for m, k in LAYER_SHAPES] for _ in range(layers_rotated)]
    xs = {k: syn.activations(1, k, gen) for k in (4096, 11008)}
    ys = {m: torch.empty(1, m, dtype=torch.float16, device=dev) for m in (4096, 11008)}
    lib = capi()

    def run():
        st = torch.cuda.current_stream().cuda_stream
        for lw in layers:
            for (q, sc), (m, k) in zip(lw, LAYER_SHAPES):
                check(lib.gdsllm_fused_int8_gemv(q.data_ptr(), sc.data_ptr(), xs[k].data_ptr(), ys[m].data_ptr(),
                                                 m, k, 1, k, m, st))

    def run_ref():
        for (q, sc), (m, k) in zip(layers[0], LAYER_SHAPES):
            F.linear(xs[k], (q.float() * sc).half())

    ms = _replay_ms(run, reps) / layers_rotated
    run_ref()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(ref_reps):
        run_ref()
    torch.cuda.synchronize()
    ref_ms = (time.perf_counter() - t0) * 1e3 / ref_reps
    nbytes = sum(m * k + 2 * k + 2 * k + 2 * m for m, k in LAYER_SHAPES)
    return {"us_per_layer": round(ms * 1e3, 3), "bytes_per_layer": nbytes,
            "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1), "pct_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / 80, 1),
            "layers_rotated": layers_rotated, "reference_expression_us_per_layer": round(ref_ms * 1e3, 1)}


def bench_moe(dev, calls: int = 64, reps: int = 20):
    """Affine-Q4 top-10 expert-gather MLP, 512 experts, hidden 4096, ffn 1024,
    group 64, batch 1; every call in the graph uses its own fresh random
    distinct top-10 picks from the 3.6 GB resident pool."""
    import ctypes

    import torch

    from gdsllm_amd import AffineExperts, capi, check
    from gdsllm_amd import synthetic as syn

    E, H, Fd, g, k = 512, 4096, 1024, 64, 10
    gen = torch.Generator(device=dev).manual_seed(1002)
    pools = [syn.affine_q4_weights([E, Fd, H], g, gen), syn.affine_q4_weights([E, Fd, H], g, gen),
             syn.affine_q4_weights([E, H, Fd], g, gen)]

    def experts(p):
        w, sc, bi = p
        e, n, kw = w.shape
        kk = kw * 8
        return AffineExperts(w.data_ptr(), sc.data_ptr(), bi.data_ptr(), n * kw * 4, n * (kk // g) * 2,
                             n * (kk // g) * 2, e, n, kk, g)

    gate, up, down = (experts(p) for p in pools)
    cg = torch.Generator().manual_seed(1003)
    idx = torch.stack([torch.randperm(E, generator=cg)[:k] for _ in range(calls)]).to(torch.int32).to(dev)
    wts = torch.softmax(torch.randn(calls, k, generator=cg), -1).to(torch.float16).to(dev)
    x = syn.activations(1, H, gen)
    y = torch.empty(calls, H, dtype=torch.float16, device=dev)
    ws_bytes = capi().gdsllm_moe_gather_workspace_size(k, Fd)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

    def run():
        s = torch.cuda.current_stream().cuda_stream
        for i in range(calls):
            check(capi().gdsllm_moe_gather_affine_q4(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down),
                                                     x.data_ptr(), idx[i].data_ptr(), wts[i].data_ptr(), k,
                                                     y[i].data_ptr(), ws.data_ptr(), ws_bytes, s))

    ms = _replay_ms(run, reps) / calls
    per_expert = 2 * (Fd * H // 2 + 2 * 2 * Fd * H // g) + (H * Fd // 2 + 2 * 2 * H * Fd // g)
    nbytes = k * per_expert + 2 * H + 2 * H
    out = {"us_per_call": round(ms * 1e3, 3), "bytes_per_call": nbytes,
           "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1), "pct_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / 80, 1),
           "launches_per_call": 2, "pool_bytes": sum(t.numel() * t.element_size() for p in pools for t in p)}

    # The whole decode MoE step on the device, no host round trip: fp16 router
    # GEMV (512 x 4096), top-k + softmax, the top-10 gather, the shared expert
    # (ffn 1024, as a one-expert gather), the shared-gate GEMV and the combine.
    # Every call routes its own token and reads its own router and shared
    # expert (as the layers of a model do), so those come from HBM too.
    router = (torch.randn(calls, E, H, generator=gen, device=dev) * 0.02).to(torch.float16)
    sgate = (torch.randn(calls, H, generator=gen, device=dev) * 0.02).to(torch.float16)
    shared = [syn.affine_q4_weights([calls, Fd, H], g, gen), syn.affine_q4_weights([calls, Fd, H], g, gen),
              syn.affine_q4_weights([calls, H, Fd], g, gen)]
    sh_g, sh_u, sh_d = (experts(p) for p in shared)
    xs = syn.activations(calls, H, gen)
    logits = torch.empty(calls, E, dtype=torch.float16, device=dev)
    ridx = torch.empty(calls, k, dtype=torch.int32, device=dev)
    rw = torch.empty(calls, k, dtype=torch.float16, device=dev)
    eo, so, yy = (torch.empty(calls, H, dtype=torch.float16, device=dev) for _ in range(3))
    gl = torch.empty(calls, 1, dtype=torch.float16, device=dev)
    sidx = torch.arange(calls, dtype=torch.int32, device=dev)
    sw = torch.ones(calls, dtype=torch.float16, device=dev)
    ws1_bytes = capi().gdsllm_moe_gather_workspace_size(1, Fd)
    ws1 = torch.empty(ws1_bytes, dtype=torch.uint8, device=dev)

    def step():
        s = torch.cuda.current_stream().cuda_stream
        for i in range(calls):
            xi = xs[i].data_ptr()
            check(capi().gdsllm_gemv_f16(router[i].data_ptr(), xi, logits[i].data_ptr(), E, H, 1, H, E, s))
            check(capi().gdsllm_moe_route_topk(logits[i].data_ptr(), E, 1, E, k, ridx[i].data_ptr(),
                                               rw[i].data_ptr(), s))
            check(capi().gdsllm_moe_gather_affine_q4(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down), xi,
                                                     ridx[i].data_ptr(), rw[i].data_ptr(), k, eo[i].data_ptr(),
                                                     ws.data_ptr(), ws_bytes, s))
            check(capi().gdsllm_moe_gather_affine_q4(ctypes.byref(sh_g), ctypes.byref(sh_u), ctypes.byref(sh_d), xi,
                                                     sidx[i:].data_ptr(), sw[i:].data_ptr(), 1, so[i].data_ptr(),
                                                     ws1.data_ptr(), ws1_bytes, s))
            check(capi().gdsllm_gemv_f16(sgate[i].data_ptr(), xi, gl[i].data_ptr(), 1, H, 1, H, 1, s))
            check(capi().gdsllm_moe_combine(eo[i].data_ptr(), so[i].data_ptr(), gl[i].data_ptr(), yy[i].data_ptr(), H,
                                            1, s))

    ms2 = _replay_ms(step, reps) / calls

    # The same step with the shared expert, its gate and the combine fused
    # into the gather's two launches (gdsllm_moe_step_affine_q4): 4 launches.
    def one_expert(e, i):
        w, sc, bi = (t[i] for t in shared[e])
        n, kw = w.shape
        kk = kw * 8
        return AffineExperts(w.data_ptr(), sc.data_ptr(), bi.data_ptr(), n * kw * 4, n * (kk // g) * 2,
                             n * (kk // g) * 2, 1, n, kk, g)

    sh_one = [[one_expert(e, i) for e in range(3)] for i in range(calls)]
    wsf_bytes = capi().gdsllm_moe_step_workspace_size(k, Fd)
    wsf = torch.empty(wsf_bytes, dtype=torch.uint8, device=dev)
    yf = torch.empty(calls, H, dtype=torch.float16, device=dev)

    def step_fused():
        s = torch.cuda.current_stream().cuda_stream
        for i in range(calls):
            xi = xs[i].data_ptr()
            check(capi().gdsllm_gemv_f16(router[i].data_ptr(), xi, logits[i].data_ptr(), E, H, 1, H, E, s))
            check(capi().gdsllm_moe_route_topk(logits[i].data_ptr(), E, 1, E, k, ridx[i].data_ptr(),
                                               rw[i].data_ptr(), s))
            sg_, su_, sd_ = sh_one[i]
            check(capi().gdsllm_moe_step_affine_q4(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down),
                                                   ctypes.byref(sg_), ctypes.byref(su_), ctypes.byref(sd_), xi,
                                                   ridx[i].data_ptr(), rw[i].data_ptr(), k, sgate[i].data_ptr(),
                                                   yf[i].data_ptr(), wsf.data_ptr(), wsf_bytes, s))

    ms3 = _replay_ms(step_fused, reps) / calls
    torch.cuda.synchronize()
    nbytes2 = E * H * 2 + (k + 1) * per_expert + H * 2 + 2 * H * 2
    includes = ("fp16 router GEMV 512x4096, top-k+softmax, top-10 gather, shared expert (ffn 1024), "
                "shared-gate GEMV, combine+clamp")
    out["decode_step"] = {
        "us_per_token_layer": round(ms3 * 1e3, 3), "bytes_per_token_layer": nbytes2,
        "GB_s": round(nbytes2 / (ms3 * 1e-3) / 1e9, 1), "pct_of_hbm_peak": round(nbytes2 / (ms3 * 1e-3) / 1e9 / 80, 1),
        "launches": 4, "host_syncs": 0, "includes": includes,
        "separate_launches": {"us_per_token_layer": round(ms2 * 1e3, 3), "launches": 8},
        "bit_identical_to_separate": bool(torch.equal(yf.view(torch.int16), yy.view(torch.int16)))}
    return out


LAYER_70B = [(8192, 8192), (1024, 8192), (1024, 8192), (8192, 8192), (28672, 8192), (28672, 8192), (8192, 28672)]


def bench_70b_layer(dev, layers_rotated: int = 2, reps: int = 20):
    """Q4_0 LLaMA-70B decoder layer (7 GEMVs, 481 MB of weights) at batch
    1, 2, 4, 8, rotating over `layers_rotated` distinct layers."""
    import torch

    from gdsllm_amd import synthetic as syn

    gen = torch.Generator(device=dev).manual_seed(1004)
    layers = [[syn.q4_0_weights(m, k, gen) for m, k in LAYER_70B] for _ in range(layers_rotated)]
    wbytes = sum(m * (k // 32) * 18 for m, k in LAYER_70B)
    out = {}
    for B in (1, 2, 4, 8):
        xs = {k: syn.activations(B, k, gen) for k in (8192, 28672)}
        ys = {m: torch.empty(B, m, dtype=torch.float16, device=dev) for m in (1024, 8192, 28672)}

        def run():
            for lw in layers:
                for w, (m, k) in zip(lw, LAYER_70B):
                    _gemv_call("q4_0", w, xs[k], ys[m], m, k, B)

        ms = _replay_ms(run, reps) / layers_rotated
        nbytes = wbytes + sum(B * (2 * k + 2 * m) for m, k in LAYER_70B)
        out[f"b{B}"] = {"us_per_layer": round(ms * 1e3, 3), "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "pct_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / 80, 1), "bytes_per_layer": nbytes}
    out["layers_rotated"] = layers_rotated
    return out


def bench_prefill(dev, layers, lm_head, tokens: int = 512, reps: int = 3):
    """LLaMA-7B Q4_0 prefill chunk of 512 tokens through the MFMA dequant-GEMM:
    7 projections per layer x 32 layers + lm_head, one graph per chunk."""
    import torch

    from gdsllm_amd import capi, check
    from gdsllm_amd import synthetic as syn

    gen = torch.Generator(device=dev).manual_seed(1005)
    xs = {k: syn.activations(tokens, k, gen) for k in (4096, 11008)}
    ys = {m: torch.empty(tokens, m, dtype=torch.float16, device=dev) for m in (4096, 11008, 32000)}

    def gemm(w, m, k):
        check(capi().gdsllm_dequant_gemm_q4_0(w.data_ptr(), xs[k].data_ptr(), ys[m].data_ptr(), m, k, tokens, k, m,
                                              torch.cuda.current_stream().cuda_stream))

    def run():
        for lw in layers:
            for w, (m, k) in zip(lw, LAYER_SHAPES):
                gemm(w, m, k)
        gemm(lm_head, *LM_HEAD)

    ms = _replay_ms(run, reps, warm=1)
    flops = 2 * tokens * (N_LAYERS * sum(m * k for m, k in LAYER_SHAPES) + LM_HEAD[0] * LM_HEAD[1])
    return {"ms_per_chunk": round(ms, 3), "tokens": tokens, "tok_s": round(tokens / (ms * 1e-3), 1),
            "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1), "flop_per_chunk": flops,
            "pct_of_fp16_dense_peak": round(flops / (ms * 1e-3) / 1e12 / 25, 1)}


def bench_load(dev, layers: int = 2, reps: int = 3, tokens: int = 512, emb_reps: int = 20):
    """Converted LLaMA-7B Q4_0 directory (files written first, so they are page-
    cache resident): one layer file (113 MB) into HBM through
    ModelWeights.load_layer (pread -> pinned staging -> hipMemcpyAsync), and the
    embedding lookup of a 512-token chunk from the 32000 x 4096 Q4_0 table:
    row gather against the reference's whole-table dequant + F.embedding."""
    import shutil
    import tempfile

    import torch
    import torch.nn.functional as F

    from gdsllm_amd.runtime import ext
    from gdsllm_amd.runtime.scheduler import _embed_tokens
    from gdsllm_amd.runtime.torch_bridge import ModelWeights
    from gdsllm_amd.synthetic_model import write_llama

    d = tempfile.mkdtemp(prefix="gdsllm_load_", dir="/dev/shm" if os.path.isdir("/dev/shm") else None)
    try:
        write_llama(d, "q4_0", layers=layers, hidden=4096, ffn=11008, vocab=32000, seed=1006)
        mw = ModelWeights(d)
        mw.init_gds()
        times = []
        for _ in range(reps):
            for i in range(layers):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                tensors, handle = mw.load_layer(i)
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
                del tensors, handle
        times.sort()
        size = mw.layers[0].size_bytes
        emb, emb_handle = mw.load_special("embed_tokens")
        w = emb["model.embed_tokens.weight"]
        ids = torch.randint(0, 32000, (1, tokens), device=dev, generator=torch.Generator(device=dev).manual_seed(7))

        def timed(fn):
            fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(emb_reps):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) * 1e3 / emb_reps

        gather_us = timed(lambda: _embed_tokens(ids, emb))
        full_us = timed(lambda: F.embedding(ids, ext().dequant_gguf(w["buffer"], w["shape"], "q4_0", w["offset"])))
        return {"layer_file_bytes": size, "load_ms_median": round(times[len(times) // 2] * 1e3, 3),
                "load_GB_s": round(size / times[len(times) // 2] / 1e9, 2),
                "embed_512_gather_us": round(gather_us, 2), "embed_512_full_table_dequant_us": round(full_us, 2),
                "source": "page-cache resident files (tmpfs when /dev/shm exists)"}
    finally:
        shutil.rmtree(d, ignore_errors=True)


def cpu_baseline(weights_dev, x_dev, y_gpu, seconds: float):
    """Oracle-side torch restatement of dequant -> F.linear (fp32) on the host
    cores, timed over a bounded number of calls; also checks the GPU result."""
    import numpy as np
    import torch

    from oracle import cpu_baseline as cb
    from oracle import quant as oq

    w = weights_dev.cpu()
    x = x_dev.cpu()
    y_cpu = cb.q4_0_gemv(w, x, M0, K0)  # warm-up
    calls, t0 = 0, time.perf_counter()
    while True:
        cb.q4_0_gemv(w, x, M0, K0)
        calls += 1
        el = time.perf_counter() - t0
        if (el >= seconds and calls >= 3) or calls >= 200:
            break
    per_call = el / calls
    deq = cb.dequant_q4_0(w).view(M0, K0).numpy()
    xn = x.numpy()
    ref, norms = oq.gemv(deq, xn), oq.row_norms(deq, xn)
    rel, mx = oq.gemv_errors(y_gpu.cpu().numpy().astype(np.float64), ref, norms)
    rel_c, _ = oq.gemv_errors(y_cpu.numpy().astype(np.float64), ref, norms)
    return {
        "value": round(ALGO_BYTES_CFG0 / per_call / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(per_call * 1e6, 1),
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{calls} calls of the 11008x4096 Q4_0 b=1 GEMV (bit-exact torch dequant + fp32 F.linear), "
                  f"one weight copy, {el:.1f} s",
    }, {"gpu_rel_l2": rel, "gpu_max_norm": mx, "cpu_rel_l2": rel_c,
        "ok": bool(rel <= oq.GEMV_REL_L2 and mx <= oq.GEMV_MAX_NORM)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=6400, help="timed GEMV launches")
    ap.add_argument("--warmup", type=int, default=640, help="untimed GEMV launches")
    ap.add_argument("--copies", type=int, default=16, help="distinct weight copies rotated over")
    ap.add_argument("--chunk", type=int, default=64, help="launches per captured graph")
    ap.add_argument("--sweep-tokens", type=int, default=100, help="timed 7B decode-sweep tokens (0 = skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--configs", default="q8,moe,70b,prefill,load,int8",
                    help="comma list of extra workloads to measure: q8 (Q8_0 7B layer), moe (top-10 expert "
                         "gather), 70b (Q4_0 70B layer, B=1..8), prefill (512-token MFMA GEMM), load (7B layer "
                         "file -> HBM, embedding row gather), int8 (per-column int8 7B layer); '' = none")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the GEMV would shard by output rows; see the design notes).", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0 or args.copies < 1 or args.chunk < 1:
        print("bench.py: --steps >= 1, --warmup >= 0, --copies >= 1, --chunk >= 1", file=sys.stderr)
        return 2

    import torch

    _ensure_built()
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")

    g = bench_gemv(args, dev)
    ms_total = g["ms"]
    us_per_call = ms_total * 1e3 / args.steps
    gbs = ALGO_BYTES_CFG0 / (us_per_call * 1e-6) / 1e9
    print(f"# q4_0 gemv 11008x4096 b=1: {us_per_call:.3f} us/call, {gbs:.1f} GB/s "
          f"({100 * gbs / HBM_PEAK_GBS:.1f}% of {HBM_PEAK_GBS:.0f})", file=sys.stderr, flush=True)

    sweep, sweep_weights = None, None
    if args.sweep_tokens > 0:
        ms_tok, ms_unf, sweep_weights = bench_decode_sweep(args, dev)
        sb = sweep_bytes()
        sweep = {"tok_s": round(1e3 / ms_tok, 1), "ms_per_token": round(ms_tok, 4), "launches_per_token": 129,
                 "bytes_per_token": sb, "GB_s": round(sb / (ms_tok * 1e-3) / 1e9, 1),
                 "fusion": "q/k/v grouped launch; gate+up+SiLU launch writing h; o, down, lm_head single",
                 "unfused": {"tok_s": round(1e3 / ms_unf, 1), "ms_per_token": round(ms_unf, 4),
                             "launches_per_token": 225, "GB_s": round(sb / (ms_unf * 1e-3) / 1e9, 1)}}
        print(f"# 7B decode sweep: {ms_tok:.4f} ms/token, {sweep['tok_s']} tok/s, {sweep['GB_s']} GB/s "
              f"(unfused 225 launches: {sweep['unfused']['tok_s']} tok/s)", file=sys.stderr, flush=True)

    wanted = {c.strip() for c in args.configs.split(",") if c.strip()}
    unknown = wanted - {"q8", "moe", "70b", "prefill", "load", "int8"}
    if unknown:
        print(f"bench.py: unknown --configs entries {sorted(unknown)}", file=sys.stderr)
        return 2
    configs = {}
    runs = [("q8", "q8_0_layer_7b_b1", lambda: bench_q8_layer(dev)),
            ("moe", "moe_affine_q4_top10", lambda: bench_moe(dev)),
            ("70b", "q4_0_layer_70b", lambda: bench_70b_layer(dev)),
            ("prefill", "prefill_7b_512",
             lambda: bench_prefill(dev, *sweep_weights) if sweep_weights is not None else None),
            ("load", "load_7b_q4_0", lambda: bench_load(dev)),
            ("int8", "int8_layer_7b_b1", lambda: bench_int8_layer(dev))]
    for key, name, fn in runs:
        if key in wanted:
            res = fn()
            if res is not None:
                configs[name] = res
                print(f"# {name}: {res}", file=sys.stderr, flush=True)
            torch.cuda.empty_cache()
    sweep_weights = None

    cpu, parity = None, None
    if args.cpu_seconds > 0:
        cpu, parity = cpu_baseline(g["weights0"], g["x"], g["y0"], args.cpu_seconds)
        print(f"# cpu baseline: {cpu['us_per_call']} us/call on {cpu['cores']} threads; parity {parity}",
              file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_total / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0->fp16, fp32 acc",
        "data": "synthetic",
        "config": {"workload": "GGUF Q4_0 fused dequant+GEMV, W 11008x4096 (LLaMA-7B gate_proj), batch 1",
                   "weight_copies_rotated": args.copies, "graph_chunk": args.chunk,
                   "algorithmic_bytes_per_step": ALGO_BYTES_CFG0},
        "us_per_call": round(us_per_call, 3),
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "decode_sweep_7b": sweep,
        "configs": configs or None,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    if parity is not None and not parity["ok"]:
        print("bench.py: GPU result does not match the oracle", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
