#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matvec hot path (one GPU).

Headline workload: GGUF Q4_0 fused dequant+GEMV at the LLaMA-7B gate_proj
shape, W = 11008 x 4096 (Q4_0 blocks: fp16 d ~ U(0.005, 0.02), uniform 4-bit
codes), x fp16 [1, 4096] ~ N(0, 1), y fp16 [1, 11008], fp32 accumulation.
Weights rotate over `--copies` distinct HBM-resident copies (16 x 25.4 MB =
406 MB, more than the 256 MB Infinity Cache), so every launch streams its
weights from HBM.  One step = one pass over the copies: `--copies` fused GEMV
launches through the C ABI, one per copy (a step count of 20 times 320
launches, so the timed region is not dominated by the fixed cost of
starting it).  The K timed steps are replayed from HIP graphs of `--chunk`
launches (rounded up to whole passes), bracketed by HIP events on the
launch stream; `value` is the per-launch rate.

Also reported (same JSON line): the LLaMA-7B Q4_0 decode weight sweep, all 32
layers resident (7 projection GEMVs per layer + lm_head 32000 x 4096, one HIP
graph per token) as tokens/s, fused (q/k/v grouped, gate+up+SiLU in one
launch: 129 launches) and unfused (225 launches), the fused sweep at batch 4
and 8 (tokens/s over the batch), and the CPU baseline (torch restatement of
dequant -> F.linear in fp32 on the host cores).

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


def _gpu_delay() -> None:
    """Keeps the GPU busy for a few milliseconds so that everything enqueued
    after it (the start event, the graph replays, the end event) is queued
    before the GPU reaches the start event: the timed region then holds GPU
    time only, not host enqueue latency."""
    import torch

    torch.cuda._sleep(5_000_000)


def _capture(fn):
    import torch

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def bench_gemv(args, dev):
    """Exactly `steps` passes over the weight copies (steps x copies
    launches), all replayed from HIP graphs: L // c replays of a graph of
    c = min(L, chunk rounded up to whole passes) launches, then one graph of
    the remaining L % c launches, L the launch count (whole passes, so the
    rotation runs on across graphs)."""
    import torch

    from gdsllm_amd import synthetic as syn

    gemv = Q4Gemv()
    copies = [syn.q4_0_weights(M0, K0, torch.Generator(device=dev).manual_seed(1000 + i)) for i in range(args.copies)]
    x = syn.activations(1, K0, torch.Generator(device=dev).manual_seed(999))
    ys = torch.empty(args.copies, M0, dtype=torch.float16, device=dev)
    n = args.copies

    for i in range(max(args.warmup, 1) * n):
        gemv(copies[i % n], x, ys[i % n], M0, K0)
    torch.cuda.synchronize()

    K = args.steps * n
    c = min(K, -(-args.chunk // n) * n)
    reps, rem = divmod(K, c)

    def launches(count):
        return lambda: [gemv(copies[i % n], x, ys[i % n], M0, K0) for i in range(count)]

    full = _capture(launches(c))
    tail = _capture(launches(rem)) if rem else None
    full.replay()
    if tail is not None:
        tail.replay()
    torch.cuda.synchronize()

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _gpu_delay()
    start.record()
    for _ in range(reps):
        full.replay()
    if tail is not None:
        tail.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    return {"ms": ms, "launches_timed": reps * c + rem, "graph_launches": c, "weights0": copies[0], "x": x,
            "y0": ys[0].clone()}


def bench_decode_sweep(args, dev):
    """LLaMA-7B Q4_0 decode weight sweep, one HIP graph per token, timed two ways.

    unfused: 225 single GEMV launches (7 per layer + lm_head), every GEMV
    reading a synthetic x of its in_dim.
    fused: the runtime's DecodeSweep, 129 launches with the reference layer's
    data flow (llama.py:212-256): q/k/v in one grouped launch on the attention
    input, o on the attention output, gate+up+SiLU in one launch writing h,
    down on that h; lm_head last.  Same weights, same 224 + 1 projections.
    The fused sweep is also timed at batch 4 and 8 (one decode step of B
    sequences per replay).  Returns (ms fused, ms unfused, weights, {B: ms per
    step})."""
    import torch

    from gdsllm_amd import synthetic as syn

    gemv = Q4Gemv()
    gen = torch.Generator(device=dev).manual_seed(2004)
    layers = [[syn.q4_0_weights(m, k, gen) for m, k in LAYER_SHAPES] for _ in range(N_LAYERS)]
    lm_head = syn.q4_0_weights(*LM_HEAD, gen)
    xs = {k: syn.activations(1, k, gen) for k in (4096, 11008)}
    ys = {m: torch.empty(1, m, dtype=torch.float16, device=dev) for m in (4096, 11008, 32000)}

    def token_unfused():
        for lw in layers:
            for w, (m, k) in zip(lw, LAYER_SHAPES):
                gemv(w, xs[k], ys[m], m, k)
        gemv(lm_head, xs[LM_HEAD[1]], ys[LM_HEAD[0]], *LM_HEAD)

    # fused: the runtime's decode-step driver (one HIP graph per token)
    from gdsllm_amd.runtime import ext
    from gdsllm_amd.runtime.scheduler import DecodeSweep

    names = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
             "mlp.up_proj", "mlp.down_proj")

    def entry(w, m, k):
        return {"buffer": ext().GdsBufferHandle.from_tensor(w), "shape": [m, k], "gguf_type": "q4_0", "offset": 0}

    layer_entries = [{f"{n}.weight": entry(w, m, k) for n, w, (m, k) in zip(names, lw, LAYER_SHAPES)} for lw in layers]
    head_entry = entry(lm_head, *LM_HEAD)
    sweep = DecodeSweep(layer_entries, head_entry, batch=1, device=dev)
    for b in [*sweep.attn_in, *sweep.attn_out, *sweep.mlp_in, sweep.final_in]:
        b.copy_(syn.activations(1, b.shape[1], gen))
    sweep.run()
    torch.cuda.synchronize()

    ms_unfused = _replay_ms(token_unfused, args.sweep_tokens)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        sweep.run()
    torch.cuda.synchronize()
    _gpu_delay()
    start.record()
    for _ in range(args.sweep_tokens):
        sweep.run()
    end.record()
    torch.cuda.synchronize()
    ms_fused = start.elapsed_time(end) / args.sweep_tokens

    # the same weights at batch 4 and 8 (one decode step of B sequences per
    # replay: grouped q/k/v and gate/up/SiLU on the batched kernel)
    batched = {}
    for B in (4, 8):
        sw = DecodeSweep(layer_entries, head_entry, batch=B, device=dev)
        for b in [*sw.attn_in, *sw.attn_out, *sw.mlp_in, sw.final_in]:
            b.copy_(syn.activations(B, b.shape[1], gen))
        for _ in range(3):
            sw.run()
        torch.cuda.synchronize()
        _gpu_delay()
        start.record()
        for _ in range(args.sweep_tokens):
            sw.run()
        end.record()
        torch.cuda.synchronize()
        batched[B] = start.elapsed_time(end) / args.sweep_tokens
        del sw
    return ms_fused, ms_unfused, (layers, lm_head), batched


_EAGER = False  # --profile-case: launch eagerly instead of replaying graphs


def _replay_ms(capture, reps: int, warm: int = 3) -> float:
    """Captures `capture()` (launches on the current stream) into a HIP graph
    once, replays it `warm` times untimed, then `reps` times between HIP
    events on the launch stream; returns ms per replay.  With _EAGER set,
    `capture()` itself runs once untimed and `reps` times timed, so a profiler
    sees plain kernel dispatches."""
    import torch

    capture()
    torch.cuda.synchronize()
    if _EAGER:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            capture()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps
    graph = _capture(capture)
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _gpu_delay()
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
    `layers_rotated` distinct layers (3 x 215 MB > the 256 MB Infinity Cache);
    also with the decode-step fusions (4 launches per layer)."""
    import ctypes

    import torch

    from gdsllm_amd import capi, check
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

    # q/k/v in one grouped launch, o, gate/up/SiLU writing h, down on h
    lib = capi()
    h = torch.empty(1, 11008, dtype=torch.float16, device=dev)
    yq, yk, yv = (torch.empty(1, 4096, dtype=torch.float16, device=dev) for _ in range(3))
    dims = (ctypes.c_int64 * 3)(4096, 4096, 4096)
    outs = (ctypes.c_void_p * 3)(yq.data_ptr(), yk.data_ptr(), yv.data_ptr())
    groups = [(ctypes.c_void_p * 3)(lw[0].data_ptr(), lw[1].data_ptr(), lw[2].data_ptr()) for lw in layers]

    def run_fused():
        st = torch.cuda.current_stream().cuda_stream
        for lw, grp in zip(layers, groups):
            check(lib.gdsllm_fused_q8_0_gemv_group(3, grp, outs, dims, xs[4096].data_ptr(), 4096, 1, 4096, st))
            _gemv_call("q8_0", lw[3], xs[4096], ys[4096], 4096, 4096, 1)
            check(lib.gdsllm_fused_q8_0_gate_up_silu(lw[4].data_ptr(), lw[5].data_ptr(), xs[4096].data_ptr(),
                                                     h.data_ptr(), 11008, 4096, 1, 4096, 11008, st))
            _gemv_call("q8_0", lw[6], h, ys[4096], 4096, 11008, 1)

    msf = _replay_ms(run_fused, reps) / layers_rotated
    fbytes = sum(m * (k // 32) * 34 for m, k in LAYER_SHAPES) + 2 * (4096 + 3 * 4096 + 2 * 4096 + 4096 + 11008 +
                                                                    11008 + 4096)
    return {"us_per_layer": round(ms * 1e3, 3), "bytes_per_layer": nbytes,
            "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1), "pct_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / 80, 1),
            "layers_rotated": layers_rotated,
            "fused_4_launches": {"us_per_layer": round(msf * 1e3, 3), "bytes_per_layer": fbytes,
                                 "GB_s": round(fbytes / (msf * 1e-3) / 1e9, 1),
                                 "pct_of_hbm_peak": round(fbytes / (msf * 1e-3) / 1e9 / 80, 1)}}


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


def bench_moe(dev, calls: int = 64, reps: int = 20, decode_step: bool = True):
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
    if not decode_step:
        return out

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

    # The same step with the routing folded in (gdsllm_moe_step_routed_affine_q4):
    # router GEMV, then the gate/up launch whose waves take the top-k
    # themselves, then down: 3 launches.
    wsr_bytes = capi().gdsllm_moe_step_routed_workspace_size(k, Fd, E)
    wsr = torch.empty(wsr_bytes, dtype=torch.uint8, device=dev)
    ridx3 = torch.empty(calls, k, dtype=torch.int32, device=dev)
    rw3 = torch.empty(calls, k, dtype=torch.float16, device=dev)
    y3 = torch.empty(calls, H, dtype=torch.float16, device=dev)

    def step_routed():
        s = torch.cuda.current_stream().cuda_stream
        for i in range(calls):
            sg_, su_, sd_ = sh_one[i]
            check(capi().gdsllm_moe_step_routed_affine_q4(router[i].data_ptr(), ctypes.byref(gate), ctypes.byref(up),
                                                          ctypes.byref(down), ctypes.byref(sg_), ctypes.byref(su_),
                                                          ctypes.byref(sd_), xs[i].data_ptr(), k,
                                                          sgate[i].data_ptr(), y3[i].data_ptr(), ridx3[i].data_ptr(),
                                                          rw3[i].data_ptr(), wsr.data_ptr(), wsr_bytes, s))

    ms4 = _replay_ms(step_routed, reps) / calls
    torch.cuda.synchronize()
    nbytes2 = E * H * 2 + (k + 1) * per_expert + H * 2 + 2 * H * 2
    includes = ("fp16 router GEMV 512x4096, top-k+softmax, top-10 gather, shared expert (ffn 1024), "
                "shared-gate GEMV, combine+clamp")
    out["decode_step"] = {
        "us_per_token_layer": round(ms3 * 1e3, 3), "bytes_per_token_layer": nbytes2,
        "GB_s": round(nbytes2 / (ms3 * 1e-3) / 1e9, 1), "pct_of_hbm_peak": round(nbytes2 / (ms3 * 1e-3) / 1e9 / 80, 1),
        "launches": 4, "host_syncs": 0, "includes": includes,
        "separate_launches": {"us_per_token_layer": round(ms2 * 1e3, 3), "launches": 8},
        "bit_identical_to_separate": bool(torch.equal(yf.view(torch.int16), yy.view(torch.int16))),
        "routed": {"us_per_token_layer": round(ms4 * 1e3, 3), "launches": 3,
                   "GB_s": round(nbytes2 / (ms4 * 1e-3) / 1e9, 1),
                   "pct_of_hbm_peak": round(nbytes2 / (ms4 * 1e-3) / 1e9 / 80, 1),
                   "bit_identical_to_fused": bool(torch.equal(y3.view(torch.int16), yf.view(torch.int16)) and
                                                  torch.equal(ridx3, ridx) and
                                                  torch.equal(rw3.view(torch.int16), rw.view(torch.int16)))}}
    return out


# bytes of the top-10 affine-Q4 gather's two launches (512 experts, hidden
# 4096, ffn 1024, group 64): gate and up rows of 10 experts with their scales
# and biases, plus x; down rows of 10 experts with scales and biases, plus h
MOE_GATE_UP_BYTES = 10 * 2 * (1024 * 4096 // 2 + 2 * 1024 * (4096 // 64) * 2) + 4096 * 2
MOE_DOWN_BYTES = 10 * (4096 * 1024 // 2 + 2 * 4096 * (1024 // 64) * 2) + 10 * 1024 * 2


def bench_ceiling(dev, copies: int = 16, calls: int = 64, reps: int = 10):
    """What one launch can do on this device, for the headline's size:
    a plain read of 25,392,640 B (the headline call's algorithmic bytes,
    rotating over `copies` slices of one 406 MB buffer, as the headline
    rotates its weights) at several grid sizes, one launch reading all 406 MB,
    the time per launch of an empty kernel, and plain reads of the expert
    gather's two launches' bytes, all back to back in HIP graphs."""
    import torch

    from gdsllm_amd import capi, check

    lib = capi()
    nb = ALGO_BYTES_CFG0
    buf = torch.randint(0, 256, (copies * nb,), dtype=torch.uint8, device=dev,
                        generator=torch.Generator(device=dev).manual_seed(1010))
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    key = 0x9E3779B9

    def read_ms(nbytes, wg, n, rot):
        def run():
            st = torch.cuda.current_stream().cuda_stream
            for i in range(n):
                check(lib.gdsllm_read_stream(buf.data_ptr() + (i % rot) * nbytes, nbytes, wg, key, sink.data_ptr(),
                                             st))
        return _replay_ms(run, reps) / n

    by_wg = {wg: read_ms(nb, wg, calls, copies) * 1e3 for wg in (1024, 2048, 4096, 8192)}
    best_wg = min(by_wg, key=by_wg.get)
    us = by_wg[best_wg]
    whole = {wg: read_ms(copies * nb, wg, 4, 1) * 1e3 for wg in (4096, 16384, 65536)}
    best_whole = min(whole, key=whole.get)

    def empty_us(wg):
        def run():
            st = torch.cuda.current_stream().cuda_stream
            for _ in range(calls):
                check(lib.gdsllm_empty_launch(wg, st))
        return _replay_ms(run, reps) / calls * 1e3

    # The top-10 expert gather's two launches as plain reads of their bytes
    # (gate/up rows of 10 experts + x; down rows + h), each rotating over
    # slices of the same buffer; a plain read over the same bytes scattered at
    # fresh expert places in the 3.6 GB pool measured within 4% of this.
    moe = {}
    for name, nbytes in (("gate_up", MOE_GATE_UP_BYTES), ("down", MOE_DOWN_BYTES)):
        rot = (copies * nb) // nbytes
        t = {wg: read_ms(nbytes, wg, calls, rot) * 1e3 for wg in (2048, 4096, 8192, 16384)}
        w = min(t, key=t.get)
        moe[name] = {"bytes": nbytes, "us": round(t[w], 3), "GB_s": round(nbytes / (t[w] * 1e-6) / 1e9, 1),
                     "workgroups": w}
    moe["two_launches_us"] = round(moe["gate_up"]["us"] + moe["down"]["us"], 3)

    return {"read_25MB": {"bytes": nb, "us": round(us, 3), "GB_s": round(nb / (us * 1e-6) / 1e9, 1),
                          "frac_of_peak": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "workgroups": best_wg,
                          "us_by_workgroups": {str(k): round(v, 3) for k, v in by_wg.items()}},
            "read_406MB_one_launch": {"bytes": copies * nb, "us": round(whole[best_whole], 2),
                                      "GB_s": round(copies * nb / (whole[best_whole] * 1e-6) / 1e9, 1),
                                      "workgroups": best_whole},
            "empty_launch_us": {"256_workgroups": round(empty_us(256), 3), "2048_workgroups": round(empty_us(2048), 3)},
            "read_moe_gather_bytes": moe,
            "method": "16-byte non-temporal loads, 256-thread workgroups, grid-stride, 4 loads in flight per thread; "
                      "graph replays between HIP events"}


LAYER_70B = [(8192, 8192), (1024, 8192), (1024, 8192), (8192, 8192), (28672, 8192), (28672, 8192), (8192, 28672)]


def bench_70b_layer(dev, layers_rotated: int = 2, reps: int = 20):
    """Q4_0 LLaMA-70B decoder layer (7 GEMVs, 481 MB of weights) at batch
    1, 2, 4, 8, rotating over `layers_rotated` distinct layers, as 7 launches
    and with the decode-step fusions (4 launches per layer)."""
    import ctypes

    import torch

    from gdsllm_amd import capi, check
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
        # the same layer with the decode-step fusions of the 7B sweep:
        # q/k/v in one grouped launch, gate/up/SiLU in one launch writing
        # h, down on h: 4 launches instead of 7
        h = torch.empty(B, 28672, dtype=torch.float16, device=dev)
        lib = capi()
        yq, yk, yv = (torch.empty(B, m, dtype=torch.float16, device=dev) for m in (8192, 1024, 1024))
        dims = (ctypes.c_int64 * 3)(8192, 1024, 1024)
        outs = (ctypes.c_void_p * 3)(yq.data_ptr(), yk.data_ptr(), yv.data_ptr())
        groups = [(ctypes.c_void_p * 3)(lw[0].data_ptr(), lw[1].data_ptr(), lw[2].data_ptr()) for lw in layers]

        def run_fused():
            st = torch.cuda.current_stream().cuda_stream
            for lw, grp in zip(layers, groups):
                check(lib.gdsllm_fused_q4_0_gemv_group(3, grp, outs, dims, xs[8192].data_ptr(), 8192, B, 8192, st))
                _gemv_call("q4_0", lw[3], xs[8192], ys[8192], 8192, 8192, B)
                check(lib.gdsllm_fused_q4_0_gate_up_silu(lw[4].data_ptr(), lw[5].data_ptr(), xs[8192].data_ptr(),
                                                         h.data_ptr(), 28672, 8192, B, 8192, 28672, st))
                _gemv_call("q4_0", lw[6], h, ys[8192], 8192, 28672, B)

        msf = _replay_ms(run_fused, reps) / layers_rotated
        fbytes = wbytes + B * 2 * (8192 + (8192 + 1024 + 1024) + 2 * 8192 + 8192 + 28672 + 28672 + 8192)
        out[f"b{B}"]["fused_4_launches"] = {
            "us_per_layer": round(msf * 1e3, 3), "GB_s": round(fbytes / (msf * 1e-3) / 1e9, 1),
            "pct_of_hbm_peak": round(fbytes / (msf * 1e-3) / 1e9 / 80, 1), "bytes_per_layer": fbytes}
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

    # The same chunk with each layer's gate and up projections and the SiLU in
    # one launch (gdsllm_dequant_gemm_gate_up_silu_q4_0) writing h, the down
    # projection's input: 6 launches per layer, the MLP's real data flow.
    h = torch.empty(tokens, 11008, dtype=torch.float16, device=dev)

    def run_fused_mlp():
        st = torch.cuda.current_stream().cuda_stream
        for lw in layers:
            for w, (m, k) in zip(lw[:4], LAYER_SHAPES[:4]):
                gemm(w, m, k)
            check(capi().gdsllm_dequant_gemm_gate_up_silu_q4_0(lw[4].data_ptr(), lw[5].data_ptr(), xs[4096].data_ptr(),
                                                                h.data_ptr(), 11008, 4096, tokens, 4096, 11008, st))
            check(capi().gdsllm_dequant_gemm_q4_0(lw[6].data_ptr(), h.data_ptr(), ys[4096].data_ptr(), 4096, 11008,
                                                  tokens, 11008, 4096, st))
        gemm(lm_head, *LM_HEAD)

    ms_fused = _replay_ms(run_fused_mlp, reps, warm=1)

    # Per shape: the fused kernel against the reference's route, the bit-exact
    # dequant into an fp16 scratch matrix followed by the vendor GEMM
    # (hipBLASLt through torch.mm), runtime/llama.py:160-166.
    lib = capi()
    per_shape = {}
    shapes = [((4096, 4096), layers[0][0]), ((11008, 4096), layers[0][4]), ((4096, 11008), layers[0][6]),
              (LM_HEAD, lm_head)]
    for (m, k), w in shapes:
        wdq = torch.empty(m, k, dtype=torch.float16, device=dev)
        yr = torch.empty(tokens, m, dtype=torch.float16, device=dev)

        def fused():
            gemm(w, m, k)

        def dequant():
            check(lib.gdsllm_dequant_q4_0(w.data_ptr(), wdq.data_ptr(), m * k // 32,
                                          torch.cuda.current_stream().cuda_stream))

        def matmul():
            torch.mm(xs[k], wdq.t(), out=yr)

        def route():
            dequant()
            matmul()

        f_us, d_us, mm_us, r_us = (_replay_ms(fn, 20) * 1e3 for fn in (fused, dequant, matmul, route))
        fl = 2 * tokens * m * k
        per_shape[f"{m}x{k}"] = {"fused_us": round(f_us, 2), "fused_TFLOP_s": round(fl / (f_us * 1e-6) / 1e12, 1),
                                 "dequant_then_hipblaslt_us": round(r_us, 2), "dequant_us": round(d_us, 2),
                                 "hipblaslt_fp16_gemm_us": round(mm_us, 2), "fused_faster": bool(f_us < r_us)}
        del wdq, yr
    # The MLP input of a layer: gate and up projections and h = silu(g) * u.
    # Fused: one launch.  The reference's route: both projections as dequant +
    # vendor GEMM, then torch's F.silu and product on the fp16 outputs.
    m, k = LAYER_SHAPES[4]
    wg_, wu_ = layers[0][4], layers[0][5]
    wdq = torch.empty(m, k, dtype=torch.float16, device=dev)
    g_, u_ = (torch.empty(tokens, m, dtype=torch.float16, device=dev) for _ in range(2))

    def gate_up_fused():
        check(lib.gdsllm_dequant_gemm_gate_up_silu_q4_0(wg_.data_ptr(), wu_.data_ptr(), xs[k].data_ptr(), h.data_ptr(),
                                                        m, k, tokens, k, m, torch.cuda.current_stream().cuda_stream))

    def gate_up_route():
        for w, out in ((wg_, g_), (wu_, u_)):
            check(lib.gdsllm_dequant_q4_0(w.data_ptr(), wdq.data_ptr(), m * k // 32,
                                          torch.cuda.current_stream().cuda_stream))
            torch.mm(xs[k], wdq.t(), out=out)
        torch.nn.functional.silu(g_).mul_(u_)

    f_us, r_us = (_replay_ms(fn, 20) * 1e3 for fn in (gate_up_fused, gate_up_route))
    fl = 2 * 2 * tokens * m * k
    per_shape[f"gate_up_silu_{m}x{k}"] = {"fused_us": round(f_us, 2), "fused_TFLOP_s": round(fl / (f_us * 1e-6) / 1e12, 1),
                                          "dequant_then_hipblaslt_silu_us": round(r_us, 2),
                                          "fused_faster": bool(f_us < r_us)}
    del wdq, g_, u_
    return {"ms_per_chunk": round(ms, 3), "tokens": tokens, "tok_s": round(tokens / (ms * 1e-3), 1),
            "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1), "flop_per_chunk": flops,
            "pct_of_fp16_dense_peak": round(flops / (ms * 1e-3) / 1e12 / 25, 1), "launches_per_layer": 7,
            "fused_gate_up_silu": {"ms_per_chunk": round(ms_fused, 3), "tok_s": round(tokens / (ms_fused * 1e-3), 1),
                                   "TFLOP_s": round(flops / (ms_fused * 1e-3) / 1e12, 1),
                                   "pct_of_fp16_dense_peak": round(flops / (ms_fused * 1e-3) / 1e12 / 25, 1),
                                   "launches_per_layer": 6, "writes": "h = silu(gate x) * (up x), as the MLP uses it"},
            "per_shape": per_shape}


def bench_prefill_formats(dev, tokens: int = 512, reps: int = 20):
    """Q8_0 and affine-Q4 (group 64) prefill on the MFMA dequant-GEMM at the
    LLaMA-7B projection shapes with a 512-token chunk, per shape against the
    reference's route: the dequant kernel into an fp16 scratch matrix, then the
    vendor fp16 GEMM (hipBLASLt through torch.mm), runtime/llama.py:160-166 and
    runtime/qwen_moe.py:69-73."""
    import torch

    from gdsllm_amd import capi, check
    from gdsllm_amd import synthetic as syn

    lib = capi()
    gen = torch.Generator(device=dev).manual_seed(1007)
    xs = {k: syn.activations(tokens, k, gen) for k in (4096, 11008)}
    out = {}
    layer_fused = {"q8_0": 0.0, "affine_g64": 0.0}
    layer_route = {"q8_0": 0.0, "affine_g64": 0.0}
    for m, k in sorted(set(LAYER_SHAPES)):
        n_in_layer = LAYER_SHAPES.count((m, k))
        y = torch.empty(tokens, m, dtype=torch.float16, device=dev)
        wdq = torch.empty(m, k, dtype=torch.float16, device=dev)
        w8 = syn.q8_0_weights(m, k, gen)
        aw, asc, ab = syn.affine_q4_weights([m, k], 64, gen)
        st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
        runs = {
            "q8_0": (lambda: check(lib.gdsllm_dequant_gemm_q8_0(w8.data_ptr(), xs[k].data_ptr(), y.data_ptr(), m, k,
                                                                 tokens, k, m, st())),
                     lambda: check(lib.gdsllm_dequant_q8_0(w8.data_ptr(), wdq.data_ptr(), m * k // 32, st()))),
            "affine_g64": (lambda: check(lib.gdsllm_dequant_gemm_affine_q4(aw.data_ptr(), asc.data_ptr(), ab.data_ptr(),
                                                                           xs[k].data_ptr(), y.data_ptr(), m, k, 64,
                                                                           tokens, k, m, st())),
                           lambda: check(lib.gdsllm_dequant_affine_q4(aw.data_ptr(), asc.data_ptr(), ab.data_ptr(),
                                                                      wdq.data_ptr(), m * k, k, 64, st()))),
        }
        mm_us = _replay_ms(lambda: torch.mm(xs[k], wdq.t(), out=y), reps) * 1e3
        fl = 2 * tokens * m * k
        for fmt, (fused, dq) in runs.items():
            f_us = _replay_ms(fused, reps) * 1e3
            d_us = _replay_ms(dq, reps) * 1e3
            r_us = _replay_ms(lambda: (dq(), torch.mm(xs[k], wdq.t(), out=y)), reps) * 1e3
            out.setdefault(fmt, {})[f"{m}x{k}"] = {
                "fused_us": round(f_us, 2), "fused_TFLOP_s": round(fl / (f_us * 1e-6) / 1e12, 1),
                "dequant_then_hipblaslt_us": round(r_us, 2), "dequant_us": round(d_us, 2),
                "hipblaslt_fp16_gemm_us": round(mm_us, 2), "fused_faster": bool(f_us < r_us)}
            layer_fused[fmt] += n_in_layer * f_us
            layer_route[fmt] += n_in_layer * r_us
        del w8, aw, asc, ab, wdq, y
    for fmt in out:
        out[fmt]["layer_7b_512_tokens"] = {"fused_us": round(layer_fused[fmt], 1),
                                           "dequant_then_hipblaslt_us": round(layer_route[fmt], 1)}
    return out


def bench_moe_prefill(dev, tokens: int = 512, reps: int = 5, reference: bool = True):
    """Routed-expert MLP of a 512-token prefill chunk over the resident
    512-expert affine-Q4 pool (hidden 4096, ffn 1024, group 64, top-10, random
    distinct picks per token): the grouped MFMA path (4 launches, no host
    sync) against the reference's route for the same chunk, the per-expert loop
    of runtime/qwen_moe.py:475-492 (host sync per slot, dequant of each expert's
    three matrices, three fp16 GEMMs, weighted scatter-add)."""
    import ctypes

    import torch

    from gdsllm_amd import AffineExperts, capi, check
    from gdsllm_amd import synthetic as syn

    E, H, Fd, g, k = 512, 4096, 1024, 64, 10
    gen = torch.Generator(device=dev).manual_seed(1008)
    pools = [syn.affine_q4_weights([E, Fd, H], g, gen), syn.affine_q4_weights([E, Fd, H], g, gen),
             syn.affine_q4_weights([E, H, Fd], g, gen)]

    def experts(p):
        w, sc, bi = p
        e, n, kw = w.shape
        kk = kw * 8
        return AffineExperts(w.data_ptr(), sc.data_ptr(), bi.data_ptr(), n * kw * 4, n * (kk // g) * 2,
                             n * (kk // g) * 2, e, n, kk, g)

    gate, up, down = (experts(p) for p in pools)
    cg = torch.Generator().manual_seed(1009)
    idx = torch.stack([torch.randperm(E, generator=cg)[:k] for _ in range(tokens)]).to(torch.int32).to(dev)
    wts = torch.softmax(torch.randn(tokens, k, generator=cg), -1).to(torch.float16).to(dev)
    x = syn.activations(tokens, H, gen)
    y = torch.empty(tokens, H, dtype=torch.float16, device=dev)
    lib = capi()
    ws_bytes = lib.gdsllm_moe_prefill_workspace_size(tokens, k, Fd, H, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

    def run():
        check(lib.gdsllm_moe_prefill_affine_q4(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down), x.data_ptr(),
                                               H, idx.data_ptr(), wts.data_ptr(), tokens, k, y.data_ptr(), H,
                                               ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream))

    ms = _replay_ms(run, reps)
    used = sorted(set(idx.reshape(-1).tolist()))
    per_expert = 3 * (Fd * H // 2 + 2 * 2 * Fd * H // g)
    wbytes = len(used) * per_expert
    flops = 2 * tokens * k * 3 * Fd * H
    res = {"us_per_chunk": round(ms * 1e3, 1), "tokens": tokens, "top_k": k, "experts_used": len(used),
           "weight_bytes": wbytes, "weight_GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
           "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1), "launches": 4, "host_syncs": 0}
    if not reference:
        return res

    # the reference's route, eagerly (it syncs to the host for every expert id)
    gd = torch.empty(Fd, H, dtype=torch.float16, device=dev)
    ud = torch.empty(Fd, H, dtype=torch.float16, device=dev)
    dd = torch.empty(H, Fd, dtype=torch.float16, device=dev)

    def deq(pool, e, out, n, kk):
        w, sc, bi = (t[e] for t in pool)
        check(lib.gdsllm_dequant_affine_q4(w.data_ptr(), sc.data_ptr(), bi.data_ptr(), out.data_ptr(), n * kk, kk, g,
                                           torch.cuda.current_stream().cuda_stream))

    def reference_route():
        eo = torch.zeros(tokens, H, dtype=torch.float16, device=dev)
        for j in range(k):
            ids = idx[:, j]
            for e in ids.unique().tolist():
                mask = ids == e
                xs_ = x[mask]
                deq(pools[0], e, gd, Fd, H)
                gate_o = torch.nn.functional.linear(xs_, gd)
                deq(pools[1], e, ud, Fd, H)
                up_o = torch.nn.functional.linear(xs_, ud)
                deq(pools[2], e, dd, H, Fd)
                down_o = torch.nn.functional.linear(torch.nn.functional.silu(gate_o) * up_o, dd)
                eo[mask] += wts[mask, j].unsqueeze(-1) * down_o
        return eo

    reference_route()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ref = reference_route()
    torch.cuda.synchronize()
    ref_ms = (time.perf_counter() - t0) * 1e3
    rel = float(torch.linalg.vector_norm((y.float() - ref.float())) / torch.linalg.vector_norm(ref.float()))
    res.update({"reference_route_ms": round(ref_ms, 2), "speedup_vs_reference_route": round(ref_ms / ms, 1),
                "rel_l2_vs_reference_route": rel})
    return res


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


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _median_s(fn, seconds: float, min_runs: int = 10, max_runs: int = 200, warm: int = 2) -> tuple[float, int]:
    """Median wall time of fn() over at least min_runs timed runs after `warm`
    untimed ones, continuing while the time budget lasts (at most max_runs)."""
    for _ in range(warm):
        fn()
    times, t_all = [], time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_all < seconds and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(weights_dev, x_dev, y_gpu, seconds: float):
    """Oracle-side torch restatement of the reference's route for one Q4_0
    projection (bit-exact dequant, then F.linear in fp32) on the host cores:
    dequant-only and dequant + matmul timed separately as medians of >= 10 runs
    after 2 warm-ups; also checks the GPU result against the oracle.  Threads:
    os.cpu_count(), limited to the cores this process may run on and to
    OMP_NUM_THREADS when set (the host share a one-GPU job is given)."""
    import numpy as np
    import torch

    from oracle import cpu_baseline as cb
    from oracle import quant as oq

    ncpu = os.cpu_count() or 1
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else ncpu
    threads = min(ncpu, allowed)
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, max(1, int(os.environ["OMP_NUM_THREADS"])))
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        w = weights_dev.cpu()
        x = x_dev.cpu()
        deq_s, deq_runs = _median_s(lambda: cb.dequant_q4_0(w), seconds / 3)
        tot_s, tot_runs = _median_s(lambda: cb.q4_0_gemv(w, x, M0, K0), seconds * 2 / 3)
        used = torch.get_num_threads()
        y_cpu = cb.q4_0_gemv(w, x, M0, K0)
    finally:
        torch.set_num_threads(prev)
    deq = cb.dequant_q4_0(w).view(M0, K0).numpy()
    xn = x.numpy()
    ref, norms = oq.gemv(deq, xn), oq.row_norms(deq, xn)
    rel, mx = oq.gemv_errors(y_gpu.cpu().numpy().astype(np.float64), ref, norms)
    rel_c, _ = oq.gemv_errors(y_cpu.numpy().astype(np.float64), ref, norms)
    return {
        "value": round(ALGO_BYTES_CFG0 / tot_s / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(tot_s * 1e6, 1),
        "dequant_only_us": round(deq_s * 1e6, 1),
        "cores": used,
        "os_cpu_count": ncpu,
        "cpus_allowed": allowed,
        "torch_threads": used,
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": f"11008x4096 Q4_0 b=1 GEMV (bit-exact torch dequant, then fp32 F.linear, fp16 out), one weight "
                  f"copy: median of {tot_runs} calls (dequant alone: median of {deq_runs}) after 2 warm-ups",
    }, {"gpu_rel_l2": rel, "gpu_max_norm": mx, "cpu_rel_l2": rel_c,
        "ok": bool(rel <= oq.GEMV_REL_L2 and mx <= oq.GEMV_MAX_NORM)}


CPU_ROW_CAP = 4096  # rows of one matrix timed on the host; the time scales linearly with rows


def _q8_bytes(m: int, k: int) -> int:
    return m * (k // 32) * 34


def cpu_baseline_configs(seconds_per_shape: float) -> dict:
    """The CPU restatement of the reference's route (bit-exact dequant, then
    F.linear in fp32; oracle/cpu_baseline.py) for the other workloads, each
    as dequant-only and dequant + GEMV time and GB/s over the GPU's
    algorithmic bytes: the Q8_0 LLaMA-7B layer (7 GEMVs), the top-10
    affine-Q4 expert gather (the reference's per-expert decode loop,
    runtime/qwen_moe.py:455-474), the Q4_0 LLaMA-70B layer at batch 1, and
    the LLaMA-7B Q4_0 decode sweep as the sum of its 224 + 1 GEMVs.  Each
    distinct matrix shape is timed once (median of >= 10 runs after 2
    warm-ups, at most CPU_ROW_CAP rows, the time scaled by rows / timed rows)
    and the shapes are summed with their counts.  Runs on the threads the
    caller has set."""
    import torch

    from gdsllm_amd import synthetic as syn
    from oracle import cpu_baseline as cb

    gen = torch.Generator().manual_seed(1050)
    cache = {}

    def shape_s(kind, m, k):
        if (kind, m, k) in cache:
            return cache[(kind, m, k)]
        r = min(m, CPU_ROW_CAP)
        x = syn.activations(1, k, gen)
        if kind == "q4_0":
            w = syn.q4_0_weights(r, k, gen)
            dq, tot = (lambda: cb.dequant_q4_0(w)), (lambda: cb.q4_0_gemv(w, x, r, k))
        else:
            w = syn.q8_0_weights(r, k, gen)
            dq, tot = (lambda: cb.dequant_q8_0(w)), (lambda: cb.q8_0_gemv(w, x, r, k))
        d_s, _ = _median_s(dq, seconds_per_shape / 3)
        t_s, _ = _median_s(tot, seconds_per_shape * 2 / 3)
        cache[(kind, m, k)] = (d_s * m / r, t_s * m / r)
        return cache[(kind, m, k)]

    def layer(kind, shapes):
        d = sum(shape_s(kind, m, k)[0] for m, k in shapes)
        t = sum(shape_s(kind, m, k)[1] for m, k in shapes)
        return d, t

    def entry(d_s, t_s, nbytes, **extra):
        return {"us": round(t_s * 1e6, 1), "GB_s": round(nbytes / t_s / 1e9, 3),
                "dequant_only_us": round(d_s * 1e6, 1), "dequant_only_GB_s": round(nbytes / d_s / 1e9, 3),
                "algorithmic_bytes": nbytes, **extra}

    out = {}
    d, t = layer("q8_0", LAYER_SHAPES)
    out["q8_0_layer_7b_b1"] = entry(d, t, sum(_q8_bytes(m, k) + 2 * k + 2 * m for m, k in LAYER_SHAPES))
    # top-10 expert gather: the selected experts' matrices only (what the loop reads)
    E, H, Fd, g, k = 10, 4096, 1024, 64, 10
    pools = [syn.affine_q4_weights(sh, g, gen) for sh in ([E, Fd, H], [E, Fd, H], [E, H, Fd])]
    xm = syn.activations(1, H, gen)
    wts = torch.softmax(torch.randn(k, generator=gen), 0).to(torch.float16)
    idx = list(range(k))
    def dq_moe():
        for p in pools:
            for e in idx:
                cb.dequant_affine_q4(p[0][e], p[1][e], p[2][e], g)

    gather = lambda: cb.moe_gather_decode(*pools, xm, idx, wts, g)  # noqa: E731
    for _ in range(3):  # the allocator's first passes over these temporaries are slower
        dq_moe()
        gather()
    d_s, _ = _median_s(dq_moe, seconds_per_shape / 3)
    t_s, _ = _median_s(gather, seconds_per_shape * 2 / 3)
    out["moe_affine_q4_top10"] = entry(d_s, t_s, MOE_GATE_UP_BYTES + MOE_DOWN_BYTES - 10 * 1024 * 2 + 4096 * 2)
    d, t = layer("q4_0", LAYER_70B)
    out["q4_0_layer_70b_b1"] = entry(d, t, sum(q4_bytes(m, k) + 2 * k + 2 * m for m, k in LAYER_70B))
    d, t = layer("q4_0", LAYER_SHAPES)
    dl, tl = shape_s("q4_0", *LM_HEAD)
    d, t = N_LAYERS * d + dl, N_LAYERS * t + tl
    out["decode_sweep_7b"] = entry(d, t, sweep_bytes(), tok_s=round(1.0 / t, 3))
    out["sample"] = (f"each distinct matrix shape once: median of >= 10 runs after 2 warm-ups on at most "
                     f"{CPU_ROW_CAP} rows, scaled by rows; layers and the sweep as the sum of their GEMVs; "
                     f"the expert gather as the reference's loop over 10 experts")
    return out


def profile_case(case: str, reps: int, dev) -> int:
    """One workload launched `reps` times eagerly (no graph), for a profiler's
    kernel trace or counters; prints one JSON line and returns 0.
      gemm:M,K,T / gemm_q8:M,K,T / gemm_aff:M,K,T   Q4_0 / Q8_0 / affine-Q4 g64
                                                    prefill dequant-GEMM
      gemv:M,K,B                                    Q4_0 fused GEMV
      moe                                           top-10 gather, `reps` calls
      moe_step                                      the decode MoE step, 8-launch
                                                    and 4-launch forms, `reps` calls each
      moe_prefill                                   grouped MoE prefill, 512 tokens
      q8_layer                                      Q8_0 LLaMA-7B layer at batch 1, as 7
                                                    GEMVs and as 4 fused launches, `reps`
                                                    passes over 3 layers each"""
    import torch

    from gdsllm_amd import capi, check
    from gdsllm_amd import synthetic as syn

    global _EAGER
    _EAGER = True
    kind, _, spec = case.partition(":")
    st = torch.cuda.current_stream().cuda_stream
    gen = torch.Generator(device=dev).manual_seed(1020)
    lib = capi()
    if kind in ("gemm", "gemv", "gemm_q8", "gemm_aff"):
        m, k, t = (int(v) for v in spec.split(","))
        x = syn.activations(t, k, gen)
        y = torch.empty(t, m, dtype=torch.float16, device=dev)
        if kind == "gemm_aff":
            aw, asc, ab = syn.affine_q4_weights([m, k], 64, gen)
            launch = lambda: check(lib.gdsllm_dequant_gemm_affine_q4(  # noqa: E731
                aw.data_ptr(), asc.data_ptr(), ab.data_ptr(), x.data_ptr(), y.data_ptr(), m, k, 64, t, k, m, st))
        else:
            w = syn.q8_0_weights(m, k, gen) if kind == "gemm_q8" else syn.q4_0_weights(m, k, gen)
            fn = {"gemm": lib.gdsllm_dequant_gemm_q4_0, "gemm_q8": lib.gdsllm_dequant_gemm_q8_0,
                  "gemv": lib.gdsllm_fused_q4_0_gemv}[kind]
            launch = lambda: check(fn(w.data_ptr(), x.data_ptr(), y.data_ptr(), m, k, t, k, m, st))  # noqa: E731
    elif kind in ("moe", "moe_step"):
        res = bench_moe(dev, calls=reps, reps=1, decode_step=kind == "moe_step")
        res = res.get("decode_step", res)
        print(json.dumps({"profile_case": case, "calls": reps, "result": res}), flush=True)
        return 0
    elif kind == "moe_prefill":
        res = bench_moe_prefill(dev, reps=reps, reference=False)
        print(json.dumps({"profile_case": case, "chunks": reps, "result": res}), flush=True)
        return 0
    elif kind == "q8_layer":
        res = bench_q8_layer(dev, reps=reps)
        print(json.dumps({"profile_case": case, "passes": reps, "result": res}), flush=True)
        return 0
    else:
        print(f"bench.py: unknown --profile-case {case!r}", file=sys.stderr)
        return 2
    launch()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        launch()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    print(json.dumps({"profile_case": case, "launches": reps, "wall_us_per_launch": round(el * 1e6 / reps, 2)}),
          flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400, help="timed passes over the weight copies")
    ap.add_argument("--warmup", type=int, default=40, help="untimed passes over the weight copies")
    ap.add_argument("--copies", type=int, default=16, help="distinct weight copies rotated over")
    ap.add_argument("--chunk", type=int, default=64, help="launches per captured graph")
    ap.add_argument("--sweep-tokens", type=int, default=100, help="timed 7B decode-sweep tokens (0 = skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--cpu-config-seconds", type=float, default=1.0,
                    help="CPU baseline budget per matrix shape of the other workloads (0 = skip)")
    ap.add_argument("--profile-case", default="",
                    help="run only one workload, eagerly, for a profiler: gemm:M,K,T (Q4_0 prefill GEMM), "
                         "gemv:M,K,B (Q4_0 GEMV), moe (top-10 gather, fresh picks per call); then exit")
    ap.add_argument("--profile-reps", type=int, default=10, help="launches of --profile-case")
    ap.add_argument("--configs", default="ceiling,q8,moe,70b,prefill,prefill_fmt,moe_prefill,load",
                    help="comma list of extra workloads to measure: ceiling (plain read of the headline's bytes, "
                         "empty launch), q8 (Q8_0 7B layer), moe (top-10 expert "
                         "gather), 70b (Q4_0 70B layer, B=1..8), prefill (512-token MFMA GEMM), prefill_fmt (Q8_0 "
                         "and affine-Q4 prefill GEMMs), moe_prefill (512-token grouped-expert MLP), load (7B layer "
                         "file -> HBM, embedding row gather), int8 (per-column int8 7B layer); '' = none")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              "(the GEMV would shard by output rows, one row range per GPU).", file=sys.stderr)
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
    if args.profile_case:
        return profile_case(args.profile_case, args.profile_reps, dev)

    g = bench_gemv(args, dev)
    ms_total = g["ms"]
    us_per_call = ms_total * 1e3 / g["launches_timed"]
    gbs = ALGO_BYTES_CFG0 / (us_per_call * 1e-6) / 1e9
    print(f"# q4_0 gemv 11008x4096 b=1: {us_per_call:.3f} us/call, {gbs:.1f} GB/s "
          f"({100 * gbs / HBM_PEAK_GBS:.1f}% of {HBM_PEAK_GBS:.0f})", file=sys.stderr, flush=True)

    sweep, sweep_weights = None, None
    if args.sweep_tokens > 0:
        ms_tok, ms_unf, sweep_weights, batched = bench_decode_sweep(args, dev)
        sb = sweep_bytes()
        sweep = {"tok_s": round(1e3 / ms_tok, 1), "ms_per_token": round(ms_tok, 4), "launches_per_token": 129,
                 "bytes_per_token": sb, "GB_s": round(sb / (ms_tok * 1e-3) / 1e9, 1),
                 "fusion": "q/k/v grouped launch; gate+up+SiLU launch writing h; o, down, lm_head single",
                 "unfused": {"tok_s": round(1e3 / ms_unf, 1), "ms_per_token": round(ms_unf, 4),
                             "launches_per_token": 225, "GB_s": round(sb / (ms_unf * 1e-3) / 1e9, 1)}}
        for B, ms_b in batched.items():
            sweep[f"batch_{B}"] = {"tok_s": round(B * 1e3 / ms_b, 1), "ms_per_step": round(ms_b, 4),
                                   "launches_per_step": 129, "GB_s": round(sb / (ms_b * 1e-3) / 1e9, 1)}
        print(f"# 7B decode sweep: {ms_tok:.4f} ms/token, {sweep['tok_s']} tok/s, {sweep['GB_s']} GB/s "
              f"(unfused 225 launches: {sweep['unfused']['tok_s']} tok/s)", file=sys.stderr, flush=True)

    wanted = {c.strip() for c in args.configs.split(",") if c.strip()}
    unknown = wanted - {"ceiling", "q8", "moe", "70b", "prefill", "prefill_fmt", "moe_prefill", "load", "int8"}
    if unknown:
        print(f"bench.py: unknown --configs entries {sorted(unknown)}", file=sys.stderr)
        return 2
    configs = {}
    runs = [("ceiling", "ceiling_single_launch", lambda: bench_ceiling(dev, args.copies)),
            ("q8", "q8_0_layer_7b_b1", lambda: bench_q8_layer(dev)),
            ("moe", "moe_affine_q4_top10", lambda: bench_moe(dev)),
            ("70b", "q4_0_layer_70b", lambda: bench_70b_layer(dev)),
            ("prefill", "prefill_7b_512",
             lambda: bench_prefill(dev, *sweep_weights) if sweep_weights is not None else None),
            ("prefill_fmt", "prefill_q8_0_affine_7b_512", lambda: bench_prefill_formats(dev)),
            ("moe_prefill", "moe_prefill_affine_q4_512", lambda: bench_moe_prefill(dev)),
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
        if args.cpu_config_seconds > 0:
            prev = torch.get_num_threads()
            torch.set_num_threads(cpu["torch_threads"])
            try:
                cpu["configs"] = cpu_baseline_configs(args.cpu_config_seconds)
            finally:
                torch.set_num_threads(prev)
            print(f"# cpu baseline configs: {cpu['configs']}", file=sys.stderr, flush=True)

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
                   "weight_copies_rotated": args.copies, "launches_per_step": args.copies,
                   "graph_launches": g["graph_launches"], "launches_timed": g["launches_timed"],
                   "algorithmic_bytes_per_launch": ALGO_BYTES_CFG0,
                   "algorithmic_bytes_per_step": ALGO_BYTES_CFG0 * args.copies},
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
