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
layers resident (7 projection GEMVs per layer + lm_head 32000 x 4096 = 225
launches per token, one HIP graph per token) as tokens/s, and the CPU baseline
(torch restatement of dequant -> F.linear in fp32 on the host cores).

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
    """LLaMA-7B Q4_0 decode weight sweep: 225 GEMVs per token, one graph."""
    import torch

    from gdsllm_amd import synthetic as syn

    gemv = Q4Gemv()
    gen = torch.Generator(device=dev).manual_seed(2004)
    layers = [[syn.q4_0_weights(m, k, gen) for m, k in LAYER_SHAPES] for _ in range(N_LAYERS)]
    lm_head = syn.q4_0_weights(*LM_HEAD, gen)
    xs = {k: syn.activations(1, k, gen) for k in (4096, 11008)}
    ys = {m: torch.empty(1, m, dtype=torch.float16, device=dev) for m in (4096, 11008, 32000)}

    def token():
        for lw in layers:
            for w, (m, k) in zip(lw, LAYER_SHAPES):
                gemv(w, xs[k], ys[m], m, k)
        gemv(lm_head, xs[LM_HEAD[1]], ys[LM_HEAD[0]], *LM_HEAD)

    token()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        token()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.sweep_tokens):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.sweep_tokens
    del layers, lm_head
    return ms


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

    sweep = None
    if args.sweep_tokens > 0:
        ms_tok = bench_decode_sweep(args, dev)
        sb = sweep_bytes()
        sweep = {"tok_s": round(1e3 / ms_tok, 1), "ms_per_token": round(ms_tok, 4), "launches_per_token": 225,
                 "bytes_per_token": sb, "GB_s": round(sb / (ms_tok * 1e-3) / 1e9, 1)}
        print(f"# 7B decode sweep: {ms_tok:.4f} ms/token, {sweep['tok_s']} tok/s, {sweep['GB_s']} GB/s",
              file=sys.stderr, flush=True)

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
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
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
