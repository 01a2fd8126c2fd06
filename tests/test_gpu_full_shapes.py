"""Parity at the benchmark configurations' own shapes, where the launch
geometry and the kernel chosen differ from the smaller test shapes:

* the LLaMA-70B layer projections (q/o 8192x8192, k/v 1024x8192, gate/up
  28672x8192, down 8192x28672) at batch 1, 2, 4 and 8, and the layer's
  decode-step fusions at batch 1 and 2 (q/k/v in one grouped launch,
  gate/up/SiLU in one launch);
* the LLaMA-7B projections and lm_head at batch 3, 4 and 8;
* the LLaMA-7B lm_head 32000x4096 as the batch-1 GEMV and as the 512-token
  prefill GEMM, and the 512-token GEMMs of gate/up 11008x4096 and down
  4096x11008.

Weights are generated on the device (same distributions as the benchmark);
the whole matrix is multiplied, and a seeded sample of 512 output rows (every
row when there are at most 1024) is checked against the oracle's float64
product over those rows' exact dequantized weights, under the GEMV tolerance
(relative L2 <= 2e-3, per-row error <= 1e-2 of ||w_r * x||).  Every output
must be finite.
"""

import numpy as np
import pytest
import torch

from helpers import assert_gemv_close, capi, check, oq, ptr, stream, syn, to_np

pytestmark = pytest.mark.gpu

LAYER_70B = [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)]
LAYER_7B = [(4096, 4096), (11008, 4096), (4096, 11008), (32000, 4096)]


def _weights(M, K, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return syn.q4_0_weights(M, K, g)


def _sample_rows(M, seed, n=512):
    if M <= 1024:
        return np.arange(M)
    return np.sort(np.random.default_rng(seed).choice(M, n, replace=False))


def _check_rows(y, w, x, rows, K, what):
    yn = to_np(y).astype(np.float32)
    assert np.isfinite(yn).all(), f"{what}: non-finite output"
    deq = oq.dequant_q4_0(to_np(w[torch.as_tensor(rows, device=w.device)])).reshape(len(rows), K)
    rel, mx = assert_gemv_close(yn[:, rows].astype(np.float16), deq, to_np(x), what)
    print(f"{what}: rel_l2={rel:.2e} max_norm={mx:.2e}")


@pytest.mark.parametrize("B", [3, 4, 8])
@pytest.mark.parametrize("M,K", LAYER_7B, ids=[f"{m}x{k}" for m, k in LAYER_7B])
def test_q4_0_gemv_7b_batched_shapes(gpu, M, K, B):
    """The LLaMA-7B projections at batch 3-8, as the batched decode sweep runs
    them: the x-in-registers kernel's two-workgroup form (11008 and 32000
    rows), the 16-wave form (4096x4096 at batch 3-4), the code kernel with
    16-row tiles over 4096 rows (the down projection; 4096x4096 at batch
    8)."""
    seed = 3600 + M // 1024 + K // 1024 + B
    w = _weights(M, K, seed, gpu)
    x = syn.activations(B, K, torch.Generator().manual_seed(seed + 1))
    xd = x.to(gpu)
    y = torch.empty(B, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_q4_0_gemv(ptr(w), ptr(xd), ptr(y), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    _check_rows(y, w, x, _sample_rows(M, seed), K, f"7B {M}x{K} B={B}")


@pytest.mark.parametrize("B", [1, 2, 4, 8])
@pytest.mark.parametrize("M,K", LAYER_70B, ids=[f"{m}x{k}" for m, k in LAYER_70B])
def test_q4_0_gemv_70b_layer_shapes(gpu, M, K, B):
    seed = 3000 + M // 1024 + K // 1024 + B
    w = _weights(M, K, seed, gpu)
    x = syn.activations(B, K, torch.Generator().manual_seed(seed + 1))
    xd = x.to(gpu)
    y = torch.empty(B, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_q4_0_gemv(ptr(w), ptr(xd), ptr(y), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    _check_rows(y, w, x, _sample_rows(M, seed), K, f"70B {M}x{K} B={B}")


def test_q4_0_lm_head_gemv(gpu):
    """LLaMA-7B lm_head 32000x4096 at batch 1 (the last GEMV of a decode step)."""
    M, K = 32000, 4096
    w = _weights(M, K, 3101, gpu)
    x = syn.activations(1, K, torch.Generator().manual_seed(3102))
    xd = x.to(gpu)
    y = torch.empty(1, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_q4_0_gemv(ptr(w), ptr(xd), ptr(y), M, K, 1, K, M, stream()))
    torch.cuda.synchronize()
    _check_rows(y, w, x, _sample_rows(M, 3101), K, "lm_head B=1")


PREFILL_7B = [(32000, 4096), (11008, 4096), (4096, 11008)]


@pytest.mark.parametrize("M,K", PREFILL_7B, ids=[f"{m}x{k}" for m, k in PREFILL_7B])
def test_q4_0_prefill_gemm_512_tokens(gpu, M, K):
    T = 512
    seed = 3200 + M // 1024 + K // 1024
    w = _weights(M, K, seed, gpu)
    x = syn.activations(T, K, torch.Generator().manual_seed(seed + 1))
    xd = x.to(gpu)
    y = torch.empty(T, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_dequant_gemm_q4_0(ptr(w), ptr(xd), ptr(y), M, K, T, K, M, stream()))
    torch.cuda.synchronize()
    _check_rows(y, w, x, _sample_rows(M, seed), K, f"prefill T{T} {M}x{K}")


@pytest.mark.parametrize("B", [1, 2, 4, 8])
def test_q4_0_70b_qkv_group_and_gate_up_silu(gpu, B):
    """The fused 70B layer of the benchmark: q, k, v (8192, 1024, 1024 rows x
    8192) in one grouped launch and h = silu(gate x) * (up x) for 28672 x 8192
    in one launch, against the oracle on sampled rows (h from the oracle's
    fp16 g and u with torch's fp16 SiLU and product)."""
    import ctypes

    seed = 3300 + B
    Ms = (8192, 1024, 1024)
    ws = [_weights(M, 8192, seed + i, gpu) for i, M in enumerate(Ms)]
    x = syn.activations(B, 8192, torch.Generator().manual_seed(seed + 5))
    xd = x.to(gpu)
    ys = [torch.empty(B, M, dtype=torch.float16, device=gpu) for M in Ms]
    check(capi().gdsllm_fused_q4_0_gemv_group(3, (ctypes.c_void_p * 3)(*[ptr(w) for w in ws]),
                                              (ctypes.c_void_p * 3)(*[ptr(y) for y in ys]),
                                              (ctypes.c_int64 * 3)(*Ms), ptr(xd), 8192, B, 8192, stream()))
    F = 28672
    wg, wu = _weights(F, 8192, seed + 6, gpu), _weights(F, 8192, seed + 7, gpu)
    h = torch.empty(B, F, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_q4_0_gate_up_silu(ptr(wg), ptr(wu), ptr(xd), ptr(h), F, 8192, B, 8192, F, stream()))
    torch.cuda.synchronize()
    for i, (w, y, M) in enumerate(zip(ws, ys, Ms)):
        _check_rows(y, w, x, _sample_rows(M, seed + i), 8192, f"70B qkv group[{i}] {M}x8192 B={B}")
    rows = _sample_rows(F, seed + 8)
    hn = to_np(h).astype(np.float64)[:, rows]
    assert np.isfinite(hn).all(), "non-finite h"
    idx = torch.as_tensor(rows, device=gpu)
    gq = oq.gemv(oq.dequant_q4_0(to_np(wg[idx])).reshape(len(rows), 8192), to_np(x)).astype(np.float16)
    uq = oq.gemv(oq.dequant_q4_0(to_np(wu[idx])).reshape(len(rows), 8192), to_np(x)).astype(np.float16)
    h_ref = (oq.silu_fp16(gq).astype(np.float32) * uq.astype(np.float32)).astype(np.float64)
    rel = float(np.linalg.norm(hn - h_ref) / np.linalg.norm(h_ref))
    print(f"70B gate_up_silu 28672x8192 B={B}: rel L2 {rel:.2e}")
    assert rel <= oq.GEMV_REL_L2, f"h rel L2 {rel:.3e}"

