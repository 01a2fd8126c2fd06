"""Parity of the top-k expert-gather MLP and the MFMA prefill dequant-GEMM."""

import numpy as np
import pytest
import torch

from helpers import (affine_dequant_np, assert_gemv_close, capi, check, check_moe, gen, moe_gather, moe_pool, oq, ptr,
                     stream, syn, to_np)

pytestmark = pytest.mark.gpu


MOE_CASES = [
    # row-span path: 64 lanes per gate/up row (1-4 chunks each), 16/32/64 lanes per down row, 1-8 slots
    (16, 4096, 1024, 64, 10), (6, 2048, 512, 64, 5), (10, 8192, 2048, 128, 8), (8, 6144, 1024, 32, 3),
    (20, 2048, 1024, 64, 16), (4, 2048, 512, 32, 1),
    # general path
    (8, 512, 256, 32, 3), (12, 1024, 512, 128, 1), (6, 2048, 256, 64, 4),
]


@pytest.mark.parametrize("E,H,F,g,top_k", MOE_CASES, ids=[f"E{e}_H{h}_F{f}_g{g}_k{k}" for e, h, f, g, k in MOE_CASES])
def test_moe_gather(gpu, E, H, F, g, top_k):
    gate, up, down = moe_pool(E, H, F, g, 4000 + E + top_k)
    x = syn.activations(1, H, gen(4100 + E))
    idx = torch.randperm(E, generator=gen(4200 + E))[:top_k].to(torch.int32)
    wts = torch.softmax(torch.randn(top_k, generator=gen(4300)), 0).to(torch.float16)
    y, ws, hk = moe_gather(tuple(t.to(gpu) for t in gate), tuple(t.to(gpu) for t in up),
                           tuple(t.to(gpu) for t in down), x.to(gpu), idx.to(gpu), wts.to(gpu), g, return_workspace=True)
    check_moe(y, ws, gate, up, down, x, to_np(idx), wts, g, E, hk)


@pytest.mark.parametrize("H,F", [(512, 256), (2048, 1024)], ids=["general", "rows"])
def test_moe_gather_skips_out_of_range_experts(gpu, H, F):
    E, g = 6, 64
    gate, up, down = moe_pool(E, H, F, g, 77)
    x = syn.activations(1, H, gen(78))
    idx = torch.tensor([2, -1, 5, 6, 0], dtype=torch.int32)
    wts = torch.tensor([0.3, 0.2, 0.2, 0.2, 0.1], dtype=torch.float16)
    y, ws, hk = moe_gather(tuple(t.to(gpu) for t in gate), tuple(t.to(gpu) for t in up),
                           tuple(t.to(gpu) for t in down), x.to(gpu), idx.to(gpu), wts.to(gpu), g, return_workspace=True)
    check_moe(y, ws, gate, up, down, x, to_np(idx), wts, g, E, hk)


def test_moe_gather_cfg2_full_pool(gpu):
    """512-expert pool (3.6 GB) generated on the device; the oracle sees only the 10 picked experts."""
    E, H, F, g, top_k = 512, 4096, 1024, 64, 10
    gate, up, down = moe_pool(E, H, F, g, 1002, device=gpu)
    x = syn.activations(1, H, gen(1003))
    idx = torch.randperm(E, generator=gen(1004))[:top_k].to(torch.int32)
    wts = torch.softmax(torch.randn(top_k, generator=gen(1005)), 0).to(torch.float16)
    y, ws, hk = moe_gather(gate, up, down, x.to(gpu), idx.to(gpu), wts.to(gpu), g, return_workspace=True)
    sel = sorted(set(int(e) for e in idx))
    remap = {e: i for i, e in enumerate(sel)}
    small = [tuple(t[sel].cpu() for t in pool) for pool in (gate, up, down)]
    assert hk is not None, "the 512-expert shape must take the row-span path"
    check_moe(y, ws, *small, x, np.array([remap[int(e)] for e in idx]), wts, g, len(sel), hk)
    del gate, up, down
    torch.cuda.empty_cache()


# (T, M, K): single step (K = 32), K not a multiple of 64, ragged token and row
# tiles, and shapes large enough for the 256-token workgroup tiles
# (1100 x 8200 and 2048 x 4096 give at least one tile per CU).
GEMM_CASES = [(1, 128, 64), (3, 130, 32), (7, 300, 256), (40, 200, 96), (64, 128, 4096), (100, 260, 1024),
              (512, 4096, 4096), (33, 11008, 4096), (512, 512, 11008), (1100, 8200, 512), (2048, 4096, 4096)]


@pytest.mark.parametrize("T,M,K", GEMM_CASES, ids=[f"T{t}_{m}x{k}" for t, m, k in GEMM_CASES])
def test_dequant_gemm_q4_0(gpu, T, M, K):
    w = syn.q4_0_weights(M, K, gen(5000 + M))
    x = syn.activations(T, K, gen(5001 + T))
    deq = oq.dequant_q4_0(to_np(w)).reshape(M, K)
    xd = x.to(gpu)
    y = torch.empty(T, M, dtype=torch.float16, device=gpu)
    wd = w.to(gpu)  # held across the call: a freed copy could be reused before the kernel reads it
    check(capi().gdsllm_dequant_gemm_q4_0(ptr(wd), ptr(xd), ptr(y), M, K, T, K, M, stream()))
    torch.cuda.synchronize()
    assert_gemv_close(to_np(y), deq, to_np(x), f"gemm T{T} {M}x{K}")


def test_dequant_gemm_strided(gpu):
    """x rows and y rows with leading dimensions wider than the rows."""
    T, M, K, ldx, ldy = 70, 390, 512, 520, 397
    w = syn.q4_0_weights(M, K, gen(5100))
    xfull = syn.activations(T, ldx, gen(5101))
    x = xfull[:, :K]
    deq = oq.dequant_q4_0(to_np(w)).reshape(M, K)
    xd = xfull.to(gpu)
    y = torch.full((T, ldy), 7.0, dtype=torch.float16, device=gpu)
    wd = w.to(gpu)  # held across the call: a freed copy could be reused before the kernel reads it
    check(capi().gdsllm_dequant_gemm_q4_0(ptr(wd), ptr(xd), ptr(y), M, K, T, ldx, ldy, stream()))
    torch.cuda.synchronize()
    yh = to_np(y)
    assert_gemv_close(yh[:, :M].copy(), deq, to_np(x).copy(), "gemm strided")
    assert (yh[:, M:] == 7.0).all(), "padding columns of y were written"


def test_dequant_gemm_rejects_unsupported(gpu):
    y = torch.empty(8, dtype=torch.float16, device=gpu)
    assert capi().gdsllm_dequant_gemm_q4_0(ptr(y), ptr(y), ptr(y), 4, 96, 2, 100, 4, stream()) == 2
    assert b"aligned" in capi().gdsllm_last_error()
