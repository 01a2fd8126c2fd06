"""The MoE gather entry point that allocates nothing
(gdsllm_moe_gather_affine_q4_noalloc) against the workspace entry point
(gdsllm_moe_gather_affine_q4) through the C ABI: bit-identical outputs on two
calls in a row, the second with a smaller problem (fewer experts, a narrower
expert FFN), so the fixed workspace holds the first call's contents when the
second starts."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import capi, check, experts_struct, gen, moe_gather, ptr, stream, syn, to_np

pytestmark = pytest.mark.gpu


def _pool(E, H, F, g, seed, dev):
    gg = torch.Generator(device=dev).manual_seed(seed)
    return tuple(syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F]))


def _noalloc(pool, x, idx, w, g):
    gate, up, down = (experts_struct(*p, g) for p in pool)
    y = torch.empty(down.out_dim, dtype=torch.float16, device=x.device)
    check(capi().gdsllm_moe_gather_affine_q4_noalloc(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down), ptr(x),
                                                     ptr(idx), ptr(w), idx.numel(), ptr(y), stream()))
    torch.cuda.synchronize()
    return y


# (E, H, F, g, top_k): the 512-expert configuration's shape, then smaller ones
# on both kernel paths (row-span: H % 2048 == 0; general: H = 512)
CALLS = [[(64, 4096, 1024, 64, 10), (32, 2048, 512, 64, 4)],
         [(16, 512, 256, 32, 6), (16, 512, 128, 32, 3)]]


@pytest.mark.parametrize("calls", CALLS, ids=["rows_path", "general_path"])
def test_noalloc_matches_workspace_entry_point(gpu, calls):
    assert capi().gdsllm_moe_gather_noalloc_max_bytes() == 1 << 20
    results = []
    for i, (E, H, F, g, k) in enumerate(calls):
        pool = _pool(E, H, F, g, 7100 + i, gpu)
        x = syn.activations(1, H, gen(7200 + i)).to(gpu)
        idx = torch.randperm(E, generator=gen(7300 + i))[:k].to(torch.int32).to(gpu)
        w = torch.softmax(torch.randn(k, generator=gen(7400 + i)), 0).to(torch.float16).to(gpu)
        got = _noalloc(pool, x, idx, w, g)
        want = moe_gather(*pool, x, idx, w, g)
        results.append((got, want))
    for got, want in results:
        assert np.isfinite(to_np(got)).all()
        np.testing.assert_array_equal(to_np(got).view(np.uint16), to_np(want).view(np.uint16))
