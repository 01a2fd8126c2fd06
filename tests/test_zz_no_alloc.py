"""The MoE gather entry point that allocates nothing
(gdsllm_moe_gather_affine_q4_noalloc) against the workspace entry point
(gdsllm_moe_gather_affine_q4) through the C ABI: bit-identical outputs on two
calls in a row, the second with a smaller problem (fewer experts, a narrower
expert FFN), so the fixed workspace holds the first call's contents when the
second starts; and, in a fresh process, the entry point's first call on the
device made inside a HIP graph capture, the graph then replayed on new inputs
written in place."""

import ctypes
import json
import os
import subprocess
import sys

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


# Run in a fresh process, so that the capture below is the process's first
# call of the entry point: its per-device set-up (the address of the fixed
# workspace, the kernels' LDS attribute) then happens inside the capture.
_CAPTURE_SCRIPT = r"""
import ctypes, json, sys
import torch
sys.path[:0] = [sys.argv[1], sys.argv[2]]
from helpers import capi, check, experts_struct, gen, moe_gather, ptr, syn
dev = torch.device("cuda:0")
E, H, F, g, k = 64, 4096, 1024, 64, 10
gg = torch.Generator(device=dev).manual_seed(7700)
pool = tuple(syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F]))
gate, up, down = (experts_struct(*p, g) for p in pool)
x = torch.zeros(1, H, dtype=torch.float16, device=dev)
idx = torch.zeros(k, dtype=torch.int32, device=dev)
w = torch.zeros(k, dtype=torch.float16, device=dev)
y = torch.empty(H, dtype=torch.float16, device=dev)
graph = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
with torch.cuda.stream(s):
    with torch.cuda.graph(graph, stream=s):
        check(capi().gdsllm_moe_gather_affine_q4_noalloc(
            ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down), ptr(x), ptr(idx), ptr(w), k, ptr(y),
            torch.cuda.current_stream().cuda_stream))
torch.cuda.synchronize()
same = []
for rep in range(4):
    x.copy_(syn.activations(1, H, gen(7800 + rep)).to(dev))
    idx.copy_(torch.randperm(E, generator=gen(7900 + rep))[:k].to(torch.int32).to(dev))
    w.copy_(torch.softmax(torch.randn(k, generator=gen(8000 + rep)), 0).to(torch.float16).to(dev))
    y.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    want = moe_gather(*pool, x, idx, w, g)
    same.append(bool(torch.equal(y.view(torch.int16), want.view(torch.int16))))
print(json.dumps({"replays_bit_identical": same}))
"""


def test_noalloc_first_use_inside_graph_capture(gpu):
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    out = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, here, root], capture_output=True, text=True,
                         timeout=240)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    assert res["replays_bit_identical"] == [True] * 4, res
