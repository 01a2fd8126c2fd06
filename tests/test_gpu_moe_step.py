"""The fused decode MoE step (gdsllm_moe_step_affine_q4): routed top-k experts,
the shared expert and its fp16 gate logit in one gate/up launch, their down
rows with the sigmoid-gated combine in one more (runtime/qwen_moe.py:455-513
after routing).

Its output is bit-identical to the separate launches it replaces (the top-k
gather, a one-expert gather of the shared expert, gdsllm_gemv_f16 for the
gate logit and the combine): the shared expert occupies its own lane slot and
the logit follows gemv_f16's summation order, so every sum is formed in the
same order.  The oracle composition bounds both under a relative-L2
tolerance."""

import ctypes

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from gdsllm_amd import capi, check
from helpers import affine_dequant_np, experts_struct, gen, moe_gather, oq, ptr, stream, syn, to_np

pytestmark = pytest.mark.gpu


def _dev(parts, gpu):
    return tuple(t.to(gpu) for t in parts)


def _shared_stacked(parts):
    return tuple(t.unsqueeze(0) for t in parts)


def _step(routed, shared, x, idx, w, sgw, g, top_k, gpu):
    structs = [experts_struct(*p, g) for p in routed + shared]
    F = structs[0].out_dim
    ws_bytes = capi().gdsllm_moe_step_workspace_size(top_k, F)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device=gpu)  # NaN-filled: every read slot must be written
    y = torch.empty(structs[2].out_dim, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_moe_step_affine_q4(*(ctypes.byref(s) for s in structs), ptr(x), ptr(idx), ptr(w), top_k,
                                           ptr(sgw), ptr(y), ptr(ws), ws_bytes, stream()))
    torch.cuda.synchronize()
    return y


def _separate(routed, shared, x, idx, w, sgw, g, gpu):
    eo = moe_gather(*routed, x, idx, w, g)
    one = torch.zeros(1, dtype=torch.int32, device=gpu)
    unit = torch.ones(1, dtype=torch.float16, device=gpu)
    so = moe_gather(*shared, x, one, unit, g)
    H = eo.numel()
    gl = torch.empty(1, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_gemv_f16(ptr(sgw), ptr(x), ptr(gl), 1, H, 1, H, 1, stream()))
    y = torch.empty_like(eo)
    check(capi().gdsllm_moe_combine(ptr(eo), ptr(so), ptr(gl), ptr(y), H, 1, stream()))  # hidden, n_tok
    torch.cuda.synchronize()
    return y


def _gate_row(x, logit):
    """fp16 gate row whose dot with x is about `logit`."""
    xf = x.float().reshape(-1)
    return (xf * (logit / float((xf * xf).sum()))).to(torch.float16)


# (E, H, F, top_k): one to eight lane slots, 4 / 2 / 1 experts per lane group
CASES = [(8, 2048, 512, 1), (16, 2048, 512, 3), (64, 2048, 512, 4), (128, 2048, 512, 8), (64, 4096, 512, 10),
         (32, 2048, 1024, 2), (32, 4096, 1024, 5), (16, 6144, 1024, 3), (16, 2048, 2048, 1), (16, 8192, 2048, 7),
         (512, 2048, 512, 31)]


@pytest.mark.parametrize("E,H,F,k", CASES)
def test_moe_step_matches_separate_launches(gpu, E, H, F, k):
    g = 64
    gg = gen(9100 + E + H + F + k)
    routed_cpu = [syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F])]
    shared_cpu = [_shared_stacked(syn.affine_q4_weights(s, g, gg)) for s in ([F, H], [F, H], [H, F])]
    routed = [_dev(p, gpu) for p in routed_cpu]
    shared = [_dev(p, gpu) for p in shared_cpu]
    x = syn.activations(1, H, gen(9200 + k)).to(gpu)
    picks = torch.randperm(E, generator=gen(9300 + k))[:k].to(torch.int32)
    rw = torch.softmax(torch.randn(k, generator=gen(9400 + k)), 0).to(torch.float16)
    sgw_cpu = (torch.randn(H, generator=gen(9500 + k)) * 0.02).to(torch.float16)
    idx, w, sgw = picks.to(gpu), rw.to(gpu), sgw_cpu.to(gpu)

    y = _step(routed, shared, x, idx, w, sgw, g, k, gpu)
    want = _separate(routed, shared, x, idx, w, sgw, g, gpu)
    np.testing.assert_array_equal(to_np(y).view(np.uint16), to_np(want).view(np.uint16))

    def dq(p, e):
        return affine_dequant_np(*(t[e] for t in p), g).reshape(p[0].shape[1], -1)

    xn = to_np(x).reshape(-1)
    eo, _ = oq.moe_gather(xn, lambda e: dq(routed_cpu[0], e), lambda e: dq(routed_cpu[1], e),
                          lambda e: dq(routed_cpu[2], e), to_np(picks), to_np(rw))
    so, _ = oq.moe_gather(xn, lambda e: dq(shared_cpu[0], e), lambda e: dq(shared_cpu[1], e),
                          lambda e: dq(shared_cpu[2], e), np.zeros(1, np.int32), np.ones(1, np.float16))
    gl = oq.gemv(to_np(sgw_cpu).reshape(1, -1), xn)[0].astype(np.float16)
    ref = oq.moe_combine(eo.astype(np.float16)[None], so.astype(np.float16)[None], gl).astype(np.float64)
    got = to_np(y).astype(np.float64)
    rel = float(np.linalg.norm(got - ref.reshape(-1)) / np.linalg.norm(ref))
    print(f"moe step E{E} H{H} F{F} k{k}: rel L2 {rel:.2e}")
    assert np.all(np.isfinite(got)) and rel <= oq.GEMV_REL_L2, f"rel L2 {rel:.3e}"


def test_moe_step_invalid_indices_and_clamp(gpu):
    """Out-of-range expert indices contribute nothing (as in the gather), and a
    large shared gate drives outputs past fp16 range into the +-65504 clamp."""
    E, H, F, k, g = 16, 2048, 512, 6, 64
    gg = gen(9500)
    routed = [_dev(syn.affine_q4_weights(s, g, gg), gpu) for s in ([E, F, H], [E, F, H], [E, H, F])]
    # shared down rows scaled up so fp16(sigmoid(g) * shared) overflows for some rows
    sgw, suw, sdw = (_shared_stacked(syn.affine_q4_weights(s, g, gg)) for s in ([F, H], [F, H], [H, F]))
    sdw = (sdw[0], (sdw[1].float() * 2000).to(torch.float16), (sdw[2].float() * 2000).to(torch.float16))
    shared = [_dev(p, gpu) for p in (sgw, suw, sdw)]
    x = syn.activations(1, H, gen(9501)).to(gpu)
    idx = torch.tensor([3, -1, 15, 16, 7, 1 << 20], dtype=torch.int32, device=gpu)
    w = torch.full((k,), 1.0 / k, dtype=torch.float16, device=gpu)
    sgw = _gate_row(x, 4.0)
    y = _step(routed, shared, x, idx, w, sgw, g, k, gpu)
    want = _separate(routed, shared, x, idx, w, sgw, g, gpu)
    yn = to_np(y)
    np.testing.assert_array_equal(yn.view(np.uint16), to_np(want).view(np.uint16))
    assert np.any(np.abs(yn) == 65504.0) and np.all(np.isfinite(yn))


def test_moe_step_two_calls_share_nothing(gpu):
    """A second call with fewer experts on the same workspace gives the result
    a fresh workspace gives (no state carried from the first)."""
    E, H, F, g = 32, 2048, 1024, 64
    gg = gen(9600)
    routed = [_dev(syn.affine_q4_weights(s, g, gg), gpu) for s in ([E, F, H], [E, F, H], [E, H, F])]
    shared = [_dev(_shared_stacked(syn.affine_q4_weights(s, g, gg)), gpu) for s in ([F, H], [F, H], [H, F])]
    x = syn.activations(1, H, gen(9601)).to(gpu)
    sgw = _gate_row(x, -0.5)
    structs = [experts_struct(*p, g) for p in routed + shared]
    ws_bytes = capi().gdsllm_moe_step_workspace_size(8, F)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    outs = []
    for k in (8, 3):
        idx = torch.arange(k, dtype=torch.int32, device=gpu) * 3
        w = torch.full((k,), 1.0 / k, dtype=torch.float16, device=gpu)
        y = torch.empty(H, dtype=torch.float16, device=gpu)
        check(capi().gdsllm_moe_step_affine_q4(*(ctypes.byref(s) for s in structs), ptr(x), ptr(idx), ptr(w), k,
                                               ptr(sgw), ptr(y), ptr(ws), ws_bytes, stream()))
        torch.cuda.synchronize()
        outs.append((y, _separate(routed, shared, x, idx, w, sgw, g, gpu)))
    for y, want in outs:
        np.testing.assert_array_equal(to_np(y).view(np.uint16), to_np(want).view(np.uint16))


def _routed_step(router, routed, shared, x, sgw, g, top_k, gpu):
    structs = [experts_struct(*p, g) for p in routed + shared]
    E, F = structs[0].num_experts, structs[0].out_dim
    ws_bytes = capi().gdsllm_moe_step_routed_workspace_size(top_k, F, E)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device=gpu)
    y = torch.empty(structs[2].out_dim, dtype=torch.float16, device=gpu)
    idx = torch.full((top_k,), -7, dtype=torch.int32, device=gpu)
    w = torch.full((top_k,), float("nan"), dtype=torch.float16, device=gpu)
    check(capi().gdsllm_moe_step_routed_affine_q4(ptr(router), *(ctypes.byref(s) for s in structs), ptr(x), top_k,
                                                  ptr(sgw), ptr(y), ptr(idx), ptr(w), ptr(ws), ws_bytes, stream()))
    torch.cuda.synchronize()
    return y, idx, w


# (E, H, F, top_k, ties): the cfg2 layer (512 experts, top-10), small pools,
# and routers whose top logits tie (equal rows: the lower expert index first)
ROUTED_CASES = [(512, 4096, 1024, 10, False), (64, 2048, 512, 4, False), (8, 2048, 512, 1, False),
                (128, 4096, 512, 8, True), (512, 2048, 512, 31, True)]


@pytest.mark.parametrize("E,H,F,k,ties", ROUTED_CASES)
def test_moe_step_routed_matches_route_then_step(gpu, E, H, F, k, ties):
    """The routed step (router GEMV, then the gate/up launch taking the top-k
    itself, then down) gives the picks and weights of gemv_f16 +
    moe_route_topk and the output of the fused step on them, bit for bit."""
    g = 64
    gg = gen(9700 + E + H + F + k)
    routed = [_dev(syn.affine_q4_weights(s, g, gg), gpu) for s in ([E, F, H], [E, F, H], [E, H, F])]
    shared = [_dev(_shared_stacked(syn.affine_q4_weights(s, g, gg)), gpu) for s in ([F, H], [F, H], [H, F])]
    x = syn.activations(1, H, gen(9800 + k)).to(gpu)
    router = (torch.randn(E, H, generator=gen(9900 + k)) * 0.02).to(torch.float16)
    if ties:
        hot = _gate_row(x.cpu(), 8.0)
        for e in (E - 1, 5, 2, E // 2):  # equal top logits at four experts
            router[e] = hot
    router = router.to(gpu)
    sgw = (torch.randn(H, generator=gen(9950 + k)) * 0.02).to(torch.float16).to(gpu)

    y, idx, w = _routed_step(router, routed, shared, x, sgw, g, k, gpu)

    logits = torch.empty(E, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_gemv_f16(ptr(router), ptr(x), ptr(logits), E, H, 1, H, E, stream()))
    ridx = torch.empty(k, dtype=torch.int32, device=gpu)
    rw = torch.empty(k, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_moe_route_topk(ptr(logits), E, 1, E, k, ptr(ridx), ptr(rw), stream()))
    torch.cuda.synchronize()
    want = _step(routed, shared, x, ridx, rw, sgw, g, k, gpu)
    assert torch.equal(idx, ridx), f"picks {idx.tolist()} != {ridx.tolist()}"
    assert torch.equal(w.view(torch.int16), rw.view(torch.int16))
    if ties:
        top = sorted((E - 1, 5, 2, E // 2))[:min(k, 4)]
        assert idx[:len(top)].tolist() == top, "equal logits must come out lowest index first"
    np.testing.assert_array_equal(to_np(y).view(np.uint16), to_np(want).view(np.uint16))


# Drawn layers: expert count, hidden/ffn, group size, top-k and tied router
# rows, pools generated on the device (the properties compare two device paths
# bit for bit, so no oracle pass is needed)
STEP_DIMS = [(2048, 512), (4096, 512), (2048, 1024), (4096, 1024), (6144, 1024), (8192, 512)]


@settings(max_examples=25, deadline=None, derandomize=True, database=None, print_blob=True,
          suppress_health_check=[HealthCheck.function_scoped_fixture, HealthCheck.too_slow])
@given(E8=st.integers(1, 32), dims=st.sampled_from(STEP_DIMS), g=st.sampled_from([32, 64, 128]),
       k=st.integers(1, 12), ties=st.booleans(), seed=st.integers(0, 2 ** 16))
def test_moe_step_property(gpu, E8, dims, g, k, ties, seed):
    """Over drawn layers: the fused step is bit-identical to the separate
    launches on the same picks, and the routed step gives the picks, weights
    and output of router GEMV + top-k + fused step, bit for bit."""
    E = 8 * E8
    H, F = dims
    k = min(k, E, 31 if F == 512 else 15)
    gg = torch.Generator(device=gpu).manual_seed(seed)
    routed = [syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F])]
    shared = [_shared_stacked(syn.affine_q4_weights(s, g, gg)) for s in ([F, H], [F, H], [H, F])]
    x = syn.activations(1, H, gen(seed + 1)).to(gpu)
    picks = torch.randperm(E, generator=gen(seed + 2))[:k].to(torch.int32).to(gpu)
    rw = torch.softmax(torch.randn(k, generator=gen(seed + 3)), 0).to(torch.float16).to(gpu)
    sgw = (torch.randn(H, generator=gen(seed + 4)) * 0.02).to(torch.float16).to(gpu)
    what = f"E{E} H{H} F{F} g{g} k{k}"
    y = _step(routed, shared, x, picks, rw, sgw, g, k, gpu)
    want = _separate(routed, shared, x, picks, rw, sgw, g, gpu)
    np.testing.assert_array_equal(to_np(y).view(np.uint16), to_np(want).view(np.uint16), err_msg=what)

    router = (torch.randn(E, H, generator=gen(seed + 5)) * 0.02).to(torch.float16)
    if ties:
        hot = _gate_row(x.cpu(), 8.0)
        for e in {E - 1, E // 2, 0}:
            router[e] = hot
    router = router.to(gpu)
    y2, idx, w = _routed_step(router, routed, shared, x, sgw, g, k, gpu)
    logits = torch.empty(E, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_gemv_f16(ptr(router), ptr(x), ptr(logits), E, H, 1, H, E, stream()))
    ridx = torch.empty(k, dtype=torch.int32, device=gpu)
    rw2 = torch.empty(k, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_moe_route_topk(ptr(logits), E, 1, E, k, ptr(ridx), ptr(rw2), stream()))
    torch.cuda.synchronize()
    want2 = _step(routed, shared, x, ridx, rw2, sgw, g, k, gpu)
    assert torch.equal(idx, ridx), f"{what}: picks {idx.tolist()} != {ridx.tolist()}"
    assert torch.equal(w.view(torch.int16), rw2.view(torch.int16)), f"{what}: weights differ"
    np.testing.assert_array_equal(to_np(y2).view(np.uint16), to_np(want2).view(np.uint16), err_msg=what)
    del routed, shared
