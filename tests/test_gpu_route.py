"""On-device MoE routing and epilogue against the oracle, through the C ABI:
the fp16 router GEMV (tolerance of the GEMV kernels), top-k + softmax
(indices exact; weights equal to the oracle's from the same logits, within
one fp16 ulp for the rare last-bit difference of exp between numpy and the
device), and the shared-expert combine (exact but for the same exp ulp)."""

import numpy as np
import pytest
import torch

from helpers import assert_gemv_close, capi, check, gen, on_gpu, oq, ptr, stream, syn, to_np

pytestmark = pytest.mark.gpu

F16_CASES = [(512, 4096, 1), (512, 4096, 3), (512, 2048, 8), (1, 4096, 1), (100, 1000, 2), (37, 100, 1), (9, 20, 4),
             (60, 1024, 1), (48, 8192, 2), (16, 12288, 3), (2048, 4096, 1)]


@pytest.mark.parametrize("M,K,B", F16_CASES, ids=[f"{m}x{k}_b{b}" for m, k, b in F16_CASES])
@pytest.mark.parametrize("w_off", [0, 2])
def test_gemv_f16(gpu, M, K, B, w_off):
    g = gen(6000 + M + K + B)
    w = (torch.randn(M, K, generator=g, device=g.device) * 0.05).to(torch.float16)
    x = syn.activations(B, K, gen(6001 + K))
    wd = on_gpu(w.view(torch.uint8).reshape(-1), gpu, pad_front=w_off).view(torch.float16)
    xd = x.to(gpu)
    y = torch.empty(B, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_gemv_f16(ptr(wd), ptr(xd), ptr(y), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    assert_gemv_close(to_np(y), to_np(w), to_np(x), f"gemv_f16 {M}x{K} b{B} off{w_off}")


def _ulp_close(got: np.ndarray, want: np.ndarray, what: str, min_exact: float = 0.95):
    g, w = got.astype(np.float16), want.astype(np.float16)
    same = (g.view(np.uint16) == w.view(np.uint16)) | (np.isnan(g) & np.isnan(w))
    gi = g.view(np.int16).astype(np.int32)
    wi = w.view(np.int16).astype(np.int32)
    ulps = np.abs(gi - wi)
    assert np.all(same | (ulps <= 1)), f"{what}: differs by more than one fp16 ulp"
    assert same.mean() >= min_exact, f"{what}: only {same.mean():.3f} bit-exact"


def _route(logits: torch.Tensor, k: int):
    n, E = logits.shape
    idx = torch.empty(n, k, dtype=torch.int32, device=logits.device)
    w = torch.empty(n, k, dtype=torch.float16, device=logits.device)
    check(capi().gdsllm_moe_route_topk(ptr(logits), E, n, E, k, ptr(idx), ptr(w), stream()))
    torch.cuda.synchronize()
    return to_np(idx), to_np(w)


ROUTE_CASES = [(512, 10, 1), (512, 10, 4), (100, 1, 2), (64, 64, 1), (4096, 64, 1), (2048, 8, 3), (7, 3, 2)]


@pytest.mark.parametrize("E,k,n", ROUTE_CASES, ids=[f"E{e}_k{k}_n{n}" for e, k, n in ROUTE_CASES])
def test_route_topk(gpu, E, k, n):
    g = gen(6100 + E + k + n)
    logits = torch.randn(n, E, generator=g, device=g.device).to(torch.float16)
    idx, w = _route(logits.to(gpu), k)
    ridx, rw = oq.route_topk(to_np(logits), k)
    np.testing.assert_array_equal(idx, ridx)
    _ulp_close(w, rw, f"route E{E} k{k}")


def test_route_topk_ties_and_specials(gpu):
    rng = np.random.default_rng(61)
    v = (rng.integers(-3, 4, size=(5, 300)).astype(np.float16) * np.float16(0.25))
    v[0, [5, 77, 200]] = np.float16(np.nan)
    v[1, [3, 4]] = np.float16(np.inf)
    v[2, :] = np.float16(-np.inf)
    v[2, [10, 20]] = np.float16(-1.0)
    v[3, ::2] = np.float16(-0.0)
    v[3, 1::2] = np.float16(0.0)
    v[4, :] = np.float16(1.0)
    logits = torch.from_numpy(v)
    idx, w = _route(logits.to(gpu), 12)
    ridx, rw = oq.route_topk(v, 12)
    np.testing.assert_array_equal(idx, ridx)
    _ulp_close(w, rw, "route ties/specials", min_exact=1.0)


def test_route_from_router_gemv(gpu):
    """Router logits from gdsllm_gemv_f16 on a random fp16 router, then top-k on
    those logits: the picks and weights equal the oracle's from the same logits."""
    H, E, k = 4096, 512, 10
    g = gen(6200)
    router = (torch.randn(E, H, generator=g, device=g.device) * 0.02).to(torch.float16).to(gpu)
    x = syn.activations(1, H, gen(6201)).to(gpu)
    logits = torch.empty(1, E, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_gemv_f16(ptr(router), ptr(x), ptr(logits), E, H, 1, H, E, stream()))
    idx, w = _route(logits, k)
    ridx, rw = oq.route_topk(to_np(logits), k)
    np.testing.assert_array_equal(idx, ridx)
    _ulp_close(w, rw, "routed from gemv")
    assert_gemv_close(to_np(logits), to_np(router), to_np(x), "router logits")


@pytest.mark.parametrize("H,n", [(4096, 1), (2048, 3), (5, 2)])
def test_moe_combine(gpu, H, n):
    g = gen(6300 + H + n)
    eo = (torch.randn(n, H, generator=g, device=g.device) * 4).to(torch.float16)
    so = (torch.randn(n, H, generator=g, device=g.device) * 4).to(torch.float16)
    gl = (torch.randn(n, generator=g, device=g.device) * 3).to(torch.float16)
    if H > 4:
        eo[0, :3] = torch.tensor([float("inf"), float("nan"), -60000.0], dtype=torch.float16)
        so[0, 2] = -60000.0
        gl[0] = 20.0  # sigmoid rounds to 1: -60000 + -60000 overflows and clamps
    eo_d, so_d, gl_d = eo.to(gpu), so.to(gpu), gl.to(gpu)
    y = torch.empty(n, H, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_moe_combine(ptr(eo_d), ptr(so_d), ptr(gl_d), ptr(y), H, n, stream()))
    torch.cuda.synchronize()
    want = oq.moe_combine(to_np(eo), to_np(so), to_np(gl))
    _ulp_close(to_np(y), want, f"combine H{H} n{n}", min_exact=0.98)
    if H > 4:
        got = to_np(y)
        assert got[0, 0] == np.float16(65504.0) and np.isnan(got[0, 1]) and got[0, 2] == np.float16(-65504.0)
