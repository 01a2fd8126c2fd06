"""Activations the reference's fp32 loops handle without loss, on every fused
GEMV path (row-span batch 1-2, the batched Q4_0 code and x-in-registers
kernels, the batched Q8_0 MFMA kernel, the staged kernel for x off the 16-byte
grid, the generic kernel for in_dim % 256 != 0, the affine GEMV and the MoE
gather):

* +-inf and NaN: the reference gives +-inf where the weight is nonzero, NaN
  where it is 0 or where +inf and -inf terms meet (runtime/fused_gemv.cu:69-70,
  runtime/affine_q4_dequant.cu:125-126); the non-finite pattern must match
  exactly (oracle.quant.gemv_ieee);
* +-65504 next to N(0, 1) values, large all-positive outlier columns, all
  subnormal x, and a small outlier over a tiny background: finite outputs
  within the GEMV tolerance (relative L2 <= 2e-3, per row <= 1e-2 of
  ||w_r * x||), including rows whose weight at the outlier is 0.
"""

import ctypes

import numpy as np
import pytest
import torch

from helpers import affine_dequant_np, capi, check, experts_struct, gen, oq, ptr, stream, syn, to_np

pytestmark = pytest.mark.gpu

CASES = ["inf", "max", "outliers", "subnormal", "tiny_outlier"]


def make_x(case: str, B: int, K: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(B, K))
    if case == "inf":
        for b in range(B):
            p = (131 * b + 17) % K
            kind = b % 4
            if kind == 0:
                x[b, p] = np.inf
            elif kind == 1:
                x[b, p], x[b, (p + K // 2) % K] = -np.inf, np.inf
            elif kind == 2:
                x[b, p] = np.nan
            # kind 3: a finite row beside the others
    elif case == "max":
        for b in range(B):
            x[b, (97 * b + 13) % K] = 65504.0 if b % 2 == 0 else -65504.0
    elif case == "outliers":
        cols = [5, 77, K // 3, K - 3]
        x[:, cols] = rng.uniform(300, 3000, size=(B, len(cols)))
    elif case == "subnormal":
        x = rng.integers(1, 1024, size=(B, K)) * np.where(rng.integers(0, 2, size=(B, K)) == 1, 1.0, -1.0) * 2.0 ** -24
    elif case == "tiny_outlier":
        x = x * 2.0 ** -10
        x[:, K // 2 + 1] = 16.0
    return x.astype(np.float16)


def assert_matches_reference(y16: np.ndarray, w: np.ndarray, x: np.ndarray, what: str) -> None:
    """y16 [B, n] from the kernel against the reference's IEEE results on the
    rows of w [n, K]: identical NaN / signed-inf pattern, fp16 overflow where
    the exact value lies beyond the fp16 range, and the GEMV tolerance on every
    batch row whose x is finite."""
    y = np.asarray(y16, dtype=np.float16).astype(np.float64)
    ref = oq.gemv_ieee(w, x)
    nan = np.isnan(ref)
    bad_nan = np.isnan(y) != nan
    assert not bad_nan.any(), f"{what}: NaN pattern differs at {np.argwhere(bad_nan)[:8].tolist()}"
    inf = np.isinf(ref)
    assert np.array_equal(y[inf], ref[inf]), f"{what}: infinite outputs differ"
    over = np.isfinite(ref) & (np.abs(ref) >= 65520.0 * (1 + 1e-3))
    assert np.array_equal(y[over], np.sign(ref[over]) * np.inf), f"{what}: fp16 overflow differs"
    for b in range(x.shape[0]):
        if not np.isfinite(x[b].astype(np.float64)).all():
            continue
        ok = np.abs(ref[b]) < 65504.0
        assert np.isfinite(y[b, ok]).all(), f"{what}: batch row {b} non-finite where the reference is finite"
        norms = oq.row_norms(w, x[b:b + 1])[0]
        rel, mx = oq.gemv_errors(y[b, ok][None, :], ref[b, ok][None, :], norms[ok][None, :])
        assert rel <= oq.GEMV_REL_L2 and mx <= oq.GEMV_MAX_NORM, \
            f"{what}: batch row {b}: rel L2 {rel:.3e}, max normalized {mx:.3e}"


def _rows(M: int, seed: int, n: int = 512) -> np.ndarray:
    return np.arange(M) if M <= n else np.sort(np.random.default_rng(seed).choice(M, n, replace=False))


# (fmt, M, K, B, x byte offset): which kernel serves each is noted
GGUF = [
    ("q4_0", 512, 4096, 1, 0), ("q4_0", 300, 11008, 2, 0),   # row-span, one and three windows
    ("q4_0", 9000, 4096, 3, 0), ("q4_0", 9000, 4096, 8, 0),  # x in registers (uneven 32-row tiles)
    ("q4_0", 1024, 8192, 4, 0),                              # x in registers (few tiles)
    ("q4_0", 8192, 4096, 5, 0), ("q4_0", 256, 16384, 8, 0),  # code kernel
    ("q4_0", 8192, 4096, 3, 0),                              # code kernel, x rows 0-3 only
    ("q4_0", 512, 4096, 4, 2),                               # staged (x off the 16-byte grid)
    ("q4_0", 64, 4128, 3, 0),                                # generic (in_dim % 256 != 0)
    ("q8_0", 512, 4096, 1, 0), ("q8_0", 300, 11008, 2, 0),   # row-span
    ("q8_0", 512, 4096, 6, 0),                               # MFMA on exact weights
    ("q8_0", 512, 4096, 3, 2),                               # staged
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("fmt,M,K,B,xoff", GGUF, ids=[f"{f}_{m}x{k}_b{b}_x{o}" for f, m, k, b, o in GGUF])
def test_gguf_gemv_extreme_x(gpu, fmt, M, K, B, xoff, case):
    seed = 8000 + M + K + B
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    w = make(M, K, torch.Generator(device=gpu).manual_seed(seed))
    x = make_x(case, B, K, seed + 1)
    buf = torch.zeros(B * K + 16, dtype=torch.float16, device=gpu)
    xd = buf[xoff // 2: xoff // 2 + B * K]
    xd.copy_(torch.from_numpy(x.reshape(-1)).to(gpu))
    y = torch.empty(B, M, dtype=torch.float16, device=gpu)
    fn = capi().gdsllm_fused_q4_0_gemv if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv
    check(fn(ptr(w), ptr(xd), ptr(y), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    rows = _rows(M, seed)
    deq = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(w[torch.as_tensor(rows, device=gpu)]))
    assert_matches_reference(to_np(y)[:, rows], deq.reshape(len(rows), K), x, f"{fmt} {M}x{K} B={B} {case}")


AFFINE = [(1024, 4096, 64, 1), (4096, 1024, 64, 2), (1024, 4096, 128, 3), (512, 2048, 64, 8), (40, 96, 32, 2)]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("M,K,g,B", AFFINE, ids=[f"{m}x{k}_g{g}_b{b}" for m, k, g, b in AFFINE])
def test_affine_gemv_extreme_x(gpu, M, K, g, B, case):
    seed = 8100 + M + K + B
    words, scales, biases = syn.affine_q4_weights([M, K], g, gen(seed))
    x = make_x(case, B, K, seed + 1)
    xd = torch.from_numpy(x).to(gpu)
    y = torch.empty(B, M, dtype=torch.float16, device=gpu)
    wd, sd, bd = words.to(gpu), scales.to(gpu), biases.to(gpu)
    check(capi().gdsllm_fused_affine_q4_gemv(ptr(wd), ptr(sd), ptr(bd), ptr(xd), ptr(y), M, K, g, B, K, M, stream()))
    torch.cuda.synchronize()
    deq = affine_dequant_np(words, scales, biases, g).reshape(M, K)
    assert_matches_reference(to_np(y), deq, x, f"affine {M}x{K} g{g} B={B} {case}")


@pytest.mark.parametrize("case", ["inf", "max", "outliers", "tiny_outlier"])
@pytest.mark.parametrize("H,F", [(4096, 1024), (512, 256)], ids=["rows", "general"])
def test_moe_gather_phase1_extreme_x(gpu, H, F, case):
    """The gather's gate/up rows (phase 1, kept in the workspace) follow the
    reference's GEMV on extreme x; the output is finite wherever the expert
    intermediate values are."""
    E, g, k = 12, 64, 5
    gg = gen(8200 + H)
    pools = [syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F])]
    x = make_x(case, 1, H, 8201 + H)
    idx = torch.tensor([3, 0, 11, 7, 5], dtype=torch.int32)
    wts = torch.softmax(torch.randn(k, generator=gen(8202)), 0).to(torch.float16)
    dp = [tuple(t.to(gpu) for t in p) for p in pools]
    structs = [experts_struct(*p, g) for p in dp]
    ws_bytes = capi().gdsllm_moe_gather_workspace_size(k, F)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=gpu)
    y = torch.empty(H, dtype=torch.float16, device=gpu)
    xd, idxd, wd = torch.from_numpy(x.reshape(-1)).to(gpu), idx.to(gpu), wts.to(gpu)
    check(capi().gdsllm_moe_gather_affine_q4(*(ctypes.byref(s) for s in structs), ptr(xd), ptr(idxd), ptr(wd), k,
                                             ptr(y), ptr(ws), ws_bytes, stream()))
    torch.cuda.synchronize()
    gu = to_np(ws[: k * 2 * F * 2].view(torch.float16).view(k, 2, F))
    for j, e in enumerate(idx.tolist()):
        for part in range(2):
            wt, st, bt = (t[e] for t in pools[part])
            deq = affine_dequant_np(wt, st, bt, g).reshape(F, H)
            assert_matches_reference(gu[j, part][None, :], deq, x, f"moe {case} slot {j} {'gate' if part == 0 else 'up'}")


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("M,K,B", [(1000, 4096, 5), (200, 8192, 3), (40, 256, 8)], ids=["1000x4096_b5", "200x8192_b3",
                                                                                       "40x256_b8"])
def test_q4_0_group_gate_up_extreme_x(gpu, M, K, B, case):
    """Batch 3-8 groups and gate/up pairs (the x-in-registers kernel, which
    takes the offset-corrected products only where a wave's slice of x has no
    dominant block and no non-finite value): gate and up from the grouped
    launch follow the reference; h from the pair launch follows silu(g) * u
    of those outputs (the same per-row sums) with torch's fp16 semantics,
    NaN and infinities included."""
    seed = 8300 + M + B
    gg = torch.Generator(device=gpu).manual_seed(seed)
    wg, wu = syn.q4_0_weights(M, K, gg), syn.q4_0_weights(M, K, gg)
    x = make_x(case, B, K, seed + 1)
    xd = torch.from_numpy(x).to(gpu)
    g, u, h = (torch.empty(B, M, dtype=torch.float16, device=gpu) for _ in range(3))
    check(capi().gdsllm_fused_q4_0_gemv_group(2, (ctypes.c_void_p * 2)(ptr(wg), ptr(wu)),
                                              (ctypes.c_void_p * 2)(ptr(g), ptr(u)), (ctypes.c_int64 * 2)(M, M),
                                              ptr(xd), K, B, K, stream()))
    check(capi().gdsllm_fused_q4_0_gate_up_silu(ptr(wg), ptr(wu), ptr(xd), ptr(h), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    rows = _rows(M, seed)
    idx = torch.as_tensor(rows, device=gpu)
    for t, w, part in ((g, wg, "gate"), (u, wu, "up")):
        deq = oq.dequant_q4_0(to_np(w[idx])).reshape(len(rows), K)
        assert_matches_reference(to_np(t)[:, rows], deq, x, f"group {part} {M}x{K} B={B} {case}")
    gn, un, hn = to_np(g), to_np(u), to_np(h).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        sg = oq.silu_fp16(gn)
        href = (sg.astype(np.float32) * un.astype(np.float32)).astype(np.float16).astype(np.float64)
        bound = oq.fp16_ulp(sg) * np.abs(un.astype(np.float64)) + oq.fp16_ulp(href)
    assert np.array_equal(np.isnan(hn), np.isnan(href)), f"h NaN pattern differs ({case})"
    inf = np.isinf(href)
    assert np.array_equal(hn[inf], href[inf]), f"h infinities differ ({case})"
    fin = np.isfinite(href) & np.isfinite(bound)
    bad = np.abs(hn[fin] - href[fin]) > bound[fin]
    assert not bad.any(), f"{int(bad.sum())} h values off ({case})"
