"""Property tests over drawn shapes (Hypothesis): every dispatch path of the
fused GEMVs, the grouped and gate/up launches and the dequant kernels, through
the C ABI, against the oracle.

Each example draws out_dim, in_dim, batch, the x and y row strides and an
x start off the 16-byte grid, so the planner's choices (row-span, code and
x-in-registers kernels, their 8/12/16-wave forms, staged and generic paths)
are all reached over the run, and checks two properties: the result is
within the oracle tolerance (per-row error beyond one fp16 ulp <= 1e-2 of
||w_r * x||, and relative L2 <= 2e-3 over 256 or more outputs;
oracle.quant.gemv_errors), and nothing
outside the output rows is written (y padding columns keep a sentinel).
Dequantization is checked bit for bit.  The draws are derandomized, so a run
is reproducible and a failure names its example.
"""

import ctypes

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from helpers import (affine_dequant_np, capi, check, check_moe, check_moe_prefill, check_sort, gen, moe_gather,
                     moe_pool, moe_prefill, oq, ptr, stream, syn, to_np)

pytestmark = pytest.mark.gpu

PROPS = settings(max_examples=120, deadline=None, derandomize=True, database=None, print_blob=True,
                 suppress_health_check=[HealthCheck.function_scoped_fixture, HealthCheck.too_slow])
SENTINEL = 7.0

# in_dim: multiples of 256 (the fast kernels) and of 32 only (the generic path)
in_dims = st.one_of(st.integers(1, 36).map(lambda v: 256 * v), st.integers(1, 200).map(lambda v: 32 * v))


def _x_strided(B, K, ldx, x_off, seed, dev):
    """x rows ldx elements apart, starting x_off elements into the allocation."""
    x = syn.activations(B, K, gen(seed))
    buf = torch.zeros(x_off + B * ldx + 8, dtype=torch.float16)
    for b in range(B):
        buf[x_off + b * ldx: x_off + b * ldx + K] = x[b]
    return x, buf.to(dev), x_off


def _gemv_close(y_test, w_fp16, x_fp16, what):
    """The parity bound of the GEMV tests: per row, the error beyond one fp16
    ulp within 1e-2 of ||w_r * x|| (a row whose terms cancel has no relative
    precision to keep); over at least 256 outputs also relative L2 <= 2e-3."""
    y_ref = oq.gemv(w_fp16, x_fp16)
    rel, mx = oq.gemv_errors(np.asarray(y_test, dtype=np.float64), y_ref, oq.row_norms(w_fp16, x_fp16))
    assert np.all(np.isfinite(y_test)), f"{what}: non-finite output"
    assert mx <= oq.GEMV_MAX_NORM, f"{what}: max normalized error {mx:.3e} > {oq.GEMV_MAX_NORM}"
    if y_ref.size >= 256:
        assert rel <= oq.GEMV_REL_L2, f"{what}: rel L2 {rel:.3e} > {oq.GEMV_REL_L2}"


def _y_padded(B, M, ldy, dev):
    return torch.full((B * ldy + 8,), SENTINEL, dtype=torch.float16, device=dev)


def _y_rows(y, B, M, ldy):
    yh = to_np(y)
    rows = np.stack([yh[b * ldy: b * ldy + M] for b in range(B)])
    pad = np.concatenate([yh[b * ldy + M: (b + 1) * ldy] for b in range(B)] + [yh[B * ldy:]])
    return rows, pad


@PROPS
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), M=st.integers(1, 700), K=in_dims, B=st.integers(1, 8),
       ldx_pad=st.integers(0, 9), ldy_pad=st.integers(0, 5), x_off=st.sampled_from([0, 0, 0, 8, 1, 3]),
       seed=st.integers(0, 2 ** 16))
def test_gguf_gemv_property(gpu, fmt, M, K, B, ldx_pad, ldy_pad, x_off, seed):
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    w = make(M, K, gen(seed))
    ldx, ldy = K + ldx_pad, M + ldy_pad
    x, xbuf, off = _x_strided(B, K, ldx, x_off, seed + 1, gpu)
    y = _y_padded(B, M, ldy, gpu)
    fn = capi().gdsllm_fused_q4_0_gemv if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv
    wd = w.to(gpu)  # device copies stay referenced until the launch has run
    check(fn(ptr(wd), xbuf.data_ptr() + 2 * off, ptr(y), M, K, B, ldx, ldy, stream()))
    torch.cuda.synchronize()
    rows, pad = _y_rows(y, B, M, ldy)
    what = f"{fmt} {M}x{K} B{B} ldx {ldx} ldy {ldy} x+{off}"
    assert np.all(pad == SENTINEL), f"{what}: written outside the output rows"
    _gemv_close(rows, dq(to_np(w)).reshape(M, K), to_np(x), what)


# Matrices with thousands of rows: the launch plans that need many row groups
# or tiles per CU (the 12-wave gate/up pairs, the two-workgroup batched form,
# 16-row code-kernel tiles, two stage buffers per wave)
LARGE = settings(PROPS, max_examples=12)
large_rows = st.integers(4000, 13000)
large_in = st.sampled_from([1024, 2048, 3072, 4096, 5120])


@LARGE
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), M=large_rows, K=large_in, B=st.integers(1, 8),
       seed=st.integers(0, 2 ** 16))
def test_gguf_gemv_large_property(gpu, fmt, M, K, B, seed):
    test_gguf_gemv_property.hypothesis.inner_test(gpu, fmt, M, K, B, 0, 3, 0, seed)


@LARGE
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), M=large_rows, K=large_in, B=st.integers(1, 8),
       seed=st.integers(0, 2 ** 16))
def test_gate_up_silu_large_property(gpu, fmt, M, K, B, seed):
    test_gate_up_silu_property.hypothesis.inner_test(gpu, fmt, M, K, B, 2, seed)


@PROPS
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), Ms=st.lists(st.integers(0, 500), min_size=1, max_size=4),
       K=in_dims, B=st.integers(1, 8), seed=st.integers(0, 2 ** 16))
def test_gemv_group_property(gpu, fmt, Ms, K, B, seed):
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    n = len(Ms)
    ws = [make(M, K, gen(seed + i)) if M else None for i, M in enumerate(Ms)]
    x = syn.activations(B, K, gen(seed + 10))
    xd = x.to(gpu)
    wd = [w.to(gpu) if w is not None else None for w in ws]
    ys = [_y_padded(B, M, M, gpu) for M in Ms]
    fn = capi().gdsllm_fused_q4_0_gemv_group if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv_group
    check(fn(n, (ctypes.c_void_p * n)(*[ptr(w) if w is not None else None for w in wd]),
             (ctypes.c_void_p * n)(*[ptr(y) for y in ys]), (ctypes.c_int64 * n)(*Ms), ptr(xd), K, B, K, stream()))
    torch.cuda.synchronize()
    for i, M in enumerate(Ms):
        rows, pad = _y_rows(ys[i], B, M, M)
        what = f"{fmt} group[{i}] of {Ms} x {K} B{B}"
        assert np.all(pad == SENTINEL), f"{what}: written past its rows"
        if M:
            _gemv_close(rows, dq(to_np(ws[i])).reshape(M, K), to_np(x), what)


@PROPS
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), M=st.integers(1, 600), K=in_dims, B=st.integers(1, 8),
       ldh_pad=st.integers(0, 4), seed=st.integers(0, 2 ** 16))
def test_gate_up_silu_property(gpu, fmt, M, K, B, ldh_pad, seed):
    """h = fp16(silu(g) * u) against the oracle's g and u, element by element
    within the GEMV tolerance carried through silu and the product (a g or u
    that cancels to near zero has no relative precision), and over many
    elements by relative L2; a batch 3-8 shape the pair launch does not serve
    is refused with GDSLLM_ERR_UNSUPPORTED and writes nothing."""
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    wg, wu = make(M, K, gen(seed)), make(M, K, gen(seed + 1))
    x = syn.activations(B, K, gen(seed + 2))
    ldh = M + ldh_pad
    h = _y_padded(B, M, ldh, gpu)
    fn = capi().gdsllm_fused_q4_0_gate_up_silu if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gate_up_silu
    wgd, wud, xd = wg.to(gpu), wu.to(gpu), x.to(gpu)
    rc = fn(ptr(wgd), ptr(wud), ptr(xd), ptr(h), M, K, B, K, ldh, stream())
    torch.cuda.synchronize()
    what = f"{fmt} gate/up {M}x{K} B{B} ldh {ldh}"
    served = B <= 2 and K % 256 == 0 or (B <= 8 and fmt == "q4_0" and K % 256 == 0 and K <= 8192)
    if not served:
        assert rc == 2, f"{what}: expected GDSLLM_ERR_UNSUPPORTED (2), got {rc}"
        assert np.all(to_np(h) == SENTINEL), f"{what}: a refused call wrote h"
        return
    check(rc)
    rows, pad = _y_rows(h, B, M, ldh)
    assert np.all(pad == SENTINEL), f"{what}: written outside h's rows"
    _h_close(rows, dq(to_np(wg)).reshape(M, K), dq(to_np(wu)).reshape(M, K), to_np(x), what)


@PROPS
@given(g=st.sampled_from([32, 64, 128]), M=st.integers(1, 500), kg=st.integers(1, 40), B=st.integers(1, 8),
       ldx_pad=st.integers(0, 9), ldy_pad=st.integers(0, 5), seed=st.integers(0, 2 ** 16))
def test_affine_gemv_property(gpu, g, M, kg, B, ldx_pad, ldy_pad, seed):
    K = g * kg
    words, scales, biases = syn.affine_q4_weights([M, K], g, gen(seed))
    ldx, ldy = K + ldx_pad, M + ldy_pad
    x, xbuf, off = _x_strided(B, K, ldx, 0, seed + 1, gpu)
    y = _y_padded(B, M, ldy, gpu)
    wd, sd, bd = words.to(gpu), scales.to(gpu), biases.to(gpu)
    check(capi().gdsllm_fused_affine_q4_gemv(ptr(wd), ptr(sd), ptr(bd), xbuf.data_ptr(), ptr(y), M, K, g, B, ldx, ldy,
                                             stream()))
    torch.cuda.synchronize()
    rows, pad = _y_rows(y, B, M, ldy)
    what = f"affine g{g} {M}x{K} B{B} ldx {ldx} ldy {ldy}"
    assert np.all(pad == SENTINEL), f"{what}: written outside the output rows"
    _gemv_close(rows, affine_dequant_np(words, scales, biases, g).reshape(M, K), to_np(x), what)


@PROPS
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), nblk=st.integers(1, 5000), seed=st.integers(0, 2 ** 16))
def test_gguf_dequant_property(gpu, fmt, nblk, seed):
    """Bit for bit, on raw blocks with every scale bit pattern allowed
    (subnormal, infinite and NaN scales included)."""
    bb = 18 if fmt == "q4_0" else 34
    raw = torch.randint(0, 256, (nblk * bb,), dtype=torch.uint8, generator=gen(seed))
    out = torch.full((nblk * 32 + 8,), SENTINEL, dtype=torch.float16, device=gpu)
    fn = capi().gdsllm_dequant_q4_0 if fmt == "q4_0" else capi().gdsllm_dequant_q8_0
    rd = raw.to(gpu)
    check(fn(ptr(rd), ptr(out), nblk, stream()))
    torch.cuda.synchronize()
    got = to_np(out).view(np.uint16)
    ref = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(raw)).reshape(-1).view(np.uint16)
    assert np.array_equal(got[: nblk * 32], ref), f"{fmt} {nblk} blocks: bits differ"
    assert np.all(to_np(out)[nblk * 32:] == SENTINEL), f"{fmt} {nblk} blocks: written past the end"


@PROPS
@given(g=st.sampled_from([32, 64, 128]), rows=st.integers(1, 300), kg=st.integers(1, 24), seed=st.integers(0, 2 ** 16))
def test_affine_dequant_property(gpu, g, rows, kg, seed):
    cols = g * kg
    words, scales, biases = syn.affine_q4_weights([rows, cols], g, gen(seed))
    n = rows * cols
    out = torch.full((n + 8,), SENTINEL, dtype=torch.float16, device=gpu)
    wd, sd, bd = words.to(gpu), scales.to(gpu), biases.to(gpu)
    check(capi().gdsllm_dequant_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(out), n, cols, g, stream()))
    torch.cuda.synchronize()
    ref = affine_dequant_np(words, scales, biases, g).reshape(-1).view(np.uint16)
    assert np.array_equal(to_np(out)[:n].view(np.uint16), ref), f"affine g{g} {rows}x{cols}: bits differ"
    assert np.all(to_np(out)[n:] == SENTINEL), f"affine g{g} {rows}x{cols}: written past the end"


GEMM_FORMATS = ["q4_0", "q8_0", "aff32", "aff64", "aff128"]


@PROPS
@given(fmt=st.sampled_from(GEMM_FORMATS), M=st.integers(1, 700), K=in_dims, T=st.integers(1, 300),
       ldx_pad=st.integers(0, 3), ldy_pad=st.integers(0, 5), seed=st.integers(0, 2 ** 16))
def test_dequant_gemm_property(gpu, fmt, M, K, T, ldx_pad, ldy_pad, seed):
    """The prefill dequant-GEMM (every tile shape the planner picks) on T
    tokens; Q8_0 and affine weights off the 256 grid are refused with
    GDSLLM_ERR_UNSUPPORTED and write nothing."""
    g = int(fmt[3:]) if fmt.startswith("aff") else 0
    if g and K % g:
        K = max(g, K // g * g)
    ldx, ldy = K + 8 * ldx_pad, M + ldy_pad
    x, xbuf, _ = _x_strided(T, K, ldx, 0, seed + 1, gpu)
    y = _y_padded(T, M, ldy, gpu)
    what = f"{fmt} gemm {M}x{K} T{T} ldx {ldx} ldy {ldy}"
    if g:
        words, scales, biases = syn.affine_q4_weights([M, K], g, gen(seed))
        wd, sd, bd = words.to(gpu), scales.to(gpu), biases.to(gpu)
        rc = capi().gdsllm_dequant_gemm_affine_q4(ptr(wd), ptr(sd), ptr(bd), xbuf.data_ptr(), ptr(y), M, K, g, T, ldx,
                                                  ldy, stream())
        deq = affine_dequant_np(words, scales, biases, g).reshape(M, K)
    else:
        w = (syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights)(M, K, gen(seed))
        wd = w.to(gpu)
        fn = capi().gdsllm_dequant_gemm_q4_0 if fmt == "q4_0" else capi().gdsllm_dequant_gemm_q8_0
        rc = fn(ptr(wd), xbuf.data_ptr(), ptr(y), M, K, T, ldx, ldy, stream())
        deq = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(w)).reshape(M, K)
    torch.cuda.synchronize()
    if fmt != "q4_0" and K % 256:
        assert rc == 2, f"{what}: expected GDSLLM_ERR_UNSUPPORTED (2), got {rc}"
        assert np.all(to_np(y) == SENTINEL), f"{what}: a refused call wrote y"
        return
    check(rc)
    rows, pad = _y_rows(y, T, M, ldy)
    assert np.all(pad == SENTINEL), f"{what}: written outside the output rows"
    _gemv_close(rows, deq, to_np(x), what)


def _h_close(hk, wgq, wuq, x, what):
    """h = fp16(fp16(silu(g)) * u) of the gate/up launches against the
    oracle's g and u: per element within the GEMV bound on g and u (one fp16
    ulp plus 1e-2 of ||w_r * x||) carried through silu (slope below 1.1) and
    the product, plus the roundings of silu and of h; relative L2 over 256
    or more outputs."""
    gx, ux = oq.gemv(wgq, x), oq.gemv(wuq, x)
    gq, uq = gx.astype(np.float16), ux.astype(np.float16)
    h_oracle = (oq.silu_fp16(gq).astype(np.float32) * uq.astype(np.float32)).astype(np.float64)
    hk = np.asarray(hk, dtype=np.float64)
    dg = oq.fp16_ulp(gx) + oq.GEMV_MAX_NORM * oq.row_norms(wgq, x)
    du = oq.fp16_ulp(ux) + oq.GEMV_MAX_NORM * oq.row_norms(wuq, x)
    sx = gx / (1.0 + np.exp(-np.clip(gx, -60, 60)))
    ds = 1.1 * dg + oq.fp16_ulp(sx)
    bound = np.abs(sx) * du + np.abs(ux) * ds + ds * du + 2 * oq.fp16_ulp(h_oracle)
    bad = np.abs(hk - h_oracle) > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} h values beyond the carried GEMV tolerance"
    if hk.size >= 256:
        rel = float(np.linalg.norm(hk - h_oracle) / max(np.linalg.norm(h_oracle), 1e-30))
        assert rel <= oq.GEMV_REL_L2, f"{what}: h rel L2 {rel:.3e}"


@PROPS
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), F=st.integers(1, 600), kb=st.integers(1, 24), T=st.integers(1, 200),
       ldh_pad=st.integers(0, 5), seed=st.integers(0, 2 ** 16))
def test_gate_up_silu_gemm_property(gpu, fmt, F, kb, T, ldh_pad, seed):
    """The prefill gate/up/SiLU launch: h rows of T tokens."""
    K = 256 * kb
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    wg, wu = make(F, K, gen(seed)), make(F, K, gen(seed + 1))
    x = syn.activations(T, K, gen(seed + 2))
    ldh = F + ldh_pad
    h = _y_padded(T, F, ldh, gpu)
    wgd, wud, xd = wg.to(gpu), wu.to(gpu), x.to(gpu)
    fn = (capi().gdsllm_dequant_gemm_gate_up_silu_q4_0 if fmt == "q4_0"
          else capi().gdsllm_dequant_gemm_gate_up_silu_q8_0)
    check(fn(ptr(wgd), ptr(wud), ptr(xd), ptr(h), F, K, T, K, ldh, stream()))
    torch.cuda.synchronize()
    rows, pad = _y_rows(h, T, F, ldh)
    what = f"{fmt} gate/up/SiLU GEMM {F}x{K} T{T} ldh {ldh}"
    assert np.all(pad == SENTINEL), f"{what}: written outside h's rows"
    _h_close(rows, dq(to_np(wg)).reshape(F, K), dq(to_np(wu)).reshape(F, K), to_np(x), what)


# (hidden, ffn) pairs: the row-span gather (hidden % 2048 == 0, ffn/32 in
# {16, 32, 64}) and the general path
MOE_DIMS = [(2048, 512), (2048, 1024), (4096, 512), (4096, 1024), (512, 256), (1024, 512), (768, 256), (2048, 256)]


@settings(PROPS, max_examples=30)
@given(dims=st.sampled_from(MOE_DIMS), g=st.sampled_from([32, 64, 128]), E=st.integers(1, 24),
       k=st.integers(1, 12), bad=st.sampled_from([None, None, None, -1, "E"]), seed=st.integers(0, 2 ** 16))
def test_moe_gather_property(gpu, dims, g, E, k, bad, seed):
    """The top-k expert gather over drawn pools and picks (distinct experts,
    now and then one index outside [0, E)), checked phase by phase and end to
    end against the oracle."""
    H, F = dims
    k = min(k, E)
    gate, up, down = moe_pool(E, H, F, g, seed)
    x = syn.activations(1, H, gen(seed + 1))
    idx = torch.randperm(E, generator=gen(seed + 2))[:k].to(torch.int32)
    if bad is not None:
        idx[int(seed % k)] = -1 if bad == -1 else E
    wts = torch.softmax(torch.randn(k, generator=gen(seed + 3)), 0).to(torch.float16)
    dev = [tuple(t.to(gpu) for t in p) for p in (gate, up, down)]
    y, ws, hk = moe_gather(*dev, x.to(gpu), idx.to(gpu), wts.to(gpu), g, return_workspace=True)
    if all(int(e) < 0 or int(e) >= E for e in idx):
        assert np.all(to_np(y) == 0), "no valid expert: the output is zero"
        return
    check_moe(y, ws, gate, up, down, x, to_np(idx), wts, g, E, hk)


@PROPS
@given(E=st.integers(1, 4096), k=st.integers(1, 64), n=st.integers(1, 8), ld_pad=st.integers(0, 7),
       kind=st.sampled_from(["normal", "ties", "specials"]), seed=st.integers(0, 2 ** 16))
def test_route_topk_property(gpu, E, k, n, ld_pad, kind, seed):
    """On-device top-k + softmax of fp16 logit rows ld apart: the picks equal
    the oracle's (value descending, ties to the lower index, NaN above every
    number, -0 == +0); every weight within one fp16 ulp of the oracle's (the
    device's exp may round the last bit differently)."""
    k = min(k, E)
    ld = E + ld_pad
    rng = np.random.default_rng(seed)
    if kind == "normal":
        v = rng.standard_normal((n, E)).astype(np.float16)
    elif kind == "ties":
        v = (rng.integers(-3, 4, size=(n, E)) * 0.25).astype(np.float16)
    else:
        v = rng.standard_normal((n, E)).astype(np.float16)
        specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 65504.0, -65504.0], dtype=np.float16)
        mask = rng.random((n, E)) < 0.1
        v[mask] = rng.choice(specials, size=int(mask.sum()))
    buf = np.zeros((n, ld), dtype=np.float16)
    buf[:, :E] = v
    logits = torch.from_numpy(buf).reshape(-1).to(gpu)
    idx = torch.empty(n, k, dtype=torch.int32, device=gpu)
    w = torch.empty(n, k, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_moe_route_topk(ptr(logits), E, n, ld, k, ptr(idx), ptr(w), stream()))
    torch.cuda.synchronize()
    ridx, rw = oq.route_topk(v, k)
    what = f"route E{E} k{k} n{n} ld{ld} {kind}"
    np.testing.assert_array_equal(to_np(idx), ridx, err_msg=what)
    got, want = to_np(w).astype(np.float16), np.asarray(rw, dtype=np.float16)
    same = (got.view(np.uint16) == want.view(np.uint16)) | (np.isnan(got) & np.isnan(want))
    ulps = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert np.all(same | (ulps <= 1)), f"{what}: a weight differs by more than one fp16 ulp"


@PROPS
@given(fmt=st.sampled_from(["q4_0", "q8_0"]), vocab=st.integers(1, 3000), hb=st.integers(1, 64),
       n=st.integers(1, 300), seed=st.integers(0, 2 ** 16))
def test_embed_rows_property(gpu, fmt, vocab, hb, n, seed):
    """Row gather of a GGUF table: each row bit-identical to the whole-table
    dequant's row, ids outside [0, vocab) give zeros."""
    hidden = 64 * hb
    raw = (syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights)(vocab, hidden, gen(seed))
    table = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(raw)).reshape(vocab, hidden)
    ids = torch.randint(-3, vocab + 3, (n,), generator=gen(seed + 1), dtype=torch.int64)
    src, ids_dev = raw.to(gpu), ids.to(gpu)
    out = torch.full((n * hidden + 8,), SENTINEL, dtype=torch.float16, device=gpu)
    fn = capi().gdsllm_embed_q4_0 if fmt == "q4_0" else capi().gdsllm_embed_q8_0
    check(fn(ptr(src), ptr(ids_dev), n, vocab, hidden, ptr(out), stream()))
    torch.cuda.synchronize()
    got = to_np(out)
    rows = got[: n * hidden].reshape(n, hidden).view(np.uint16)
    ok_ids = (ids >= 0) & (ids < vocab)
    want = np.zeros((n, hidden), dtype=np.uint16)
    want[ok_ids.numpy()] = table[ids[ok_ids].numpy()].view(np.uint16)
    assert np.array_equal(rows, want), f"{fmt} vocab {vocab} hidden {hidden} n {n}: rows differ"
    assert np.all(got[n * hidden:] == SENTINEL), f"{fmt}: written past the last row"


@PROPS
@given(M=st.integers(1, 700), kc=st.integers(1, 300), B=st.integers(1, 8), ldx_pad=st.integers(0, 9),
       ldy_pad=st.integers(0, 5), seed=st.integers(0, 2 ** 16))
def test_int8_gemv_property(gpu, M, kc, B, ldx_pad, ldy_pad, seed):
    """Per-column int8 weights (fast path for in_dim % 16 == 0 with aligned
    rows, the general kernel otherwise)."""
    K = 8 * kc
    q, sc = syn.int8_weights(M, K, gen(seed))
    ldx, ldy = K + ldx_pad, M + ldy_pad
    x, xbuf, _ = _x_strided(B, K, ldx, 0, seed + 1, gpu)
    y = _y_padded(B, M, ldy, gpu)
    qd, sd = q.to(gpu), sc.to(gpu)
    check(capi().gdsllm_fused_int8_gemv(ptr(qd), ptr(sd), xbuf.data_ptr(), ptr(y), M, K, B, ldx, ldy, stream()))
    torch.cuda.synchronize()
    rows, pad = _y_rows(y, B, M, ldy)
    what = f"int8 {M}x{K} B{B} ldx {ldx} ldy {ldy}"
    assert np.all(pad == SENTINEL), f"{what}: written outside the output rows"
    _gemv_close(rows, oq.dequant_int8(to_np(q), to_np(sc)), to_np(x), what)


# (hidden, ffn): both multiples of 256, as the grouped prefill requires
PREFILL_DIMS = [(512, 256), (1024, 256), (1024, 512), (2048, 512), (768, 512)]


@settings(PROPS, max_examples=25)
@given(dims=st.sampled_from(PREFILL_DIMS), g=st.sampled_from([32, 64, 128]), E=st.integers(1, 40),
       k=st.integers(1, 10), T=st.integers(1, 120), bad=st.integers(0, 3), seed=st.integers(0, 2 ** 16))
def test_moe_prefill_property(gpu, dims, g, E, k, T, bad, seed):
    """The grouped-expert MoE prefill over drawn pools, token counts and picks
    (distinct experts per token, `bad` entries replaced by indices outside [0,
    E)): the device sort, each down row, the fp16 combine bit for bit, and the
    end result against the oracle."""
    H, F = dims
    k = min(k, E)
    gg = gen(seed)
    pools = [syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F])]
    x = syn.activations(T, H, gen(seed + 1))
    rng = np.random.default_rng(seed + 2)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    for i in range(min(bad, T * k - 1)):
        idx.flat[int(rng.integers(1, T * k))] = -1 if i % 2 else E + i
    wts = torch.softmax(torch.randn(T, k, generator=gen(seed + 3)), -1).to(torch.float16)
    dev = [tuple(t.to(gpu) for t in p) for p in pools]
    y, tok, pos, tiles, hbuf, dbuf = moe_prefill(*dev, x.to(gpu), torch.from_numpy(idx).to(gpu), wts.to(gpu), g, T, k)
    check_sort(idx, tok, pos, tiles, E)
    check_moe_prefill(y, tok, pos, hbuf, dbuf, *pools, x, idx, to_np(wts), g, E)
