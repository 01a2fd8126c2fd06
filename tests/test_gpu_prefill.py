"""Parity of the MFMA prefill dequant-GEMM for Q8_0 and affine-Q4 weights (the
Q4_0 cases live in test_gpu_moe_gemm.py), tile-width invariance, and the
grouped-expert MoE prefill, against the oracle, through the C ABI.

The dense GEMMs replace the reference's prefill route dequant -> F.linear
(runtime/llama.py:160-166, runtime/qwen_moe.py:69-73); the MoE prefill
replaces the per-expert loop of runtime/qwen_moe.py:475-492.
"""


import numpy as np
import pytest
import torch

from helpers import (affine_dequant_np, assert_gemv_close, capi, check, check_moe_prefill, check_sort, gen, moe_prefill,
                     oq, ptr, stream, syn, to_np)

pytestmark = pytest.mark.gpu

# (T, M, K): one stage pair, ragged token and row tiles, LLaMA-7B layer shapes
# at a 512-token chunk (the Q8_0 layer of the benchmark's Q8_0 model)
Q8_CASES = [(1, 128, 256), (7, 300, 256), (64, 128, 4096), (100, 260, 1024), (33, 11008, 4096),
            (512, 4096, 4096), (512, 11008, 4096), (512, 4096, 11008)]


@pytest.mark.parametrize("T,M,K", Q8_CASES, ids=[f"T{t}_{m}x{k}" for t, m, k in Q8_CASES])
def test_dequant_gemm_q8_0(gpu, T, M, K):
    w = syn.q8_0_weights(M, K, gen(5200 + M + K))
    x = syn.activations(T, K, gen(5201 + T))
    deq = oq.dequant_q8_0(to_np(w)).reshape(M, K)
    wd, xd = w.to(gpu), x.to(gpu)
    y = torch.empty(T, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_dequant_gemm_q8_0(ptr(wd), ptr(xd), ptr(y), M, K, T, K, M, stream()))
    torch.cuda.synchronize()
    rel, mx = assert_gemv_close(to_np(y), deq, to_np(x), f"q8_0 gemm T{T} {M}x{K}")
    print(f"q8_0 gemm T{T} {M}x{K}: rel={rel:.2e} max={mx:.2e}")


AFF_CASES = [(5, 200, 256, 64), (64, 1024, 4096, 64), (512, 4096, 1024, 64), (100, 260, 2048, 128),
             (70, 384, 512, 32), (512, 1024, 4096, 128), (33, 512, 1024, 32)]


@pytest.mark.parametrize("T,M,K,g", AFF_CASES, ids=[f"T{t}_{m}x{k}_g{g}" for t, m, k, g in AFF_CASES])
def test_dequant_gemm_affine_q4(gpu, T, M, K, g):
    words, scales, biases = syn.affine_q4_weights([M, K], g, gen(5300 + M + g))
    x = syn.activations(T, K, gen(5301 + T))
    deq = affine_dequant_np(words, scales, biases, g).reshape(M, K)
    wd, sd, bd, xd = words.to(gpu), scales.to(gpu), biases.to(gpu), x.to(gpu)
    y = torch.empty(T, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_dequant_gemm_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(xd), ptr(y), M, K, g, T, K, M, stream()))
    torch.cuda.synchronize()
    rel, mx = assert_gemv_close(to_np(y), deq, to_np(x), f"affine gemm T{T} {M}x{K} g{g}")
    print(f"affine gemm T{T} {M}x{K} g{g}: rel={rel:.2e} max={mx:.2e}")


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_dequant_gemm_tile_width_keeps_bits(gpu, fmt):
    """8192 rows at 512 tokens take the 128x128 tile, 64 tokens the 128x64
    tile: the same MFMA sequence per output, so the shared rows are equal bit
    for bit (and within the GEMV tolerance of the oracle).  11008 rows at 512
    tokens take the 256-row tile, whose two K halves add the same products in
    another order: within fp32 reassociation of the 64-token result (one fp16
    ulp plus 2^-16 of ||w_r * x||)."""
    K = 4096
    for M in (8192, 11008):
        w = (syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights)(M, K, gen(5400 + M))
        x = syn.activations(512, K, gen(5401))
        wd, xd = w.to(gpu), x.to(gpu)
        fn = capi().gdsllm_dequant_gemm_q4_0 if fmt == "q4_0" else capi().gdsllm_dequant_gemm_q8_0
        y = torch.empty(512, M, dtype=torch.float16, device=gpu)
        y64 = torch.empty(64, M, dtype=torch.float16, device=gpu)
        check(fn(ptr(wd), ptr(xd), ptr(y), M, K, 512, K, M, stream()))
        check(fn(ptr(wd), ptr(xd), ptr(y64), M, K, 64, K, M, stream()))
        torch.cuda.synchronize()
        deq = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(w)).reshape(M, K)
        if M == 8192:
            assert torch.equal(y[:64].view(torch.int16), y64.view(torch.int16)), "tile width changed the result"
        else:
            a, b = to_np(y)[:64].astype(np.float64), to_np(y64).astype(np.float64)
            bound = oq.fp16_ulp(np.maximum(np.abs(a), np.abs(b))) + oq.row_norms(deq, to_np(x)[:64]) * 2.0 ** -16
            bad = np.abs(a - b) > bound
            assert not bad.any(), f"{int(bad.sum())} outputs apart beyond reassociation, first at {np.argwhere(bad)[0]}"
        assert_gemv_close(to_np(y)[448:], deq, to_np(x)[448:], f"{fmt} gemm {M} rows, last token tile")


# (T, M, K) that the planner gives 256-row tiles on a 256-CU MI355X (the
# 128-row tiles would take two rounds of the CUs, these one): ragged last row
# tile (10000 = 39 x 256 + 16, 12000 = 46 x 256 + 224), ragged last token
# tile, one and four W groups.  Every case also holds on other CU counts: the
# oracle checks whichever tile the planner takes.
ROW256_CASES = [(512, 10000, 256), (500, 12000, 1024), (300, 12000, 1024)]


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0", "affine32", "affine64", "affine128"])
@pytest.mark.parametrize("T,M,K", ROW256_CASES, ids=[f"T{t}_{m}x{k}" for t, m, k in ROW256_CASES])
def test_dequant_gemm_256_row_tile(gpu, fmt, T, M, K):
    x = syn.activations(T, K, gen(5451 + T))
    xd = x.to(gpu)
    y = torch.full((T, M + 3), 7.0, dtype=torch.float16, device=gpu)
    if fmt.startswith("affine"):
        g = int(fmt[6:])
        words, scales, biases = syn.affine_q4_weights([M, K], g, gen(5452 + M + g))
        deq = affine_dequant_np(words, scales, biases, g).reshape(M, K)
        wd, sd, bd = words.to(gpu), scales.to(gpu), biases.to(gpu)
        check(capi().gdsllm_dequant_gemm_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(xd), ptr(y), M, K, g, T, K, M + 3,
                                                   stream()))
    else:
        w = (syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights)(M, K, gen(5450 + M + K))
        deq = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(w)).reshape(M, K)
        wd = w.to(gpu)
        fn = capi().gdsllm_dequant_gemm_q4_0 if fmt == "q4_0" else capi().gdsllm_dequant_gemm_q8_0
        check(fn(ptr(wd), ptr(xd), ptr(y), M, K, T, K, M + 3, stream()))
    torch.cuda.synchronize()
    yh = to_np(y)
    rel, mx = assert_gemv_close(yh[:, :M].copy(), deq, to_np(x), f"{fmt} gemm T{T} {M}x{K}")
    assert (yh[:, M:] == 7.0).all(), "columns past the rows were written"
    print(f"{fmt} gemm 256-row tile T{T} {M}x{K}: rel={rel:.2e} max={mx:.2e}")


@pytest.mark.parametrize("fmt", ["q8_0", "affine"])
def test_dequant_gemm_strided(gpu, fmt):
    """x and y rows with leading dimensions wider than the rows; columns past
    the rows are left alone."""
    T, M, K, ldx, ldy, g = 70, 390, 512, 520, 397, 64
    xfull = syn.activations(T, ldx, gen(5500))
    x = xfull[:, :K]
    xd = xfull.to(gpu)
    y = torch.full((T, ldy), 7.0, dtype=torch.float16, device=gpu)
    if fmt == "q8_0":
        w = syn.q8_0_weights(M, K, gen(5501))
        deq = oq.dequant_q8_0(to_np(w)).reshape(M, K)
        wd = w.to(gpu)
        check(capi().gdsllm_dequant_gemm_q8_0(ptr(wd), ptr(xd), ptr(y), M, K, T, ldx, ldy, stream()))
    else:
        words, scales, biases = syn.affine_q4_weights([M, K], g, gen(5502))
        deq = affine_dequant_np(words, scales, biases, g).reshape(M, K)
        wd, sd, bd = words.to(gpu), scales.to(gpu), biases.to(gpu)
        check(capi().gdsllm_dequant_gemm_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(xd), ptr(y), M, K, g, T, ldx, ldy,
                                                   stream()))
    torch.cuda.synchronize()
    yh = to_np(y)
    assert_gemv_close(yh[:, :M].copy(), deq, to_np(x).copy(), f"{fmt} gemm strided")
    assert (yh[:, M:] == 7.0).all(), "padding columns of y were written"


BIG_X_FMTS = ["q4_0", "q8_0", "affine64", "gate_up_q4_0"]


@pytest.mark.parametrize("fmt", BIG_X_FMTS)
def test_dequant_gemm_x_beyond_4gib(gpu, fmt):
    """x rows 2^23 elements apart over 300 tokens (5 GB): token tiles past
    4 GiB of x read their own rows.  The outputs equal bit for bit those of
    the same call on a compact copy of x (the same tiles and products), and
    sampled rows are checked against the oracle."""
    T, M, K, g = 300, 256, 4096, 64
    ldx = 1 << 23
    x = syn.activations(T, K, gen(5700))
    xbig = torch.empty(T, ldx, dtype=torch.float16, device=gpu)
    assert xbig.numel() * 2 > (1 << 32)
    xbig[:, :K].copy_(x.to(gpu))
    xd = x.to(gpu)
    y_big = torch.full((T, M), float("nan"), dtype=torch.float16, device=gpu)
    y_ref = torch.full((T, M), float("nan"), dtype=torch.float16, device=gpu)
    if fmt in ("q4_0", "q8_0", "gate_up_q4_0"):
        make = syn.q8_0_weights if fmt == "q8_0" else syn.q4_0_weights
        w = make(M, K, gen(5701))
        wd = w.to(gpu)
        deq = (oq.dequant_q8_0 if fmt == "q8_0" else oq.dequant_q4_0)(to_np(w)).reshape(M, K)
        if fmt == "gate_up_q4_0":
            wu = syn.q4_0_weights(M, K, gen(5702))
            wud = wu.to(gpu)
            fn = capi().gdsllm_dequant_gemm_gate_up_silu_q4_0
            for xx, lx, yy in ((xbig, ldx, y_big), (xd, K, y_ref)):
                check(fn(ptr(wd), ptr(wud), ptr(xx), ptr(yy), M, K, T, lx, M, stream()))
        else:
            fn = capi().gdsllm_dequant_gemm_q8_0 if fmt == "q8_0" else capi().gdsllm_dequant_gemm_q4_0
            for xx, lx, yy in ((xbig, ldx, y_big), (xd, K, y_ref)):
                check(fn(ptr(wd), ptr(xx), ptr(yy), M, K, T, lx, M, stream()))
    else:
        words, scales, biases = syn.affine_q4_weights([M, K], g, gen(5703))
        deq = affine_dequant_np(words, scales, biases, g).reshape(M, K)
        wd, sd, bd = words.to(gpu), scales.to(gpu), biases.to(gpu)
        for xx, lx, yy in ((xbig, ldx, y_big), (xd, K, y_ref)):
            check(capi().gdsllm_dequant_gemm_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(xx), ptr(yy), M, K, g, T, lx, M,
                                                       stream()))
    torch.cuda.synchronize()
    del xbig
    assert torch.equal(y_big.view(torch.int16), y_ref.view(torch.int16)), "x beyond 4 GiB changed the result"
    rows = np.array([0, 1, 63, 64, 127, 128, 191, 192, 255, 256, 299])
    if fmt == "gate_up_q4_0":
        du = oq.dequant_q4_0(to_np(wu)).reshape(M, K)
        xr = to_np(x)[rows]
        gq = oq.gemv(deq, xr).astype(np.float16)
        uq = oq.gemv(du, xr).astype(np.float16)
        h = (oq.silu_fp16(gq).astype(np.float32) * uq.astype(np.float32)).astype(np.float64)
        rel = float(np.linalg.norm(to_np(y_big)[rows].astype(np.float64) - h) / np.linalg.norm(h))
        assert rel <= oq.GEMV_REL_L2, f"h rel L2 {rel:.3e}"
    else:
        assert_gemv_close(to_np(y_big)[rows].copy(), deq, to_np(x)[rows].copy(), f"{fmt} gemm, x beyond 4 GiB")


def test_dequant_gemm_unsupported_shapes(gpu):
    """Shapes off the MFMA kernels' grid are refused as unsupported (the caller
    keeps the dequant route), before any launch."""
    y = torch.empty(64, dtype=torch.float16, device=gpu)
    assert capi().gdsllm_dequant_gemm_q8_0(ptr(y), ptr(y), ptr(y), 4, 96, 2, 96, 4, stream()) == 2
    assert b"multiple of 256" in capi().gdsllm_last_error()
    assert capi().gdsllm_dequant_gemm_affine_q4(ptr(y), ptr(y), ptr(y), ptr(y), ptr(y), 4, 256, 256, 2, 256, 4,
                                                stream()) == 2
    assert b"group_size" in capi().gdsllm_last_error()
    # Q8_0 rows whose 32-bit in-tile offsets would pass 4 GiB (in_dim from 15,852,288 on)
    big_k = 15_852_288
    assert capi().gdsllm_dequant_gemm_q8_0(ptr(y), ptr(y), ptr(y), 256, big_k, 2, big_k, 256, stream()) == 2
    assert b"in_dim too large" in capi().gdsllm_last_error()


# ------------------------------------------------------------ MoE prefill --


PREFILL_CASES = [(16, 1024, 512, 64, 4, 37), (64, 2048, 1024, 64, 10, 100), (8, 512, 256, 32, 3, 9),
                 (32, 1024, 256, 128, 8, 65), (4, 1024, 512, 64, 2, 300)]


@pytest.mark.parametrize("E,H,F,g,k,T", PREFILL_CASES, ids=[f"E{e}_H{h}_F{f}_g{g}_k{k}_T{t}" for e, h, f, g, k, t in PREFILL_CASES])
def test_moe_prefill(gpu, E, H, F, g, k, T):
    gg = gen(5600 + E + T)
    gate = syn.affine_q4_weights([E, F, H], g, gg)
    up = syn.affine_q4_weights([E, F, H], g, gg)
    down = syn.affine_q4_weights([E, H, F], g, gg)
    x = syn.activations(T, H, gen(5601 + T))
    idx = np.stack([np.random.default_rng(5602 + t).choice(E, k, replace=False) for t in range(T)]).astype(np.int32)
    wts = torch.softmax(torch.randn(T, k, generator=gen(5603)), -1).to(torch.float16)
    dev = [tuple(t.to(gpu) for t in p) for p in (gate, up, down)]
    y, tok, pos, tiles, hbuf, dbuf = moe_prefill(*dev, x.to(gpu), torch.from_numpy(idx).to(gpu), wts.to(gpu), g, T, k)
    check_sort(idx, tok, pos, tiles, E)
    check_moe_prefill(y, tok, pos, hbuf, dbuf, gate, up, down, x, idx, to_np(wts), g, E)
    # a second run gives the same bits (positions inside an expert may differ)
    y2 = moe_prefill(*dev, x.to(gpu), torch.from_numpy(idx).to(gpu), wts.to(gpu), g, T, k)[0]
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_moe_prefill_out_of_range_experts(gpu):
    E, H, F, g, k, T = 6, 512, 256, 64, 3, 11
    gg = gen(5700)
    pools = [syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F])]
    x = syn.activations(T, H, gen(5701))
    idx = np.stack([np.random.default_rng(5702 + t).choice(E, k, replace=False) for t in range(T)]).astype(np.int32)
    idx[0, 1], idx[3, 0], idx[7, 2] = -1, E, 1 << 20
    wts = torch.softmax(torch.randn(T, k, generator=gen(5703)), -1).to(torch.float16)
    dev = [tuple(t.to(gpu) for t in p) for p in pools]
    y, tok, pos, tiles, hbuf, dbuf = moe_prefill(*dev, x.to(gpu), torch.from_numpy(idx).to(gpu), wts.to(gpu), g, T, k)
    check_sort(idx, tok, pos, tiles, E)
    check_moe_prefill(y, tok, pos, hbuf, dbuf, *pools, x, idx, to_np(wts), g, E)


def test_moe_prefill_cfg2_pool_512_tokens(gpu):
    """The 512-expert pool of the MoE configuration (3.6 GB, generated on the
    device) with a 512-token chunk at top-10: the sort and the combine are
    checked for every token, the GEMMs and the end result on 8 sampled tokens
    (the oracle only dequantizes the experts those tokens pick)."""
    E, H, F, g, k, T = 512, 4096, 1024, 64, 10, 512
    gd = torch.Generator(device=gpu).manual_seed(5800)
    dev = [syn.affine_q4_weights(s, g, gd) for s in ([E, F, H], [E, F, H], [E, H, F])]
    x = syn.activations(T, H, gen(5801))
    idx = np.stack([np.random.default_rng(5802 + t).choice(E, k, replace=False) for t in range(T)]).astype(np.int32)
    wts = torch.softmax(torch.randn(T, k, generator=gen(5803)), -1).to(torch.float16)
    y, tok, pos, tiles, hbuf, dbuf = moe_prefill(*dev, x.to(gpu), torch.from_numpy(idx).to(gpu), wts.to(gpu), g, T, k)
    check_sort(idx, tok, pos, tiles, E)
    sample = sorted(np.random.default_rng(5804).choice(T, 8, replace=False).tolist())

    class Lazy:
        """pool[e] on the CPU, only for the experts the sample touches"""
        def __init__(self, t):
            self.t, self.shape = t, t.shape

        def __getitem__(self, e):
            return self.t[e].cpu()

    pools = [tuple(Lazy(t) for t in p) for p in dev]
    check_moe_prefill(y, tok, pos, hbuf, dbuf, *pools, x, idx, to_np(wts), g, E, sample=sample)
    del dev
    torch.cuda.empty_cache()


def test_runtime_moe_prefill_matches_per_expert_route(gpu, tmp_path):
    """moe_mlp_selective on a prefill chunk: the resident stacked experts (one
    grouped GEMM per phase) and the reference's per-expert buffers from
    load_experts (the MFMA GEMM per projection) against the oracle."""
    from gdsllm_amd.runtime import qwen_moe as qm
    from gdsllm_amd.runtime.torch_bridge import ModelWeights
    from gdsllm_amd.synthetic_model import write_moe_layer

    E, H, F, g, k, T = 8, 2048, 512, 64, 4, 40
    d = str(tmp_path / "moe")
    raw = write_moe_layer(d, experts=E, hidden=H, ffn=F, group=g, seed=5900)
    mw = ModelWeights(d)
    part, _h = mw.load_layer_partial(0)
    full, _hf = mw.load_layer(0)
    x = syn.activations(T, H, gen(5901))
    xd = x.to(gpu).view(1, T, H)
    idx = np.stack([np.random.default_rng(5902 + t).choice(E, k, replace=False) for t in range(T)]).astype(np.int64)
    wts = torch.softmax(torch.randn(T, k, generator=gen(5903)), -1).to(torch.float16)
    it, wt = torch.from_numpy(idx).to(gpu).view(1, T, k), wts.to(gpu).view(1, T, k)
    y_res = qm.moe_mlp_selective(xd, full, None, it, wt, k)
    experts, _eh = mw.load_experts(0, sorted(set(idx.reshape(-1).tolist())))
    y_exp = qm.moe_mlp_selective(xd, part, experts, it, wt, k)
    torch.cuda.synchronize()

    def fn(proj):
        def f(e):
            w, s, b = (t[e] for t in raw[f"mlp.switch_mlp.{proj}"])
            return affine_dequant_np(w, s, b, g).reshape(w.shape[0], -1)
        return f

    ref, _ = oq.moe_prefill(to_np(x), fn("gate_proj"), fn("up_proj"), fn("down_proj"), idx, to_np(wts))
    ref = np.clip(ref, np.float16(-65504), np.float16(65504)).astype(np.float64)
    for name, y in (("resident", y_res), ("per-expert", y_exp)):
        got = to_np(y).reshape(T, H).astype(np.float64)
        rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
        print(f"runtime moe prefill {name}: rel L2 {rel:.2e}")
        assert np.isfinite(got).all() and rel <= oq.GEMV_REL_L2, f"{name}: rel L2 {rel:.3e}"


def test_runtime_q8_0_prefill_projection(gpu):
    """dequant_linear on a Q8_0 weight with a prefill chunk the MFMA GEMM
    serves faster (8192 rows, 128 tokens) takes it."""
    from gdsllm_amd.runtime import ext
    from gdsllm_amd.runtime import llama

    M, K, T = 8192, 4096, 128
    assert llama.prefill_takes_fused_gemm(M, T, K, "q8_0")
    w = syn.q8_0_weights(M, K, gen(6000))
    handle = ext().GdsBufferHandle.from_tensor(w.reshape(-1).to(gpu))
    meta = {"buffer": handle, "shape": [M, K], "gguf_type": "q8_0", "offset": 0}
    x = syn.activations(T, K, gen(6001))
    y = llama.dequant_linear(x.to(gpu).view(2, T // 2, K), {"p.weight": meta}, "p")
    torch.cuda.synchronize()
    assert y.shape == (2, T // 2, M)
    assert_gemv_close(to_np(y).reshape(T, M), oq.dequant_q8_0(to_np(w)).reshape(M, K), to_np(x), "q8_0 dequant_linear")


@pytest.mark.parametrize("fmt,T,F,K", [("q4_0", 64, 4096, 1024), ("q8_0", 96, 8192, 512), ("q4_0", 8, 256, 512)])
def test_runtime_mlp_prefill(gpu, fmt, T, F, K):
    """runtime mlp on a prefill chunk over GGUF weights: where the rule sends
    the projections to the fused GEMM, gate/up/SiLU is one launch
    (fused_gate_up_silu_gemm) and down follows; else the reference's three
    projections and elementwise SiLU.  Against the oracle composition: g and u
    rounded to fp16, torch's fp16 SiLU and product, then down."""
    from gdsllm_amd.runtime import ext, llama

    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    shapes = {"mlp.gate_proj": (F, K), "mlp.up_proj": (F, K), "mlp.down_proj": (K, F)}
    weights, mats = {}, {}
    for i, (name, (m, k)) in enumerate(shapes.items()):
        w = make(m, k, gen(6100 + i))
        mats[name] = dq(to_np(w)).reshape(m, k)
        weights[f"{name}.weight"] = {"buffer": ext().GdsBufferHandle.from_tensor(w.reshape(-1).to(gpu)),
                                     "shape": [m, k], "gguf_type": fmt, "offset": 0}
    fused = llama.prefill_takes_fused_gemm(F, T, K, fmt)
    assert fused == (F >= 2048), "the cases pick both routes"
    calls = []
    real = ext().fused_gate_up_silu_gemm

    def spy(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    ext().fused_gate_up_silu_gemm = spy
    try:
        x = syn.activations(T, K, gen(6110))
        y = llama.mlp(x.to(gpu).view(1, T, K), weights)
        torch.cuda.synchronize()
    finally:
        ext().fused_gate_up_silu_gemm = real
    assert len(calls) == (1 if fused else 0)
    assert y.shape == (1, T, K)
    g = oq.gemv(mats["mlp.gate_proj"], to_np(x)).astype(np.float16)
    u = oq.gemv(mats["mlp.up_proj"], to_np(x)).astype(np.float16)
    h = (oq.silu_fp16(g).astype(np.float32) * u.astype(np.float32)).astype(np.float16)
    want = oq.gemv(mats["mlp.down_proj"], h)
    got = to_np(y).reshape(T, K).astype(np.float64)
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    print(f"mlp prefill {fmt} T{T} {F}x{K}: rel L2 {rel:.2e} ({'fused' if fused else 'route'})")
    assert np.isfinite(got).all() and rel <= oq.GEMV_REL_L2, f"mlp rel L2 {rel:.3e}"


# (fmt, T, F, K): the 7B gate/up shape at a 512-token chunk (128-token tiles)
# and at 64 tokens (64-token tiles), ragged rows and tokens, a short K
# 6000 rows at 500-512 tokens: 128 + 128-row gate/up tiles on a 256-CU GPU
# (one round of 188 tiles against two of 376), ragged last tile
GATE_UP_CASES = [("q4_0", 512, 11008, 4096), ("q4_0", 64, 11008, 4096), ("q4_0", 7, 300, 256),
                 ("q4_0", 100, 1000, 512), ("q8_0", 512, 11008, 4096), ("q8_0", 33, 260, 1024),
                 ("q4_0", 512, 6000, 1024), ("q8_0", 500, 6000, 512)]


@pytest.mark.parametrize("fmt,T,F,K", GATE_UP_CASES, ids=[f"{f}_T{t}_{m}x{k}" for f, t, m, k in GATE_UP_CASES])
def test_dequant_gemm_gate_up_silu(gpu, fmt, T, F, K):
    """h = fp16(fp16(silu(g)) * u) for a prefill chunk in one launch.  (1)
    Against g and u from the dense GEMM: within one fp16 ulp of silu times |u|
    plus one ulp of h (the room the device's expf leaves against numpy's),
    plus what fp32 reassociation of g and u allows (one fp16 ulp plus 2^-16
    of ||w_r * x|| each, carried through silu (slope below 1.1) and the
    product): the two launches may add a row's products in different orders
    (128- or 256-row tiles, 2 or 4 K parts).  (2) End to end against the
    oracle's g and u: relative L2 of h."""
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    gemm = capi().gdsllm_dequant_gemm_q4_0 if fmt == "q4_0" else capi().gdsllm_dequant_gemm_q8_0
    fused = (capi().gdsllm_dequant_gemm_gate_up_silu_q4_0 if fmt == "q4_0"
             else capi().gdsllm_dequant_gemm_gate_up_silu_q8_0)
    wg, wu = make(F, K, gen(5600 + F)), make(F, K, gen(5601 + K))
    x = syn.activations(T, K, gen(5602 + T))
    wgd, wud, xd = wg.to(gpu), wu.to(gpu), x.to(gpu)
    h = torch.full((T, F), float("nan"), dtype=torch.float16, device=gpu)
    check(fused(ptr(wgd), ptr(wud), ptr(xd), ptr(h), F, K, T, K, F, stream()))
    g = torch.empty(T, F, dtype=torch.float16, device=gpu)
    u = torch.empty(T, F, dtype=torch.float16, device=gpu)
    check(gemm(ptr(wgd), ptr(xd), ptr(g), F, K, T, K, F, stream()))
    check(gemm(ptr(wud), ptr(xd), ptr(u), F, K, T, K, F, stream()))
    torch.cuda.synchronize()
    hk = to_np(h).astype(np.float64)
    assert np.all(np.isfinite(hk)), "h not written everywhere"
    gn, un = to_np(g), to_np(u)
    dg, du = dq(to_np(wg)).reshape(F, K), dq(to_np(wu)).reshape(F, K)
    eg = oq.fp16_ulp(gn) + oq.row_norms(dg, to_np(x)) * 2.0 ** -16
    eu = oq.fp16_ulp(un) + oq.row_norms(du, to_np(x)) * 2.0 ** -16
    sg = oq.silu_fp16(gn)
    href = (sg.astype(np.float32) * un.astype(np.float32)).astype(np.float16)
    ua, sa = np.abs(un.astype(np.float64)), np.abs(sg.astype(np.float64))
    bound = (oq.fp16_ulp(sg) * ua + oq.fp16_ulp(href) + 1.1 * eg * (ua + eu) + sa * eu
             + oq.fp16_ulp(sa + 1.1 * eg) * (ua + eu))
    bad = np.abs(hk - href.astype(np.float64)) > bound
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} h values off; first at {np.argwhere(bad)[0]}"
    rows = np.arange(T) if T <= 64 else np.random.default_rng(T).choice(T, 64, replace=False)
    xr = to_np(x)[rows]
    gq = oq.gemv(dg, xr).astype(np.float16)
    uq = oq.gemv(du, xr).astype(np.float16)
    h_oracle = (oq.silu_fp16(gq).astype(np.float32) * uq.astype(np.float32)).astype(np.float64)
    rel = float(np.linalg.norm(hk[rows] - h_oracle) / np.linalg.norm(h_oracle))
    print(f"gate_up_silu {fmt} T{T} {F}x{K}: rel L2 {rel:.2e}")
    assert rel <= oq.GEMV_REL_L2, f"h end-to-end rel L2 {rel:.3e}"
