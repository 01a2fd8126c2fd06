"""Parity of the fused GEMV kernels (Q4_0, Q8_0, affine-Q4) with the oracle,
through the C ABI.  Tolerance: relative L2 <= 2e-3 and per-row error /
||w_r * x||_2 <= 1e-2 (oracle.quant.GEMV_REL_L2 / GEMV_MAX_NORM)."""

import numpy as np
import pytest
import torch

from helpers import (affine_dequant_np, affine_gemv, assert_gemv_close, capi, check, gen, gguf_gemv, on_gpu, oq, ptr,
                     stream, syn, to_np)

pytestmark = pytest.mark.gpu

GGUF_SHAPES = [
    (1, 256), (5, 256), (64, 512), (33, 4096), (4096, 4096), (300, 11008), (130, 8192), (17, 28672),
    # more row groups than resident waves at one window per row: two stage buffers per wave
    (16001, 2048),
    # in_dim % 256 != 0: generic path
    (10, 32), (7, 96), (9, 4128),
]


def _gguf_case(fmt, M, K, B, seed):
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    w = make(M, K, gen(seed))
    x = syn.activations(B, K, gen(seed + 1))
    deq = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(w)).reshape(M, K)
    return w, x, deq


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("M,K", GGUF_SHAPES, ids=[f"{m}x{k}" for m, k in GGUF_SHAPES])
def test_gguf_gemv_b1(gpu, fmt, M, K):
    w, x, deq = _gguf_case(fmt, M, K, 1, 1000 + M + K)
    y = gguf_gemv(fmt, w.to(gpu), x.to(gpu), M, K)
    assert_gemv_close(to_np(y), deq, to_np(x), f"{fmt} {M}x{K}")


# K = 256 (one super-block: most waves of a batched workgroup have no stage),
# ragged row tiles at both tile heights (8200 rows: 32-row tiles with a part
# tile), in_dim % 256 != 0 (generic kernel); super-blocks per row not a
# multiple of the 8 waves (5120: waves with 3 and 2, 2816: 2 and 1) and more
# tiles than workgroups (4100 x 6144).  Rows 8200, 9000, 8300, 8500 and 13003
# split unevenly into 32-row tiles over 256 compute units, so batch 3-8 Q4_0
# takes the x-in-registers kernel there (with part tiles, 1 super-block per
# row, and 20 / 11 super-blocks over 8 waves)
# 24 x 8192, 50 x 5120 and 3000 x 7936 take the 16-wave x-in-registers
# variant (2, 1 and 0 super-blocks per wave, a part tile), as does 2500 x
# 3072 at batch 3-4 (12 super-blocks over 16 waves); 4090 x 9216 takes the
# code kernel with 16-row tiles (one per CU, a part tile), and 9000 x 5120,
# 13003 x 1024 and 8300 x 256 the x-in-registers kernel's two-workgroup form
BATCHED_SHAPES = [(70, 4096), (33, 11008), (20, 96), (24, 8192), (9, 28672), (13003, 1024), (40, 256), (8200, 512),
                  (50, 5120), (1000, 2816), (4100, 6144), (9000, 5120), (8300, 256), (8500, 2816), (3000, 7936),
                  (2500, 3072), (4090, 9216)]


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("B", [2, 3, 4, 5, 7, 8])
@pytest.mark.parametrize("M,K", BATCHED_SHAPES, ids=[f"{m}x{k}" for m, k in BATCHED_SHAPES])
def test_gguf_gemv_batched(gpu, fmt, B, M, K):
    w, x, deq = _gguf_case(fmt, M, K, B, 2000 + B + M)
    y = gguf_gemv(fmt, w.to(gpu), x.to(gpu), M, K)
    assert_gemv_close(to_np(y), deq, to_np(x), f"{fmt} B={B} {M}x{K}")


def test_q4_0_gemv_cfg0_full(gpu):
    """The headline shape: LLaMA-7B gate_proj 11008x4096 at batch 1."""
    w, x, deq = _gguf_case("q4_0", 11008, 4096, 1, 1000)
    y = gguf_gemv("q4_0", w.to(gpu), x.to(gpu), 11008, 4096)
    rel, mx = assert_gemv_close(to_np(y), deq, to_np(x), "cfg0")
    print(f"cfg0 rel_l2={rel:.2e} max_norm={mx:.2e}")


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("B", [2, 4])
@pytest.mark.parametrize("w_off", [2, 0])
def test_gguf_gemv_misaligned_inputs(gpu, fmt, B, w_off):
    """Weights off the 16-byte grid take the generic kernel; x off the 8-byte grid
    takes the element-wise staging (batch 3-8: the staged kernel instead of the
    MFMA one); both must agree with the oracle."""
    M, K = 40, 512
    w, x, deq = _gguf_case(fmt, M, K, B, 77 + B)
    wd = on_gpu(w, gpu, pad_front=w_off)
    xbuf = torch.zeros(B * K + 8, dtype=torch.float16, device=gpu)
    xd = xbuf[1:1 + B * K]
    xd.copy_(x.reshape(-1).to(gpu))
    y = torch.empty(B, M, dtype=torch.float16, device=gpu)
    fn = capi().gdsllm_fused_q4_0_gemv if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv
    check(fn(ptr(wd), ptr(xd), ptr(y), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    assert_gemv_close(to_np(y), deq, to_np(x), f"{fmt} misaligned B={B}")


@pytest.mark.parametrize("B", [2, 3])
def test_gguf_gemv_strided_batch(gpu, B):
    """ldx / ldy larger than the row: rows of x and y taken from wider buffers."""
    M, K = 50, 256
    w, x, deq = _gguf_case("q4_0", M, K, B, 91)
    xw = torch.zeros(B, K + 64, dtype=torch.float16)
    xw[:, :K] = x
    xd = xw.to(gpu)
    y = torch.full((B, M + 10), 7.0, dtype=torch.float16, device=gpu)
    wd = w.to(gpu)  # held across the call: a freed copy could be reused before the kernel reads it
    check(capi().gdsllm_fused_q4_0_gemv(ptr(wd), ptr(xd), ptr(y), M, K, B, K + 64, M + 10, stream()))
    torch.cuda.synchronize()
    yn = to_np(y)
    assert np.all(yn[:, M:] == 7.0), "wrote outside the output rows"
    assert_gemv_close(yn[:, :M], deq, to_np(x), "strided")


@pytest.mark.parametrize("B", [3, 8])
def test_q4_0_batched_strided_x_in_registers(gpu, B):
    """ldx / ldy larger than the row on a shape that takes the x-in-registers
    kernel (9000 rows: 282 tiles of 32 over 256 CUs): x rows come from a wider
    buffer and nothing outside y's rows is written."""
    M, K = 9000, 1536
    w, x, deq = _gguf_case("q4_0", M, K, B, 93 + B)
    xw = torch.zeros(B, K + 128, dtype=torch.float16)
    xw[:, :K] = x
    xd, wd = xw.to(gpu), w.to(gpu)
    y = torch.full((B, M + 24), 7.0, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_q4_0_gemv(ptr(wd), ptr(xd), ptr(y), M, K, B, K + 128, M + 24, stream()))
    torch.cuda.synchronize()
    yn = to_np(y)
    assert np.all(yn[:, M:] == 7.0), "wrote outside the output rows"
    assert_gemv_close(yn[:, :M], deq, to_np(x), f"strided x-in-registers B={B}")


def test_gguf_gemv_closed_forms(gpu):
    """All nibbles 8 -> y = 0 up to the fp32 cancellation of the nibble-offset
    correction (1032*sum(x) per block, |err| ~ 2^-24 * 1032 * |sum x| * d, far
    below one fp16 ulp of a real output); one-hot x -> y = column k of the fp16
    weights exactly (every term is an exact small integer times d)."""
    M, K = 64, 1024
    w = syn.q4_0_weights(M, K, gen(5)).view(-1, 18).clone()
    w[:, 2:] = 0x88
    x = syn.activations(1, K, gen(6))
    y = gguf_gemv("q4_0", w.reshape(M, -1).to(gpu), x.to(gpu), M, K)
    bound = 1e-5 * float(np.abs(to_np(x).astype(np.float64)).sum())
    assert np.max(np.abs(to_np(y).astype(np.float64))) <= bound
    w2 = syn.q4_0_weights(M, K, gen(8))
    deq = oq.dequant_q4_0(to_np(w2)).reshape(M, K)
    for k in (0, 15, 16, 31, 517, K - 1):
        e = torch.zeros(1, K, dtype=torch.float16)
        e[0, k] = 1.0
        y = gguf_gemv("q4_0", w2.to(gpu), e.to(gpu), M, K)
        assert np.array_equal(to_np(y)[0], deq[:, k]), f"column {k}"


AFFINE_SHAPES = [(1024, 4096, 64), (4096, 1024, 64), (64, 4096, 128), (33, 256, 32), (7, 2048, 64), (5, 96, 32),
                 # row-span geometries: 3 / 4 chunks per lane, 16 lanes per row, partial last chunk column
                 (21, 6144, 64), (10, 8192, 128), (19, 512, 32), (13, 3072, 64), (6, 1536, 32),
                 # generic path: in_dim % 32 != 0 or group_size % 32 != 0
                 (9, 104, 8), (6, 128, 16)]


@pytest.mark.parametrize("M,K,g", AFFINE_SHAPES, ids=[f"{m}x{k}g{g}" for m, k, g in AFFINE_SHAPES])
@pytest.mark.parametrize("B", [1, 2, 3, 8])
def test_affine_gemv(gpu, M, K, g, B):
    w, s, b = syn.affine_q4_weights([M, K], g, gen(3000 + M + K + g))
    x = syn.activations(B, K, gen(3001 + B))
    deq = affine_dequant_np(w, s, b, g).reshape(M, K)
    y = affine_gemv(w.to(gpu), s.to(gpu), b.to(gpu), x.to(gpu), M, K, g)
    assert_gemv_close(to_np(y), deq, to_np(x), f"affine {M}x{K} g{g} B{B}")


def test_capi_rejects_bad_shapes_before_launch(gpu):
    lib = capi()
    y = torch.empty(4, dtype=torch.float16, device=gpu)
    assert lib.gdsllm_fused_q4_0_gemv(ptr(y), ptr(y), ptr(y), 4, 48, 1, 48, 4, stream()) == 1
    assert b"multiple of 32" in lib.gdsllm_last_error()
    assert lib.gdsllm_fused_q8_0_gemv(ptr(y), ptr(y), ptr(y), 4, 64, 9, 64, 4, stream()) == 1
    assert lib.gdsllm_fused_affine_q4_gemv(ptr(y), ptr(y), ptr(y), ptr(y), ptr(y), 4, 96, 64, 1, 96, 4, stream()) == 1
    # zero-sized problems are no-ops, as in the reference launchers
    assert lib.gdsllm_fused_q4_0_gemv(None, None, None, 0, 64, 1, 64, 0, stream()) == 0


GROUP_CASES = [((256, 64, 64), 512, 1), ((4096, 1024, 1024), 4096, 1), ((33, 7, 129), 1024, 2), ((100,), 256, 1),
               ((8, 16, 24, 40), 2048, 2), ((5, 0, 9), 512, 1),
               # batch 3-8: Q4_0 takes the x-in-registers kernel over the matrices'
               # 16-row tiles (part tiles, an empty matrix, 1-2 super-blocks per
               # wave, 0 for most waves at in_dim 256); in_dim 544 and 8448 fall
               # back to one GEMV per matrix
               ((33, 7, 129), 1024, 3), ((8, 16, 24, 40), 2048, 5), ((5, 0, 9), 256, 8), ((1000, 200, 200), 4096, 4),
               ((300, 40), 8192, 8), ((17, 64), 7936, 7), ((40, 9), 544, 4), ((20, 30), 8448, 3)]


def _xreg_group(fmt, K, B):
    """Whether a Q4_0 group or gate/up pair at batch 3-8 takes the x-in-registers kernel."""
    return fmt == "q4_0" and B >= 3 and K % 256 == 0 and K <= 8192


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("Ms,K,B", GROUP_CASES, ids=[f"{'-'.join(map(str, m))}x{k}_b{b}" for m, k, b in GROUP_CASES])
def test_gemv_group(gpu, fmt, Ms, K, B):
    """n matrices sharing x in one call: each output matches the oracle, and is
    bit-identical to the single-matrix GEMV of the same matrix (the rows of a
    group are computed exactly like the rows of one matrix), except where a
    Q4_0 group at batch 3-8 takes the x-in-registers kernel: the same block
    products summed in another order than the single GEMV's kernel, so within
    one fp16 ulp plus 2^-16 of ||w_r * x|| of it."""
    import ctypes

    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    ws = [make(M, K, gen(6000 + 17 * i + M)) if M else torch.empty(0, dtype=torch.uint8) for i, M in enumerate(Ms)]
    x = syn.activations(B, K, gen(6100 + K + B))
    xd = x.to(gpu)
    wd = [w.to(gpu) for w in ws]
    ys = [torch.full((B, max(M, 1)), 7.0, dtype=torch.float16, device=gpu) for M in Ms]
    n = len(Ms)
    fn = capi().gdsllm_fused_q4_0_gemv_group if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv_group
    arr_w = (ctypes.c_void_p * n)(*[ptr(w) if M else None for w, M in zip(wd, Ms)])
    arr_y = (ctypes.c_void_p * n)(*[ptr(y) for y in ys])
    dims = (ctypes.c_int64 * n)(*Ms)
    check(fn(n, arr_w, arr_y, dims, ptr(xd), K, B, K, stream()))
    torch.cuda.synchronize()
    for i, M in enumerate(Ms):
        if M == 0:
            assert np.all(to_np(ys[i]) == 7.0), "an empty matrix must not be written"
            continue
        y = to_np(ys[i])
        deq = dq(to_np(ws[i])).reshape(M, K)
        assert_gemv_close(y, deq, to_np(x), f"{fmt} group[{i}] {M}x{K} B{B}")
        single = to_np(gguf_gemv(fmt, wd[i], xd, M, K))
        if not _xreg_group(fmt, K, B):
            assert np.array_equal(y, single), f"group[{i}] differs from the single GEMV"
            continue
        a, b = y.astype(np.float64), single.astype(np.float64)
        bound = oq.fp16_ulp(np.maximum(np.abs(a), np.abs(b))) + oq.row_norms(deq, to_np(x)) * 2.0 ** -16
        bad = np.abs(a - b) > bound
        assert not bad.any(), f"group[{i}]: {int(bad.sum())} outputs apart beyond reassociation"


# Fewer row groups than compute units and in_dim over 2-4 windows of 4096:
# the single-matrix launch splits the windows over waves (2 windows; 3 with a
# ragged last one; 4), and a group of two matrices keeps them in one wave.
SPLIT_SHAPES = [(1024, 8192), (200, 11008), (37, 16384), (513, 12288), (4, 8192)]


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("M,K", SPLIT_SHAPES, ids=[f"{m}x{k}" for m, k in SPLIT_SHAPES])
def test_gemv_split_windows(gpu, fmt, B, M, K):
    """Window sums added in window order after the stages: within the GEMV
    tolerance of the oracle, and within fp32 reassociation of the unsplit
    kernel (the same products; one fp16 ulp plus 2^-16 of ||w_r * x||)."""
    import ctypes

    w, x, deq = _gguf_case(fmt, M, K, B, 6500 + M + K + B)
    wd, xd = w.to(gpu), x.to(gpu)
    y = gguf_gemv(fmt, wd, xd, M, K)
    assert_gemv_close(to_np(y), deq, to_np(x), f"{fmt} split {M}x{K} B{B}")
    ys = [torch.empty(B, M, dtype=torch.float16, device=gpu) for _ in range(2)]
    fn = capi().gdsllm_fused_q4_0_gemv_group if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv_group
    check(fn(2, (ctypes.c_void_p * 2)(ptr(wd), ptr(wd)), (ctypes.c_void_p * 2)(*[ptr(t) for t in ys]),
             (ctypes.c_int64 * 2)(M, M), ptr(xd), K, B, K, stream()))
    torch.cuda.synchronize()
    a, b = to_np(y).astype(np.float64), to_np(ys[0]).astype(np.float64)
    norms = oq.row_norms(deq, to_np(x))
    bound = oq.fp16_ulp(np.maximum(np.abs(a), np.abs(b))) + norms * 2.0 ** -16
    bad = np.abs(a - b) > bound
    assert not bad.any(), f"{int(bad.sum())} outputs apart beyond reassociation, first at {np.argwhere(bad)[0]}"


GATE_UP_CASES = [(300, 1024, 1), (11008, 4096, 1), (7, 256, 2), (1025, 2048, 2), (4096, 11008, 1), (16001, 1024, 1),
                 # batch 1 on one 12-wave workgroup per CU (11008 x 4096 too)
                 (11501, 2048, 1),
                 # batch 3-8: Q4_0 pairs 8 gate and 8 up rows per tile of the
                 # x-in-registers kernel (part tiles at 300, 1037, 7 and 129
                 # rows); Q8_0 and in_dim 11008 are refused
                 (300, 1024, 3), (11008, 4096, 4), (1037, 8192, 8), (7, 256, 5), (129, 7936, 7), (4096, 11008, 3)]


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("M,K,B", GATE_UP_CASES, ids=[f"{m}x{k}_b{b}" for m, k, b in GATE_UP_CASES])
def test_gate_up_silu(gpu, fmt, M, K, B):
    """h = fp16(silu(g) * u) in one call.  (1) Against g, u from the single
    GEMV (same per-row sums, bit for bit): h within one fp16 ulp of silu times
    |u| plus one ulp of h, the room the device's expf leaves against numpy's.
    (2) End to end against the oracle's g, u: relative L2 of h.  At batch 3-8
    g and u come from the grouped launch of the two matrices, whose rows the
    pair launch computes the same way; the shapes no batch 3-8 launch serves
    are refused with GDSLLM_ERR_UNSUPPORTED."""
    import ctypes

    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    wg, wu = make(M, K, gen(7000 + M)), make(M, K, gen(7001 + K))
    x = syn.activations(B, K, gen(7002 + B))
    wgd, wud, xd = wg.to(gpu), wu.to(gpu), x.to(gpu)
    h = torch.empty(B, M, dtype=torch.float16, device=gpu)
    fn = capi().gdsllm_fused_q4_0_gate_up_silu if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gate_up_silu
    rc = fn(ptr(wgd), ptr(wud), ptr(xd), ptr(h), M, K, B, K, M, stream())
    if B >= 3 and not _xreg_group(fmt, K, B):
        assert rc == 2, f"batch {B} {fmt} {M}x{K}: expected GDSLLM_ERR_UNSUPPORTED (2), got {rc}"
        return
    check(rc)
    torch.cuda.synchronize()
    hk = to_np(h).astype(np.float64)
    if B >= 3:
        gd, ud = (torch.empty(B, M, dtype=torch.float16, device=gpu) for _ in range(2))
        check(capi().gdsllm_fused_q4_0_gemv_group(2, (ctypes.c_void_p * 2)(ptr(wgd), ptr(wud)),
                                                  (ctypes.c_void_p * 2)(ptr(gd), ptr(ud)), (ctypes.c_int64 * 2)(M, M),
                                                  ptr(xd), K, B, K, stream()))
        torch.cuda.synchronize()
        g, u = to_np(gd), to_np(ud)
    else:
        g, u = to_np(gguf_gemv(fmt, wgd, xd, M, K)), to_np(gguf_gemv(fmt, wud, xd, M, K))
    sg = oq.silu_fp16(g)
    href = (sg.astype(np.float32) * u.astype(np.float32)).astype(np.float16)
    bound = oq.fp16_ulp(sg) * np.abs(u.astype(np.float64)) + oq.fp16_ulp(href)
    bad = np.abs(hk - href.astype(np.float64)) > bound
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} h values off; first at {np.argwhere(bad)[0]}"
    gq = oq.gemv(dq(to_np(wg)).reshape(M, K), to_np(x)).astype(np.float16)
    uq = oq.gemv(dq(to_np(wu)).reshape(M, K), to_np(x)).astype(np.float16)
    h_oracle = (oq.silu_fp16(gq).astype(np.float32) * uq.astype(np.float32)).astype(np.float64)
    rel = float(np.linalg.norm(hk - h_oracle) / np.linalg.norm(h_oracle))
    assert rel <= oq.GEMV_REL_L2, f"h end-to-end rel L2 {rel:.3e}"


@pytest.mark.parametrize("B", [3, 8])
def test_batched_group_and_pair_strides_and_alignment(gpu, B):
    """Batch 3-8 Q4_0 group and gate/up pair with x rows ldx > in_dim apart
    and h rows ldh > out_dim apart (the pair writes only its columns), then
    x off the 16-byte grid: the group falls back to one GEMV per matrix (the
    single GEMVs' bits), the pair is refused with GDSLLM_ERR_UNSUPPORTED."""
    import ctypes

    M, K = 300, 2048
    ldx, ldh = K + 72, M + 40
    wg, wu = syn.q4_0_weights(M, K, gen(7300)), syn.q4_0_weights(M, K, gen(7301))
    x = syn.activations(B, K, gen(7302))
    wgd, wud = wg.to(gpu), wu.to(gpu)
    xbuf = torch.zeros(B * ldx + 8, dtype=torch.float16, device=gpu)
    xs = xbuf[: B * ldx].view(B, ldx)
    xs[:, :K].copy_(x.to(gpu))
    g, u = (torch.empty(B, M, dtype=torch.float16, device=gpu) for _ in range(2))
    grp = capi().gdsllm_fused_q4_0_gemv_group
    check(grp(2, (ctypes.c_void_p * 2)(ptr(wgd), ptr(wud)), (ctypes.c_void_p * 2)(ptr(g), ptr(u)),
              (ctypes.c_int64 * 2)(M, M), ptr(xs), K, B, ldx, stream()))
    hbuf = torch.full((B, ldh), 5.0, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_q4_0_gate_up_silu(ptr(wgd), ptr(wud), ptr(xs), ptr(hbuf), M, K, B, ldx, ldh, stream()))
    torch.cuda.synchronize()
    dq = oq.dequant_q4_0
    for t, w, part in ((g, wg, "gate"), (u, wu, "up")):
        assert_gemv_close(to_np(t), dq(to_np(w)).reshape(M, K), to_np(x), f"strided group {part} B{B}")
    hk = to_np(hbuf).astype(np.float64)
    assert np.all(hk[:, M:] == 5.0), "the pair wrote past out_dim"
    sg = oq.silu_fp16(to_np(g))
    href = (sg.astype(np.float32) * to_np(u).astype(np.float32)).astype(np.float16)
    bound = oq.fp16_ulp(sg) * np.abs(to_np(u).astype(np.float64)) + oq.fp16_ulp(href)
    assert not (np.abs(hk[:, :M] - href.astype(np.float64)) > bound).any(), "strided pair h"
    # x off the 16-byte grid (ldx stays a multiple of 8 elements)
    xo = xbuf[1: 1 + B * ldx].view(B, ldx)
    xo[:, :K].copy_(x.to(gpu))
    g2, u2 = (torch.empty(B, M, dtype=torch.float16, device=gpu) for _ in range(2))
    check(grp(2, (ctypes.c_void_p * 2)(ptr(wgd), ptr(wud)), (ctypes.c_void_p * 2)(ptr(g2), ptr(u2)),
              (ctypes.c_int64 * 2)(M, M), ptr(xo), K, B, ldx, stream()))
    gs = torch.empty(B, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_q4_0_gemv(ptr(wgd), ptr(xo), ptr(gs), M, K, B, ldx, M, stream()))
    torch.cuda.synchronize()
    assert torch.equal(g2, gs), "unaligned x: the group's fallback differs from the single GEMV"
    assert_gemv_close(to_np(u2), dq(to_np(wu)).reshape(M, K), to_np(x), f"unaligned group up B{B}")
    rc = capi().gdsllm_fused_q4_0_gate_up_silu(ptr(wgd), ptr(wud), ptr(xo), ptr(hbuf), M, K, B, ldx, ldh, stream())
    assert rc == 2, f"unaligned x at batch {B}: expected GDSLLM_ERR_UNSUPPORTED (2), got {rc}"
