"""Per-column int8 weights (runtime/llama.py:162-165): the bit-exact dequant
and the fused GEMV through the C ABI, the extension's int8_linear op, and the
runtime dispatch, against the oracle (oracle/quant.py dequant_int8, gemv)."""

import numpy as np
import pytest
import torch

from gdsllm_amd.runtime import ext
from gdsllm_amd.runtime.llama import dequant_linear
from helpers import assert_gemv_close, capi, check, gen, on_gpu, oq, ptr, stream, syn, to_np

pytestmark = pytest.mark.gpu


def _case(M, K, seed, s_range=(0.001, 0.004)):
    q, s = syn.int8_weights(M, K, gen(seed), s_range)
    return q, s, oq.dequant_int8(to_np(q), to_np(s))


@pytest.mark.parametrize("M,K", [(1, 16), (3, 48), (5, 40), (64, 4096), (4096, 11008), (11008, 4096)])
def test_dequant_int8_bit_exact(gpu, M, K):
    q, s, want = _case(M, K, 10 + M + K)
    out = torch.empty(M, K, dtype=torch.float16, device=gpu)
    qd, sd = q.to(gpu), s.to(gpu)  # held across the call: a freed copy could be reused by the next one
    check(capi().gdsllm_dequant_int8(ptr(qd), ptr(sd), ptr(out), M, K, stream()))
    torch.cuda.synchronize()
    assert np.array_equal(to_np(out).view(np.uint16), want.view(np.uint16)), f"{M}x{K}"


def test_dequant_int8_special_scales(gpu):
    """Signed zeros, subnormal, huge (overflow to inf) and negative scales round
    like the reference's fp32 product + .half()."""
    special = np.array([0.0, -0.0, -0.5, 6.0e-8, -3.0e-6, 65504.0, -65504.0, 1.0, 0.0123, 7.1e3,
                        1e-3, -1e-3, 2.0, -2.0, 0.25, 300.0], dtype=np.float16)
    q = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8).view(256, 1).repeat(1, 16)
    s = torch.from_numpy(special.reshape(1, 16))
    want = oq.dequant_int8(to_np(q), special)
    qd = q.to(gpu)
    for pad in (0, 2):  # fast path, then the element-wise path (scale off the 16-byte grid)
        sd = on_gpu(s, gpu, pad_front=pad)
        out = torch.empty(256, 16, dtype=torch.float16, device=gpu)
        check(capi().gdsllm_dequant_int8(ptr(qd), ptr(sd), ptr(out), 256, 16, stream()))
        torch.cuda.synchronize()
        assert np.array_equal(to_np(out).view(np.uint16), want.view(np.uint16)), f"pad {pad}"


@pytest.mark.parametrize("B", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("M,K", [(1, 16), (7, 48), (33, 4096), (4096, 11008), (300, 40), (257, 1040)])
def test_int8_gemv(gpu, B, M, K):
    q, s, w = _case(M, K, 20 + M + K + B)
    x = syn.activations(B, K, gen(21 + B))
    y = torch.empty(B, M, dtype=torch.float16, device=gpu)
    qd, sd, xd = q.to(gpu), s.to(gpu), x.to(gpu)
    check(capi().gdsllm_fused_int8_gemv(ptr(qd), ptr(sd), ptr(xd), ptr(y), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    assert_gemv_close(to_np(y), w, to_np(x), f"int8 B={B} {M}x{K}")


def test_int8_gemv_strided_and_misaligned(gpu):
    """x / y rows from wider buffers; x off the 16-byte grid takes the generic
    kernel; both agree with the oracle and write nothing outside y's rows."""
    M, K, B = 50, 256, 3
    q, s, w = _case(M, K, 31)
    x = syn.activations(B, K, gen(32))
    xw = torch.zeros(B, K + 64, dtype=torch.float16)
    xw[:, :K] = x
    y = torch.full((B, M + 10), 7.0, dtype=torch.float16, device=gpu)
    qd, sd, xd = q.to(gpu), s.to(gpu), xw.to(gpu)
    check(capi().gdsllm_fused_int8_gemv(ptr(qd), ptr(sd), ptr(xd), ptr(y), M, K, B, K + 64, M + 10, stream()))
    torch.cuda.synchronize()
    yn = to_np(y)
    assert np.all(yn[:, M:] == 7.0)
    assert_gemv_close(yn[:, :M], w, to_np(x), "int8 strided")
    xbuf = torch.zeros(B * K + 8, dtype=torch.float16, device=gpu)
    xm = xbuf[1:1 + B * K]
    xm.copy_(x.reshape(-1).to(gpu))
    y2 = torch.empty(B, M, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_fused_int8_gemv(ptr(qd), ptr(sd), ptr(xm), ptr(y2), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    assert_gemv_close(to_np(y2), w, to_np(x), "int8 misaligned x")


@pytest.mark.parametrize("rows", [1, 4, 20])
def test_int8_linear_op_and_dispatch(gpu, rows):
    """gds_io_ext.int8_linear and dequant_linear on an int8 weight dict: the
    fused GEMV for up to 8 rows of x, the bit-exact dequant + GEMM above."""
    M, K = 96, 512
    q, s, w = _case(M, K, 40 + rows)
    x = syn.activations(rows, K, gen(41 + rows))
    qd, sd, xd = q.to(gpu), s.to(gpu), x.to(gpu)
    weights = {"mlp.down_proj.weight": qd, "mlp.down_proj.scale": sd}
    y = dequant_linear(xd.view(1, rows, K), weights, "mlp.down_proj")
    assert y.shape == (1, rows, M) and y.dtype == torch.float16
    assert_gemv_close(to_np(y).reshape(rows, M), w, to_np(x), f"dequant_linear int8 rows={rows}")
    y2 = ext().int8_linear(qd, sd, xd)
    assert y2.shape == (rows, M)
    assert_gemv_close(to_np(y2), w, to_np(x), f"int8_linear rows={rows}")
    full = ext().dequant_int8(qd, sd)
    assert np.array_equal(to_np(full).view(np.uint16), w.view(np.uint16))


def test_int8_linear_prefill_row_chunks(gpu):
    """Above 512 MiB of fp16 weights, prefill dequantizes in row chunks: rows on
    both sides of every chunk boundary agree with the oracle."""
    M, K, rows = 40000, 8192, 9
    g = torch.Generator().manual_seed(51)
    q = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    s = torch.empty(1, K).uniform_(0.001, 0.004, generator=g).to(torch.float16)
    x = syn.activations(rows, K, gen(52))
    qd, sd, xd = q.to(gpu), s.to(gpu), x.to(gpu)
    y = to_np(ext().int8_linear(qd, sd, xd))
    assert y.shape == (rows, M)
    step = (512 << 20) // (2 * K)
    check_rows = sorted({0, step - 1, step, M - 1})
    w = oq.dequant_int8(to_np(q[check_rows]), to_np(s))
    assert_gemv_close(y[:, check_rows], w, to_np(x), "int8 prefill chunk boundaries")
