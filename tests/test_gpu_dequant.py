"""Bit-exact parity of the HIP dequant kernels with the oracle (through the C ABI)."""

import numpy as np
import pytest
import torch

from helpers import affine_dequant_np, double_rounding_cases, capi, check, gen, on_gpu, oq, ptr, stream, syn, to_np

pytestmark = pytest.mark.gpu


def _bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def _dequant_gguf(fmt, raw_cpu, dev, pad_src=0, pad_dst=0):
    nblk = raw_cpu.numel() // (18 if fmt == "q4_0" else 34)
    src = on_gpu(raw_cpu, dev, pad_src)
    dst_buf = torch.zeros(nblk * 32 + 16, dtype=torch.float16, device=dev)
    dst = dst_buf[pad_dst:pad_dst + nblk * 32]
    fn = capi().gdsllm_dequant_q4_0 if fmt == "q4_0" else capi().gdsllm_dequant_q8_0
    check(fn(ptr(src), ptr(dst), nblk, stream()))
    torch.cuda.synchronize()
    return to_np(dst)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("rows,cols", [(1, 32), (1, 64), (3, 96), (7, 4096), (11008, 4096)])
def test_gguf_dequant_bit_exact(gpu, fmt, rows, cols):
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    raw = make(rows, cols, gen(100 + rows + cols))
    got = _dequant_gguf(fmt, raw, gpu)
    ref = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(raw))
    assert np.array_equal(_bits(got), _bits(ref)), f"{fmt} {rows}x{cols}: dequant differs from oracle"


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("pad_src,pad_dst", [(2, 0), (0, 1), (1, 3)])
def test_gguf_dequant_misaligned_paths(gpu, fmt, pad_src, pad_dst):
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    raw = make(5, 96, gen(7))
    got = _dequant_gguf(fmt, raw, gpu, pad_src, pad_dst)
    ref = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(raw))
    assert np.array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_gguf_dequant_special_scales(gpu, fmt):
    """Signed zeros, subnormal / huge / negative scales (overflow to inf) round like the reference."""
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    bb = 18 if fmt == "q4_0" else 34
    raw = make(1, 32 * 8, gen(3)).view(-1, bb).clone()
    specials = np.array([0.0, -0.0, -0.5, 6.0e-8, -3.0e-6, 65504.0, -65504.0, 1.0], dtype=np.float16)
    raw[:, :2] = torch.from_numpy(specials.view(np.uint8).reshape(8, 2).copy())
    raw[0, 2:] = 0x88  # q = 8 everywhere: d*(q-8) = +-0 in Q4_0
    got = _dequant_gguf(fmt, raw.reshape(-1), gpu)
    ref = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(raw.reshape(-1)))
    assert np.array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_gguf_dequant_nonfinite_scales(gpu, fmt):
    """Infinite and NaN scales: +-inf where the reference's fp32 product is
    infinite, NaN where it is NaN (inf * 0 at q = 8, any NaN d).  NaN payloads
    differ between processors (x86, this GPU and CUDA each make their own
    default NaN), so NaN outputs are compared as NaN and every other output
    bit for bit.  Q8_0 codes include -128 and 127."""
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    bb = 18 if fmt == "q4_0" else 34
    raw = make(1, 32 * 8, gen(4)).view(-1, bb).clone()
    specials = np.array([np.inf, -np.inf, np.nan, -np.nan, 1.0, -1.0, np.inf, 2.0], dtype=np.float16)
    bits = specials.view(np.uint16).copy()
    bits[7] = 0x7C01  # signaling NaN
    raw[:, :2] = torch.from_numpy(bits.view(np.uint8).reshape(8, 2).copy())
    raw[0, 2:] = 0x88 if fmt == "q4_0" else 0  # d*0: NaN for an infinite d
    raw[6, 2:] = torch.tensor([0x80, 0x7F] * ((bb - 2) // 2), dtype=torch.uint8) if fmt == "q8_0" else 0x0F
    got = _dequant_gguf(fmt, raw.reshape(-1), gpu)
    ref = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(raw.reshape(-1)))
    nan = np.isnan(ref)
    assert nan.any() and np.isinf(ref).any()
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(_bits(got)[~nan], _bits(ref)[~nan])


@pytest.mark.parametrize("rows,cols,g", [(1, 64, 64), (4, 1024, 64), (1024, 4096, 64), (3, 256, 128), (5, 96, 32),
                                         (2, 64, 8), (3, 48, 16)])
def test_affine_dequant_bit_exact(gpu, rows, cols, g):
    w, s, b = syn.affine_q4_weights([rows, cols], g, gen(rows * 7 + cols))
    wd, sd, bd = w.to(gpu), s.to(gpu), b.to(gpu)
    out = torch.empty(rows * cols, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_dequant_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(out), rows * cols, cols, g, stream()))
    torch.cuda.synchronize()
    ref = affine_dequant_np(w, s, b, g)
    assert np.array_equal(_bits(to_np(out)), _bits(ref))


def test_affine_dequant_misaligned_dst(gpu):
    w, s, b = syn.affine_q4_weights([3, 128], 64, gen(11))
    wd, sd, bd = w.to(gpu), s.to(gpu), b.to(gpu)
    buf = torch.zeros(3 * 128 + 8, dtype=torch.float16, device=gpu)
    out = buf[1:1 + 3 * 128]
    check(capi().gdsllm_dequant_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(out), 3 * 128, 128, 64, stream()))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(to_np(out)), _bits(affine_dequant_np(w, s, b, 64)))


def test_affine_dequant_special_values(gpu):
    w, s, b = syn.affine_q4_weights([1, 8 * 64], 64, gen(5))
    s[:] = torch.tensor([0.0, -0.0, 65504.0, -1.0, 6.0e-8, 0.25, 1e-3, -2.0], dtype=torch.float16)
    b[:] = torch.tensor([-0.0, 0.0, 65504.0, 1.0, -6.0e-8, -1e4, 3.0, 0.5], dtype=torch.float16)
    wd, sd, bd = w.to(gpu), s.to(gpu), b.to(gpu)
    out = torch.empty(8 * 64, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_dequant_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(out), 8 * 64, 8 * 64, 64, stream()))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(to_np(out)), _bits(affine_dequant_np(w, s, b, 64)))


def test_affine_dequant_rounds_through_fp32(gpu):
    """Values where rounding nib*s+b straight to fp16 differs from the
    reference's fp32-then-fp16: the kernel must give the latter."""
    nib, scales, biases = double_rounding_cases(256, 21)
    n = len(nib)
    wd = torch.from_numpy(nib.view(np.int32).copy()).to(gpu)  # element 8i = nib, other nibbles 0
    sd, bd = torch.from_numpy(scales.copy()).to(gpu), torch.from_numpy(biases.copy()).to(gpu)
    out = torch.empty(8 * n, dtype=torch.float16, device=gpu)
    check(capi().gdsllm_dequant_affine_q4(ptr(wd), ptr(sd), ptr(bd), ptr(out), 8 * n, 8, 8, stream()))
    torch.cuda.synchronize()
    ref = oq.dequant_affine_q4(nib, scales, biases, 8 * n, 8)
    assert np.array_equal(_bits(to_np(out)), _bits(ref))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("vocab,hidden,n", [(300, 64, 37), (97, 192, 5), (1000, 4096, 129), (3, 64, 1)])
def test_embed_rows_bit_exact(gpu, fmt, vocab, hidden, n):
    """Row gather of a GGUF table through the C ABI: each row is bit-identical
    to that row of the whole-table dequant; ids outside [0, vocab) give zeros."""
    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    raw = make(vocab, hidden, gen(300 + vocab + hidden))
    table = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(raw)).reshape(vocab, hidden)
    ids = torch.randint(-2, vocab + 2, (n,), generator=gen(301 + n), dtype=torch.int64)
    ids[0] = vocab - 1
    src, ids_dev = on_gpu(raw, gpu), ids.to(gpu)
    out = torch.full((n, hidden), float("nan"), dtype=torch.float16, device=gpu)
    fn = capi().gdsllm_embed_q4_0 if fmt == "q4_0" else capi().gdsllm_embed_q8_0
    check(fn(ptr(src), ptr(ids_dev), n, vocab, hidden, ptr(out), stream()))
    torch.cuda.synchronize()
    got = _bits(to_np(out))
    for r, t in enumerate(ids.tolist()):
        want = _bits(table[t]) if 0 <= t < vocab else np.zeros(hidden, np.uint16)
        assert np.array_equal(got[r], want), f"{fmt} row {r} (token {t})"
