"""CPU baseline of the quantized GEMVs — TEST / BENCH INFRASTRUCTURE ONLY.

Only `bench.py`'s cpu_baseline leg and `tests/` use this module; the product
(`gdsllm_amd/`) never imports it.

The reference has no CPU path for these formats (its dequant exists only as
CUDA, runtime/gguf_dequant.cu:76-118), so the CPU baseline is a multithreaded
torch restatement of what its decode path computes for one Q4_0 projection:
the bit-exact fp16 dequant of runtime/gguf_dequant.cu:84-107 followed by
F.linear in fp32 and a cast to fp16 (the dequant -> F.linear route of
runtime/llama.py:160-166, with fp32 accumulation).  The same for Q8_0
(gguf_dequant.cu:40-57) and affine-Q4 (affine_q4_dequant.cu:50-58), and the
decode MoE loop of runtime/qwen_moe.py:455-474 over those GEMVs.
tests/test_oracle.py pins every dequant bit for bit against oracle.quant and
the GEMVs and the MoE loop against the oracle's tolerance.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def dequant_q4_0(raw: torch.Tensor) -> torch.Tensor:
    """uint8 Q4_0 blocks (any shape, 18 bytes per block) -> fp16 [n_blocks*32].

    d*(q-8) is exact in fp32 (11-bit by 4-bit), so casting the fp32 product to
    fp16 is the single round-to-nearest-even the CUDA kernel performs."""
    b = raw.reshape(-1, 18)
    d = b[:, :2].contiguous().view(torch.float16).to(torch.float32)  # [n, 1]
    qs = b[:, 2:].to(torch.int16)
    lo = ((qs & 15) - 8).to(torch.float32)
    hi = ((qs >> 4) - 8).to(torch.float32)
    return torch.cat([d * lo, d * hi], dim=1).to(torch.float16).reshape(-1)


def q4_0_gemv(raw: torch.Tensor, x: torch.Tensor, out_dim: int, in_dim: int) -> torch.Tensor:
    """y = fp16(x . dequant(W)^T) with fp32 accumulation; x fp16 [B, in_dim]."""
    w = dequant_q4_0(raw).view(out_dim, in_dim)
    return F.linear(x.to(torch.float32), w.to(torch.float32)).to(torch.float16)


def dequant_q8_0(raw: torch.Tensor) -> torch.Tensor:
    """uint8 Q8_0 blocks (34 bytes: fp16 d, i8 qs[32]) -> fp16 [n_blocks*32]
    (runtime/gguf_dequant.cu:40-57): d*q is exact in fp32, one fp16 rounding."""
    b = raw.reshape(-1, 34)
    d = b[:, :2].contiguous().view(torch.float16).to(torch.float32)
    q = b[:, 2:].contiguous().view(torch.int8).to(torch.float32)
    return (d * q).to(torch.float16).reshape(-1)


def q8_0_gemv(raw: torch.Tensor, x: torch.Tensor, out_dim: int, in_dim: int) -> torch.Tensor:
    w = dequant_q8_0(raw).view(out_dim, in_dim)
    return F.linear(x.to(torch.float32), w.to(torch.float32)).to(torch.float16)


def dequant_affine_q4(words: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int) -> torch.Tensor:
    """Affine-Q4 words (uint32 bits as int32 [rows, cols/8], nibbles LSB first)
    and fp16 scales/biases [rows, cols/g] -> fp16 [rows, cols]
    (runtime/affine_q4_dequant.cu:50-58: nib*s + b in fp32, then one fp16
    rounding; nib*s is exact, so fp32 fma and mul+add agree)."""
    rows = words.shape[0]
    w = words.reshape(rows, -1).to(torch.int32)
    per_word = group_size // 8  # words per group (converter group sizes are multiples of 8)
    s = scales.reshape(rows, -1).to(torch.float32).repeat_interleave(per_word, dim=1)
    b = biases.reshape(rows, -1).to(torch.float32).repeat_interleave(per_word, dim=1)
    out = torch.empty(rows, w.shape[1], 8, dtype=torch.float16)
    for n in range(8):  # nibble n of each word (an arithmetic int32 shift keeps the low bits)
        out[:, :, n] = (((w >> (4 * n)) & 15).to(torch.float32) * s + b).to(torch.float16)
    return out.reshape(rows, -1)


def affine_gemv(words, scales, biases, x: torch.Tensor, group_size: int) -> torch.Tensor:
    w = dequant_affine_q4(words, scales, biases, group_size)
    return F.linear(x.to(torch.float32), w.to(torch.float32)).to(torch.float16)


def moe_gather_decode(gate, up, down, x: torch.Tensor, idx, weights: torch.Tensor, group_size: int) -> torch.Tensor:
    """The decode branch of moe_mlp_selective (runtime/qwen_moe.py:455-474) for
    one token: for each selected expert in pick order, gate and up GEMVs,
    h = silu(g) * u, the down GEMV, and acc += w_k * down, every op's result an
    fp16 tensor as in the reference.  gate/up/down: (words, scales, biases) of
    the selected experts, indexed by idx."""
    acc = torch.zeros(1, down[0].shape[1], dtype=torch.float16)
    for k, e in enumerate(idx):
        g = affine_gemv(gate[0][e], gate[1][e], gate[2][e], x, group_size)
        u = affine_gemv(up[0][e], up[1][e], up[2][e], x, group_size)
        h = (F.silu(g.to(torch.float32)).to(torch.float16).to(torch.float32) * u.to(torch.float32)).to(torch.float16)
        d = affine_gemv(down[0][e], down[1][e], down[2][e], h, group_size)
        acc = (acc.to(torch.float32) + (weights[k].to(torch.float32) * d.to(torch.float32)).to(torch.float16)
               .to(torch.float32)).to(torch.float16)
    return acc
