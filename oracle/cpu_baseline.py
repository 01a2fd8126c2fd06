"""CPU baseline of the quantized GEMV — TEST / BENCH INFRASTRUCTURE ONLY.

Only `bench.py`'s cpu_baseline leg and `tests/` use this module; the product
(`gdsllm_amd/`) never imports it.

The reference has no CPU path for these formats (its dequant exists only as
CUDA, runtime/gguf_dequant.cu:76-118), so the CPU baseline is a multithreaded
torch restatement of what its decode path computes for one Q4_0 projection:
the bit-exact fp16 dequant of runtime/gguf_dequant.cu:84-107 followed by
F.linear in fp32 and a cast to fp16 (the dequant -> F.linear route of
runtime/llama.py:160-166, with fp32 accumulation).  tests/test_oracle.py pins
its dequant bit for bit against oracle.quant.dequant_q4_0.
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
