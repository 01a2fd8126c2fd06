"""Embedding lookup and lm_head projection of the layer-by-layer schedulers.

Mirrors _embed_tokens and _lm_head_proj of the reference's
runtime/scheduler.py:22-69 (same names, arguments and tensor keys).  Two
changes, both on the fast side of the same contract:
  * a GGUF embedding table is no longer dequantized whole every forward pass
    (32000 x 4096 x 2 B = 262 MB written and re-read per step for LLaMA-7B):
    only the looked-up rows are, bit for bit the values the full dequant
    would give (gds_io_ext.embed_gguf);
  * a GGUF lm_head goes through dequant_linear, i.e. the fused dequant+GEMV
    at decode and the MFMA dequant-GEMM for Q4_0 prefill, instead of dequant
    into a temporary plus F.linear; an int8 lm_head goes through
    gds_io_ext.int8_linear instead of an fp32 copy of the matrix.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import ext
from .llama import dequant_linear


def _embed_tokens(token_ids: torch.Tensor, tensors: dict, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """token_ids [B, S] -> hidden states [B, S, H] fp16 (runtime/scheduler.py:22-44)."""
    w = tensors["model.embed_tokens.weight"]
    if isinstance(w, dict) and "gguf_type" in w:
        return ext().embed_gguf(w["buffer"], token_ids, w["shape"], w["gguf_type"], w["offset"])
    if w.dtype == torch.int8:
        scale = tensors["model.embed_tokens.scale"]
        return (F.embedding(token_ids, w).float() * scale).half()
    return F.embedding(token_ids, w)


def _lm_head_proj(h: torch.Tensor, tensors: dict, key: str = "lm_head.weight",
                  scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """h [B, S, H] -> logits [B, S, vocab] (runtime/scheduler.py:47-69); `key`
    names the tied embedding table when lm_head shares it."""
    w = tensors[key]
    if isinstance(w, dict) and "gguf_type" in w:
        return dequant_linear(h, {key: w}, key[: -len(".weight")], scratch)
    if w.dtype == torch.int8:
        return ext().int8_linear(w, tensors[key[: -len(".weight")] + ".scale"], h)
    return F.linear(h, w)
