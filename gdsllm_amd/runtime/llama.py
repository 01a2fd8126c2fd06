"""GGUF projection dispatch of the LLaMA forward pass, over the gfx950 kernels.

Mirrors runtime/llama.py:106-166 of the reference: same function names,
arguments and weight-metadata dicts ({"buffer", "shape", "gguf_type",
"offset"}, built at runtime/torch_bridge.py:125-132), same decode/prefill rule
(x.shape[1] == 1 -> fused dequant+GEMV).  Differences, all on the fast side of
the same contract:
  * decode with batch > 1 (x [B, 1, K], B <= 8) runs one batched fused GEMV
    instead of failing the reference's x.view(-1) size check;
  * Q4_0 and Q8_0 prefill run the fused MFMA dequant-GEMM instead of
    dequant + GEMM where that is faster (prefill_takes_fused_gemm: chunks of
    up to 512 tokens over matrices of 2048 rows or more); the dequant route
    stays for the other chunks and for shapes the kernel does not serve;
  * per-column int8 weights (runtime/llama.py:162-165) go through
    gds_io_ext.int8_linear: a fused GEMV at decode, a bit-exact dequant and one
    GEMM at prefill, instead of an fp32 copy of the whole matrix per call.

The decode step's fused launches are exposed as the reference's own units:
qkv_projections (the three dequant_linear calls of runtime/llama.py:212-214 in
one launch) and mlp (runtime/llama.py:247-256: gate, up and F.silu(gate)*up in
one launch, then down).
"""

from __future__ import annotations

from typing import Dict, Optional

import torch
import torch.nn.functional as F

from . import ext


def _dequant_gguf(meta: dict, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp16 dequantization of a GGUF tensor (runtime/llama.py:106-119)."""
    return ext().dequant_gguf(meta["buffer"], meta["shape"], meta["gguf_type"], meta["offset"], scratch)


def _fused_dequant_gemv(x: torch.Tensor, meta: dict) -> torch.Tensor:
    """Fused dequant + GEMV for decode (runtime/llama.py:122-141).

    x: (batch, 1, in_dim) fp16 -> (batch, 1, out_dim) fp16.
    """
    batch = x.shape[0] if x.dim() == 3 else 1
    out = ext().fused_dequant_gemv(
        meta["buffer"], x.reshape(batch, -1), meta["shape"], meta["gguf_type"], meta["offset"]
    )
    return out.unsqueeze(1)


# Measured on MI355X (Q4_0 and Q8_0, LLaMA-7B/70B projection shapes, 64 to
# 2048 tokens), fused MFMA dequant-GEMM against the bit-exact dequant into a
# scratch matrix + hipBLASLt: the fused GEMM wins up to 512 tokens (11008 x
# 4096 Q4_0 at 512: 69 against 73 us; 28672 x 8192 at 128: 108 against 235
# us) and loses from 1024 on (11008 x 4096 Q4_0 at 2048: 217 against 182 us;
# it dequantizes every weight once per 128-token tile, the route once per
# call), on matrices under 2048 rows (1024 x 8192 at 512: 51 against 39 us)
# and where its tiles leave most compute units idle (4096 x 11008 at 64
# tokens: 32 tiles, 63 against 53 us).
FUSED_GEMM_MAX_TOKENS = 512
FUSED_GEMM_MIN_ROWS = 2048
FUSED_GEMM_MIN_TILES = 64  # 128-row x 64-token tiles


def prefill_takes_fused_gemm(out_dim: int, tokens: int) -> bool:
    """Whether a prefill projection of `tokens` rows of x onto `out_dim` rows
    of quantized weights takes the fused MFMA dequant-GEMM (else dequant +
    F.linear)."""
    tiles = -(-out_dim // 128) * -(-tokens // 64)
    return tokens <= FUSED_GEMM_MAX_TOKENS and out_dim >= FUSED_GEMM_MIN_ROWS and tiles >= FUSED_GEMM_MIN_TILES


def _fused_dequant_gemm(x: torch.Tensor, meta: dict) -> Optional[torch.Tensor]:
    """Prefill Q4_0 / Q8_0 projection on the MFMA dequant-GEMM: (B, S, K) ->
    (B, S, M); None for a shape or alignment the kernels do not serve."""
    return ext().fused_dequant_gemm(meta["buffer"], x, meta["shape"], meta["gguf_type"], meta["offset"])


def dequant_linear(
    x: torch.Tensor, weights: Dict[str, torch.Tensor], name: str, scratch: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """F.linear with on-the-fly dequantization (runtime/llama.py:144-166)."""
    w = weights[f"{name}.weight"]
    if isinstance(w, dict) and "gguf_type" in w:
        if x.shape[1] == 1 and x.shape[0] <= 8:
            return _fused_dequant_gemv(x, w)
        if prefill_takes_fused_gemm(int(w["shape"][0]), x.numel() // x.shape[-1]):
            out = _fused_dequant_gemm(x, w)
            if out is not None:
                return out
        w = _dequant_gguf(w, scratch)
    elif w.dtype == torch.int8:
        # per-column int8: fused GEMV for up to 8 rows of x, else the bit-exact
        # dequant and one GEMM (no fp32 copy of the matrix)
        return ext().int8_linear(w, weights[f"{name}.scale"], x)
    return F.linear(x, w)


def _gguf_decode(x: torch.Tensor, metas) -> bool:
    """Decode (x [B, 1, K], B <= 8) over GGUF weights of one type sharing a buffer device."""
    return (x.dim() == 3 and x.shape[1] == 1 and x.shape[0] <= 8 and
            all(isinstance(m, dict) and "gguf_type" in m for m in metas) and
            len({m["gguf_type"] for m in metas}) == 1)


def qkv_projections(x: torch.Tensor, weights: Dict, scratch: Optional[torch.Tensor] = None):
    """(xq, xk, xv) = the q/k/v projections of runtime/llama.py:212-214; at
    decode over GGUF weights one grouped launch reads x once for all three."""
    names = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")
    metas = [weights[f"{n}.weight"] for n in names]
    if _gguf_decode(x, metas):
        batch = x.shape[0]
        outs = ext().fused_dequant_gemv_group([m["buffer"] for m in metas], x.reshape(batch, -1),
                                              [list(m["shape"]) for m in metas], metas[0]["gguf_type"],
                                              [m["offset"] for m in metas])
        return tuple(o.unsqueeze(1) for o in outs)
    return tuple(dequant_linear(x, weights, n, scratch) for n in names)


def mlp(x: torch.Tensor, weights: Dict, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """SwiGLU MLP (runtime/llama.py:247-256).  At decode over GGUF weights,
    h = fp16(silu(gate x) * (up x)) comes from one launch that never writes
    gate or up (torch's fp16 rounding of silu and of the product), then down."""
    g, u = weights["mlp.gate_proj.weight"], weights["mlp.up_proj.weight"]
    if _gguf_decode(x, (g, u)) and list(g["shape"]) == list(u["shape"]):
        batch = x.shape[0]
        h = ext().fused_gate_up_silu(g["buffer"], u["buffer"], x.reshape(batch, -1), list(g["shape"]),
                                     g["gguf_type"], g["offset"], u["offset"])
        if h is not None:
            return dequant_linear(h.unsqueeze(1), weights, "mlp.down_proj", scratch)
    gate = dequant_linear(x, weights, "mlp.gate_proj", scratch)
    up = dequant_linear(x, weights, "mlp.up_proj", scratch)
    return dequant_linear(F.silu(gate) * up, weights, "mlp.down_proj", scratch)
