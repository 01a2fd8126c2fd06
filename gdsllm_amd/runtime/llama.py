"""GGUF projection dispatch of the LLaMA forward pass, over the gfx950 kernels.

Mirrors runtime/llama.py:106-166 of the reference: same function names,
arguments and weight-metadata dicts ({"buffer", "shape", "gguf_type",
"offset"}, built at runtime/torch_bridge.py:125-132), same decode/prefill rule
(x.shape[1] == 1 -> fused dequant+GEMV).  Differences, all on the fast side of
the same contract:
  * decode with batch > 1 (x [B, 1, K], B <= 8) runs one batched fused GEMV
    instead of failing the reference's x.view(-1) size check;
  * Q4_0 and Q8_0 prefill run the fused MFMA dequant-GEMM instead of
    dequant + GEMM where that measured faster (prefill_takes_fused_gemm, per
    format, rows, in_dim and chunk length); the dequant route stays for the
    other chunks and for shapes the kernel does not serve;
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


# Measured on MI355X: the fused MFMA dequant-GEMM against the bit-exact dequant
# into a scratch matrix + hipBLASLt (the reference's route), Q4_0, Q8_0 and
# affine-Q4 g64 over 4096x4096, 11008x4096, 4096x11008, 32000x4096, 8192x8192,
# 1024x8192, 28672x8192, 8192x28672 and 2048x4096 at 64 to 1024 tokens.
#  * Q4_0 and affine-Q4: the fused GEMM wins wherever its 128-row x 64-token
#    tiles number at least 32 (64 over an in_dim past 8192, where each tile is
#    long, or over 2048 rows), on 2048 rows or more, for chunks of up to 512
#    tokens, and for longer chunks over up to 8192 rows (8192x28672 at 1024
#    tokens: 464 against 503 us); it loses on 1024 rows (1024x8192 at 512
#    tokens: 51 against 40 us), where few tiles leave most compute units idle
#    (4096x11008 at 64 tokens: 62 against 53 us), and at 1024 tokens over
#    11008 rows or more (11008x4096: 132 against 108 us), where it dequantizes
#    every weight once per token tile and the route once per call.
#  * Q8_0 (a W stage twice Q4_0's): the fused GEMM wins on 8192 rows or more
#    up to 512 tokens (28672x8192 at 128 tokens: 97 against 247 us), except
#    512 tokens over an in_dim of 4096 on fewer than 16384 rows (11008x4096:
#    82 against 76 us); on 4096 rows the two are within 10% either way and the
#    route is taken.
FUSED_GEMM_MAX_TOKENS = 512
FUSED_GEMM_MIN_ROWS = 2048


def prefill_takes_fused_gemm(out_dim: int, tokens: int, in_dim: int = 4096, gguf_type: str = "q4_0") -> bool:
    """Whether a prefill projection of `tokens` rows of x onto `out_dim` rows
    of quantized weights (in_dim columns; gguf_type "q4_0", "q8_0" or
    "affine_q4") takes the fused MFMA dequant-GEMM (else dequant + F.linear)."""
    if gguf_type == "q8_0":
        return (tokens <= FUSED_GEMM_MAX_TOKENS and out_dim >= 8192 and
                not (in_dim <= 4096 and tokens > 256 and out_dim < 16384))
    tiles = -(-out_dim // 128) * -(-tokens // 64)
    min_tiles = 64 if in_dim > 8192 or out_dim <= 2048 else 32
    return (out_dim >= FUSED_GEMM_MIN_ROWS and tiles >= min_tiles and
            (tokens <= FUSED_GEMM_MAX_TOKENS or out_dim <= 8192))


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
        if prefill_takes_fused_gemm(int(w["shape"][0]), x.numel() // x.shape[-1], int(w["shape"][1]), w["gguf_type"]):
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


def _gguf_pair(g, u) -> bool:
    """gate and up: GGUF weights of one type and shape on one device."""
    return (isinstance(g, dict) and isinstance(u, dict) and "gguf_type" in g and
            g.get("gguf_type") == u.get("gguf_type") and list(g["shape"]) == list(u["shape"]) and
            g["buffer"].device_id == u["buffer"].device_id)


def mlp(x: torch.Tensor, weights: Dict, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """SwiGLU MLP (runtime/llama.py:247-256).  Over GGUF weights h =
    fp16(silu(gate x) * (up x)) comes from one launch that never writes gate
    or up (torch's fp16 rounding of silu and of the product), then down: the
    fused GEMV at decode, the fused MFMA GEMM for a prefill chunk where the
    projections take it (prefill_takes_fused_gemm)."""
    g, u = weights["mlp.gate_proj.weight"], weights["mlp.up_proj.weight"]
    if _gguf_decode(x, (g, u)) and list(g["shape"]) == list(u["shape"]):
        batch = x.shape[0]
        h = ext().fused_gate_up_silu(g["buffer"], u["buffer"], x.reshape(batch, -1), list(g["shape"]),
                                     g["gguf_type"], g["offset"], u["offset"])
        if h is not None:
            return dequant_linear(h.unsqueeze(1), weights, "mlp.down_proj", scratch)
    elif (x.shape[1] > 1 or x.shape[0] > 8) and _gguf_pair(g, u) and g["gguf_type"] in ("q4_0", "q8_0") and \
            prefill_takes_fused_gemm(int(g["shape"][0]), x.numel() // x.shape[-1], int(g["shape"][1]), g["gguf_type"]):
        h = ext().fused_gate_up_silu_gemm(g["buffer"], u["buffer"], x, list(g["shape"]), g["gguf_type"],
                                          g["offset"], u["offset"])
        if h is not None:
            return dequant_linear(h, weights, "mlp.down_proj", scratch)
    gate = dequant_linear(x, weights, "mlp.gate_proj", scratch)
    up = dequant_linear(x, weights, "mlp.up_proj", scratch)
    return dequant_linear(F.silu(gate) * up, weights, "mlp.down_proj", scratch)
