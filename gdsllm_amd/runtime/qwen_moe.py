"""Affine-Q4 projection dispatch and the MoE MLP of the Qwen-MoE forward pass.

Mirrors runtime/qwen_moe.py:20-73 and :386-513 of the reference (same names,
arguments and metadata dicts {"buffer", "shape", "quant_type",
"weight_offset", "scale_offset", "bias_offset", "group_size"}).

The MoE path changes shape, not contract: instead of syncing the selected
expert ids to the host and running 3 GEMV launches per expert over per-expert
buffers (runtime/qwen_moe.py:455-474), the stacked [E, N, K] expert tensors
stay resident; decode reads the selected experts by index on the device
(`moe_gather`, `moe_step`), and a prefill chunk groups its tokens by expert on
the device and runs one grouped MFMA GEMM per phase (`moe_prefill_affine_q4`,
for the loop of runtime/qwen_moe.py:475-492).  The reference's per-expert
route (expert_tensors from load_experts) is still accepted; its prefill
projections run on the MFMA dequant-GEMM.
"""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F

from . import ext
from .llama import prefill_takes_fused_gemm


def _dequant_affine_q4(meta: dict, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """runtime/qwen_moe.py:20-35."""
    return ext().dequant_affine_q4(
        meta["buffer"], meta["shape"], meta["weight_offset"], meta["scale_offset"], meta["bias_offset"],
        meta["group_size"], scratch,
    )


def _fused_affine_q4_gemv(x: torch.Tensor, meta: dict) -> torch.Tensor:
    """runtime/qwen_moe.py:38-55: (batch, 1, in_dim) -> (batch, 1, out_dim)."""
    batch = x.shape[0] if x.dim() == 3 else 1
    out = ext().fused_affine_q4_gemv(
        meta["buffer"], x.reshape(batch, -1), meta["shape"], meta["weight_offset"], meta["scale_offset"],
        meta["bias_offset"], meta["group_size"],
    )
    return out.unsqueeze(1)


def _fused_affine_q4_gemm(x: torch.Tensor, meta: dict) -> Optional[torch.Tensor]:
    """Prefill affine-Q4 projection on the MFMA dequant-GEMM: (..., K) -> (..., M);
    None for a shape, grouping or alignment the kernel does not serve."""
    return ext().fused_affine_q4_gemm(
        meta["buffer"], x, meta["shape"], meta["weight_offset"], meta["scale_offset"], meta["bias_offset"],
        meta["group_size"],
    )


def _affine_linear(x: torch.Tensor, meta: dict, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.linear(x, dequant(meta)) for a prefill chunk: the fused GEMM where it
    is the faster route (llama.prefill_takes_fused_gemm), else the
    reference's dequant -> F.linear (runtime/qwen_moe.py:72-73)."""
    if prefill_takes_fused_gemm(int(meta["shape"][0]), x.numel() // x.shape[-1], int(meta["shape"][1]), "affine_q4"):
        out = _fused_affine_q4_gemm(x, meta)
        if out is not None:
            return out
    return F.linear(x, _dequant_affine_q4(meta, scratch))


def affine_q4_linear(x: torch.Tensor, weights: Dict, name: str, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """runtime/qwen_moe.py:58-73: fused GEMV for decode, the MFMA dequant-GEMM
    (or dequant + F.linear) otherwise."""
    w = weights[f"{name}.weight"]
    if isinstance(w, dict) and w.get("quant_type") == "affine_q4":
        if x.shape[1] == 1 and x.shape[0] <= 8:
            return _fused_affine_q4_gemv(x, w)
        return _affine_linear(x, w, scratch)
    return F.linear(x, w)


def _router_logits(x: torch.Tensor, weights: Dict, scratch: Optional[torch.Tensor]) -> torch.Tensor:
    """F.linear(x, router) (runtime/qwen_moe.py:405-408) on the device: the fp16
    router through gemv_f16, an affine-Q4 router through its fused GEMV."""
    router_w = weights["mlp.gate.weight"]
    if isinstance(router_w, dict):
        return affine_q4_linear(x, weights, "mlp.gate", scratch)
    if x.numel() // x.shape[-1] > 8:
        return F.linear(x, router_w)  # a prefill chunk: one library GEMM
    return ext().gemv_f16(router_w, x)


def moe_route(
    x: torch.Tensor,
    weights: Dict,
    num_experts_per_token: int,
    scratch: Optional[torch.Tensor] = None,
    sync_unique: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor, Optional[list]]:
    """runtime/qwen_moe.py:386-416: router logits -> top-k -> fp16(softmax_fp32).

    Logits, picks and weights stay on the device (gemv_f16 + moe_route_topk;
    indices int32, ties to the lower expert index).  The sorted list of unique
    experts needs the picks on the host: with sync_unique=False it is not built
    (None) and nothing waits for the device, which is all the resident decode
    path needs.
    """
    logits = _router_logits(x, weights, scratch)
    top_idx, top_w = ext().moe_route_topk(logits, num_experts_per_token)
    unique = sorted(set(top_idx.reshape(-1).tolist())) if sync_unique else None
    return top_idx, top_w, unique


_EXPERT_PROJ = ("mlp.switch_mlp.gate_proj", "mlp.switch_mlp.up_proj", "mlp.switch_mlp.down_proj")


def moe_gather(x: torch.Tensor, weights: Dict, top_k_indices: torch.Tensor, top_k_weights: torch.Tensor) -> torch.Tensor:
    """Decode expert MLP over resident stacked experts: sum_k w_k * down_k(silu(gate_k x) * up_k x).

    x: (1, 1, hidden); weights holds the three stacked affine_q4 entries
    (shape [E, N, K]).  Returns (1, 1, hidden) fp16.
    """
    g, u, d = (weights[f"{p}.weight"] for p in _EXPERT_PROJ)
    out = ext().moe_gather_affine_q4(
        x.reshape(-1),
        g["buffer"], g["shape"], g["weight_offset"], g["scale_offset"], g["bias_offset"],
        u["buffer"], u["shape"], u["weight_offset"], u["scale_offset"], u["bias_offset"],
        d["buffer"], d["shape"], d["weight_offset"], d["scale_offset"], d["bias_offset"],
        g["group_size"], top_k_indices.reshape(-1), top_k_weights.reshape(-1),
    )
    return out.view(1, 1, -1)


_SHARED_PROJ = ("mlp.shared_expert.gate_proj", "mlp.shared_expert.up_proj", "mlp.shared_expert.down_proj")


def _entry(m: dict) -> tuple:
    return (m["buffer"], list(m["shape"]), m["weight_offset"], m["scale_offset"], m["bias_offset"], m["group_size"])


def moe_step(x: torch.Tensor, weights: Dict, top_k_indices: torch.Tensor, top_k_weights: torch.Tensor):
    """The decode MoE MLP of runtime/qwen_moe.py:455-513 for one token in two
    launches: one for the gate/up rows of the top-k experts and the shared
    expert (and the fp16 shared-expert gate logit), one for their down rows
    with the sigmoid-gated combine and clamp.  Returns (1, 1, hidden), or
    None when the layer has no affine_q4 shared expert with an fp16 gate or its
    shapes are outside the fused kernels (the caller then runs the separate
    launches)."""
    shared = [weights.get(f"{p}.weight") for p in _SHARED_PROJ]
    sg = weights.get("mlp.shared_expert_gate.weight")
    if any(not isinstance(m, dict) for m in shared) or not isinstance(sg, torch.Tensor):
        return None
    routed = [weights[f"{p}.weight"] for p in _EXPERT_PROJ]
    out = ext().moe_step_affine_q4(
        x.reshape(-1), [_entry(m) for m in routed + shared],
        top_k_indices.reshape(-1), top_k_weights.reshape(-1), sg.reshape(-1),
    )
    return None if out is None else out.view(1, 1, -1)


def _expert_meta(stacked: dict, e: int) -> dict:
    """One expert's slice of a stacked [E, N, K] affine_q4 entry (runtime/torch_bridge.py:326-337)."""
    E, N, K = stacked["shape"]
    g = stacked["group_size"]
    return {
        "buffer": stacked["buffer"],
        "shape": [N, K],
        "quant_type": "affine_q4",
        "weight_offset": stacked["weight_offset"] + e * N * (K // 8) * 4,
        "scale_offset": stacked["scale_offset"] + e * N * (K // g) * 2,
        "bias_offset": stacked["bias_offset"] + e * N * (K // g) * 2,
        "group_size": g,
    }


def moe_mlp_selective(
    x: torch.Tensor,
    weights: Dict,
    expert_tensors: Optional[Dict[str, dict]],
    top_k_indices: torch.Tensor,
    top_k_weights: torch.Tensor,
    num_experts_per_token: int,
    scratch: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """runtime/qwen_moe.py:419-513.  expert_tensors=None selects the resident
    stacked experts in `weights` (decode: one on-device gather)."""
    batch, seq_len, hidden = x.shape
    x_flat = x.view(-1, hidden)
    n_tok = x_flat.shape[0]
    resident = expert_tensors is None
    if resident and n_tok == 1:
        fused = moe_step(x, weights, top_k_indices, top_k_weights)
        if fused is not None:
            return fused
    expert_output = None
    if resident and n_tok == 1:
        expert_output = moe_gather(x, weights, top_k_indices, top_k_weights).view(1, hidden)
    elif resident:
        # prefill over the resident pools: tokens grouped by expert on the
        # device, one grouped MFMA GEMM per phase, no host sync
        expert_output = ext().moe_prefill_affine_q4(
            x_flat, [_entry(weights[f"{p}.weight"]) for p in _EXPERT_PROJ],
            top_k_indices.reshape(n_tok, num_experts_per_token), top_k_weights.reshape(n_tok, num_experts_per_token),
        )
    if expert_output is None:
        def meta(proj: str, e: int) -> dict:
            if resident:
                return _expert_meta(weights[f"mlp.switch_mlp.{proj}.weight"], e)
            return expert_tensors[f"{proj}.{e}"]

        expert_output = torch.zeros(n_tok, hidden, device=x.device, dtype=x.dtype)
        idx = top_k_indices.view(n_tok, num_experts_per_token)
        wts = top_k_weights.view(n_tok, num_experts_per_token)
        for k in range(num_experts_per_token):
            ids, ew = idx[:, k], wts[:, k]
            if n_tok == 1:
                e = int(ids[0].item())
                gate = _fused_affine_q4_gemv(x_flat.view(1, 1, -1), meta("gate_proj", e))
                up = _fused_affine_q4_gemv(x_flat.view(1, 1, -1), meta("up_proj", e))
                down = _fused_affine_q4_gemv(F.silu(gate) * up, meta("down_proj", e))
                expert_output += ew.unsqueeze(-1) * down.view(n_tok, -1)
            else:
                for e_t in ids.unique():
                    e = int(e_t.item())
                    mask = ids == e
                    xs = x_flat[mask]
                    gate = _affine_linear(xs, meta("gate_proj", e), scratch)
                    up = _affine_linear(xs, meta("up_proj", e), scratch)
                    down = _affine_linear(F.silu(gate) * up, meta("down_proj", e), scratch)
                    expert_output[mask] += ew[mask].unsqueeze(-1) * down
    expert_output = expert_output.view(batch, seq_len, hidden)

    if "mlp.shared_expert.gate_proj.weight" not in weights:
        return expert_output.clamp(min=-65504.0, max=65504.0)
    shared_gate = affine_q4_linear(x, weights, "mlp.shared_expert.gate_proj", scratch)
    shared_up = affine_q4_linear(x, weights, "mlp.shared_expert.up_proj", scratch)
    shared_out = affine_q4_linear(F.silu(shared_gate) * shared_up, weights, "mlp.shared_expert.down_proj", scratch)
    sg = weights["mlp.shared_expert_gate.weight"]
    if isinstance(sg, dict):
        gate_logit = affine_q4_linear(x, weights, "mlp.shared_expert_gate", scratch)
    else:
        gate_logit = ext().gemv_f16(sg, x)
    # expert_output + sigmoid(gate) * shared_out, clamped (runtime/qwen_moe.py:508-513), in one kernel
    return ext().moe_combine(expert_output, shared_out, gate_logit)
