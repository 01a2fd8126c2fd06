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

DecodeSweep drives the projection work of a cached decode step (the
reference's CachedScheduler.forward) as one HIP graph per token.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

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


_LAYER_PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
_UNSUPPORTED = 2  # GDSLLM_ERR_UNSUPPORTED: a valid request no fused kernel serves


def _ptr(meta: dict) -> int:
    return int(meta["buffer"].data_ptr) + int(meta["offset"])


class DecodeSweep:
    """The projection work of one decode step of CachedScheduler.forward
    (runtime/scheduler.py:303-386) over resident GGUF layers, captured once
    into a HIP graph and replayed per token.

    Per layer, as transformer_block issues them (runtime/llama.py:259-285 via
    :212-214 and :247-256): q/k/v on the attention input in one grouped
    launch, o_proj on the attention output, gate/up/SiLU on the MLP input in
    one launch writing h, down_proj on h; after the last layer, lm_head on
    the final hidden state: 4 launches per layer + 1 (129 for LLaMA-7B, where
    the reference issues 7 per layer + a dequant and a GEMM for lm_head).

    Attention, RoPE, the norms and the residual adds are not matvec work and
    stay with the caller, which writes each layer's inputs (attn_in[l],
    attn_out[l], mlp_in[l]: fp16 [batch, hidden]; final_in: [batch, hidden])
    before run() and reads q[l], k[l], v[l], o[l], h[l], down[l] and logits.

    layers[l]: the layer's weight dict (entries {"buffer", "shape",
    "gguf_type", "offset"} as ModelWeights.load_layer gives them); lm_head:
    the lm_head entry.  All weights one GGUF type; batch 1-8.  Where the
    fused gate/up/SiLU launch does not serve the shape (Q8_0 at batch 3-8, a
    hidden size it refuses) the layer's MLP input runs through the gate and
    up GEMVs into scratch rows and h = silu(g) * u comes from torch's fp16
    ops, the reference's own composition (runtime/llama.py:253-256): 5
    launches per layer instead of 4, in the same graph.
    """

    def __init__(self, layers: Sequence[dict], lm_head: dict, batch: int = 1, device=None, use_graph: bool = True):
        from gdsllm_amd import capi

        if not layers:
            raise ValueError("DecodeSweep: no layers")
        if not 1 <= batch <= 8:
            raise ValueError("DecodeSweep: batch must be in [1, 8]")
        metas = [[lw[f"{p}.weight"] for p in _LAYER_PROJ] for lw in layers]
        fmt = lm_head.get("gguf_type")
        for lm in metas:
            for m in lm:
                if not isinstance(m, dict) or m.get("gguf_type") != fmt:
                    raise ValueError("DecodeSweep: every projection and lm_head must be one GGUF type")
        if fmt not in ("q4_0", "q8_0"):
            raise ValueError(f"DecodeSweep: unsupported GGUF type {fmt!r}")
        self.lib, self.fmt, self.batch, self.use_graph = capi(), fmt, batch, use_graph
        self.metas, self.lm_head = metas, lm_head
        dev = torch.device(device) if device is not None else torch.device("cuda", lm_head["buffer"].device_id)
        H = int(metas[0][0]["shape"][1])
        Fd = int(metas[0][4]["shape"][0])
        for lm in metas:
            if any(int(m["shape"][1]) != H for m in lm[:6]) or int(lm[6]["shape"][1]) != Fd or \
                    int(lm[6]["shape"][0]) != H or [int(v) for v in lm[5]["shape"]] != [Fd, H]:
                raise ValueError("DecodeSweep: layer shapes disagree")
        self.hidden, self.ffn, self.vocab = H, Fd, int(lm_head["shape"][0])

        def buf(n):
            return torch.zeros(batch, n, dtype=torch.float16, device=dev)

        L = len(metas)
        self.attn_in = [buf(H) for _ in range(L)]
        self.attn_out = [buf(int(lm[3]["shape"][1])) for lm in metas]
        self.mlp_in = [buf(H) for _ in range(L)]
        self.final_in = buf(int(lm_head["shape"][1]))
        self.q, self.k, self.v, self.o = ([buf(int(lm[i]["shape"][0])) for lm in metas] for i in range(4))
        self.h = [buf(Fd) for _ in range(L)]
        # gate and up rows for layers whose fused gate/up/SiLU launch is refused
        self._g, self._u = buf(Fd), buf(Fd)
        self.fused_gate_up = True
        self.down = [buf(H) for _ in range(L)]
        self.logits = buf(self.vocab)
        c_vp, c_i64 = ctypes.c_void_p, ctypes.c_int64
        self._qkv = [((c_vp * 3)(*[_ptr(m) for m in lm[:3]]),
                      (c_vp * 3)(self.q[i].data_ptr(), self.k[i].data_ptr(), self.v[i].data_ptr()),
                      (c_i64 * 3)(*[int(m["shape"][0]) for m in lm[:3]])) for i, lm in enumerate(metas)]
        self._graph = None

    def _launch_all(self) -> None:
        from gdsllm_amd import check

        lib, B = self.lib, self.batch
        gemv = lib.gdsllm_fused_q4_0_gemv if self.fmt == "q4_0" else lib.gdsllm_fused_q8_0_gemv
        group = lib.gdsllm_fused_q4_0_gemv_group if self.fmt == "q4_0" else lib.gdsllm_fused_q8_0_gemv_group
        gate_up = lib.gdsllm_fused_q4_0_gate_up_silu if self.fmt == "q4_0" else lib.gdsllm_fused_q8_0_gate_up_silu
        s = torch.cuda.current_stream().cuda_stream
        H, Fd = self.hidden, self.ffn
        for i, lm in enumerate(self.metas):
            w3, y3, m3 = self._qkv[i]
            check(group(3, w3, y3, m3, self.attn_in[i].data_ptr(), H, B, H, s))
            mo, ko = (int(v) for v in lm[3]["shape"])
            check(gemv(_ptr(lm[3]), self.attn_out[i].data_ptr(), self.o[i].data_ptr(), mo, ko, B, ko, mo, s))
            rc = gate_up(_ptr(lm[4]), _ptr(lm[5]), self.mlp_in[i].data_ptr(), self.h[i].data_ptr(), Fd, H, B, H, Fd, s)
            if rc == _UNSUPPORTED:
                # refused before any launch: the reference's composition
                self.fused_gate_up = False
                x = self.mlp_in[i].data_ptr()
                check(gemv(_ptr(lm[4]), x, self._g.data_ptr(), Fd, H, B, H, Fd, s))
                check(gemv(_ptr(lm[5]), x, self._u.data_ptr(), Fd, H, B, H, Fd, s))
                torch.mul(F.silu(self._g), self._u, out=self.h[i])
            elif rc != 0:
                check(rc)
            check(gemv(_ptr(lm[6]), self.h[i].data_ptr(), self.down[i].data_ptr(), H, Fd, B, Fd, H, s))
        mv, kv = self.vocab, int(self.lm_head["shape"][1])
        check(gemv(_ptr(self.lm_head), self.final_in.data_ptr(), self.logits.data_ptr(), mv, kv, B, kv, mv, s))

    def run(self) -> None:
        """One token's projections on the current stream (asynchronous)."""
        if not self.use_graph:
            self._launch_all()
            return
        if self._graph is None:
            self._launch_all()  # loads the kernels and plans the launches outside capture
            torch.cuda.current_stream().synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._launch_all()
            self._graph = graph
        self._graph.replay()

    @property
    def launches_per_token(self) -> int:
        """Projection launches per token (the SiLU and product of a refused
        gate/up/SiLU launch not counted)."""
        return (4 if self.fused_gate_up else 5) * len(self.metas) + 1
