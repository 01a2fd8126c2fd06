"""The runtime's prefill route choice (CPU): dequant_linear and
affine_q4_linear take the fused MFMA dequant-GEMM for the chunks where it was
measured faster than the reference's dequant -> F.linear route
(runtime/llama.py:160-166, runtime/qwen_moe.py:69-73), and that route
otherwise; a chunk the fused GEMM declines (None) falls back to the route.
The extension is replaced by a recorder, so no kernel runs."""

from __future__ import annotations

import pytest
import torch

from gdsllm_amd.runtime import llama, qwen_moe


class Recorder:
    def __init__(self, fused_result=True):
        self.calls = []
        self.fused_result = fused_result

    def fused_dequant_gemm(self, buf, x, shape, gguf_type, offset):
        self.calls.append("fused")
        if not self.fused_result:
            return None
        return torch.zeros(*x.shape[:-1], shape[0], dtype=x.dtype)

    fused_affine_q4_gemm = None

    def dequant_gguf(self, buf, shape, gguf_type, offset, scratch):
        self.calls.append("dequant")
        return torch.zeros(shape, dtype=torch.float32)

    def dequant_affine_q4(self, buf, shape, wo, so, bo, g, scratch):
        self.calls.append("dequant")
        return torch.zeros(shape, dtype=torch.float32)


@pytest.mark.parametrize("M,T,fused", [
    (11008, 512, True), (4096, 128, True), (32000, 512, True), (28672, 64, True),
    (11008, 1024, False), (4096, 2048, False),   # long chunks: dequant once, then the library GEMM
    (1024, 512, False), (1024, 64, False),        # short matrices
    (4096, 64, False),                            # 32 tiles: most compute units idle
])
def test_gguf_prefill_route(monkeypatch, M, T, fused):
    rec = Recorder()
    monkeypatch.setattr(llama, "ext", lambda: rec)
    K = 256
    meta = {"buffer": object(), "shape": [M, K], "gguf_type": "q4_0", "offset": 0}
    x = torch.zeros(1, T, K)
    y = llama.dequant_linear(x, {"p.weight": meta}, "p")
    assert y.shape == (1, T, M)
    assert rec.calls == (["fused"] if fused else ["dequant"])
    assert llama.prefill_takes_fused_gemm(M, T) == fused


def test_gguf_prefill_falls_back_when_fused_declines(monkeypatch):
    rec = Recorder(fused_result=False)
    monkeypatch.setattr(llama, "ext", lambda: rec)
    meta = {"buffer": object(), "shape": [4096, 256], "gguf_type": "q8_0", "offset": 0}
    y = llama.dequant_linear(torch.zeros(2, 256, 256), {"p.weight": meta}, "p")
    assert y.shape == (2, 256, 4096)
    assert rec.calls == ["fused", "dequant"]


@pytest.mark.parametrize("M,T,fused", [(4096, 512, True), (4096, 1024, False), (1024, 256, False)])
def test_affine_prefill_route(monkeypatch, M, T, fused):
    rec = Recorder()

    def fused_affine(buf, x, shape, wo, so, bo, g):
        rec.calls.append("fused")
        return torch.zeros(*x.shape[:-1], shape[0], dtype=x.dtype)

    rec.fused_affine_q4_gemm = fused_affine
    monkeypatch.setattr(qwen_moe, "ext", lambda: rec)
    K = 256
    meta = {"buffer": object(), "shape": [M, K], "quant_type": "affine_q4", "weight_offset": 0,
            "scale_offset": 0, "bias_offset": 0, "group_size": 64}
    y = qwen_moe.affine_q4_linear(torch.zeros(1, T, K), {"p.weight": meta}, "p")
    assert y.shape == (1, T, M)
    assert rec.calls == (["fused"] if fused else ["dequant"])
