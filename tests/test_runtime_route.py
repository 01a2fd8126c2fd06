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


# (format, out_dim, in_dim, tokens, fused faster): the choices the route rule
# must make, each from the MI355X measurement of both routes that the rule in
# runtime/llama.py summarizes (fused / route us per call in the comments).
ROUTE_TABLE = [
    ("q4_0", 4096, 4096, 64, True),        # 29.9 / 34.4
    ("q4_0", 11008, 4096, 512, True),      # 70.4 / 73.9
    ("q4_0", 11008, 4096, 1024, False),    # 132.2 / 108.1
    ("q4_0", 4096, 11008, 64, False),      # 62.5 / 52.8: 32 long tiles
    ("q4_0", 4096, 11008, 128, True),      # 63.7 / 72.4
    ("q4_0", 4096, 11008, 1024, True),     # 107.8 / 117.6
    ("q4_0", 32000, 4096, 1024, False),    # 289.6 / 265.9
    ("q4_0", 8192, 28672, 1024, True),     # 463.7 / 502.9
    ("q4_0", 28672, 8192, 64, True),       # 58.1 / 229.3
    ("q4_0", 1024, 8192, 512, False),      # 50.8 / 40.3
    ("q4_0", 2048, 4096, 128, False),      # 29.9 / 27.6
    ("q4_0", 2048, 4096, 512, True),       # 32.7 / 34.8
    ("q8_0", 11008, 4096, 512, False),     # 82.1 / 76.1
    ("q8_0", 11008, 4096, 256, True),      # 52.6 / 68.6
    ("q8_0", 4096, 11008, 256, False),     # 79.7 / 71.7
    ("q8_0", 4096, 4096, 64, False),       # 34.5 / 31.3
    ("q8_0", 28672, 8192, 128, True),      # 96.6 / 247.2
    ("q8_0", 8192, 8192, 512, True),       # 98.4 / 106.3
    ("q8_0", 8192, 8192, 1024, False),     # 164.4 / 155.6
    ("q8_0", 32000, 4096, 256, True),      # 89.0 / 150.8
    ("affine_q4", 4096, 4096, 1024, True),     # 50.9 / 54.4
    ("affine_q4", 28672, 8192, 1024, False),   # 537.1 / 501.7
    ("affine_q4", 1024, 8192, 128, False),     # 47.6 / 28.4
]


@pytest.mark.parametrize("fmt,M,K,T,fused", ROUTE_TABLE, ids=[f"{f}_{m}x{k}_T{t}" for f, m, k, t, _ in ROUTE_TABLE])
def test_prefill_route_rule(fmt, M, K, T, fused):
    assert llama.prefill_takes_fused_gemm(M, T, K, fmt) == fused


@pytest.mark.parametrize("fmt,M,T,fused", [
    ("q4_0", 11008, 512, True), ("q4_0", 4096, 128, True), ("q4_0", 32000, 512, True), ("q4_0", 28672, 64, True),
    ("q4_0", 11008, 1024, False), ("q4_0", 32000, 2048, False),   # long chunks: dequant once, then the library GEMM
    ("q4_0", 1024, 512, False), ("q4_0", 1024, 64, False),        # short matrices
    ("q4_0", 2048, 64, False),                                    # 16 tiles: most compute units idle
    ("q8_0", 11008, 512, False), ("q8_0", 11008, 256, True), ("q8_0", 4096, 128, False),
])
def test_gguf_prefill_route(monkeypatch, fmt, M, T, fused):
    """dequant_linear takes the route the rule names for its weight's format
    and shape (in_dim 256 here: the rule reads in_dim only past 8192)."""
    rec = Recorder()
    monkeypatch.setattr(llama, "ext", lambda: rec)
    K = 256
    meta = {"buffer": object(), "shape": [M, K], "gguf_type": fmt, "offset": 0}
    x = torch.zeros(1, T, K)
    y = llama.dequant_linear(x, {"p.weight": meta}, "p")
    assert y.shape == (1, T, M)
    assert rec.calls == (["fused"] if fused else ["dequant"])
    assert llama.prefill_takes_fused_gemm(M, T, K, fmt) == fused


def test_gguf_prefill_falls_back_when_fused_declines(monkeypatch):
    rec = Recorder(fused_result=False)
    monkeypatch.setattr(llama, "ext", lambda: rec)
    meta = {"buffer": object(), "shape": [8192, 256], "gguf_type": "q8_0", "offset": 0}
    y = llama.dequant_linear(torch.zeros(2, 64, 256), {"p.weight": meta}, "p")
    assert y.shape == (2, 64, 8192)
    assert rec.calls == ["fused", "dequant"]


@pytest.mark.parametrize("M,T,fused", [(4096, 512, True), (4096, 1024, True), (11008, 1024, False), (1024, 256, False)])
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


class _Buf:
    device_id = 0


def _sweep_layer(fmt, H, F):
    from gdsllm_amd.runtime.scheduler import _LAYER_PROJ

    shapes = [[H, H]] * 4 + [[F, H]] * 2 + [[H, F]]
    return {f"{p}.weight": {"buffer": _Buf(), "shape": s, "gguf_type": fmt, "offset": 0}
            for p, s in zip(_LAYER_PROJ, shapes)}


@pytest.mark.parametrize("fmt,H,B,ok", [("q4_0", 512, 3, True), ("q4_0", 8192, 8, True), ("q8_0", 512, 3, True),
                                        ("q4_0", 8448, 4, True), ("q8_0", 544, 8, True), ("q8_0", 512, 2, True),
                                        ("q4_0", 512, 9, False), ("q4_0", 512, 0, False), ("q5_0", 512, 1, False)])
def test_decode_sweep_batch_rule(monkeypatch, fmt, H, B, ok):
    """DecodeSweep takes batch 1-8 for both GGUF types (a gate/up/SiLU launch
    the fused kernel refuses runs as two GEMVs and torch's SiLU and product);
    other batches and types are refused before any device memory is
    allocated."""
    from gdsllm_amd.runtime import scheduler

    class Stop(Exception):
        pass

    def no_alloc(*a, **k):
        raise Stop()

    monkeypatch.setattr(scheduler.torch, "zeros", no_alloc)
    lm = {"buffer": _Buf(), "shape": [640, H], "gguf_type": fmt, "offset": 0}
    with pytest.raises(Stop if ok else ValueError):
        scheduler.DecodeSweep([_sweep_layer(fmt, H, 2 * H)], lm, batch=B, device="cpu")
