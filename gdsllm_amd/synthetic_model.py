"""Synthetic converted model directories (loader tests and the load benchmark).

Writes metadata.json plus .bin files with the byte layout the reference's
converters produce (tools/convert_gguf.py:76-89, 378-431, 434-470, 540-575 for
GGUF LLaMA; tools/convert_qwen_moe.py:157-276 for affine-Q4 expert stacks):
every tensor at a 4 KiB-aligned offset and zero-padded to a 4 KiB multiple,
GGUF blocks verbatim, fp16 norms, the LLaMA layer tensors in the converter's
order.  Returns the raw tensors so the tests can check the loaded buffers
against the oracle on exactly these bytes.
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

from . import synthetic as syn

ALIGN = 4096

# tools/convert_gguf.py:44-54
LLAMA_LAYER_ORDER = [
    "input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
    "self_attn.o_proj.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
    "mlp.down_proj.weight",
]


def _pad(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


class _BinWriter:
    """Appends tensors to one .bin file at 4 KiB-aligned offsets."""

    def __init__(self, path: str):
        self.f = open(path, "wb")

    def put(self, data: bytes):
        off = self.f.tell()
        self.f.write(data)
        pad = _pad(len(data)) - len(data)
        if pad:
            self.f.write(b"\0" * pad)
        return off, _pad(len(data))

    def close(self) -> int:
        size = self.f.tell()
        self.f.close()
        return size


def _bytes(t: torch.Tensor) -> bytes:
    return t.contiguous().cpu().view(torch.uint8).numpy().tobytes()


def _plain_entry(name, shape, dtype, off, size, padded):
    return {"name": name, "shape": list(shape), "dtype": dtype, "offset": off, "size_bytes": size,
            "padded_size": padded, "quant": None}


def _gguf_entry(name, shape, quant, off, size, padded):
    return {"name": name, "shape": list(shape), "dtype": f"gguf_{quant}", "offset": off, "size_bytes": size,
            "padded_size": padded, "quant": quant, "block_size": 32}


def _quant(rows, cols, quant, gen):
    return syn.q4_0_weights(rows, cols, gen) if quant == "q4_0" else syn.q8_0_weights(rows, cols, gen)


def write_llama(model_dir: str, quant: str = "q4_0", layers: int = 2, hidden: int = 512, ffn: int = 1024,
                vocab: int = 640, seed: int = 0) -> dict:
    """A GGUF-converted LLaMA directory.  Returns {"layers": [{name: raw tensor}],
    "embed": raw, "norm": fp16, "lm_head": raw, "shapes": {name: [rows, cols]}}."""
    os.makedirs(model_dir, exist_ok=True)
    g = torch.Generator().manual_seed(seed)
    shapes = {"self_attn.q_proj.weight": (hidden, hidden), "self_attn.k_proj.weight": (hidden, hidden),
              "self_attn.v_proj.weight": (hidden, hidden), "self_attn.o_proj.weight": (hidden, hidden),
              "mlp.gate_proj.weight": (ffn, hidden), "mlp.up_proj.weight": (ffn, hidden),
              "mlp.down_proj.weight": (hidden, ffn)}
    raw_layers, layer_metas = [], []
    for i in range(layers):
        path = f"layer_{i:03d}.bin"
        w = _BinWriter(os.path.join(model_dir, path))
        raw, metas = {}, []
        for name in LLAMA_LAYER_ORDER:
            if name.endswith("layernorm.weight"):
                t = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.float16)
                off, padded = w.put(_bytes(t))
                metas.append(_plain_entry(name, [hidden], "float16", off, hidden * 2, padded))
            else:
                rows, cols = shapes[name]
                t = _quant(rows, cols, quant, g)
                b = _bytes(t)
                off, padded = w.put(b)
                metas.append(_gguf_entry(name, [rows, cols], quant, off, len(b), padded))
            raw[name] = t
        layer_metas.append({"index": i, "path": path, "size_bytes": w.close(), "tensors": metas})
        raw_layers.append(raw)

    def special(fname, name, t, shape, q):
        w = _BinWriter(os.path.join(model_dir, fname))
        b = _bytes(t)
        off, padded = w.put(b)
        entry = _gguf_entry(name, shape, q, off, len(b), padded) if q else _plain_entry(name, shape, "float16", off,
                                                                                        len(b), padded)
        return {"path": fname, "size_bytes": w.close(), "tensors": [entry]}

    embed = _quant(vocab, hidden, quant, g)
    norm = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.float16)
    lm_head = _quant(vocab, hidden, quant, g)
    metadata = {
        "model": "llama", "dtype": quant, "quantization": quant, "alignment": ALIGN,
        "num_layers": layers, "hidden_size": hidden, "intermediate_size": ffn, "vocab_size": vocab,
        "num_heads": hidden // 64, "num_kv_heads": hidden // 64, "head_dim": 64, "rms_norm_eps": 1e-5,
        "rope_theta": 10000.0, "max_seq_len": 2048, "lm_head_tied": False,
        "files": {
            "embed_tokens": special("embed_tokens.bin", "model.embed_tokens.weight", embed, [vocab, hidden], quant),
            "final_norm": special("final_norm.bin", "model.norm.weight", norm, [hidden], None),
            "lm_head": special("lm_head.bin", "lm_head.weight", lm_head, [vocab, hidden], quant),
            "layers": layer_metas,
        },
    }
    with open(os.path.join(model_dir, "metadata.json"), "w") as f:
        json.dump(metadata, f, indent=2)
    return {"layers": raw_layers, "embed": embed, "norm": norm, "lm_head": lm_head, "shapes": shapes}


def write_moe_layer(model_dir: str, experts: int = 8, hidden: int = 2048, ffn: int = 512, group: int = 64,
                    seed: int = 1) -> dict:
    """One Qwen-MoE-style layer: a norm, an fp16 router, and stacked affine-Q4
    switch_mlp gate/up/down [E, N, K] (weight entry + .scales + .biases entries,
    tools/convert_qwen_moe.py:205-263).  Returns {name: (words, scales, biases)}
    for the expert stacks and the router."""
    os.makedirs(model_dir, exist_ok=True)
    g = torch.Generator().manual_seed(seed)
    w = _BinWriter(os.path.join(model_dir, "layer_000.bin"))
    metas, raw = [], {}
    norm = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.float16)
    off, padded = w.put(_bytes(norm))
    metas.append(_plain_entry("input_layernorm.weight", [hidden], "float16", off, hidden * 2, padded))
    router = (0.02 * torch.randn(experts, hidden, generator=g)).to(torch.float16)
    off, padded = w.put(_bytes(router))
    metas.append(_plain_entry("mlp.gate.weight", [experts, hidden], "float16", off, router.numel() * 2, padded))
    raw["mlp.gate.weight"] = router
    for proj, (n, k) in (("gate_proj", (ffn, hidden)), ("up_proj", (ffn, hidden)), ("down_proj", (hidden, ffn))):
        words, scales, biases = syn.affine_q4_weights([experts, n, k], group, g)
        prefix = f"mlp.switch_mlp.{proj}"
        wb, sb, bb = _bytes(words), _bytes(scales), _bytes(biases)
        w_off, w_pad = w.put(wb)
        s_off, s_pad = w.put(sb)
        b_off, b_pad = w.put(bb)
        metas.append({"name": f"{prefix}.weight", "shape": [experts, n, k], "dtype": "uint32", "offset": w_off,
                      "size_bytes": len(wb), "padded_size": w_pad, "quant": "affine_q4", "group_size": group,
                      "scale_shape": list(scales.shape), "scale_offset": s_off, "scale_size_bytes": len(sb),
                      "scale_padded_size": s_pad, "bias_shape": list(biases.shape), "bias_offset": b_off,
                      "bias_size_bytes": len(bb), "bias_padded_size": b_pad})
        metas.append(_plain_entry(f"{prefix}.scales", scales.shape, "float16", s_off, len(sb), s_pad))
        metas.append(_plain_entry(f"{prefix}.biases", biases.shape, "float16", b_off, len(bb), b_pad))
        raw[prefix] = (words, scales, biases)
    size = w.close()
    metadata = {"model": "qwen3_moe", "quantization": "affine_q4", "alignment": ALIGN, "num_layers": 1,
                "hidden_size": hidden, "num_experts": experts, "moe_intermediate_size": ffn,
                "files": {"embed_tokens": None, "final_norm": None, "lm_head": None,
                          "layers": [{"index": 0, "path": "layer_000.bin", "size_bytes": size,
                                      "layer_type": "full_attention", "tensors": metas}]}}
    with open(os.path.join(model_dir, "metadata.json"), "w") as f:
        json.dump(metadata, f, indent=2)
    return raw


def file_bytes(path: str, offset: int, size: int) -> np.ndarray:
    with open(path, "rb") as f:
        f.seek(offset)
        return np.frombuffer(f.read(size), dtype=np.uint8)
