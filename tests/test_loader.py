"""Model-directory loader, host side (no GPU): metadata.json parsing, the
byte regions a partial layer load reads, and the on-disk layout of the
synthetic converted directories the GPU loader tests use."""

import json
import os

import numpy as np
import pytest

from gdsllm_amd.runtime.torch_bridge import ModelWeights, TensorMeta, merge_regions, parse_tensors
from gdsllm_amd.synthetic_model import ALIGN, LLAMA_LAYER_ORDER, file_bytes, write_llama, write_moe_layer


def test_merge_regions():
    assert merge_regions([]) == []
    assert merge_regions([(8192, 12288), (0, 4096)]) == [(0, 4096), (8192, 12288)]
    assert merge_regions([(0, 4096), (4096, 8192)]) == [(0, 8192)]  # touching ranges join
    assert merge_regions([(0, 10000), (4096, 8192), (9000, 20000), (30000, 40000)]) == [(0, 20000), (30000, 40000)]


def test_tensor_end_covers_scale_and_bias():
    t = TensorMeta(name="w", shape=[4, 8], dtype="uint32", offset=0, size_bytes=100, padded_size=4096,
                   quant="affine_q4", scale_offset=4096, scale_padded_size=4096, bias_offset=8192,
                   bias_padded_size=4096)
    assert t.end() == 12288
    assert TensorMeta(name="n", shape=[8], dtype="float16", offset=4096, size_bytes=16, padded_size=4096).end() == 8192


def test_parse_tensors_ignores_unknown_keys():
    (t,) = parse_tensors([{"name": "a", "shape": [2, 32], "dtype": "gguf_q4_0", "offset": 0, "size_bytes": 36,
                           "padded_size": 4096, "quant": "q4_0", "block_size": 32}])
    assert t.quant == "q4_0" and t.scale_offset is None and t.group_size is None


@pytest.mark.parametrize("quant", ["q4_0", "q8_0"])
def test_llama_directory_layout_and_metadata(tmp_path, quant):
    d = str(tmp_path / quant)
    raw = write_llama(d, quant=quant, layers=2, hidden=256, ffn=512, vocab=320, seed=3)
    mw = ModelWeights(d)
    assert mw.num_layers == 2
    assert mw.config["hidden_size"] == 256 and "files" not in mw.config and "alignment" not in mw.config
    bpb = 18 if quant == "q4_0" else 34
    for i, layer in enumerate(mw.layers):
        assert [t.name for t in layer.tensors] == LLAMA_LAYER_ORDER
        assert layer.size_bytes == os.path.getsize(os.path.join(d, layer.path))
        for t in layer.tensors:
            assert t.offset % ALIGN == 0 and t.padded_size % ALIGN == 0 and t.padded_size >= t.size_bytes
            if t.quant:
                rows, cols = t.shape
                assert t.size_bytes == rows * cols // 32 * bpb
                got = file_bytes(os.path.join(d, layer.path), t.offset, t.size_bytes)
                assert np.array_equal(got, raw["layers"][i][t.name].numpy().reshape(-1))
    for name in ModelWeights.SPECIAL_FILES:
        assert mw.special[name] is not None
    (emb,) = mw.special["embed_tokens"].tensors
    assert emb.quant == quant and emb.shape == [320, 256]


def test_moe_directory_layout_and_partial_regions(tmp_path):
    d = str(tmp_path / "moe")
    write_moe_layer(d, experts=4, hidden=512, ffn=256, group=64)
    mw = ModelWeights(d)
    (layer,) = mw.layers
    assert mw.special["embed_tokens"] is None
    names = {t.name: t for t in layer.tensors}
    gate = names["mlp.switch_mlp.gate_proj.weight"]
    assert gate.quant == "affine_q4" and gate.shape == [4, 256, 512] and gate.group_size == 64
    assert gate.size_bytes == 4 * 256 * 512 // 2 and gate.scale_size_bytes == 4 * 256 * (512 // 64) * 2
    # what load_layer_partial reads: everything but the expert stacks, as one region
    keep = [t for t in layer.tensors if not t.name.startswith("mlp.switch_mlp.")]
    assert merge_regions((t.offset, t.end()) for t in keep) == [(0, names["mlp.gate.weight"].end())]
    with open(os.path.join(d, "metadata.json")) as f:
        assert json.load(f)["files"]["layers"][0]["layer_type"] == "full_attention"
