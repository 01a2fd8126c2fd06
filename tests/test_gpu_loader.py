"""Converted model directory -> HBM -> kernels: the loader's parity tests.

Synthetic directories in the converters' on-disk format (gdsllm_amd/synthetic_model.py)
are loaded with ModelWeights / LayerCache, and every projection, the
embedding rows, lm_head and the stacked-expert gather are computed from the
loaded buffers and checked against the oracle on the bytes that were written.
"""

import numpy as np
import pytest
import torch

from gdsllm_amd.runtime import ext
from gdsllm_amd.runtime.llama import dequant_linear
from gdsllm_amd.runtime.qwen_moe import _fused_affine_q4_gemv, moe_gather
from gdsllm_amd.runtime.scheduler import _embed_tokens, _lm_head_proj
from gdsllm_amd.runtime.torch_bridge import LayerCache, ModelWeights
from gdsllm_amd.synthetic_model import write_llama, write_moe_layer
from helpers import affine_dequant_np, assert_gemv_close, gen, oq, syn, to_np

pytestmark = pytest.mark.gpu


def _deq(raw: torch.Tensor, quant: str, rows: int, cols: int) -> np.ndarray:
    fn = oq.dequant_q4_0 if quant == "q4_0" else oq.dequant_q8_0
    return fn(raw.numpy().reshape(-1)).reshape(rows, cols)


@pytest.mark.parametrize("quant", ["q4_0", "q8_0"])
def test_llama_directory_projections(gpu, tmp_path, quant):
    d = str(tmp_path / quant)
    raw = write_llama(d, quant=quant, layers=2, hidden=512, ffn=1024, vocab=640, seed=11)
    mw = ModelWeights(d)
    mw.init_gds()
    assert mw.is_driver_open()
    cache = LayerCache(mw)
    cache.preload()
    st = cache.stats
    assert st["cached_layers"] == 2 and st["cached_specials"] == 3 and st["misses"] == 5
    for i in range(2):
        tensors = cache.get_layer(i)
        for norm in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            assert torch.equal(tensors[norm].cpu().view(torch.int16), raw["layers"][i][norm].view(torch.int16))
        for name, (M, K) in raw["shapes"].items():
            w = _deq(raw["layers"][i][name], quant, M, K)
            x = syn.activations(1, K, gen(100 * i + M + K))
            y = dequant_linear(x.to(gpu).view(1, 1, K), tensors, name[: -len(".weight")])
            assert y.shape == (1, 1, M)
            assert_gemv_close(to_np(y).reshape(1, M), w, to_np(x), f"layer {i} {name} decode")
            if quant == "q4_0":  # prefill through the MFMA dequant-GEMM
                xp = syn.activations(40, K, gen(200 * i + M))
                yp = dequant_linear(xp.to(gpu).view(1, 40, K), tensors, name[: -len(".weight")])
                assert_gemv_close(to_np(yp).reshape(40, M), w, to_np(xp), f"layer {i} {name} prefill")
    assert cache.stats["hits"] == 2
    mw.shutdown_gds()


@pytest.mark.parametrize("quant", ["q4_0", "q8_0"])
def test_embedding_rows_and_lm_head(gpu, tmp_path, quant):
    d = str(tmp_path / quant)
    raw = write_llama(d, quant=quant, layers=1, hidden=512, ffn=1024, vocab=640, seed=12)
    mw = ModelWeights(d)
    emb, h_emb = mw.load_special("embed_tokens")
    table = _deq(raw["embed"], quant, 640, 512)
    ids = torch.tensor([[0, 5, 639, 17, 5], [3, 3, 640, 1, -2]], dtype=torch.int64)
    h = _embed_tokens(ids.to(gpu), emb)
    assert h.shape == (2, 5, 512) and h.dtype == torch.float16
    got = to_np(h).reshape(10, 512).view(np.uint16)
    for r, t in enumerate(ids.reshape(-1).tolist()):
        want = table[t].view(np.uint16) if 0 <= t < 640 else np.zeros(512, np.uint16)
        assert np.array_equal(got[r], want), f"embedding row for token {t}"
    head, h_head = mw.load_special("lm_head")
    x = syn.activations(1, 512, gen(13))
    logits = _lm_head_proj(x.to(gpu).view(1, 1, 512), head)
    assert logits.shape == (1, 1, 640)
    assert_gemv_close(to_np(logits).reshape(1, 640), _deq(raw["lm_head"], quant, 640, 512), to_np(x), "lm_head")
    norm, _ = mw.load_special("final_norm")
    assert torch.equal(norm["model.norm.weight"].cpu().view(torch.int16), raw["norm"].view(torch.int16))


def test_moe_partial_layer_experts_and_gather(gpu, tmp_path):
    E, H, F, g = 8, 2048, 512, 64
    d = str(tmp_path / "moe")
    raw = write_moe_layer(d, experts=E, hidden=H, ffn=F, group=g, seed=14)
    mw = ModelWeights(d)
    part, handles = mw.load_layer_partial(0)
    assert set(part) == {"input_layernorm.weight", "mlp.gate.weight"} and len(handles) == 1
    assert torch.equal(part["mlp.gate.weight"].cpu().view(torch.int16), raw["mlp.gate.weight"].view(torch.int16))
    x = syn.activations(1, H, gen(15))
    xd = x.to(gpu).view(1, 1, H)
    picks = [1, 6]
    experts, eh = mw.load_experts(0, picks)
    assert len(eh) == 6 and set(experts) == {f"{p}.{e}" for p in ("gate_proj", "up_proj", "down_proj") for e in picks}
    for e in picks:
        for proj, K in (("gate_proj", H), ("up_proj", H), ("down_proj", F)):
            words, scales, biases = (t[e] for t in raw[f"mlp.switch_mlp.{proj}"])
            w = affine_dequant_np(words, scales, biases, g).reshape(-1, K)
            xin = x if K == H else syn.activations(1, F, gen(16 + e))
            y = _fused_affine_q4_gemv(xin.to(gpu).view(1, 1, K), experts[f"{proj}.{e}"])
            assert_gemv_close(to_np(y).reshape(1, -1), w, to_np(xin), f"expert {e} {proj}")
    # the whole layer resident: the on-device gather reads the stacked experts by index
    whole, _ = mw.load_layer(0)
    idx = torch.tensor(picks, dtype=torch.int32)
    wts = torch.tensor([0.625, 0.375], dtype=torch.float16)
    y = moe_gather(xd, whole, idx.to(gpu), wts.to(gpu))

    def expert_fn(proj, K):
        def f(e):
            words, scales, biases = (t[e] for t in raw[f"mlp.switch_mlp.{proj}"])
            return affine_dequant_np(words, scales, biases, g).reshape(-1, K)
        return f

    ref, _ = oq.moe_gather(to_np(x).reshape(-1), expert_fn("gate_proj", H), expert_fn("up_proj", H),
                           expert_fn("down_proj", F), np.array(picks), to_np(wts))
    rel = float(np.linalg.norm(to_np(y).astype(np.float64).reshape(-1) - ref) / np.linalg.norm(ref))
    assert rel <= oq.GEMV_REL_L2, f"gather from the loaded layer: rel L2 {rel:.3e}"


def test_region_loads_round_to_4k(gpu, tmp_path):
    d = str(tmp_path / "r")
    write_llama(d, quant="q4_0", layers=1, hidden=512, ffn=1024, vocab=640, seed=17)
    path = f"{d}/layer_000.bin"
    h = ext().load_file_region(path, 5000, 4096)
    assert h.size == 8192 and h.device_id == 0 and not h.registered
    with open(path, "rb") as f:
        f.seek(4096)
        want = np.frombuffer(f.read(5000), dtype=np.uint8)
    got = to_np(ext().view_tensor(h, [5000], "uint8", 0))
    assert np.array_equal(got, want)


def test_multi_chunk_reads_and_short_read(gpu, tmp_path):
    """Reads spanning many 8 MiB staging chunks (split over the reader
    threads) at an unaligned offset, and the end-of-file count."""
    path = str(tmp_path / "big.bin")
    n = 5 * (8 << 20) + 12345
    data = np.random.default_rng(18).integers(0, 256, n + 5000, dtype=np.uint8)
    data.tofile(path)
    h = ext().load_file_region(path, n, 4103)
    assert np.array_equal(to_np(ext().view_tensor(h, [n], "uint8", 0)), data[4103:4103 + n])
    whole = ext().load_file(path, n + 5000)
    assert np.array_equal(to_np(ext().view_tensor(whole, [n + 5000], "uint8", 0)), data)
    with pytest.raises(RuntimeError, match=f"expected {n + 5001} bytes, got {n + 5000}"):
        ext().load_file(path, n + 5001)
    t = ext().load_tensor(path, [3, 1000], "float16", (8 << 20) * 3 - 10)
    want = data[(8 << 20) * 3 - 10:][:6000].view(np.float16).reshape(3, 1000)
    assert np.array_equal(to_np(t).view(np.uint16), want.view(np.uint16))
