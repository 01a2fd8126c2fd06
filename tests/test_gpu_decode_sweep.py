"""The decode-step projection driver (gdsllm_amd.runtime.scheduler.DecodeSweep,
the projection work of the reference's CachedScheduler.forward,
runtime/scheduler.py:303-386) and the fused decode units of runtime/llama.py
(qkv_projections, mlp), against the oracle:

* LLaMA-7B Q4_0 shapes, two layers plus lm_head 32000x4096, replayed from its
  HIP graph on two tokens with different inputs (every output checked on
  sampled rows, so the graph reads the inputs written before each run);
* LLaMA-7B Q4_0 shapes at batch 4 (the batch 3-8 grouped and paired launches);
* a converted Q8_0 directory loaded by ModelWeights at batch 2 without the
  graph, and at batch 3 (gate/up/SiLU as two GEMVs and torch's SiLU and
  product) under the graph;
* qkv_projections and mlp at decode against the reference composition.
"""

import numpy as np
import pytest
import torch

from helpers import assert_gemv_close, gen, oq, syn, to_np

pytestmark = pytest.mark.gpu

PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
        "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def _layer(gpu, shapes, fmt, seed):
    """One layer's 7 projections packed in one device buffer (as a layer file is)."""
    from gdsllm_amd.runtime import ext

    make = syn.q4_0_weights if fmt == "q4_0" else syn.q8_0_weights
    g = torch.Generator(device=gpu).manual_seed(seed)
    mats = [make(m, k, g) for m, k in shapes]
    buf, offs = syn.pack_buffer(mats)
    h = ext().GdsBufferHandle.from_tensor(buf)
    return {f"{p}.weight": {"buffer": h, "shape": [m, k], "gguf_type": fmt, "offset": o}
            for p, (m, k), o in zip(PROJ, shapes, offs)}, mats


def _rows(M, seed, n=256):
    return np.arange(M) if M <= n else np.sort(np.random.default_rng(seed).choice(M, n, replace=False))


def _check(y, w_raw, x, fmt, K, what, seed):
    """y [B, M] device output vs the oracle on sampled rows of w_raw [M, row bytes]."""
    rows = _rows(w_raw.shape[0], seed)
    deq = (oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0)(to_np(w_raw[torch.as_tensor(rows, device=w_raw.device)]))
    assert_gemv_close(to_np(y)[:, rows], deq.reshape(len(rows), K), to_np(x), what)


def _check_h(h, wg_raw, wu_raw, x, fmt, K, what, seed):
    rows = _rows(wg_raw.shape[0], seed)
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    sel = torch.as_tensor(rows, device=wg_raw.device)
    g = oq.gemv(dq(to_np(wg_raw[sel])).reshape(len(rows), K), to_np(x)).astype(np.float16)
    u = oq.gemv(dq(to_np(wu_raw[sel])).reshape(len(rows), K), to_np(x)).astype(np.float16)
    want = (oq.silu_fp16(g).astype(np.float32) * u.astype(np.float32)).astype(np.float64)
    got = to_np(h)[:, rows].astype(np.float64)
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    assert np.isfinite(got).all() and rel <= oq.GEMV_REL_L2, f"{what}: h rel L2 {rel:.3e}"


def _fill(sweep, seed):
    g = torch.Generator().manual_seed(seed)
    for bufs in (sweep.attn_in, sweep.attn_out, sweep.mlp_in):
        for b in bufs:
            b.copy_(syn.activations(b.shape[0], b.shape[1], g))
    sweep.final_in.copy_(syn.activations(sweep.final_in.shape[0], sweep.final_in.shape[1], g))


def _check_sweep(sweep, mats, head, fmt, tag):
    H, Fd = sweep.hidden, sweep.ffn
    for i, m in enumerate(mats):
        for j, y in enumerate((sweep.q[i], sweep.k[i], sweep.v[i])):
            _check(y, m[j], sweep.attn_in[i].cpu(), fmt, H, f"{tag} layer {i} {PROJ[j]}", 10 + i)
        _check(sweep.o[i], m[3], sweep.attn_out[i].cpu(), fmt, H, f"{tag} layer {i} o_proj", 20 + i)
        _check_h(sweep.h[i], m[4], m[5], sweep.mlp_in[i].cpu(), fmt, H, f"{tag} layer {i} gate/up", 30 + i)
        _check(sweep.down[i], m[6], sweep.h[i].cpu(), fmt, Fd, f"{tag} layer {i} down_proj", 40 + i)
    _check(sweep.logits, head, sweep.final_in.cpu(), fmt, sweep.final_in.shape[1], f"{tag} lm_head", 50)


@pytest.mark.parametrize("B", [1, 4])
def test_decode_sweep_llama7b_shapes_graph(gpu, B):
    """Batch 1 (row-span launches) and batch 4 (the grouped q/k/v and the
    gate/up/SiLU launches of the x-in-registers kernel)."""
    from gdsllm_amd.runtime import ext
    from gdsllm_amd.runtime.scheduler import DecodeSweep

    shapes = [(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008)]
    layers, mats = zip(*(_layer(gpu, shapes, "q4_0", 9000 + i) for i in range(2)))
    head = syn.q4_0_weights(32000, 4096, torch.Generator(device=gpu).manual_seed(9100))
    lm = {"buffer": ext().GdsBufferHandle.from_tensor(head), "shape": [32000, 4096], "gguf_type": "q4_0", "offset": 0}
    sweep = DecodeSweep(list(layers), lm, batch=B)
    assert sweep.launches_per_token == 9
    for token in range(2):
        _fill(sweep, 9200 + token)
        sweep.run()
        torch.cuda.synchronize()
        _check_sweep(sweep, mats, head, "q4_0", f"B={B} token {token}")


@pytest.mark.parametrize("B,graph", [(2, False), (3, True)])
def test_decode_sweep_loaded_q8_0(gpu, tmp_path, B, graph):
    """A converted Q8_0 directory at batch 2 (fused gate/up/SiLU) and at batch
    3, where the fused launch is refused and the sweep runs the two GEMVs and
    torch's SiLU and product, captured in the token's graph and replayed for
    two tokens."""
    from gdsllm_amd.runtime.scheduler import DecodeSweep
    from gdsllm_amd.runtime.torch_bridge import ModelWeights
    from gdsllm_amd.synthetic_model import write_llama

    d = str(tmp_path / "q8")
    write_llama(d, quant="q8_0", layers=2, hidden=512, ffn=1024, vocab=640, seed=9300)
    mw = ModelWeights(d)
    loaded = [mw.load_layer(i) for i in range(2)]
    head, _hh = mw.load_special("lm_head")
    layers = [t for t, _h in loaded]
    sweep = DecodeSweep(layers, head["lm_head.weight"], batch=B, use_graph=graph)
    for token in range(2 if graph else 1):
        _fill(sweep, 9301 + token)
        sweep.run()
        torch.cuda.synchronize()
    assert sweep.fused_gate_up == (B <= 2)
    assert sweep.launches_per_token == (4 if B <= 2 else 5) * 2 + 1

    def raw(meta):
        from gdsllm_amd.runtime import ext

        m, k = meta["shape"]
        return ext().view_tensor(meta["buffer"], [m, k // 32 * 34], "uint8", meta["offset"])

    mats = [[raw(lw[f"{p}.weight"]) for p in PROJ] for lw in layers]
    _check_sweep(sweep, mats, raw(head["lm_head.weight"]), "q8_0", f"q8_0 b{B}")


@pytest.mark.parametrize("fmt,B", [("q4_0", 1), ("q8_0", 2), ("q4_0", 6), ("q8_0", 3)])
def test_qkv_projections_and_mlp_decode(gpu, fmt, B):
    from gdsllm_amd.runtime import llama

    shapes = [(1024, 1024), (256, 1024), (256, 1024), (1024, 1024), (2816, 1024), (2816, 1024), (1024, 2816)]
    weights, mats = _layer(gpu, shapes, fmt, 9400 + B)
    x = syn.activations(B, 1024, gen(9401))
    xq, xk, xv = llama.qkv_projections(x.to(gpu).view(B, 1, 1024), weights)
    assert xq.shape == (B, 1, 1024) and xk.shape == (B, 1, 256) and xv.shape == (B, 1, 256)
    for j, y in enumerate((xq, xk, xv)):
        _check(y.view(B, -1), mats[j], x, fmt, 1024, f"{fmt} {PROJ[j]}", 60 + j)
    y = llama.mlp(x.to(gpu).view(B, 1, 1024), weights)
    torch.cuda.synchronize()
    assert y.shape == (B, 1, 1024)
    # reference composition: the fused h, then down (h checked against the oracle separately)
    dq = oq.dequant_q4_0 if fmt == "q4_0" else oq.dequant_q8_0
    g = oq.gemv(dq(to_np(mats[4])).reshape(2816, 1024), to_np(x)).astype(np.float16)
    u = oq.gemv(dq(to_np(mats[5])).reshape(2816, 1024), to_np(x)).astype(np.float16)
    h = (oq.silu_fp16(g).astype(np.float32) * u.astype(np.float32)).astype(np.float16)
    want = oq.gemv(dq(to_np(mats[6])).reshape(1024, 2816), h)
    got = to_np(y).reshape(B, 1024).astype(np.float64)
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    print(f"mlp {fmt} B{B}: rel L2 {rel:.2e}")
    assert np.isfinite(got).all() and rel <= oq.GEMV_REL_L2, f"mlp rel L2 {rel:.3e}"
