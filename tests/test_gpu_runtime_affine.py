"""The reference's affine-Q4 call forms through the runtime mirror
(gdsllm_amd/runtime/qwen_moe.py), on the device, against the oracle:

* affine_q4_linear (runtime/qwen_moe.py:58-73) at decode (x [B, 1, K], the
  fused GEMV) and at prefill (x [B, S, K], S > 1);
* moe_mlp_selective with per-expert buffers from ModelWeights.load_experts
  (the reference scheduler's route, runtime/qwen_moe.py:455-492 and
  runtime/torch_bridge.py:284-362), for one token and for several, with the
  shared expert and the sigmoid-gated combine.
"""

import numpy as np
import pytest
import torch

from helpers import affine_dequant_np, assert_gemv_close, gen, oq, syn, to_np

pytestmark = pytest.mark.gpu


def _affine_meta(gpu, M, K, g, seed):
    from gdsllm_amd.runtime import ext

    words, scales, biases = syn.affine_q4_weights([M, K], g, gen(seed))
    buf, offs = syn.pack_buffer([words, scales, biases])
    handle = ext().GdsBufferHandle.from_tensor(buf.to(gpu))
    meta = {"buffer": handle, "shape": [M, K], "quant_type": "affine_q4", "weight_offset": offs[0],
            "scale_offset": offs[1], "bias_offset": offs[2], "group_size": g}
    return meta, affine_dequant_np(words, scales, biases, g).reshape(M, K)


@pytest.mark.parametrize("B,S", [(1, 1), (4, 1), (1, 33), (2, 17)])
@pytest.mark.parametrize("M,K,g", [(1024, 2048, 64), (512, 1024, 128)])
def test_affine_q4_linear(gpu, M, K, g, B, S):
    from gdsllm_amd.runtime import qwen_moe as qm

    meta, w = _affine_meta(gpu, M, K, g, 7700 + M + K + g)
    x = syn.activations(B * S, K, gen(7701 + B * S))
    y = qm.affine_q4_linear(x.to(gpu).view(B, S, K), {"proj.weight": meta}, "proj")
    torch.cuda.synchronize()
    assert y.shape == (B, S, M) and y.dtype == torch.float16
    rel, mx = assert_gemv_close(to_np(y).reshape(B * S, M), w, to_np(x), f"affine_q4_linear B{B} S{S}")
    print(f"affine_q4_linear {M}x{K} g{g} B{B} S{S}: rel={rel:.2e} max={mx:.2e}")


@pytest.mark.parametrize("n_tok", [1, 5])
def test_moe_mlp_selective_loaded_experts(gpu, tmp_path, n_tok):
    from gdsllm_amd.runtime import ext
    from gdsllm_amd.runtime import qwen_moe as qm
    from gdsllm_amd.runtime.torch_bridge import ModelWeights
    from gdsllm_amd.synthetic_model import write_moe_layer

    E, H, F, Fs, g, k = 8, 2048, 512, 512, 64, 4
    d = str(tmp_path / "moe")
    raw = write_moe_layer(d, experts=E, hidden=H, ffn=F, group=g, seed=7800 + n_tok)
    mw = ModelWeights(d)
    part, _h = mw.load_layer_partial(0)
    # shared expert and its gate (the reference keeps them in the partial layer)
    gg = gen(7801)
    shared = [syn.affine_q4_weights(s, g, gg) for s in ([Fs, H], [Fs, H], [H, Fs])]
    sbuf, soffs = syn.pack_buffer([t for p in shared for t in p])
    sh = ext().GdsBufferHandle.from_tensor(sbuf.to(gpu))
    names = ["mlp.shared_expert.gate_proj", "mlp.shared_expert.up_proj", "mlp.shared_expert.down_proj"]
    for i, (n, shape) in enumerate(zip(names, ([Fs, H], [Fs, H], [H, Fs]))):
        part[f"{n}.weight"] = {"buffer": sh, "shape": shape, "quant_type": "affine_q4",
                               "weight_offset": soffs[3 * i], "scale_offset": soffs[3 * i + 1],
                               "bias_offset": soffs[3 * i + 2], "group_size": g}
    sgate = (torch.randn(1, H, generator=gg) * 0.02).to(torch.float16)
    part["mlp.shared_expert_gate.weight"] = sgate.to(gpu)

    x = syn.activations(n_tok, H, gen(7802 + n_tok))
    xd = x.to(gpu).view(1, n_tok, H)
    rng = np.random.default_rng(7803)
    picks = np.stack([rng.choice(E, k, replace=False) for _ in range(n_tok)]).astype(np.int64)
    wts = torch.softmax(torch.randn(n_tok, k, generator=gen(7804)), -1).to(torch.float16)
    experts, _eh = mw.load_experts(0, sorted(set(picks.reshape(-1).tolist())))
    y = qm.moe_mlp_selective(xd, part, experts, torch.from_numpy(picks).to(gpu).view(1, n_tok, k),
                             wts.to(gpu).view(1, n_tok, k), k)
    torch.cuda.synchronize()
    assert y.shape == (1, n_tok, H) and y.dtype == torch.float16

    def expert_fn(proj, K):
        def f(e):
            words, scales, biases = (t[e] for t in raw[f"mlp.switch_mlp.{proj}"])
            return affine_dequant_np(words, scales, biases, g).reshape(-1, K)
        return f

    def dq(p):
        return affine_dequant_np(*p, g).reshape(p[0].shape[0], -1)

    got = to_np(y).reshape(n_tok, H).astype(np.float64)
    for t in range(n_tok):
        xn = to_np(x)[t]
        eo, _ = oq.moe_gather(xn, expert_fn("gate_proj", H), expert_fn("up_proj", H), expert_fn("down_proj", F),
                              picks[t], to_np(wts)[t])
        so, _ = oq.moe_gather(xn, lambda e: dq(shared[0]), lambda e: dq(shared[1]), lambda e: dq(shared[2]),
                              np.zeros(1, np.int64), np.ones(1, np.float16))
        gl = oq.gemv(to_np(sgate), xn)[0].astype(np.float16)
        want = oq.moe_combine(eo.astype(np.float16)[None], so.astype(np.float16)[None], gl).astype(np.float64)
        rel = float(np.linalg.norm(got[t] - want.reshape(-1)) / np.linalg.norm(want))
        print(f"moe_mlp_selective n_tok={n_tok} token {t}: rel L2 {rel:.2e}")
        assert np.isfinite(got[t]).all() and rel <= oq.GEMV_REL_L2, f"token {t}: rel L2 {rel:.3e}"
