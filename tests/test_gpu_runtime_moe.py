"""The Qwen-MoE MLP of the runtime mirror (gdsllm_amd/runtime/qwen_moe.py) on a
synthetic layer, end to end on the device: moe_route (fp16 router GEMV +
top-k + softmax, no host sync) and moe_mlp_selective with resident stacked
experts, the shared expert and the combine, against the oracle composition of
runtime/qwen_moe.py:386-513 (router picks compared exactly on the device's
own logits; the MLP output under a relative-L2 bound)."""

import numpy as np
import pytest
import torch

from helpers import affine_dequant_np, assert_gemv_close, gen, oq, syn, to_np

pytestmark = pytest.mark.gpu


def _layer(gpu, E, H, F, Fs, g, seed):
    from gdsllm_amd.runtime import ext

    gg = gen(seed)
    projs = [syn.affine_q4_weights(s, g, gg) for s in ([E, F, H], [E, F, H], [E, H, F], [Fs, H], [Fs, H], [H, Fs])]
    router = (torch.randn(E, H, generator=gg) * 0.05).to(torch.float16)
    shared_gate = (torch.randn(1, H, generator=gg) * 0.02).to(torch.float16)
    buf, offs = syn.pack_buffer([t for p in projs for t in p])
    handle = ext().GdsBufferHandle.from_tensor(buf.to(gpu))

    def meta(i, shape):
        return {"buffer": handle, "shape": shape, "quant_type": "affine_q4", "weight_offset": offs[3 * i],
                "scale_offset": offs[3 * i + 1], "bias_offset": offs[3 * i + 2], "group_size": g}

    names = ["mlp.switch_mlp.gate_proj", "mlp.switch_mlp.up_proj", "mlp.switch_mlp.down_proj",
             "mlp.shared_expert.gate_proj", "mlp.shared_expert.up_proj", "mlp.shared_expert.down_proj"]
    shapes = [[E, F, H], [E, F, H], [E, H, F], [Fs, H], [Fs, H], [H, Fs]]
    weights = {f"{n}.weight": meta(i, s) for i, (n, s) in enumerate(zip(names, shapes))}
    weights["mlp.gate.weight"] = router.to(gpu)
    weights["mlp.shared_expert_gate.weight"] = shared_gate.to(gpu)
    return weights, projs, router, shared_gate, handle


@pytest.mark.parametrize("E,H,F,Fs,g,k", [(32, 1024, 256, 256, 64, 4), (64, 2048, 512, 512, 64, 10)])
def test_runtime_moe_mlp_decode(gpu, E, H, F, Fs, g, k):
    from gdsllm_amd.runtime import ext
    from gdsllm_amd.runtime import qwen_moe as qm

    weights, projs, router, shared_gate, _handle = _layer(gpu, E, H, F, Fs, g, 7000 + E)
    x = syn.activations(1, H, gen(7001 + E)).view(1, 1, H)
    xd = x.to(gpu)

    idx, w, unique = qm.moe_route(xd, weights, k, sync_unique=False)
    assert unique is None and idx.dtype == torch.int32 and idx.shape == (1, 1, k)
    y = qm.moe_mlp_selective(xd, weights, None, idx, w, k)
    torch.cuda.synchronize()
    assert y.shape == (1, 1, H) and y.dtype == torch.float16

    xn = to_np(x).reshape(-1)
    # router: logits from the same kernel, picks and weights exactly the oracle's on them
    logits = to_np(ext().gemv_f16(weights["mlp.gate.weight"], xd)).reshape(1, E)
    assert_gemv_close(logits, to_np(router), xn[None, :], "router logits")
    ridx, rw = oq.route_topk(logits, k)
    np.testing.assert_array_equal(to_np(idx).reshape(1, k), ridx)
    assert np.all(np.abs(to_np(w).reshape(1, k).astype(np.float64) - rw.astype(np.float64))
                  <= oq.fp16_ulp(rw.astype(np.float64)))

    def dq(p, e=None):
        t = [a[e] if e is not None else a for a in p]
        return affine_dequant_np(*t, g).reshape(t[0].shape[0], -1)

    def expert(i):
        return lambda e: dq(projs[i], e) if 0 <= e < E else None

    eo, _ = oq.moe_gather(xn, expert(0), expert(1), expert(2), ridx[0], rw[0])
    eo = eo.astype(np.float16)
    sg = oq.gemv(dq(projs[3]), xn)[0].astype(np.float16)
    su = oq.gemv(dq(projs[4]), xn)[0].astype(np.float16)
    sh = (oq.silu_fp16(sg).astype(np.float32) * su.astype(np.float32)).astype(np.float16)
    so = oq.gemv(dq(projs[5]), sh)[0].astype(np.float16)
    gl = oq.gemv(to_np(shared_gate), xn)[0].astype(np.float16)
    want = oq.moe_combine(eo[None, :], so[None, :], gl).astype(np.float64).reshape(-1)
    got = to_np(y).astype(np.float64).reshape(-1)
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    print(f"runtime moe rel={rel:.2e}")
    assert np.all(np.isfinite(got)) and rel <= oq.GEMV_REL_L2, f"runtime MoE MLP rel L2 {rel:.3e}"
