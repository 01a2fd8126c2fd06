"""Numpy restatement of the reference's quantized-matvec arithmetic.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the checker for the HIP
kernels, never called by the product.

Every function cites the reference code it restates.  Dequantization is
bit-exact (same fp32 operations, same single round-to-nearest-even to fp16 as
the CUDA kernels); matrix-vector products are computed in float64 over those
exact fp16 weights, and kernels are compared against them under the stated
tolerance (GEMV_REL_L2 / GEMV_MAX_NORM).
"""

from __future__ import annotations

import numpy as np

Q4_0_BLOCK_BYTES = 18  # runtime/gguf_dequant.cu:73-74
Q8_0_BLOCK_BYTES = 34  # runtime/gguf_dequant.cu:29-30
QK = 32                # weights per GGUF block

# GEMV / GEMM acceptance: relative L2 over the whole output, and the largest
# per-row error normalized by that row's ||w_r * x||_2.
GEMV_REL_L2 = 2e-3
GEMV_MAX_NORM = 1e-2


def _blocks(raw, block_bytes: int) -> np.ndarray:
    a = np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray)) else np.asarray(raw, dtype=np.uint8)
    if a.size % block_bytes:
        raise ValueError(f"byte count {a.size} is not a multiple of {block_bytes}")
    return a.reshape(-1, block_bytes)


def dequant_q4_0(raw) -> np.ndarray:
    """kernel_dequant_q4_0 (runtime/gguf_dequant.cu:76-108).

    Block = fp16 d (little endian) + 16 bytes qs.  out[32b+j] = fp16(f32(d) *
    f32((qs[j] & 15) - 8)), out[32b+j+16] = fp16(f32(d) * f32((qs[j] >> 4) - 8))
    (the code's j / j+16 order, :105-106 — not the even/odd wording of its
    header comment, :18-19).  The fp32 product is exact, so one RNE rounding.
    """
    b = _blocks(raw, Q4_0_BLOCK_BYTES)
    d = np.ascontiguousarray(b[:, :2]).view(np.float16)[:, 0].astype(np.float32)[:, None]
    qs = b[:, 2:]
    lo = (qs & 15).astype(np.float32) - 8.0
    hi = (qs >> 4).astype(np.float32) - 8.0
    out = np.empty((b.shape[0], QK), dtype=np.float16)
    out[:, :16] = (d * lo).astype(np.float16)
    out[:, 16:] = (d * hi).astype(np.float16)
    return out.reshape(-1)


def dequant_q8_0(raw) -> np.ndarray:
    """kernel_dequant_q8_0 (runtime/gguf_dequant.cu:32-58): out[32b+i] = fp16(f32(d) * f32(qs[i]))."""
    b = _blocks(raw, Q8_0_BLOCK_BYTES)
    d = np.ascontiguousarray(b[:, :2]).view(np.float16)[:, 0].astype(np.float32)[:, None]
    qs = np.ascontiguousarray(b[:, 2:]).view(np.int8).astype(np.float32)
    return (d * qs).astype(np.float16).reshape(-1)


def dequant_int8(w_int8, scale_fp16) -> np.ndarray:
    """Per-column int8 weights as runtime/llama.py:162-165 dequantizes them:
    (w.float() * scale).half(), scale [1, in_dim] broadcast over the rows
    (layout from tools/convert_weights.py:55-83).  An int8 times an fp16 value
    is exact in fp32, so this is one RNE rounding of q * s."""
    q = np.asarray(w_int8, dtype=np.int8).astype(np.float32)
    s = np.asarray(scale_fp16, dtype=np.float16).reshape(1, -1).astype(np.float32)
    return (q * s).astype(np.float16)


def quantize_int8(w_fp16) -> tuple[np.ndarray, np.ndarray]:
    """quantize_tensor_int8 of tools/convert_weights.py:55-83 for a 2-D tensor:
    scale = max_r |W[r, c]| / 127 per column (at least 1e-10),
    q = clip(round(W / scale), -128, 127); returns (q int8, scale fp16 [1, cols])."""
    w = np.asarray(w_fp16, dtype=np.float16).astype(np.float32)
    scale = np.maximum(np.abs(w).max(axis=0, keepdims=True) / 127.0, 1e-10)
    q = np.clip(np.round(w / scale), -128, 127).astype(np.int8)
    return q, scale.astype(np.float16)


def unpack_affine_nibbles(words: np.ndarray) -> np.ndarray:
    """uint32 words -> nibbles, element 8w+n = (word >> 4n) & 15 (LSB first;
    runtime/affine_q4_dequant.cu:50-58, tools/convert_qwen_moe.py:170-179)."""
    w = np.asarray(words, dtype=np.uint32).reshape(-1)
    shifts = (4 * np.arange(8, dtype=np.uint32))[None, :]
    return ((w[:, None] >> shifts) & np.uint32(15)).astype(np.uint8).reshape(-1)


def dequant_affine_q4(words, scales, biases, num_elements: int, group_size: int) -> np.ndarray:
    """kernel_dequant_affine_q4 (runtime/affine_q4_dequant.cu:28-59).

    Group G = flat_index // group_size; out = fp16(f32(nib) * f32(s[G]) + f32(b[G])):
    the product is exact, the add rounds once in fp32, the cast once to fp16
    (two roundings, as the kernel does — restated in fp32, not fp64).  The two
    roundings differ from one when nib*s sits exactly on an fp16 tie and a bias
    below half an fp32 ulp of it nudges the exact sum off the tie.
    """
    nib = unpack_affine_nibbles(words)[:num_elements].astype(np.float32)
    g = np.arange(num_elements) // group_size
    s = np.asarray(scales, dtype=np.float16).reshape(-1)[g].astype(np.float32)
    b = np.asarray(biases, dtype=np.float16).reshape(-1)[g].astype(np.float32)
    v = (nib * s).astype(np.float32) + b
    return v.astype(np.float32).astype(np.float16)


def gemv(w_fp16: np.ndarray, x_fp16: np.ndarray) -> np.ndarray:
    """y[b, r] = sum_k W[r, k] * x[b, k] in float64 over the exact fp16 values.

    The fused kernels (runtime/fused_gemv.cu:27-105, 142-205;
    runtime/affine_q4_dequant.cu:79-158) accumulate the same products in fp32
    and round once to fp16; this is the exact value they approximate.
    """
    w = np.asarray(w_fp16, dtype=np.float16).astype(np.float64)
    x = np.atleast_2d(np.asarray(x_fp16, dtype=np.float16)).astype(np.float64)
    return x @ w.T


def gemv_ieee(w_fp16: np.ndarray, x_fp16: np.ndarray, rows_per_chunk: int = 256) -> np.ndarray:
    """gemv with IEEE special values kept: y[b, r] = sum_k W[r, k] * x[b, k] as
    float64 products summed element by element (no BLAS, which may skip zero
    operands), so 0 * inf = NaN and inf + -inf = NaN exactly as the
    reference's fp32 loop produces them (runtime/fused_gemv.cu:69-70,
    runtime/affine_q4_dequant.cu:125-126; the IEEE results do not depend on
    the summation order).  Finite sums equal gemv's."""
    w = np.asarray(w_fp16, dtype=np.float16).astype(np.float64)
    x = np.atleast_2d(np.asarray(x_fp16, dtype=np.float16)).astype(np.float64)
    out = np.empty((x.shape[0], w.shape[0]))
    with np.errstate(invalid="ignore", over="ignore"):
        for r0 in range(0, w.shape[0], rows_per_chunk):
            out[:, r0:r0 + rows_per_chunk] = (x[:, None, :] * w[None, r0:r0 + rows_per_chunk, :]).sum(-1)
    return out


def row_norms(w_fp16: np.ndarray, x_fp16: np.ndarray) -> np.ndarray:
    """||w_r * x_b||_2 for every (b, r): the scale of the fp32 accumulation error of row r."""
    w = np.asarray(w_fp16, dtype=np.float16).astype(np.float64)
    x = np.atleast_2d(np.asarray(x_fp16, dtype=np.float16)).astype(np.float64)
    return np.sqrt((x * x) @ (w * w).T)


def fp16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of the fp16 grid at |v| (float64): the size of one output rounding step."""
    with np.errstate(over="ignore"):
        h = np.abs(np.asarray(v, dtype=np.float64)).astype(np.float16)
    return np.spacing(h).astype(np.float64)


def gemv_errors(y_test, y_ref: np.ndarray, norms: np.ndarray) -> tuple[float, float]:
    """(relative L2 error, max per-row accumulation error / ||w_r * x||) of a kernel result.

    Every kernel (the reference's included, runtime/fused_gemv.cu:102) rounds
    its fp32 sum once to fp16, an error of up to one fp16 ulp of the result
    that does not shrink with ||w_r * x||: when the terms of a row share a sign
    (affine weights have mean ~7.5*scale + bias) |y_r| reaches 50x ||w_r * x||
    and the correctly rounded fp16 value alone would exceed the 1e-2 bound.
    The per-row figure therefore charges only what exceeds one fp16 ulp of
    y_ref; the relative L2 figure charges everything.
    """
    y = np.asarray(y_test, dtype=np.float64).reshape(y_ref.shape)
    diff = y - y_ref
    rel = float(np.linalg.norm(diff) / max(np.linalg.norm(y_ref), 1e-30))
    excess = np.maximum(np.abs(diff) - fp16_ulp(y_ref), 0.0)
    mx = float(np.max(excess / np.maximum(norms, 1e-30))) if diff.size else 0.0
    return rel, mx


def silu_fp16(g_fp16: np.ndarray) -> np.ndarray:
    """torch F.silu on an fp16 tensor: x / (1 + exp(-x)) in fp32, rounded to fp16."""
    g = np.asarray(g_fp16, dtype=np.float16).astype(np.float32)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float16)


def moe_gather(x, gate, up, down, idx, routing_weights):
    """Decode branch of moe_mlp_selective (runtime/qwen_moe.py:455-474).

    gate/up/down: callables e -> fp16 dequantized [out, in] matrix of expert e.
    For each k: g = fp16(gate_e . x), u = fp16(up_e . x) (the fused GEMV outputs),
    h = fp16(fp16(silu(g)) * u), then sum_k w_k * (down_e . h).  Returns
    (float64 exact weighted sum given the fp16 intermediates, the intermediates h).
    Indices outside the expert range contribute nothing.
    """
    x = np.asarray(x, dtype=np.float16).reshape(-1)
    acc = None
    hs = []
    for k, e in enumerate(np.asarray(idx).reshape(-1)):
        e = int(e)
        wg, wu, wd = gate(e), up(e), down(e)
        if wg is None:
            hs.append(None)
            continue
        g = gemv(wg, x)[0].astype(np.float16)
        u = gemv(wu, x)[0].astype(np.float16)
        h = (silu_fp16(g).astype(np.float32) * u.astype(np.float32)).astype(np.float16)
        hs.append(h)
        y = gemv(wd, h)[0] * float(np.float16(np.asarray(routing_weights).reshape(-1)[k]))
        acc = y if acc is None else acc + y
    if acc is None:
        acc = np.zeros(0)
    return acc, hs


def moe_prefill(x, gate, up, down, idx, routing_weights):
    """Prefill branch of moe_mlp_selective (runtime/qwen_moe.py:475-492).

    x fp16 [T, H]; gate/up/down: callables e -> fp16 dequantized [out, in]
    matrix of expert e (None for an index outside the pool, which then
    contributes nothing); idx [T, k], routing_weights fp16 [T, k].  Follows the
    reference loop: for each slot k, for each unique expert e of that slot,
    the tokens routed to e get g = fp16(F.linear(x_sel, gate_e)),
    u = fp16(F.linear(x_sel, up_e)), h = fp16(fp16(silu(g)) * u),
    d = fp16(F.linear(h, down_e)), then expert_output[mask] =
    fp16(expert_output[mask] + fp16(w * d)) (fp16 tensor ops: fp32 math, one
    rounding each).  The products are float64 over the exact fp16 operands.
    Returns (expert_output fp16 [T, H], {(t, j): (h, d)}).
    """
    x = np.asarray(x, dtype=np.float16)
    idx = np.asarray(idx).reshape(x.shape[0], -1)
    w = np.asarray(routing_weights, dtype=np.float16).reshape(idx.shape)
    T, k = idx.shape
    out = np.zeros(x.shape, dtype=np.float16)
    inter = {}
    for j in range(k):
        ids = idx[:, j]
        for e in np.unique(ids):
            e = int(e)
            wg, wu, wd = gate(e), up(e), down(e)
            if wg is None:
                continue
            toks = np.nonzero(ids == e)[0]
            xs = x[toks]
            g = (xs.astype(np.float64) @ wg.astype(np.float64).T).astype(np.float16)
            u = (xs.astype(np.float64) @ wu.astype(np.float64).T).astype(np.float16)
            h = (silu_fp16(g).astype(np.float32) * u.astype(np.float32)).astype(np.float16)
            d = (h.astype(np.float64) @ wd.astype(np.float64).T).astype(np.float16)
            prod = (w[toks, j].astype(np.float32)[:, None] * d.astype(np.float32)).astype(np.float16)
            out[toks] = (out[toks].astype(np.float32) + prod.astype(np.float32)).astype(np.float16)
            for r, t in enumerate(toks):
                inter[(int(t), j)] = (h[r], d[r])
    return out, inter


def moe_prefill_combine(d_rows, pos, routing_weights):
    """The combine step of moe_prefill alone, from given per-entry down
    outputs: out[t] = fold over j of fp16(out + fp16(w[t][j] * d_rows[pos[t][j]]))
    starting from fp16 zeros, skipping pos < 0 (runtime/qwen_moe.py:490-492)."""
    d_rows = np.asarray(d_rows, dtype=np.float16)
    pos = np.asarray(pos).reshape(len(pos), -1) if np.asarray(pos).ndim == 2 else np.asarray(pos)
    w = np.asarray(routing_weights, dtype=np.float16).reshape(pos.shape)
    T, k = pos.shape
    out = np.zeros((T, d_rows.shape[1]), dtype=np.float16)
    for j in range(k):
        ok = pos[:, j] >= 0
        prod = (w[ok, j].astype(np.float32)[:, None] * d_rows[pos[ok, j]].astype(np.float32)).astype(np.float16)
        out[ok] = (out[ok].astype(np.float32) + prod.astype(np.float32)).astype(np.float16)
    return out


def route_topk(logits, k: int):
    """moe_route (runtime/qwen_moe.py:408-412): torch.topk(logits, k) then
    F.softmax(top.float(), dim=-1).type_as(x), per row of fp16 logits [n, E].

    Pick order: value descending, ties to the lower expert index, NaN above
    every number, -0 equal to +0.  Softmax in float32: exp(l - max) / sum,
    rounded to fp16.  Returns (idx int32 [n, k], weights fp16 [n, k]).
    """
    L = np.asarray(logits, dtype=np.float16).astype(np.float32)
    n, E = L.shape
    idx = np.empty((n, k), dtype=np.int32)
    w = np.empty((n, k), dtype=np.float16)
    for t in range(n):
        v = L[t]
        nan = np.isnan(v)
        order = sorted(range(E), key=lambda e: (0, 0.0, e) if nan[e] else (1, -float(v[e]), e))
        sel = np.asarray(order[:k], dtype=np.int64)
        idx[t] = sel
        top = v[sel]
        with np.errstate(invalid="ignore", over="ignore"):
            ex = np.exp((top - top[0]).astype(np.float32)).astype(np.float32)
            total = np.float32(0.0)
            for val in ex:
                total = np.float32(total + val)
            w[t] = (ex / total).astype(np.float16)
    return idx, w


def moe_combine(expert_out, shared_out, gate_logit):
    """runtime/qwen_moe.py:508-513 on fp16 tensors [n, hidden] with one gate
    logit per row: sw = fp16(sigmoid(g)) (fp32 math), s = fp16(sw * shared),
    r = fp16(expert + s), then clamp to +-65504 (NaN stays NaN)."""
    eo = np.asarray(expert_out, dtype=np.float16).astype(np.float32)
    so = np.asarray(shared_out, dtype=np.float16).astype(np.float32)
    g = np.asarray(gate_logit, dtype=np.float16).astype(np.float32).reshape(-1, 1)
    with np.errstate(over="ignore", invalid="ignore"):
        sw = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float16).astype(np.float32)
        s = (sw * so).astype(np.float16).astype(np.float32)
        r = (eo + s).astype(np.float16)
    return np.clip(r, np.float16(-65504.0), np.float16(65504.0))
