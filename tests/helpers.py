"""Shared helpers for the parity tests: seeded inputs, calls through the C ABI,
oracle comparisons."""

from __future__ import annotations

import ctypes
import functools

import numpy as np
import torch

from gdsllm_amd import AffineExperts, capi, check
from gdsllm_amd import synthetic as syn
from oracle import quant as oq


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def on_gpu(t: torch.Tensor, dev, pad_front: int = 0) -> torch.Tensor:
    """Copy to the GPU; with pad_front > 0 the data starts pad_front bytes into
    a larger allocation (to exercise misaligned entry paths).  Returns a view
    whose data_ptr() is the shifted start."""
    if pad_front == 0:
        return t.contiguous().to(dev)
    raw = t.contiguous().view(torch.uint8).reshape(-1)
    buf = torch.zeros(raw.numel() + pad_front + 64, dtype=torch.uint8, device=dev)
    buf[pad_front:pad_front + raw.numel()] = raw.to(dev)
    return buf[pad_front:pad_front + raw.numel()]


def assert_gemv_close(y_test: np.ndarray, w_fp16: np.ndarray, x_fp16: np.ndarray, what: str = "") -> tuple:
    y_ref = oq.gemv(w_fp16, x_fp16)
    norms = oq.row_norms(w_fp16, x_fp16)
    rel, mx = oq.gemv_errors(y_test.astype(np.float64), y_ref, norms)
    assert np.all(np.isfinite(y_test)), f"{what}: non-finite output"
    assert rel <= oq.GEMV_REL_L2, f"{what}: rel L2 {rel:.3e} > {oq.GEMV_REL_L2}"
    assert mx <= oq.GEMV_MAX_NORM, f"{what}: max normalized error {mx:.3e} > {oq.GEMV_MAX_NORM}"
    return rel, mx


def gguf_gemv(fmt: str, w_dev: torch.Tensor, x_dev: torch.Tensor, M: int, K: int) -> torch.Tensor:
    """y [B, M] via gdsllm_fused_{fmt}_gemv; x_dev is [B, K] contiguous."""
    B = x_dev.shape[0]
    y = torch.empty(B, M, dtype=torch.float16, device=x_dev.device)
    fn = capi().gdsllm_fused_q4_0_gemv if fmt == "q4_0" else capi().gdsllm_fused_q8_0_gemv
    check(fn(ptr(w_dev), ptr(x_dev), ptr(y), M, K, B, K, M, stream()))
    torch.cuda.synchronize()
    return y


def affine_gemv(words, scales, biases, x_dev, M, K, g) -> torch.Tensor:
    B = x_dev.shape[0]
    y = torch.empty(B, M, dtype=torch.float16, device=x_dev.device)
    check(capi().gdsllm_fused_affine_q4_gemv(ptr(words), ptr(scales), ptr(biases), ptr(x_dev), ptr(y), M, K, g, B, K, M,
                                             stream()))
    torch.cuda.synchronize()
    return y


def experts_struct(words: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int) -> AffineExperts:
    E, N, kw = words.shape
    K = kw * 8
    return AffineExperts(ptr(words), ptr(scales), ptr(biases), N * kw * 4, N * (K // group_size) * 2,
                         N * (K // group_size) * 2, E, N, K, group_size)


def moe_gather(gate, up, down, x_dev, idx_dev, w_dev, group_size, return_workspace: bool = False):
    """y [hidden] via gdsllm_moe_gather_affine_q4; optionally also the fp16
    workspace [top_k][2][ffn] holding the phase-1 gate/up outputs."""
    g, u, d = (experts_struct(*p, group_size) for p in (gate, up, down))
    top_k = idx_dev.numel()
    ws_bytes = capi().gdsllm_moe_gather_workspace_size(top_k, g.out_dim)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x_dev.device)
    y = torch.empty(d.out_dim, dtype=torch.float16, device=x_dev.device)
    check(capi().gdsllm_moe_gather_affine_q4(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), ptr(x_dev), ptr(idx_dev),
                                             ptr(w_dev), top_k, ptr(y), ptr(ws), ws_bytes, stream()))
    torch.cuda.synchronize()
    if return_workspace:
        F = g.out_dim
        gu = ws[: top_k * 2 * F * 2].view(torch.float16).view(top_k, 2, F)
        h = ws[top_k * 2 * F * 2: top_k * 3 * F * 2].view(torch.float16).view(top_k, F) if writes_h(g, top_k) else None
        return y, gu, h
    return y


def writes_h(gate: AffineExperts, top_k: int) -> bool:
    """Whether the gather takes its row-span path, which also stores h = fp16(fp16(silu(g)) * u)
    after the gate/up outputs in the workspace (hidden % 2048 == 0 and <= 8192, ffn/32 in {16, 32, 64},
    at most 8 expert slots per lane)."""
    H, F = gate.in_dim, gate.out_dim
    cpr = F // 32
    if H % 2048 or H > 8192 or cpr not in (16, 32, 64):
        return False
    return -(-top_k // (64 // cpr)) <= 8


def affine_dequant_np(words: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int) -> np.ndarray:
    n = words.numel() * 8
    return oq.dequant_affine_q4(to_np(words).view(np.uint32), to_np(scales), to_np(biases), n, group_size)


def double_rounding_cases(n: int, seed: int):
    """(nib, scale, bias) triples for which fp16(nib*s+b) rounded once differs
    from rounding to fp32 first (nib*s on an fp16 tie, |b| below half an fp32
    ulp of it).  Found by vectorized sampling; every returned case is checked
    with exact float64 arithmetic (the sums below are exact in float64)."""
    rng = np.random.default_rng(seed)
    found = []
    while sum(len(f[0]) for f in found) < n:
        m = 1 << 20
        s = rng.integers(0x3C00, 0x7000, m, dtype=np.uint16).view(np.float16)  # 1 .. 8192
        nib = rng.integers(1, 16, m)
        b = (rng.integers(0x0400, 0x1C00, m, dtype=np.uint16) | (rng.integers(0, 2, m, dtype=np.uint16) << 15))
        b = b.view(np.float16)  # |b| in [2^-14, 2^-6)
        exact = nib * s.astype(np.float64) + b.astype(np.float64)
        with np.errstate(over="ignore"):
            once = exact.astype(np.float16)
            twice = exact.astype(np.float32).astype(np.float16)
        sel = np.isfinite(once) & (once.view(np.uint16) != twice.view(np.uint16))
        found.append((nib[sel], s[sel], b[sel]))
    nib = np.concatenate([f[0] for f in found])[:n]
    s = np.concatenate([f[1] for f in found])[:n]
    b = np.concatenate([f[2] for f in found])[:n]
    return nib.astype(np.uint32), s, b


def moe_pool(E, H, F, g, seed, device="cpu"):
    """Stacked affine-Q4 gate, up [E, F, H] and down [E, H, F] pools (words, scales, biases)."""
    gg = gen(seed) if device == "cpu" else torch.Generator(device=device).manual_seed(seed)
    gate = syn.affine_q4_weights([E, F, H], g, gg)
    up = syn.affine_q4_weights([E, F, H], g, gg)
    down = syn.affine_q4_weights([E, H, F], g, gg)
    return gate, up, down


def expert_fn(pool, g, E):
    """e -> expert e's dequantized fp16 matrix (None outside [0, E)), for the oracle."""
    def f(e):
        if e < 0 or e >= E:
            return None
        w, s, b = (t[e].cpu() for t in pool)
        N = w.shape[0]
        return affine_dequant_np(w, s, b, g).reshape(N, -1)
    return f


def check_moe(y, ws, gate, up, down, x, idx, wts, g, E, hk=None):
    """Three checks.  (1) phase 1: the fp16 gate/up rows in the workspace match
    the oracle GEMVs under the GEMV tolerance, and h (when the kernel stores it)
    is within one fp16 ulp of fp16(fp16(silu(g)) * u) built from those rows.
    (2) phase 2: y matches the oracle's weighted down-projection of the
    kernel's h (or of h built from its g/u), under the GEMV tolerance.  (3) end
    to end: y matches the all-oracle result in relative L2 (one-ulp fp16
    differences in g/u move h, so the per-row bound is not applied end to end)."""
    xn = to_np(x).reshape(-1)
    gf, uf, dn = expert_fn(gate, g, E), expert_fn(up, g, E), expert_fn(down, g, E)
    wsn = to_np(ws)
    hkn = to_np(hk) if hk is not None else None
    for k, e in enumerate(idx):
        e = int(e)
        if gf(e) is None:
            assert np.all(wsn[k] == 0), "rows of an out-of-range expert must be zero"
            continue
        assert_gemv_close(wsn[k, 0][None, :], gf(e), xn[None, :], f"gate k={k}")
        assert_gemv_close(wsn[k, 1][None, :], uf(e), xn[None, :], f"up k={k}")
    ref2 = None
    norm2 = 0.0
    for k, e in enumerate(idx):
        e = int(e)
        if gf(e) is None:
            continue
        h = (oq.silu_fp16(wsn[k, 0]).astype(np.float32) * wsn[k, 1].astype(np.float32)).astype(np.float16)
        if hkn is not None:
            # expf on the GPU and numpy's exp may round fp32 exp(-g) differently, which
            # can move fp16(silu(g)) by one ulp; h = fp16(silu * u) then moves by up to
            # that ulp times |u| plus its own rounding step
            sg = oq.silu_fp16(wsn[k, 0])
            bound = oq.fp16_ulp(sg) * np.abs(wsn[k, 1].astype(np.float64)) + oq.fp16_ulp(h)
            bad = np.abs(hkn[k].astype(np.float64) - h.astype(np.float64)) > bound
            if bad.any():
                i = int(np.argmax(bad))
                raise AssertionError(f"h k={k}: {int(bad.sum())} of {bad.size} differ; first n={i}: kernel {hkn[k][i]} "
                                     f"expected {h[i]} from g={wsn[k, 0][i]} u={wsn[k, 1][i]}; bad n: {np.nonzero(bad)[0][:16]}")
            h = hkn[k]
        wk = float(np.float16(to_np(wts)[k]))
        part = oq.gemv(dn(e), h)[0] * wk
        ref2 = part if ref2 is None else ref2 + part
        norm2 = norm2 + (wk ** 2) * oq.row_norms(dn(e), h)[0] ** 2
    rel2, mx2 = oq.gemv_errors(to_np(y).astype(np.float64), ref2, np.sqrt(norm2))
    assert rel2 <= oq.GEMV_REL_L2, f"moe phase-2 rel L2 {rel2:.3e}"
    assert mx2 <= oq.GEMV_MAX_NORM, f"moe phase-2 max normalized {mx2:.3e}"
    ref, _ = oq.moe_gather(xn, gf, uf, dn, idx, to_np(wts))
    rel = float(np.linalg.norm(to_np(y).astype(np.float64) - ref) / np.linalg.norm(ref))
    assert rel <= oq.GEMV_REL_L2, f"moe end-to-end rel L2 {rel:.3e}"
    print(f"moe phase2 rel={rel2:.2e} max={mx2:.2e} end-to-end rel={rel:.2e}")
    return rel2, mx2


def prefill_layout(T, k, F, H, E):
    """Byte offsets of the library's MoE-prefill workspace regions (tok, pos,
    tiles, ntiles, h, d), 256-byte aligned, in the order the library lays them out."""
    up = lambda v: (v + 255) & ~255  # noqa: E731
    n = T * k
    max_tiles = n // 32 + min(E, n) + 1
    o, out = 0, {}
    for name, size in (("tok", 4 * n), ("pos", 4 * n), ("tiles", 16 * max_tiles), ("ntiles", 16), ("h", 2 * n * F),
                       ("d", 2 * n * H)):
        out[name] = o
        o = up(o + size)
    out["total"] = o
    return out


def moe_prefill(gate, up, down, xd, idx_d, w_d, g, T, k):
    gs, us, ds = (experts_struct(*p, g) for p in (gate, up, down))
    E, F, H = gs.num_experts, gs.out_dim, gs.in_dim
    ws_bytes = capi().gdsllm_moe_prefill_workspace_size(T, k, F, H, E)
    L = prefill_layout(T, k, F, H, E)
    assert ws_bytes == L["total"]
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=xd.device)
    y = torch.full((T, H), 3.0, dtype=torch.float16, device=xd.device)
    check(capi().gdsllm_moe_prefill_affine_q4(ctypes.byref(gs), ctypes.byref(us), ctypes.byref(ds), ptr(xd), H,
                                              ptr(idx_d), ptr(w_d), T, k, ptr(y), H, ptr(ws), ws_bytes, stream()))
    torch.cuda.synchronize()
    n = T * k
    part = lambda name, dt, count: ws[L[name]:L[name] + count * dt.itemsize].view(dt)  # noqa: E731
    tok = to_np(part("tok", torch.int32, n))
    pos = to_np(part("pos", torch.int32, n)).reshape(T, k)
    ntiles = int(to_np(part("ntiles", torch.int32, 1))[0])
    tiles = to_np(part("tiles", torch.int32, 4 * ntiles)).reshape(ntiles, 4)
    hbuf = to_np(part("h", torch.float16, n * F)).reshape(n, F)
    dbuf = to_np(part("d", torch.float16, n * H)).reshape(n, H)
    return y, tok, pos, tiles, hbuf, dbuf


def check_sort(idx, tok, pos, tiles, E, BT=32):
    """Every in-range entry (t, j) has a position p with tok[p] == t; positions
    are a permutation of 0 .. n_valid-1; the tiles cover each expert's positions
    in runs of at most BT."""
    T, k = idx.shape
    valid = (idx >= 0) & (idx < E)
    assert (pos[~valid] == -1).all()
    pv = pos[valid]
    assert sorted(pv.tolist()) == list(range(int(valid.sum())))
    for t, j in zip(*np.nonzero(valid)):
        assert tok[pos[t, j]] == t
    owner = np.full(int(valid.sum()), -1)
    owner[pv] = idx[valid]
    covered = np.zeros(len(owner), bool)
    for e, p0, cnt, _ in tiles:
        assert 1 <= cnt <= BT and (owner[p0:p0 + cnt] == e).all()
        assert not covered[p0:p0 + cnt].any()
        covered[p0:p0 + cnt] = True
    assert covered.all()


def dq_fn(pool, g):
    @functools.lru_cache(maxsize=None)
    def f(e):
        if e < 0 or e >= pool[0].shape[0]:
            return None
        w, s, b = (t[e].cpu() for t in pool)
        return affine_dequant_np(w, s, b, g).reshape(w.shape[0], -1)
    return lambda e: f(int(e))


def check_moe_prefill(y, tok, pos, hbuf, dbuf, gate, up, down, x, idx, wts, g, E, sample=None):
    T, k = idx.shape
    gf, uf, dn = dq_fn(gate, g), dq_fn(up, g), dq_fn(down, g)
    toks = range(T) if sample is None else sample
    xn = to_np(x)
    # (1) phase 2: each down row against the oracle product of the kernel's own h
    for t in toks:
        for j in range(k):
            e = int(idx[t, j])
            if gf(e) is None:
                continue
            p = pos[t, j]
            assert_gemv_close(dbuf[p][None, :], dn(e), hbuf[p][None, :], f"down t{t} j{j}")
    # (2) the combine, replayed from the kernel's down rows: bit for bit
    want = oq.moe_prefill_combine(dbuf, pos, wts)
    assert np.array_equal(to_np(y).view(np.uint16), want.view(np.uint16)), "combine differs from the fp16 fold"
    # (3) h and end to end against the all-oracle prefill on the sampled tokens
    sel = np.asarray(list(toks))
    ref, inter = oq.moe_prefill(xn[sel], gf, uf, dn, idx[sel], wts[sel])
    hk = np.stack([hbuf[pos[t, j]] for t in sel for j in range(k) if gf(int(idx[t, j])) is not None]).astype(np.float64)
    hr = np.stack([inter[(r, j)][0] for r in range(len(sel)) for j in range(k) if (r, j) in inter]).astype(np.float64)
    relh = float(np.linalg.norm(hk - hr) / np.linalg.norm(hr))
    got = to_np(y)[sel].astype(np.float64)
    rel = float(np.linalg.norm(got - ref.astype(np.float64)) / np.linalg.norm(ref.astype(np.float64)))
    print(f"moe prefill: h rel L2 {relh:.2e}, expert_output rel L2 {rel:.2e}")
    assert relh <= oq.GEMV_REL_L2, f"h rel L2 {relh:.3e}"
    assert np.isfinite(got).all() and rel <= oq.GEMV_REL_L2, f"expert_output rel L2 {rel:.3e}"


__all__ = [
    "gen", "stream", "ptr", "to_np", "on_gpu", "assert_gemv_close", "gguf_gemv", "affine_gemv", "moe_gather",
    "experts_struct", "writes_h", "affine_dequant_np", "double_rounding_cases", "syn", "oq", "capi", "check",
    "moe_pool", "expert_fn", "check_moe", "prefill_layout", "moe_prefill", "check_sort", "dq_fn", "check_moe_prefill",
]
