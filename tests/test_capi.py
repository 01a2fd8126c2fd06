"""The C ABI boundary on the CPU: the library loads, exports exactly what
include/gdsllm_amd.h declares, and rejects invalid calls before touching the
device (every call below fails validation or is a no-op, so no HIP work is
issued and no GPU is needed)."""

import ctypes
import re
from pathlib import Path

import pytest

import gdsllm_amd
from gdsllm_amd import AffineExperts, capi

HEADER = Path(__file__).resolve().parents[1] / "include" / "gdsllm_amd.h"


def declared_functions() -> dict:
    """name -> (return type, argument list text) for every function prototype in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"(int|size_t|const char\*)\s+(gdsllm_\w+)\s*\(([^;]*?)\)\s*;", text, re.S):
        out[m.group(2)] = (m.group(1), " ".join(m.group(3).split()))
    return out


def test_header_declares_the_entry_points():
    names = set(declared_functions())
    assert {"gdsllm_fused_q4_0_gemv", "gdsllm_fused_q8_0_gemv", "gdsllm_fused_affine_q4_gemv", "gdsllm_dequant_q4_0",
            "gdsllm_dequant_q8_0", "gdsllm_dequant_affine_q4", "gdsllm_moe_gather_affine_q4", "gdsllm_moe_step_affine_q4",
            "gdsllm_dequant_gemm_q4_0"} <= names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(gdsllm_amd.LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"


def test_ctypes_table_matches_header():
    decl = declared_functions()
    assert set(gdsllm_amd.SIGNATURES) == set(decl), "gdsllm_amd.SIGNATURES and the header disagree"
    for name, (ret, args) in decl.items():
        n_args = 0 if args in ("void", "") else args.count(",") + 1
        assert len(gdsllm_amd.SIGNATURES[name][1]) == n_args, name


def test_version_and_empty_error():
    lib = capi()
    assert lib.gdsllm_version().startswith(b"gdsllm_amd")
    assert isinstance(lib.gdsllm_last_error(), bytes)


def _err():
    return capi().gdsllm_last_error().decode()


@pytest.mark.parametrize("name", ["gdsllm_fused_q4_0_gemv", "gdsllm_fused_q8_0_gemv"])
def test_gguf_gemv_validation(name):
    fn = getattr(capi(), name)
    assert fn(8, 8, 8, 4, 48, 1, 48, 4, None) == 1 and "multiple of 32" in _err()
    assert fn(8, 8, 8, 4, 64, 9, 64, 4, None) == 1 and "batch" in _err()
    assert fn(8, 8, 8, 4, 64, 0, 64, 4, None) == 1
    assert fn(8, 8, 8, -1, 64, 1, 64, 4, None) == 1 and "negative" in _err()
    assert fn(None, 8, 8, 4, 64, 1, 64, 4, None) == 1 and "null" in _err()
    assert fn(8, 8, 8, 4, 64, 2, 32, 4, None) == 1 and "ldx" in _err()
    assert fn(8, 9, 8, 4, 64, 1, 64, 4, None) == 1 and "aligned" in _err()
    # empty problems are silent no-ops, as in the reference launchers (fused_gemv.cu:111)
    assert fn(None, None, None, 0, 64, 1, 64, 0, None) == 0
    assert fn(None, None, None, 4, 0, 1, 0, 4, None) == 0


def test_affine_gemv_validation():
    fn = capi().gdsllm_fused_affine_q4_gemv
    assert fn(16, 16, 16, 16, 16, 4, 96, 64, 1, 96, 4, None) == 1 and "group_size" in _err()
    assert fn(16, 16, 16, 16, 16, 4, 64, 12, 1, 64, 4, None) == 1
    assert fn(16, 16, 16, 16, 16, 4, 64, 64, 9, 64, 4, None) == 1
    assert fn(16, 16, 16, 16, None, 4, 64, 64, 1, 64, 4, None) == 1 and "null" in _err()  # y missing
    assert fn(None, None, None, None, None, 0, 64, 64, 1, 64, 0, None) == 0


def test_dequant_validation():
    lib = capi()
    assert lib.gdsllm_dequant_q4_0(8, 8, -1, None) == 1
    assert lib.gdsllm_dequant_q4_0(None, 8, 4, None) == 1 and "null" in _err()
    assert lib.gdsllm_dequant_q4_0(None, None, 0, None) == 0
    assert lib.gdsllm_dequant_q8_0(8, None, 4, None) == 1
    a = lib.gdsllm_dequant_affine_q4
    assert a(16, 16, 16, 16, 64, 64, 12, None) == 2 and "multiple of 8" in _err()
    assert a(16, 16, 16, 16, 64, 96, 64, None) == 1 and "in_dim" in _err()
    assert a(16, 16, 16, 16, 72, 64, 64, None) == 1
    assert a(17, 16, 16, 16, 64, 64, 64, None) == 1 and "misaligned" in _err()
    assert a(None, None, None, None, 0, 64, 64, None) == 0


def test_gemv_group_validation():
    lib = capi()
    for name in ("gdsllm_fused_q4_0_gemv_group", "gdsllm_fused_q8_0_gemv_group"):
        fn = getattr(lib, name)
        w = (ctypes.c_void_p * 5)(*([16] * 5))
        y = (ctypes.c_void_p * 5)(*([16] * 5))
        dims = (ctypes.c_int64 * 5)(*([4] * 5))
        assert fn(0, w, y, dims, 16, 64, 1, 64, None) == 1 and "n must be" in _err()
        assert fn(5, w, y, dims, 16, 64, 1, 64, None) == 1
        assert fn(2, None, y, dims, 16, 64, 1, 64, None) == 1 and "null" in _err()
        assert fn(2, w, y, dims, 16, 48, 1, 48, None) == 1 and "multiple of 32" in _err()
        assert fn(2, w, y, dims, 16, 64, 9, 64, None) == 1 and "batch" in _err()
        zero = (ctypes.c_int64 * 2)(0, 0)
        assert fn(2, w, y, zero, 16, 64, 1, 64, None) == 0  # nothing to compute


def test_gate_up_silu_validation():
    lib = capi()
    for name in ("gdsllm_fused_q4_0_gate_up_silu", "gdsllm_fused_q8_0_gate_up_silu"):
        fn = getattr(lib, name)
        assert fn(16, 16, 16, 16, 4, 48, 1, 48, 4, None) == 1 and "multiple of 32" in _err()
        assert fn(None, 16, 16, 16, 4, 256, 1, 256, 4, None) == 1 and "null" in _err()
        # batch 3-8: Q4_0 with in_dim <= 8192 only (the launch itself needs a GPU)
        assert fn(16, 16, 16, 16, 4, 8448, 3, 8448, 4, None) == 2 and "batch 3-8" in _err()
        if "q8_0" in name:
            assert fn(16, 16, 16, 16, 4, 256, 3, 256, 4, None) == 2 and "batch 3-8" in _err()
        assert fn(16, 16, 18, 16, 4, 256, 1, 256, 4, None) == 2  # x off the 16-byte grid
        assert fn(16, 16, 16, 16, 4, 96, 1, 96, 4, None) == 2  # in_dim % 256 != 0
        assert fn(None, None, None, None, 0, 256, 1, 256, 0, None) == 0


def test_gemm_validation():
    g = capi().gdsllm_dequant_gemm_q4_0
    assert g(16, 16, 16, 4, 96, 2, 100, 4, None) == 2 and "aligned" in _err()
    assert g(16, 16, 16, 4, 48, 2, 48, 4, None) == 1 and "multiple of 32" in _err()
    assert g(16, 16, 16, 4, 64, 2, 32, 4, None) == 1 and "ldx" in _err()
    assert g(16, 24, 16, 4, 64, 2, 64, 4, None) == 2 and "aligned" in _err()
    assert g(None, None, None, 4, 64, 0, 64, 4, None) == 0


def test_gemm_other_formats_validation():
    q8 = capi().gdsllm_dequant_gemm_q8_0
    assert q8(16, 16, 16, 4, 48, 2, 48, 4, None) == 1 and "multiple of 32" in _err()
    assert q8(16, 16, 16, -4, 256, 2, 256, 4, None) == 1 and "negative" in _err()
    assert q8(None, 16, 16, 4, 256, 2, 256, 4, None) == 1 and "null" in _err()
    assert q8(16, 16, 16, 4, 96, 2, 96, 4, None) == 2 and "multiple of 256" in _err()
    assert q8(16, 24, 16, 4, 256, 2, 256, 4, None) == 2 and "aligned" in _err()
    assert q8(None, None, None, 4, 256, 0, 256, 4, None) == 0
    a = capi().gdsllm_dequant_gemm_affine_q4
    assert a(16, 16, 16, 16, 16, 4, 256, 12, 2, 256, 4, None) == 1 and "group_size" in _err()
    assert a(16, 16, 16, 16, 16, 4, 256, 96, 2, 256, 4, None) == 1 and "group_size" in _err()
    assert a(16, None, 16, 16, 16, 4, 256, 64, 2, 256, 4, None) == 1 and "null" in _err()
    assert a(16, 16, 16, 16, 16, 4, 512, 256, 2, 512, 4, None) == 2 and "group_size" in _err()
    assert a(16, 16, 16, 16, 16, 4, 192, 64, 2, 192, 4, None) == 2 and "multiple of 256" in _err()
    assert a(16, 18, 16, 16, 16, 4, 256, 64, 2, 256, 4, None) == 2 and "aligned" in _err()
    assert a(16, 20, 20, 16, 16, 4, 256, 32, 2, 256, 4, None) == 2 and "16-byte aligned" in _err()  # group 32


def test_moe_prefill_validation():
    lib = capi()
    ws = lib.gdsllm_moe_prefill_workspace_size
    assert ws(512, 10, 1024, 4096, 512) > 512 * 10 * (1024 + 4096) * 2
    assert ws(-1, 10, 1024, 4096, 512) == 0
    fn = lib.gdsllm_moe_prefill_affine_q4
    gate, up, down = _experts(), _experts(), _experts(N=512, K=256)
    need = ws(4, 2, 256, 512, 8)
    args = lambda g, u, d, x=16, k=2, t=4, wsb=need: (ctypes.byref(g) if g else None, ctypes.byref(u), ctypes.byref(d),  # noqa: E731
                                                      x, 512, 16, 16, t, k, 16, 512, 256, wsb, None)
    assert fn(*args(None, up, down)) == 1 and "gate is null" in _err()
    assert fn(*args(gate, up, _experts(N=512, K=512))) == 1 and "disagree" in _err()
    assert fn(*args(gate, up, down, k=0)) == 1 and "top_k" in _err()
    assert fn(*args(gate, up, down, t=0)) == 0  # nothing to compute
    assert fn(*args(gate, up, down, x=None)) == 1 and "null" in _err()
    assert fn(*args(gate, up, down, wsb=need - 1)) == 1 and "workspace" in _err()
    assert fn(*args(gate, up, _experts(N=512, K=256, g=256))) == 1  # down grouping differs
    odd = _experts(N=192, K=512)
    assert fn(*args(odd, _experts(N=192, K=512), _experts(N=512, K=192, g=64))) == 2 and "multiples of 256" in _err()


def _experts(w=16, s=16, b=16, E=8, N=256, K=512, g=64, ws=None):
    return AffineExperts(w, s, b, ws if ws is not None else N * K // 2, N * K // g * 2, N * K // g * 2, E, N, K, g)


def test_moe_gather_validation():
    lib = capi()
    gate, up = _experts(), _experts()
    down = _experts(N=512, K=256)
    ws = lib.gdsllm_moe_gather_workspace_size(3, 256)
    assert ws >= 3 * 2 * 256 * 2 and ws % 256 == 0
    call = lambda g, u, d, k=3, wsb=ws, idx=16: lib.gdsllm_moe_gather_affine_q4(  # noqa: E731
        ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), 16, idx, 16, k, 16, 16, wsb, None)
    assert call(gate, up, down, k=0) == 1 and "top_k" in _err()
    assert call(gate, up, down, k=65) == 1
    assert call(gate, up, _experts(N=256, K=512)) == 1 and "disagree" in _err()
    assert call(gate, up, down, wsb=ws - 256) == 1 and "workspace" in _err()
    assert call(_experts(g=48), up, down) == 1
    assert call(_experts(w=8), up, down) == 1 and "16-byte" in _err()
    assert call(gate, up, down, idx=18) == 1 and "misaligned" in _err()
    assert lib.gdsllm_moe_gather_affine_q4(None, ctypes.byref(up), ctypes.byref(down), 16, 16, 16, 3, 16, 16, ws,
                                           None) == 1


def test_moe_step_validation():
    """The fused decode step checks its arguments, and answers UNSUPPORTED (2)
    for shapes outside its kernels before touching the device."""
    lib = capi()
    H, F = 2048, 512
    gate, up, down = _experts(N=F, K=H), _experts(N=F, K=H), _experts(N=H, K=F)
    sg, su, sd = _experts(E=1, N=F, K=H), _experts(E=1, N=F, K=H), _experts(E=1, N=H, K=F)
    ws = lib.gdsllm_moe_step_workspace_size(4, F)
    assert ws >= lib.gdsllm_moe_gather_workspace_size(5, F) + 2

    def call(g=gate, u=up, d=down, a=sg, b=su, c=sd, k=4, wsb=ws, sgw=16, x=16):
        return lib.gdsllm_moe_step_affine_q4(*(ctypes.byref(e) for e in (g, u, d, a, b, c)), x, 16, 16, k, sgw, 16,
                                             16, wsb, None)

    assert call(k=0) == 1 and "top_k" in _err()
    assert call(k=64) == 1
    assert call(wsb=lib.gdsllm_moe_gather_workspace_size(5, F)) == 1 and "workspace" in _err()
    assert call(d=_experts(N=F, K=H)) == 1 and "disagree" in _err()
    assert call(c=_experts(E=1, N=1024, K=F)) == 1 and "shared" in _err()
    assert call(sgw=None) == 1 and "null" in _err()
    assert call(sgw=17) == 1 and "misaligned" in _err()
    assert call(x=8) == 2  # x off the 16-byte grid: separate launches
    assert call(sgw=8) == 2  # gate row off the 16-byte grid
    small = dict(g=_experts(N=F, K=1024), u=_experts(N=F, K=1024), d=_experts(N=1024, K=F),
                 a=_experts(E=1, N=F, K=1024), b=_experts(E=1, N=F, K=1024), c=_experts(E=1, N=1024, K=F))
    assert call(**small) == 2 and "separate" in _err()  # hidden not a multiple of 2048
    wide = dict(a=_experts(E=1, N=1024, K=H), b=_experts(E=1, N=1024, K=H), c=_experts(E=1, N=H, K=1024))
    assert call(**wide) == 2  # shared width differs from the routed width
    assert call(k=32, wsb=lib.gdsllm_moe_step_workspace_size(32, F)) == 2  # 33 slots, 4 per lane group: > 8


@pytest.mark.parametrize("name", ["gdsllm_dequant_gemm_gate_up_silu_q4_0", "gdsllm_dequant_gemm_gate_up_silu_q8_0"])
def test_gate_up_silu_gemm_validation(name):
    """Every call fails validation before any launch."""
    fn = getattr(capi(), name)
    assert fn(16, 16, 16, 16, 64, 100, 8, 100, 64, None) == 1 and "multiple of 32" in _err()
    assert fn(16, 16, 16, 16, -1, 256, 8, 256, 64, None) == 1 and "negative" in _err()
    assert fn(16, 16, 16, 16, 0, 256, 8, 256, 64, None) == 0  # empty: nothing to do
    assert fn(16, None, 16, 16, 64, 256, 8, 256, 64, None) == 1 and "null" in _err()
    assert fn(16, 24, 16, 16, 64, 256, 8, 256, 64, None) == 2 and "aligned" in _err()
    assert fn(16, 16, 16, 16, 64, 96, 8, 96, 64, None) == 2 and "256" in _err()
    assert fn(16, 16, 16, 16, 64, 256, 8, 200, 64, None) == 1 and "ldx" in _err()


def test_moe_step_routed_validation():
    """The routed step checks the router arguments and every step argument
    before it launches anything: each call below fails validation."""
    lib = capi()
    H, F, E = 2048, 512, 64
    gate, up, down = _experts(E=E, N=F, K=H), _experts(E=E, N=F, K=H), _experts(E=E, N=H, K=F)
    sg, su, sd = _experts(E=1, N=F, K=H), _experts(E=1, N=F, K=H), _experts(E=1, N=H, K=F)
    ws = lib.gdsllm_moe_step_routed_workspace_size(4, F, E)
    assert ws >= lib.gdsllm_moe_step_workspace_size(4, F) + 2 * E

    def call(router=16, g=gate, u=up, d=down, a=sg, b=su, c=sd, k=4, wsb=ws, sgw=16, x=16, idx=16, w=16):
        return lib.gdsllm_moe_step_routed_affine_q4(router, *(ctypes.byref(e) for e in (g, u, d, a, b, c)), x, k, sgw,
                                                    16, idx, w, 16, wsb, None)

    assert call(router=None) == 1 and "null" in _err()
    assert call(idx=None) == 1 and "null" in _err()
    assert call(k=0) == 1 and "top_k" in _err()
    assert call(k=65) == 1 and "top_k" in _err()
    assert call(router=8) == 1 and "misaligned" in _err()
    assert call(idx=18) == 1 and "misaligned" in _err()
    assert call(wsb=ws - 256) == 1 and "workspace" in _err()
    odd = dict(g=_experts(E=60, N=F, K=H), u=_experts(E=60, N=F, K=H), d=_experts(E=60, N=H, K=F))
    assert call(**odd, wsb=lib.gdsllm_moe_step_routed_workspace_size(4, F, 60)) == 2 and "512" in _err()
    big = dict(g=_experts(E=1024, N=F, K=H), u=_experts(E=1024, N=F, K=H), d=_experts(E=1024, N=H, K=F))
    assert call(**big, wsb=lib.gdsllm_moe_step_routed_workspace_size(4, F, 1024)) == 2
    # step checks, before the router GEMV is launched
    assert call(d=_experts(E=E, N=F, K=H)) == 1 and "disagree" in _err()
    assert call(sgw=None) == 1 and "null" in _err()
    assert call(k=32, wsb=lib.gdsllm_moe_step_routed_workspace_size(32, F, E)) == 2  # 33 slots: separate launches


@pytest.mark.parametrize("name", ["gdsllm_embed_q4_0", "gdsllm_embed_q8_0"])
def test_embed_validation(name):
    fn = getattr(capi(), name)
    assert fn(None, None, 0, 10, 64, None, None) == 0  # no tokens: nothing to do
    assert fn(16, 16, -1, 10, 64, 16, None) == 1 and "negative" in _err()
    assert fn(None, 16, 4, 10, 64, 16, None) == 1 and "null" in _err()
    assert fn(16, 16, 4, 10, 96, 16, None) == 2 and "multiple of 64" in _err()
    assert fn(16, 16, 65536, 10, 64, 16, None) == 1 and "65535" in _err()
    assert fn(18, 16, 4, 10, 64, 16, None) == 1 and "aligned" in _err()
    assert fn(16, 16, 4, 10, 64, 24, None) == 1 and "aligned" in _err()
    assert fn(16, 12, 4, 10, 64, 16, None) == 1 and "aligned" in _err()


def test_int8_validation():
    lib = capi()
    g = lib.gdsllm_fused_int8_gemv
    assert g(16, 16, 16, 16, 4, 64, 0, 64, 4, None) == 1 and "batch" in _err()
    assert g(16, 16, 16, 16, 4, 64, 9, 64, 4, None) == 1
    assert g(16, 16, 16, 16, -1, 64, 1, 64, 4, None) == 1 and "negative" in _err()
    assert g(None, 16, 16, 16, 4, 64, 1, 64, 4, None) == 1 and "null" in _err()
    assert g(16, 16, 16, 16, 4, 64, 2, 32, 4, None) == 1 and "ldx" in _err()
    assert g(16, 16, 17, 16, 4, 64, 1, 64, 4, None) == 1 and "aligned" in _err()
    assert g(None, None, None, None, 0, 64, 1, 64, 0, None) == 0  # empty problems are no-ops
    d = lib.gdsllm_dequant_int8
    assert d(16, 16, 16, -1, 4, None) == 1 and "negative" in _err()
    assert d(None, 16, 16, 2, 4, None) == 1 and "null" in _err()
    assert d(16, 17, 16, 2, 4, None) == 1 and "aligned" in _err()
    assert d(None, None, None, 0, 4, None) == 0


def test_buffer_validation():
    lib = capi()
    assert lib.gdsllm_buffer_alloc(4096, 0, None, None) == 1
    p = ctypes.c_void_p(1)
    assert lib.gdsllm_buffer_alloc(4096, -1, ctypes.byref(p), None) == 1 and p.value is None
    n = ctypes.c_int64(7)
    assert lib.gdsllm_buffer_read_file(None, 10, b"/dev/null", 4, 0, 0, 0, ctypes.byref(n)) == 1 and n.value == 0
    assert lib.gdsllm_buffer_read_file(16, 10, None, 4, 0, 0, 0, None) == 1
    assert lib.gdsllm_buffer_read_file(16, 10, b"/dev/null", 8, 0, 4, 0, None) == 1 and "exceed" in _err()
    assert lib.gdsllm_buffer_read_file(16, 10, b"/dev/null", 4, -1, 0, 0, None) == 1
    assert lib.gdsllm_buffer_read_file(16, 10, b"/no/such/file", 4, 0, 0, 0, None) == 4 and "cannot open" in _err()
    assert lib.gdsllm_buffer_free(None, 0) == 0


def test_extension_module_surface():
    """The pybind module exports the reference's functions with their argument names."""
    from gdsllm_amd.runtime import ext

    m = ext()
    expected = {
        "init": [], "shutdown": [], "is_driver_open": [],
        "load_file": ["filepath", "size_bytes", "device_id"],
        "load_file_region": ["filepath", "size_bytes", "file_offset", "device_id"],
        "load_expert": ["filepath", "w_file_offset", "w_size", "s_file_offset", "s_size", "b_file_offset", "b_size",
                        "device_id"],
        "view_tensor": ["handle", "shape", "dtype", "offset"],
        "load_tensor": ["filepath", "shape", "dtype", "file_offset", "size_bytes", "device_id"],
        "dequant_gguf": ["handle", "shape", "gguf_type", "offset", "output"],
        "fused_dequant_gemv": ["handle", "x", "weight_shape", "gguf_type", "offset"],
        "dequant_affine_q4": ["handle", "weight_shape", "weight_offset", "scale_offset", "bias_offset", "group_size",
                              "output"],
        "fused_affine_q4_gemv": ["handle", "x", "weight_shape", "weight_offset", "scale_offset", "bias_offset",
                                 "group_size"],
        # extensions of this library
        "embed_gguf": ["handle", "token_ids", "shape", "gguf_type", "offset"],
        "dequant_int8": ["weight", "scale", "output"],
        "int8_linear": ["weight", "scale", "x"],
        "moe_step_affine_q4": ["x", "entries", "top_k_indices", "top_k_weights", "shared_gate_weight"],
        "fused_dequant_gemv_group": ["handles", "x", "weight_shapes", "gguf_type", "offsets"],
        "fused_gate_up_silu": ["gate_handle", "up_handle", "x", "weight_shape", "gguf_type", "gate_offset",
                               "up_offset"],
    }
    for name, args in expected.items():
        fn = getattr(m, name)
        doc = fn.__doc__ or ""
        for a in args:
            assert re.search(rf"\b{a}\b", doc), f"{name}: argument {a} missing from the signature"
    assert hasattr(m, "GdsBufferHandle")
    for prop in ("size", "device_id", "registered"):
        assert hasattr(m.GdsBufferHandle, prop)


def test_extension_rejects_invalid_handle():
    import torch

    from gdsllm_amd.runtime import ext

    m = ext()
    x = torch.zeros(64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="invalid buffer handle"):
        m.fused_dequant_gemv(None, x, [4, 64], "q4_0", 0)
    with pytest.raises(RuntimeError, match="invalid buffer handle"):
        m.dequant_gguf(None, [4, 64], "q4_0", 0)
    with pytest.raises(RuntimeError, match="invalid buffer handle"):
        m.fused_affine_q4_gemv(None, x, [4, 64], 0, 0, 0, 64)
    with pytest.raises(RuntimeError, match="invalid buffer handle"):
        m.view_tensor(None, [4], "float16", 0)


def test_route_and_combine_validation():
    lib = capi()
    assert lib.gdsllm_gemv_f16(16, 16, 16, 4, 8, 9, 8, 4, None) == 1 and "batch" in _err()
    assert lib.gdsllm_gemv_f16(16, 16, 16, -1, 8, 1, 8, 4, None) == 1
    assert lib.gdsllm_gemv_f16(None, None, None, 0, 8, 1, 8, 4, None) == 0
    assert lib.gdsllm_gemv_f16(None, 16, 16, 4, 8, 1, 8, 4, None) == 1 and "null" in _err()
    assert lib.gdsllm_gemv_f16(16, 16, 16, 4, 8, 2, 4, 4, None) == 1 and "ldx" in _err()
    idx = 16
    assert lib.gdsllm_moe_route_topk(16, 512, 1, 512, 65, idx, 16, None) == 1 and "top_k" in _err()
    assert lib.gdsllm_moe_route_topk(16, 8, 1, 8, 9, idx, 16, None) == 1 and "top_k" in _err()
    assert lib.gdsllm_moe_route_topk(16, 5000, 1, 5000, 8, idx, 16, None) == 1 and "num_experts" in _err()
    assert lib.gdsllm_moe_route_topk(16, 512, 1, 100, 8, idx, 16, None) == 1 and "ld_logits" in _err()
    assert lib.gdsllm_moe_route_topk(16, 512, 0, 512, 8, idx, 16, None) == 0
    assert lib.gdsllm_moe_route_topk(None, 512, 1, 512, 8, idx, 16, None) == 1 and "null" in _err()
    assert lib.gdsllm_moe_combine(16, 16, 16, 16, -1, 1, None) == 1
    assert lib.gdsllm_moe_combine(16, 16, 16, 16, 0, 1, None) == 0
    assert lib.gdsllm_moe_combine(16, None, 16, 16, 8, 1, None) == 1 and "null" in _err()
    assert lib.gdsllm_moe_combine(16, 17, 16, 16, 8, 1, None) == 1 and "aligned" in _err()


def test_measurement_helpers_validation():
    lib = capi()
    assert lib.gdsllm_read_stream(16, 64, 0, 1, 16, None) == 1 and "workgroups" in _err()
    assert lib.gdsllm_read_stream(16, -16, 4, 1, 16, None) == 1
    assert lib.gdsllm_read_stream(None, 0, 4, 1, None, None) == 0  # nothing to read
    assert lib.gdsllm_read_stream(None, 64, 4, 1, 16, None) == 1 and "null" in _err()
    assert lib.gdsllm_read_stream(16, 40, 4, 1, 16, None) == 1 and "aligned" in _err()
    assert lib.gdsllm_read_stream(8, 64, 4, 1, 16, None) == 1 and "aligned" in _err()
    assert lib.gdsllm_empty_launch(0, None) == 1 and "workgroups" in _err()


def test_moe_gather_noalloc_validation():
    """The scratch-backed gather rejects what its fixed 1 MiB workspace cannot
    hold, and every argument error, before any HIP call."""
    lib = capi()
    assert lib.gdsllm_moe_gather_noalloc_max_bytes() == 1 << 20
    H = 2048
    big = [_experts(E=64, N=n, K=kk) for n, kk in ((4096, H), (4096, H), (H, 4096))]
    rc = lib.gdsllm_moe_gather_affine_q4_noalloc(*(ctypes.byref(e) for e in big), 16, 16, 16, 64, 16, None)
    assert rc == 1 and "fixed workspace" in _err()  # 64 * 3 * 4096 * 2 bytes > 1 MiB
    ok_shape = [_experts(N=n, K=kk) for n, kk in ((1024, H), (1024, H), (H, 1024))]
    call = lambda k=10, idx=16, x=16: lib.gdsllm_moe_gather_affine_q4_noalloc(  # noqa: E731
        *(ctypes.byref(e) for e in ok_shape), x, idx, 16, k, 16, None)
    assert call(k=0) == 1 and "top_k" in _err()
    assert call(idx=18) == 1 and "misaligned" in _err()
    assert call(x=None) == 1 and "null" in _err()
