"""gdsllm_amd — MI355X (gfx950) quantized-weight matvec for GdsLLM.

  libgdsllm_amd.so        hand-written HIP kernels behind the C ABI of
                          include/gdsllm_amd.h
  runtime.gds_io_ext      PyTorch-ROCm extension with the reference's
                          gds_io_ext op signatures, over that C ABI
  runtime.llama / .qwen_moe   the reference's dispatch functions over it
  capi()                  ctypes handle on the C ABI (argtypes declared)

Build in-tree with `python -m gdsllm_amd.build`.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libgdsllm_amd.so")

_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p


class AffineExperts(ctypes.Structure):
    """gdsllm_affine_experts (include/gdsllm_amd.h)."""

    _fields_ = [
        ("weight", _c_vp), ("scales", _c_vp), ("biases", _c_vp),
        ("weight_stride", _c_i64), ("scale_stride", _c_i64), ("bias_stride", _c_i64),
        ("num_experts", _c_i64), ("out_dim", _c_i64), ("in_dim", _c_i64), ("group_size", _c_i64),
    ]


# name -> (restype, argtypes); must match include/gdsllm_amd.h
SIGNATURES = {
    "gdsllm_last_error": (ctypes.c_char_p, []),
    "gdsllm_version": (ctypes.c_char_p, []),
    "gdsllm_buffer_alloc": (ctypes.c_int, [ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(_c_vp), ctypes.POINTER(ctypes.c_size_t)]),
    "gdsllm_buffer_free": (ctypes.c_int, [_c_vp, ctypes.c_int]),
    "gdsllm_buffer_read_file": (ctypes.c_int, [_c_vp, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t, _c_i64, _c_i64, ctypes.c_int, ctypes.POINTER(_c_i64)]),
    "gdsllm_dequant_q4_0": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_vp]),
    "gdsllm_dequant_q8_0": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_vp]),
    "gdsllm_embed_q4_0": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp]),
    "gdsllm_embed_q8_0": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp]),
    "gdsllm_dequant_int8": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_int8_gemv": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_dequant_affine_q4": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_q4_0_gemv": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_q8_0_gemv": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_q4_0_gemv_group": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_c_vp), ctypes.POINTER(_c_vp), ctypes.POINTER(_c_i64), _c_vp, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_q8_0_gemv_group": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_c_vp), ctypes.POINTER(_c_vp), ctypes.POINTER(_c_i64), _c_vp, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_q4_0_gate_up_silu": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_q8_0_gate_up_silu": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_fused_affine_q4_gemv": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_moe_gather_workspace_size": (ctypes.c_size_t, [_c_i64, _c_i64]),
    "gdsllm_moe_gather_affine_q4": (ctypes.c_int, [ctypes.POINTER(AffineExperts)] * 3 + [_c_vp, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp, ctypes.c_size_t, _c_vp]),
    "gdsllm_moe_gather_noalloc_max_bytes": (ctypes.c_size_t, []),
    "gdsllm_moe_gather_affine_q4_noalloc": (ctypes.c_int, [ctypes.POINTER(AffineExperts)] * 3 + [_c_vp, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp]),
    "gdsllm_moe_step_affine_q4": (ctypes.c_int, [ctypes.POINTER(AffineExperts)] * 6 + [_c_vp, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp, _c_vp, ctypes.c_size_t, _c_vp]),
    "gdsllm_moe_step_workspace_size": (ctypes.c_size_t, [_c_i64, _c_i64]),
    "gdsllm_moe_step_routed_affine_q4": (ctypes.c_int, [_c_vp] + [ctypes.POINTER(AffineExperts)] * 6 + [_c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, ctypes.c_size_t, _c_vp]),
    "gdsllm_moe_step_routed_workspace_size": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64]),
    "gdsllm_dequant_gemm_q4_0": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_dequant_gemm_q8_0": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_dequant_gemm_affine_q4": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_dequant_gemm_gate_up_silu_q4_0": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_dequant_gemm_gate_up_silu_q8_0": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_moe_prefill_workspace_size": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "gdsllm_moe_prefill_affine_q4": (ctypes.c_int, [ctypes.POINTER(AffineExperts)] * 3 + [_c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, ctypes.c_size_t, _c_vp]),
    "gdsllm_gemv_f16": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "gdsllm_moe_route_topk": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp]),
    "gdsllm_moe_combine": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "gdsllm_read_stream": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, ctypes.c_uint32, _c_vp, _c_vp]),
    "gdsllm_empty_launch": (ctypes.c_int, [_c_i64, _c_vp]),
}

_LIB = None


def capi() -> ctypes.CDLL:
    """The C ABI library with restype/argtypes set for every entry point."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built; run `python -m gdsllm_amd.build`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


class CapiError(RuntimeError):
    pass


def check(rc: int) -> None:
    """Raise CapiError with the library's message for a non-zero status."""
    if rc != 0:
        raise CapiError(f"status {rc}: {capi().gdsllm_last_error().decode()}")
