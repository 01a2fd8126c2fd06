"""Host side of the hot path: the `gds_io_ext` extension module and the model
code that calls it (mirrors of the reference's runtime/llama.py and
runtime/qwen_moe.py dispatch functions).

The extension is built in-tree by `python -m gdsllm_amd.build`; importing an op
without it raises ImportError — there is no CPU fallback.
"""

from __future__ import annotations

import importlib

_EXT = None


def ext():
    """The compiled `gds_io_ext` module (HIP kernels behind the C ABI)."""
    global _EXT
    if _EXT is None:
        try:
            import torch  # noqa: F401  (loads libc10 / libtorch before the extension)
            _EXT = importlib.import_module("gdsllm_amd.runtime.gds_io_ext")
        except ImportError as e:  # pragma: no cover - exercised only on a broken install
            raise ImportError(
                "gdsllm_amd.runtime.gds_io_ext is not built; run `python -m gdsllm_amd.build` "
                f"(ROCm + hipcc required): {e}"
            ) from e
    return _EXT
