"""Model-directory loader: converted GdsLLM weights into HBM-resident buffers.

Same surface as the reference's runtime/torch_bridge.py (ModelWeights,
LayerCache, the TensorMeta / LayerMeta / FileMeta records, the metadata dicts
handed to the projection ops), so its schedulers run unchanged.  The files are
the ones the reference's converters write (tools/convert_gguf.py:378-431,
tools/convert_qwen_moe.py:205-276): per-layer .bin files of 4 KiB-aligned
tensors described by metadata.json.

What differs is where the bytes go.  The reference streams layers from NVMe
with cuFile for every forward pass that misses its VRAM cache; here a buffer
is filled once by pread + hipMemcpy (gds_io_ext.load_file*, double-buffered
through pinned staging) and, with 288 GB of HBM per MI355X, a whole model's
layers normally stay resident: LayerCache.preload() loads everything that fits
and the quantized tensors are consumed in place by the fused kernels (the
stacked [E, N, K] expert tensors included, which the on-device gather reads by
index instead of loading experts one by one).
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import torch

from . import ext


@dataclass
class TensorMeta:
    """One tensor entry of metadata.json (runtime/torch_bridge.py:16-35)."""

    name: str
    shape: List[int]
    dtype: str
    offset: int
    size_bytes: int
    padded_size: int
    quant: Optional[str] = None
    scale_shape: Optional[List[int]] = None
    scale_offset: Optional[int] = None
    scale_size_bytes: Optional[int] = None
    scale_padded_size: Optional[int] = None
    group_size: Optional[int] = None
    bias_shape: Optional[List[int]] = None
    bias_offset: Optional[int] = None
    bias_size_bytes: Optional[int] = None
    bias_padded_size: Optional[int] = None

    def end(self) -> int:
        """First byte past this tensor and its scale / bias regions."""
        e = self.offset + self.padded_size
        for off, size in ((self.scale_offset, self.scale_padded_size), (self.bias_offset, self.bias_padded_size)):
            if off is not None and size is not None:
                e = max(e, off + size)
        return e


@dataclass
class LayerMeta:
    index: int
    path: str
    size_bytes: int
    layer_type: Optional[str] = None
    tensors: List[TensorMeta] = field(default_factory=list)


@dataclass
class FileMeta:
    path: str
    size_bytes: int
    tensors: List[TensorMeta] = field(default_factory=list)


_TENSOR_KEYS = tuple(TensorMeta.__dataclass_fields__)


def parse_tensors(entries: Iterable[dict]) -> List[TensorMeta]:
    """TensorMeta records from metadata.json tensor entries; keys the record
    does not know (e.g. GGUF "block_size") are ignored."""
    return [TensorMeta(**{k: e.get(k) for k in _TENSOR_KEYS}) for e in entries]


def merge_regions(spans: Iterable[Tuple[int, int]]) -> List[Tuple[int, int]]:
    """Sorted, merged [start, end) byte ranges; touching ranges join."""
    out: List[List[int]] = []
    for start, end in sorted(spans):
        if out and start <= out[-1][1]:
            out[-1][1] = max(out[-1][1], end)
        else:
            out.append([start, end])
    return [(s, e) for s, e in out]


def _scale_name(name: str) -> str:
    """'self_attn.q_proj.weight' -> 'self_attn.q_proj.scale' (runtime/torch_bridge.py:172)."""
    return name[: -len(".weight")] + ".scale" if name.endswith(".weight") else name + ".scale"


class ModelWeights:
    """metadata.json of a converted model directory and its loaders
    (runtime/torch_bridge.py:78-402)."""

    SPECIAL_FILES = ("embed_tokens", "final_norm", "lm_head")

    def __init__(self, model_dir: str, device_id: int = 0):
        with open(os.path.join(model_dir, "metadata.json"), "r") as f:
            self.metadata = json.load(f)
        self.model_dir = model_dir
        self.device_id = device_id
        self._ext = None
        files = self.metadata["files"]
        self.layers: List[LayerMeta] = [
            LayerMeta(index=lm["index"], path=lm["path"], size_bytes=lm["size_bytes"],
                      layer_type=lm.get("layer_type"), tensors=parse_tensors(lm["tensors"]))
            for lm in files["layers"]
        ]
        self.special: Dict[str, Optional[FileMeta]] = {}
        for name in self.SPECIAL_FILES:
            raw = files.get(name)
            self.special[name] = None if raw is None else FileMeta(
                path=raw["path"], size_bytes=raw["size_bytes"], tensors=parse_tensors(raw["tensors"]))

    # -- driver ------------------------------------------------------------------------
    def init_gds(self):
        """Binds the extension (runtime/torch_bridge.py:113-117); the name is kept
        for the reference's callers, there is no cuFile driver on ROCm."""
        self._ext = ext()
        self._ext.init()

    def shutdown_gds(self):
        if self._ext is not None:
            self._ext.shutdown()
            self._ext = None

    def is_driver_open(self) -> bool:
        return self._ext is not None and self._ext.is_driver_open()

    def _bound(self):
        if self._ext is None:
            self.init_gds()
        return self._ext

    # -- entries -----------------------------------------------------------------------
    def _entry(self, handle, t: TensorMeta, offset: int, scale_off=None, bias_off=None):
        """What a projection op receives for tensor t living at `offset` of
        `handle` (runtime/torch_bridge.py:125-145)."""
        if t.quant in ("q4_0", "q8_0"):
            return {"buffer": handle, "shape": t.shape, "gguf_type": t.quant, "offset": offset}
        if t.quant == "affine_q4":
            return {"buffer": handle, "shape": t.shape, "quant_type": "affine_q4", "weight_offset": offset,
                    "scale_offset": t.scale_offset if scale_off is None else scale_off,
                    "bias_offset": t.bias_offset if bias_off is None else bias_off, "group_size": t.group_size}
        return self._bound().view_tensor(handle, t.shape, t.dtype, offset)

    def _add(self, tensors: dict, handle, t: TensorMeta, locate=None):
        """Adds t (and the fp16 scale view of an int8 tensor); `locate` maps a
        file offset to (handle, buffer offset) when the file was loaded in pieces."""
        where = locate or (lambda off: (handle, off))
        h, off = where(t.offset)
        if t.quant == "affine_q4":
            _, soff = where(t.scale_offset)
            _, boff = where(t.bias_offset)
            tensors[t.name] = self._entry(h, t, off, soff, boff)
        else:
            tensors[t.name] = self._entry(h, t, off)
        if t.quant == "int8" and t.scale_offset is not None:
            sh, soff = where(t.scale_offset)
            tensors[_scale_name(t.name)] = self._bound().view_tensor(sh, t.scale_shape, "float16", soff)

    # -- loaders -----------------------------------------------------------------------
    def load_layer(self, layer_index: int):
        """Whole layer file in one buffer -> (tensors, handle); keep the handle
        alive while the tensors are used (runtime/torch_bridge.py:147-178)."""
        layer = self.layers[layer_index]
        handle = self._bound().load_file(os.path.join(self.model_dir, layer.path), layer.size_bytes, self.device_id)
        tensors: dict = {}
        for t in layer.tensors:
            self._add(tensors, handle, t)
        return tensors, handle

    def load_layer_partial(self, layer_index: int, exclude_prefixes: Sequence[str] = ("mlp.switch_mlp.",)):
        """The layer's tensors except those whose name starts with one of
        exclude_prefixes, read as merged contiguous file regions, one buffer each
        (runtime/torch_bridge.py:180-282) -> (tensors, handles)."""
        layer = self.layers[layer_index]
        keep = [t for t in layer.tensors if not any(t.name.startswith(p) for p in exclude_prefixes)]
        if not keep:
            return {}, []
        path = os.path.join(self.model_dir, layer.path)
        pieces = []
        for start, end in merge_regions((t.offset, t.end()) for t in keep):
            pieces.append((start, end, self._bound().load_file_region(path, end - start, start, self.device_id)))

        def locate(file_offset: int):
            for start, end, h in pieces:
                if start <= file_offset < end:
                    return h, file_offset - start
            raise ValueError(f"File offset {file_offset} not in any loaded region")

        tensors: dict = {}
        for t in keep:
            self._add(tensors, None, t, locate)
        return tensors, [h for _, _, h in pieces]

    def load_experts(self, layer_index: int, expert_indices: Sequence[int],
                     proj_names: Sequence[str] = ("mlp.switch_mlp.gate_proj", "mlp.switch_mlp.up_proj",
                                                  "mlp.switch_mlp.down_proj")):
        """Weight + scales + biases of each listed expert of each stacked
        affine-Q4 projection, one buffer per (projection, expert)
        (runtime/torch_bridge.py:284-362) -> ({"gate_proj.5": meta, ...}, handles).
        Expert e's share of each region is e * (region bytes / E), as the
        reference computes it."""
        layer = self.layers[layer_index]
        path = os.path.join(self.model_dir, layer.path)
        by_name = {t.name: t for t in layer.tensors}
        out: dict = {}
        handles = []
        for proj in proj_names:
            t = by_name.get(f"{proj}.weight")
            if t is None or t.quant != "affine_q4":
                continue
            E = t.shape[0]
            w_each, s_each, b_each = t.padded_size // E, t.scale_size_bytes // E, t.bias_size_bytes // E
            short = proj.rsplit(".", 1)[-1]
            for e in expert_indices:
                h, w_off, s_off, b_off = self._bound().load_expert(
                    path, t.offset + e * w_each, w_each, t.scale_offset + e * s_each, s_each,
                    t.bias_offset + e * b_each, b_each, self.device_id)
                handles.append(h)
                out[f"{short}.{e}"] = {"buffer": h, "shape": t.shape[1:], "quant_type": "affine_q4",
                                       "weight_offset": w_off, "scale_offset": s_off, "bias_offset": b_off,
                                       "group_size": t.group_size}
        return out, handles

    def load_special(self, name: str):
        """embed_tokens / final_norm / lm_head file -> (tensors, handle)
        (runtime/torch_bridge.py:364-385)."""
        meta = self.special.get(name)
        if meta is None:
            raise ValueError(f"Special file '{name}' not available")
        handle = self._bound().load_file(os.path.join(self.model_dir, meta.path), meta.size_bytes, self.device_id)
        tensors: dict = {}
        for t in meta.tensors:
            self._add(tensors, handle, t)
        return tensors, handle

    @property
    def num_layers(self) -> int:
        return len(self.layers)

    @property
    def config(self) -> dict:
        return {k: v for k, v in self.metadata.items() if k not in ("files", "alignment")}


class LayerCache:
    """Layers and special files kept in HBM, least recently used evicted first
    when free device memory runs short (runtime/torch_bridge.py:404-589)."""

    def __init__(self, model_weights: ModelWeights, device: int = 0):
        self._weights = model_weights
        self._device = device
        self._layers: Dict[int, tuple] = {}
        self._specials: Dict[str, tuple] = {}
        self._lru: List[int] = []
        self._temp_handle = None
        self._hits = self._misses = self._evictions = self._used = 0

    def _free_vram(self) -> int:
        return torch.cuda.mem_get_info(self._device)[0]

    def _fits(self, size_bytes: int, min_free: int) -> bool:
        return self._free_vram() >= size_bytes + min_free

    def _touch(self, idx: int):
        if idx in self._lru:
            self._lru.remove(idx)
        self._lru.append(idx)

    def _drop(self, idx: int):
        del self._layers[idx]
        if idx in self._lru:
            self._lru.remove(idx)
        self._used -= self._weights.layers[idx].size_bytes
        self._evictions += 1
        torch.cuda.empty_cache()

    def _evict_lru_layer(self) -> bool:
        while self._lru:
            victim = self._lru[0]
            if victim in self._layers:
                self._drop(victim)
                return True
            self._lru.pop(0)
        return False

    def _load_evicting(self, load):
        while True:
            try:
                return load()
            except RuntimeError as e:
                if "out of memory" not in str(e).lower() or not self._evict_lru_layer():
                    raise

    def get_layer(self, idx: int, min_free: int = 0) -> dict:
        """The layer's tensors, loaded on a miss and cached when
        layer size + min_free fits in free device memory."""
        if idx in self._layers:
            self._hits += 1
            self._touch(idx)
            return self._layers[idx][0]
        self._misses += 1
        tensors, handle = self._load_evicting(lambda: self._weights.load_layer(idx))
        size = self._weights.layers[idx].size_bytes
        if self._fits(size, min_free):
            self._layers[idx] = (tensors, handle)
            self._used += size
            self._touch(idx)
        else:
            self._temp_handle = handle
        return tensors

    def get_special(self, name: str, min_free: int = 0) -> dict:
        if name in self._specials:
            self._hits += 1
            return self._specials[name][0]
        self._misses += 1
        tensors, handle = self._load_evicting(lambda: self._weights.load_special(name))
        size = self._weights.special[name].size_bytes
        if self._fits(size, min_free):
            self._specials[name] = (tensors, handle)
            self._used += size
        else:
            self._temp_handle = handle
        return tensors

    def preload(self, min_free: int = 0):
        """Special files, then layers in order, while they fit."""
        for name in ModelWeights.SPECIAL_FILES:
            if self._weights.special.get(name) is not None:
                self.get_special(name, min_free=min_free)
        for idx in range(self._weights.num_layers):
            if not self._fits(self._weights.layers[idx].size_bytes, min_free):
                break
            self.get_layer(idx, min_free=min_free)

    def ensure_free_vram(self, needed_bytes: int):
        """Evicts the highest-indexed cached layers (needed last in a forward
        pass) until needed_bytes are free."""
        torch.cuda.empty_cache()
        while self._free_vram() < needed_bytes and self._layers:
            self.evict_layer(max(self._layers))

    def evict_layer(self, idx: int) -> bool:
        if idx not in self._layers:
            return False
        self._drop(idx)
        return True

    def release_temp(self):
        self._temp_handle = None
        torch.cuda.empty_cache()

    def evict_all(self):
        self._layers.clear()
        self._specials.clear()
        self._lru.clear()
        self._temp_handle = None
        self._used = 0
        torch.cuda.empty_cache()

    @property
    def stats(self) -> dict:
        return {"cached_layers": len(self._layers), "total_layers": self._weights.num_layers,
                "cached_specials": len(self._specials), "vram_used_mb": self._used / (1024 * 1024),
                "vram_free_mb": self._free_vram() / (1024 * 1024), "hits": self._hits, "misses": self._misses,
                "evictions": self._evictions}
