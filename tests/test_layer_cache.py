"""LayerCache on the CPU with a stubbed ModelWeights: the out-of-memory ->
evict least recently used layer -> retry path of get_layer / get_special
(runtime/torch_bridge.py:471-480, 502-509 of the reference), the re-raise when
nothing is left to evict, errors that are not out-of-memory, the caching
decision on free memory after the load, and the stats counters
(torch_bridge.py:578-589).

The stub models device memory as a byte budget: a loaded layer's handle holds
its bytes until the last reference to it goes away, and a load that does not
fit raises RuntimeError("... out of memory ..."), as torch does for a failed
device allocation.
"""

from __future__ import annotations

import types
import weakref

import pytest

from gdsllm_amd.runtime.torch_bridge import LayerCache

MB = 1 << 20


class Handle:
    """Stands for a GdsBufferHandle: holds its bytes while referenced."""

    def __init__(self, what: str):
        self.what = what


class FakeDevice:
    def __init__(self, capacity: int):
        self.capacity = capacity
        self.used = 0

    def alloc(self, size: int, what: str):
        if self.used + size > self.capacity:
            raise RuntimeError(f"HIP out of memory. Tried to allocate {size} bytes for {what}")
        self.used += size
        handle = Handle(what)
        weakref.finalize(handle, self._free, size)
        return handle

    def _free(self, size: int):
        self.used -= size


class StubWeights:
    """The parts of ModelWeights that LayerCache uses."""

    SPECIAL_FILES = ("embed_tokens", "final_norm", "lm_head")

    def __init__(self, dev: FakeDevice, layer_sizes, special_sizes=None, fail=None):
        self.dev = dev
        self.layers = [types.SimpleNamespace(size_bytes=s) for s in layer_sizes]
        self.special = {k: types.SimpleNamespace(size_bytes=v) for k, v in (special_sizes or {}).items()}
        self.num_layers = len(layer_sizes)
        self.loads = []
        self.fail = fail  # an exception to raise on the next load, once

    def load_layer(self, idx: int):
        self.loads.append(idx)
        if self.fail is not None:
            e, self.fail = self.fail, None
            raise e
        handle = self.dev.alloc(self.layers[idx].size_bytes, f"layer {idx}")
        return {"layer": idx}, handle

    def load_special(self, name: str):
        self.loads.append(name)
        handle = self.dev.alloc(self.special[name].size_bytes, name)
        return {"special": name}, handle


def make_cache(capacity_mb: int, layer_mb, special_mb=None):
    dev = FakeDevice(capacity_mb * MB)
    w = StubWeights(dev, [m * MB for m in layer_mb], {k: v * MB for k, v in (special_mb or {}).items()})
    cache = LayerCache(w, device=0)
    cache._free_vram = lambda: dev.capacity - dev.used  # the device's free memory
    return cache, w, dev


def test_lru_eviction_on_out_of_memory_then_retry():
    cache, w, dev = make_cache(40, [10] * 5 + [20])
    for i in (0, 1, 2):
        assert cache.get_layer(i) == {"layer": i}
    # cached while free memory after the load covers one more layer: 0, 1, 2
    assert sorted(cache._layers) == [0, 1, 2]
    assert cache.get_layer(0) == {"layer": 0}  # hit: LRU order 1, 2, 0
    # layer 3 fits (40 MB) but is not cached: nothing would be left free
    assert cache.get_layer(3) == {"layer": 3}
    assert 3 not in cache._layers and cache._temp_handle is not None
    # layer 4: 30 cached + 10 temporary = 40 used; the load fails, layer 1
    # (least recently used) is evicted, the retry loads it; it replaces
    # layer 3 as the temporary one
    w.loads.clear()
    assert cache.get_layer(4) == {"layer": 4}
    assert w.loads == [4, 4]
    assert sorted(cache._layers) == [0, 2] and cache._lru == [2, 0]
    assert dev.used == 30 * MB
    # a hit on layer 2 makes layer 0 the least recently used
    assert cache.get_layer(2) == {"layer": 2}
    assert cache._lru == [0, 2]
    # layer 5 (20 MB): 30 used, the load fails, layer 0 goes, the retry fits
    w.loads.clear()
    assert cache.get_layer(5) == {"layer": 5}
    assert w.loads == [5, 5]
    assert sorted(cache._layers) == [2]
    st = cache.stats
    assert (st["hits"], st["misses"], st["evictions"]) == (2, 6, 2)
    assert st["cached_layers"] == 1 and st["total_layers"] == 6
    assert st["vram_used_mb"] == 10.0 and st["vram_free_mb"] == 10.0


def test_out_of_memory_reraised_when_nothing_is_left_to_evict():
    cache, w, dev = make_cache(25, [10, 10, 30])
    cache.get_layer(0)
    cache.get_layer(1)
    assert sorted(cache._layers) == [0]  # layer 1 left only 5 MB free
    w.loads.clear()
    with pytest.raises(RuntimeError, match="out of memory"):
        cache.get_layer(2)  # 30 MB never fits: layer 0 evicted, then re-raised
    assert w.loads == [2, 2]
    assert cache._layers == {} and cache._lru == []
    assert cache.stats["evictions"] == 1


def test_other_errors_are_not_retried():
    cache, w, dev = make_cache(100, [10, 10])
    cache.get_layer(0)
    w.fail = RuntimeError("read failed: short file")
    w.loads.clear()
    with pytest.raises(RuntimeError, match="short file"):
        cache.get_layer(1)
    assert w.loads == [1]
    assert sorted(cache._layers) == [0] and cache.stats["evictions"] == 0


def test_special_load_evicts_layers_and_min_free():
    cache, w, dev = make_cache(45, [10] * 4, {"embed_tokens": 20})
    for i in range(3):
        cache.get_layer(i)
    assert sorted(cache._layers) == [0, 1, 2]
    # 30 used; the 20 MB embedding fails, evicting layer 0 frees room
    w.loads.clear()
    assert cache.get_special("embed_tokens") == {"special": "embed_tokens"}
    assert w.loads == ["embed_tokens", "embed_tokens"]
    assert sorted(cache._layers) == [1, 2]
    assert "embed_tokens" not in cache._specials  # 5 MB free after it: kept as the temporary
    cache.release_temp()
    assert dev.used == 20 * MB
    assert cache.get_special("embed_tokens") == {"special": "embed_tokens"}  # a miss again
    assert cache.stats["misses"] == 5 and cache.stats["hits"] == 0
    # min_free: a layer is cached only if free >= size + min_free after loading
    cache.release_temp()
    cache.get_layer(3, min_free=10 * MB)  # 15 MB free after the load
    assert 3 not in cache._layers
    cache.release_temp()
    cache.get_layer(3, min_free=0)
    assert 3 in cache._layers


def test_ensure_free_vram_evicts_highest_index_first():
    cache, w, dev = make_cache(100, [10] * 5)
    for i in range(5):
        cache.get_layer(i)
    assert sorted(cache._layers) == [0, 1, 2, 3, 4]
    cache.ensure_free_vram(75 * MB)  # 50 free: evict 4, then 3, then 2
    assert sorted(cache._layers) == [0, 1]
    assert cache._lru == [0, 1]
    assert cache.evict_layer(7) is False
    cache.evict_all()
    assert cache._layers == {} and cache.stats["vram_used_mb"] == 0
