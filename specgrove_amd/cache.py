"""Persistent per-request KV arena and the per-wave tree-row cache.

Mirrors the reference's persistent Target cache
(continuous_tree_block_decode.py:126-261): one preallocated arena per layer,
``key_storage[l]`` / ``value_storage[l]`` of shape ``[Hkv, slots * capacity, D]``,
request ``slot`` owning ``[slot * capacity, slot * capacity + length)``.

What changes for the packed verification wave:

* the wave no longer copies every prefix into a packed ``DynamicCache``
  (``_pack_cache_sequence``, :313-361).  ``TreeVerifyCache`` only records the
  new tree rows' K/V of each layer (the rows whose KV is computed by this
  wave); the attention kernel reads each request's prefix in place from the
  arena;
* ``append_packed_sequence`` (:215-261) scatters the kept rows of every layer
  with a single ``sg_kv_commit`` launch instead of 4 launches per layer and
  two host-built index tensors.

Error behaviour is the reference's: metadata mismatches raise ValueError,
capacity overflow raises RuntimeError("Persistent request KV capacity
exhausted") before anything is written.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from . import ops


def _cache_length(cache) -> int:
    """Cached tokens of a request cache (DynamicCache or arena view)."""
    if hasattr(cache, "get_seq_length"):
        return int(cache.get_seq_length())
    return int(cache.layers[0].keys.shape[-2])


class PersistentRequestCacheLayer:
    """Request-local view of one layer of the arena (reference :126-150)."""

    def __init__(self, cache: "PersistentRequestCache", layer_index: int):
        self._cache = cache
        self._layer_index = layer_index

    def _span(self):
        pool = self._cache.pool
        start = self._cache.slot * pool.capacity
        return start, start + pool.lengths[self._cache.slot]

    @property
    def keys(self) -> torch.Tensor:
        start, end = self._span()
        return self._cache.pool.key_storage[self._layer_index][:, start:end].unsqueeze(0)

    @property
    def values(self) -> torch.Tensor:
        start, end = self._span()
        return self._cache.pool.value_storage[self._layer_index][:, start:end].unsqueeze(0)


class PersistentRequestCache:
    """Cache-compatible request view whose history is never recopied
    (reference :153-164)."""

    def __init__(self, pool: "PersistentRequestCachePool", slot: int):
        self.pool = pool
        self.slot = slot
        self.layers = [PersistentRequestCacheLayer(self, i)
                       for i in range(len(pool.key_storage))]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.pool.lengths[self.slot]


class PersistentRequestCachePool:
    """Preallocated Target KV arena shared by independent requests
    (reference :167-213).

    ``caches`` are per-request caches holding one request each (a transformers
    ``DynamicCache`` after prefill, or anything with ``layers[l].keys/values``
    of shape [1, Hkv, L, D]).  Besides the host ``lengths`` list, the pool
    keeps device copies of the lengths and slot offsets for the kernels.
    """

    def __init__(self, caches: Sequence, capacity: int):
        if not caches:
            raise ValueError("At least one cache is required")
        lengths = [_cache_length(cache) for cache in caches]
        if capacity < max(lengths):
            raise ValueError("Persistent cache capacity is below the prefix")
        layer_count = len(caches[0].layers)
        if any(len(cache.layers) != layer_count for cache in caches):
            raise ValueError("Target caches have different layer counts")
        self.capacity = int(capacity)
        self.lengths = list(lengths)
        self.key_storage: list[torch.Tensor] = []
        self.value_storage: list[torch.Tensor] = []
        for layer_index in range(layer_count):
            example = caches[0].layers[layer_index]
            if example.keys.shape[0] != 1:
                raise ValueError("Expected one request per source cache")
            shape = (example.keys.shape[1], len(caches) * self.capacity, example.keys.shape[-1])
            keys = torch.empty(shape, dtype=example.keys.dtype, device=example.keys.device)
            values = torch.empty(shape, dtype=example.values.dtype,
                                 device=example.values.device)
            for slot, (cache, length) in enumerate(zip(caches, lengths)):
                source = cache.layers[layer_index]
                start = slot * self.capacity
                keys[:, start:start + length].copy_(source.keys[0])
                values[:, start:start + length].copy_(source.values[0])
            self.key_storage.append(keys)
            self.value_storage.append(values)
        self.device = self.key_storage[0].device
        self.caches = tuple(PersistentRequestCache(self, slot) for slot in range(len(caches)))
        self._lengths_dev = None
        self._k_ptrs = None
        self._v_ptrs = None

    # -- device mirrors ---------------------------------------------------
    def _device_state(self):
        if self._lengths_dev is None:
            dev = self.device
            self._lengths_dev = torch.tensor(self.lengths, dtype=torch.int32, device=dev)
            self._k_ptrs = ops.pointer_array(self.key_storage, dev)
            self._v_ptrs = ops.pointer_array(self.value_storage, dev)
        return self._lengths_dev, self._k_ptrs, self._v_ptrs

    def slot_starts(self, caches: Sequence[PersistentRequestCache]) -> list[int]:
        return [cache.slot * self.capacity for cache in caches]

    # -- commit -----------------------------------------------------------
    def append_packed_sequence(self, packed: "TreeVerifyCache",
                               caches: Sequence[PersistentRequestCache],
                               packed_old_length: int, query_offsets: Sequence[int],
                               keep_query_rows: Sequence[Sequence[int]], device) -> None:
        """Scatter only newly accepted query KV rows back to the arena
        (reference :215-261), all layers in one sg_kv_commit call.

        ``packed`` is the wave's TreeVerifyCache: its layer l holds the new
        rows' K/V [1, Hkv, R, D], so the source row of request i's kept local
        row k is ``query_offsets[i] + k`` (the reference's
        ``packed_old_length + query_offsets[i] + k`` in its concatenated
        cache; ``packed_old_length`` must equal the wave's prefix total).
        """
        if not (len(caches) == len(query_offsets) == len(keep_query_rows) and caches):
            raise ValueError("Persistent cache append metadata disagree")
        if int(packed_old_length) != packed.prefix_total:
            raise ValueError("Persistent cache append metadata disagree")
        if len(packed.layers) != len(self.key_storage):
            raise ValueError("Persistent cache append metadata disagree")
        rows_total = packed.num_rows
        n = len(caches)
        # Request i's packed rows are [query_offsets[i], query_offsets[i+1]) (the
        # offsets are the prefix sums of the wave's block sizes).
        row_offset = np.zeros(n + 1, np.int64)
        row_offset[:n] = np.asarray(query_offsets, np.int64)
        row_offset[n] = rows_total
        if (np.diff(row_offset) < 0).any() or row_offset[0] < 0:
            raise ValueError("Persistent cache append metadata disagree")
        increments = []
        for i, (cache, rows) in enumerate(zip(caches, keep_query_rows)):
            if cache.pool is not self:
                raise ValueError("Persistent cache belongs to another pool")
            increment = len(rows)
            if self.lengths[cache.slot] + increment > self.capacity:
                raise RuntimeError("Persistent request KV capacity exhausted")
            if any(not 0 <= int(r) < row_offset[i + 1] - row_offset[i] for r in rows):
                raise ValueError("Persistent cache append metadata disagree")
            increments.append((cache.slot, increment))
        keep_stride = max(1, max(len(rows) for rows in keep_query_rows))
        keep = np.full((n, keep_stride), -1, np.int32)
        for i, rows in enumerate(keep_query_rows):
            keep[i, :len(rows)] = [int(r) for r in rows]
        slots = [cache.slot for cache in caches]
        lengths_dev, k_ptrs, v_ptrs = self._device_state()
        dev = self.device
        # Commit runs over the caller's subset of slots: gather their lengths,
        # advance them in the kernel, and scatter them back.
        slot_index = torch.tensor(slots, dtype=torch.long, device=dev)
        sub_lengths = lengths_dev.index_select(0, slot_index).contiguous()
        k0 = self.key_storage[0]
        kt = packed.layers[0].tree_keys
        ops.kv_commit(
            k_ptrs, v_ptrs, packed.key_pointers(), packed.value_pointers(),
            num_kv_heads=k0.shape[0], head_dim=k0.shape[2],
            cache_head_stride=k0.stride(0), cache_token_stride=k0.stride(1),
            tree_row_stride=kt.stride(0), tree_head_stride=kt.stride(1),
            row_offset=torch.from_numpy(row_offset.astype(np.int32)).to(dev),
            keep_rows=torch.from_numpy(keep).to(dev),
            keep_len=torch.tensor([len(r) for r in keep_query_rows], dtype=torch.int32,
                                  device=dev),
            prefix_start=torch.tensor([s * self.capacity for s in slots], dtype=torch.int64,
                                      device=dev),
            lengths=sub_lengths, capacity=self.capacity)
        lengths_dev.index_copy_(0, slot_index, sub_lengths)
        for slot, increment in increments:
            self.lengths[slot] += increment


class _TreeLayer:
    """New rows of one layer: keys/values [1, Hkv, R, D] as the model wrote them."""

    def __init__(self, keys: torch.Tensor, values: torch.Tensor):
        self.keys = keys
        self.values = values

    @property
    def tree_keys(self) -> torch.Tensor:  # [R, Hkv, D] view
        return self.keys[0].transpose(0, 1)

    @property
    def tree_values(self) -> torch.Tensor:
        return self.values[0].transpose(0, 1)


class TreeVerifyCache:
    """Cache object of one packed verification wave (replaces the packed
    ``DynamicCache`` built by ``_pack_cache_sequence``).

    ``update`` records the wave's new K/V rows of a layer and returns them
    unchanged; the attention function reads the requests' prefixes from the
    pool's arena.  ``prefix_total`` is the reference's packed prefix length
    (sum of the chosen requests' cached lengths), kept for the commit call.
    """

    def __init__(self, pool: PersistentRequestCachePool,
                 caches: Sequence[PersistentRequestCache]):
        self.pool = pool
        self.caches = tuple(caches)
        self.prefix_lengths = tuple(pool.lengths[c.slot] for c in self.caches)
        self.prefix_total = int(sum(self.prefix_lengths))
        self.layers: list[_TreeLayer] = []

    @property
    def num_rows(self) -> int:
        return int(self.layers[0].keys.shape[-2]) if self.layers else 0

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs=None):
        if key_states.shape[0] != 1 or value_states.shape != key_states.shape:
            raise ValueError("Expected one packed sequence of new rows")
        # One layout for K and V ([1, Hkv, R, D] contiguous): the kernels take a
        # single row/head stride pair for both.
        key_states = key_states.contiguous()
        value_states = value_states.contiguous()
        if layer_idx == len(self.layers):
            self.layers.append(_TreeLayer(key_states, value_states))
        elif layer_idx < len(self.layers):
            self.layers[layer_idx] = _TreeLayer(key_states, value_states)
        else:
            raise ValueError("Layers must be updated in order")
        return key_states, value_states

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.prefix_total

    def key_pointers(self) -> torch.Tensor:
        return ops.pointer_array([layer.tree_keys for layer in self.layers], self.pool.device)

    def value_pointers(self) -> torch.Tensor:
        return ops.pointer_array([layer.tree_values for layer in self.layers], self.pool.device)


def pack_cache_sequence(caches: Sequence[PersistentRequestCache], cache_factory=None,
                        device=None):
    """Drop-in for ``_pack_cache_sequence`` (reference :313-361) on arena
    caches: returns ``(TreeVerifyCache, lengths, offsets, total)`` without
    copying any prefix.  ``cache_factory`` is accepted for signature
    compatibility and unused."""
    if not caches:
        raise ValueError("At least one cache is required")
    pool = caches[0].pool
    if any(not isinstance(c, PersistentRequestCache) or c.pool is not pool for c in caches):
        raise ValueError("Packed tree verification needs caches of one persistent pool")
    packed = TreeVerifyCache(pool, caches)
    offsets = []
    total = 0
    for length in packed.prefix_lengths:
        offsets.append(total)
        total += length
    return packed, packed.prefix_lengths, tuple(offsets), total
