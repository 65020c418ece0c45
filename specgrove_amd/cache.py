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

import weakref
from typing import Sequence

import numpy as np
import torch

from . import ops

_COMMIT_KEEP_STRIDE = 32  # kept rows per request the pool's commit buffers hold at first


class DeviceStatus:
    """A status word that kernels set on a violated contract (SG_EINVAL,
    SG_ERANGE), read back without a synchronisation of its own.

    ``after_launch()`` enqueues a copy of the word into pinned host memory
    right behind the kernel; ``check()`` reads that copy once it has landed
    -- by the next wave the verifier's device-to-host transfer has waited for
    it -- and raises RuntimeError if a kernel reported an error.  The word is
    never cleared: an error stays reported.
    """

    def __init__(self, device, what: str):
        self.what = what
        self.dev = torch.zeros(1, dtype=torch.int32, device=device)
        self.host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.event = torch.cuda.Event()
        self.pending = False

    def after_launch(self) -> None:
        self.host.copy_(self.dev, non_blocking=True)
        self.event.record()
        self.pending = True

    def check(self) -> None:
        if self.pending:
            self.event.synchronize()
            self.pending = False
        code = int(self.host[0])
        if code != 0:
            raise RuntimeError(f"{self.what} reported error {code} on the device")


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
    of shape [1, Hkv, L, D]).  The arena of every layer is one slice of a
    single ``[2, layers, Hkv, slots * capacity, D]`` allocation (K then V), so
    the per-layer ``key_storage[l]`` / ``value_storage[l]`` views the reference
    exposes are contiguous and the kernels get one pointer per layer; each
    request's prefill is copied in with one stacked copy over all its layers.
    ``lengths`` (host) are the cached lengths per slot.
    """

    def __init__(self, caches: Sequence, capacity: int):
        if not caches:
            raise ValueError("At least one cache is required")
        lengths = [_cache_length(cache) for cache in caches]
        if capacity < max(lengths):
            raise ValueError("Persistent cache capacity is below the prefix")
        layers = len(caches[0].layers)
        if any(len(cache.layers) != layers for cache in caches):
            raise ValueError("Target caches have different layer counts")
        first = caches[0].layers
        if any(layer.keys.shape[0] != 1 for cache in caches for layer in cache.layers):
            raise ValueError("Expected one request per source cache")
        hkv, dim = first[0].keys.shape[1], first[0].keys.shape[-1]
        self.capacity = int(capacity)
        self.lengths = list(lengths)
        arena = torch.empty((2, layers, hkv, len(caches) * self.capacity, dim),
                            dtype=first[0].keys.dtype, device=first[0].keys.device)
        for slot, (cache, length) in enumerate(zip(caches, lengths)):
            if length == 0:
                continue
            at = slice(slot * self.capacity, slot * self.capacity + length)
            arena[0, :, :, at] = torch.stack([layer.keys[0] for layer in cache.layers])
            arena[1, :, :, at] = torch.stack([layer.values[0] for layer in cache.layers])
        self._arena = arena
        self.key_storage: list[torch.Tensor] = list(arena[0].unbind(0))
        self.value_storage: list[torch.Tensor] = list(arena[1].unbind(0))
        self.device = arena.device
        self.caches = tuple(PersistentRequestCache(self, slot) for slot in range(len(caches)))
        self._k_ptrs = None
        self._v_ptrs = None
        self._commit = None          # prepared commit call and its metadata buffers
        self._status = None          # DeviceStatus of the commits, made by the first one

    @property
    def status(self) -> DeviceStatus:
        if self._status is None:
            self._status = DeviceStatus(self.device, "KV commit")
        return self._status

    # -- device mirrors ---------------------------------------------------
    def _device_pointers(self):
        """Per-layer arena bases on the device, built once per pool."""
        if self._k_ptrs is None:
            self._k_ptrs = ops.pointer_array(self.key_storage, self.device)
            self._v_ptrs = ops.pointer_array(self.value_storage, self.device)
        return self._k_ptrs, self._v_ptrs

    def slot_starts(self, caches: Sequence[PersistentRequestCache]) -> list[int]:
        return [cache.slot * self.capacity for cache in caches]

    # -- commit -----------------------------------------------------------
    def _commit_call(self, layers: int, keep_stride: int) -> dict:
        """The pool's commit call, bound once to persistent metadata buffers
        sized for every slot (rebuilt only when a wave has more layers or
        longer keep lists than they hold).  Layout (int64 words): the wave's
        tree-row pointers per layer (K, then V), the slot starts, then int32
        pairs: row offsets [slots+1], kept rows [slots, stride], keep lengths
        [slots], current lengths [slots]."""
        c = self._commit
        if c is not None and c["layers"] == layers and c["stride"] >= keep_stride:
            return c
        cap = len(self.caches)
        stride = max(keep_stride, _COMMIT_KEEP_STRIDE, c["stride"] if c else 0)
        words32 = (cap + 1) + cap * stride + 2 * cap
        words32 += words32 % 2
        total = 2 * layers + cap + words32 // 2
        dev = torch.zeros(total, dtype=torch.int64, device=self.device)
        host = torch.zeros(total, dtype=torch.int64, pin_memory=True)
        d32 = dev[2 * layers + cap:].view(torch.int32)
        base = cap + 1 + cap * stride
        k_ptrs, v_ptrs = self._device_pointers()
        k0 = self.key_storage[0]
        call = ops.prepare_kv_commit(
            k_ptrs[:layers], v_ptrs[:layers], dev[:layers], dev[layers:2 * layers],
            num_kv_heads=k0.shape[0], head_dim=k0.shape[2],
            cache_head_stride=k0.stride(0), cache_token_stride=k0.stride(1),
            tree_row_stride=k0.shape[2], tree_head_stride=k0.shape[2],
            row_offset=d32[:cap + 1], keep_rows=d32[cap + 1:base].view(cap, stride),
            keep_len=d32[base:base + cap], prefix_start=dev[2 * layers:2 * layers + cap],
            lengths=d32[base + cap:base + 2 * cap], capacity=self.capacity,
            status=self.status.dev)
        copied = torch.cuda.Event()
        copied.record()
        self._commit = dict(call=call, dev=dev, host=host, layers=layers, slots=cap,
                            stride=stride, copied=copied)
        return self._commit

    def check_status(self) -> None:
        """Raise if a commit kernel reported an error (waits for the last
        commit's status copy)."""
        if self._status is not None:
            self._status.check()

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

        The call is prepared once per pool; the wave's metadata travels in
        one host-to-device copy from pinned memory.  The host checks below
        reject every case the kernel would report; a device-side error of the
        previous commit still raises here (``status``).
        """
        if not (len(caches) == len(query_offsets) == len(keep_query_rows) and caches):
            raise ValueError("Persistent cache append metadata disagree")
        if len({id(c) for c in caches}) != len(caches):
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
        commit = self._commit_call(len(packed.layers), keep_stride)
        self.status.check()
        # The pinned staging buffer is rewritten only after the previous
        # wave's copy out of it has completed.
        commit["copied"].synchronize()
        slots = [cache.slot for cache in caches]
        layers, cap, stride = commit["layers"], commit["slots"], commit["stride"]
        host64 = commit["host"].numpy()
        host32 = host64[2 * layers + cap:].view(np.int32)
        host64[:layers] = [layer.tree_keys.data_ptr() for layer in packed.layers]
        host64[layers:2 * layers] = [layer.tree_values.data_ptr() for layer in packed.layers]
        host64[2 * layers:2 * layers + n] = [s * self.capacity for s in slots]
        host32[:n + 1] = row_offset
        keep = host32[cap + 1:cap + 1 + cap * stride].reshape(cap, stride)
        keep[:n] = -1
        for i, rows in enumerate(keep_query_rows):
            keep[i, :len(rows)] = [int(r) for r in rows]
        base = cap + 1 + cap * stride
        host32[base:base + n] = [len(r) for r in keep_query_rows]
        host32[base + cap:base + cap + n] = [self.lengths[s] for s in slots]
        commit["dev"].copy_(commit["host"], non_blocking=True)
        commit["copied"].record()
        kt = packed.layers[0].tree_keys
        commit["call"].set(num_requests=n, tree_row_stride=kt.stride(0),
                           tree_head_stride=kt.stride(1))()
        self.status.after_launch()
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


class PackedPrefix:
    """The chosen requests' prefixes concatenated along the sequence, one
    ``[Hkv, P, D]`` buffer per layer: the packed cache of the reference's
    non-persistent wave (``_pack_cache_sequence``, :313-361), with the same
    ``key_storage`` / ``value_storage`` interface as the persistent arena."""

    def __init__(self, key_storage: list[torch.Tensor], value_storage: list[torch.Tensor]):
        self.key_storage = key_storage
        self.value_storage = value_storage
        self.device = key_storage[0].device


class TreeVerifyCache:
    """Cache object of one packed verification wave (replaces the packed
    ``DynamicCache`` built by ``_pack_cache_sequence``).

    ``update`` records the wave's new K/V rows of a layer and returns them
    unchanged; the attention function reads the requests' prefixes where they
    lie: in the persistent pool's arena (``pool`` set; request i's prefix
    starts at its slot) or in a ``PackedPrefix`` (non-persistent waves;
    request i's prefix starts at its packed offset).  ``prefix_total`` is the
    reference's packed prefix length (sum of the chosen requests' cached
    lengths), kept for the commit and split calls.
    """

    def __init__(self, pool: PersistentRequestCachePool | None,
                 caches: Sequence, prefix: "PackedPrefix | None" = None,
                 prefix_lengths: Sequence[int] | None = None):
        self.pool = pool
        self.caches = tuple(caches)
        if pool is not None:
            self.prefix_source = pool
            self.prefix_lengths = tuple(pool.lengths[c.slot] for c in self.caches)
            self.prefix_starts = tuple(c.slot * pool.capacity for c in self.caches)
        else:
            self.prefix_source = prefix
            self.prefix_lengths = tuple(int(v) for v in prefix_lengths)
            starts, total = [], 0
            for length in self.prefix_lengths:
                starts.append(total)
                total += length
            self.prefix_starts = tuple(starts)
        self.prefix_total = int(sum(self.prefix_lengths))
        self.device = self.prefix_source.device
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
        return ops.pointer_array([layer.tree_keys for layer in self.layers], self.device)

    def value_pointers(self) -> torch.Tensor:
        return ops.pointer_array([layer.tree_values for layer in self.layers], self.device)


# The non-persistent packed wave of a request cache, for pack_block_inputs,
# which the reference calls right after _pack_cache_sequence with the same
# request caches but without the packed cache (CTBD:1772-1787).
_WAVE_ATTR = "_specgrove_packed_wave"


def packed_wave_of(cache) -> "TreeVerifyCache | None":
    ref = getattr(cache, _WAVE_ATTR, None)
    return ref() if ref is not None else None


def pack_cache_sequence(caches: Sequence, cache_factory=None, device=None):
    """Drop-in for ``_pack_cache_sequence`` (reference :313-361).

    Arena caches of one persistent pool: returns ``(TreeVerifyCache, lengths,
    offsets, total)`` without copying any prefix.  Other request caches
    (``layers[l].keys/values`` [1, Hkv, L, D], e.g. DynamicCache; the
    non-persistent path): their prefixes are concatenated into one
    ``PackedPrefix`` per layer -- the reference's copy -- and the request
    caches remember the wave for ``pack_block_inputs``.  ``cache_factory`` is
    accepted for signature compatibility and unused.
    """
    if not caches:
        raise ValueError("At least one cache is required")
    if isinstance(caches[0], PersistentRequestCache):
        pool = caches[0].pool
        if any(not isinstance(c, PersistentRequestCache) or c.pool is not pool for c in caches):
            raise ValueError("Packed tree verification needs caches of one persistent pool")
        packed = TreeVerifyCache(pool, caches)
    else:
        lengths = [_cache_length(c) for c in caches]
        layer_count = len(caches[0].layers)
        if any(len(c.layers) != layer_count for c in caches):
            raise ValueError("Target caches have different layer counts")
        keys, values = [], []
        for layer_index in range(layer_count):
            k = [c.layers[layer_index].keys for c in caches]
            v = [c.layers[layer_index].values for c in caches]
            if any(t.shape[0] != 1 for t in k):
                raise ValueError("Expected one request per source cache")
            dev = k[0].device if device is None else torch.device(device)
            keys.append(torch.cat([t[0] for t in k], dim=1).to(dev).contiguous())
            values.append(torch.cat([t[0] for t in v], dim=1).to(dev).contiguous())
        packed = TreeVerifyCache(None, caches, PackedPrefix(keys, values), lengths)
        for c in caches:
            setattr(c, _WAVE_ATTR, weakref.ref(packed))
    offsets, total = [], 0
    for length in packed.prefix_lengths:
        offsets.append(total)
        total += length
    return packed, packed.prefix_lengths, tuple(offsets), total


class RequestCache:
    """Minimal per-request cache (``layers[l].keys/values`` [1, Hkv, L, D],
    ``update``, ``get_seq_length``), the default ``cache_factory`` of
    ``split_compacted_sequence_caches``."""

    def __init__(self):
        self.layers: list[_TreeLayer] = []

    def update(self, keys: torch.Tensor, values: torch.Tensor, layer_idx: int,
               cache_kwargs=None):
        if layer_idx == len(self.layers):
            self.layers.append(_TreeLayer(keys, values))
        elif layer_idx < len(self.layers):
            layer = self.layers[layer_idx]
            layer.keys = torch.cat((layer.keys, keys), dim=-2)
            layer.values = torch.cat((layer.values, values), dim=-2)
        else:
            raise ValueError("Layers must be updated in order")
        return self.layers[layer_idx].keys, self.layers[layer_idx].values

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self.layers[layer_idx].keys.shape[-2]) if self.layers else 0


def split_compacted_sequence_caches(packed: TreeVerifyCache, cache_factory,
                                    cache_offsets: Sequence[int], old_lengths: Sequence[int],
                                    packed_old_length: int, query_offsets: Sequence[int],
                                    keep_query_rows: Sequence[Sequence[int]], device,
                                    status: DeviceStatus | None = None):
    """Drop-in for ``_split_compacted_sequence_caches`` (reference :409-450):
    every request's new cache = its old prefix + its kept query rows, for all
    layers in one ``sg_kv_split`` call.

    The new caches are views of one ``[Hkv, sum(L_i + |keep_i|), D]`` buffer
    per layer (as the reference's slices of its one gather per layer), handed
    to ``cache_factory()`` caches through ``update`` (``RequestCache`` when
    ``cache_factory`` is None).  The source row of request i's kept row k is
    ``query_offsets[i] + k`` of the wave's new rows (the reference's
    ``packed_old_length + query_offsets[i] + k``).

    The checks below reject every kept row or size the kernel would report;
    with ``status`` (a ``DeviceStatus``, e.g. the wave loop's) a device-side
    report is also read back and raised by its next ``check()``.
    """
    count = len(cache_offsets)
    if not (count == len(old_lengths) == len(query_offsets) == len(keep_query_rows)
            and count > 0):
        raise ValueError("Packed cache split metadata disagree")
    if (int(packed_old_length) != packed.prefix_total
            or tuple(int(v) for v in old_lengths) != packed.prefix_lengths
            or tuple(int(v) for v in cache_offsets) != tuple(
                np.cumsum([0] + list(packed.prefix_lengths[:-1])).tolist())
            or not packed.layers):
        raise ValueError("Packed cache split metadata disagree")
    rows_total = packed.num_rows
    row_offset = np.zeros(count + 1, np.int64)
    row_offset[:count] = np.asarray(query_offsets, np.int64)
    row_offset[count] = rows_total
    if (np.diff(row_offset) < 0).any() or row_offset[0] < 0:
        raise ValueError("Packed cache split metadata disagree")
    for i, rows in enumerate(keep_query_rows):
        if any(not 0 <= int(r) < row_offset[i + 1] - row_offset[i] for r in rows):
            raise ValueError("Packed cache split metadata disagree")
    sizes = [int(L) + len(k) for L, k in zip(old_lengths, keep_query_rows)]
    out_offset = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    total = int(sum(sizes))
    source = packed.prefix_source
    k0 = source.key_storage[0]
    hkv, dim = k0.shape[0], k0.shape[2]
    dev = packed.device
    out_k = [torch.empty((hkv, total, dim), dtype=k0.dtype, device=dev)
             for _ in packed.layers]
    out_v = [torch.empty_like(t) for t in out_k]
    keep_stride = max(1, max(len(k) for k in keep_query_rows))
    keep = np.full((count, keep_stride), -1, np.int32)
    for i, rows in enumerate(keep_query_rows):
        keep[i, :len(rows)] = [int(r) for r in rows]
    meta = torch.from_numpy(np.concatenate([
        np.asarray(packed.prefix_starts, np.int64), out_offset])).to(dev)
    meta32 = torch.from_numpy(np.concatenate([
        np.asarray(old_lengths, np.int32), row_offset.astype(np.int32),
        np.asarray([len(k) for k in keep_query_rows], np.int32), keep.reshape(-1)])).to(dev)
    kt = packed.layers[0].tree_keys
    ops.kv_split(
        ops.pointer_array(source.key_storage[:len(packed.layers)], dev),
        ops.pointer_array(source.value_storage[:len(packed.layers)], dev),
        packed.key_pointers(), packed.value_pointers(),
        ops.pointer_array(out_k, dev), ops.pointer_array(out_v, dev),
        num_kv_heads=hkv, head_dim=dim,
        prefix_head_stride=k0.stride(0), prefix_token_stride=k0.stride(1),
        tree_row_stride=kt.stride(0), tree_head_stride=kt.stride(1),
        out_head_stride=out_k[0].stride(0), out_token_stride=out_k[0].stride(1),
        cache_offset=meta[:count], old_length=meta32[:count],
        row_offset=meta32[count:2 * count + 1], keep_len=meta32[2 * count + 1:3 * count + 1],
        keep_rows=meta32[3 * count + 1:].view(count, keep_stride),
        out_offset=meta[count:], max_tokens=max(sizes),
        status=status.dev if status is not None else None)
    if status is not None:
        status.after_launch()
    results = []
    for i in range(count):
        cache = cache_factory() if cache_factory is not None else RequestCache()
        a, b = int(out_offset[i]), int(out_offset[i]) + sizes[i]
        for layer_index in range(len(packed.layers)):
            cache.update(out_k[layer_index][:, a:b].unsqueeze(0),
                         out_v[layer_index][:, a:b].unsqueeze(0), layer_index)
        results.append(cache)
    return tuple(results)
