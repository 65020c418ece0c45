"""Packed-row builder and the transformers attention plug of the packed
verification wave.

The reference builds, per wave (continuous_tree_block_decode.py:500-546):

* ``ids`` = [root] + tree tokens of every chosen request, packed;
* ``positions`` = ``round_prefix_len + depth``;
* a dense additive mask ``[1, 1, R, P + R]`` (own prefix and own tree
  ancestors visible);

and runs the Target model's SDPA over all ``P + R`` keys of a packed cache.
``pack_block_inputs`` produces the same ``ids`` / ``positions`` /
``query_offsets`` but replaces the dense mask by a ``PackedTreeMask``: row
offsets, request-local parent indices, the requests' arena slots and prefix
lengths, and the attention work plan -- O(R + n) integers instead of
O(R * (P + R)).

Passed as ``attention_mask={"full_attention": mask}``, transformers' decoder
forwards the object untouched to every layer's attention function, which
``register()`` installs as ``attn_implementation="specgrove_hip"``
(transformers' ``AttentionInterface``, the plug point of engine.py:278-281).
The function then calls the HIP kernel with the layer's arena as the prefix
K/V and the wave's new rows (returned by ``TreeVerifyCache.update``) as the
tree K/V.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from . import ops

IMPLEMENTATION = "specgrove_hip"


@dataclass
class PackedTreeMask:
    """Compact replacement of the packed dense mask."""
    pool: object                    # the prefixes: a PersistentRequestCachePool (arena per
                                    # layer) or a PackedPrefix (non-persistent wave); both
                                    # expose key_storage[l] / value_storage[l] [Hkv, T, D]
    row_offset: torch.Tensor        # [n+1] i32, device
    parent: torch.Tensor            # [R] i32, request-local parents, -1 for roots
    prefix_start: torch.Tensor      # [n] i64, slot * capacity
    prefix_len: torch.Tensor        # [n] i32
    row_offset_host: np.ndarray
    prefix_len_host: np.ndarray
    plans: dict = field(default_factory=dict)

    @property
    def num_rows(self) -> int:
        return int(self.row_offset_host[-1])

    def plan(self, num_q_heads: int, num_kv_heads: int, head_dim: int) -> ops.AttnPlan:
        """Work plan of this wave for a head configuration (built once and
        shared by every layer)."""
        key = (num_q_heads, num_kv_heads, head_dim)
        if key not in self.plans:
            self.plans[key] = ops.plan_attention(
                self.row_offset_host, self.prefix_len_host, num_q_heads, num_kv_heads,
                head_dim).to(self.row_offset.device)
        return self.plans[key]


def build_tree_mask(pool, caches: Sequence, parents_list: Sequence[Sequence[int]],
                    device, prefix_start: Sequence[int] | None = None,
                    prefix_len: Sequence[int] | None = None) -> PackedTreeMask:
    """Compact mask of one wave: request i uses arena slot ``caches[i].slot``
    with its current length as prefix (or, for a non-persistent wave, the
    given ``prefix_start`` / ``prefix_len`` in ``pool``, a PackedPrefix) and
    the tree ``parents_list[i]`` (local parent indices, root -1, parents
    before children)."""
    rows = [len(p) for p in parents_list]
    row_offset = np.zeros(len(rows) + 1, np.int32)
    np.cumsum(rows, out=row_offset[1:])
    parent = np.concatenate([np.asarray(p, np.int32) for p in parents_list]) if rows else \
        np.zeros(0, np.int32)
    for p in parents_list:
        if len(p) == 0 or p[0] != -1 or any(not 0 <= q < k for k, q in enumerate(p[1:], 1)):
            raise ValueError("Tree parents must precede their children")
    if prefix_start is None:
        prefix_len = np.asarray([pool.lengths[c.slot] for c in caches], np.int32)
        prefix_start = np.asarray([c.slot * pool.capacity for c in caches], np.int64)
    else:
        prefix_len = np.asarray(prefix_len, np.int32)
        prefix_start = np.asarray(prefix_start, np.int64)
    dev = torch.device(device)
    # One host-to-device copy for the whole wave: prefix starts (int64), then
    # row offsets, prefix lengths and parents as int32 pairs.
    n = len(rows)
    words32 = np.concatenate([row_offset, prefix_len, parent]).astype(np.int32)
    if words32.size % 2:
        words32 = np.concatenate([words32, np.zeros(1, np.int32)])
    host = np.concatenate([prefix_start.astype(np.int64), words32.view(np.int64)])
    meta = torch.from_numpy(host).to(dev)
    meta32 = meta[n:].view(torch.int32)
    return PackedTreeMask(
        pool=pool,
        row_offset=meta32[:n + 1],
        parent=meta32[2 * n + 1:2 * n + 1 + parent.size],
        prefix_start=meta[:n],
        prefix_len=meta32[n + 1:2 * n + 1],
        row_offset_host=row_offset,
        prefix_len_host=prefix_len,
    )


def pack_block_inputs(states, blocks, cache_lengths: Sequence[int],
                      cache_offsets: Sequence[int], packed_cache_length: int, dtype, device):
    """Drop-in for ``_packed_block_inputs`` (reference :500-546).

    Same ``ids`` [1, R], ``positions`` [1, R] and ``query_offsets``; the
    third result is ``{"full_attention": PackedTreeMask}`` instead of the
    dense ``[1, 1, R, P + R]`` mask.  ``states[i].target_cache`` must be a
    view of one persistent pool, or the request caches just packed by
    ``pack_cache_sequence`` (non-persistent wave, prefixes at
    ``cache_offsets``); ``packed_cache_length`` and ``dtype`` are accepted for
    signature compatibility.
    """
    block_rows = tuple(len(block.nodes) for block in blocks)
    query_offsets = []
    total = 0
    for rows in block_rows:
        query_offsets.append(total)
        total += rows
    ids = np.empty(total, np.int64)
    positions = np.empty(total, np.int64)
    for state, block, old_length, q0 in zip(states, blocks, cache_lengths, query_offsets):
        rows = len(block.nodes)
        root = (state.generated[-1] if state.block_root == 0
                else state.tree.tokens[state.block_root - 1])
        ids[q0:q0 + rows] = [root] + list(block.tokens)
        positions[q0:q0 + rows] = np.asarray(block.depths, np.int64) + state.round_prefix_len
    caches = [state.target_cache for state in states]
    parents_list = [list(block.parents) for block in blocks]
    if hasattr(caches[0], "pool") and hasattr(caches[0], "slot"):
        pool = caches[0].pool
        if any(getattr(c, "pool", None) is not pool for c in caches):
            raise ValueError("Packed tree verification needs caches of one persistent pool")
        if any(pool.lengths[c.slot] != int(L) for c, L in zip(caches, cache_lengths)):
            raise ValueError("Cache lengths disagree with the persistent pool")
        mask = build_tree_mask(pool, caches, parents_list, device)
    else:
        # Non-persistent wave: the prefixes were packed by pack_cache_sequence.
        from .cache import packed_wave_of
        wave = packed_wave_of(caches[0])
        if wave is None or any(packed_wave_of(c) is not wave for c in caches) \
                or tuple(wave.caches) != tuple(caches):
            raise ValueError("Request caches were not packed together by pack_cache_sequence")
        if (tuple(int(v) for v in cache_lengths) != wave.prefix_lengths
                or tuple(int(v) for v in cache_offsets) != wave.prefix_starts):
            raise ValueError("Cache lengths disagree with the packed wave")
        mask = build_tree_mask(wave.prefix_source, caches, parents_list, device,
                               prefix_start=wave.prefix_starts, prefix_len=wave.prefix_lengths)
    dev = torch.device(device)
    return (torch.from_numpy(ids).to(dev).unsqueeze(0),
            torch.from_numpy(positions).to(dev).unsqueeze(0),
            {"full_attention": mask}, tuple(query_offsets))


def tree_attention_forward(module, query: torch.Tensor, key: torch.Tensor,
                           value: torch.Tensor, attention_mask, scaling: float | None = None,
                           dropout: float = 0.0, **kwargs):
    """transformers attention function (``ALL_ATTENTION_FUNCTIONS`` signature).

    query [1, Hq, R, D]; key/value [1, Hkv, R, D] are the wave's new rows
    (``TreeVerifyCache.update`` returns them); ``attention_mask`` is the
    wave's PackedTreeMask.  Returns ([1, R, Hq, D], None).
    """
    if not isinstance(attention_mask, PackedTreeMask):
        raise ValueError("specgrove_hip attention needs a PackedTreeMask "
                         "(attention_mask={'full_attention': mask})")
    if dropout != 0.0:
        raise ValueError("specgrove_hip attention does not implement dropout")
    if kwargs.get("sliding_window") is not None:
        raise ValueError("specgrove_hip attention does not implement sliding windows")
    mask = attention_mask
    if query.shape[0] != 1 or key.shape[0] != 1:
        raise ValueError("Packed verification runs one packed sequence")
    hq, rows, dim = query.shape[1], query.shape[2], query.shape[3]
    hkv = key.shape[1]
    if rows != mask.num_rows or key.shape[2] != rows:
        raise ValueError("Packed rows disagree with the tree mask")
    layer = module.layer_idx
    k_cache = mask.pool.key_storage[layer]
    v_cache = mask.pool.value_storage[layer]
    plan = mask.plan(hq, hkv, dim)
    out = torch.empty((1, rows, hq, dim), dtype=query.dtype, device=query.device)
    ops.tree_attention(query[0].transpose(0, 1), k_cache, v_cache, key[0].transpose(0, 1),
                       value[0].transpose(0, 1), mask.row_offset, mask.prefix_start,
                       mask.prefix_len, mask.parent, plan, out=out[0],
                       scale=scaling if scaling is not None else dim ** -0.5)
    return out, None


def register() -> str:
    """Install the attention function under ``attn_implementation="specgrove_hip"``."""
    from transformers import AttentionInterface
    AttentionInterface.register(IMPLEMENTATION, tree_attention_forward)
    return IMPLEMENTATION
