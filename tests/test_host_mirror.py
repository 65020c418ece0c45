"""Host-side drop-in layer (packed-row builder, persistent pool, verifier,
transformers plug) checked on the CPU: argument validation and error classes
follow the reference wrappers, the compact mask encodes exactly the
reference's dense packed mask, and the transformers decoder routes every
layer to the plug.  No kernel runs here (the GPU tests run them)."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from specgrove_amd import attention, verify
from specgrove_amd.cache import (PersistentRequestCachePool, TreeVerifyCache,
                                 pack_cache_sequence)
from specgrove_amd import workloads as W


class _Layer:
    def __init__(self, keys, values):
        self.keys, self.values = keys, values


class _Cache:
    """Minimal per-request cache: layers[l].keys/values [1, Hkv, L, D]."""

    def __init__(self, layers):
        self.layers = layers

    def get_seq_length(self):
        return int(self.layers[0].keys.shape[-2])


def _pool(lengths, layers=2, hkv=2, dim=8, capacity=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    caches = [_Cache([_Layer(torch.randn(1, hkv, L, dim, generator=g),
                             torch.randn(1, hkv, L, dim, generator=g)) for _ in range(layers)])
              for L in lengths]
    return PersistentRequestCachePool(caches, capacity), caches


def _states_blocks(pool, trees, rng):
    states, blocks = [], []
    for i, parents in enumerate(trees):
        depths = W.depths_of(parents)
        tokens = W.random_tokens(parents, 4096, rng)
        states.append(SimpleNamespace(generated=[int(rng.integers(0, 4096))], block_root=0,
                                      tree=None, round_prefix_len=pool.lengths[i] + 3,
                                      target_cache=pool.caches[i]))
        blocks.append(SimpleNamespace(nodes=list(range(len(parents))), parents=parents,
                                      tokens=tokens, depths=depths))
    return states, blocks


def test_pool_copies_prefixes_into_slots():
    pool, caches = _pool([5, 9, 3])
    for slot, cache in enumerate(caches):
        for layer in range(2):
            view = pool.caches[slot].layers[layer].keys
            assert torch.equal(view, cache.layers[layer].keys)
    assert pool.lengths == [5, 9, 3]
    with pytest.raises(ValueError):
        PersistentRequestCachePool(caches, 4)  # capacity below the prefix
    with pytest.raises(ValueError):
        PersistentRequestCachePool([], 8)


def test_packed_inputs_match_the_reference_dense_mask(oracle):
    rng = np.random.default_rng(7)
    pool, _ = _pool([5, 9, 3, 12])
    trees = [W.random_parent_tree(n, rng) for n in (4, 1, 7, 3)]
    states, blocks = _states_blocks(pool, trees, rng)
    lengths = [pool.lengths[i] for i in range(4)]
    offsets = list(np.cumsum([0] + lengths[:-1]))
    ids, positions, mask, qoff = attention.pack_block_inputs(
        states, blocks, lengths, offsets, sum(lengths), torch.bfloat16, "cpu")
    ref_ids, ref_pos = oracle.packed_ids_positions(
        [s.generated[-1] for s in states], [b.tokens for b in blocks],
        [b.depths for b in blocks], [s.round_prefix_len for s in states])
    assert ids[0].tolist() == list(ref_ids) and positions[0].tolist() == list(ref_pos)
    assert list(qoff) == [0, 4, 5, 12]
    m = mask["full_attention"]
    # Rebuild the dense mask from the compact one and compare with the oracle's.
    R, P = m.num_rows, sum(lengths)
    dense = np.full((R, P + R), -np.inf)
    ro, par = m.row_offset.numpy(), m.parent.numpy()
    for i in range(4):
        vis = oracle.visibility(par[ro[i]:ro[i + 1]])
        for k in range(ro[i + 1] - ro[i]):
            dense[ro[i] + k, offsets[i]:offsets[i] + m.prefix_len[i].item()] = 0
            dense[ro[i] + k, P + ro[i]:P + ro[i + 1]][vis[k]] = 0
    assert np.array_equal(dense, oracle.packed_dense_mask(lengths, [b.parents for b in blocks]))
    assert m.prefix_start.tolist() == [i * pool.capacity for i in range(4)]


def test_packed_inputs_reject_bad_trees_and_foreign_pools():
    rng = np.random.default_rng(1)
    pool, _ = _pool([5, 6])
    states, blocks = _states_blocks(pool, [[-1, 0], [-1, 0, 1]], rng)
    blocks[1].parents = [-1, 2, 0]
    with pytest.raises(ValueError):
        attention.pack_block_inputs(states, blocks, [5, 6], [0, 5], 11, torch.bfloat16, "cpu")
    other, _ = _pool([5, 6])
    states[1].target_cache = other.caches[1]
    blocks[1].parents = [-1, 0, 1]
    with pytest.raises(ValueError):
        attention.pack_block_inputs(states, blocks, [5, 6], [0, 5], 11, torch.bfloat16, "cpu")


def test_tree_cache_records_new_rows_and_commit_checks():
    pool, _ = _pool([5, 60])
    packed, lengths, offsets, total = pack_cache_sequence(pool.caches)
    assert lengths == (5, 60) and offsets == (0, 5) and total == 65
    rows = torch.randn(1, 2, 6, 8).transpose(1, 2).transpose(1, 2)  # a strided view
    k, v = packed.update(rows, rows.clone(), 0)
    assert k.is_contiguous() and packed.num_rows == 6
    packed.update(rows, rows, 1)
    with pytest.raises(ValueError):
        packed.update(rows, rows, 3)
    # metadata mismatches -> ValueError, capacity -> RuntimeError; nothing launched
    with pytest.raises(ValueError):
        pool.append_packed_sequence(packed, pool.caches, 64, [0, 3], [[0], [0]], "cpu")
    with pytest.raises(ValueError):
        pool.append_packed_sequence(packed, pool.caches, 65, [0, 3], [[0, 3], [0]], "cpu")
    with pytest.raises(ValueError):
        pool.append_packed_sequence(packed, pool.caches[:1], 65, [0, 3], [[0]], "cpu")
    with pytest.raises(RuntimeError, match="capacity exhausted"):
        pool.append_packed_sequence(packed, pool.caches, 65, [0, 3], [[0], [0, 1, 2, 3, 4]],
                                    "cpu")
    assert pool.lengths == [5, 60]


def test_verifier_validation_follows_the_reference():
    x = torch.zeros(3, 16)
    gens = [torch.Generator()]
    with pytest.raises(ValueError):  # host tensor
        verify.tree_verify_hip_rejection_batched([[-1, 0, 0]], [[1, 2]], x, generators=gens)
    with pytest.raises(ValueError):  # parent after child
        verify._topology([-1, 2, 0], [1, 2])
    with pytest.raises(ValueError):  # repeated child token
        verify._topology([-1, 0, 0], [1, 1])
    with pytest.raises(ValueError):  # token count
        verify._topology([-1, 0], [1, 2])
    assert verify._topology([-1, 0, 1, 0], [3, 4, 5])[2] == 2
    assert verify.VERIFIER_NAME == "hip_tree_rejection"


def test_transformers_routes_every_layer_to_the_plug():
    """A Qwen3 decoder with attn_implementation='specgrove_hip' hands the
    compact mask and the new rows to the plug; on host tensors the plug
    refuses loudly (no CPU fallback)."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(hidden_size=64, intermediate_size=128, num_attention_heads=4,
                                   num_key_value_heads=2, head_dim=64, num_hidden_layers=2,
                                   vocab_size=256, rope_theta=1e6, max_position_embeddings=256)
    torch.manual_seed(0)
    model = transformers.Qwen3ForCausalLM(cfg).eval()
    attention.register()
    model.config._attn_implementation = attention.IMPLEMENTATION
    pool, _ = _pool([5, 7], layers=2, hkv=2, dim=64)
    rng = np.random.default_rng(3)
    states, blocks = _states_blocks(pool, [[-1, 0, 0], [-1, 0]], rng)
    ids, positions, mask, _ = attention.pack_block_inputs(states, blocks, [5, 7], [0, 5], 12,
                                                          torch.float32, "cpu")
    ids = ids % 256
    packed, *_ = pack_cache_sequence(pool.caches)
    seen = []
    original = attention.tree_attention_forward

    def spy(module, q, k, v, m, **kw):
        seen.append((module.layer_idx, tuple(q.shape), tuple(k.shape), m is mask["full_attention"]))
        return original(module, q, k, v, m, **kw)

    from transformers import AttentionInterface
    AttentionInterface.register(attention.IMPLEMENTATION, spy)
    try:
        with pytest.raises(ValueError, match="HIP device"):
            model.model(input_ids=ids, position_ids=positions, attention_mask=mask,
                        past_key_values=packed, use_cache=True)
    finally:
        attention.register()
    assert seen == [(0, (1, 4, 5, 64), (1, 2, 5, 64), True)]
    assert len(packed.layers) == 1 and packed.layers[0].keys.shape == (1, 2, 5, 64)


def test_non_persistent_pack_concatenates_in_requested_order():
    """pack_cache_sequence on plain request caches builds one packed prefix
    per layer in the requested order (the reference's pack-order fixture,
    test_continuous_tree_block_decode.py:248-267) and pack_block_inputs finds
    it through the request caches."""
    from specgrove_amd.cache import PackedPrefix
    first = torch.tensor([1, 2], dtype=torch.float32).reshape(1, 1, 2, 1)
    second = torch.tensor([3, 4, 5], dtype=torch.float32).reshape(1, 1, 3, 1)
    caches = [_Cache([_Layer(first, -first)]), _Cache([_Layer(second, -second)])]
    packed, lengths, offsets, total = pack_cache_sequence(tuple(reversed(caches)))
    assert lengths == (3, 2) and offsets == (0, 3) and total == 5
    assert isinstance(packed.prefix_source, PackedPrefix) and packed.pool is None
    assert packed.prefix_source.key_storage[0].flatten().tolist() == [3, 4, 5, 1, 2]
    assert packed.prefix_source.value_storage[0].flatten().tolist() == [-3, -4, -5, -1, -2]
    states = [SimpleNamespace(generated=[7], block_root=0, tree=None, round_prefix_len=L,
                              target_cache=c) for c, L in zip(reversed(caches), (3, 2))]
    blocks = [SimpleNamespace(nodes=[0, 1], parents=[-1, 0], tokens=[9], depths=[0, 1])] * 2
    ids, positions, mask, qoff = attention.pack_block_inputs(
        states, blocks, lengths, offsets, total, torch.float32, "cpu")
    assert mask["full_attention"].prefix_start.tolist() == [0, 3]
    assert mask["full_attention"].prefix_len.tolist() == [3, 2]
    with pytest.raises(ValueError, match="packed together"):
        attention.pack_block_inputs(states[:1], blocks[:1], lengths[:1], offsets[:1], 3,
                                    torch.float32, "cpu")


def test_non_persistent_split_validates_like_the_reference():
    from specgrove_amd.cache import split_compacted_sequence_caches
    first = torch.zeros((1, 1, 2, 8))
    second = torch.zeros((1, 1, 3, 8))
    caches = [_Cache([_Layer(first, first)]), _Cache([_Layer(second, second)])]
    packed, lengths, offsets, total = pack_cache_sequence(caches)
    packed.update(torch.zeros((1, 1, 5, 8)), torch.zeros((1, 1, 5, 8)), 0)
    for args in (((0, 2), (2, 3), 5, (0, 3), ((0, 2),)),          # fewer keep lists
                 ((0, 2), (2, 3), 6, (0, 3), ((0, 2), (1,))),     # wrong packed length
                 ((0, 1), (2, 3), 5, (0, 3), ((0, 2), (1,))),     # wrong offsets
                 ((0, 2), (2, 3), 5, (0, 3), ((0, 3), (1,)))):    # row outside request 0
        with pytest.raises(ValueError, match="split metadata disagree"):
            split_compacted_sequence_caches(packed, None, args[0], args[1], args[2], args[3],
                                            args[4], "cpu")
