"""Pins of the packing, commit and attention oracles against the reference's
own integer fixtures (transcribed in golden/reference_fixtures.json) and
against an explicit float64 loop implementation of masked attention."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from specgrove_amd import workloads as W

FX = json.loads((Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())


def test_visibility_fixture(oracle):
    fx = FX["padded_mask_visibility"]
    vis = oracle.visibility(fx["parents"])[:4, :4]
    assert vis.astype(int).tolist() == fx["visibility_4x4"]


def test_packed_mask_is_request_local(oracle):
    fx = FX["packed_mask_request_local"]
    block = fx["parents"][:fx["block_rows"]]
    mask = oracle.packed_dense_mask(fx["cache_lengths"], [block, block])
    assert list(mask.shape) == fx["expect_shape"]
    for r0, r1, c0, c1 in fx["finite"]:
        assert np.isfinite(mask[r0:r1, c0:c1]).all()
    for r0, r1, c0, c1 in fx["neg_inf"]:
        assert np.isneginf(mask[r0:r1, c0:c1]).all()


def test_continuation_positions(oracle):
    fx = FX["continuation_positions"]
    nodes = list(range(fx["block_root"], fx["block_root"] + fx["row_cap"]))
    depths = [fx["tree_depths"][k] for k in nodes]
    _, positions = oracle.packed_ids_positions([0], [[0] * (len(nodes) - 1)], [depths],
                                               [fx["round_prefix_len"]])
    assert positions.tolist() == fx["positions"]


def test_bulk_split_fixture(oracle):
    """oracle.kv_split reproduces the reference's bulk split fixture exactly
    (keys and values of both requests)."""
    fx = FX["bulk_split"]
    packed = np.asarray(fx["packed_keys"], np.float64)
    P = fx["packed_old_length"]
    prefix = packed[:P].reshape(1, 1, P, 1)
    tree = packed[P:].reshape(1, -1, 1, 1)
    row_offset = fx["query_offsets"] + [tree.shape[1]]
    out = oracle.kv_split(prefix, -prefix, tree, -tree, fx["cache_offsets"],
                          fx["old_lengths"], row_offset, fx["keep_query_rows"])
    for i, (keys, values) in enumerate(out):
        assert keys.reshape(-1).tolist() == fx["keys"][i]
        assert values.reshape(-1).tolist() == fx["values"][i]


def test_bulk_split_fixture_via_commit(oracle):
    """Old prefix rows + kept query rows == the reference's split fixture."""
    fx = FX["bulk_split"]
    packed = np.asarray(fx["packed_keys"], np.float64)
    n = len(fx["old_lengths"])
    cap = 8
    arena = np.zeros((1, 1, n * cap, 1))
    lengths = np.zeros(n, np.int64)
    for i, (off, length) in enumerate(zip(fx["cache_offsets"], fx["old_lengths"])):
        arena[0, 0, i * cap:i * cap + length, 0] = packed[off:off + length]
        lengths[i] = length
    tree = packed[fx["packed_old_length"]:].reshape(1, -1, 1, 1)
    row_offset = fx["query_offsets"] + [tree.shape[1]]
    arena_v = -arena
    oracle.kv_commit(arena, arena_v, lengths, cap, range(n), tree, -tree, row_offset,
                     fx["keep_query_rows"])
    for i in range(n):
        got = arena[0, 0, i * cap:i * cap + lengths[i], 0].tolist()
        assert got == fx["keys"][i]
        assert arena_v[0, 0, i * cap:i * cap + lengths[i], 0].tolist() == fx["values"][i]


def test_persistent_append_fixture(oracle):
    fx = FX["persistent_append"]
    cap = fx["capacity"]
    n = len(fx["prefixes"])
    arena = np.zeros((1, 1, n * cap, 1))
    lengths = np.zeros(n, np.int64)
    for i, prefix in enumerate(fx["prefixes"]):
        arena[0, 0, i * cap:i * cap + len(prefix), 0] = prefix
        lengths[i] = len(prefix)
    packed = np.asarray(fx["packed_keys"], np.float64)
    tree = packed[fx["packed_old_length"]:].reshape(1, -1, 1, 1)
    arena_v = -arena
    oracle.kv_commit(arena, arena_v, lengths, cap, range(n), tree, -tree,
                     fx["query_offsets"] + [tree.shape[1]], fx["keep_query_rows"])
    assert lengths.tolist() == fx["lengths"]
    for i in range(n):
        assert arena[0, 0, i * cap:i * cap + lengths[i], 0].tolist() == fx["keys"][i]
        assert arena_v[0, 0, i * cap:i * cap + lengths[i], 0].tolist() == fx["values"][i]


def test_capacity_fixture(oracle):
    fx = FX["capacity_exhausted"]
    keep = [list(range(fx["keep_rows"]))]
    tree = np.arange(fx["keep_rows"], dtype=np.float64).reshape(1, -1, 1, 1)
    for cap, ok in ((fx["small_capacity"], False), (fx["fixed_capacity"], True)):
        arena = np.zeros((1, 1, cap, 1))
        lengths = np.asarray([fx["prefix_length"]])
        if ok:
            oracle.kv_commit(arena, arena.copy(), lengths, cap, [0], tree, tree,
                             [0, fx["keep_rows"]], keep)
            assert lengths[0] == fx["fixed_length_after"]
        else:
            with pytest.raises(RuntimeError, match="capacity exhausted"):
                oracle.kv_commit(arena, arena.copy(), lengths, cap, [0], tree, tree,
                                 [0, fx["keep_rows"]], keep)


def _tiny_inputs(seed, **kw):
    wl = W.tiny_attention_workload(seed=seed, **kw)
    q, kc, vc, kt, vt = wl.make_tensors("cpu", seed)
    ks = [kc[:, int(s):int(s) + int(L)] for s, L in zip(wl.prefix_start, wl.prefix_len)]
    vs = [vc[:, int(s):int(s) + int(L)] for s, L in zip(wl.prefix_start, wl.prefix_len)]
    return wl, q, ks, vs, kt, vt


def test_dense_attention_matches_float64_loops(oracle):
    wl, q, ks, vs, kt, vt = _tiny_inputs(4, num_requests=3, rows=6, prefix_lo=3, prefix_hi=9)
    dense = oracle.attention_dense(q, ks, vs, kt, vt, wl.parents).numpy()
    brute = oracle.attention_bruteforce(q.float().numpy(), [k.float().numpy() for k in ks],
                                        [v.float().numpy() for v in vs], kt.float().numpy(),
                                        vt.float().numpy(), wl.row_offset, wl.parents)
    assert np.max(np.abs(dense - brute)) < 1e-5


def test_per_request_mode_equals_dense_mode(oracle):
    wl, q, ks, vs, kt, vt = _tiny_inputs(7)
    dense = oracle.attention_dense(q, ks, vs, kt, vt, wl.parents)
    per = oracle.attention_per_request(q, ks, vs, kt, vt, wl.row_offset, wl.parents)
    stacked = torch.cat([per[i] for i in range(wl.num_requests)])
    assert torch.allclose(dense, stacked, atol=1e-5)


def test_dense_oracle_request_isolation(oracle):
    wl, q, ks, vs, kt, vt = _tiny_inputs(8)
    base = oracle.attention_dense(q, ks, vs, kt, vt, wl.parents)
    ks2 = list(ks)
    ks2[2] = torch.full_like(ks[2], 3.0)
    kt2 = kt.clone()
    r0, r1 = int(wl.row_offset[2]), int(wl.row_offset[3])
    kt2[r0:r1] = -4.0
    poisoned = oracle.attention_dense(q, ks2, vs, kt2, vt, wl.parents)
    mask = torch.ones(wl.total_rows, dtype=torch.bool)
    mask[r0:r1] = False
    assert torch.equal(base[mask], poisoned[mask])
    assert not torch.equal(base[~mask], poisoned[~mask])
