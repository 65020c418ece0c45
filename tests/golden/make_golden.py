"""Writes the committed golden vectors of this directory.

  reference_fixtures.json  integer fixtures transcribed from the reference's
                           own tests (file:line cited per entry); they are
                           data, not code, and pin the oracle's packing,
                           commit and sampling-law restatements.
  sampler_tiny.npz         seeded sampler problem (vocab 4096, 6 requests)
                           with the oracle's outputs; pins the oracle across
                           edits and is replayed on the GPU.

Run from the repository root: python -m tests.golden.make_golden
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

REFERENCE_FIXTURES = {
    "_source": "code/natural/tests/gbv_paper/ in the reference snapshot",
    "packed_mask_request_local": {
        "cite": "test_continuous_tree_block_decode.py:171-192",
        "parents": [-1, 0, 0, 1, 3],
        "block_rows": 4,
        "cache_lengths": [7, 5],
        "expect_shape": [8, 20],
        "finite": [[0, 4, 0, 7], [4, 8, 7, 12]],
        "neg_inf": [[0, 4, 7, 12], [0, 4, 16, 20], [4, 8, 0, 7], [4, 8, 12, 16]],
    },
    "padded_mask_visibility": {
        "cite": "test_continuous_tree_block_decode.py:133-153",
        "parents": [-1, 0, 0, 1, 3],
        "visibility_4x4": [[1, 0, 0, 0], [1, 1, 0, 0], [1, 0, 1, 0], [1, 1, 0, 1]],
    },
    "continuation_positions": {
        "cite": "test_continuous_tree_block_decode.py:156-168",
        "tree_parents": [-1, 0, 1, 2, 3],
        "tree_depths": [0, 1, 2, 3, 4],
        "block_root": 2,
        "row_cap": 3,
        "round_prefix_len": 7,
        "positions": [9, 10, 11],
    },
    "bulk_split": {
        "cite": "test_continuous_tree_block_decode.py:195-215",
        "packed_keys": list(range(10)),
        "cache_offsets": [0, 2],
        "old_lengths": [2, 3],
        "packed_old_length": 5,
        "query_offsets": [0, 3],
        "keep_query_rows": [[0, 2], [1]],
        "keys": [[0, 1, 5, 7], [2, 3, 4, 9]],
        "values": [[0, -1, -5, -7], [-2, -3, -4, -9]],
    },
    "persistent_append": {
        "cite": "test_continuous_tree_block_decode.py:218-245",
        "prefixes": [[1, 2], [3, 4, 5]],
        "capacity": 8,
        "packed_keys": list(range(10)),
        "packed_old_length": 5,
        "query_offsets": [0, 3],
        "keep_query_rows": [[0, 2], [1]],
        "lengths": [4, 4],
        "keys": [[1, 2, 5, 7], [3, 4, 5, 9]],
        "values": [[-1, -2, -5, -7], [-3, -4, -5, -9]],
    },
    "pack_order": {
        "cite": "test_continuous_tree_block_decode.py:248-267",
        "prefixes": [[1, 2], [3, 4, 5]],
        "order": [1, 0],
        "lengths": [3, 2],
        "offsets": [0, 3],
        "total": 5,
        "keys": [3, 4, 5, 1, 2],
    },
    "capacity_exhausted": {
        "cite": "test_audited_global_tree_matrix.py:67-84",
        "prefix_length": 162,
        "keep_rows": 16,
        "small_capacity": 177,
        "fixed_capacity": 211,
        "fixed_length_after": 178,
    },
    "exit_law": {
        "cite": "test_audited_global_tree_matrix.py:48-64",
        "parents": [-1, 0, 0, 1],
        "tokens": [0, 1, 1],
        "probabilities": [[0.6, 0.4], [0.25, 0.75], [0.9, 0.1], [0.3, 0.7]],
        "law": [[[0, 0], 0.15], [[0, 1, 0], 0.135], [[0, 1, 1], 0.315],
                [[1, 0], 0.36], [[1, 1], 0.04]],
    },
    "greedy_walk": {
        "cite": "test_continuous_tree_block_decode.py:49-72",
        "parents": [-1, 0, 0, 1],
        "tokens": [4, 5, 6],
        "argmax": [4, 6, 0, 7],
        "nodes": [1, 3],
        "accepted": [4, 6],
        "bonus": 7,
    },
}


def write_reference_fixtures() -> Path:
    path = HERE / "reference_fixtures.json"
    path.write_text(json.dumps(REFERENCE_FIXTURES, indent=1, sort_keys=True) + "\n")
    return path


def write_sampler_tiny() -> Path:
    import sys
    sys.path.insert(0, str(HERE.parents[1]))
    from oracle import oracle
    from tests.sampler_cases import tree_problem
    case = tree_problem(2024, num_requests=6, nodes=[16, 1, 9, 16, 3, 12], vocab=4096)
    nodes, length, bonus, m, z = oracle.tree_sample(
        case["logits"], case["row_offset"], case["parent"], case["token"],
        case["uniforms"], case["max_depth"])
    path = HERE / "sampler_tiny.npz"
    np.savez_compressed(
        path, logits=case["logits"], row_offset=case["row_offset"], parent=case["parent"],
        token=case["token"], uniforms=case["uniforms"],
        max_depth=np.int32(case["max_depth"]), accept_nodes=nodes, accept_len=length,
        bonus=bonus, row_max=m, row_sum=z)
    return path


if __name__ == "__main__":
    print(write_reference_fixtures())
    print(write_sampler_tiny())
