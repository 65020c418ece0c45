"""Seeded sampler problems shared by the CPU and GPU sampler tests."""
from __future__ import annotations

import numpy as np

from specgrove_amd import workloads as W


def tree_problem(seed: int, num_requests: int, nodes, vocab: int, *, child_boost: float = 6.0,
                 logit_std: float = 3.0, random_trees: bool = True, extreme_uniforms=False,
                 trees=None):
    """Logits with each child token boosted in its parent's row (so routes accept).

    ``nodes`` is an int or a per-request list; ``trees`` (parent lists) replaces
    the generated trees when given.  Returns a dict of numpy arrays: logits
    [R, V] f32, row_offset, parent, token (i32), uniforms [n, U] f32,
    max_depth, parents/tokens lists.
    """
    rng = np.random.default_rng(seed)
    if trees is not None:
        sizes = [len(p) for p in trees]
    else:
        sizes = [nodes] * num_requests if np.isscalar(nodes) else list(nodes)
    parents, tokens = [], []
    for k, size in enumerate(sizes):
        if trees is not None:
            p = list(trees[k])
        else:
            p = (W.random_parent_tree(size, rng, max_depth=8) if random_trees
                 else W.canonical_tree(size, rng))
        parents.append(p)
        tokens.append(W.random_tokens(p, vocab, rng))
    rows = sum(sizes)
    logits = (rng.standard_normal((rows, vocab)) * logit_std).astype(np.float32)
    offset = 0
    for p, t in zip(parents, tokens):
        for k in range(1, len(p)):
            logits[offset + p[k], t[k - 1]] += np.float32(child_boost)
        offset += len(p)
    max_depth = max(max(W.depths_of(p)) for p in parents)
    stride = 2 * (max_depth + 1)
    uniforms = rng.random((len(sizes), stride), dtype=np.float32)
    if extreme_uniforms:
        uniforms[0::3] = 0.0
        uniforms[1::3] = np.float32(1.0 - 2.0 ** -24)
    parent = np.concatenate([np.asarray(p, np.int32) for p in parents])
    token = np.concatenate([np.asarray([0] + list(t), np.int32) for t in tokens])
    row_offset = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    return dict(logits=logits, row_offset=row_offset, parent=parent.astype(np.int32),
                token=token.astype(np.int32), uniforms=uniforms, max_depth=max_depth,
                parents=parents, tokens=tokens)
