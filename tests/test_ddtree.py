"""DDTree proposal trees and the occupancy controls on the CPU.

Pins for ``ddtree.probability_tree`` (the reference's tree.py:148-212):

* the reference tests' fixtures (code/natural/tests/gbv_paper/
  test_continuous_tree_block_decode.py, T_CTBD below): the two-depth tree of
  :390-399 and the canonical-prefix property of :402-410, with the same
  seeded draft;
* brute force without rewards: the tree's nodes are the ``budget``
  highest-scoring token prefixes among all prefixes whose token at each depth
  lies in that depth's top ``cap`` tokens, in decreasing score;
* with rewards (which break that ordering), an explicit best-first search
  over the whole frontier -- every child of every chosen node -- instead of
  the builder's lazy sibling offers.

Random drafts are continuous, so no two scores tie.
"""
import itertools
import math
import random
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from specgrove_amd import ddtree
from specgrove_amd import scheduler as S


def _paths(tree):
    """Token path of every node (root = ())."""
    paths = [()]
    for node in range(1, len(tree.parents)):
        paths.append(paths[tree.parents[node]] + (tree.tokens[node - 1],))
    return paths


def _draft(rng, length, vocab, peak=0.0):
    logits = rng.standard_normal((length, vocab)) * 1.5
    if peak:
        logits[:, 0] += peak
    q = np.exp(logits - logits.max(1, keepdims=True))
    return torch.from_numpy(q / q.sum(1, keepdims=True))


def _ranked(q, caps):
    """Per depth, the top ``cap`` (log probability, token) pairs, descending."""
    out = []
    for d, cap in enumerate(caps):
        order = np.argsort(-q[d].numpy(), kind="stable")[:cap]
        out.append([(math.log(float(q[d, t])), int(t)) for t in order])
    return out


def test_two_depth_fixture():
    # T_CTBD:390-399: q = [[.75, .25], [.5, .5]], budget 2.
    q = torch.tensor([[0.75, 0.25], [0.50, 0.50]], dtype=torch.float64)
    tree = ddtree.probability_tree(q, 2)
    # The .75 token, then its child beats the .25 sibling (.375 > .25).
    assert tree.parents == [-1, 0, 1] and tree.depths == [0, 1, 2]
    assert tree.tokens[0] == 0 and tree.tokens[1] in (0, 1)
    assert tree.draft_prefix_log_masses == [0.0, math.log(0.75), math.log(0.75) + math.log(0.5)]
    assert S.draft_tree_expected_tokens(tree) == pytest.approx(1.0 + 0.75 + 0.375, abs=1e-12)


def test_canonical_budget_is_prefix_of_larger_tree():
    # T_CTBD:402-410 with the same seeded draft.
    generator = torch.Generator().manual_seed(17)
    q = torch.softmax(torch.randn((4, 32), generator=generator), -1).double()
    full = ddtree.probability_tree(q, 12)
    prefix = S.prefix_tree(full, 5)
    direct = ddtree.probability_tree(q, 5)
    assert prefix.tokens == direct.tokens
    assert prefix.parents == direct.parents
    assert prefix.depths == direct.depths
    assert prefix.draft_prefix_log_masses == direct.draft_prefix_log_masses


@pytest.mark.parametrize("seed", range(12))
def test_without_rewards_the_tree_is_the_top_prefixes(seed):
    rng = np.random.default_rng(seed)
    length, vocab = int(rng.integers(1, 5)), int(rng.integers(2, 7))
    budget = int(rng.integers(1, 30))
    caps = None
    if seed % 2:
        caps = tuple(int(rng.integers(1, vocab + 1)) for _ in range(length))
    q = _draft(rng, length, vocab)
    tree = ddtree.probability_tree(q, budget, rank_caps=caps)
    eff = [min(c, budget, vocab) for c in (caps or (vocab,) * length)]
    ranked = _ranked(q, eff)
    scored = []
    for depth in range(1, length + 1):
        for combo in itertools.product(*(ranked[d] for d in range(depth))):
            scored.append((sum(lp for lp, _ in combo), tuple(t for _, t in combo)))
    scored.sort(key=lambda x: -x[0])
    want = [p for _, p in scored[:budget]]
    got = _paths(tree)[1:]
    assert got == want
    for node, path in enumerate(_paths(tree)[1:], 1):
        assert tree.depths[node] == len(path)
        assert tree.draft_prefix_log_masses[node] == pytest.approx(
            sum(math.log(float(q[d, t])) for d, t in enumerate(path)), rel=0, abs=1e-12)


@pytest.mark.parametrize("seed", range(12))
def test_with_rewards_matches_explicit_frontier_search(seed):
    rng = np.random.default_rng(100 + seed)
    length, vocab = int(rng.integers(2, 6)), int(rng.integers(2, 8))
    budget = int(rng.integers(1, 40))
    schedule = tuple(float(v) for v in rng.normal(0.0, 1.5, length))
    caps = tuple(int(rng.integers(1, vocab + 1)) for _ in range(length))
    q = _draft(rng, length, vocab)
    tree = ddtree.probability_tree(q, budget, depth_reward_schedule=schedule, rank_caps=caps)
    ranked = _ranked(q, [min(c, budget, vocab) for c in caps])
    # nodes as (path, score); frontier = every child of a chosen node
    chosen = [((), 0.0)]
    taken = {()}
    while len(chosen) - 1 < budget:
        best = None
        for path, score in chosen:
            d = len(path)
            if d >= length:
                continue
            for lp, t in ranked[d]:
                child = path + (t,)
                if child in taken:
                    continue
                s = score + lp + schedule[d]
                if best is None or s > best[1]:
                    best = (child, s)
        if best is None:
            break
        chosen.append(best)
        taken.add(best[0])
    assert _paths(tree) == [p for p, _ in chosen]
    assert tree.draft_prefix_log_masses == pytest.approx([s for _, s in chosen], abs=1e-12)


def test_adaptive_budget():
    rng = np.random.default_rng(3)
    confident = _draft(rng, 6, 16, peak=9.0)
    unsure = _draft(rng, 6, 16)
    small = ddtree.probability_tree(confident, 20, adaptive_min_budget=6, confidence_threshold=0.9)
    big = ddtree.probability_tree(unsure, 20, adaptive_min_budget=6, confidence_threshold=0.9)
    assert len(small.tokens) == 6 and len(big.tokens) == 20
    # the smaller budget only truncates the same best-first order
    assert small.parents == ddtree.probability_tree(confident, 20).parents[:7]
    with pytest.raises(ValueError, match="confidence threshold"):
        ddtree.probability_tree(confident, 20, adaptive_min_budget=6)


def test_controls_are_validated():
    q = torch.full((3, 5), 0.2, dtype=torch.float64)
    with pytest.raises(ValueError, match="depth reward must be finite"):
        ddtree.probability_tree(q, 4, depth_reward=math.inf)
    with pytest.raises(ValueError, match="depth-reward schedule"):
        ddtree.probability_tree(q, 4, depth_reward_schedule=(0.0, 1.0))
    for caps in ((1, 2), (1, 0, 1), (1, True, 1), (1, 1.5, 1)):
        with pytest.raises(ValueError, match="rank caps"):
            ddtree.probability_tree(q, 4, rank_caps=caps)
    with pytest.raises(ValueError, match="budget"):
        ddtree.probability_tree(q, 0)
    with pytest.raises(ValueError, match="requests, depths, vocab"):
        ddtree.probability_trees(q, [3])


def test_batched_trees_equal_single_trees_and_proposer():
    rng = np.random.default_rng(9)
    q = torch.stack([_draft(rng, 5, 40) for _ in range(6)]).float()
    budgets = [3, 17, 1, 31, 8, 12]
    many = ddtree.probability_trees(q, budgets, rank_caps=(4, 4, 3, 2, 2))
    for k, b in enumerate(budgets):
        one = ddtree.probability_tree(q[k], b, rank_caps=(4, 4, 3, 2, 2))
        assert many[k] == one
        assert len(one.tokens) <= b
    # float32 drafts: logarithms taken in float32, as the reference does
    assert many[1].draft_prefix_log_masses[1] == float(torch.log(q[1, 0].max()))
    seen = []
    proposer = ddtree.DDTreeProposer(lambda states: (seen.append(len(states)), q[:len(states)])[1])
    trees = proposer.propose_many([SimpleNamespace()] * 3, [2, 4, 6])
    assert seen == [3] and [len(t.tokens) for t in trees] == [2, 4, 6]
    assert proposer.canonical
    assert not ddtree.DDTreeProposer(None, depth_reward=0.5).canonical


def test_occupancy_row_cap_fixture():
    # T_CTBD:328-335
    assert S.effective_row_cap(16, 46, 4, 16, 24, 8) == 16
    assert S.effective_row_cap(16, 46, 4, 9, 24, 8) == 16
    assert S.effective_row_cap(16, 46, 4, 8, 24, 8) == 24
    assert S.effective_row_cap(16, 46, 4, 5, 24, 8) == 24
    assert S.effective_row_cap(16, 46, 4, 4, 24, 8) == 46
    assert S.effective_row_cap(16, 46, 4, 1, 24, 8) == 46
    assert S.effective_row_cap(24, None, None, 1) == 24


def test_occupancy_tree_budget_fixtures():
    # T_CTBD:356-361
    assert S.effective_tree_budget(45, 11, 45, 4, 16) == 11
    assert S.effective_tree_budget(45, 11, 45, 4, 5) == 11
    assert S.effective_tree_budget(45, 11, 45, 4, 4) == 45
    assert S.effective_tree_budget(45, 11, 45, 4, 1) == 45
    assert S.effective_tree_budget(45, None, None, None, 16) == 45
    # T_CTBD:364-368
    assert S.adaptive_expansion_eligible(16, (4, 4), True)
    assert S.adaptive_expansion_eligible(8, (4, 4), True)
    assert not S.adaptive_expansion_eligible(4, (4, 4), True)
    assert S.adaptive_expansion_eligible(4, (4, 4), False)
    with pytest.raises(ValueError):
        S.adaptive_expansion_eligible(0, (4,), False)
    # T_CTBD:371-387
    states = [SimpleNamespace(request_id=0, generated=[0] * 40, age=0),
              SimpleNamespace(request_id=1, generated=[0] * 20, age=0),
              SimpleNamespace(request_id=2, generated=[0] * 30, age=0),
              SimpleNamespace(request_id=3, generated=[0] * 20, age=0)]
    assert S.effective_tree_budgets(states, 45, 11, 45, 4, 4, 2) == (11, 45, 11, 45)
    assert S.effective_tree_budgets(states, 45, 11, 45, 4, 5, 2) == (11, 11, 11, 11)
    assert S.effective_tree_budgets(states, 45, 11, 45, 4, 4, None) == (45, 45, 45, 45)


def test_tail_budget_ties_go_to_older_then_lower_ids():
    rng = random.Random(4)
    for _ in range(50):
        states = [SimpleNamespace(request_id=i, generated=[0] * rng.randrange(3),
                                  age=rng.randrange(3)) for i in range(6)]
        slots = rng.randrange(1, 6)
        got = S.effective_tree_budgets(states, 9, 3, 9, 8, 6, slots)
        order = sorted(range(6), key=lambda i: (len(states[i].generated), -states[i].age, i))
        assert [i for i in range(6) if got[i] == 9] == sorted(order[:slots])
