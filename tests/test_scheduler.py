"""Host scheduler (tree blocks, tiers, wave selection, tier allocation) on the
CPU.  Expected values are the reference tests' own fixtures, cited by file
and line (code/natural/tests/gbv_paper/...), plus a brute-force enumeration
of the allocator's objective written here from its specification."""
import itertools
import math
import random
from types import SimpleNamespace

import pytest

from specgrove_amd import scheduler as S

PARENTS = [-1, 0, 0, 1, 1, 2, 3, 3]      # test_tree_block_skip.py:16-18
TOKENS = [1, 2, 3, 4, 5, 6, 7]
DEPTHS = [0, 1, 1, 2, 2, 2, 3, 3]


def test_local_blocks_are_connected_and_ancestor_closed():
    # test_tree_block_skip.py:21-29
    assert S.local_tree_block(PARENTS, TOKENS, DEPTHS, 0, 4).nodes == (0, 1, 2, 3)
    block = S.local_tree_block(PARENTS, TOKENS, DEPTHS, 3, 8)
    assert block.nodes == (3, 6, 7)
    assert block.parents == (-1, 0, 0)
    assert block.tokens == (6, 7)
    assert block.depths == (2, 3, 3)


def test_local_block_is_the_id_order_prefix_of_the_subtree():
    rng = random.Random(5)
    for _ in range(200):
        n = rng.randrange(1, 40)
        parents = [-1] + [rng.randrange(0, k) for k in range(1, n)]
        depths = [0] * n
        for k in range(1, n):
            depths[k] = depths[parents[k]] + 1
        tokens = list(range(1, n))
        root = rng.randrange(0, n)
        cap = rng.randrange(1, n + 2)

        def below(node):
            while node > root:
                node = parents[node]
            return node == root
        want = [v for v in range(root, n) if below(v)][:cap]
        block = S.local_tree_block(parents, tokens, depths, root, cap)
        assert list(block.nodes) == want
        for row, node in enumerate(block.nodes[1:], 1):
            assert block.nodes[block.parents[row]] == parents[node]


def test_child_lookup():
    # test_tree_block_skip.py:94-96
    assert S.child_for_edge(PARENTS, TOKENS, 1, 4) == 4
    assert S.child_for_edge(PARENTS, TOKENS, 1, 8) is None


def test_tree_validation_errors():
    with pytest.raises(ValueError, match="topologically"):
        S.local_tree_block([-1, 1], [3], [0, 1], 0, 2)
    with pytest.raises(ValueError, match="repeat a child token"):
        S.local_tree_block([-1, 0, 0], [3, 3], [0, 1, 1], 0, 2)
    with pytest.raises(ValueError, match="controls"):
        S.local_tree_block(PARENTS, TOKENS, DEPTHS, 0, 0)


def test_prefix_tree_is_the_first_budget_nodes():
    tree = S.DraftTree(PARENTS, TOKENS, DEPTHS, [0.0, -0.1, -0.2, -0.3, -0.4, -0.5, -0.6, -0.7])
    tier = S.prefix_tree(tree, 4)
    assert tier.parents == PARENTS[:5] and tier.tokens == TOKENS[:4] and tier.depths == DEPTHS[:5]
    assert tier.draft_prefix_log_masses == [0.0, -0.1, -0.2, -0.3, -0.4]
    assert S.draft_tree_expected_tokens(tier) == 1.0 + sum(
        math.exp(v) for v in (-0.1, -0.2, -0.3, -0.4))
    with pytest.raises(ValueError):
        S.prefix_tree(tree, 8)


def _state(rid, generated, age, tree=True, block_root=0, budget=None, done=False):
    t = S.DraftTree(PARENTS, TOKENS, DEPTHS) if tree else None
    return SimpleNamespace(request_id=rid, generated=[0] * generated, age=age, tree=t,
                           block_root=block_root, proposal_tree_budget=budget, done=done,
                           continuation=t is not None and block_root != 0)


def test_select_ready_orders_continuations_then_age_and_respects_budgets():
    states = [_state(0, 3, 1), _state(1, 3, 4), _state(2, 3, 0, block_root=3),
              _state(3, 3, 9, done=True), _state(4, 3, 2, tree=False), _state(5, 3, 4)]
    chosen, blocks = S.select_ready(states, row_cap=4, slot_capacity=None, row_budget=10)
    # continuation 2 (3 rows), then ages 4 (ids 1, 5: 4 rows each -> 5 overflows)
    assert [s.request_id for s in chosen] == [2, 1]
    assert [b.nodes for b in blocks] == [(3, 6, 7), (0, 1, 2, 3)]
    assert [s.age for s in states] == [2, 0, 0, 9, 2, 5]
    chosen, _ = S.select_ready(states, row_cap=2, slot_capacity=2, row_budget=None)
    assert [s.request_id for s in chosen] == [2, 5]


def test_global_tree_budget_allocator_fixtures():
    # test_continuous_tree_block_decode.py:413-458
    two = [SimpleNamespace(generated=[0], age=0), SimpleNamespace(generated=[0], age=0)]
    assert S.allocate_global_tree_budgets(
        two, (1, 3), ((2.0, 2.1), (2.0, 2.1)), row_budget=8, fixed_row_equivalent=1.0,
        criticality_weight=0.0, max_new_tokens=8) == (1, 1)
    assert S.allocate_global_tree_budgets(
        two, (1, 3), ((2.0, 4.0), (2.0, 2.1)), row_budget=6, fixed_row_equivalent=32.0,
        criticality_weight=0.0, max_new_tokens=8) == (3, 1)
    lag = [SimpleNamespace(generated=[0] * 4, age=0), SimpleNamespace(generated=[0] * 2, age=0)]
    assert S.allocate_global_tree_budgets(
        lag, (1, 3), ((2.0, 3.0), (2.0, 3.0)), row_budget=6, fixed_row_equivalent=32.0,
        criticality_weight=2.0, max_new_tokens=8) == (1, 3)
    curve = ((2, 1.0), (4, 1.0))
    assert S.global_wave_cost(3, None, curve) == 1.0
    assert S.allocate_global_tree_budgets(
        [SimpleNamespace(generated=[0], age=0)], (1, 3), ((2.0, 3.0),), row_budget=4,
        fixed_row_equivalent=None, criticality_weight=0.0, max_new_tokens=8,
        row_cost_curve=curve) == (3,)


def test_allocator_matches_brute_force():
    """The allocation maximises reward / wave cost over every feasible tier
    choice (ties: fewer rows, then smaller tiers), checked by enumeration."""
    rng = random.Random(20260916)
    options = (11, 23, 45)
    curve = ((12, 24.0), (46, 24.5), (96, 25.0), (193, 28.0), (384, 40.0))
    for trial in range(40):
        count = rng.randrange(1, 5)
        states = [SimpleNamespace(generated=[0] * rng.randrange(1, 64), age=rng.randrange(5))
                  for _ in range(count)]
        utilities = [sorted(1 + rng.random() * 5 for _ in options) for _ in states]
        row_budget = rng.randrange(count * 12, 194)
        use_curve = trial % 2 == 0
        lead = max(len(s.generated) for s in states)
        oldest = max(1, max(s.age for s in states))
        weights = [1 + (lead - len(s.generated)) / 64 + s.age / oldest for s in states]
        best = None
        for alloc in itertools.product(options, repeat=count):
            rows = sum(b + 1 for b in alloc)
            if rows > row_budget:
                continue
            reward = sum(w * u[options.index(b)] for w, u, b in zip(weights, utilities, alloc))
            cost = (S.global_wave_cost(rows, None, curve) if use_curve
                    else S.global_wave_cost(rows, 20.0, None))
            key = (reward / cost, -rows, tuple(-b for b in alloc))
            if best is None or key > best[0]:
                best = (key, alloc)
        got = S.allocate_global_tree_budgets(
            states, options, utilities, row_budget=row_budget,
            fixed_row_equivalent=None if use_curve else 20.0, criticality_weight=1,
            max_new_tokens=64, row_cost_curve=curve if use_curve else None)
        assert got == best[1]


def test_allocator_rejects_bad_problems():
    st = [SimpleNamespace(generated=[0], age=0)]
    with pytest.raises(ValueError):
        S.allocate_global_tree_budgets(st, (3, 1), ((2.0, 2.0),), row_budget=8,
                                       fixed_row_equivalent=1.0, criticality_weight=0.0,
                                       max_new_tokens=8)
    with pytest.raises(ValueError):
        S.allocate_global_tree_budgets(st, (1, 3), ((0.5, 2.0),), row_budget=8,
                                       fixed_row_equivalent=1.0, criticality_weight=0.0,
                                       max_new_tokens=8)
    with pytest.raises(ValueError):
        S.normalize_row_cost_curve(((4, 1.0), (2, 2.0)))


def test_admission_and_tier_gates():
    # test_continuous_tree_block_decode.py:461-497
    states = [SimpleNamespace(request_id=0, generated=[0] * 4, age=9),
              SimpleNamespace(request_id=1, generated=[0] * 2, age=0),
              SimpleNamespace(request_id=2, generated=[0] * 2, age=3),
              SimpleNamespace(request_id=3, generated=[0] * 3, age=20)]
    admitted = S.admit_global_proposal_states(states, row_budget=4, minimum_tree_budget=1)
    assert tuple(s.request_id for s in admitted) == (1, 2)
    assert S.globally_feasible_budget_options(
        (11, 23, 45), request_count=4, row_budget=193, require_tier_fit=True) == (11, 23, 45)
    assert S.globally_feasible_budget_options(
        (11, 23, 45), request_count=8, row_budget=193, require_tier_fit=True) == (11, 23)
    assert S.globally_feasible_budget_options(
        (11, 23, 45), request_count=16, row_budget=193, require_tier_fit=True) == (11,)
    assert S.active_global_tree_budget_options(
        (11, 23, 45), active_count=9, expansion_active_limit=8) == (11,)
    assert S.active_global_tree_budget_options(
        (11, 23, 45), active_count=8, expansion_active_limit=8) == (11, 23, 45)
