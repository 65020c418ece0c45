"""The wave loop's host decisions on the CPU: the option contract, the
proposal step (occupancy tree budgets, global admission and tiers) and the
occupancy row cap of the selection, without running a wave.  Expected
values follow the reference's rules (continuous_tree_block_decode.py,
CTBD below) applied by hand to the same states."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from specgrove_amd import ddtree
from specgrove_amd import decode as D


class _Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.w = torch.nn.Parameter(torch.zeros(1))


class _Cache:
    def __init__(self, n):
        self.n = n

    def get_seq_length(self):
        return self.n


def _states(lengths):
    return [D.DecodeRequest(i, [5] * g, _Cache(40 + i), None) for i, g in enumerate(lengths)]


def _proposer(vocab=64, depth=5, seed=0):
    rng = np.random.default_rng(seed)
    calls = []

    def draft(states):
        calls.append(tuple(s.request_id for s in states))
        logits = torch.from_numpy(rng.standard_normal((len(states), depth, vocab)) * 2)
        return torch.softmax(logits, -1)
    return ddtree.DDTreeProposer(draft), calls


def _loop(propose, **kw):
    kw.setdefault("max_new_tokens", 32)
    return D.WaveLoop(_Model(), propose, persistent=False, **kw)


def test_contract():
    p, _ = _proposer()
    good = dict(tree_budget=12, row_cap=4, row_budget=64)
    _loop(p, **good)
    bad = [
        dict(row_budget=2),                                   # budget below the row cap
        dict(tree_budget=None),                               # batched proposer, no budget
        dict(low_occupancy_row_cap=8),                        # cap without threshold
        dict(low_occupancy_row_cap=2, low_occupancy_threshold=2),   # below row_cap
        dict(low_occupancy_row_cap=16, low_occupancy_threshold=2,
             mid_occupancy_row_cap=20, mid_occupancy_threshold=4),  # mid above low
        dict(low_occupancy_row_cap=16, low_occupancy_threshold=4,
             mid_occupancy_row_cap=8, mid_occupancy_threshold=4),   # thresholds not increasing
        dict(proposal_tree_budget=13),                        # above the tree budget
        dict(low_occupancy_tree_budget=12),                   # budget without threshold
        dict(proposal_tree_budget=4, low_occupancy_tree_budget=3,
             low_occupancy_tree_threshold=2),                 # expansion below the base
        dict(proposal_tree_budget=4, low_occupancy_tree_budget=12,
             low_occupancy_tree_threshold=2, low_occupancy_expansion_slots=3),
        dict(global_tree_budget_options=(3, 7)),              # row_cap != options[0] + 1
        dict(global_tree_criticality_weight=1.0),             # global control without options
        dict(continuation_ready_threshold=-1),
    ]
    for b in bad:
        with pytest.raises(ValueError, match="experiment contract"):
            _loop(p, **{**good, **b})
    g = dict(tree_budget=12, row_cap=4, row_budget=64, global_tree_budget_options=(3, 7),
             continuation_ready_threshold=0, global_tree_fixed_row_equivalent=8.0)
    _loop(p, **g)
    for b in (dict(continuation_ready_threshold=None), dict(global_tree_budget_options=(3, 13)),
              dict(global_tree_fixed_row_equivalent=None),
              dict(global_tree_row_cost_curve=((4, 1.0), (64, 2.0))),
              dict(global_tree_fixed_row_equivalent=None, global_tree_row_cost_curve=((5, 1.0),
                                                                                    (64, 2.0)))):
        with pytest.raises(ValueError, match="experiment contract"):
            _loop(p, **{**g, **b})
    with pytest.raises(ValueError, match="canonical DDTree"):
        _loop(ddtree.DDTreeProposer(None, depth_reward=0.5), **g)


def test_occupancy_tree_budgets_and_counts():
    p, calls = _proposer()
    loop = _loop(p, tree_budget=12, row_cap=13, row_budget=64, proposal_tree_budget=4,
                 low_occupancy_tree_budget=12, low_occupancy_tree_threshold=2,
                 low_occupancy_expansion_slots=1)
    states = _states([3, 1, 2])
    loop.attach(states)
    loop._propose(states)                         # 3 active > threshold 2: base budget
    assert [len(s.tree.tokens) for s in states] == [4, 4, 4]
    assert [s.proposal_tree_budget for s in states] == [4, 4, 4]
    assert [s.round_prefix_len for s in states] == [40, 41, 42]
    states[0].done = True
    for s in states[1:]:
        s.tree = None
    states[1].generated = [5] * 3
    states[2].generated = [5]                      # fewest tokens: request 2 expands
    loop._propose(states)
    assert [len(s.tree.tokens) for s in states[1:]] == [4, 12]
    assert calls == [(0, 1, 2), (1, 2)]
    assert dict(loop.tree_budget_counts) == {4: 4, 12: 1}


def test_drain_rule_disables_expansions_for_small_runs():
    p, _ = _proposer()
    kw = dict(tree_budget=12, row_cap=4, row_budget=64, proposal_tree_budget=4,
              low_occupancy_tree_budget=12, low_occupancy_tree_threshold=2,
              low_occupancy_row_cap=16, low_occupancy_threshold=2,
              adaptive_expansion_requires_drain=True)
    small, big = _loop(p, **kw), _loop(p, **kw)
    small.attach(_states([1, 1]))
    big.attach(_states([1, 1, 1]))
    assert not small.expansion_eligible and big.expansion_eligible
    states = _states([1, 1])
    small._propose(states)
    assert [len(s.tree.tokens) for s in states] == [4, 4]
    small._select(states)
    assert dict(small.row_cap_counts) == {4: 1}


def test_occupancy_row_cap_in_selection():
    p, _ = _proposer(depth=8, vocab=8)
    loop = _loop(p, tree_budget=40, row_cap=4, row_budget=100, low_occupancy_row_cap=24,
                 low_occupancy_threshold=2, mid_occupancy_row_cap=12, mid_occupancy_threshold=3)
    states = _states([1, 1, 1, 1])
    loop.attach(states)
    loop._propose(states)
    sizes = []
    for active in (4, 3, 2):
        for s in states[active:]:
            s.done = True
        _, chosen, blocks = loop._select(states)
        sizes.append([len(b.nodes) for b in blocks])
    assert sizes == [[4] * 4, [12] * 3, [24] * 2]
    assert dict(loop.row_cap_counts) == {4: 1, 12: 1, 24: 1}


def test_global_admission_defers_and_allocates_tiers():
    p, calls = _proposer(depth=6, vocab=32)
    loop = _loop(p, tree_budget=15, row_cap=2, row_budget=12,
                 global_tree_budget_options=(1, 3, 7), continuation_ready_threshold=0,
                 global_tree_fixed_row_equivalent=4.0, global_tree_criticality_weight=1.0)
    states = _states([6, 2, 4, 2, 9, 3, 7, 1])
    loop.attach(states)
    loop._propose(states)
    # row_budget // 2 = 6 requests draft: the six with the fewest tokens (CTBD:648-667)
    admitted = sorted(range(8), key=lambda i: (len(states[i].generated), i))[:6]
    assert calls == [tuple(sorted(admitted))]
    for i, s in enumerate(states):
        if i in admitted:
            assert s.tree is not None and s.proposal_tree_budget in (1, 3, 7)
            assert len(s.tree.tokens) == s.proposal_tree_budget
        else:
            assert s.tree is None and s.age == 1
    assert loop.tree_budget_counts[0] == 2
    assert sum(s.proposal_tree_budget + 1 for s in states if s.tree) <= 12
    # the selection takes each admitted request's whole tier
    _, chosen, blocks = loop._select(states)
    assert all(len(b.nodes) == s.proposal_tree_budget + 1 for s, b in zip(chosen, blocks))


def test_result_fields_follow_the_reference_order():
    names = [f.name for f in D.DecodeResult.__dataclass_fields__.values()]
    assert names == ["outputs", "request_rounds", "wall_ms", "prefill_ms", "proposal_ms",
                     "target_ms", "pack_ms", "select_commit_ms", "physical_target_calls",
                     "physical_target_rows", "useful_target_rows", "padded_target_rows",
                     "effective_row_cap_counts", "effective_tree_budget_counts",
                     "gated_continuations"]
    loop = _loop(lambda s: None, row_cap=4)
    loop.calls, loop.rows, loop.useful_rows = 3, 40, 40
    loop.row_cap_counts = {4: 3}
    res = loop.result([SimpleNamespace(generated=[1, 2], rounds=[])], 0.5)
    assert res.wall_ms == 500.0 and res.padded_target_rows == 0
    assert res.target_calls == 3 and res.effective_row_cap_counts == ((4, 3),)
