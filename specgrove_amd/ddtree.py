"""DDTree proposal trees for the packed verification waves.

Restates the reference's tree builder ``probability_tree``
(code/natural/src/gbv_experiments/tree.py:148-212, TREE below) and the
proposal step that calls it for every request needing a tree
(``_propose_many``, continuous_tree_block_decode.py:798-870, CTBD below):

* the draft's per-depth probabilities ``q [L, V]`` are cut to their sorted
  top ``min(budget, V)`` tokens per depth (TREE:187-188);
* nodes are added best first by score = log reach probability plus the
  per-depth rewards, up to ``budget`` nodes; a popped node offers its next
  sibling (rank + 1 under the same parent, within the depth's rank cap) and
  its first child (rank 0 one depth down) as candidates (TREE:200-211), so
  parents always precede their children;
* ties are broken by (parent, depth, rank), the order of the reference's
  heap tuples, which decides the tree whenever two scores are equal;
* ``adaptive_min_budget`` shrinks the budget when the mean greedy log
  probability of the first four depths reaches ``log(confidence_threshold)``
  (TREE:189-197).

The wave builds all its trees with one top-k launch over ``[B, L, V]`` and one
device-to-host transfer (``probability_trees``); the expansion itself is a
few hundred heap operations per request on the host.
"""
from __future__ import annotations

import heapq
import math
from numbers import Integral
from typing import Callable, Sequence

import torch

from .scheduler import DraftTree

__all__ = ["probability_tree", "probability_trees", "DDTreeProposer"]


def _controls(length: int, vocab: int, budget: int, depth_reward: float,
              depth_reward_schedule, rank_caps):
    """Validated per-depth rewards and rank caps (TREE:169-186), with the
    reference's messages."""
    if not math.isfinite(depth_reward):
        raise ValueError("Tree depth reward must be finite")
    if depth_reward_schedule is not None and (
            len(depth_reward_schedule) != length
            or any(not math.isfinite(v) for v in depth_reward_schedule)):
        raise ValueError("Invalid tree depth-reward schedule")
    if rank_caps is not None and (
            len(rank_caps) != length
            or any(not isinstance(v, Integral) or isinstance(v, bool) or v < 1
                   for v in rank_caps)):
        raise ValueError("Invalid per-depth tree rank caps")
    if isinstance(budget, bool) or not isinstance(budget, Integral) or budget < 1:
        raise ValueError("Tree budget must be a positive integer")
    rewards = (tuple(float(v) for v in depth_reward_schedule)
               if depth_reward_schedule is not None else (float(depth_reward),) * length)
    caps = (tuple(min(int(v), budget, vocab) for v in rank_caps) if rank_caps is not None
            else (min(budget, vocab),) * length)
    return rewards, caps


def _expand(logs: Sequence[Sequence[float]], ids: Sequence[Sequence[int]], budget: int,
            rewards: Sequence[float], caps: Sequence[int],
            adaptive_min_budget: int | None, confidence_threshold: float | None) -> DraftTree:
    """Best-first expansion over sorted per-depth log probabilities ``logs``
    and token ids ``ids`` (one row per depth, descending)."""
    length = len(logs)
    if adaptive_min_budget is not None:
        if confidence_threshold is None:
            raise ValueError("Adaptive tree budget requires a confidence threshold")
        depths_seen = min(4, length)
        greedy = sum(logs[d][0] for d in range(depths_seen)) / depths_seen
        if greedy >= math.log(confidence_threshold):
            budget = adaptive_min_budget
    parents, tokens, depths, masses = [-1], [], [0], [0.0]
    # Candidate = (-score, parent node, depth index, rank); score is the log
    # reach mass of the parent + the token's log probability + the depth's
    # reward.  Each (parent, depth, rank) is offered once, so the key is
    # unique and its tuple order is the reference's tie-break.
    frontier = [(-(logs[0][0] + rewards[0]), 0, 0, 0)]
    while frontier and len(tokens) < budget:
        neg, parent, depth, rank = heapq.heappop(frontier)
        score = -neg
        node = len(parents)
        parents.append(parent)
        tokens.append(int(ids[depth][rank]))
        depths.append(depth + 1)
        masses.append(score)
        parent_score = masses[parent]
        if rank + 1 < caps[depth]:
            heapq.heappush(frontier, (-((parent_score + logs[depth][rank + 1]) + rewards[depth]),
                                      parent, depth, rank + 1))
        if depth + 1 < length:
            heapq.heappush(frontier, (-((score + logs[depth + 1][0]) + rewards[depth + 1]),
                                      node, depth + 1, 0))
    return DraftTree(parents=parents, tokens=tokens, depths=depths,
                     draft_prefix_log_masses=masses)


def probability_tree(q: torch.Tensor, budget: int, depth_reward: float = 0.0,
                     depth_reward_schedule: Sequence[float] | None = None,
                     rank_caps: Sequence[int] | None = None,
                     adaptive_min_budget: int | None = None,
                     confidence_threshold: float | None = None) -> DraftTree:
    """Best-first prefix tree of ``budget`` draft nodes over the draft's
    per-depth probabilities ``q [L, V]`` (TREE:148-212).

    ``depth_reward = 0`` is DDTree's product-probability tree; node k's
    ``draft_prefix_log_masses[k]`` is its score (log reach probability plus
    the rewards along its path).  The logarithms are taken in ``q``'s dtype
    on its device, as the reference does.
    """
    return probability_trees(q[None], [budget], depth_reward=depth_reward,
                             depth_reward_schedule=depth_reward_schedule,
                             rank_caps=rank_caps, adaptive_min_budget=adaptive_min_budget,
                             confidence_threshold=confidence_threshold)[0]


def probability_trees(q: torch.Tensor, budgets: Sequence[int], **controls) -> list[DraftTree]:
    """``probability_tree`` for every request of a wave: ``q [B, L, V]``,
    one budget per request.  One top-k over the whole batch and one
    device-to-host transfer; the same controls for every request."""
    if q.ndim != 3 or q.shape[0] != len(budgets) or q.shape[1] < 1 or q.shape[2] < 1:
        raise ValueError("Draft probabilities must be [requests, depths, vocab]")
    batch, length, vocab = q.shape
    checked = [_controls(length, vocab, b, controls.get("depth_reward", 0.0),
                         controls.get("depth_reward_schedule"), controls.get("rank_caps"))
               for b in budgets]
    k = min(max(int(b) for b in budgets), vocab)
    values, indices = torch.topk(q, k, dim=-1, sorted=True)
    host = torch.cat([values.log().double().reshape(batch, -1),
                      indices.double().reshape(batch, -1)], dim=1).cpu().tolist()
    trees = []
    for row, b, (rewards, caps) in zip(host, budgets, checked):
        width = min(int(b), vocab)
        logs = [row[d * k:d * k + width] for d in range(length)]
        ids = [[int(v) for v in row[length * k + d * k:length * k + d * k + width]]
               for d in range(length)]
        trees.append(_expand(logs, ids, int(b), rewards, caps,
                             controls.get("adaptive_min_budget"),
                             controls.get("confidence_threshold")))
    return trees


class DDTreeProposer:
    """Proposal step of the wave loop from a draft model's probabilities.

    ``draft_probabilities(states) -> q [len(states), L, V]`` runs the draft
    once for every request that needs a tree (the reference's one padded
    draft forward, CTBD:798-870); ``propose_many(states, budgets)`` cuts
    them into trees with ``probability_trees``.  ``canonical`` is whether
    the trees are DDTree's product-probability trees (no rewards, caps or
    adaptive budget), which global tier budgeting requires
    (CTBD:810-818).
    """

    def __init__(self, draft_probabilities: Callable[[Sequence], torch.Tensor], *,
                 depth_reward: float = 0.0,
                 depth_reward_schedule: Sequence[float] | None = None,
                 rank_caps: Sequence[int] | None = None,
                 adaptive_min_budget: int | None = None,
                 confidence_threshold: float | None = None):
        self.draft_probabilities = draft_probabilities
        self.controls = dict(depth_reward=depth_reward,
                             depth_reward_schedule=depth_reward_schedule,
                             rank_caps=rank_caps, adaptive_min_budget=adaptive_min_budget,
                             confidence_threshold=confidence_threshold)

    @property
    def canonical(self) -> bool:
        c = self.controls
        return (c["depth_reward"] == 0.0 and c["depth_reward_schedule"] is None
                and c["rank_caps"] is None and c["adaptive_min_budget"] is None)

    def propose_many(self, states: Sequence, budgets: Sequence[int]) -> list[DraftTree]:
        if not states:
            return []
        q = self.draft_probabilities(states)
        return probability_trees(q, list(budgets), **self.controls)
