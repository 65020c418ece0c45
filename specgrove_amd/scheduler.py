"""Host scheduling of the packed verification waves: which requests verify in
a wave, with which slice of their draft tree.

Restates, for the drop-in wave loop (``specgrove_amd.decode``), the
reference's host scheduler (paths relative to the reference snapshot,
CTBD = code/natural/src/gbv_experiments/continuous_tree_block_decode.py,
TBS = code/natural/src/gbv_experiments/tree_block_skip.py):

* tree blocks -- ``local_tree_block`` (TBS:95-125): the first ``row_cap``
  nodes of the remaining subtree below a root in best-first node order, as a
  block with local parents; ``tree_block_from_nodes`` (TBS:128-150);
  ``child_for_edge`` (TBS:250-258);
* tiers -- ``prefix_tree`` (CTBD:571-586): the first ``budget`` nodes of a
  canonical best-first tree (ancestor-closed because parents precede
  children);
* ``select_ready`` (CTBD:1158-1195): continuations first, then the oldest,
  under a slot cap and a shared row budget; ages advance for the ones left
  out;
* occupancy controls -- ``effective_row_cap`` (CTBD:1198-1216),
  ``effective_tree_budget(s)`` (:1247-1300) and
  ``adaptive_expansion_eligible`` (:1303-1314): larger blocks and trees
  only when few requests are ready or active;
* global tree budgets -- ``admit_global_proposal_states`` (CTBD:648-667),
  ``globally_feasible_budget_options`` (:670-690),
  ``active_global_tree_budget_options`` (:693-703), ``global_wave_cost``
  (:619-641) with ``normalize_row_cost_curve`` (:589-616), and
  ``allocate_global_tree_budgets`` (:706-795): a multiple-choice knapsack
  over the wave's rows that maximises expected accepted tokens per unit of
  wave cost.

Error classes and messages follow the reference's, so callers' handling is
unchanged.  Everything here is host Python over small integer lists (at most
a few hundred requests and a few thousand rows per wave).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from numbers import Integral
from typing import Sequence

__all__ = [
    "TreeBlock", "DraftTree", "local_tree_block", "tree_block_from_nodes", "child_for_edge",
    "prefix_tree", "select_ready", "effective_row_cap", "effective_tree_budget",
    "effective_tree_budgets", "adaptive_expansion_eligible", "admit_global_proposal_states",
    "globally_feasible_budget_options", "active_global_tree_budget_options",
    "normalize_row_cost_curve", "global_wave_cost", "allocate_global_tree_budgets",
]


# --------------------------------------------------------------------------
# trees and blocks
# --------------------------------------------------------------------------

@dataclass(frozen=True)
class TreeBlock:
    """A connected, ancestor-closed block of a draft tree: ``nodes`` in the
    tree's numbering (``nodes[0] == root``), ``parents`` local to the block
    (root -1), the non-root nodes' ``tokens`` and every node's global
    ``depths``."""
    root: int
    nodes: tuple[int, ...]
    parents: tuple[int, ...]
    tokens: tuple[int, ...]
    depths: tuple[int, ...]


@dataclass
class DraftTree:
    """A draft tree in best-first order: node 0 is the root (the newest
    committed token), ``parents[k] < k``, ``tokens[k - 1]`` is node k's draft
    token and ``depths[k]`` its depth.  ``draft_prefix_log_masses`` (optional)
    holds the log draft probability of reaching each node, for tier
    utilities."""
    parents: list[int]
    tokens: list[int]
    depths: list[int]
    draft_prefix_log_masses: list[float] | None = None


def _check_tree(parents: Sequence[int], tokens: Sequence[int]) -> None:
    bad = (not parents or len(tokens) != len(parents) - 1 or parents[0] != -1)
    if not bad:
        for node in range(1, len(parents)):
            p = parents[node]
            if isinstance(p, bool) or not isinstance(p, Integral) or not 0 <= p < node:
                bad = True
                break
    if bad:
        raise ValueError("Invalid topologically ordered tree")
    edges = set()
    for node in range(1, len(parents)):
        edge = (int(parents[node]), int(tokens[node - 1]))
        if edge in edges:
            raise ValueError("A tree parent cannot repeat a child token")
        edges.add(edge)


def _is_index(value) -> bool:
    return isinstance(value, Integral) and not isinstance(value, bool)


def tree_block_from_nodes(parents: Sequence[int], tokens: Sequence[int],
                          depths: Sequence[int], root: int,
                          nodes: Sequence[int]) -> TreeBlock:
    """The block of an ancestor-closed, ascending node list starting at
    ``root`` (TBS:128-150)."""
    _check_tree(parents, tokens)
    nodes = tuple(int(v) for v in nodes)
    if (len(depths) != len(parents) or not nodes or nodes[0] != root
            or any(b <= a for a, b in zip(nodes, nodes[1:]))):
        raise ValueError("Invalid explicit tree block")
    row_of = {node: row for row, node in enumerate(nodes)}
    local_parents = [-1]
    for node in nodes[1:]:
        row = row_of.get(int(parents[node]))
        if row is None:
            raise AssertionError("Tree block is not ancestor closed")
        local_parents.append(row)
    return TreeBlock(root=root, nodes=nodes, parents=tuple(local_parents),
                     tokens=tuple(int(tokens[node - 1]) for node in nodes[1:]),
                     depths=tuple(int(depths[node]) for node in nodes))


def local_tree_block(parents: Sequence[int], tokens: Sequence[int], depths: Sequence[int],
                     root: int, row_cap: int) -> TreeBlock:
    """The first ``row_cap`` nodes (root included) of ``root``'s subtree in
    node order (TBS:95-125).  Node ids are best-first, so every prefix of a
    subtree's id order is ancestor-closed."""
    _check_tree(parents, tokens)
    if (len(depths) != len(parents) or not _is_index(root) or not 0 <= root < len(parents)
            or not _is_index(row_cap) or row_cap < 1):
        raise ValueError("Invalid local tree-block controls")
    root, row_cap = int(root), int(row_cap)
    # A node belongs to the subtree iff its parent does (parents precede
    # children), so one forward pass marks the whole subtree.
    inside = {root}
    nodes = [root]
    for node in range(root + 1, len(parents)):
        if len(nodes) == row_cap:
            break
        if int(parents[node]) in inside:
            inside.add(node)
            nodes.append(node)
    return tree_block_from_nodes(parents, tokens, depths, root, nodes)


def child_for_edge(parents: Sequence[int], tokens: Sequence[int], parent: int,
                   token: int) -> int | None:
    """The child of ``parent`` whose draft token is ``token``, if any
    (TBS:250-258)."""
    for node in range(parent + 1, len(parents)):
        if int(parents[node]) == parent and int(tokens[node - 1]) == token:
            return node
    return None


def prefix_tree(tree: DraftTree, budget: int) -> DraftTree:
    """The tier of ``budget`` draft nodes (``budget + 1`` rows with the root):
    the first nodes of the canonical best-first tree (CTBD:571-586)."""
    if budget < 1 or budget > len(tree.tokens):
        raise ValueError("DDTree prefix budget is outside the source tree")
    if any(p > budget for p in tree.parents[1:budget + 1]):
        raise RuntimeError("Canonical DDTree prefix is not ancestor closed")
    masses = tree.draft_prefix_log_masses
    return DraftTree(parents=list(tree.parents[:budget + 1]), tokens=list(tree.tokens[:budget]),
                     depths=list(tree.depths[:budget + 1]),
                     draft_prefix_log_masses=(list(masses[:budget + 1])
                                              if masses is not None else None))


def draft_tree_expected_tokens(tree: DraftTree) -> float:
    """Expected accepted draft tokens plus the bonus under the draft itself:
    1 + sum of the reach probabilities of the non-root nodes (CTBD:560-568),
    the utility of a tier."""
    masses = tree.draft_prefix_log_masses
    if masses is None or len(masses) != len(tree.parents):
        raise ValueError("Global tree budgeting requires DDTree prefix masses")
    value = 1.0 + sum(math.exp(m) for m in masses[1:])
    if not math.isfinite(value) or value < 1.0:
        raise FloatingPointError("Invalid draft-tree expected-token utility")
    return value


# --------------------------------------------------------------------------
# wave selection
# --------------------------------------------------------------------------

def select_ready(states: Sequence, row_cap: int, slot_capacity: int | None,
                 row_budget: int | None = None, use_proposal_tree_budget: bool = False):
    """Requests and blocks of the next wave (CTBD:1158-1195).

    Ready requests (not done, with a tree) are taken continuations first,
    then by decreasing age, then by request id.  Each contributes the block
    of at most ``row_cap`` rows (its tier's rows when
    ``use_proposal_tree_budget``) below its current block root; a request
    whose block would overflow ``row_budget`` is skipped, and selection stops
    at ``slot_capacity`` requests.  Chosen requests' ages reset to 0, the
    others' grow by one.  Returns (chosen states, blocks).
    """
    ready = [s for s in states if not s.done and s.tree is not None]
    ready.sort(key=lambda s: (0 if s.continuation else 1, -s.age, s.request_id))
    chosen, blocks = [], []
    used = 0
    for state in ready:
        cap = (state.proposal_tree_budget + 1
               if use_proposal_tree_budget and state.proposal_tree_budget is not None
               else row_cap)
        block = local_tree_block(state.tree.parents, state.tree.tokens, state.tree.depths,
                                 state.block_root, cap)
        if slot_capacity is not None and len(chosen) >= slot_capacity:
            break
        if row_budget is not None and used + len(block.nodes) > row_budget:
            continue
        chosen.append(state)
        blocks.append(block)
        used += len(block.nodes)
    picked = {s.request_id for s in chosen}
    for state in ready:
        state.age = 0 if state.request_id in picked else state.age + 1
    return chosen, blocks


def effective_row_cap(row_cap: int, low_occupancy_row_cap: int | None,
                      low_occupancy_threshold: int | None, ready_count: int,
                      mid_occupancy_row_cap: int | None = None,
                      mid_occupancy_threshold: int | None = None) -> int:
    """Rows per request block for the next wave (CTBD:1198-1216): the
    low-occupancy cap at or below ``low_occupancy_threshold`` ready requests,
    else the mid-occupancy cap at or below ``mid_occupancy_threshold``, else
    ``row_cap`` -- larger blocks only when the saved rows could not admit
    another request anyway."""
    if (low_occupancy_row_cap is not None and low_occupancy_threshold is not None
            and ready_count <= low_occupancy_threshold):
        return low_occupancy_row_cap
    if (mid_occupancy_row_cap is not None and mid_occupancy_threshold is not None
            and ready_count <= mid_occupancy_threshold):
        return mid_occupancy_row_cap
    return row_cap


def effective_tree_budget(default_budget: int, proposal_tree_budget: int | None,
                          low_occupancy_tree_budget: int | None,
                          low_occupancy_tree_threshold: int | None, active_count: int) -> int:
    """Draft-tree size at the current occupancy (CTBD:1247-1260): the
    low-occupancy budget at or below ``low_occupancy_tree_threshold`` active
    requests, else ``proposal_tree_budget`` or the default."""
    if (low_occupancy_tree_budget is not None and low_occupancy_tree_threshold is not None
            and active_count <= low_occupancy_tree_threshold):
        return low_occupancy_tree_budget
    return proposal_tree_budget or default_budget


def effective_tree_budgets(states: Sequence, default_budget: int,
                           proposal_tree_budget: int | None,
                           low_occupancy_tree_budget: int | None,
                           low_occupancy_tree_threshold: int | None, active_count: int,
                           low_occupancy_expansion_slots: int | None) -> tuple[int, ...]:
    """Per-request tree budgets (CTBD:1263-1300): when the occupancy calls
    for the larger tree and ``low_occupancy_expansion_slots`` is below the
    number of requests, only that many requests get it -- those with the
    fewest generated tokens (the most remaining work), then the oldest, then
    the lowest id; the others keep the base budget."""
    base = proposal_tree_budget or default_budget
    expanded = effective_tree_budget(default_budget, proposal_tree_budget,
                                     low_occupancy_tree_budget, low_occupancy_tree_threshold,
                                     active_count)
    if (expanded == base or low_occupancy_expansion_slots is None
            or low_occupancy_expansion_slots >= len(states)):
        return (expanded,) * len(states)
    ranked = sorted(states, key=lambda s: (len(s.generated), -s.age, s.request_id))
    chosen = {s.request_id for s in ranked[:low_occupancy_expansion_slots]}
    return tuple(expanded if s.request_id in chosen else base for s in states)


def adaptive_expansion_eligible(initial_count: int, thresholds: Sequence[int],
                                requires_drain: bool) -> bool:
    """Whether the occupancy-dependent expansions may apply to a run of
    ``initial_count`` requests (CTBD:1303-1314): with ``requires_drain``,
    only when the run starts above every threshold (a drained tail, not a
    small run)."""
    if initial_count < 1 or any(t < 1 for t in thresholds):
        raise ValueError("Invalid adaptive expansion occupancy")
    return not requires_drain or not thresholds or initial_count > max(thresholds)


def admit_global_proposal_states(states: Sequence, *, row_budget: int,
                                 minimum_tree_budget: int) -> tuple:
    """At most ``row_budget // (minimum_tree_budget + 1)`` requests may draft
    for the next wave: the most lagging (fewest generated tokens), then the
    oldest, then the lowest id (CTBD:648-667).  Original order is kept."""
    minimum_rows = minimum_tree_budget + 1
    capacity = row_budget // minimum_rows
    if row_budget < minimum_rows or capacity < 1:
        raise ValueError("Global row budget cannot admit one minimum tree")
    if len(states) <= capacity:
        return tuple(states)
    order = sorted(states, key=lambda s: (len(s.generated), -s.age, s.request_id))
    admitted = {s.request_id for s in order[:capacity]}
    return tuple(s for s in states if s.request_id in admitted)


def globally_feasible_budget_options(budget_options: Sequence[int], *, request_count: int,
                                     row_budget: int | None,
                                     require_tier_fit: bool) -> tuple[int, ...]:
    """Tiers small enough to give every request of the wave that tier
    (CTBD:670-690)."""
    options = tuple(int(v) for v in budget_options)
    if (not options or request_count < 1 or row_budget is None or row_budget < 1
            or not isinstance(require_tier_fit, bool)):
        raise ValueError("Invalid global tree-budget tier gate")
    if not require_tier_fit:
        return options
    fits = tuple(b for b in options if request_count * (b + 1) <= row_budget)
    if not fits:
        raise RuntimeError("No tree-budget tier can cover the admitted wave")
    return fits


def active_global_tree_budget_options(budget_options: Sequence[int], *, active_count: int,
                                      expansion_active_limit: int | None) -> tuple[int, ...]:
    """Only the smallest tier while more than ``expansion_active_limit``
    requests are active (CTBD:693-703)."""
    options = tuple(int(v) for v in budget_options)
    if (not options or active_count < 1
            or (expansion_active_limit is not None and expansion_active_limit < 1)):
        raise ValueError("Invalid active-request global tree-budget gate")
    if expansion_active_limit is not None and active_count > expansion_active_limit:
        return (options[0],)
    return options


# --------------------------------------------------------------------------
# global tree budgets
# --------------------------------------------------------------------------

def normalize_row_cost_curve(curve) -> tuple[tuple[int, float], ...] | None:
    """A measured wave-cost curve: (rows, cost) points with rows strictly and
    cost weakly increasing, rows >= 1, costs finite and positive
    (CTBD:589-616)."""
    if curve is None:
        return None
    try:
        points = tuple((int(p[0]), float(p[1])) for p in curve)
        widths = [len(p) for p in curve]
    except (IndexError, TypeError, ValueError) as error:
        raise ValueError("Invalid global Target row-cost curve") from error
    valid = bool(points) and all(w == 2 for w in widths) and all(
        r >= 1 and math.isfinite(c) and c > 0 for r, c in points) and all(
        a[0] < b[0] and a[1] <= b[1] for a, b in zip(points, points[1:]))
    if not valid:
        raise ValueError("Invalid global Target row-cost curve")
    return points


def global_wave_cost(rows: int, fixed_row_equivalent: float | None,
                     row_cost_curve: Sequence[tuple[int, float]] | None) -> float:
    """Cost of a wave of ``rows`` packed rows: linear interpolation of the
    measured curve (flat outside it), or ``fixed_row_equivalent + rows``
    without one (CTBD:619-641)."""
    if rows < 1:
        raise ValueError("A Target wave must contain at least one row")
    if row_cost_curve is None:
        if (fixed_row_equivalent is None or not math.isfinite(fixed_row_equivalent)
                or fixed_row_equivalent <= 0):
            raise ValueError("Missing global Target cost model")
        return fixed_row_equivalent + rows
    points = tuple(row_cost_curve)
    if rows <= points[0][0]:
        return points[0][1]
    for (r0, c0), (r1, c1) in zip(points, points[1:]):
        if rows <= r1:
            return c0 + (rows - r0) / (r1 - r0) * (c1 - c0)
    return points[-1][1]


_TIE = 1e-12


def allocate_global_tree_budgets(states: Sequence, budget_options: Sequence[int],
                                 utilities: Sequence[Sequence[float]], *,
                                 row_budget: int | None, fixed_row_equivalent: float | None,
                                 criticality_weight: float, max_new_tokens: int | None,
                                 row_cost_curve=None) -> tuple[int, ...]:
    """One tier per request for the next wave (CTBD:706-795).

    Request j's tier b costs ``b + 1`` rows and is worth ``w_j * u_j(b)``,
    where ``w_j = 1 + criticality_weight * (lag_j / max_new_tokens +
    age_j / max_age)`` favours lagging and older requests.  Over every exact
    total of rows within ``row_budget`` the best-rewarded allocation is kept
    (a dense table indexed by rows; ties within 1e-12 go to the
    lexicographically smaller allocation); the wave then takes the total whose
    reward per unit of ``global_wave_cost`` is largest, preferring fewer rows
    and then smaller tiers.
    """
    options = tuple(int(v) for v in budget_options)
    curve = normalize_row_cost_curve(row_cost_curve)
    valid = (
        bool(states) and bool(options) and tuple(sorted(set(options))) == options
        and options[0] >= 1 and row_budget is not None
        and row_budget >= len(states) * (options[0] + 1)
        and (fixed_row_equivalent is None) != (curve is None)
        and (fixed_row_equivalent is None or (math.isfinite(fixed_row_equivalent)
                                              and fixed_row_equivalent > 0))
        and math.isfinite(criticality_weight) and criticality_weight >= 0
        and max_new_tokens is not None and max_new_tokens >= 1
        and len(utilities) == len(states)
        and all(len(u) == len(options) for u in utilities)
        and all(math.isfinite(v) and v >= 1.0 for u in utilities for v in u))
    if not valid:
        raise ValueError("Invalid global tree-budget allocation problem")
    progress = [len(s.generated) for s in states]
    lead = max(progress)
    oldest = max(1, max(s.age for s in states))
    weights = [1.0 + criticality_weight * ((lead - g) / max_new_tokens + s.age / oldest)
               for s, g in zip(states, progress)]
    # best[r] = (reward, allocation) over the requests seen so far using r rows.
    best: list[tuple[float, tuple[int, ...]] | None] = [None] * (row_budget + 1)
    best[0] = (0.0, ())
    for weight, values in zip(weights, utilities):
        nxt: list[tuple[float, tuple[int, ...]] | None] = [None] * (row_budget + 1)
        for used, entry in enumerate(best):
            if entry is None:
                continue
            reward, allocation = entry
            for b, value in zip(options, values):
                rows = used + b + 1
                if rows > row_budget:
                    continue
                cand = (reward + weight * value, allocation + (b,))
                cur = nxt[rows]
                if (cur is None or cand[0] > cur[0] + _TIE
                        or (abs(cand[0] - cur[0]) <= _TIE and cand[1] < cur[1])):
                    nxt[rows] = cand
        best = nxt
    choice = None
    for rows, entry in enumerate(best):
        if entry is None:
            continue
        key = (entry[0] / global_wave_cost(rows, fixed_row_equivalent, curve), -rows,
               tuple(-b for b in entry[1]))
        if choice is None or key > choice[0]:
            choice = (key, entry[1])
    if choice is None:
        raise RuntimeError("Global tree-budget allocator found no feasible wave")
    return choice[1]
