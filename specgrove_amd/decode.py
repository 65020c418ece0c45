"""The packed verification wave loop on the drop-in path.

Restates the verify-and-commit core of the reference's decoder
``generate_continuous_tree_blocks`` (paths relative to the reference snapshot:
CTBD = code/natural/src/gbv_experiments/continuous_tree_block_decode.py; wave
loop :1640-2248; TREE = code/natural/src/gbv_experiments/tree.py) with this
repository's plugs in every slot:

  proposals   ``ddtree.DDTreeProposer`` (the DDTree builder over the draft
              model's per-depth probabilities, TREE:148-212) or any
              ``propose(state) -> DraftTree``; tree budgets from the
              occupancy controls (CTBD:1247-1300) or the global tier
              allocator (``scheduler.allocate_global_tree_budgets``,
              CTBD:706-795) after admission (:648-667);
  selection   ``scheduler.select_ready`` (CTBD:1158-1195) with the
              occupancy row cap (``scheduler.effective_row_cap``,
              CTBD:1198-1216);
  pack        ``cache.pack_cache_sequence`` + ``attention.pack_block_inputs``
              (CTBD:1772-1787) -- persistent arena or packed prefixes;
  target      the caller's transformers model, configured with
              ``attn_implementation="specgrove_hip"`` (CTBD:1791-1794);
  verify      ``verify.tree_verify_hip_rejection_batched`` on the wave's
              logits (CTBD:1845-2107, verifier ``"hip_tree_rejection"``);
  commit      ``PersistentRequestCachePool.append_packed_sequence`` or
              ``cache.split_compacted_sequence_caches`` with keep rows
              ``[0] + accepted`` (CTBD:2108-2143);
  tokens      accepted tokens + bonus, truncated at ``max_new_tokens`` and the
              first stop id, or a continuation block when the bonus edge is a
              tree edge and the gate allows it (CTBD:2186-2248).

Draft conditioning (feature chunks of the kept rows) and the draft models'
own caches are the proposer's business and are not restated; the run's
accounting is the reference's ``ContinuousDecodeResult`` (CTBD:103-123).
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import Callable, Sequence

import torch

from . import attention, cache as cache_mod, scheduler, verify


@dataclass
class DecodeRequest:
    """Per-request state of the wave loop (the fields of the reference's
    ``ContinuousDecodeRequest``, CTBD:74-100, that the verification path
    reads or writes).  ``generated[-1]`` is the newest committed token, whose
    K/V is not cached yet: it is the root row of the request's next block."""
    request_id: int
    generated: list[int]
    target_cache: object
    generator: torch.Generator
    tree: scheduler.DraftTree | None = None
    proposal_tree_budget: int | None = None
    round_prefix_len: int = 0
    block_root: int = 0
    accepted_nodes: list[int] = field(default_factory=list)
    accepted_tokens: list[int] = field(default_factory=list)
    round_block_rows: list[int] = field(default_factory=list)
    rounds: list[dict] = field(default_factory=list)
    done: bool = False
    age: int = 0

    @property
    def continuation(self) -> bool:
        return self.tree is not None and self.block_root != 0


@dataclass(frozen=True)
class DecodeResult:
    """Outputs and accounting of a decode, with the fields of the reference's
    ``ContinuousDecodeResult`` (CTBD:103-123) in its order, so run summaries
    read it unchanged.  Stage times are host wall times in ms; the packed
    layout pads nothing, so ``padded_target_rows`` is 0."""
    outputs: tuple[tuple[int, ...], ...]
    request_rounds: tuple[tuple[dict, ...], ...]
    wall_ms: float
    prefill_ms: float
    proposal_ms: float
    target_ms: float
    pack_ms: float
    select_commit_ms: float
    physical_target_calls: int
    physical_target_rows: int
    useful_target_rows: int
    padded_target_rows: int
    effective_row_cap_counts: tuple[tuple[int, int], ...]
    effective_tree_budget_counts: tuple[tuple[int, int], ...]
    gated_continuations: int

    @property
    def output_tokens(self) -> int:
        return sum(len(o) for o in self.outputs)

    @property
    def target_calls(self) -> int:
        return self.physical_target_calls

    @property
    def target_rows(self) -> int:
        return self.physical_target_rows


@dataclass(frozen=True)
class WaveRecord:
    """What one wave did, for callers that check or log waves."""
    chosen: tuple
    blocks: tuple
    logits: torch.Tensor
    results: tuple
    keep_rows: tuple
    query_offsets: tuple
    prefix_lengths: tuple
    generator_states: tuple  # each chosen request's generator state before its draws


def continue_existing_tree(ready_count: int, blocks_verified: int, *,
                           continuation_ready_threshold: int | None,
                           max_continuation_blocks: int | None) -> bool:
    """Whether a bonus token that is a tree edge continues in the same tree
    (CTBD:1219-1245): not above ``continuation_ready_threshold`` ready
    requests, and at most ``max_continuation_blocks`` continuations per round.
    Stopping early only commits the already sampled token as the round's
    bonus, so the output law does not change."""
    if ready_count < 1 or blocks_verified < 1:
        raise ValueError("Continuation gate requires positive runtime counts")
    if continuation_ready_threshold is not None and ready_count > continuation_ready_threshold:
        return False
    if max_continuation_blocks is not None and blocks_verified - 1 >= max_continuation_blocks:
        return False
    return True


def commit_tokens(accepted_tokens: Sequence[int], bonus: int, room: int,
                  stops: set[int]) -> list[int]:
    """Tokens a finished round appends (CTBD:2217-2223): the accepted draft
    tokens and the bonus, at most ``room`` of them, cut after the first stop
    id."""
    committed = (list(accepted_tokens) + [int(bonus)])[:room]
    for k, token in enumerate(committed):
        if token in stops:
            return committed[:k + 1]
    return committed


def _cache_length(cache) -> int:
    return int(cache.get_seq_length())


_CONTRACT = "Invalid continuous DDTree/DFlash experiment contract"


class WaveLoop:
    """One packed verification wave at a time over a set of requests.

    ``step(states)`` runs one wave over the given requests (fresh trees for
    those without one, selection, pack, target, verify, commit, token commit)
    and returns the requests it finished.  ``generate_tree_waves`` loops it
    until every request is done; the open-loop serving wrapper interleaves it
    with admissions (``specgrove_amd.serving``).

    ``propose`` is either ``propose(state) -> DraftTree`` (one tree per
    request, budgets ignored) or an object with ``propose_many(states,
    budgets)`` such as ``ddtree.DDTreeProposer`` (one draft pass for every
    request needing a tree, trees of the budgets the occupancy controls or the
    global allocator pick).  The keyword options and their contract are the
    reference's (CTBD:1317-1520) for the packed layout; ``tree_budget`` is the
    variant's tree budget.
    """

    def __init__(self, model, propose, *,
                 max_new_tokens: int, stop_ids: Sequence[int] = (), row_cap: int = 64,
                 row_budget: int | None = None, slot_capacity: int | None = None,
                 persistent: bool = True, capacity: int | None = None, cache_factory=None,
                 tree_budget: int | None = None,
                 low_occupancy_row_cap: int | None = None,
                 low_occupancy_threshold: int | None = None,
                 mid_occupancy_row_cap: int | None = None,
                 mid_occupancy_threshold: int | None = None,
                 proposal_tree_budget: int | None = None,
                 low_occupancy_tree_budget: int | None = None,
                 low_occupancy_tree_threshold: int | None = None,
                 low_occupancy_expansion_slots: int | None = None,
                 adaptive_expansion_requires_drain: bool = False,
                 global_tree_budget_options: Sequence[int] | None = None,
                 global_tree_fixed_row_equivalent: float | None = None,
                 global_tree_row_cost_curve=None,
                 global_tree_require_tier_fit: bool = False,
                 global_tree_expansion_active_limit: int | None = None,
                 global_tree_criticality_weight: float = 0.0,
                 continuation_ready_threshold: int | None = None,
                 max_continuation_blocks: int | None = 0,
                 on_wave: Callable[[WaveRecord], None] | None = None):
        options = (tuple(int(v) for v in global_tree_budget_options)
                   if global_tree_budget_options is not None else None)
        curve = scheduler.normalize_row_cost_curve(global_tree_row_cost_curve)
        adaptive_cap = any(v is not None for v in (low_occupancy_row_cap, low_occupancy_threshold,
                                                   mid_occupancy_row_cap,
                                                   mid_occupancy_threshold))
        budget = tree_budget
        batched = hasattr(propose, "propose_many")
        bad = (
            max_new_tokens < 1 or row_cap < 1
            or (row_budget is not None and row_budget < row_cap)
            or (persistent and capacity is None)
            or (adaptive_cap and (
                low_occupancy_row_cap is None or low_occupancy_threshold is None
                or (mid_occupancy_row_cap is None) != (mid_occupancy_threshold is None)
                or low_occupancy_row_cap < row_cap or low_occupancy_threshold < 1
                or (mid_occupancy_row_cap is not None and (
                    mid_occupancy_row_cap < row_cap
                    or mid_occupancy_row_cap > low_occupancy_row_cap
                    or mid_occupancy_threshold <= low_occupancy_threshold))
                or row_budget is None or row_budget < low_occupancy_row_cap))
            or (continuation_ready_threshold is not None and continuation_ready_threshold < 0)
            or (max_continuation_blocks is not None and max_continuation_blocks < 0)
            or (budget is not None and budget < 1)
            or (batched and options is None and budget is None)
            or (proposal_tree_budget is not None and (
                budget is None or not 1 <= proposal_tree_budget <= budget))
            or ((low_occupancy_tree_budget is None) != (low_occupancy_tree_threshold is None))
            or (low_occupancy_tree_budget is not None and (
                proposal_tree_budget is None
                or not proposal_tree_budget <= low_occupancy_tree_budget <= budget
                or low_occupancy_tree_threshold < 1))
            or (low_occupancy_expansion_slots is not None and (
                low_occupancy_tree_budget is None or low_occupancy_expansion_slots < 1
                or low_occupancy_expansion_slots > low_occupancy_tree_threshold))
            or not isinstance(adaptive_expansion_requires_drain, bool)
            or (options is not None and (
                adaptive_cap or proposal_tree_budget is not None
                or low_occupancy_tree_budget is not None
                or low_occupancy_expansion_slots is not None
                or not options or tuple(sorted(set(options))) != options or options[0] < 1
                or (budget is not None and options[-1] > budget)
                or row_cap != options[0] + 1
                or row_budget is None or options[0] + 1 > row_budget
                or continuation_ready_threshold != 0
                or not isinstance(global_tree_require_tier_fit, bool)
                or (global_tree_expansion_active_limit is not None
                    and global_tree_expansion_active_limit < 1)
                or (global_tree_fixed_row_equivalent is None) == (curve is None)
                or (global_tree_fixed_row_equivalent is not None
                    and (not math.isfinite(global_tree_fixed_row_equivalent)
                         or global_tree_fixed_row_equivalent <= 0))
                or (curve is not None and (curve[0][0] > options[0] + 1
                                           or curve[-1][0] < row_budget))
                or not math.isfinite(global_tree_criticality_weight)
                or global_tree_criticality_weight < 0))
            or (options is None and (
                global_tree_fixed_row_equivalent is not None or curve is not None
                or global_tree_require_tier_fit
                or global_tree_expansion_active_limit is not None
                or global_tree_criticality_weight != 0.0)))
        if bad:
            raise ValueError(_CONTRACT)
        if options is not None and batched and not getattr(propose, "canonical", True):
            raise ValueError("Global budgeting requires canonical DDTree proposal masses")
        self.model, self.propose = model, propose
        self.max_new_tokens, self.stops = max_new_tokens, {int(t) for t in stop_ids}
        self.row_cap, self.row_budget, self.slot_capacity = row_cap, row_budget, slot_capacity
        self.persistent, self.capacity, self.cache_factory = persistent, capacity, cache_factory
        self.tree_budget = budget
        self.low_occupancy_row_cap, self.low_occupancy_threshold = (low_occupancy_row_cap,
                                                                    low_occupancy_threshold)
        self.mid_occupancy_row_cap, self.mid_occupancy_threshold = (mid_occupancy_row_cap,
                                                                    mid_occupancy_threshold)
        self.proposal_tree_budget = proposal_tree_budget
        self.low_occupancy_tree_budget = low_occupancy_tree_budget
        self.low_occupancy_tree_threshold = low_occupancy_tree_threshold
        self.low_occupancy_expansion_slots = low_occupancy_expansion_slots
        self.adaptive_expansion_requires_drain = adaptive_expansion_requires_drain
        self.global_options = options
        self.global_fixed_row_equivalent, self.global_row_cost_curve = (
            global_tree_fixed_row_equivalent, curve)
        self.global_require_tier_fit = global_tree_require_tier_fit
        self.global_expansion_active_limit = global_tree_expansion_active_limit
        self.global_criticality_weight = global_tree_criticality_weight
        self.continuation_ready_threshold = continuation_ready_threshold
        self.max_continuation_blocks = max_continuation_blocks
        self.on_wave = on_wave
        self.device = next(model.parameters()).device
        self.dtype = next(model.parameters()).dtype
        self.pool = None
        self.split_status = (cache_mod.DeviceStatus(self.device, "KV split")
                             if not persistent and self.device.type == "cuda" else None)
        self.expansion_eligible = True
        self.stage = {"prefill": 0.0, "proposal": 0.0, "target": 0.0, "pack": 0.0,
                      "select_commit": 0.0}
        self.calls = 0
        self.rows = 0
        self.useful_rows = 0
        self.row_cap_counts: dict[int, int] = {}
        self.tree_budget_counts: dict[int, int] = {}
        self.gated_continuations = 0

    def attach(self, states: Sequence[DecodeRequest]) -> None:
        """Mark finished requests done and, with a persistent arena, move the
        requests' prefilled caches into one pool (the reference builds the
        pool once after prefill and counts it as prefill, CTBD:1604-1620).
        The occupancy expansions' drain rule is decided on the first call
        (CTBD:1636-1639)."""
        t0 = time.perf_counter()
        for s in states:
            if len(s.generated) >= self.max_new_tokens or (s.generated and
                                                            s.generated[-1] in self.stops):
                s.done = True
        if self.persistent:
            self.pool = cache_mod.PersistentRequestCachePool(
                [s.target_cache for s in states], self.capacity)
            for s, c in zip(states, self.pool.caches):
                s.target_cache = c
        if self.calls == 0 and not self.stage["prefill"]:
            thresholds = tuple(v for v in (self.low_occupancy_threshold,
                                           self.mid_occupancy_threshold,
                                           self.low_occupancy_tree_threshold) if v is not None)
            self.expansion_eligible = scheduler.adaptive_expansion_eligible(
                len(states), thresholds, self.adaptive_expansion_requires_drain)
        self.stage["prefill"] += time.perf_counter() - t0

    def _trees(self, states: Sequence[DecodeRequest], budgets: Sequence[int]) -> list:
        if hasattr(self.propose, "propose_many"):
            return list(self.propose.propose_many(states, budgets))
        return [self.propose(s) for s in states]

    def _propose(self, states: Sequence[DecodeRequest]) -> None:
        """Trees for the requests that need one (CTBD:1640-1739): admission
        and tier allocation under global budgeting, otherwise the occupancy
        tree budgets."""
        active_count = sum(not s.done for s in states)
        fresh = [s for s in states if not s.done and s.tree is None
                 and len(s.generated) < self.max_new_tokens and s.generated[-1] not in self.stops]
        if not fresh:
            return
        if self.global_options is not None:
            wave_options = scheduler.active_global_tree_budget_options(
                self.global_options, active_count=active_count,
                expansion_active_limit=self.global_expansion_active_limit)
            admitted = list(scheduler.admit_global_proposal_states(
                fresh, row_budget=self.row_budget, minimum_tree_budget=self.global_options[0]))
            deferred = len(fresh) - len(admitted)
            if deferred:
                # budget 0 counts deferred admissions, as the reference's telemetry does
                self.tree_budget_counts[0] = self.tree_budget_counts.get(0, 0) + deferred
            taken = {s.request_id for s in admitted}
            for s in fresh:
                if s.request_id not in taken:
                    s.age += 1
            if not admitted:
                return
            options = scheduler.globally_feasible_budget_options(
                wave_options, request_count=len(admitted), row_budget=self.row_budget,
                require_tier_fit=self.global_require_tier_fit)
            full = self._trees(admitted, [options[-1]] * len(admitted))
            candidates = [[scheduler.prefix_tree(t, b) for b in options] for t in full]
            utilities = [[scheduler.draft_tree_expected_tokens(t) for t in c] for c in candidates]
            budgets = scheduler.allocate_global_tree_budgets(
                admitted, options, utilities, row_budget=self.row_budget,
                fixed_row_equivalent=self.global_fixed_row_equivalent,
                criticality_weight=self.global_criticality_weight,
                max_new_tokens=self.max_new_tokens, row_cost_curve=self.global_row_cost_curve)
            index = {b: k for k, b in enumerate(options)}
            trees = [c[index[b]] for c, b in zip(candidates, budgets)]
            chosen = admitted
        else:
            if self.tree_budget is not None:
                eligible = self.expansion_eligible
                budgets = scheduler.effective_tree_budgets(
                    fresh, self.tree_budget, self.proposal_tree_budget,
                    self.low_occupancy_tree_budget if eligible else None,
                    self.low_occupancy_tree_threshold if eligible else None,
                    active_count, self.low_occupancy_expansion_slots)
            else:
                budgets = (None,) * len(fresh)
            trees = self._trees(fresh, budgets)
            chosen = fresh
        for s, tree, b in zip(chosen, trees, budgets):
            s.tree = tree
            s.proposal_tree_budget = b
            s.round_prefix_len = _cache_length(s.target_cache)
            s.block_root = 0
            s.accepted_nodes.clear()
            s.accepted_tokens.clear()
            s.round_block_rows.clear()
            key = int(b) if b is not None else len(tree.tokens)
            self.tree_budget_counts[key] = self.tree_budget_counts.get(key, 0) + 1

    def _select(self, states: Sequence[DecodeRequest]):
        """The wave's requests and blocks under the occupancy row cap
        (CTBD:1740-1766); returns (ready count, chosen, blocks)."""
        ready_count = sum(not s.done and s.tree is not None for s in states)
        eligible = self.expansion_eligible
        cap = scheduler.effective_row_cap(
            self.row_cap, self.low_occupancy_row_cap if eligible else None,
            self.low_occupancy_threshold if eligible else None, ready_count,
            self.mid_occupancy_row_cap if eligible else None,
            self.mid_occupancy_threshold if eligible else None)
        chosen, blocks = scheduler.select_ready(
            states, cap, self.slot_capacity, self.row_budget,
            use_proposal_tree_budget=self.global_options is not None)
        if not chosen:
            raise RuntimeError("No ready request can make progress")
        self.row_cap_counts[cap] = self.row_cap_counts.get(cap, 0) + 1
        return ready_count, chosen, blocks

    def step(self, states: Sequence[DecodeRequest]) -> list[DecodeRequest]:
        """One wave over ``states``; returns the requests it finished."""
        t0 = time.perf_counter()
        self._propose(states)
        self.stage["proposal"] += time.perf_counter() - t0
        t0 = time.perf_counter()
        ready_count, chosen, blocks = self._select(states)
        caches = [s.target_cache for s in chosen]
        packed, lengths, offsets, total = cache_mod.pack_cache_sequence(
            caches, self.cache_factory, self.device)
        ids, positions, mask, qoff = attention.pack_block_inputs(
            chosen, blocks, lengths, offsets, total, self.dtype, self.device)
        self.stage["pack"] += time.perf_counter() - t0

        t0 = time.perf_counter()
        with torch.no_grad():
            hidden = self.model.model(input_ids=ids, position_ids=positions,
                                      attention_mask=mask, past_key_values=packed,
                                      use_cache=True).last_hidden_state
            logits = self.model.get_output_embeddings()(hidden)[0]
        gen_states = tuple(s.generator.get_state() for s in chosen) if self.on_wave else ()
        results = verify.tree_verify_hip_rejection_batched(
            [b.parents for b in blocks], [b.tokens for b in blocks], logits,
            generators=[s.generator for s in chosen], validate=False)
        self.stage["target"] += time.perf_counter() - t0
        self.calls += 1
        wave_rows = sum(len(b.nodes) for b in blocks)
        self.rows += wave_rows
        self.useful_rows += wave_rows

        t0 = time.perf_counter()
        keeps = [[0] + list(nodes) for nodes, _, _ in results]
        if self.pool is not None:
            self.pool.append_packed_sequence(packed, caches, total, qoff, keeps, self.device)
        else:
            if self.split_status is not None:
                self.split_status.check()
            new = cache_mod.split_compacted_sequence_caches(
                packed, self.cache_factory, offsets, lengths, total, qoff, keeps, self.device,
                status=self.split_status)
            for s, c in zip(chosen, new):
                s.target_cache = c
        if self.on_wave is not None:
            self.on_wave(WaveRecord(tuple(chosen), tuple(blocks), logits, tuple(results),
                                    tuple(tuple(k) for k in keeps), tuple(qoff),
                                    tuple(lengths), gen_states))
        finished = []
        for s, block, (local_nodes, local_tokens, bonus) in zip(chosen, blocks, results):
            if self._commit(s, block, local_nodes, local_tokens, bonus, ready_count):
                finished.append(s)
        self.stage["select_commit"] += time.perf_counter() - t0
        return finished

    def _commit(self, s: DecodeRequest, block, local_nodes, local_tokens, bonus,
                ready_count: int) -> bool:
        """Token bookkeeping of one verified block (CTBD:2186-2248); True when
        the request finished."""
        mapped = [block.nodes[n] for n in local_nodes]
        s.round_block_rows.append(len(block.nodes))
        if s.block_root:
            s.accepted_nodes.append(s.block_root)
            s.accepted_tokens.append(s.tree.tokens[s.block_root - 1])
        s.accepted_nodes.extend(mapped)
        s.accepted_tokens.extend(int(t) for t in local_tokens)
        terminal = mapped[-1] if mapped else s.block_root
        nxt = scheduler.child_for_edge(s.tree.parents, s.tree.tokens, terminal, int(bonus))
        if nxt is not None:
            if nxt in block.nodes:
                raise AssertionError("Cascade exited through a verified edge")
            if continue_existing_tree(
                    ready_count, len(s.round_block_rows),
                    continuation_ready_threshold=self.continuation_ready_threshold,
                    max_continuation_blocks=self.max_continuation_blocks):
                s.block_root = nxt
                return False
            self.gated_continuations += 1
        committed = commit_tokens(s.accepted_tokens, bonus,
                                  self.max_new_tokens - len(s.generated), self.stops)
        s.generated.extend(committed)
        s.rounds.append({"committed_tokens": len(committed),
                         "accepted_draft_tokens": len(s.accepted_nodes),
                         "block_rows": list(s.round_block_rows),
                         "continuation_blocks": len(s.round_block_rows) - 1,
                         "gated_continuation": nxt is not None})
        s.tree = None
        s.proposal_tree_budget = None
        s.age = 0
        if len(s.generated) >= self.max_new_tokens or s.generated[-1] in self.stops:
            s.done = True
            return True
        return False

    def check_status(self) -> None:
        """Raise if a commit or split kernel of this loop reported an error."""
        if self.pool is not None:
            self.pool.check_status()
        if self.split_status is not None:
            self.split_status.check()

    def result(self, states: Sequence[DecodeRequest], wall_s: float) -> "DecodeResult":
        """The run's outputs and accounting (CTBD:2252-2270)."""
        return DecodeResult(
            outputs=tuple(tuple(s.generated) for s in states),
            request_rounds=tuple(tuple(s.rounds) for s in states),
            wall_ms=1000 * wall_s, prefill_ms=1000 * self.stage["prefill"],
            proposal_ms=1000 * self.stage["proposal"], target_ms=1000 * self.stage["target"],
            pack_ms=1000 * self.stage["pack"],
            select_commit_ms=1000 * self.stage["select_commit"],
            physical_target_calls=self.calls, physical_target_rows=self.rows,
            useful_target_rows=self.useful_rows, padded_target_rows=self.rows - self.useful_rows,
            effective_row_cap_counts=tuple(sorted(self.row_cap_counts.items())),
            effective_tree_budget_counts=tuple(sorted(self.tree_budget_counts.items())),
            gated_continuations=self.gated_continuations)


def generate_tree_waves(model, states: Sequence[DecodeRequest], propose, *,
                        max_waves: int = 100000, **options) -> DecodeResult:
    """Decode until every request is done, one packed verification wave at a
    time.  ``states`` hold the prefilled target caches (one request each) and
    ``generated == [first sampled token]``; ``model`` is a transformers causal
    LM on the GPU whose attention implementation is ``"specgrove_hip"``.

    ``propose``: see ``WaveLoop``.  Options (``WaveLoop``, named as the
    reference's): ``max_new_tokens``, ``stop_ids``, ``row_cap``,
    ``row_budget``, ``slot_capacity``; ``persistent`` moves the caches into
    one ``PersistentRequestCachePool`` of ``capacity`` tokens per request (the
    reference's ``persistent_request_target_cache``), otherwise every wave
    packs prefixes and splits the caches again; ``tree_budget`` with
    ``proposal_tree_budget``, ``low_occupancy_tree_budget`` /
    ``low_occupancy_tree_threshold`` / ``low_occupancy_expansion_slots``
    size the trees by occupancy; ``low_occupancy_row_cap`` /
    ``low_occupancy_threshold`` / ``mid_occupancy_row_cap`` /
    ``mid_occupancy_threshold`` widen the blocks at low occupancy;
    ``global_tree_budget_options`` (sorted tiers, with ``row_budget``, one
    cost model -- ``global_tree_fixed_row_equivalent`` or
    ``global_tree_row_cost_curve`` -- ``row_cap == options[0] + 1`` and
    ``continuation_ready_threshold == 0``) cuts each fresh tree to the tier
    the allocator picks, and trees then need ``draft_prefix_log_masses``;
    ``continuation_ready_threshold`` / ``max_continuation_blocks`` gate
    continuation blocks; ``on_wave`` receives a ``WaveRecord`` per wave.
    """
    loop = WaveLoop(model, propose, **options)
    wall0 = time.perf_counter()
    loop.attach(states)
    waves = 0
    while not all(s.done for s in states):
        waves += 1
        if waves > max_waves:
            raise RuntimeError("Decode did not finish within max_waves")
        loop.step(states)
    torch.cuda.synchronize(loop.device)
    loop.check_status()
    return loop.result(states, time.perf_counter() - wall0)
