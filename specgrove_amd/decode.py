"""The packed verification wave loop on the drop-in path.

Restates the verify-and-commit core of the reference's decoder
``generate_continuous_tree_blocks`` (paths relative to the reference snapshot:
CTBD = code/natural/src/gbv_experiments/continuous_tree_block_decode.py; wave
loop :1640-2248) with this repository's plugs in every slot:

  proposals   a caller-supplied ``propose(state) -> DraftTree`` (the
              reference's draft model and DDTree builder, out of scope here),
              optionally cut to tiers by the global tier allocator
              (``scheduler.allocate_global_tree_budgets``, CTBD:706-795);
  selection   ``scheduler.select_ready`` (CTBD:1158-1195);
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
own caches are the proposer's business and are not restated.
"""
from __future__ import annotations

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
    """Outputs and accounting of a decode (the reference's
    ``ContinuousDecodeResult``, CTBD:103-123, fields on this path)."""
    outputs: tuple[tuple[int, ...], ...]
    request_rounds: tuple[tuple[dict, ...], ...]
    wall_ms: float
    target_ms: float
    pack_ms: float
    select_commit_ms: float
    target_calls: int
    target_rows: int

    @property
    def output_tokens(self) -> int:
        return sum(len(o) for o in self.outputs)


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


class WaveLoop:
    """One packed verification wave at a time over a set of requests.

    ``step(states)`` runs one wave over the given requests (fresh trees for
    those without one, selection, pack, target, verify, commit, token commit)
    and returns the requests it finished.  ``generate_tree_waves`` loops it
    until every request is done; the open-loop serving wrapper interleaves it
    with admissions (``specgrove_amd.serving``).
    """

    def __init__(self, model, propose: Callable[[DecodeRequest], scheduler.DraftTree], *,
                 max_new_tokens: int, stop_ids: Sequence[int] = (), row_cap: int = 64,
                 row_budget: int | None = None, slot_capacity: int | None = None,
                 persistent: bool = True, capacity: int | None = None, cache_factory=None,
                 global_tiers: Sequence[int] | None = None,
                 fixed_row_equivalent: float | None = None, row_cost_curve=None,
                 criticality_weight: float = 0.0,
                 continuation_ready_threshold: int | None = None,
                 max_continuation_blocks: int | None = 0,
                 on_wave: Callable[[WaveRecord], None] | None = None):
        if max_new_tokens < 1 or row_cap < 1:
            raise ValueError("max_new_tokens and row_cap must be positive")
        if persistent and capacity is None:
            raise ValueError("A persistent arena needs a capacity")
        if global_tiers is not None and row_budget is None:
            raise ValueError("Global tiers need a row budget")
        self.model, self.propose = model, propose
        self.max_new_tokens, self.stops = max_new_tokens, {int(t) for t in stop_ids}
        self.row_cap, self.row_budget, self.slot_capacity = row_cap, row_budget, slot_capacity
        self.persistent, self.capacity, self.cache_factory = persistent, capacity, cache_factory
        self.global_tiers = global_tiers
        self.fixed_row_equivalent, self.row_cost_curve = fixed_row_equivalent, row_cost_curve
        self.criticality_weight = criticality_weight
        self.continuation_ready_threshold = continuation_ready_threshold
        self.max_continuation_blocks = max_continuation_blocks
        self.on_wave = on_wave
        self.device = next(model.parameters()).device
        self.dtype = next(model.parameters()).dtype
        self.pool = None
        self.stage = {"target": 0.0, "pack": 0.0, "select_commit": 0.0}
        self.calls = 0
        self.rows = 0

    def attach(self, states: Sequence[DecodeRequest]) -> None:
        """Mark finished requests done and, with a persistent arena, move the
        requests' prefilled caches into one pool (the reference builds the
        pool once after prefill, CTBD:1604-1620)."""
        for s in states:
            if len(s.generated) >= self.max_new_tokens or (s.generated and
                                                            s.generated[-1] in self.stops):
                s.done = True
        if self.persistent:
            self.pool = cache_mod.PersistentRequestCachePool(
                [s.target_cache for s in states], self.capacity)
            for s, c in zip(states, self.pool.caches):
                s.target_cache = c

    def _propose(self, states: Sequence[DecodeRequest]) -> None:
        fresh = [s for s in states if not s.done and s.tree is None]
        for s in fresh:
            s.tree = self.propose(s)
            s.proposal_tree_budget = None
            s.round_prefix_len = _cache_length(s.target_cache)
            s.block_root = 0
            s.accepted_nodes.clear()
            s.accepted_tokens.clear()
            s.round_block_rows.clear()
        if self.global_tiers is None or not fresh:
            return
        options = scheduler.globally_feasible_budget_options(
            self.global_tiers, request_count=len(fresh), row_budget=self.row_budget,
            require_tier_fit=False)
        utilities = [[scheduler.draft_tree_expected_tokens(scheduler.prefix_tree(s.tree, b))
                      for b in options] for s in fresh]
        tiers = scheduler.allocate_global_tree_budgets(
            fresh, options, utilities, row_budget=self.row_budget,
            fixed_row_equivalent=self.fixed_row_equivalent,
            criticality_weight=self.criticality_weight, max_new_tokens=self.max_new_tokens,
            row_cost_curve=self.row_cost_curve)
        for s, b in zip(fresh, tiers):
            s.tree = scheduler.prefix_tree(s.tree, b)
            s.proposal_tree_budget = b

    def step(self, states: Sequence[DecodeRequest]) -> list[DecodeRequest]:
        """One wave over ``states``; returns the requests it finished."""
        t0 = time.perf_counter()
        self._propose(states)
        chosen, blocks = scheduler.select_ready(
            states, self.row_cap, self.slot_capacity, self.row_budget,
            use_proposal_tree_budget=self.global_tiers is not None)
        if not chosen:
            raise RuntimeError("No ready request fits the wave's row budget")
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
        self.rows += sum(len(b.nodes) for b in blocks)

        t0 = time.perf_counter()
        keeps = [[0] + list(nodes) for nodes, _, _ in results]
        if self.pool is not None:
            self.pool.append_packed_sequence(packed, caches, total, qoff, keeps, self.device)
        else:
            new = cache_mod.split_compacted_sequence_caches(
                packed, self.cache_factory, offsets, lengths, total, qoff, keeps, self.device)
            for s, c in zip(chosen, new):
                s.target_cache = c
        if self.on_wave is not None:
            self.on_wave(WaveRecord(tuple(chosen), tuple(blocks), logits, tuple(results),
                                    tuple(tuple(k) for k in keeps), tuple(qoff),
                                    tuple(lengths), gen_states))
        finished = []
        for s, block, (local_nodes, local_tokens, bonus) in zip(chosen, blocks, results):
            if self._commit(s, block, local_nodes, local_tokens, bonus, len(chosen)):
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


def generate_tree_waves(model, states: Sequence[DecodeRequest],
                        propose: Callable[[DecodeRequest], scheduler.DraftTree], *,
                        max_waves: int = 100000, **options) -> DecodeResult:
    """Decode until every request is done, one packed verification wave at a
    time.  ``states`` hold the prefilled target caches (one request each) and
    ``generated == [first sampled token]``; ``model`` is a transformers causal
    LM on the GPU whose attention implementation is ``"specgrove_hip"``.

    Options (``WaveLoop``): ``max_new_tokens``, ``stop_ids``, ``row_cap``,
    ``row_budget``, ``slot_capacity``; ``persistent`` moves the caches into
    one ``PersistentRequestCachePool`` of ``capacity`` tokens per request (the
    reference's ``persistent_request_target_cache``), otherwise every wave
    packs prefixes and splits the caches again; ``global_tiers`` (sorted tier
    sizes, with ``row_budget`` and one cost model, ``fixed_row_equivalent``
    or ``row_cost_curve``) cuts each fresh tree to the tier the allocator
    picks, and trees then need ``draft_prefix_log_masses``;
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
    return DecodeResult(
        outputs=tuple(tuple(s.generated) for s in states),
        request_rounds=tuple(tuple(s.rounds) for s in states),
        wall_ms=1000 * (time.perf_counter() - wall0),
        target_ms=1000 * loop.stage["target"], pack_ms=1000 * loop.stage["pack"],
        select_commit_ms=1000 * loop.stage["select_commit"],
        target_calls=loop.calls, target_rows=loop.rows)
