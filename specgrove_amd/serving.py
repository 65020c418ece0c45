"""Open-loop serving over the packed verification waves: requests arrive over
time, are admitted at wave boundaries up to a concurrency limit, and report
queueing, time-to-first-token, per-output-token and end-to-end latencies.

Restates the arrival plumbing of the reference's serving decoder
(code/serving/src/gbv_experiments/continuous_tree_block_decode.py, SCTBD
below; admission :1680-1715, prefill at wave boundaries :1557-1622,
per-request metrics :2352-2380) around this repository's wave loop
(``decode.WaveLoop``).  As in the reference (:1526-1531), open-loop serving
uses the non-persistent cache path: every wave packs the admitted requests'
prefixes and splits the caches again, so requests can join and leave between
waves.

``PackedPrefill`` is the reference's ``batched_prefill`` (:1557-1609) on this
path: the newly admitted prompts run through the target in one packed
sequence, each prompt a causal chain of rows (parent = previous token) for the
tree attention kernel -- in chunks of at most 256 rows per request, each chunk
attending to the request's earlier chunks as its cached prefix -- and each
request's first token is drawn from its last prompt row by the tree sampler as
a one-node walk with the request's generator.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import Callable, Sequence

import numpy as np
import torch

from . import attention, cache as cache_mod, verify
from .decode import DecodeRequest, WaveLoop

_CHUNK_ROWS = 256  # rows per request and prefill chunk (the attention kernel's tree limit)


class PackedPrefill:
    """Prefill of newly admitted requests in packed waves (SCTBD:1557-1609).

    ``PackedPrefill(model, prompts)(new_states)`` fills every state's
    ``target_cache`` (a ``cache_factory()`` cache, ``RequestCache`` by
    default) with its prompt's K/V and sets ``generated = [first token]``,
    drawn at temperature 1 from the last prompt row's logits with the
    request's generator (the same law as the reference's ``sample(
    probabilities(...))``; the draw is the sampler's one-node walk, so it
    consumes two uniforms of the generator).  ``model`` is the causal LM with
    ``attn_implementation="specgrove_hip"``; ``prompts[request_id]`` are the
    prompt token lists.  ``on_chunk`` (optional) receives, per packed prefill
    wave, the chunk's request ids, row counts and logits of the requests'
    final rows with the generator states before the draws (for checking the
    draws).
    """

    def __init__(self, model, prompts, cache_factory=None, on_chunk=None):
        self.model, self.prompts = model, prompts
        self.cache_factory, self.on_chunk = cache_factory, on_chunk
        self.seconds = 0.0

    def __call__(self, states: Sequence[DecodeRequest]) -> None:
        if not states:
            return
        t0 = time.perf_counter()
        model = self.model
        device = next(model.parameters()).device
        cfg = model.config
        hkv = cfg.num_key_value_heads
        dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        dtype = next(model.parameters()).dtype
        prompts = [list(self.prompts[s.request_id]) for s in states]
        if any(len(p) < 1 for p in prompts):
            raise ValueError("Each prompt must have at least one token")
        caches: list = [None] * len(states)
        done = [0] * len(states)
        while True:
            wave = [i for i, p in enumerate(prompts) if done[i] < len(p)]
            if not wave:
                break
            rows = [min(_CHUNK_ROWS, len(prompts[i]) - done[i]) for i in wave]
            lengths = [done[i] for i in wave]
            layers = cfg.num_hidden_layers
            keys, values = [], []
            for layer in range(layers):
                parts_k = [caches[i].layers[layer].keys[0] for i in wave if caches[i] is not None]
                parts_v = [caches[i].layers[layer].values[0] for i in wave if caches[i] is not None]
                if parts_k:
                    keys.append(torch.cat(parts_k, dim=1).contiguous())
                    values.append(torch.cat(parts_v, dim=1).contiguous())
                else:  # no request has a cached prefix yet: nothing is read from it
                    keys.append(torch.zeros((hkv, 1, dim), dtype=dtype, device=device))
                    values.append(torch.zeros((hkv, 1, dim), dtype=dtype, device=device))
            prefix = cache_mod.PackedPrefix(keys, values)
            packed = cache_mod.TreeVerifyCache(None, [object() for _ in wave], prefix, lengths)
            parents = [[-1] + list(range(r - 1)) for r in rows]
            mask = attention.build_tree_mask(prefix, None, parents, device,
                                             prefix_start=packed.prefix_starts,
                                             prefix_len=lengths)
            ids = np.concatenate([prompts[i][done[i]:done[i] + r] for i, r in zip(wave, rows)])
            pos = np.concatenate([np.arange(done[i], done[i] + r) for i, r in zip(wave, rows)])
            with torch.no_grad():
                hidden = model.model(
                    input_ids=torch.from_numpy(ids.astype(np.int64)).to(device)[None],
                    position_ids=torch.from_numpy(pos.astype(np.int64)).to(device)[None],
                    attention_mask={"full_attention": mask}, past_key_values=packed,
                    use_cache=True).last_hidden_state[0]
            offsets = np.concatenate([[0], np.cumsum(rows)[:-1]]).tolist()
            new = cache_mod.split_compacted_sequence_caches(
                packed, self.cache_factory, packed.prefix_starts, lengths, packed.prefix_total,
                offsets, [list(range(r)) for r in rows], device)
            for i, c in zip(wave, new):
                caches[i] = c
            finishing = [(k, i) for k, i in enumerate(wave) if done[i] + rows[k] == len(prompts[i])]
            if finishing:
                last = torch.tensor([offsets[k] + rows[k] - 1 for k, _ in finishing],
                                    device=device)
                with torch.no_grad():
                    logits = model.get_output_embeddings()(hidden.index_select(0, last))
                gens = [states[i].generator for _, i in finishing]
                if self.on_chunk is not None:
                    self.on_chunk([states[i].request_id for _, i in finishing], rows, logits,
                                  [g.get_state() for g in gens])
                draws = verify.tree_verify_hip_rejection_batched(
                    [[-1]] * len(finishing), [[]] * len(finishing), logits,
                    generators=gens, validate=False)
                for (_, i), (_, _, anchor) in zip(finishing, draws):
                    states[i].generated = [int(anchor)]
            for k, i in enumerate(wave):
                done[i] += rows[k]
        for s, c in zip(states, caches):
            s.target_cache = c
        self.seconds += time.perf_counter() - t0


@dataclass(frozen=True)
class ServingResult:
    """Outputs and per-request timing of an open-loop run (the reference's
    ``request_metrics``: arrival, admission, first token and completion times
    in ms from the start, and queue, TTFT, end-to-end, service and TPOT)."""
    outputs: tuple[tuple[int, ...], ...]
    request_metrics: tuple[dict, ...]
    wall_ms: float
    target_calls: int
    target_rows: int
    max_concurrent: int
    admissions: tuple[dict, ...] = ()


def serve_open_loop(model, states: Sequence[DecodeRequest],
                    arrival_times_s: Sequence[float],
                    propose, prefill: Callable[[Sequence[DecodeRequest]], None], *,
                    max_active_requests: int, clock: Callable[[], float] = time.perf_counter,
                    sleep: Callable[[float], None] = time.sleep, **loop_options) -> ServingResult:
    """Serve ``states`` arriving at ``arrival_times_s`` (seconds from the
    start, non-decreasing).

    At every wave boundary the requests that have arrived are admitted in
    arrival order while fewer than ``max_active_requests`` are active;
    ``prefill(new_states)`` then fills each one's ``target_cache`` with its
    prompt and sets ``generated = [first token]`` (the reference samples it
    from the prefill logits), which is the request's first-token time.  The
    admitted, unfinished requests then run one wave of ``WaveLoop`` (options
    as for ``decode.generate_tree_waves``; ``persistent`` must be False).
    With nothing active, the loop sleeps until the next arrival.

    ``admissions`` records every wave boundary that admitted requests: its
    time, the active count before it, the requests that had arrived and were
    waiting, and the ones admitted (the first ``max_active_requests - active``
    of the waiting ones in arrival order, SCTBD:1684-1694).
    """
    arrivals = tuple(float(v) for v in arrival_times_s)
    if (len(arrivals) != len(states) or not states
            or any(not math.isfinite(v) or v < 0 for v in arrivals)
            or tuple(sorted(arrivals)) != arrivals
            or max_active_requests is None or max_active_requests < 1
            or loop_options.get("persistent", False)):
        raise ValueError("Invalid open-loop serving contract")
    loop = WaveLoop(model, propose, persistent=False, **{
        k: v for k, v in loop_options.items() if k != "persistent"})
    n = len(states)
    admitted_at: list[float | None] = [None] * n
    first_at: list[float | None] = [None] * n
    done_at: list[float | None] = [None] * n
    index = {id(s): k for k, s in enumerate(states)}
    start = clock()
    peak = 0
    log: list[dict] = []
    while not all(s.done for s in states):
        now = clock() - start
        active = [s for k, s in enumerate(states) if admitted_at[k] is not None and not s.done]
        room = max_active_requests - len(active)
        arrived = [k for k in range(n) if admitted_at[k] is None and arrivals[k] <= now]
        new = arrived[:max(0, room)]
        if new:
            t = clock() - start
            log.append({"at_ms": 1000 * now, "active_before": len(active),
                        "waiting": tuple(states[k].request_id for k in arrived),
                        "admitted": tuple(states[k].request_id for k in new)})
            for k in new:
                admitted_at[k] = t
            prefill([states[k] for k in new])
            torch.cuda.synchronize(loop.device)
            t = clock() - start
            for k in new:
                first_at[k] = t
            loop.attach([states[k] for k in new])
            for k in new:
                if states[k].done:
                    done_at[k] = t
        active = [s for k, s in enumerate(states) if admitted_at[k] is not None and not s.done]
        peak = max(peak, len(active))
        if not active:
            pending = [arrivals[k] for k in range(n) if admitted_at[k] is None]
            if not pending:
                break
            sleep(max(0.0, min(pending) - (clock() - start)))
            continue
        finished = loop.step(active)
        if finished:
            torch.cuda.synchronize(loop.device)
            t = clock() - start
            for s in finished:
                done_at[index[id(s)]] = t
    wall = clock() - start
    loop.check_status()
    if any(v is None for v in admitted_at + first_at + done_at):
        raise RuntimeError("Open-loop request timing is incomplete")
    metrics = []
    for k, s in enumerate(states):
        tokens = len(s.generated)
        metrics.append({
            "request_id": s.request_id,
            "arrival_ms": 1000 * arrivals[k],
            "admitted_ms": 1000 * admitted_at[k],
            "first_token_ms": 1000 * first_at[k],
            "completed_ms": 1000 * done_at[k],
            "queue_ms": 1000 * (admitted_at[k] - arrivals[k]),
            "ttft_ms": 1000 * (first_at[k] - arrivals[k]),
            "e2e_ms": 1000 * (done_at[k] - arrivals[k]),
            "service_ms": 1000 * (done_at[k] - admitted_at[k]),
            "tpot_ms": 1000 * (done_at[k] - first_at[k]) / (tokens - 1) if tokens > 1 else 0.0,
            "output_tokens": tokens,
        })
    return ServingResult(outputs=tuple(tuple(s.generated) for s in states),
                         request_metrics=tuple(metrics), wall_ms=1000 * wall,
                         target_calls=loop.calls, target_rows=loop.rows, max_concurrent=peak,
                         admissions=tuple(log))
