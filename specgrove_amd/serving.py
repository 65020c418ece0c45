"""Open-loop serving over the packed verification waves: requests arrive over
time, are admitted at wave boundaries up to a concurrency limit, and report
queueing, time-to-first-token, per-output-token and end-to-end latencies.

Restates the arrival plumbing of the reference's serving decoder
(code/serving/src/gbv_experiments/continuous_tree_block_decode.py; admission
:1680-1715, prefill at wave boundaries :1557-1622, per-request metrics
:2352-2380) around this repository's wave loop (``decode.WaveLoop``).  As in
the reference (:1526-1531), open-loop serving uses the non-persistent cache
path: every wave packs the admitted requests' prefixes and splits the caches
again, so requests can join and leave between waves.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import Callable, Sequence

import torch

from .decode import DecodeRequest, WaveLoop


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
    while not all(s.done for s in states):
        now = clock() - start
        active = [s for k, s in enumerate(states) if admitted_at[k] is not None and not s.done]
        room = max_active_requests - len(active)
        arrived = [k for k in range(n) if admitted_at[k] is None and arrivals[k] <= now]
        new = arrived[:max(0, room)]
        if new:
            t = clock() - start
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
                         target_calls=loop.calls, target_rows=loop.rows, max_concurrent=peak)
