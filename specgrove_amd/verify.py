"""Temperature-1 tree verifier on the HIP sampler (verifier name
``"hip_tree_rejection"``).

Mirrors the reference's batched logits verifiers
(fused_tree_sampling.py:2468-2533, ``tree_verify_ancestral_logits_fused_scan_batched``,
and the sparse-exit wrapper :2255-2373): the same topology validation
(``_topology``, :2089-2102) with the same exception classes, one uniform draw
per request from the request's own ``torch.Generator``, one kernel launch for
the whole wave and one device-to-host transfer, and the same
``(nodes, tokens, bonus)`` results.

Differences, by design:

* the sampler reads fp32, bf16 or f16 logits and does its own fp32 softmax with the
  reference's law (sampling.py:903-950): routing by ``u[2d]`` over the
  children's cumulative mass, residual draw by ``u[2d+1]`` over the
  complement of the children (fused_tree_sampling.py:683-824); the
  arithmetic is fixed so that the CPU restatement reproduces it bit for bit;
* uniforms are fp32 (``torch.rand(..., dtype=torch.float32)``), and
  ``probability_dtype`` must be ``torch.float32``;
* ragged batches (trees of different sizes and depths) run in one launch:
  ``all_logits`` is either ``[B, N, V]`` (equal trees) or the packed wave
  ``[1, R, V]`` / ``[R, V]`` with the requests' rows in order.
"""
from __future__ import annotations

import array
import itertools
import math
from typing import Sequence

import numpy as np
import torch

from . import ops

VERIFIER_NAME = "hip_tree_rejection"


def _topology(parents, tokens):
    """Validation and depth of one tree (reference fused_tree_sampling.py:2089-2102)."""
    parents = list(parents)
    tokens = list(tokens)
    node_count = len(parents)
    if (node_count < 1 or len(tokens) != node_count - 1
            or parents[0] != -1
            or any(parent < 0 or parent >= node for node, parent in enumerate(parents[1:], 1))
            or len(set(zip(parents[1:], tokens))) != len(tokens)):
        raise ValueError("Invalid probability-tree topology")
    depths = [0] * node_count
    for node in range(1, node_count):
        depths[node] = depths[parents[node]] + 1
    return parents, tokens, max(depths)


def _draw_uniforms(topologies, generators, device):
    """Each request's 2*(depth+1) fp32 uniforms from its own generator (the
    reference's per-request draw), written straight into its row of one
    [n, 2*(max_depth+1)] tensor; returns (uniforms, max_depth)."""
    max_depth = max(depth for _, _, depth in topologies)
    uniforms = torch.zeros((len(topologies), 2 * (max_depth + 1)), dtype=torch.float32,
                           device=device)
    for i, ((_, _, depth), generator) in enumerate(zip(topologies, generators)):
        torch.rand(2 * (depth + 1), dtype=torch.float32, device=device, generator=generator,
                   out=uniforms[i, :2 * (depth + 1)])
    return uniforms, max_depth


_SIDE_STREAMS: dict = {}


def _draw_uniforms_beside(topologies, generators, device):
    """_draw_uniforms on a side stream (default priority, one per device), so
    that the per-request draws -- many tiny launches -- run beside the work
    already queued on the current stream instead of after it.  They read
    nothing the current stream writes (a generator's state lives on the host)
    and write only their own new tensor, so the side stream waits for
    nothing; the current stream waits for them before anything it enqueues
    later."""
    main = torch.cuda.current_stream(device)
    side = _SIDE_STREAMS.get(main.device_index)
    if side is None:
        side = _SIDE_STREAMS[main.device_index] = torch.cuda.Stream(device)
    with torch.cuda.stream(side):
        uniforms, max_depth = _draw_uniforms(topologies, generators, device)
    main.wait_stream(side)
    uniforms.record_stream(main)
    return uniforms, max_depth


def tree_verify_hip_rejection_batched(parents_batch: Sequence[Sequence[int]],
                                      tokens_batch: Sequence[Sequence[int]],
                                      all_logits: torch.Tensor, temperature: float = 1.0,
                                      probability_dtype=torch.float32, generators=None,
                                      validate: bool = True):
    """Sample every request's accepted path and bonus token in one launch.

    Returns a list of ``(nodes, tokens, bonus)``: accepted local node ids in
    root-to-leaf order, their tokens, and the bonus (residual) token.
    """
    count = len(parents_batch)
    if (count < 1 or len(tokens_batch) != count or generators is None
            or len(generators) != count or not isinstance(all_logits, torch.Tensor)
            or not all_logits.is_cuda or not all_logits.is_floating_point()):
        raise ValueError("Batched tree-rejection inputs are inconsistent")
    if (not isinstance(temperature, (float, int)) or not math.isfinite(float(temperature))
            or float(temperature) != 1.0):
        raise ValueError("The HIP tree verifier samples at temperature 1")
    if probability_dtype != torch.float32:
        raise ValueError("The HIP tree verifier uses fp32 probability arithmetic")
    topologies = [_topology(p, t) for p, t in zip(parents_batch, tokens_batch)]
    rows = [len(p) for p, _, _ in topologies]
    total = sum(rows)
    if all_logits.dim() == 3 and all_logits.shape[0] == count and count > 1:
        if any(r != all_logits.shape[1] for r in rows):
            raise ValueError("Batched tree-rejection tensor shape mismatch")
        logits = all_logits.reshape(count * all_logits.shape[1], all_logits.shape[2])
    elif all_logits.dim() == 3 and all_logits.shape[0] == 1:
        logits = all_logits[0]
    elif all_logits.dim() == 2:
        logits = all_logits
    elif all_logits.dim() == 3 and count == 1:
        logits = all_logits[0]
    else:
        raise ValueError("Batched tree-rejection tensor shape mismatch")
    if logits.shape[0] != total or logits.shape[1] < 1:
        raise ValueError("Batched tree-rejection tensor shape mismatch")
    vocab = logits.shape[1]
    if any(token < 0 or token >= vocab for _, tokens, _ in topologies for token in tokens):
        raise ValueError("Tree token is outside the Target vocabulary")
    # fp32, bf16 and f16 rows are read as they are (the 16-bit types widen to
    # fp32 exactly inside the kernels); other types are rounded to fp32.
    if logits.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        logits = logits.float()
    if logits.stride(1) != 1 or logits.stride(0) < logits.shape[1]:
        logits = logits.contiguous()
    if validate and not bool(torch.isfinite(logits).all()):
        raise FloatingPointError("Invalid Target logits for the HIP tree verifier")

    device = logits.device
    # Beside the work that produces the logits, when that is still running.
    uniforms, max_depth = _draw_uniforms_beside(topologies, generators, device)
    row_offset = np.zeros(count + 1, np.int32)
    np.cumsum(rows, out=row_offset[1:])
    parent = np.concatenate([np.asarray(p, np.int32) for p, _, _ in topologies])
    token = np.concatenate([np.asarray([-1] + list(t), np.int32) for _, t, _ in topologies])
    meta = torch.from_numpy(np.concatenate([row_offset, parent, token])).to(device)
    n1 = count + 1
    result = ops.tree_sample(logits, meta[:n1], meta[n1:n1 + total], meta[n1 + total:],
                             uniforms, max_depth)
    # One device-to-host transfer for the whole wave.
    host = torch.cat([result.accept_len, result.bonus, result.accept_nodes.reshape(-1),
                      result.status]).tolist()
    lengths, bonuses = host[:count], host[count:2 * count]
    nodes_flat = host[2 * count:2 * count + count * result.accept_nodes.shape[1]]
    if host[-1] != 0:
        raise RuntimeError("HIP tree sampler returned invalid control values")
    width = result.accept_nodes.shape[1]
    results = []
    for i, ((_, tokens, depth), accepted, bonus) in enumerate(zip(topologies, lengths, bonuses)):
        if not 0 <= accepted <= depth or not 0 <= bonus < vocab:
            raise RuntimeError("HIP tree sampler returned invalid control values")
        nodes = [int(v) for v in nodes_flat[i * width:i * width + accepted]]
        results.append((nodes, [tokens[node - 1] for node in nodes], int(bonus)))
    return results


def tree_verify_hip_rejection(parents, tokens, all_logits: torch.Tensor,
                              generator=None, validate: bool = True):
    """Per-request convention ``f(parents, tokens, values[rows, V], generator,
    validate) -> (nodes, tokens, bonus)`` (reference sampling.py:903-950)."""
    return tree_verify_hip_rejection_batched([parents], [tokens], all_logits,
                                             generators=[generator], validate=validate)[0]


LAZY_VERIFIER_NAME = "hip_lazy_projection"


def _head_weight(lm_head):
    """The [V, H] bf16 weight of an ``nn.Linear`` vocabulary head (no bias),
    the weight tensor itself, or its ``ops.PackedLmHead`` (used as it is)."""
    if isinstance(lm_head, ops.PackedLmHead):
        return lm_head
    weight = getattr(lm_head, "weight", lm_head)
    if getattr(lm_head, "bias", None) is not None:
        raise ValueError("The HIP lazy projection supports a vocabulary head without bias")
    if (not isinstance(weight, torch.Tensor) or weight.dim() != 2 or not weight.is_cuda
            or weight.dtype != torch.bfloat16):
        raise ValueError("The HIP lazy projection needs a bf16 [V, H] head weight on the GPU")
    return weight if weight.stride(1) == 1 else weight.contiguous()


def _lazy_hidden(final_hidden: torch.Tensor, count: int, rows: Sequence[int], weight):
    """The packed [R, H] rows of final_hidden when its shape fits the trees'
    row counts and the head's hidden size, else None (the caller's checks
    raise)."""
    total = sum(rows)
    hidden_size = final_hidden.shape[-1]
    if final_hidden.dim() == 3 and final_hidden.shape[0] == count and count > 1:
        if any(r != final_hidden.shape[1] for r in rows):
            return None
        hidden = final_hidden.reshape(count * final_hidden.shape[1], hidden_size)
    elif final_hidden.dim() == 3 and final_hidden.shape[0] == 1:
        hidden = final_hidden[0]
    elif final_hidden.dim() == 2:
        hidden = final_hidden
    else:
        return None
    if hidden.shape[0] != total or hidden_size != weight.shape[1]:
        return None
    return hidden if hidden.stride(1) == 1 else hidden.contiguous()


def _lazy_rows(parents_batch):
    """From the trees' parent lists alone: row_offset [n+1], parent [R] and
    the internal rows' packed indices (nodes with a child), which is all the
    internal-row projection needs.  Edges that are not parent < node are
    skipped, so lists that the topology check would reject still give
    in-range indices; raises TypeError or ValueError when the lists do not
    convert to integers."""
    rows = [len(p) for p in parents_batch]
    count = len(rows)
    if count < 1 or min(rows) < 1:
        raise ValueError("not a batch of trees")
    total = sum(rows)
    row_offset = np.zeros(count + 1, np.int32)
    np.cumsum(rows, out=row_offset[1:])
    # One pass over the Python lists (int32 range enforced by fromiter).
    parent = np.fromiter(itertools.chain.from_iterable(parents_batch), np.int32, total)
    gpar = parent + np.repeat(row_offset[:-1], rows)  # packed index of each parent
    edge = (parent >= 0) & (gpar < np.arange(total, dtype=np.int32))
    internal = np.zeros(total, bool)
    internal[gpar[edge]] = True
    return row_offset, parent, np.flatnonzero(internal).astype(np.int32)


def _lazy_meta(parents_batch, tokens_batch, rows=None):
    """The lazy walk's packed metadata from the trees' parent and token lists:
    row_offset [n+1], parent [R], token [R] (-1 at each root), row_map [R]
    (each node's row among the projected internal rows, else -1), the
    internal rows' packed indices, and each row's request.  ``rows``: the
    result of _lazy_rows for the same parents, when already computed.  Raises
    TypeError or ValueError when the lists do not convert to integers."""
    row_offset, parent, internal_rows = rows if rows is not None else _lazy_rows(parents_batch)
    count = row_offset.size - 1
    total = int(row_offset[-1])
    owner = np.repeat(np.arange(count, dtype=np.int32), np.diff(row_offset))
    if len(tokens_batch) != count or sum(len(t) for t in tokens_batch) != total - count:
        raise ValueError("not a batch of trees")
    # array.fromlist converts each list in one C loop (int32 range enforced).
    token = array.array("i")
    for t in tokens_batch:
        token.append(-1)
        token.fromlist(t if isinstance(t, list) else list(t))
    token = np.frombuffer(token, np.int32)
    row_map = np.full(total, -1, np.int32)
    row_map[internal_rows] = np.arange(internal_rows.size, dtype=np.int32)
    return row_offset, parent, token, row_map, internal_rows, owner


def tree_verify_hip_lazy_projection_batched(parents_batch: Sequence[Sequence[int]],
                                            tokens_batch: Sequence[Sequence[int]],
                                            final_hidden: torch.Tensor, lm_head,
                                            temperature: float = 1.0,
                                            probability_dtype=torch.float32,
                                            generators=None, validate: bool = True):
    """Lazy vocabulary projection with exact sparse-exit routing on the HIP
    kernels (reference ``tree_verify_ancestral_lazy_projection_sparse_exit_batched``,
    fused_tree_sampling.py:2840-3031; law sampling.py:738-832).

    All internal rows of the wave (nodes with children) are projected by one
    ``sg_lm_head`` call, whose epilogue leaves their softmax statistics; the
    walks route on them, and a walk that reaches a leaf leaves it for a second
    projection of only the reached leaves, from whose rows the bonus is drawn
    (``u[2d+1]`` over the whole row).  The output law is that of projecting
    every row: a leaf row cannot influence which leaf is reached.

    ``final_hidden`` is ``[B, N, H]`` (equal trees, as the reference) or the
    packed wave ``[R, H]`` / ``[1, R, H]``; ``lm_head`` an ``nn.Linear``
    without bias, its bf16 ``[V, H]`` weight, or that weight packed once by
    ``ops.pack_lm_head`` (same results, faster weight reads).  Returns, per request,
    ``(nodes, tokens, bonus, stats)`` with the reference's projection counts.
    """
    count = len(parents_batch)
    if (count < 1 or len(tokens_batch) != count or generators is None
            or len(generators) != count or not isinstance(final_hidden, torch.Tensor)
            or not final_hidden.is_cuda or final_hidden.dtype != torch.bfloat16):
        raise ValueError("Batched lazy-projection inputs are inconsistent")
    if (not isinstance(temperature, (float, int)) or not math.isfinite(float(temperature))
            or float(temperature) != 1.0):
        raise ValueError("The HIP lazy projection samples at temperature 1")
    if probability_dtype != torch.float32:
        raise ValueError("The HIP lazy projection uses fp32 probability arithmetic")
    weight = _head_weight(lm_head)
    # The wave's metadata is copied to the device (a synchronous copy, while
    # nothing of this call is queued yet) and the internal-row projection is
    # started before the host-side validation below, so that the two overlap.
    # The row indices come from the unvalidated parents (non-edges skipped,
    # every index in range; the kernel also bounds-checks each one); an
    # invalid call then raises below, with the same errors in the same order,
    # before anything is sampled.
    # Only the internal rows (from the parent lists) come before the launch;
    # the tokens and the walk's other metadata are built while the GPU
    # projects, and reach it by a non-blocking copy from pinned memory queued
    # behind the projection (a pageable copy there would hold the host until
    # the projection ends).
    early, early_meta, early_head = None, None, None
    try:
        early_hidden = _lazy_hidden(final_hidden, count, [len(p) for p in parents_batch], weight)
        if early_hidden is not None:
            early_rows = _lazy_rows(parents_batch)
            if early_rows[2].size:
                early_head = ops.lm_head(early_hidden, weight,
                                         torch.from_numpy(early_rows[2]).to(early_hidden.device))
            early = _lazy_meta(parents_batch, tokens_batch, early_rows)
            early_meta = torch.from_numpy(np.concatenate(early[:5])).pin_memory().to(
                early_hidden.device, non_blocking=True)
    except (TypeError, ValueError, OverflowError):
        early, early_meta, early_head = None, None, None  # the checks below raise
    topologies = [_topology(p, t) for p, t in zip(parents_batch, tokens_batch)]
    rows = [len(p) for p, _, _ in topologies]
    total = sum(rows)
    hidden_size = final_hidden.shape[-1]
    if final_hidden.dim() == 3 and final_hidden.shape[0] == count and count > 1:
        if any(r != final_hidden.shape[1] for r in rows):
            raise ValueError("Batched lazy-projection hidden shape mismatch")
        hidden = final_hidden.reshape(count * final_hidden.shape[1], hidden_size)
    elif final_hidden.dim() == 3 and final_hidden.shape[0] == 1:
        hidden = final_hidden[0]
    elif final_hidden.dim() == 2:
        hidden = final_hidden
    else:
        raise ValueError("Batched lazy-projection hidden shape mismatch")
    if hidden.shape[0] != total or hidden_size != weight.shape[1]:
        raise ValueError("Batched lazy-projection hidden shape mismatch")
    if hidden.stride(1) != 1:
        hidden = hidden.contiguous()
    vocab = weight.shape[0]
    if any(token < 0 or token >= vocab for _, tokens, _ in topologies for token in tokens):
        raise ValueError("Tree token is outside the Target vocabulary")

    device = hidden.device
    # Internal nodes (those with children) in ascending packed order.  The
    # trees are valid now, so the metadata built before the checks is theirs.
    if early_meta is not None:
        row_offset, parent, token, row_map, internal_rows, owner = early
        meta = early_meta
    else:
        row_offset, parent, token, row_map, internal_rows, owner = _lazy_meta(
            [p for p, _, _ in topologies], [t for _, t, _ in topologies])
        meta = torch.from_numpy(np.concatenate([row_offset, parent, token, row_map,
                                                internal_rows])).to(device)
    internal_counts = np.bincount(owner[internal_rows], minlength=count).tolist()
    n1 = count + 1
    meta_row_offset = meta[:n1]
    meta_parent = meta[n1:n1 + total]
    meta_token = meta[n1 + total:n1 + 2 * total]
    meta_row_map = meta[n1 + 2 * total:n1 + 3 * total]
    meta_internal = meta[n1 + 3 * total:]

    def projection_check(head: "ops.LmHeadResult") -> torch.Tensor:
        """[head status, valid]: the head's status word (0 = every row index
        in range) always; with ``validate`` also 1 when the statistics are
        finite with positive sums.  The statistics checks (a few reductions)
        are skipped without ``validate``, as the reference skips its."""
        if not validate:
            return head.status.reshape(1)
        ok = (torch.isfinite(head.row_max).all() & torch.isfinite(head.row_sum).all()
              & (head.row_sum > 0).all())
        return torch.cat([head.status.reshape(1), ok.to(torch.int32).reshape(1)])

    if internal_rows.size:
        head = early_head if early_head is not None else ops.lm_head(hidden, weight,
                                                                     meta_internal)
    # Drawn after the projection is enqueued, on a side stream: their host
    # work and their tiny kernels both overlap the projection.
    uniforms, max_depth = _draw_uniforms_beside(topologies, generators, device)
    if internal_rows.size:
        logits, row_max, row_sum = head.logits, head.row_max, head.row_sum
        check = projection_check(head)
    else:  # no tree has an edge: every walk ends at its (unprojected) root
        logits = torch.zeros((1, vocab), dtype=torch.bfloat16, device=device)
        row_max = torch.zeros(1, dtype=torch.float32, device=device)
        row_sum = torch.ones(1, dtype=torch.float32, device=device)
        check = torch.tensor([0, 1][:2 if validate else 1], dtype=torch.int32, device=device)
    result = ops.tree_sample_projected(logits, meta_row_offset, meta_parent, meta_token,
                                       uniforms, max_depth, row_max=row_max, row_sum=row_sum,
                                       row_map=meta_row_map)
    # One device-to-host transfer for the walks.
    width = result.accept_nodes.shape[1]
    host = torch.cat([result.accept_len, result.bonus, result.terminal_leaf,
                      result.accept_nodes.reshape(-1), result.status, check]).tolist()
    lengths = host[:count]
    bonuses = host[count:2 * count]
    leaves = host[2 * count:3 * count]
    nodes_flat = host[3 * count:3 * count + count * width]
    tail = host[3 * count + count * width:]  # sampler status, head status[, valid]
    if tail[1] != 0:
        raise RuntimeError("HIP LM head reported an out-of-range row index")
    if validate and tail[2] != 1:
        raise FloatingPointError("Invalid batched internal probabilities")
    if tail[0] != 0:
        raise RuntimeError("HIP tree sampler returned invalid control values")

    leaf_requests = [i for i in range(count) if leaves[i] >= 0]
    if leaf_requests:
        # Second projection: the reached leaves only; each draws its bonus from
        # the whole row with its exit uniform u[2d+1] (a one-node walk).
        m = len(leaf_requests)
        leaf_rows = [int(row_offset[i]) + leaves[i] for i in leaf_requests]
        exit_cols = [2 * lengths[i] + 1 for i in leaf_requests]
        leaf_meta = torch.tensor(leaf_rows + list(range(m + 1)) + [-1] * m + [0] * m
                                 + leaf_requests + exit_cols, dtype=torch.int32)
        leaf_meta = leaf_meta.to(device)
        leaf_index = leaf_meta[:m]
        single_offset = leaf_meta[m:2 * m + 1]
        single_parent = leaf_meta[2 * m + 1:3 * m + 1]
        single_token = leaf_meta[3 * m + 1:4 * m + 1]
        req_idx = leaf_meta[4 * m + 1:5 * m + 1].long()
        col_idx = leaf_meta[5 * m + 1:].long()
        leaf_uniforms = torch.zeros((m, 2), dtype=torch.float32, device=device)
        leaf_uniforms[:, 1] = uniforms[req_idx, col_idx]
        leaf_head = ops.lm_head(hidden, weight, leaf_index)
        leaf = ops.tree_sample_projected(leaf_head.logits, single_offset, single_parent,
                                         single_token, leaf_uniforms, 0,
                                         row_max=leaf_head.row_max, row_sum=leaf_head.row_sum)
        leaf_host = torch.cat([leaf.bonus, leaf.accept_len, leaf.status,
                               projection_check(leaf_head)]).tolist()
        leaf_tail = leaf_host[2 * m:]  # sampler status, head status[, valid]
        if leaf_tail[1] != 0:
            raise RuntimeError("HIP LM head reported an out-of-range row index")
        if validate and leaf_tail[2] != 1:
            raise FloatingPointError("Invalid lazy-projection leaf probabilities")
        if leaf_tail[0] != 0 or any(v != 0 for v in leaf_host[m:2 * m]):
            raise RuntimeError("HIP tree sampler returned invalid control values")
        for i, bonus in zip(leaf_requests, leaf_host[:m]):
            bonuses[i] = bonus

    results = []
    for i, ((parents, tokens, depth), accepted, bonus) in enumerate(
            zip(topologies, lengths, bonuses)):
        if not 0 <= accepted <= depth or not 0 <= bonus < vocab:
            raise RuntimeError("HIP tree sampler returned invalid control values")
        nodes = [int(v) for v in nodes_flat[i * width:i * width + accepted]]
        if leaves[i] >= 0 and leaves[i] != (nodes[-1] if nodes else 0):
            raise RuntimeError("HIP tree sampler returned an invalid leaf")
        leaf_projected = int(leaves[i] >= 0)
        results.append((nodes, [tokens[node - 1] for node in nodes], int(bonus), {
            "internal_projected_rows": internal_counts[i],
            "leaf_projected_rows": leaf_projected,
            "projected_rows": internal_counts[i] + leaf_projected,
            "total_tree_rows": rows[i],
            "lm_head_rows": internal_counts[i] + leaf_projected,
            "probability_rows": internal_counts[i] + leaf_projected,
            "physical_internal_projection_rows": int(internal_rows.size),
            "sparse_exit": True,
        }))
    return results
