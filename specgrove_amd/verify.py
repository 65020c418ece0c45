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
    max_depth = max(depth for _, _, depth in topologies)
    stride = 2 * (max_depth + 1)
    uniforms = torch.zeros((count, stride), dtype=torch.float32, device=device)
    for i, ((_, _, depth), generator) in enumerate(zip(topologies, generators)):
        uniforms[i, :2 * (depth + 1)] = torch.rand(2 * (depth + 1), dtype=torch.float32,
                                                   device=device, generator=generator)
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
