"""Seeded synthetic workloads for the packed verification path.

Shapes follow the five workloads the path is measured on:
  tiny      2-layer Qwen3-style decoder (hidden 256, 4 q / 2 kv heads, D 64,
            vocab 4096), 4 requests, 16-row random trees, prefixes 32-96;
  qwen3_4b  one attention layer, 32 q / 8 kv heads, D 128, 16 requests,
            prefixes U{256..2048}, tiers {16,32,64} of a 64-node canonical tree,
            512-row budget;
  qwen3_8b  one attention layer, 32 q / 8 kv heads, D 128, 64 requests,
            prefixes U{512..4096}, tiers {16,32,64,128} of a 128-node canonical
            tree (branching 1-4, depth <= 16), 2048-row budget, then a KV commit
            of 1 + a_i rows, a_i ~ U{1..8};
  sampler   64 requests x 32 nodes, vocab 151936, fp32 logits N(0, 3^2) with 1-5
            peaks +12, draft q = 0.7 softmax + 0.3 Dirichlet(0.1);
  long_ctx  128 requests, prefixes log-uniform [8192, 32768], tiers
            {1,16,32,64,128} weighted {.1,.2,.3,.25,.15}, 4096-row budget;
  tier128   the qwen3_8b shape with 16 requests all at the 128-node tier.

Row convention: a tier of k nodes is k packed rows including the root (row 0
of a request block is the newest committed token, as ids = [root] + tokens in
the reference's packed inputs, continuous_tree_block_decode.py:521-532).  When
the seeded tiers exceed the row budget, the largest tier is downgraded (ties:
lowest request id) until the wave fits.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch


# --------------------------------------------------------------------------
# trees
# --------------------------------------------------------------------------

def canonical_tree(num_nodes: int, rng: np.random.Generator, max_branch: int = 4,
                   max_depth: int = 16) -> list[int]:
    """BFS-ordered tree: each node in turn gets 1..max_branch children."""
    parents = [-1]
    depths = [0]
    frontier = 0
    while len(parents) < num_nodes:
        if frontier >= len(parents):
            raise RuntimeError("tree generation ran out of expandable nodes")
        if depths[frontier] < max_depth:
            branch = int(rng.integers(1, max_branch + 1))
            for _ in range(branch):
                if len(parents) == num_nodes:
                    break
                parents.append(frontier)
                depths.append(depths[frontier] + 1)
        frontier += 1
    return parents


def random_parent_tree(num_nodes: int, rng: np.random.Generator,
                       max_depth: int = 8) -> list[int]:
    """Node j >= 1 takes a parent uniformly among earlier nodes of depth < cap."""
    parents = [-1]
    depths = [0]
    for _ in range(1, num_nodes):
        candidates = [v for v in range(len(parents)) if depths[v] < max_depth]
        p = int(candidates[int(rng.integers(0, len(candidates)))])
        parents.append(p)
        depths.append(depths[p] + 1)
    return parents


def depths_of(parents) -> list[int]:
    depths = [0] * len(parents)
    for k in range(1, len(parents)):
        depths[k] = depths[parents[k]] + 1
    return depths


def random_tokens(parents, vocab: int, rng: np.random.Generator) -> list[int]:
    """Uniform draft tokens, distinct among the children of each parent.

    Raises ValueError when a parent has more children than the vocabulary has
    tokens (no distinct assignment exists)."""
    fanout: dict[int, int] = {}
    for k in range(1, len(parents)):
        fanout[parents[k]] = fanout.get(parents[k], 0) + 1
    if fanout and max(fanout.values()) > vocab:
        raise ValueError(f"a parent has {max(fanout.values())} children but the vocabulary "
                         f"has only {vocab} tokens")
    used: dict[int, set[int]] = {}
    tokens = []
    for k in range(1, len(parents)):
        seen = used.setdefault(parents[k], set())
        while True:
            t = int(rng.integers(0, vocab))
            if t not in seen:
                break
        seen.add(t)
        tokens.append(t)
    return tokens


def downgrade_tiers(tiers, options, budget: int) -> list[int]:
    """Downgrade the largest tier (lowest request id first) until sum <= budget."""
    options = sorted(options)
    tiers = list(tiers)
    while sum(tiers) > budget:
        biggest = max(tiers)
        if biggest == options[0]:
            raise ValueError("row budget cannot hold the smallest tiers")
        i = tiers.index(biggest)
        tiers[i] = options[options.index(biggest) - 1]
    return tiers


def random_path(parents, length: int, rng: np.random.Generator) -> list[int]:
    """Root-to-node path of up to ``length`` accepted nodes (local ids)."""
    children: dict[int, list[int]] = {}
    for k in range(1, len(parents)):
        children.setdefault(parents[k], []).append(k)
    path = []
    node = 0
    for _ in range(length):
        kids = children.get(node)
        if not kids:
            break
        node = int(kids[int(rng.integers(0, len(kids)))])
        path.append(node)
    return path


# --------------------------------------------------------------------------
# packed attention workloads
# --------------------------------------------------------------------------

@dataclass
class AttentionWorkload:
    name: str
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    prefix_len: np.ndarray            # [n] int32
    parents: list[list[int]]          # request-local parents per request
    tokens: list[list[int]]
    capacity: int                     # cache tokens per request slot
    keep: list[list[int]] = field(default_factory=list)  # [0] + accepted path

    @property
    def num_requests(self) -> int:
        return len(self.parents)

    @property
    def rows(self) -> np.ndarray:
        return np.asarray([len(p) for p in self.parents], np.int32)

    @property
    def row_offset(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.rows)]).astype(np.int32)

    @property
    def total_rows(self) -> int:
        return int(self.rows.sum())

    @property
    def parent_flat(self) -> np.ndarray:
        return np.concatenate([np.asarray(p, np.int32) for p in self.parents]).astype(np.int32)

    @property
    def prefix_start(self) -> np.ndarray:
        return (np.arange(self.num_requests, dtype=np.int64) * self.capacity).astype(np.int64)

    def algorithmic_bytes(self) -> int:
        """Prefix K+V read once, Q read, O written, tree K+V read (bf16)."""
        d = self.head_dim
        kv_prefix = int(self.prefix_len.sum()) * self.num_kv_heads * d * 2 * 2
        q_o = self.total_rows * self.num_q_heads * d * 2 * 2
        tree_kv = self.total_rows * self.num_kv_heads * d * 2 * 2
        meta = 4 * (self.total_rows + 3 * self.num_requests)
        return kv_prefix + q_o + tree_kv + meta

    def algorithmic_flops(self) -> int:
        """4*Hq*D per visible (query row, key) pair: QK^T and PV."""
        visible = 0
        for length, parents in zip(self.prefix_len, self.parents):
            depths = depths_of(parents)
            visible += len(parents) * int(length) + sum(d + 1 for d in depths)
        return 4 * self.num_q_heads * self.head_dim * visible

    def commit_bytes(self) -> int:
        rows = sum(len(k) for k in self.keep)
        return 2 * rows * self.num_kv_heads * self.head_dim * 2 * 2

    def make_tensors(self, device, seed: int, q_scale: float | None = None,
                     tree_scale: float = 1.0):
        """Q [R,Hq,D], cache K/V [Hkv, n*capacity, D], tree K/V [R,Hkv,D] (bf16).

        Values: K/V ~ N(0,1), Q ~ N(0,1)/sqrt(D) unless q_scale is given.
        Generated with a torch generator on ``device``.
        """
        gen = torch.Generator(device=device).manual_seed(seed)
        d = self.head_dim
        q_scale = (1.0 / math.sqrt(d)) if q_scale is None else q_scale
        r = self.total_rows
        bf16 = torch.bfloat16
        q = (torch.randn((r, self.num_q_heads, d), generator=gen, device=device) * q_scale).to(bf16)
        k_cache = torch.randn((self.num_kv_heads, self.num_requests * self.capacity, d),
                              generator=gen, device=device, dtype=bf16)
        v_cache = torch.randn((self.num_kv_heads, self.num_requests * self.capacity, d),
                              generator=gen, device=device, dtype=bf16)
        k_tree = (torch.randn((r, self.num_kv_heads, d), generator=gen, device=device)
                  * tree_scale).to(bf16)
        v_tree = torch.randn((r, self.num_kv_heads, d), generator=gen, device=device, dtype=bf16)
        return q, k_cache, v_cache, k_tree, v_tree


def _tiered_workload(name, seed, num_requests, prefix_lo, prefix_hi, tier_options,
                     tier_weights, budget, canonical_nodes, num_q_heads=32, num_kv_heads=8,
                     head_dim=128, log_uniform=False, accept_max=8, vocab=151936):
    rng = np.random.default_rng(seed)
    if log_uniform:
        lengths = np.exp(rng.uniform(math.log(prefix_lo), math.log(prefix_hi), num_requests))
        lengths = np.floor(lengths).astype(np.int32)
    else:
        lengths = rng.integers(prefix_lo, prefix_hi + 1, num_requests).astype(np.int32)
    canonical = canonical_tree(canonical_nodes, rng)
    weights = None if tier_weights is None else np.asarray(tier_weights) / np.sum(tier_weights)
    tiers = [int(t) for t in rng.choice(tier_options, size=num_requests, p=weights)]
    tiers = downgrade_tiers(tiers, tier_options, budget)
    parents = [canonical[:k] for k in tiers]
    tokens = [random_tokens(p, vocab, rng) for p in parents]
    keep = []
    for p in parents:
        a = int(rng.integers(1, accept_max + 1))
        keep.append([0] + random_path(p, a, rng))
    capacity = int(lengths.max()) + max(tier_options) + accept_max + 1
    capacity = (capacity + 63) // 64 * 64
    return AttentionWorkload(name, num_q_heads, num_kv_heads, head_dim, lengths, parents,
                             tokens, capacity, keep)


def qwen3_4b_workload(seed: int = 2) -> AttentionWorkload:
    return _tiered_workload("qwen3_4b_attn_16req_512rows", seed, 16, 256, 2048, [16, 32, 64],
                            None, 512, 64)


def qwen3_8b_workload(seed: int = 3) -> AttentionWorkload:
    return _tiered_workload("qwen3_8b_attn_64req_2048rows", seed, 64, 512, 4096,
                            [16, 32, 64, 128], None, 2048, 128)


def tier128_workload(seed: int = 6) -> AttentionWorkload:
    """Qwen3-8B attention shape with every request at the 128-node tier: 16
    requests, prefixes U{512..4096}, 2048 rows (the MFMA-heaviest units)."""
    return _tiered_workload("qwen3_8b_attn_16req_tier128", seed, 16, 512, 4096, [128], None,
                            2048, 128)


def long_context_workload(seed: int = 5) -> AttentionWorkload:
    return _tiered_workload("qwen3_8b_attn_128req_4096rows_8k32k", seed, 128, 8192, 32768,
                            [1, 16, 32, 64, 128], [0.1, 0.2, 0.3, 0.25, 0.15], 4096, 128,
                            log_uniform=True)


def tiny_attention_workload(seed: int = 1, num_requests: int = 4, rows: int = 16,
                            prefix_lo: int = 32, prefix_hi: int = 96, num_q_heads: int = 4,
                            num_kv_heads: int = 2, head_dim: int = 64,
                            vocab: int = 4096) -> AttentionWorkload:
    rng = np.random.default_rng(seed)
    lengths = rng.integers(prefix_lo, prefix_hi + 1, num_requests).astype(np.int32)
    parents = [random_parent_tree(rows, rng, max_depth=8) for _ in range(num_requests)]
    tokens = [random_tokens(p, vocab, rng) for p in parents]
    keep = [[0] + random_path(p, int(rng.integers(1, 9)), rng) for p in parents]
    capacity = (int(lengths.max()) + rows + 16 + 63) // 64 * 64
    return AttentionWorkload(f"tiny_attn_{num_requests}req", num_q_heads, num_kv_heads,
                             head_dim, lengths, parents, tokens, capacity, keep)


# --------------------------------------------------------------------------
# sampler workloads
# --------------------------------------------------------------------------

@dataclass
class SamplerWorkload:
    name: str
    vocab: int
    parents: list[list[int]]
    tokens: list[list[int]]

    @property
    def row_offset(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum([len(p) for p in self.parents])]).astype(np.int32)

    @property
    def total_rows(self) -> int:
        return int(sum(len(p) for p in self.parents))

    @property
    def max_depth(self) -> int:
        return max(max(depths_of(p)) for p in self.parents)

    @property
    def uniform_stride(self) -> int:
        return 2 * (self.max_depth + 1)

    def flat_parent_token(self):
        parent = np.concatenate([np.asarray(p, np.int32) for p in self.parents])
        token = np.concatenate([np.asarray([0] + list(t), np.int32) for t in self.tokens])
        return parent.astype(np.int32), token.astype(np.int32)

    def algorithmic_bytes(self) -> int:
        return self.total_rows * self.vocab * 4


def sampler_workload(device, seed: int = 4, num_requests: int = 64, nodes: int = 32,
                     vocab: int = 151936, peaks_max: int = 5, peak_boost: float = 12.0,
                     logit_std: float = 3.0, draft_mix: float = 0.3, alpha: float = 0.1):
    """Target logits and draft trees whose child tokens are drawn from q.

    Returns (workload, logits [R, V] fp32 on ``device``, uniforms [n, U] fp32
    on ``device``).  Children of a node are distinct tokens drawn without
    replacement from that node's draft distribution
    q = (1 - draft_mix) * softmax(target) + draft_mix * Dirichlet(alpha).
    """
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    parents = [canonical_tree(nodes, rng) for _ in range(num_requests)]
    rows = num_requests * nodes
    logits = torch.randn((rows, vocab), generator=gen, device=device) * logit_std
    peaks = rng.integers(1, peaks_max + 1, rows)
    peak_rows = np.repeat(np.arange(rows), peaks)
    peak_cols = rng.integers(0, vocab, int(peaks.sum()))
    logits[torch.as_tensor(peak_rows, device=device),
           torch.as_tensor(peak_cols, device=device)] += peak_boost
    tokens = []
    for i, p in enumerate(parents):
        kids: dict[int, list[int]] = {}
        for k in range(1, len(p)):
            kids.setdefault(p[k], []).append(k)
        tok = [0] * (len(p) - 1)
        for v, children in kids.items():
            row = logits[i * nodes + v]
            conc = torch.full((vocab,), alpha, device=device)
            gam = torch._standard_gamma(conc, generator=gen)
            q = (1.0 - draft_mix) * torch.softmax(row, 0) + draft_mix * gam / gam.sum()
            draws = torch.multinomial(q, len(children), replacement=False,
                                      generator=gen).tolist()
            for child, t in zip(children, draws):
                tok[child - 1] = int(t)
        tokens.append(tok)
    wl = SamplerWorkload(f"sampler_{num_requests}x{nodes}_v{vocab}", vocab, parents, tokens)
    uniforms = torch.from_numpy(
        rng.random((num_requests, wl.uniform_stride), dtype=np.float32)).to(device)
    return wl, logits.contiguous(), uniforms
