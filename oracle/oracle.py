"""CPU oracle for the packed tree-verification path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` may import this module; the product package
(``specgrove_amd``) never does.  Every function restates the reference's
semantics on the CPU and cites the reference file it follows (paths relative
to the reference snapshot, ``CTBD`` = code/natural/src/gbv_experiments/
continuous_tree_block_decode.py).

Parts:
  * packing  -- ancestor visibility (tree.py:19-26) and the dense additive
                packed mask / ids / positions (CTBD:500-546);
  * attention -- textbook masked softmax attention in fp32 on bf16-valued
                inputs, GQA head h -> kv head h // (Hq/Hkv) as transformers'
                repeat_kv (dense packed mode = the reference wave; per-request
                mode = the same math restricted to a request's own keys);
  * commit   -- the persistent-arena scatter of CTBD:215-261 with the keep rule
                of CTBD:2108-2109;
  * sampling -- ctypes binding of sg_oracle.c (explicit-uniform tree rejection
                sampler, law of sampling.py:903-950) plus the ancestral walk of
                sampling.py:937-950 on pre-drawn posterior tokens;
  * LM head  -- the statistics epilogue of the lazy projection and the walk
                over a partly projected wave (fused_tree_sampling.py:2840-3019,
                sampling.py:738-832), also in sg_oracle.c.
"""
from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path
from typing import Sequence

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libsg_oracle.so"
_lib = None


def build_oracle_library() -> Path:
    """Compile sg_oracle.c with the committed Makefile (gcc only)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build_oracle_library()
        handle = ctypes.CDLL(str(_LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        handle.sgo_exp.restype = ctypes.c_float
        handle.sgo_exp.argtypes = [ctypes.c_float]
        handle.sgo_exp_array.restype = None
        handle.sgo_exp_array.argtypes = [f32p, f32p, ctypes.c_int64]
        handle.sgo_row_stats.restype = None
        handle.sgo_row_stats.argtypes = [f32p, ctypes.c_int64, f32p, f32p]
        handle.sgo_complement_draw.restype = ctypes.c_int32
        handle.sgo_complement_draw.argtypes = [
            f32p, ctypes.c_int64, ctypes.c_float, i32p, ctypes.c_int,
            ctypes.c_float, f32p,
        ]
        handle.sgo_tree_sample.restype = ctypes.c_int
        handle.sgo_tree_sample.argtypes = [
            f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, i32p, i32p,
            i32p, f32p, ctypes.c_int32, ctypes.c_int32, i32p, i32p, i32p,
            f32p, f32p,
        ]
        handle.sgo_tree_sample_mapped.restype = ctypes.c_int
        handle.sgo_tree_sample_mapped.argtypes = [
            f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, i32p, i32p,
            i32p, f32p, ctypes.c_int32, ctypes.c_int32, i32p, f32p, f32p,
            i32p, i32p, i32p, i32p,
        ]
        handle.sgo_rows_slab_stats.restype = None
        handle.sgo_rows_slab_stats.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_int32, f32p, f32p, f32p]
        handle.sgo_slab_draw.restype = ctypes.c_int32
        handle.sgo_slab_draw.argtypes = [
            f32p, ctypes.c_int64, ctypes.c_float, f32p, i32p, ctypes.c_int,
            ctypes.c_float, f32p,
        ]
        handle.sgo_lm_head_tile_stats.restype = None
        handle.sgo_lm_head_tile_stats.argtypes = [f32p, ctypes.c_int64, f32p]
        handle.sgo_lm_head_row_stats.restype = None
        handle.sgo_lm_head_row_stats.argtypes = [f32p, ctypes.c_int64, f32p, f32p]
        _lib = handle
    return _lib


def _f32p(array: np.ndarray):
    return array.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _i32p(array: np.ndarray):
    return array.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


# --------------------------------------------------------------------------
# Sampling (sg_oracle.c)
# --------------------------------------------------------------------------

def exp_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().sgo_exp_array(_f32p(x), _f32p(out), x.size)
    return out


def row_stats(row: np.ndarray) -> tuple[float, float]:
    row = np.ascontiguousarray(row, dtype=np.float32)
    m = np.zeros(1, np.float32)
    z = np.zeros(1, np.float32)
    lib().sgo_row_stats(_f32p(row), row.size, _f32p(m), _f32p(z))
    return float(m[0]), float(z[0])


def slab_stats(logits: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Row statistics of the sampler's own statistics pass (sg_oracle.c,
    sgo_row_slab_stats): per row (max, sum of exp) and, per 2048-token slab,
    (m_s, Z_s) -- the slab max and its sum of E(x - m_s)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, vocab = logits.shape
    slabs = (vocab + 2047) // 2048
    m = np.zeros(rows, np.float32)
    z = np.zeros(rows, np.float32)
    ss = np.zeros((rows, slabs, 2), np.float32)
    lib().sgo_rows_slab_stats(_f32p(logits), vocab, vocab, rows, _f32p(m), _f32p(z), _f32p(ss))
    return m, z, ss


def slab_draw(row: np.ndarray, m: float, row_slab_stats: np.ndarray,
              child_tokens: Sequence[int], u: float) -> tuple[int, float]:
    """The exit draw from one row's slab statistics (sgo_slab_draw): the
    bonus token and the complement total C."""
    row = np.ascontiguousarray(row, dtype=np.float32)
    ss = np.ascontiguousarray(row_slab_stats, dtype=np.float32)
    children = np.ascontiguousarray(np.asarray(child_tokens, np.int32))
    total = np.zeros(1, np.float32)
    token = lib().sgo_slab_draw(_f32p(row), row.size, np.float32(m), _f32p(ss),
                                _i32p(children), children.size, np.float32(u), _f32p(total))
    return int(token), float(total[0])


def complement_draw(row: np.ndarray, m: float, child_tokens: Sequence[int],
                    u: float) -> tuple[int, float]:
    row = np.ascontiguousarray(row, dtype=np.float32)
    children = np.ascontiguousarray(np.asarray(child_tokens, np.int32))
    total = np.zeros(1, np.float32)
    token = lib().sgo_complement_draw(
        _f32p(row), row.size, np.float32(m), _i32p(children), children.size,
        np.float32(u), _f32p(total),
    )
    return int(token), float(total[0])


def tree_sample(logits: np.ndarray, row_offset: np.ndarray, parent: np.ndarray,
                token: np.ndarray, uniforms: np.ndarray, max_depth: int,
                threads: int = 1):
    """Oracle for the packed sampler.

    ``logits`` [rows, V] fp32, ``row_offset`` [n+1], ``parent``/``token``
    [rows] int32 (request-local parent, -1 root), ``uniforms`` [n, U] fp32.
    Statistics are computed here, as the sampler's own pass computes them,
    and the exit draw is the slab draw (sgo_slab_draw).  Returns
    (accept_nodes [n, max_depth], accept_len [n], bonus [n], row_m [rows],
    row_z [rows]).  Requests are independent, so ``threads`` > 1
    runs contiguous groups of requests in parallel C calls (same results).
    """
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    row_offset = np.ascontiguousarray(row_offset, dtype=np.int32)
    parent = np.ascontiguousarray(parent, dtype=np.int32)
    token = np.ascontiguousarray(token, dtype=np.int32)
    uniforms = np.ascontiguousarray(uniforms, dtype=np.float32)
    n = row_offset.size - 1
    rows = int(row_offset[-1])
    if logits.ndim != 2 or logits.shape[0] < rows or int(row_offset[0]) != 0:
        raise ValueError("logits do not cover the packed rows")
    depth_slots = max(int(max_depth), 1)
    nodes = np.full((n, depth_slots), -1, np.int32)
    length = np.zeros(n, np.int32)
    bonus = np.zeros(n, np.int32)
    row_m = np.zeros(rows, np.float32)
    row_z = np.zeros(rows, np.float32)
    vocab = logits.shape[1]

    def run(a: int, b: int) -> int:
        r0, r1 = int(row_offset[a]), int(row_offset[b])
        ro = np.ascontiguousarray(row_offset[a:b + 1] - r0)
        return lib().sgo_tree_sample(
            _f32p(logits[r0:r1]), vocab, vocab, b - a, _i32p(ro),
            _i32p(parent[r0:r1]), _i32p(token[r0:r1]), _f32p(uniforms[a:b]),
            uniforms.shape[1], int(max_depth), _i32p(nodes[a:b]), _i32p(length[a:b]),
            _i32p(bonus[a:b]), _f32p(row_m[r0:r1]), _f32p(row_z[r0:r1]),
        )

    if threads > 1 and n > 1:
        from concurrent.futures import ThreadPoolExecutor
        bounds = np.linspace(0, n, min(threads, n) + 1).astype(int)
        with ThreadPoolExecutor(len(bounds) - 1) as pool:  # ctypes releases the GIL
            statuses = list(pool.map(run, bounds[:-1], bounds[1:]))
    else:
        statuses = [run(0, n)] if n > 0 else [0]
    if any(status != 0 for status in statuses):
        raise ValueError("oracle sampler rejected its inputs")
    return nodes[:, :max_depth], length, bonus, row_m, row_z


def _parallel(count: int, threads: int, fn) -> None:
    """fn(a, b) over contiguous index ranges (ctypes releases the GIL)."""
    if count <= 0:
        return
    if threads > 1 and count > 1:
        from concurrent.futures import ThreadPoolExecutor
        bounds = np.linspace(0, count, min(threads, count) + 1).astype(int)
        with ThreadPoolExecutor(len(bounds) - 1) as pool:
            list(pool.map(fn, bounds[:-1], bounds[1:]))
    else:
        fn(0, count)


def lm_head_stats(logits: np.ndarray, threads: int = 1):
    """Statistics of the LM head's epilogue for fp32 rows ``logits`` [rows, V]
    (the bf16 logits the kernel wrote, widened): per-row 128-token tile pairs
    [rows, ceil(V/128), 2] and the merged row max / sum (sg_oracle.c:
    sgo_lm_head_tile_stats, sgo_lm_head_row_stats)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, vocab = logits.shape
    tiles = (vocab + 127) // 128
    pairs = np.zeros((rows, tiles, 2), np.float32)
    row_m = np.zeros(rows, np.float32)
    row_z = np.zeros(rows, np.float32)

    def run(a: int, b: int) -> None:
        for r in range(a, b):
            lib().sgo_lm_head_tile_stats(_f32p(logits[r]), vocab, _f32p(pairs[r]))
            lib().sgo_lm_head_row_stats(_f32p(pairs[r]), tiles, _f32p(row_m[r:r + 1]),
                                        _f32p(row_z[r:r + 1]))
    _parallel(rows, threads, run)
    return pairs, row_m, row_z


def tree_sample_mapped(logits: np.ndarray, row_offset: np.ndarray, parent: np.ndarray,
                       token: np.ndarray, uniforms: np.ndarray, max_depth: int,
                       row_map: np.ndarray | None, row_m: np.ndarray | None,
                       row_z: np.ndarray | None, threads: int = 1):
    """Oracle of the sampler over a partly projected wave.

    ``logits`` [logits rows, V] fp32; ``row_map`` [rows] gives each packed
    node's logits row (-1: not projected, only for nodes without children;
    None: row r); ``row_m``/``row_z`` [logits rows] are given statistics (the
    LM head's; the exit is then the complement draw, sgo_complement_draw) or
    None (computed as the sampler's own pass does, with the slab draw).  Returns
    (accept_nodes [n, max_depth], accept_len [n], bonus [n], terminal_leaf [n]);
    bonus is -1 where the walk ended at an unprojected leaf.
    """
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    row_offset = np.ascontiguousarray(row_offset, dtype=np.int32)
    parent = np.ascontiguousarray(parent, dtype=np.int32)
    token = np.ascontiguousarray(token, dtype=np.int32)
    uniforms = np.ascontiguousarray(uniforms, dtype=np.float32)
    n = row_offset.size - 1
    rows = int(row_offset[-1])
    vocab = logits.shape[1]
    if row_map is None:
        row_map = np.arange(rows, dtype=np.int32)
    row_map = np.ascontiguousarray(row_map, dtype=np.int32)
    if row_map.size != rows or row_map.max(initial=-1) >= logits.shape[0]:
        raise ValueError("row map does not fit the logits")
    given = row_m is not None and row_z is not None
    if given:
        row_m = np.ascontiguousarray(row_m, dtype=np.float32)
        row_z = np.ascontiguousarray(row_z, dtype=np.float32)
    depth_slots = max(int(max_depth), 1)
    nodes = np.full((n, depth_slots), -1, np.int32)
    length = np.zeros(n, np.int32)
    bonus = np.zeros(n, np.int32)
    leaf = np.full(n, -1, np.int32)
    statuses = []

    def run(a: int, b: int) -> None:
        r0, r1 = int(row_offset[a]), int(row_offset[b])
        ro = np.ascontiguousarray(row_offset[a:b + 1] - r0)
        statuses.append(lib().sgo_tree_sample_mapped(
            _f32p(logits), vocab, vocab, b - a, _i32p(ro),
            _i32p(parent[r0:r1]), _i32p(token[r0:r1]), _f32p(uniforms[a:b]),
            uniforms.shape[1], int(max_depth), _i32p(row_map[r0:r1]),
            _f32p(row_m) if given else None, _f32p(row_z) if given else None,
            _i32p(nodes[a:b]), _i32p(length[a:b]), _i32p(bonus[a:b]), _i32p(leaf[a:b])))
    _parallel(n, threads, run)
    if any(status != 0 for status in statuses):
        raise ValueError("oracle sampler rejected its inputs")
    return nodes[:, :max_depth], length, bonus, leaf


def ancestral_walk(parents: Sequence[int], tokens: Sequence[int],
                   posterior_tokens: Sequence[int]):
    """Tree walk of sampling.py:937-950 on pre-drawn per-node tokens."""
    children = {
        (int(parents[node]), int(tokens[node - 1])): node
        for node in range(1, len(parents))
    }
    nodes, accepted = [], []
    node = 0
    bonus = int(posterior_tokens[node])
    while (node, bonus) in children:
        node = children[node, bonus]
        nodes.append(node)
        accepted.append(bonus)
        bonus = int(posterior_tokens[node])
    return nodes, accepted, bonus


# --------------------------------------------------------------------------
# Packing (tree.py:19-26, CTBD:500-546)
# --------------------------------------------------------------------------

def visibility(parents: Sequence[int]) -> np.ndarray:
    """Ancestor-or-self matrix, row i = row parent[i] plus the diagonal."""
    n = len(parents)
    visible = np.zeros((n, n), dtype=bool)
    visible[0, 0] = True
    for i in range(1, n):
        visible[i] = visible[parents[i]]
        visible[i, i] = True
    return visible


def packed_dense_mask(prefix_lengths: Sequence[int],
                      parents_list: Sequence[Sequence[int]]) -> np.ndarray:
    """Dense additive mask [R, P+R] (0 visible, -inf hidden) of CTBD:500-546.

    Request i's rows see keys [c_i, c_i+L_i) of the packed prefix and the
    packed tree keys P + q_i + j for every ancestor-or-self j.
    """
    lengths = [int(v) for v in prefix_lengths]
    rows = [len(p) for p in parents_list]
    total_prefix = sum(lengths)
    total_rows = sum(rows)
    mask = np.full((total_rows, total_prefix + total_rows), -np.inf, np.float32)
    cache_offset = 0
    query_offset = 0
    for length, parents in zip(lengths, parents_list):
        n = len(parents)
        mask[query_offset:query_offset + n, cache_offset:cache_offset + length] = 0
        block = mask[query_offset:query_offset + n,
                     total_prefix + query_offset:total_prefix + query_offset + n]
        block[visibility(parents)] = 0
        cache_offset += length
        query_offset += n
    return mask


def packed_ids_positions(roots: Sequence[int], tokens_list, depths_list,
                         round_prefix_lengths: Sequence[int]):
    """ids = [root] + tokens, positions = round_prefix_len + depth (CTBD:521-532)."""
    ids = []
    positions = []
    for root, tokens, depths, prefix in zip(roots, tokens_list, depths_list,
                                            round_prefix_lengths):
        ids.extend([int(root)] + [int(t) for t in tokens])
        positions.extend(int(prefix) + int(d) for d in depths)
    return np.asarray(ids, np.int64), np.asarray(positions, np.int64)


# --------------------------------------------------------------------------
# Attention (transformers sdpa_attention_forward with an explicit mask)
# --------------------------------------------------------------------------

class DenseWave:
    """The reference packed wave's attention inputs, built once: all prefixes
    and tree rows concatenated into one packed K/V (``_pack_cache_sequence``),
    expanded to every query head (transformers' ``repeat_kv``), and the dense
    additive mask [R, P+R] (``_packed_block_inputs``), all fp32 on the CPU
    (CTBD:313-361, :500-546).  Calling it runs the masked SDPA for query rows
    [a, b) over all P+R keys."""

    def __init__(self, q, k_prefix_list, v_prefix_list, k_tree, v_tree, parents_list,
                 scale: float | None = None):
        import torch
        self.q = torch.as_tensor(q).float()
        rows, hq, dim = self.q.shape
        hkv = k_tree.shape[1]
        group = hq // hkv
        lengths = [int(k.shape[1]) for k in k_prefix_list]
        keys = torch.cat([torch.as_tensor(k).float() for k in k_prefix_list]
                         + [torch.as_tensor(k_tree).float().transpose(0, 1)], dim=1)
        values = torch.cat([torch.as_tensor(v).float() for v in v_prefix_list]
                           + [torch.as_tensor(v_tree).float().transpose(0, 1)], dim=1)
        self.mask = torch.from_numpy(packed_dense_mask(lengths, parents_list))
        self.keys = keys.repeat_interleave(group, dim=0).unsqueeze(0)
        self.values = values.repeat_interleave(group, dim=0).unsqueeze(0)
        self.scale = dim ** -0.5 if scale is None else scale
        self.rows = rows

    def __call__(self, a: int, b: int):
        """[b - a, Hq, D] fp32 output of query rows [a, b)."""
        import torch
        out = torch.nn.functional.scaled_dot_product_attention(
            self.q[a:b].transpose(0, 1).unsqueeze(0), self.keys, self.values,
            attn_mask=self.mask[a:b], scale=self.scale,
        )
        return out[0].transpose(0, 1)


def attention_dense(q, k_prefix_list, v_prefix_list, k_tree, v_tree,
                    parents_list, scale: float | None = None,
                    row_block: int | None = None):
    """Reference packed wave: one dense masked SDPA over all P+R keys.

    q [R, Hq, D]; k/v_prefix_list[i] [Hkv, L_i, D]; k/v_tree [R, Hkv, D].
    All inputs are upcast to fp32 (they hold bf16 values).  Returns [R, Hq, D]
    fp32.  Mirrors _pack_cache_sequence + _packed_block_inputs + repeat_kv +
    F.scaled_dot_product_attention(attn_mask=mask) (CTBD:313-361, :500-546).
    ``row_block`` runs the same SDPA on blocks of that many query rows (each
    row still scores all P+R keys), which bounds the score matrix's memory.
    """
    import torch
    wave = DenseWave(q, k_prefix_list, v_prefix_list, k_tree, v_tree, parents_list, scale)
    block = wave.rows if not row_block else int(row_block)
    pieces = [wave(a, min(wave.rows, a + block)) for a in range(0, wave.rows, block)]
    return torch.cat(pieces, dim=0).contiguous() if len(pieces) > 1 else pieces[0].contiguous()


def attention_per_request(q, k_prefix_list, v_prefix_list, k_tree, v_tree,
                          row_offset, parents_list, scale: float | None = None,
                          requests: Sequence[int] | None = None):
    """Same math as attention_dense restricted to each request's own keys.

    Per kv head g the request's G query heads are stacked into one [n*G, D]
    operand (row r, head h at r*G + h), scored against the prefix keys and the
    request's tree keys, masked to ancestors-or-self on the tree part,
    soft-maxed in fp32 and applied to the values: the same visible sets and
    GQA mapping as the dense wave, as plain fp32 matrix products.
    Returns a dict request -> [n_i, Hq, D] fp32 (only ``requests`` if given).
    """
    import torch
    q = torch.as_tensor(q)
    rows, hq, dim = q.shape
    hkv = k_tree.shape[1]
    group = hq // hkv
    scale = dim ** -0.5 if scale is None else scale
    out = {}
    selected = range(len(parents_list)) if requests is None else requests
    for i in selected:
        r0, r1 = int(row_offset[i]), int(row_offset[i + 1])
        n = r1 - r0
        kp = torch.as_tensor(k_prefix_list[i]).float()
        vp = torch.as_tensor(v_prefix_list[i]).float()
        length = kp.shape[1]
        hidden = ~torch.from_numpy(visibility(parents_list[i])).repeat_interleave(group, 0)
        qi = q[r0:r1].float()
        o = torch.empty(n, hq, dim)
        for g in range(hkv):
            qg = qi[:, g * group:(g + 1) * group].reshape(n * group, dim)
            kg = torch.cat([kp[g], torch.as_tensor(k_tree[r0:r1, g]).float()])
            vg = torch.cat([vp[g], torch.as_tensor(v_tree[r0:r1, g]).float()])
            scores = (qg @ kg.T) * scale
            scores[:, length:].masked_fill_(hidden, -math.inf)
            o[:, g * group:(g + 1) * group] = (
                torch.softmax(scores, dim=-1) @ vg).reshape(n, group, dim)
        out[i] = o
    return out


def attention_bruteforce(q, k_prefix_list, v_prefix_list, k_tree, v_tree,
                         row_offset, parents_list, scale: float | None = None):
    """Explicit per-row, per-head softmax loops in float64 (tiny cases only)."""
    q = np.asarray(q, np.float64)
    rows, hq, dim = q.shape
    hkv = k_tree.shape[1]
    group = hq // hkv
    scale = dim ** -0.5 if scale is None else scale
    out = np.zeros((rows, hq, dim))
    for i, parents in enumerate(parents_list):
        r0 = int(row_offset[i])
        kp = np.asarray(k_prefix_list[i], np.float64)
        vp = np.asarray(v_prefix_list[i], np.float64)
        for local in range(len(parents)):
            ancestors = []
            node = local
            while node >= 0:
                ancestors.append(node)
                node = parents[node]
            for h in range(hq):
                g = h // group
                keys = [kp[g, t] for t in range(kp.shape[1])]
                vals = [vp[g, t] for t in range(vp.shape[1])]
                for a in sorted(ancestors):
                    keys.append(np.asarray(k_tree[r0 + a, g], np.float64))
                    vals.append(np.asarray(v_tree[r0 + a, g], np.float64))
                scores = np.array([q[r0 + local, h] @ k for k in keys]) * scale
                weights = np.exp(scores - scores.max())
                weights /= weights.sum()
                out[r0 + local, h] = weights @ np.stack(vals)
    return out


# --------------------------------------------------------------------------
# KV commit (CTBD:215-261, keep rule CTBD:2108-2109)
# --------------------------------------------------------------------------

def kv_commit(arena_k: np.ndarray, arena_v: np.ndarray, lengths: np.ndarray,
              capacity: int, slots: Sequence[int], tree_k: np.ndarray,
              tree_v: np.ndarray, row_offset: Sequence[int],
              keep_rows: Sequence[Sequence[int]]):
    """Scatter kept tree rows into the arena and advance lengths, in place.

    arena_k/v [layers, Hkv, slots*capacity, D]; tree_k/v [layers, R, Hkv, D];
    keep_rows[i] = [0] + accepted local nodes.  For t < len(keep_i):
      arena[:, :, slot_i*cap + len_i + t] = tree[:, row_offset[i] + keep_i[t]].
    Raises RuntimeError when len_i + len(keep_i) > capacity (CTBD:235-236).
    """
    for i, keep in enumerate(keep_rows):
        slot = int(slots[i])
        if int(lengths[slot]) + len(keep) > capacity:
            raise RuntimeError("Persistent request KV capacity exhausted")
    for i, keep in enumerate(keep_rows):
        slot = int(slots[i])
        base = slot * capacity + int(lengths[slot])
        for t, row in enumerate(keep):
            src = int(row_offset[i]) + int(row)
            arena_k[:, :, base + t] = tree_k[:, src]
            arena_v[:, :, base + t] = tree_v[:, src]
        lengths[slot] += len(keep)
    return lengths


def kv_split(prefix_k: np.ndarray, prefix_v: np.ndarray, tree_k: np.ndarray,
             tree_v: np.ndarray, cache_offsets: Sequence[int], old_lengths: Sequence[int],
             row_offset: Sequence[int], keep_rows: Sequence[Sequence[int]]):
    """Non-persistent split (CTBD:409-450): request i's new cache is the packed
    prefix rows [c_i, c_i + L_i) followed by its kept tree rows q_i + keep_i[t].

    prefix_k/v [layers, Hkv, P, D]; tree_k/v [layers, R, Hkv, D].  Returns a
    list of (keys, values) [layers, Hkv, L_i + |keep_i|, D] per request.
    """
    out = []
    for i, keep in enumerate(keep_rows):
        c, length, q = int(cache_offsets[i]), int(old_lengths[i]), int(row_offset[i])
        rows = [q + int(r) for r in keep]
        keys = np.concatenate([prefix_k[:, :, c:c + length],
                               tree_k[:, rows].transpose(0, 2, 1, 3)], axis=2)
        values = np.concatenate([prefix_v[:, :, c:c + length],
                                 tree_v[:, rows].transpose(0, 2, 1, 3)], axis=2)
        out.append((keys, values))
    return out


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo, with its family, model
    and stepping numbers (a virtual machine may report only a generic name
    such as "AMD EPYC")."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block is enough
                key, _, value = line.partition(":")
                fields[key.strip()] = value.strip()
    except OSError:
        pass
    name = fields.get("model name")
    if not name:
        import platform
        return platform.processor() or platform.machine()
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# --------------------------------------------------------------------------
# Reference CPU path of the sampling stage (CPU baseline)
# --------------------------------------------------------------------------

def reference_sampling_wave(logits, row_offset, parents_list, tokens_list, seeds):
    """fp32 softmax over the whole wave (sampling.py:29-36 via CTBD:1821-1824),
    then per request one multinomial over its rows and the ancestral walk
    (sampling.py:903-950).  Returns [(nodes, tokens, bonus)] per request."""
    import torch
    probs = torch.softmax(torch.as_tensor(logits).to(torch.float32), dim=-1)
    results = []
    for i, (parents, tokens) in enumerate(zip(parents_list, tokens_list)):
        r0, r1 = int(row_offset[i]), int(row_offset[i + 1])
        gen = torch.Generator().manual_seed(int(seeds[i]))
        draws = torch.multinomial(probs[r0:r1], 1, generator=gen).reshape(-1).tolist()
        results.append(ancestral_walk(parents, tokens, draws))
    return results
