"""The C-ABI library loads, exports every declared symbol, and its host-side
planner produces a valid work list.  No GPU calls."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from specgrove_amd import _lib, ops
from specgrove_amd import workloads as W

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions():
    text = (ROOT / "include" / "specgrove_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(sg_\w+)\s*\(", text, re.M)))


def test_library_loads_and_struct_sizes_match():
    lib = _lib.load()
    assert lib.sg_abi_version() == _lib.SG_ABI_VERSION == 5


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    declared = _declared_functions()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), name
        assert name in _lib.EXPORTED_SYMBOLS, name


def _check_plan(wl, target):
    plan = ops.plan_attention(wl.row_offset, wl.prefix_len, wl.num_q_heads, wl.num_kv_heads,
                              wl.head_dim, target)
    header, units, merges, bins = ops.decode_plan(plan)
    assert header[0] == 0x53475041 and header[2] == plan.merges
    # work lists: one per workgroup, contiguous, non-empty, covering every unit
    # once; by default one unit per list, else at most `target` lists
    expected = min(target, len(units)) if target > 0 else len(units)
    assert header[7] == plan.units and 0 < plan.units <= expected
    assert bins[0] == 0 and bins[-1] == len(units) and (np.diff(bins) >= 1).all()
    rows_per_tile = 128 // (wl.num_q_heads // wl.num_kv_heads)
    cover = {}
    tile_of = {}  # rows per unit of each request: a full row tile, or half a
                  # tile when the planner split the rows (flags bit 1)
    for (req, g, row_begin, row_count, kb, ke, partial, flags, group, splits, first,
         _) in units.tolist():
        t = rows_per_tile // 2 if flags & 2 else rows_per_tile
        assert tile_of.setdefault(req, t) == t
        if flags & 2:  # only units of more than 64 query vectors are split by rows
            assert int(wl.rows[req]) * 128 // rows_per_tile > 64
        assert row_begin % t == 0
        assert row_count == min(t, int(wl.rows[req]) - row_begin)
        cover.setdefault((req, g, row_begin), []).append(
            (kb, ke, partial, flags, group, splits, first))
    groups = {}
    for req in range(wl.num_requests):
        for g in range(wl.num_kv_heads):
            for row_begin in range(0, int(wl.rows[req]), tile_of[req]):
                parts = sorted(cover.pop((req, g, row_begin)))
                assert parts[0][0] == 0 and parts[-1][1] == int(wl.prefix_len[req])
                for a, b in zip(parts, parts[1:]):
                    assert a[1] == b[0] and a[0] < a[1]
                assert sum(p[3] & 1 for p in parts) == 1 and parts[-1][3] & 1
                assert all(p[5] == len(parts) for p in parts)
                if len(parts) == 1:
                    assert parts[0][2] == -1 and parts[0][4] == -1
                else:
                    assert len({p[4] for p in parts}) == 1
                    slots = sorted(p[2] for p in parts)
                    assert slots == list(range(parts[0][6], parts[0][6] + len(parts)))
                    groups[parts[0][4]] = (req, g, row_begin,
                                           min(tile_of[req], int(wl.rows[req]) - row_begin),
                                           parts[0][6], len(parts))
    assert not cover
    assert sorted(groups) == list(range(plan.merges))
    for k, rec in enumerate(merges.tolist()):
        assert tuple(rec[:6]) == groups[k]
    partials = int(header[6])
    assert partials == sum(1 for u in units if u[6] >= 0)
    assert plan.workspace_bytes == partials * 128 * (wl.head_dim + 2) * 4
    # Balanced lists: no list exceeds the mean load by more than its largest unit.
    def cost(u):
        tiles = (u[5] - u[4] + 31) // 32 + ((int(wl.rows[u[0]]) + 31) // 32 if u[7] & 1 else 0)
        nq = (u[3] * (wl.num_q_heads // wl.num_kv_heads) + 31) // 32
        return 550 + 57 * tiles if nq <= 2 else 840 + 88 * tiles
    costs = [cost(u) for u in units.tolist()]
    loads = [sum(costs[bins[b]:bins[b + 1]]) for b in range(len(bins) - 1)]
    assert max(loads) <= sum(costs) / len(loads) + max(costs)
    return plan


@pytest.mark.parametrize("target", [0, 64, 4096])
def test_plan_covers_every_row_and_key_once(target):
    _check_plan(W.qwen3_8b_workload(), target)
    _check_plan(W.tiny_attention_workload(), target)


def test_plan_rejects_oversized_trees_and_bad_heads():
    with pytest.raises(ValueError):
        ops.plan_attention([0, 300], [10], 32, 8, 128)
    with pytest.raises(ValueError):
        ops.plan_attention([0, 4], [10], 30, 8, 128)
    with pytest.raises(ValueError):
        ops.plan_attention([0, 4], [10], 32, 8, 96)


def test_head_groups_beyond_16_are_rejected_not_crashed():
    """128 query heads per kv head used to reach a division by zero in the
    row-split path of the planner; groups are limited to 1..16."""
    rows = np.arange(0, 9, dtype=np.int32)
    with pytest.raises(ValueError, match="1, 2, 4, 8 or 16"):
        ops.plan_attention(rows, [65536] + [16] * 7, 128, 1, 128)
    with pytest.raises(ValueError, match="1, 2, 4, 8 or 16"):
        ops.plan_attention([0, 4], [10], 32, 1, 128)
    ops.plan_attention(rows, [65536] + [16] * 7, 16, 1, 128)  # the largest group plans


def _attn_args(**fields):
    """SgTreeAttnArgs with placeholder device pointers: every call below must
    be rejected by the host-side checks before anything touches a device."""
    a = _lib.SgTreeAttnArgs()
    a.num_requests, a.num_rows, a.num_q_heads, a.num_kv_heads, a.head_dim = 1, 4, 8, 2, 128
    a.scale = 128 ** -0.5
    for name in ("q_dev", "k_cache_dev", "v_cache_dev", "k_tree_dev", "v_tree_dev",
                 "row_offset_dev", "prefix_start_dev", "prefix_len_dev", "parent_dev",
                 "out_dev", "plan_dev"):
        setattr(a, name, 0x1000)
    a.q_row_stride, a.q_head_stride = 8 * 128, 128
    a.cache_head_stride, a.cache_token_stride = 128 * 1024, 128
    a.tree_row_stride, a.tree_head_stride = 2 * 128, 128
    a.out_row_stride, a.out_head_stride = 8 * 128, 128
    a.plan_units = 1
    for k, v in fields.items():
        setattr(a, k, v)
    return a


def test_fwd_rejects_bad_head_counts_without_crashing():
    lib = _lib.load()
    for hq, hkv in ((0, 2), (0, 0), (3, 2), (256, 2), (8, -1)):
        a = _attn_args(num_q_heads=hq, num_kv_heads=hkv)
        assert lib.sg_tree_attn_fwd(ctypes.byref(a), None) == _lib.SG_EINVAL, (hq, hkv)


def test_stale_plans_are_rejected_on_the_host():
    """A plan records its wave: the planner's header keeps the request and row
    counts and a hash of the row offsets and prefix lengths."""
    row_offset, prefix = [0, 4, 9], [100, 37]
    plan = ops.plan_attention(row_offset, prefix, 8, 2, 128)
    assert plan.num_requests == 2 and plan.num_rows == 9
    ops.check_plan(plan, row_offset, prefix)
    with pytest.raises(ValueError, match="another wave"):
        ops.check_plan(plan, row_offset, [100, 40])      # after a commit of 3 rows
    with pytest.raises(ValueError, match="another wave"):
        ops.check_plan(plan, [0, 5, 9], prefix)
    with pytest.raises(ValueError, match="another wave"):
        ops.check_plan_call(plan, 2, 10, 8, 2, 128)
    with pytest.raises(ValueError, match="head configuration"):
        ops.check_plan_call(plan, 2, 9, 16, 2, 128)
    # The C ABI checks the host copy of the plan before enqueueing anything.
    lib = _lib.load()
    for fields in ({"num_rows": 10}, {"num_requests": 3}, {"num_q_heads": 16},
                   {"plan_units": plan.units + 1}):
        base = dict(num_requests=2, num_rows=9, plan_units=plan.units,
                    plan_merges=plan.merges, plan_host=plan.host.ctypes.data)
        base.update(fields)
        a = _attn_args(**base)
        assert lib.sg_tree_attn_fwd(ctypes.byref(a), None) == _lib.SG_EINVAL, fields
        assert b"plan" in lib.sg_last_error()


def test_noalloc_sampler_rejects_oversized_waves_before_any_device_call():
    lib = _lib.load()
    a = _lib.SgTreeSampleArgs()
    per_request = lib.sg_tree_sample_workspace_bytes(1, 1, 151936)  # one row each
    a.num_requests = _lib.NOALLOC_SCRATCH_BYTES // per_request + 1
    a.num_rows = a.num_requests
    a.vocab = 151936
    a.logits_row_stride = 151936
    a.uniform_stride = 2
    for name in ("logits_dev", "row_offset_dev", "parent_dev", "token_dev", "uniforms_dev",
                 "row_max_dev", "row_sum_dev", "accept_len_dev", "bonus_dev"):
        setattr(a, name, 0x1000)
    assert lib.sg_tree_sample_noalloc(ctypes.byref(a), None) == _lib.SG_EINVAL
    assert b"static maximum" in lib.sg_last_error()
    a.num_requests = a.num_rows = 2
    a.workspace_dev, a.workspace_bytes = 0x1000, 1 << 20
    assert lib.sg_tree_sample_noalloc(ctypes.byref(a), None) == _lib.SG_EINVAL
    a.workspace_dev, a.workspace_bytes = 0, 0
    a.logits_dtype = 7
    assert lib.sg_tree_sample_noalloc(ctypes.byref(a), None) == _lib.SG_EINVAL


def test_lm_head_and_projected_sampler_reject_bad_arguments_on_the_host():
    lib = _lib.load()
    assert lib.sg_lm_head_tile_count(151936) == 1187
    assert lib.sg_lm_head_tile_count(129) == 2 and lib.sg_lm_head_tile_count(0) == -1
    a = _lib.SgLmHeadArgs()
    a.num_rows, a.hidden_size, a.vocab, a.num_hidden_rows = 4, 4096, 151936, 4
    for name in ("hidden_dev", "weight_dev", "logits_dev", "tile_stats_dev", "row_max_dev",
                 "row_sum_dev"):
        setattr(a, name, 0x1000)
    a.hidden_row_stride, a.weight_row_stride, a.logits_row_stride = 4096, 4096, 151936
    for field, value, text in (("hidden_size", 4000, b"multiple of 64"),
                               ("hidden_size", 32, b"multiple of 64"),
                               ("vocab", 0, b"vocab"),
                               ("logits_row_stride", 151930, b"strides")):
        good = getattr(a, field)
        setattr(a, field, value)
        assert lib.sg_lm_head(ctypes.byref(a), None) == _lib.SG_EINVAL, field
        assert text in lib.sg_last_error(), (field, lib.sg_last_error())
        setattr(a, field, good)
    a.hidden_dev = 0x1008  # not 16-byte aligned
    assert lib.sg_lm_head(ctypes.byref(a), None) == _lib.SG_EINVAL
    a.num_rows = 0         # nothing to project: no launch
    assert lib.sg_lm_head(ctypes.byref(a), None) == _lib.SG_OK
    s = _lib.SgTreeSampleArgs()
    s.num_requests, s.num_rows, s.vocab, s.logits_row_stride, s.uniform_stride = 1, 4, 100, 100, 2
    for name in ("logits_dev", "row_offset_dev", "parent_dev", "token_dev", "uniforms_dev",
                 "row_max_dev", "row_sum_dev", "accept_len_dev", "bonus_dev"):
        setattr(s, name, 0x1000)
    s.workspace_dev, s.workspace_bytes = 0x1000, 1 << 20
    s.logits_row_dev = 0x1000   # a row map without terminal_leaf_dev
    assert lib.sg_tree_sample(ctypes.byref(s), None) == _lib.SG_EINVAL
    assert b"terminal_leaf_dev" in lib.sg_last_error()
    s.logits_row_dev, s.num_logits_rows = 0, 3  # logits rows differ without a map
    assert lib.sg_tree_sample(ctypes.byref(s), None) == _lib.SG_EINVAL
    s.num_logits_rows, s.flags = 0, 6
    assert lib.sg_tree_sample(ctypes.byref(s), None) == _lib.SG_EINVAL


def test_packed_lm_head_rejects_bad_arguments_on_the_host():
    lib = _lib.load()
    assert lib.sg_lm_head_packed_bytes(151936, 4096) == 594 * 256 * 4096 * 2
    assert lib.sg_lm_head_packed_bytes(300, 128) == 2 * 256 * 128 * 2
    for vocab, hsize in ((0, 4096), (100, 4000), (100, 32)):
        assert lib.sg_lm_head_packed_bytes(vocab, hsize) == -1
    for args, text in (((0x1000, 4096, 0, 4096, 0x2000), b"vocab"),
                       ((0x1000, 4096, 100, 4000, 0x2000), b"multiple of 64"),
                       ((0, 4096, 100, 4096, 0x2000), b"null"),
                       ((0x1000, 4000, 100, 4096, 0x2000), b"weight_row_stride"),
                       ((0x1000, 4100, 100, 4096, 0x2000), b"weight_row_stride"),
                       ((0x1008, 4096, 100, 4096, 0x2000), b"aligned")):
        assert lib.sg_lm_head_pack_weight(*args, None) == _lib.SG_EINVAL, args
        assert text in lib.sg_last_error(), (args, lib.sg_last_error())
    a = _lib.SgLmHeadArgs()
    a.num_rows, a.hidden_size, a.vocab, a.num_hidden_rows = 4, 4096, 151936, 4
    for name in ("hidden_dev", "weight_dev", "logits_dev", "tile_stats_dev", "row_max_dev",
                 "row_sum_dev"):
        setattr(a, name, 0x1000)
    a.hidden_row_stride, a.weight_row_stride, a.logits_row_stride = 4096, 0, 151936
    a.hidden_size = 4000
    assert lib.sg_lm_head_packed(ctypes.byref(a), None) == _lib.SG_EINVAL
    a.hidden_size, a.weight_dev = 4096, 0
    assert lib.sg_lm_head_packed(ctypes.byref(a), None) == _lib.SG_EINVAL
    assert b"null" in lib.sg_last_error()
    a.num_rows = 0
    assert lib.sg_lm_head_packed(ctypes.byref(a), None) == _lib.SG_OK


def test_layer_ops_reject_bad_arguments_on_the_host():
    """The decoder-stack kernels check shapes, strides and 16-byte alignment
    before any launch (fake, never-dereferenced device addresses)."""
    lib = _lib.load()
    a = _lib.SgQkNormRopeArgs()
    a.num_rows, a.num_q_heads, a.num_kv_heads, a.head_dim, a.eps = 4, 32, 8, 128, 1e-6
    for name in ("qkv_dev", "q_norm_dev", "k_norm_dev", "inv_freq_dev", "positions_dev",
                 "q_out_dev", "k_out_dev", "v_out_dev"):
        setattr(a, name, 0x1000)
    a.qkv_row_stride, a.q_row_stride, a.kv_head_stride = 48 * 128, 32 * 128, 4 * 128
    for field, value, text in (("head_dim", 96, b"head_dim"),
                               ("qkv_row_stride", 40 * 128, b"qkv row stride"),
                               ("kv_head_stride", 3 * 128, b"head stride"),
                               ("q_row_stride", 32 * 128 + 4, b"multiples of 8"),
                               ("q_out_dev", 0x1008, b"aligned"),
                               ("k_norm_dev", 0x1004, b"aligned")):
        good = getattr(a, field)
        setattr(a, field, value)
        assert lib.sg_qk_norm_rope(ctypes.byref(a), None) == _lib.SG_EINVAL, field
        assert text in lib.sg_last_error(), (field, lib.sg_last_error())
        setattr(a, field, good)
    a.num_rows = 0  # nothing to do: no launch
    assert lib.sg_qk_norm_rope(ctypes.byref(a), None) == _lib.SG_OK


def test_product_package_never_imports_the_oracle():
    for path in (ROOT / "specgrove_amd").rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), path
