"""The C-ABI library loads, exports every declared symbol, and its host-side
planner produces a valid work list.  No GPU calls."""
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
    assert lib.sg_abi_version() == 1


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
    header, units, merges = ops.decode_plan(plan)
    assert header[0] == 0x53475041 and header[1] == plan.units and header[2] == plan.merges
    rows_per_tile = 128 // (wl.num_q_heads // wl.num_kv_heads)
    cover = {}
    for req, g, row_begin, row_count, kb, ke, partial, flags in units.tolist():
        key = (req, g, row_begin)
        assert row_begin % rows_per_tile == 0
        assert row_count == min(rows_per_tile, int(wl.rows[req]) - row_begin)
        cover.setdefault(key, []).append((kb, ke, partial, flags))
    for req in range(wl.num_requests):
        for g in range(wl.num_kv_heads):
            for row_begin in range(0, int(wl.rows[req]), rows_per_tile):
                parts = sorted(cover.pop((req, g, row_begin)))
                assert parts[0][0] == 0 and parts[-1][1] == int(wl.prefix_len[req])
                for (a0, a1, _, _), (b0, _, _, _) in zip(parts, parts[1:]):
                    assert a1 == b0 and a0 < a1
                assert sum(f & 1 for *_, f in parts) == 1
                if len(parts) == 1:
                    assert parts[0][2] == -1
                else:
                    assert all(p >= 0 for _, _, p, _ in parts)
    assert not cover
    slots = sorted(int(p) for p in units[:, 6] if p >= 0)
    assert slots == list(range(len(slots)))
    assert sum(int(m[5]) for m in merges) == len(slots)
    assert plan.workspace_bytes == len(slots) * 128 * (wl.head_dim + 2) * 4
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


def test_product_package_never_imports_the_oracle():
    for path in (ROOT / "specgrove_amd").rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), path
