"""The oracle's LM-head statistics and its walk over a partly projected wave,
pinned on the CPU.

* Statistics: the maximum is exact; the sums match float64 within fp32
  rounding; rows of equal values sum to the exact token count (every token is
  counted once: a dropped or repeated term, or a wrong tile boundary, fails);
  a spike row sums to exactly 1.
* Walk: with every row projected, the mapped walk equals the unmapped oracle
  sampler (routing and exits unchanged); with only internal rows projected,
  walks that reach a leaf stop there, and the leaf's bonus drawn from its own
  row with u[2d+1] (a one-node walk) equals the full projection's bonus --
  the lazy projection's law (reference sampling.py:738-832,
  fused_tree_sampling.py:2840-3019).
"""
import numpy as np
import pytest

from tests.sampler_cases import tree_problem


@pytest.mark.parametrize("vocab", [1, 7, 128, 129, 1000, 4096, 151936])
def test_tile_stats_against_float64(oracle, vocab):
    rng = np.random.default_rng(vocab)
    x = (rng.standard_normal((5, vocab)) * 6).astype(np.float32)
    x[1] -= 150.0
    pairs, m, z = oracle.lm_head_stats(x)
    assert pairs.shape == (5, (vocab + 127) // 128, 2)
    x64 = x.astype(np.float64)
    np.testing.assert_array_equal(m, x.max(axis=1))
    want = np.exp(x64 - x64.max(axis=1, keepdims=True)).sum(axis=1)
    np.testing.assert_allclose(z, want, rtol=2e-6)
    for t in range(pairs.shape[1]):
        seg = x64[:, 128 * t:128 * (t + 1)]
        np.testing.assert_array_equal(pairs[:, t, 0], seg.max(axis=1).astype(np.float32))
        np.testing.assert_allclose(pairs[:, t, 1],
                                   np.exp(seg - seg.max(axis=1, keepdims=True)).sum(axis=1),
                                   rtol=2e-6)


@pytest.mark.parametrize("vocab", [1, 2, 127, 128, 129, 255, 1000, 151936])
def test_constant_rows_count_every_token_once(oracle, vocab):
    x = np.full((2, vocab), 3.25, np.float32)
    x[1] = -40.0
    pairs, m, z = oracle.lm_head_stats(x)
    assert (z == np.float32(vocab)).all()
    assert (m == x[:, 0]).all()
    sizes = np.minimum(128, vocab - 128 * np.arange(pairs.shape[1]))
    assert (pairs[0, :, 1] == sizes.astype(np.float32)).all()


def test_spike_row(oracle):
    x = np.full((1, 5000), -100.0, np.float32)
    x[0, 4321] = 100.0
    _, m, z = oracle.lm_head_stats(x)
    assert m[0] == 100.0 and z[0] == 1.0


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_mapped_walk_with_every_row_equals_the_sampler(oracle, seed):
    case = tree_problem(seed, num_requests=7, nodes=[12, 1, 9, 16, 3, 12, 5], vocab=3000)
    want = oracle.tree_sample(case["logits"], case["row_offset"], case["parent"],
                              case["token"], case["uniforms"], case["max_depth"])
    nodes, length, bonus, leaf = oracle.tree_sample_mapped(
        case["logits"], case["row_offset"], case["parent"], case["token"],
        case["uniforms"], case["max_depth"], None, None, None)
    np.testing.assert_array_equal(nodes, want[0])
    np.testing.assert_array_equal(length, want[1])
    np.testing.assert_array_equal(bonus, want[2])
    assert (leaf == -1).all()
    # Given statistics (the sampler's own) give the same decisions.
    again = oracle.tree_sample_mapped(
        case["logits"], case["row_offset"], case["parent"], case["token"],
        case["uniforms"], case["max_depth"], None, want[3], want[4])
    np.testing.assert_array_equal(again[2], want[2])


def lazy_walk(oracle, case, row_m=None, row_z=None):
    """Internal rows projected, reached leaves drawn from their own rows."""
    ro, parent = case["row_offset"], case["parent"]
    rows = int(ro[-1])
    has_child = np.zeros(rows, bool)
    for i in range(len(ro) - 1):
        for k in range(1, int(ro[i + 1] - ro[i])):
            has_child[ro[i] + parent[ro[i] + k]] = True
    internal = np.flatnonzero(has_child)
    row_map = np.full(rows, -1, np.int32)
    row_map[internal] = np.arange(internal.size, dtype=np.int32)
    logits = case["logits"][internal] if internal.size else case["logits"][:1]
    stats = (None, None) if row_m is None else (row_m[internal], row_z[internal])
    nodes, length, bonus, leaf = oracle.tree_sample_mapped(
        logits, ro, parent, case["token"], case["uniforms"], case["max_depth"], row_map,
        *stats)
    reached = np.flatnonzero(leaf >= 0)
    assert (bonus[reached] == -1).all()
    if reached.size:
        leaf_rows = ro[reached] + leaf[reached]
        single = np.zeros((reached.size, 2), np.float32)
        single[:, 1] = case["uniforms"][reached, 2 * length[reached] + 1]
        lstats = (None, None) if row_m is None else (row_m[leaf_rows], row_z[leaf_rows])
        _, slen, sbonus, sleaf = oracle.tree_sample_mapped(
            case["logits"][leaf_rows], np.arange(reached.size + 1, dtype=np.int32),
            np.full(reached.size, -1, np.int32), np.zeros(reached.size, np.int32), single, 0,
            None, *lstats)
        assert (slen == 0).all() and (sleaf == -1).all()
        bonus = bonus.copy()
        bonus[reached] = sbonus
    return nodes, length, bonus, leaf


@pytest.mark.parametrize("seed", [3, 4, 5, 6])
def test_lazy_projection_law_equals_full_projection(oracle, seed):
    case = tree_problem(seed, num_requests=9, nodes=[1, 2, 16, 9, 12, 5, 16, 3, 8],
                        vocab=2500, child_boost=9.0)
    full = oracle.tree_sample_mapped(case["logits"], case["row_offset"], case["parent"],
                                     case["token"], case["uniforms"], case["max_depth"],
                                     None, None, None)
    nodes, length, bonus, leaf = lazy_walk(oracle, case)
    np.testing.assert_array_equal(nodes, full[0])
    np.testing.assert_array_equal(length, full[1])
    np.testing.assert_array_equal(bonus, full[2])
    # The boosted children make some walks reach leaves and some stop inside.
    assert (leaf >= 0).any() and (leaf < 0).any()


def test_unprojected_node_with_children_is_rejected(oracle):
    case = tree_problem(7, num_requests=2, nodes=[4, 3], vocab=600)
    row_map = np.arange(int(case["row_offset"][-1]), dtype=np.int32)
    row_map[0] = -1  # the first root has children
    with pytest.raises(ValueError):
        oracle.tree_sample_mapped(case["logits"], case["row_offset"], case["parent"],
                                  case["token"], case["uniforms"], case["max_depth"],
                                  row_map, None, None)
