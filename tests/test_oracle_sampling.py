"""Pins of the sampling oracle (CPU only).

The oracle is checked against what fixes it independently of its own code:
the reference's exact exit law (test_audited_global_tree_matrix.py:48-64),
libm/float64 exp, float64 row sums, the float64 inverse-CDF rule of
fused_tree_sampling.py:2607-2612, and the committed golden vectors.
"""
import json
from collections import Counter
from pathlib import Path

import numpy as np
import pytest

from tests.sampler_cases import tree_problem

GOLDEN = Path(__file__).parent / "golden"


def test_exp_matches_float64_exp(oracle):
    x = np.linspace(-87.0, 0.0, 1_000_001, dtype=np.float32)
    e = oracle.exp_f32(x)
    ref = np.exp(x.astype(np.float64))
    assert np.max(np.abs(e - ref) / ref) < 4e-7
    assert np.all(np.diff(e) >= 0), "exp must be monotone"
    assert oracle.exp_f32(np.array([0.0, -0.0], np.float32)).tolist() == [1.0, 1.0]
    # Into the subnormal range: monotone, within 4e-7 relative or one
    # subnormal step (2^-149) of exp, below 2^-126 from -87.5 down, and
    # exactly 0 below about -103.3 (NaN and -inf included).
    deep = np.linspace(-110.0, -87.0, 200_001, dtype=np.float32)
    ed = oracle.exp_f32(deep)
    ref = np.exp(deep.astype(np.float64))
    assert np.all(np.diff(ed) >= 0)
    assert np.all(np.abs(ed - ref) <= np.maximum(4e-7 * ref, 2.0 ** -149))
    assert np.all(ed[deep <= -87.5] < np.float32(2.0 ** -126))
    low = oracle.exp_f32(np.array([-104.5, -120.0, -1000.0, -np.inf, np.nan], np.float32))
    assert np.all(low == 0.0)
    assert oracle.exp_f32(np.array([-100.0], np.float32))[0] > 0.0
    high = oracle.exp_f32(np.array([88.0, 88.5, np.inf], np.float32))
    assert np.isfinite(high[0]) and np.all(np.isinf(high[1:]))


@pytest.mark.parametrize("vocab", [1, 7, 2048, 2049, 4096, 151936])
def test_row_stats_match_float64(oracle, vocab):
    rng = np.random.default_rng(vocab)
    for scale in (0.5, 3.0, 20.0):
        row = (rng.standard_normal(vocab) * scale).astype(np.float32)
        m, z = oracle.row_stats(row)
        assert m == row.max()
        ref = np.exp(row.astype(np.float64) - float(row.max())).sum()
        assert abs(z - ref) / ref < 2e-5


def test_reference_exit_law(oracle):
    """Monte Carlo over seeded uniforms reproduces the exact five-outcome law."""
    fx = json.loads((GOLDEN / "reference_fixtures.json").read_text())["exit_law"]
    p = np.asarray(fx["probabilities"])
    parents, tokens = fx["parents"], fx["tokens"]
    reps = 60000
    logits = np.tile(np.log(p).astype(np.float32), (reps, 1))
    row_offset = (np.arange(reps + 1) * 4).astype(np.int32)
    parent = np.tile(np.asarray(parents, np.int32), reps)
    token = np.tile(np.asarray([0] + tokens, np.int32), reps)
    u = np.random.default_rng(5).random((reps, 6), dtype=np.float32)
    nodes, length, bonus, _, _ = oracle.tree_sample(logits, row_offset, parent, token, u, 2)
    seen = Counter()
    for i in range(reps):
        seq = tuple(tokens[k - 1] for k in nodes[i, :length[i]]) + (int(bonus[i]),)
        seen[seq] += 1
    law = {tuple(k): v for k, v in fx["law"]}
    assert set(seen) <= set(law)
    for outcome, prob in law.items():
        freq = seen[outcome] / reps
        sigma = np.sqrt(prob * (1 - prob) / reps)
        assert abs(freq - prob) < 5 * sigma, (outcome, freq, prob)


def test_route_acceptance_matches_child_mass(oracle):
    """Sweeping the route uniform accepts child j on a u-interval of length p_j."""
    vocab = 64
    rng = np.random.default_rng(3)
    row = rng.standard_normal(vocab).astype(np.float32) * 2
    children = [5, 17, 40]
    row[children] += 2.0
    grid = 4000
    reps = grid
    logits = np.tile(row, (reps, 1)).reshape(reps, vocab)
    # one request per grid point: root with three leaf children
    logits = np.repeat(logits, 4, axis=0)
    row_offset = (np.arange(reps + 1) * 4).astype(np.int32)
    parent = np.tile(np.asarray([-1, 0, 0, 0], np.int32), reps)
    token = np.tile(np.asarray([0] + children, np.int32), reps)
    u = np.zeros((reps, 4), np.float32)
    u[:, 0] = (np.arange(grid, dtype=np.float64) + 0.5) / grid
    u[:, 2] = 0.5
    u[:, 1] = 0.5
    nodes, length, bonus, _, _ = oracle.tree_sample(logits, row_offset, parent, token, u, 1)
    p = np.exp(row.astype(np.float64) - row.max())
    p /= p.sum()
    for j, child in enumerate(children, start=1):
        frac = np.mean((length == 1) & (nodes[:, 0] == j))
        assert abs(frac - p[child]) <= 2.0 / grid
    exits = length == 0
    assert abs(exits.mean() - (1 - p[children].sum())) <= 2.0 / grid
    assert not np.isin(bonus[exits], children).any()


def test_complement_draw_matches_float64_inverse_cdf(oracle):
    """Away from ties the bonus is the float64 inverse-CDF token of the complement."""
    rng = np.random.default_rng(11)
    vocab = 4097
    mismatches = 0
    trials = 1500
    for k in range(trials):
        row = (rng.standard_normal(vocab) * 3).astype(np.float32)
        children = rng.choice(vocab, size=int(rng.integers(0, 5)), replace=False)
        u = np.float32(rng.random())
        m = float(row.max())
        token, total = oracle.complement_draw(row, m, children, u)
        e = np.exp(row.astype(np.float64) - m)
        e[children] = 0.0
        c = np.cumsum(e)
        thr = float(u) * c[-1]
        expect = int(np.searchsorted(c, thr, side="right"))
        assert token not in set(children.tolist())
        assert abs(total - c[-1]) / c[-1] < 1e-5
        if token != expect:
            mismatches += 1
            # only a float32 rounding tie at a token boundary may differ
            lo = min(token, expect)
            assert abs(c[lo] - thr) / c[-1] < 1e-5
    assert mismatches <= trials // 200


def test_complement_fallback_is_largest_non_child(oracle):
    vocab = 10
    row = np.full(vocab, -np.inf, np.float32)
    row[[2, 9]] = 0.0                      # all mass on the two children
    token, total = oracle.complement_draw(row, 0.0, [2, 9], np.float32(0.3))
    assert total == 0.0
    assert token == 8


def test_oracle_reproduces_golden_sampler_vectors(oracle):
    data = np.load(GOLDEN / "sampler_tiny.npz", allow_pickle=False)
    nodes, length, bonus, m, z = oracle.tree_sample(
        data["logits"], data["row_offset"], data["parent"], data["token"], data["uniforms"],
        int(data["max_depth"]))
    np.testing.assert_array_equal(nodes, data["accept_nodes"])
    np.testing.assert_array_equal(length, data["accept_len"])
    np.testing.assert_array_equal(bonus, data["bonus"])
    assert np.array_equal(z.view(np.uint32), data["row_sum"].view(np.uint32))


def test_walk_follows_tree_edges_and_uniform_layout(oracle):
    case = tree_problem(99, num_requests=12, nodes=16, vocab=512)
    nodes, length, bonus, _, _ = oracle.tree_sample(
        case["logits"], case["row_offset"], case["parent"], case["token"], case["uniforms"],
        case["max_depth"])
    for i, parents in enumerate(case["parents"]):
        path = nodes[i, :length[i]].tolist()
        node = 0
        for child in path:
            assert parents[child] == node
            node = child
        kids = [k for k in range(1, len(parents)) if parents[k] == node]
        child_tokens = {case["tokens"][i][k - 1] for k in kids}
        assert int(bonus[i]) not in child_tokens


def test_greedy_fixture_walk(oracle):
    fx = json.loads((GOLDEN / "reference_fixtures.json").read_text())["greedy_walk"]
    nodes, accepted, bonus = oracle.ancestral_walk(fx["parents"], fx["tokens"], fx["argmax"])
    assert nodes == fx["nodes"] and accepted == fx["accepted"] and bonus == fx["bonus"]


def test_oracle_rejects_short_uniforms(oracle):
    case = tree_problem(1, num_requests=2, nodes=8, vocab=64)
    with pytest.raises(ValueError):
        oracle.tree_sample(case["logits"], case["row_offset"], case["parent"], case["token"],
                           case["uniforms"][:, :1], case["max_depth"])


def test_exp_coefficients_are_the_fitted_ones():
    """The polynomial constants of the GPU header and of the C restatement are
    the binary32 rounding of oracle/fit_exp_poly.py's relative-error fit."""
    import re
    from oracle.fit_exp_poly import fit
    root = Path(__file__).resolve().parents[1]
    fitted = [float(v) for v in fit().astype(np.float32)]
    for path, prefix in ((root / "specgrove_amd/csrc/sg_math.h", "SG_C"),
                         (root / "oracle/sg_oracle.c", "SGO_C")):
        text = path.read_text()
        got = [float.fromhex(re.search(rf"#define {prefix}{j} (\S+)f", text).group(1))
               for j in range(2, 6)]
        assert got == fitted, path


@pytest.mark.parametrize("vocab", [7, 2049, 4096, 151936])
def test_slab_stats_match_float64(oracle, vocab):
    """Slab maxima exact; every 2048-token slab sum E(x - m_s) within float32
    rounding of its float64 value; the row's Z their merged total."""
    rng = np.random.default_rng(vocab + 1)
    logits = (rng.standard_normal((3, vocab)) * np.array([[0.5], [3.0], [20.0]])).astype(
        np.float32)
    logits[0, :min(vocab, 2048)] = -np.inf       # a slab with no finite logit
    m, z, ss = oracle.slab_stats(logits)
    slabs = (vocab + 2047) // 2048
    for r in range(3):
        x = logits[r].astype(np.float64)
        assert m[r] == logits[r].max()
        for s in range(slabs):
            seg = x[2048 * s:2048 * (s + 1)]
            assert ss[r, s, 0] == np.float32(seg.max())
            ref = np.exp(seg - seg.max()).sum() if np.isfinite(seg.max()) else 0.0
            assert abs(ss[r, s, 1] - ref) <= 2e-6 * max(ref, 1e-30), (r, s)
        total = sum(float(ss[r, s, 1]) * np.exp(float(ss[r, s, 0]) - float(m[r]))
                    for s in range(slabs) if np.isfinite(ss[r, s, 0]))
        assert abs(z[r] - total) <= 2e-5 * total
        # the row statistics are the pass's own
        assert (m[r], z[r]) == oracle.row_stats(logits[r])


def test_slab_draw_matches_float64_inverse_cdf(oracle):
    """Away from ties the slab draw is the float64 inverse-CDF token of the
    complement, and it agrees with the complement draw."""
    rng = np.random.default_rng(12)
    vocab = 6001
    mismatches = disagree = 0
    trials = 1200
    for k in range(trials):
        row = (rng.standard_normal(vocab) * 3).astype(np.float32)
        count = int(rng.integers(0, 6))
        if k % 3 == 0:   # several children in one slab, one on a slab edge
            base = 2048 * int(rng.integers(0, vocab // 2048))
            children = np.unique(np.concatenate([[base, base + 2047],
                                                 base + rng.integers(0, 2048, count)]))
            children = children[children < vocab]
        else:
            children = rng.choice(vocab, size=count, replace=False)
        row[children[:2]] += 4.0
        u = np.float32(rng.random())
        m, _, ss = oracle.slab_stats(row[None])
        token, total = oracle.slab_draw(row, float(m[0]), ss[0], children, u)
        e = np.exp(row.astype(np.float64) - float(m[0]))
        e[children] = 0.0
        c = np.cumsum(e)
        thr = float(u) * c[-1]
        expect = int(np.searchsorted(c, thr, side="right"))
        assert token not in set(children.tolist()) and 0 <= token < vocab
        assert abs(total - c[-1]) / c[-1] < 1e-5
        if token != expect:
            mismatches += 1
            lo = min(token, expect)
            assert abs(c[lo] - thr) / c[-1] < 1e-5
        other, _ = oracle.complement_draw(row, float(m[0]), children, u)
        disagree += other != token
    assert mismatches <= trials // 200 and disagree <= trials // 200


def test_slab_draw_fallbacks(oracle):
    vocab = 600
    row = np.full(vocab, -np.inf, np.float32)
    row[[2, 599]] = 0.0                      # all mass on the two children
    m, _, ss = oracle.slab_stats(row[None])
    token, total = oracle.slab_draw(row, float(m[0]), ss[0], [2, 599], np.float32(0.3))
    assert total == 0.0 and token == 598     # largest non-child token
    flat = np.full(vocab, -np.inf, np.float32)
    m, _, ss = oracle.slab_stats(flat[None])
    assert oracle.slab_draw(flat, float(m[0]), ss[0], [], np.float32(0.5))[0] == vocab - 1
    # u just below 1 lands on the last token with mass
    row = np.zeros(vocab, np.float32)
    row[vocab - 1] = -np.inf
    m, _, ss = oracle.slab_stats(row[None])
    token, _ = oracle.slab_draw(row, float(m[0]), ss[0], [5], np.float32(1.0 - 2 ** -24))
    assert token == vocab - 2
    token, _ = oracle.slab_draw(row, float(m[0]), ss[0], [0], np.float32(0.0))
    assert token == 1
