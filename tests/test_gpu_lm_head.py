"""GPU parity of the LM head (sg_lm_head) and of the lazy-projection walk.

* Logits: the kernel's bf16 logits against an fp32 product of the same bf16
  inputs, within bf16 rounding: |kernel - ref| <= 2**-8 * |ref| + 1e-3 * s,
  s = the largest |ref| of the case.
* Statistics: bit-exact against the oracle's restatement computed from the
  kernel's own logits (tile pairs and row max / sum).
* Lazy projection: projecting the internal rows, walking, then projecting the
  reached leaves gives exactly the decisions of projecting every row, and
  those equal the oracle's on the kernel's logits and statistics.
"""
import numpy as np
import pytest
import torch

from specgrove_amd import ops, verify
from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu


def _inputs(device, rows, hidden, vocab, seed, scale=2.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    h = torch.randn((rows, hidden), generator=g).to(torch.bfloat16)
    w = (torch.randn((vocab, hidden), generator=g) * (scale / hidden ** 0.5)).to(torch.bfloat16)
    return h.to(device), w.to(device)


def _check_head(head, hidden, weight, index, oracle, threads=8):
    sel = hidden if index is None else hidden[index.long()]
    ref = sel.float() @ weight.float().T
    got = head.logits.float()
    err = (got - ref).abs()
    bound = ref.abs() * 2.0 ** -8 + 1e-3 * ref.abs().max()
    assert bool((err <= bound).all()), float((err - bound).max())
    assert int(head.status.item()) == 0
    logits = got.cpu().numpy()
    pairs, m, z = oracle.lm_head_stats(logits, threads=threads)
    tiles = head.tile_stats.cpu().numpy()
    assert np.array_equal(tiles.view(np.uint32), pairs.view(np.uint32))
    assert np.array_equal(head.row_max.cpu().numpy().view(np.uint32), m.view(np.uint32))
    assert np.array_equal(head.row_sum.cpu().numpy().view(np.uint32), z.view(np.uint32))


@pytest.mark.parametrize("rows,hidden,vocab,gather", [
    (1, 64, 1, False), (37, 128, 1000, True), (300, 256, 2049, True),
    (513, 64, 128, False), (256, 192, 255, True), (70, 128, 1153, False),
    (260, 128, 3000, True), (129, 256, 700, True), (256, 512, 256, False)])
def test_lm_head_small_shapes(device, oracle, rows, hidden, vocab, gather):
    print(f"lm_head rows={rows} H={hidden} V={vocab} gather={gather}", flush=True)
    n_hidden = rows * 2 if gather else rows
    h, w = _inputs(device, n_hidden, hidden, vocab, seed=rows + vocab)
    index = None
    if gather:
        perm = torch.randperm(n_hidden, generator=torch.Generator().manual_seed(rows))[:rows]
        index = perm.to(torch.int32).to(device)
    head = ops.lm_head(h, w, index)
    torch.cuda.synchronize()
    _check_head(head, h, w, index, oracle)


def test_lm_head_qwen3_8b_shape(device, oracle):
    """H = 4096, V = 151,936 (Qwen3-8B's untied head), 300 gathered rows."""
    print("lm_head Qwen3-8B shape, 300 rows", flush=True)
    h, w = _inputs(device, 600, 4096, 151936, seed=8)
    index = torch.arange(1, 600, 2, dtype=torch.int32, device=device)
    head = ops.lm_head(h, w, index)
    torch.cuda.synchronize()
    _check_head(head, h, w, index, oracle)


def test_lm_head_reports_out_of_range_rows(device):
    h, w = _inputs(device, 8, 64, 300, seed=1)
    index = torch.tensor([0, 3, 8, 2], dtype=torch.int32, device=device)
    head = ops.lm_head(h, w, index)
    assert int(head.status.item()) == -1
    with pytest.raises(ValueError):
        ops.lm_head(h, w[:, :32].contiguous())  # hidden sizes disagree
    with pytest.raises(ValueError):
        ops.lm_head(h[:, :48].contiguous(), w[:, :48].contiguous())  # not a multiple of 64


def _wave(device, seed, sizes, hidden=512, vocab=151936, boost=15.0):
    """Trees whose child tokens are likely in their parent's row: each parent's
    hidden state leans towards its children's head rows."""
    rng = np.random.default_rng(seed)
    parents, tokens = [], []
    for size in sizes:
        p = W.random_parent_tree(size, rng, max_depth=8)
        parents.append(p)
        tokens.append(W.random_tokens(p, vocab, rng))
    total = sum(sizes)
    h, w = _inputs(device, total, hidden, vocab, seed=seed, scale=1.5)
    h = h.float()
    wf = w.float()
    offset = 0
    for p, t in zip(parents, tokens):
        for k in range(1, len(p)):
            row = wf[t[k - 1]]
            h[offset + p[k]] += boost * row / row.dot(row)
        offset += len(p)
    return parents, tokens, h.to(torch.bfloat16), w


def _uniforms(parents, device, seed):
    depths = [max(W.depths_of(p)) for p in parents]
    stride = 2 * (max(depths) + 1)
    u = torch.zeros((len(parents), stride), dtype=torch.float32, device=device)
    for i, d in enumerate(depths):
        g = torch.Generator(device=device).manual_seed(seed + i)
        u[i, :2 * (d + 1)] = torch.rand(2 * (d + 1), dtype=torch.float32, device=device,
                                        generator=g)
    return u, max(depths)


@pytest.mark.parametrize("seed", [0, 1])
def test_lazy_projection_equals_full_projection_and_oracle(device, oracle, seed):
    sizes = [1, 2, 16, 9, 32, 5, 16, 3, 8, 24, 12, 32, 4, 16, 7, 20]
    print(f"lazy projection wave seed={seed}, {len(sizes)} requests", flush=True)
    parents, tokens, hidden, weight = _wave(device, seed, sizes)
    uniforms, max_depth = _uniforms(parents, device, 1000 * seed)
    count = len(sizes)
    ro = np.zeros(count + 1, np.int32)
    np.cumsum(sizes, out=ro[1:])
    parent = np.concatenate([np.asarray(p, np.int32) for p in parents])
    token = np.concatenate([np.asarray([-1] + t, np.int32) for t in tokens])
    t_ro, t_parent, t_token = (torch.from_numpy(a).to(device) for a in (ro, parent, token))

    # Full projection: every row.
    full_head = ops.lm_head(hidden, weight)
    full = ops.tree_sample_projected(full_head.logits, t_ro, t_parent, t_token, uniforms,
                                     max_depth, row_max=full_head.row_max,
                                     row_sum=full_head.row_sum)
    # Oracle on the kernel's logits and its own restated statistics.
    logits = full_head.logits.float().cpu().numpy()
    _, om, oz = oracle.lm_head_stats(logits, threads=8)
    assert np.array_equal(full_head.row_sum.cpu().numpy().view(np.uint32), oz.view(np.uint32))
    o_nodes, o_len, o_bonus, o_leaf = oracle.tree_sample_mapped(
        logits, ro, parent, token, uniforms.cpu().numpy(), max_depth, None, om, oz, threads=8)
    f_len = full.accept_len.cpu().numpy()
    np.testing.assert_array_equal(f_len, o_len)
    np.testing.assert_array_equal(full.accept_nodes.cpu().numpy()[:, :max_depth], o_nodes)
    np.testing.assert_array_equal(full.bonus.cpu().numpy(), o_bonus)
    assert (full.terminal_leaf.cpu().numpy() == -1).all() and int(full.status.item()) == 0
    assert f_len.max() >= 3 and (f_len == 0).any(), f_len  # deep and stopped walks

    # Lazy projection through the verifier (same uniforms from the same seeds).
    gens = [torch.Generator(device=device).manual_seed(1000 * seed + i) for i in range(count)]
    lazy = verify.tree_verify_hip_lazy_projection_batched(parents, tokens, hidden, weight,
                                                          generators=gens)
    for i, (nodes, toks, bonus, stats) in enumerate(lazy):
        assert nodes == [int(v) for v in o_nodes[i, :o_len[i]]], i
        assert toks == [tokens[i][v - 1] for v in nodes]
        assert bonus == int(o_bonus[i]), i
        internal = len(set(parents[i][1:]))
        assert stats["internal_projected_rows"] == internal
        assert stats["projected_rows"] == internal + stats["leaf_projected_rows"]
    # Some walks reached a leaf (second projection), some stopped inside.
    reached = [s["leaf_projected_rows"] for _, _, _, s in lazy]
    assert 0 < sum(reached) < count, reached

    # The internal rows' logits of a gathered call are the full call's rows.
    internal_rows = np.flatnonzero(np.isin(np.arange(ro[-1]),
                                           [ro[i] + v for i, p in enumerate(parents)
                                            for v in set(p[1:])])).astype(np.int32)
    part = ops.lm_head(hidden, weight, torch.from_numpy(internal_rows).to(device))
    assert torch.equal(part.logits, full_head.logits[torch.from_numpy(internal_rows).long()
                                                     .to(device)])
    assert torch.equal(part.row_sum, full_head.row_sum[torch.from_numpy(internal_rows).long()
                                                       .to(device)])


def test_lazy_projection_rejects_bad_calls_after_starting_the_projection(device):
    """The verifier starts the internal-row projection before validating the
    trees; a bad tree, token or hidden shape still raises the same error,
    and the generators are left untouched."""
    sizes = [4, 3, 5]
    parents, tokens, hidden, weight = _wave(device, 7, sizes)
    gens = [torch.Generator(device=device).manual_seed(70 + i) for i in range(len(sizes))]
    states = [g.get_state().clone() for g in gens]
    bad_parent = [list(p) for p in parents]
    bad_parent[1][2] = 5                       # a parent after its node
    with pytest.raises(ValueError, match="Invalid probability-tree topology"):
        verify.tree_verify_hip_lazy_projection_batched(bad_parent, tokens, hidden, weight,
                                                       generators=gens)
    bad_token = [list(t) for t in tokens]
    bad_token[2][0] = weight.shape[0]
    with pytest.raises(ValueError, match="outside the Target vocabulary"):
        verify.tree_verify_hip_lazy_projection_batched(parents, bad_token, hidden, weight,
                                                       generators=gens)
    with pytest.raises(ValueError, match="hidden shape mismatch"):
        verify.tree_verify_hip_lazy_projection_batched(parents, tokens, hidden[:-1], weight,
                                                       generators=gens)
    torch.cuda.synchronize()
    assert all(torch.equal(g.get_state(), s) for g, s in zip(gens, states))
    # A good call after the bad ones is unaffected.
    lazy = verify.tree_verify_hip_lazy_projection_batched(parents, tokens, hidden, weight,
                                                          generators=gens)
    assert len(lazy) == len(sizes)


def test_packed_weight_layout(device):
    """sg_lm_head_pack_weight: tile t, stage s holds rows 256t.. x dims 32s..,
    row-major, zero past the vocabulary (checked against a host re-layout)."""
    g = torch.Generator(device="cpu").manual_seed(11)
    vocab, hsize = 300, 128
    w = (torch.randn(vocab, hsize + 8, generator=g) * 0.1).to(torch.bfloat16)[:, :hsize]
    packed = ops.pack_lm_head(w.to(device))
    torch.cuda.synchronize()
    tiles, steps = (vocab + 255) // 256, hsize // 32
    padded = torch.zeros(tiles * 256, hsize, dtype=torch.bfloat16)
    padded[:vocab] = w
    want = padded.view(tiles, 256, steps, 32).permute(0, 2, 1, 3).reshape(-1)
    assert packed.shape == (vocab, hsize)
    assert torch.equal(packed.packed.cpu(), want)


@pytest.mark.parametrize("rows", [40, 64, 130, 300])
@pytest.mark.parametrize("vocab", [151936, 1000])
def test_packed_lm_head_equals_row_major(device, rows, vocab):
    """The packed-weight kernel gives the row-major kernel's outputs bit for bit."""
    g = torch.Generator(device=device).manual_seed(rows + vocab)
    hidden = (torch.randn(512, 512, device=device, generator=g)).to(torch.bfloat16)
    weight = (torch.randn(vocab, 512, device=device, generator=g) * 0.05).to(torch.bfloat16)
    index = torch.randperm(512, device=device, generator=g)[:rows].to(torch.int32)
    plain = ops.lm_head(hidden, weight, index)
    packed = ops.lm_head(hidden, ops.pack_lm_head(weight), index)
    torch.cuda.synchronize()
    assert torch.equal(plain.logits, packed.logits)
    for name in ("tile_stats", "row_max", "row_sum", "status"):
        assert torch.equal(getattr(plain, name), getattr(packed, name)), name


def test_lazy_projection_with_packed_head(device):
    """The lazy verifier given the packed head decides exactly as with the
    plain weight."""
    sizes = [1, 9, 16, 3, 24, 7]
    parents, tokens, hidden, weight = _wave(device, 3, sizes)
    gens = lambda: [torch.Generator(device=device).manual_seed(300 + i)  # noqa: E731
                    for i in range(len(sizes))]
    plain = verify.tree_verify_hip_lazy_projection_batched(parents, tokens, hidden, weight,
                                                           generators=gens())
    packed = verify.tree_verify_hip_lazy_projection_batched(parents, tokens, hidden,
                                                            ops.pack_lm_head(weight),
                                                            generators=gens())
    assert [r[:3] for r in plain] == [r[:3] for r in packed]


def test_lazy_projection_validate_flag_changes_no_decision(device):
    """validate=False skips only the statistics checks (finite, positive sums):
    the decisions and projection counts equal those of validate=True."""
    sizes = [1, 9, 16, 3, 24, 7]
    parents, tokens, hidden, weight = _wave(device, 5, sizes)
    gens = lambda: [torch.Generator(device=device).manual_seed(900 + i)  # noqa: E731
                    for i in range(len(sizes))]
    checked = verify.tree_verify_hip_lazy_projection_batched(parents, tokens, hidden, weight,
                                                             generators=gens(), validate=True)
    unchecked = verify.tree_verify_hip_lazy_projection_batched(parents, tokens, hidden, weight,
                                                               generators=gens(), validate=False)
    assert checked == unchecked


@pytest.mark.parametrize("hidden_size", [512, 64])
def test_lm_head_row_tiles_agree_bit_for_bit(device, hidden_size):
    """Every kernel gives a row the same logits and statistics bit for bit:
    the 256-row ping-pong kernel (above 128 rows; the 128-row-per-wave kernel
    at a hidden size of 64), the 128-row and the 64-row tiles.  The lazy
    projection projects internal rows and reached leaves in calls of
    different sizes, so its decisions rely on this."""
    print(f"lm_head row tiles H={hidden_size}", flush=True)
    g = torch.Generator(device=device).manual_seed(hidden_size)
    hidden = torch.randn(400, hidden_size, device=device, generator=g).to(torch.bfloat16)
    weight = (torch.randn(3001, hidden_size, device=device, generator=g) * 0.05).to(torch.bfloat16)
    rows = torch.randperm(400, device=device, generator=g)[:300].to(torch.int32)
    big = ops.lm_head(hidden, weight, rows)
    torch.cuda.synchronize()
    for n in (100, 40):
        part = ops.lm_head(hidden, weight, rows[:n].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(part.logits, big.logits[:n]), n
        for name in ("tile_stats", "row_max", "row_sum"):
            assert torch.equal(getattr(part, name), getattr(big, name)[:n]), (n, name)


@pytest.mark.parametrize("vocab", [131372, 131528])
def test_lm_head_leaf_half_tiles_agree_bit_for_bit(device, oracle, vocab):
    """The 64- and 128-row kernels run the vocabulary tiles of their last,
    partial round of workgroups (above 512 and 256 tiles) as 128-token
    halves.  At 514 tiles (these two vocabularies) tiles 512 and 513 are
    split; the last half holds no token at 131,372 and 72 at 131,528.  The
    halves give the rows the same logits and statistics, bit for bit, as the
    200-row call (whole tiles), with the row-major and the packed weight."""
    print(f"lm_head leaf half tiles V={vocab}", flush=True)
    g = torch.Generator(device=device).manual_seed(vocab)
    hidden = torch.randn(256, 64, device=device, generator=g).to(torch.bfloat16)
    weight = (torch.randn(vocab, 64, device=device, generator=g) * 0.05).to(torch.bfloat16)
    rows = torch.randperm(256, device=device, generator=g)[:200].to(torch.int32)
    packed = ops.pack_lm_head(weight)
    for w in (weight, packed):
        big = ops.lm_head(hidden, w, rows)  # 200 rows at H = 64: the four-wave 256-row kernel
        torch.cuda.synchronize()
        assert big.status.item() == 0
        for n in (90, 60):  # the 128-row and the 64-row kernels, with half tiles
            part = ops.lm_head(hidden, w, rows[:n].contiguous())
            torch.cuda.synchronize()
            assert part.status.item() == 0
            assert torch.equal(part.logits, big.logits[:n]), n
            for name in ("tile_stats", "row_max", "row_sum"):
                assert torch.equal(getattr(part, name), getattr(big, name)[:n]), (n, name)
        # and the 64-row call is the fp32 product within bf16 rounding, with
        # the oracle's statistics of its logits
        _check_head(part, hidden, weight, rows[:60], oracle)
