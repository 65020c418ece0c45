"""GPU parity of the tree sampler against the CPU oracle: bit-exact."""
import os

import numpy as np
import pytest
import torch

from specgrove_amd import ops
from specgrove_amd import workloads as W
from tests.sampler_cases import tree_problem

pytestmark = pytest.mark.gpu


def _run_gpu(case, device):
    t = {k: torch.from_numpy(case[k]).to(device)
         for k in ("logits", "row_offset", "parent", "token", "uniforms")}
    res = ops.tree_sample(t["logits"], t["row_offset"], t["parent"], t["token"],
                          t["uniforms"], case["max_depth"])
    torch.cuda.synchronize()
    return {k: getattr(res, k).cpu().numpy() for k in
            ("accept_nodes", "accept_len", "bonus", "keep_rows", "row_max", "row_sum", "status")}


def _check_case(case, device, oracle):
    gpu = _run_gpu(case, device)
    nodes, length, bonus, m, z = oracle.tree_sample(
        case["logits"], case["row_offset"], case["parent"], case["token"],
        case["uniforms"], case["max_depth"])
    assert gpu["status"][0] == 0
    np.testing.assert_array_equal(gpu["row_max"], m)
    assert np.array_equal(gpu["row_sum"].view(np.uint32), z.view(np.uint32)), \
        "row sums differ in bits"
    np.testing.assert_array_equal(gpu["accept_len"], length)
    np.testing.assert_array_equal(gpu["accept_nodes"][:, :case["max_depth"]], nodes)
    np.testing.assert_array_equal(gpu["bonus"], bonus)
    keep = np.full((len(length), case["max_depth"] + 1), -1, np.int32)
    keep[:, 0] = 0
    for i, a in enumerate(length):
        keep[i, 1:1 + a] = nodes[i, :a]
    np.testing.assert_array_equal(gpu["keep_rows"], keep)
    return gpu


def test_exp_bit_exact(device, oracle):
    xs = np.concatenate([
        np.linspace(-130, 1, 400001, dtype=np.float32),
        np.array([0.0, -0.0, -87.0, np.nextafter(np.float32(-87.0), np.float32(0)),
                  np.nextafter(np.float32(-87.0), np.float32(-100)), -1e-30, 1e-30,
                  -103.0, -103.3, -104.0, -120.0, -121.0, -1e30,
                  -np.inf, np.nan, 88.0, 89.0, np.inf], np.float32),
        -np.abs(np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 30),
    ])
    got = ops.exp_probe(torch.from_numpy(xs).to(device)).cpu().numpy()
    want = oracle.exp_f32(xs)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("vocab", [1, 3, 100, 2048, 2049, 4096, 4097, 151936])
def test_row_stats_bit_exact(device, oracle, vocab):
    rng = np.random.default_rng(vocab)
    rows = 9
    x = (rng.standard_normal((rows, vocab)) * 4).astype(np.float32)
    x[1] -= 200.0                      # deep negative row
    x[2, ::7] = -np.inf                # masked tokens
    x[3, :] = 5.0                      # constant row
    m, z = ops.row_stats(torch.from_numpy(x).to(device))
    m, z = m.cpu().numpy(), z.cpu().numpy()
    for r in range(rows):
        om, oz = oracle.row_stats(x[r])
        assert m[r] == om
        assert np.float32(z[r]).view(np.uint32) == np.float32(oz).view(np.uint32), (r, z[r], oz)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_tiny_vocab_trees_bit_exact(device, oracle, seed):
    case = tree_problem(seed, num_requests=6, nodes=[16, 1, 9, 16, 3, 12], vocab=4096)
    _check_case(case, device, oracle)


@pytest.mark.parametrize("vocab,nodes", [(2, [2, 2, 1, 2, 2]), (5, [2, 3, 4, 1, 2]),
                                         (4097, [12, 12, 12, 12, 12])])
def test_odd_vocab_bit_exact(device, oracle, vocab, nodes):
    case = tree_problem(10 + vocab, num_requests=5, nodes=nodes, vocab=vocab, child_boost=2.0)
    _check_case(case, device, oracle)


def test_extreme_uniforms_bit_exact(device, oracle):
    case = tree_problem(7, num_requests=9, nodes=16, vocab=4096, extreme_uniforms=True)
    gpu = _check_case(case, device, oracle)
    assert (gpu["accept_len"][0::3] >= 1).any()


def test_qwen_vocab_bit_exact(device, oracle):
    case = tree_problem(11, num_requests=8, nodes=32, vocab=151936, random_trees=False,
                        child_boost=18.0)
    gpu = _check_case(case, device, oracle)
    assert gpu["accept_len"].max() >= 1


def test_long_context_trees_bit_exact(device, oracle):
    """The long-context wave's 128 trees (1 to 128 nodes, canonical, depth up
    to 16) with every packed row sampled, at vocabulary 8192."""
    wl = W.long_context_workload()
    case = tree_problem(31, len(wl.parents), None, 8192, trees=wl.parents, child_boost=10.0)
    assert case["logits"].shape[0] == wl.total_rows == 4096
    gpu = _check_case(case, device, oracle)
    assert gpu["accept_len"].max() >= 3


def test_exit_draws_spread_over_the_vocabulary(device, oracle):
    """Unboosted children: most walks exit at the root, and the 64 residual
    draws land in lines all over a 151,936-token row (the exit search starts
    at the first line that may hold the bonus)."""
    case = tree_problem(21, num_requests=64, nodes=3, vocab=151936, child_boost=0.0)
    gpu = _check_case(case, device, oracle)
    assert len(set((gpu["bonus"] // 256).tolist())) > 32  # many distinct lines


def test_wide_exit_node(device, oracle):
    """Roots with 200 children: the children are found by several 64-lane
    ballots, and 200 tokens are excluded from the residual draw; extreme
    uniforms included."""
    trees = [[-1] + [0] * 200 for _ in range(6)]
    case = tree_problem(22, num_requests=6, nodes=None, vocab=8192, child_boost=0.5,
                        trees=trees, extreme_uniforms=True)
    _check_case(case, device, oracle)


def test_golden_fixture(device):
    from pathlib import Path
    path = Path(__file__).parent / "golden" / "sampler_tiny.npz"
    data = np.load(path, allow_pickle=False)
    case = {k: data[k] for k in ("logits", "row_offset", "parent", "token", "uniforms")}
    case["max_depth"] = int(data["max_depth"])
    gpu = _run_gpu(case, device)
    np.testing.assert_array_equal(gpu["accept_len"], data["accept_len"])
    np.testing.assert_array_equal(gpu["accept_nodes"], data["accept_nodes"])
    np.testing.assert_array_equal(gpu["bonus"], data["bonus"])


def test_sampler_workload_full_size(device, oracle):
    """64 requests x 32 nodes, vocab 151936: every request bit-exact."""
    wl, logits, uniforms = W.sampler_workload(device)
    parent, token = wl.flat_parent_token()
    case = dict(logits=logits.cpu().numpy(), row_offset=wl.row_offset, parent=parent,
                token=token, uniforms=uniforms.cpu().numpy(), max_depth=wl.max_depth)
    gpu = _check_case(case, device, oracle)
    assert gpu["accept_len"].max() >= 1


def test_invalid_arguments_raise(device):
    logits = torch.zeros((4, 16), device=device)
    ro = torch.tensor([0, 4], dtype=torch.int32, device=device)
    par = torch.tensor([-1, 0, 0, 1], dtype=torch.int32, device=device)
    tok = torch.tensor([0, 1, 2, 3], dtype=torch.int32, device=device)
    u = torch.zeros((1, 2), device=device)
    with pytest.raises(ValueError):
        ops.tree_sample(logits, ro, par, tok, u, max_depth=2)
    with pytest.raises(ValueError):
        ops.tree_sample(logits.double(), ro, par, tok, torch.zeros((1, 6), device=device), 2)


@pytest.mark.parametrize("seed", range(8 + int(os.environ.get("SG_RANDOM_CASES", "0"))))
def test_random_trees_vocabularies_and_acceptance_rates(device, oracle, seed):
    """Random request counts, tree sizes (a lone root to 200 nodes), chains up
    to depth 40, vocabularies around the 4-token, 256-token line and
    2048-token slab edges, child boosts from none (most walks exit at the
    root) to strong (long accepted paths), and extreme uniforms on some
    seeds: bit-exact against the oracle.  SG_RANDOM_CASES=N adds N seeds."""
    rng = np.random.default_rng(1000 + seed)
    vocab = int(rng.choice([5, 255, 257, 2047, 2049, 6143, 32003, 151936]))
    n = int(rng.integers(1, 13))
    trees = []
    for _ in range(n):
        form = rng.integers(0, 3)
        size = int(rng.choice([1, 2, 9, 33, 80, 200]))
        if form == 0:
            trees.append(W.random_parent_tree(size, rng, max_depth=int(rng.integers(1, 12))))
        elif form == 1:
            depth = min(size, 41)
            trees.append([-1] + list(range(depth - 1)))
        else:
            trees.append(W.canonical_tree(size, rng))
    # child tokens are distinct per parent, so no parent may have more
    # children than the vocabulary has tokens
    widest = max(max(np.bincount(np.asarray(p[1:]), minlength=1)) if len(p) > 1 else 0
                 for p in trees)
    vocab = max(vocab, int(widest))
    case = tree_problem(2000 + seed, n, None, vocab, trees=trees,
                        child_boost=float(rng.choice([0.0, 3.0, 8.0, 14.0])),
                        logit_std=float(rng.choice([0.5, 3.0, 6.0])),
                        extreme_uniforms=bool(seed % 3 == 0))
    _check_case(case, device, oracle)


def test_reused_outputs_must_fit_the_call(device, oracle):
    """Caller-supplied outputs are checked against n, R and max_depth, and the
    status word left by an earlier broken call is cleared by the next call."""
    case = tree_problem(51, num_requests=4, nodes=[9, 5, 7, 3], vocab=1000)
    t = {k: torch.from_numpy(case[k]).to(device)
         for k in ("logits", "row_offset", "parent", "token", "uniforms")}
    res = ops.tree_sample(t["logits"], t["row_offset"], t["parent"], t["token"],
                          t["uniforms"], case["max_depth"])
    small = tree_problem(52, num_requests=2, nodes=[3, 2], vocab=1000)
    ts = {k: torch.from_numpy(small[k]).to(device)
          for k in ("logits", "row_offset", "parent", "token", "uniforms")}
    with pytest.raises(ValueError, match="out\\."):
        ops.tree_sample(ts["logits"], ts["row_offset"], ts["parent"], ts["token"],
                        ts["uniforms"], small["max_depth"], out=res)
    # A request whose rows run past num_rows is a broken walk (status EINVAL,
    # accept length -1); the next call on the same outputs starts clean.
    bad_offset = t["row_offset"].clone()
    bad_offset[-1] += 3
    parent_pad = torch.cat([t["parent"], torch.zeros(3, dtype=torch.int32, device=device)])
    token_pad = torch.cat([t["token"], torch.zeros(3, dtype=torch.int32, device=device)])
    res = ops.tree_sample(t["logits"], bad_offset, parent_pad, token_pad, t["uniforms"],
                          case["max_depth"], out=res)
    torch.cuda.synchronize()
    assert int(res.status.item()) == ops._lib.SG_EINVAL
    assert int(res.accept_len[-1].item()) == -1
    res = ops.tree_sample(t["logits"], t["row_offset"], t["parent"], t["token"],
                          t["uniforms"], case["max_depth"], out=res)
    torch.cuda.synchronize()
    assert int(res.status.item()) == 0
    nodes, length, bonus, _, _ = oracle.tree_sample(
        case["logits"], case["row_offset"], case["parent"], case["token"],
        case["uniforms"], case["max_depth"])
    np.testing.assert_array_equal(res.accept_len.cpu().numpy(), length)
    np.testing.assert_array_equal(res.bonus.cpu().numpy(), bonus)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("vocab,pad", [(6144, 64), (4100, 4), (4099, 1), (3000, 17)])
def test_padded_logits_rows(device, oracle, dtype, vocab, pad):
    """Logits rows inside a wider buffer (row stride above the vocabulary):
    the statistics and the draw read only the first `vocab` tokens of each
    row, on the 4-token vector path (stride and vocab multiples of 4) and on
    the element path, bit-exact against the oracle on the same tokens."""
    case = tree_problem(600 + vocab + pad, num_requests=5, nodes=[7, 1, 12, 4, 9], vocab=vocab)
    rows = case["logits"].shape[0]
    wide = torch.full((rows, vocab + pad), float("nan"), dtype=torch.float32)
    wide[:, :vocab] = torch.from_numpy(case["logits"])
    logits = wide.to(dtype).to(device)[:, :vocab]
    assert logits.stride(0) == vocab + pad
    res = ops.tree_sample(logits, torch.from_numpy(case["row_offset"]).to(device),
                          torch.from_numpy(case["parent"]).to(device),
                          torch.from_numpy(case["token"]).to(device),
                          torch.from_numpy(case["uniforms"]).to(device), case["max_depth"])
    torch.cuda.synchronize()
    widened = logits.float().cpu().numpy()
    nodes, length, bonus, m, z = oracle.tree_sample(
        widened, case["row_offset"], case["parent"], case["token"], case["uniforms"],
        case["max_depth"])
    assert int(res.status.item()) == 0
    np.testing.assert_array_equal(res.row_max.cpu().numpy(), m)
    assert np.array_equal(res.row_sum.cpu().numpy().view(np.uint32), z.view(np.uint32))
    np.testing.assert_array_equal(res.accept_len.cpu().numpy(), length)
    np.testing.assert_array_equal(res.accept_nodes.cpu().numpy()[:, :case["max_depth"]], nodes)
    np.testing.assert_array_equal(res.bonus.cpu().numpy(), bonus)


@pytest.mark.parametrize("vocab", [7, 2049, 4097, 6002, 151936])
def test_slab_statistics_bit_exact(device, oracle, vocab):
    """The statistics pass keeps every row's slab pairs (m_s, Z_s) behind the
    per-request region of the workspace: bit for bit the oracle's, on the
    vector path (vocab a multiple of 4) and the scalar one."""
    rng = np.random.default_rng(vocab)
    rows, n = 12, 3
    logits = (rng.standard_normal((rows, vocab)) * 4).astype(np.float32)
    logits[1, :vocab // 2] = -np.inf                 # slabs with no finite logit
    case = dict(logits=logits, row_offset=np.array([0, 4, 8, 12], np.int32),
                parent=np.tile(np.array([-1, 0, 0, 1], np.int32), 3),
                token=np.tile(np.array([0, 1, 2, 3], np.int32) % vocab, 3),
                uniforms=rng.random((n, 6), dtype=np.float32), max_depth=2)
    t = {k: torch.from_numpy(case[k]).to(device)
         for k in ("logits", "row_offset", "parent", "token", "uniforms")}
    res = ops.tree_sample(t["logits"], t["row_offset"], t["parent"], t["token"],
                          t["uniforms"], case["max_depth"])
    slabs = (vocab + 2047) // 2048
    request_floats = n * (slabs * 9 + 1028)
    ws = res.workspace.view(torch.float32).cpu().numpy()
    got = ws[request_floats:request_floats + rows * slabs * 2].reshape(rows, slabs, 2)
    m, z, want = oracle.slab_stats(logits)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(res.row_sum.cpu().numpy().view(np.uint32), z.view(np.uint32))
    _check_case(case, device, oracle)
