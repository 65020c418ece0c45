"""sg_tree_sample_noalloc (static per-GPU scratch, no device allocation)
against sg_tree_sample, bit-exact, over two calls in a row on one GPU: a full
151,936-token wave and then a smaller one, so the second call runs on the
scratch contents the first left behind.  Also checked against the oracle."""
import numpy as np
import pytest
import torch

from specgrove_amd import _lib, ops
from tests.sampler_cases import tree_problem

pytestmark = pytest.mark.gpu

FIELDS = ("accept_nodes", "accept_len", "bonus", "keep_rows", "row_max", "row_sum", "status")


def _device_case(case, device):
    return {k: torch.from_numpy(case[k]).to(device)
            for k in ("logits", "row_offset", "parent", "token", "uniforms")}


def _outputs(n, rows, max_depth, device):
    # Filled with junk so that a missing write shows up as a mismatch.
    return ops.SampleResult(
        accept_nodes=torch.full((n, max(max_depth, 1)), 77, dtype=torch.int32, device=device),
        accept_len=torch.full((n,), 77, dtype=torch.int32, device=device),
        bonus=torch.full((n,), 77, dtype=torch.int32, device=device),
        keep_rows=torch.full((n, max_depth + 1), 77, dtype=torch.int32, device=device),
        row_max=torch.full((rows,), 7.0, dtype=torch.float32, device=device),
        row_sum=torch.full((rows,), 7.0, dtype=torch.float32, device=device),
        status=torch.zeros(1, dtype=torch.int32, device=device),
    )


def _host(res):
    return {k: getattr(res, k).cpu().numpy() for k in FIELDS}


def test_noalloc_matches_the_allocating_entry_point_twice(device, oracle):
    cases = [
        tree_problem(41, num_requests=16, nodes=32, vocab=151936, random_trees=False,
                     child_boost=12.0),
        tree_problem(42, num_requests=9, nodes=[16, 1, 9, 16, 3, 12, 7, 2, 5], vocab=50000,
                     child_boost=6.0),
    ]
    for case in cases:
        print(f"noalloc case: {len(case['row_offset']) - 1} requests, vocab "
              f"{case['logits'].shape[1]}", flush=True)
        t = _device_case(case, device)
        n, rows = len(case["row_offset"]) - 1, case["logits"].shape[0]
        ref = ops.tree_sample(t["logits"], t["row_offset"], t["parent"], t["token"],
                              t["uniforms"], case["max_depth"])
        out = _outputs(n, rows, case["max_depth"], device)
        got = ops.tree_sample_noalloc(t["logits"], t["row_offset"], t["parent"], t["token"],
                                      t["uniforms"], case["max_depth"], out)
        torch.cuda.synchronize()
        want, have = _host(ref), _host(got)
        for k in FIELDS:
            assert np.array_equal(have[k].view(np.uint32) if have[k].dtype == np.float32
                                  else have[k],
                                  want[k].view(np.uint32) if want[k].dtype == np.float32
                                  else want[k]), k
        assert have["status"][0] == 0
        nodes, length, bonus, _, _ = oracle.tree_sample(
            case["logits"], case["row_offset"], case["parent"], case["token"],
            case["uniforms"], case["max_depth"])
        np.testing.assert_array_equal(have["accept_len"], length)
        np.testing.assert_array_equal(have["bonus"], bonus)
        np.testing.assert_array_equal(have["accept_nodes"][:, :case["max_depth"]], nodes)


def test_noalloc_rejects_waves_beyond_its_scratch(device):
    vocab = 151936
    per_request = int(_lib.load().sg_tree_sample_workspace_bytes(1, 1, vocab))  # one row each
    n = _lib.NOALLOC_SCRATCH_BYTES // per_request + 1
    logits = torch.zeros((n, vocab), dtype=torch.float32, device=device)
    row_offset = torch.arange(n + 1, dtype=torch.int32, device=device)
    parent = torch.full((n,), -1, dtype=torch.int32, device=device)
    token = torch.zeros(n, dtype=torch.int32, device=device)
    uniforms = torch.zeros((n, 2), dtype=torch.float32, device=device)
    out = _outputs(n, n, 0, device)
    with pytest.raises(ValueError, match="static maximum"):
        ops.tree_sample_noalloc(logits, row_offset, parent, token, uniforms, 0, out)
