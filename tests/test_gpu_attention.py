"""GPU parity of the packed tree attention against the fp32 CPU oracle.

Tolerance (bf16 inputs and output): max |gpu - ref| <= 2e-2 and
mean |gpu - ref| / mean |ref| <= 1e-2.
"""
import os

import numpy as np
import pytest
import torch

from specgrove_amd import ops
from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_REL = 1e-2


def _inputs(wl, device, seed):
    tensors = wl.make_tensors("cpu", seed)
    dev = [t.to(device) for t in tensors]
    meta = dict(
        row_offset=torch.from_numpy(wl.row_offset).to(device),
        prefix_start=torch.from_numpy(wl.prefix_start).to(device),
        prefix_len=torch.from_numpy(wl.prefix_len.astype(np.int32)).to(device),
        parent=torch.from_numpy(wl.parent_flat).to(device),
    )
    return tensors, dev, meta


def _run(wl, dev, meta, device, target_units=0):
    plan = ops.plan_attention(wl.row_offset, wl.prefix_len, wl.num_q_heads, wl.num_kv_heads,
                              wl.head_dim, target_units).to(device)
    q, kc, vc, kt, vt = dev
    out = ops.tree_attention(q, kc, vc, kt, vt, meta["row_offset"], meta["prefix_start"],
                             meta["prefix_len"], meta["parent"], plan)
    torch.cuda.synchronize()
    return out.float().cpu(), plan


def _prefix_lists(wl, tensors):
    q, kc, vc, kt, vt = tensors
    ks, vs = [], []
    for i in range(wl.num_requests):
        s = int(wl.prefix_start[i])
        L = int(wl.prefix_len[i])
        ks.append(kc[:, s:s + L])
        vs.append(vc[:, s:s + L])
    return ks, vs


def _assert_close(got, ref):
    err = (got - ref).abs()
    max_abs = err.max().item()
    mean_rel = (err.mean() / ref.abs().mean()).item()
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL, (max_abs, mean_rel)


def test_tiny_head_dim_64_dense_oracle(device, oracle):
    wl = W.tiny_attention_workload(seed=1)
    tensors, dev, meta = _inputs(wl, device, 11)
    got, _ = _run(wl, dev, meta, device)
    ks, vs = _prefix_lists(wl, tensors)
    q, kc, vc, kt, vt = tensors
    ref = oracle.attention_dense(q, ks, vs, kt, vt, wl.parents)
    _assert_close(got, ref)


def test_qwen3_4b_shape_dense_oracle(device, oracle):
    wl = W.qwen3_4b_workload()
    tensors, dev, meta = _inputs(wl, device, 12)
    got, _ = _run(wl, dev, meta, device)
    ks, vs = _prefix_lists(wl, tensors)
    q, kc, vc, kt, vt = tensors
    ref = oracle.attention_dense(q, ks, vs, kt, vt, wl.parents)
    _assert_close(got, ref)


@pytest.mark.parametrize("target_units", [64, 4096])
def test_split_plans_agree_with_oracle(device, oracle, target_units):
    wl = W.qwen3_4b_workload(seed=21)
    tensors, dev, meta = _inputs(wl, device, 13)
    got, plan = _run(wl, dev, meta, device, target_units)
    if target_units == 4096:
        assert plan.merges > 0
    ks, vs = _prefix_lists(wl, tensors)
    q, kc, vc, kt, vt = tensors
    ref = torch.cat([v for _, v in sorted(oracle.attention_per_request(
        q, ks, vs, kt, vt, wl.row_offset, wl.parents).items())])
    _assert_close(got, ref)


def test_qwen3_8b_full_size_sampled_requests_and_isolation(device, oracle):
    wl = W.qwen3_8b_workload()
    tensors, dev, meta = _inputs(wl, device, 3)
    got, _ = _run(wl, dev, meta, device)
    ks, vs = _prefix_lists(wl, tensors)
    q, kc, vc, kt, vt = tensors
    picks = [0, 5, 17, 33, 63] + [int(i) for i in np.nonzero(wl.rows == 64)[0][:2]]
    refs = oracle.attention_per_request(q, ks, vs, kt, vt, wl.row_offset, wl.parents,
                                        requests=picks)
    for i, ref in refs.items():
        r0, r1 = int(wl.row_offset[i]), int(wl.row_offset[i + 1])
        _assert_close(got[r0:r1], ref)
    # Request isolation: poisoning request 7's cache and tree rows leaves every
    # other request's output byte-identical (the reference's isolation audit).
    victim = 7
    kc2, vc2, kt2 = dev[1].clone(), dev[2].clone(), dev[3].clone()
    s, L = int(wl.prefix_start[victim]), int(wl.prefix_len[victim])
    kc2[:, s:s + L] = 7.0
    vc2[:, s:s + L] = -3.0
    r0, r1 = int(wl.row_offset[victim]), int(wl.row_offset[victim + 1])
    kt2[r0:r1] = 5.0
    poisoned, _ = _run(wl, [dev[0], kc2, vc2, kt2, dev[4]], meta, device)
    keep = torch.ones(wl.total_rows, dtype=torch.bool)
    keep[r0:r1] = False
    assert torch.equal(poisoned[keep], got[keep])
    assert not torch.equal(poisoned[~keep], got[~keep])


def test_strided_query_and_output_views(device, oracle):
    wl = W.tiny_attention_workload(seed=3, num_q_heads=8, num_kv_heads=2, head_dim=128)
    tensors, dev, meta = _inputs(wl, device, 14)
    q, kc, vc, kt, vt = dev
    # q stored head-major [Hq, R, D] and viewed as [R, Hq, D]
    q_hm = q.transpose(0, 1).contiguous().transpose(0, 1)
    plan = ops.plan_attention(wl.row_offset, wl.prefix_len, 8, 2, 128).to(device)
    out_hm = torch.empty((8, wl.total_rows, 128), dtype=torch.bfloat16, device=device)
    ops.tree_attention(q_hm, kc, vc, kt, vt, meta["row_offset"], meta["prefix_start"],
                       meta["prefix_len"], meta["parent"], plan, out=out_hm.transpose(0, 1))
    torch.cuda.synchronize()
    got = out_hm.transpose(0, 1).float().cpu()
    ks, vs = _prefix_lists(wl, tensors)
    qc, kcc, vcc, ktc, vtc = tensors
    ref = oracle.attention_dense(qc, ks, vs, ktc, vtc, wl.parents)
    _assert_close(got, ref)


def test_long_prefix_and_single_row_requests(device, oracle):
    """Tier-1 requests (root row only) and 8k-32k prefixes, sampled."""
    wl = W.long_context_workload()
    keep = [i for i in range(wl.num_requests) if wl.rows[i] == 1][:2] + [0, 1]
    sub = W.AttentionWorkload("long_sub", 32, 8, 128, wl.prefix_len[keep],
                              [wl.parents[i] for i in keep], [wl.tokens[i] for i in keep],
                              int(wl.prefix_len[keep].max()) + 192)
    tensors, dev, meta = _inputs(sub, device, 15)
    got, _ = _run(sub, dev, meta, device)
    ks, vs = _prefix_lists(sub, tensors)
    q, kc, vc, kt, vt = tensors
    refs = oracle.attention_per_request(q, ks, vs, kt, vt, sub.row_offset, sub.parents)
    for i, ref in refs.items():
        r0, r1 = int(sub.row_offset[i]), int(sub.row_offset[i + 1])
        _assert_close(got[r0:r1], ref)


def _tree_of_form(form, rows, rng):
    if rows == 0:
        return []
    if form == "chain":
        return [-1] + list(range(rows - 1))
    if form == "star":
        return [-1] + [0] * (rows - 1)
    if form == "binary":
        return [-1] + [(k - 1) // 2 for k in range(1, rows)]
    return [-1] + [int(rng.integers(0, k)) for k in range(1, rows)]


def _more_random_cases(count):
    """SG_RANDOM_CASES=N adds N seeded cases to the random test (a longer sweep)."""
    heads = [(8, 8), (16, 2), (32, 2), (4, 1), (32, 8), (64, 8), (32, 4), (16, 16), (128, 8)]
    rng = np.random.default_rng(77)
    cases = []
    for k in range(count):
        hq, hkv = heads[int(rng.integers(len(heads)))]
        cases.append((hq, hkv, int(rng.choice([64, 128])), 100 + k,
                      [None, 3.0][int(rng.integers(2))]))
    return cases


@pytest.mark.parametrize("hq,hkv,dim,seed,q_scale", [
    (8, 8, 128, 0, None), (16, 2, 64, 1, None), (32, 2, 128, 2, 3.0),
    (4, 1, 64, 3, 3.0), (32, 8, 128, 4, None), (64, 8, 64, 5, 3.0)]
    + _more_random_cases(int(os.environ.get("SG_RANDOM_CASES", "0"))))
def test_random_head_groups_prefixes_and_tree_forms(device, oracle, hq, hkv, dim, seed,
                                                    q_scale):
    """Head groups 1-16, head dims 64 and 128, prefixes of 0 to 2049 keys around
    the 32-key tile edges, chains, stars, binary and random trees from 1 to the
    256-row maximum, and an empty request.  Few units per wave, so the planner
    also splits prefixes (partials and the merge kernel).  Sharp scores
    (q_scale 3) make the running maximum jump, which forces the deferred
    softmax rescale."""
    rng = np.random.default_rng(100 + seed)
    n = 9
    prefix = rng.choice([0, 1, 31, 32, 33, 65, 127, 500, 2049], n).astype(np.int32)
    sizes = [int(x) for x in rng.choice([1, 2, 17, 33, 64, 129, 256], n)]
    sizes[seed % n] = 0
    forms = ["chain", "star", "binary", "random"]
    parents = [_tree_of_form(forms[i % 4], sizes[i], rng) for i in range(n)]
    tokens = [W.random_tokens(p, 4096, rng) for p in parents]
    capacity = (int(prefix.max()) + 256 + 63) // 64 * 64
    wl = W.AttentionWorkload(f"random_{seed}", hq, hkv, dim, prefix, parents, tokens,
                             capacity)
    tensors = wl.make_tensors("cpu", seed, q_scale=q_scale)
    dev = [t.to(device) for t in tensors]
    meta = dict(
        row_offset=torch.from_numpy(wl.row_offset).to(device),
        prefix_start=torch.from_numpy(wl.prefix_start).to(device),
        prefix_len=torch.from_numpy(wl.prefix_len.astype(np.int32)).to(device),
        parent=torch.from_numpy(wl.parent_flat).to(device),
    )
    got, plan = _run(wl, dev, meta, device)
    ks, vs = _prefix_lists(wl, tensors)
    q, kc, vc, kt, vt = tensors
    live = [i for i in range(n) if sizes[i] > 0]
    refs = oracle.attention_per_request(q, ks, vs, kt, vt, wl.row_offset, wl.parents,
                                        requests=live)
    for i in live:
        r0, r1 = int(wl.row_offset[i]), int(wl.row_offset[i + 1])
        _assert_close(got[r0:r1], refs[i])


def test_plan_of_another_wave_is_caught_on_the_device(device, oracle):
    """A plan built for other prefix lengths (as after a commit) reads no K/V
    for its mismatched units: they raise the status word and write NaN; with
    the right plan the same call is clean.  Covers plans whose prefixes are
    shorter and longer than the call's, unsplit and split (merge) plans."""
    split_wl = W.qwen3_4b_workload(seed=21)
    _, split_dev, split_meta = _inputs(split_wl, device, 17)
    wl = W.tiny_attention_workload(seed=5, num_q_heads=8, num_kv_heads=2, head_dim=128)
    tensors, dev, meta = _inputs(wl, device, 16)
    for case_wl, case_dev, case_meta, delta, target in (
            (wl, dev, meta, 3, 0), (wl, dev, meta, -5, 0),
            (split_wl, split_dev, split_meta, 3, 4096)):
        stale = ops.plan_attention(case_wl.row_offset, case_wl.prefix_len + delta,
                                   case_wl.num_q_heads, case_wl.num_kv_heads,
                                   case_wl.head_dim, target).to(device)
        assert target == 0 or stale.merges > 0
        status = torch.zeros(1, dtype=torch.int32, device=device)
        q, kc, vc, kt, vt = case_dev
        out = ops.tree_attention(q, kc, vc, kt, vt, case_meta["row_offset"],
                                 case_meta["prefix_start"], case_meta["prefix_len"],
                                 case_meta["parent"], stale, status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == ops._lib.SG_EINVAL, (delta, target)
        assert torch.isnan(out.float()).all(), (delta, target)
    q, kc, vc, kt, vt = dev
    good = ops.plan_attention(wl.row_offset, wl.prefix_len, 8, 2, 128).to(device)
    ops.check_plan(good, wl.row_offset, wl.prefix_len)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    out = ops.tree_attention(q, kc, vc, kt, vt, meta["row_offset"], meta["prefix_start"],
                             meta["prefix_len"], meta["parent"], good, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0 and torch.isfinite(out.float()).all()
    with pytest.raises(ValueError, match="another wave"):
        ops.tree_attention(q[:-1], kc, vc, kt[:-1], vt[:-1], meta["row_offset"],
                           meta["prefix_start"], meta["prefix_len"], meta["parent"], good)


def test_plan_of_a_larger_wave_without_host_copy_indexes_nothing(device):
    """Through the C ABI with no host copy of the plan, a plan built for a
    larger wave (12 requests against the call's 4; split, so it has merge
    groups) meets no host check: every unit and merge group whose request,
    kv head or partial slot the call does not have indexes nothing and only
    raises the status word, with the plan's own workspace and with one too
    small for its partials.  The same call with its own plan is then clean."""
    wl = W.tiny_attention_workload(seed=5, num_q_heads=8, num_kv_heads=2, head_dim=128)
    _, dev, meta = _inputs(wl, device, 16)
    big_wl = W.tiny_attention_workload(seed=9, num_requests=12, prefix_lo=600, prefix_hi=900,
                                       num_q_heads=8, num_kv_heads=2, head_dim=128)
    big = ops.plan_attention(big_wl.row_offset, big_wl.prefix_len, 8, 2, 128, 4096).to(device)
    assert big.merges > 0 and big.num_requests == 12
    good = ops.plan_attention(wl.row_offset, wl.prefix_len, 8, 2, 128).to(device)
    q, kc, vc, kt, vt = dev
    small_ws = torch.zeros(16, dtype=torch.uint8, device=device)
    for ws in (big.workspace, small_ws):
        print(f"larger-wave plan, workspace {ws.numel()} bytes", flush=True)
        status = torch.zeros(1, dtype=torch.int32, device=device)
        call = ops.prepare_tree_attention(q, kc, vc, kt, vt, meta["row_offset"],
                                          meta["prefix_start"], meta["prefix_len"],
                                          meta["parent"], good, status=status)
        call.set(plan_dev=big.device.data_ptr(), plan_host=None, plan_units=big.units,
                 plan_merges=big.merges, workspace_dev=ws.data_ptr(),
                 workspace_bytes=ws.numel())
        call()
        torch.cuda.synchronize()
        assert int(status.item()) == ops._lib.SG_EINVAL
    status = torch.zeros(1, dtype=torch.int32, device=device)
    out = ops.tree_attention(q, kc, vc, kt, vt, meta["row_offset"], meta["prefix_start"],
                             meta["prefix_len"], meta["parent"], good, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0 and torch.isfinite(out.float()).all()
