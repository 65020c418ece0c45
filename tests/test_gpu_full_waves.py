"""GPU parity of the whole measured waves against the oracle, every request:

* the Qwen3-8B wave (64 requests, 2,048 rows, prefixes U{512..4096}): all 64
  requests' attention, including the requests the planner splits by rows;
* a Qwen3-8B wave of 128-node trees only (16 requests, 2,048 rows), whose
  units are the MFMA-heavy ones (four q-groups per unit, both row tiles);
* the long-context wave (128 requests, prefixes log-uniform 8k-32k, 4,096
  rows): attention of all 128 requests, tree sampling of all 4,096 rows over
  a 151,936-token vocabulary (bit-exact), and the KV commit (bit-exact);
* the 64 x 32-node sampler workload at vocabulary 151,936, from fp32, bf16
  and f16 logits (the 16-bit rows widen to fp32 exactly, so the oracle runs
  on the widened rows).

Attention tolerance (bf16 in and out): max |gpu - ref| <= 2e-2 and
mean |gpu - ref| / mean |ref| <= 1e-2.
"""
import gc

import numpy as np
import pytest
import torch

from specgrove_amd import ops
from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_REL = 1e-2


def _assert_close(got, ref, what):
    err = (got - ref).abs()
    max_abs = err.max().item()
    mean_rel = (err.mean() / ref.abs().mean()).item()
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL, (what, max_abs, mean_rel)


def _meta(wl, device):
    return dict(
        row_offset=torch.from_numpy(wl.row_offset).to(device),
        prefix_start=torch.from_numpy(wl.prefix_start).to(device),
        prefix_len=torch.from_numpy(wl.prefix_len.astype(np.int32)).to(device),
        parent=torch.from_numpy(wl.parent_flat).to(device),
    )


def _attention(wl, tensors, meta, device):
    plan = ops.plan_attention(wl.row_offset, wl.prefix_len, wl.num_q_heads, wl.num_kv_heads,
                              wl.head_dim).to(device)
    q, kc, vc, kt, vt = tensors
    status = torch.zeros(1, dtype=torch.int32, device=device)
    out = ops.tree_attention(q, kc, vc, kt, vt, meta["row_offset"], meta["prefix_start"],
                             meta["prefix_len"], meta["parent"], plan, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    return out.float().cpu(), plan


def _check_requests(oracle, wl, tensors, got, requests):
    """Per-request oracle on the CPU; each request's prefix is copied from the
    device arena on its own."""
    q, kc, vc, kt, vt = tensors
    q_c, kt_c, vt_c = q.cpu(), kt.cpu(), vt.cpu()
    for i in requests:
        s, L = int(wl.prefix_start[i]), int(wl.prefix_len[i])
        ref = oracle.attention_per_request(q_c, {i: kc[:, s:s + L].cpu()},
                                           {i: vc[:, s:s + L].cpu()}, kt_c, vt_c,
                                           wl.row_offset, wl.parents, requests=[i])[i]
        r0, r1 = int(wl.row_offset[i]), int(wl.row_offset[i + 1])
        _assert_close(got[r0:r1], ref, f"request {i}")


def test_qwen3_8b_wave_all_64_requests(device, oracle):
    wl = W.qwen3_8b_workload()
    tensors = wl.make_tensors(device, seed=103)
    got, plan = _attention(wl, tensors, _meta(wl, device), device)
    _, units, _, _ = ops.decode_plan(plan)
    row_split = sorted({int(u[0]) for u in units if u[7] & 2})
    assert row_split, "the wave has row-split requests"
    print(f"row-split requests: {row_split}", flush=True)
    _check_requests(oracle, wl, tensors, got, range(wl.num_requests))


def test_qwen3_8b_tier_128_wave_all_requests(device, oracle):
    wl = W.tier128_workload()
    assert set(wl.rows.tolist()) == {128} and wl.total_rows == 2048
    tensors = wl.make_tensors(device, seed=104)
    got, _ = _attention(wl, tensors, _meta(wl, device), device)
    _check_requests(oracle, wl, tensors, got, range(wl.num_requests))


@pytest.fixture(scope="module")
def long_context(device):
    """The long-context wave's tensors (17 GB of arena) and attention output."""
    wl = W.long_context_workload()
    print("long-context wave: generating 128 requests on the device", flush=True)
    tensors = wl.make_tensors(device, seed=300)
    meta = _meta(wl, device)
    got, plan = _attention(wl, tensors, meta, device)
    state = dict(wl=wl, tensors=tensors, meta=meta, got=got, plan=plan)
    yield state
    state.clear()
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("part", range(4))
def test_long_context_attention_all_128_requests(long_context, oracle, part):
    wl = long_context["wl"]
    requests = range(part * 32, (part + 1) * 32)
    print(f"long-context attention: requests {requests.start}-{requests.stop - 1}", flush=True)
    _check_requests(oracle, wl, long_context["tensors"], long_context["got"], requests)


def test_long_context_kv_commit(long_context, device, oracle):
    """Commit of the wave's kept rows (1 + a_i per request) into the 17 GB
    arena: every request's window around its append point and every length,
    bit-exact against the oracle's scatter."""
    wl, meta = long_context["wl"], long_context["meta"]
    q, kc, vc, kt, vt = long_context["tensors"]
    n = wl.num_requests
    width = max(len(k) for k in wl.keep)
    keep = np.full((n, width), -1, np.int32)
    for i, k in enumerate(wl.keep):
        keep[i, :len(k)] = k
    lo = [max(0, int(L) - 2) for L in wl.prefix_len]
    hi = [min(wl.capacity, int(L) + width + 2) for L in wl.prefix_len]

    def windows(arena):
        return [arena[:, int(wl.prefix_start[i]) + lo[i]:int(wl.prefix_start[i]) + hi[i]]
                .cpu().view(torch.int16).numpy() for i in range(n)]

    before_k, before_v = windows(kc), windows(vc)
    lengths = meta["prefix_len"].clone()
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.kv_commit(*[ops.pointer_array([t], device) for t in (kc, vc, kt, vt)],
                  num_kv_heads=wl.num_kv_heads, head_dim=wl.head_dim,
                  cache_head_stride=kc.stride(0), cache_token_stride=kc.stride(1),
                  tree_row_stride=kt.stride(0), tree_head_stride=kt.stride(1),
                  row_offset=meta["row_offset"], keep_rows=torch.from_numpy(keep).to(device),
                  keep_len=torch.tensor([len(k) for k in wl.keep], dtype=torch.int32,
                                        device=device),
                  prefix_start=meta["prefix_start"], lengths=lengths, capacity=wl.capacity,
                  status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    after_k, after_v = windows(kc), windows(vc)
    tree_k = kt.cpu().view(torch.int16).numpy()
    tree_v = vt.cpu().view(torch.int16).numpy()
    want_len = wl.prefix_len.astype(np.int64).copy()
    for i in range(n):
        # The oracle's scatter on the window (offset so that the append point
        # lo[i] rows in matches the arena's).
        wk, wv = before_k[i][None].copy(), before_v[i][None].copy()
        length = np.array([int(wl.prefix_len[i]) - lo[i]], np.int64)
        oracle.kv_commit(wk, wv, length, hi[i] - lo[i], [0], tree_k[None], tree_v[None],
                         [int(wl.row_offset[i]), int(wl.row_offset[i + 1])], [wl.keep[i]])
        assert np.array_equal(after_k[i], wk[0]) and np.array_equal(after_v[i], wv[0]), i
        want_len[i] += len(wl.keep[i])
    assert np.array_equal(lengths.cpu().numpy(), want_len)


def test_long_context_sampling_all_4096_rows(device, oracle):
    """Tree sampling of every packed row of the long-context wave over fp32
    logits [4096, 151936] (N(0, 3^2) with each draft token boosted by 17 in its
    parent's row -- against the mass of 151,936 such logits, about e^16.4, a
    child is then accepted with probability near one half -- so that walks go
    deep), bit-exact against the oracle."""
    wl = W.long_context_workload()
    vocab = 151936
    gen = torch.Generator(device=device).manual_seed(301)
    logits = torch.randn((wl.total_rows, vocab), generator=gen, device=device) * 3.0
    rows_idx, cols_idx = [], []
    for i, (p, t) in enumerate(zip(wl.parents, wl.tokens)):
        r0 = int(wl.row_offset[i])
        rows_idx += [r0 + p[k] for k in range(1, len(p))]
        cols_idx += list(t)
    logits[torch.tensor(rows_idx, device=device), torch.tensor(cols_idx, device=device)] += 17.0
    depth = max(max(W.depths_of(p)) for p in wl.parents)
    rng = np.random.default_rng(302)
    uniforms = rng.random((wl.num_requests, 2 * (depth + 1)), dtype=np.float32)
    token = np.concatenate([np.asarray([0] + list(t), np.int32) for t in wl.tokens])
    res = ops.tree_sample(logits, torch.from_numpy(wl.row_offset).to(device),
                          torch.from_numpy(wl.parent_flat).to(device),
                          torch.from_numpy(token).to(device),
                          torch.from_numpy(uniforms).to(device), depth)
    torch.cuda.synchronize()
    host = logits.cpu().numpy()
    del logits
    print("long-context sampling: oracle over 4096 rows", flush=True)
    nodes, length, bonus, m, z = oracle.tree_sample(host, wl.row_offset, wl.parent_flat, token,
                                                    uniforms, depth,
                                                    threads=oracle.cpu_threads())
    assert int(res.status.item()) == 0
    np.testing.assert_array_equal(res.row_max.cpu().numpy(), m)
    assert np.array_equal(res.row_sum.cpu().numpy().view(np.uint32), z.view(np.uint32))
    np.testing.assert_array_equal(res.accept_len.cpu().numpy(), length)
    np.testing.assert_array_equal(res.accept_nodes.cpu().numpy()[:, :depth], nodes)
    np.testing.assert_array_equal(res.bonus.cpu().numpy(), bonus)
    assert length.max() >= 4 and (length == 0).any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_sampler_workload_64x32_v151936(device, oracle, dtype):
    """The measured sampler workload (draft tokens drawn from
    0.7 softmax + 0.3 Dirichlet(0.1)) with the logits in fp32, bf16 or f16."""
    wl, logits, uniforms = W.sampler_workload(device, seed=4)
    logits = logits.to(dtype)
    parent, token = wl.flat_parent_token()
    res = ops.tree_sample(logits, torch.from_numpy(wl.row_offset).to(device),
                          torch.from_numpy(parent).to(device), torch.from_numpy(token).to(device),
                          uniforms, wl.max_depth)
    torch.cuda.synchronize()
    widened = logits.float().cpu().numpy()
    nodes, length, bonus, m, z = oracle.tree_sample(widened, wl.row_offset, parent, token,
                                                    uniforms.cpu().numpy(), wl.max_depth,
                                                    threads=oracle.cpu_threads())
    assert int(res.status.item()) == 0
    np.testing.assert_array_equal(res.row_max.cpu().numpy(), m)
    assert np.array_equal(res.row_sum.cpu().numpy().view(np.uint32), z.view(np.uint32))
    np.testing.assert_array_equal(res.accept_len.cpu().numpy(), length)
    np.testing.assert_array_equal(res.accept_nodes.cpu().numpy()[:, :wl.max_depth], nodes)
    np.testing.assert_array_equal(res.bonus.cpu().numpy(), bonus)
    assert length.max() >= 2
