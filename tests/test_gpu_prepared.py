"""Prepared C-ABI calls (argument checks and struct built once) run the same
kernels as the checked entry points: identical attention output, with the
buffers' new contents seen on every call, and identical commits, each run
advancing the lengths again."""
import numpy as np
import pytest
import torch

from specgrove_amd import ops
from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu


def test_prepared_attention_equals_checked_call_and_sees_new_contents(device):
    wl = W.qwen3_4b_workload()
    print("prepared attention, Qwen3-4B wave", flush=True)
    q, kc, vc, kt, vt = wl.make_tensors(device, seed=7)
    row_offset = torch.from_numpy(wl.row_offset).to(device)
    prefix_start = torch.from_numpy(wl.prefix_start).to(device)
    prefix_len = torch.from_numpy(wl.prefix_len.astype(np.int32)).to(device)
    parent = torch.from_numpy(wl.parent_flat).to(device)
    plan = ops.plan_attention(wl.row_offset, wl.prefix_len, wl.num_q_heads, wl.num_kv_heads,
                              wl.head_dim, 0).to(device)
    args = (q, kc, vc, kt, vt, row_offset, prefix_start, prefix_len, parent, plan)
    want = ops.tree_attention(*args).clone()
    call = ops.prepare_tree_attention(*args)
    got = call()
    torch.cuda.synchronize()
    assert got is call.result
    assert torch.equal(got, want)
    q.mul_(-1.0)  # new contents, same storage
    want2 = ops.tree_attention(*args).clone()
    got2 = call()
    torch.cuda.synchronize()
    assert torch.equal(got2, want2) and not torch.equal(want2, want)


def test_prepared_commit_equals_checked_calls(device):
    wl = W.tiny_attention_workload(seed=9)
    print("prepared commit, tiny wave, two calls", flush=True)
    n, hkv, d = wl.num_requests, wl.num_kv_heads, wl.head_dim
    gen = torch.Generator(device="cpu").manual_seed(4)
    cache = torch.randn((2, hkv, n * wl.capacity, d), generator=gen).to(torch.bfloat16)
    tree = torch.randn((2, wl.total_rows, hkv, d), generator=gen).to(torch.bfloat16)
    keep_stride = max(len(k) for k in wl.keep)
    keep = np.full((n, keep_stride), -1, np.int32)
    for i, k in enumerate(wl.keep):
        keep[i, :len(k)] = k

    def setup():
        ck, cv = cache[0].to(device), cache[1].to(device)
        tk, tv = tree[0].to(device), tree[1].to(device)
        lengths = torch.from_numpy(wl.prefix_len.astype(np.int32)).to(device)
        ptrs = [ops.pointer_array([t], device) for t in (ck, cv, tk, tv)]
        kw = dict(num_kv_heads=hkv, head_dim=d, cache_head_stride=ck.stride(0),
                  cache_token_stride=ck.stride(1), tree_row_stride=tk.stride(0),
                  tree_head_stride=tk.stride(1),
                  row_offset=torch.from_numpy(wl.row_offset).to(device),
                  keep_rows=torch.from_numpy(keep).to(device),
                  keep_len=torch.from_numpy(np.asarray([len(k) for k in wl.keep],
                                                       np.int32)).to(device),
                  prefix_start=torch.from_numpy(wl.prefix_start).to(device),
                  lengths=lengths, capacity=wl.capacity)
        return (ck, cv, lengths), ptrs, kw

    (ak, av, alen), aptrs, akw = setup()
    ops.kv_commit(*aptrs, **akw)
    ops.kv_commit(*aptrs, **akw)
    (bk, bv, blen), bptrs, bkw = setup()
    call = ops.prepare_kv_commit(*bptrs, **bkw)
    call()
    call()
    torch.cuda.synchronize()
    assert torch.equal(alen, blen)
    np.testing.assert_array_equal(blen.cpu().numpy(),
                                  wl.prefix_len + 2 * np.asarray([len(k) for k in wl.keep]))
    assert torch.equal(ak.view(torch.int16), bk.view(torch.int16))
    assert torch.equal(av.view(torch.int16), bv.view(torch.int16))
