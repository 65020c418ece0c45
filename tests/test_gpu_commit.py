"""GPU parity of the accepted-path KV commit against the CPU oracle: bit-exact."""
import numpy as np
import pytest
import torch

from specgrove_amd import ops
from specgrove_amd import workloads as W

pytestmark = pytest.mark.gpu


def _commit_case(device, oracle, wl, layers, seed, lengths=None):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    n = wl.num_requests
    hkv, d = wl.num_kv_heads, wl.head_dim
    rows = wl.total_rows
    cache_k = torch.randn((layers, hkv, n * wl.capacity, d), generator=gen).to(torch.bfloat16)
    cache_v = torch.randn((layers, hkv, n * wl.capacity, d), generator=gen).to(torch.bfloat16)
    tree_k = torch.randn((layers, rows, hkv, d), generator=gen).to(torch.bfloat16)
    tree_v = torch.randn((layers, rows, hkv, d), generator=gen).to(torch.bfloat16)
    if lengths is None:
        lengths = wl.prefix_len.astype(np.int32)
    keep_stride = max(len(k) for k in wl.keep)
    keep = np.full((n, keep_stride), -1, np.int32)
    for i, k in enumerate(wl.keep):
        keep[i, :len(k)] = k
    keep_len = np.asarray([len(k) for k in wl.keep], np.int32)

    dk, dv = cache_k.to(device), cache_v.to(device)
    tk, tv = tree_k.to(device), tree_v.to(device)
    lengths_dev = torch.from_numpy(lengths.copy()).to(device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.kv_commit(
        ops.pointer_array([dk[l] for l in range(layers)], device),
        ops.pointer_array([dv[l] for l in range(layers)], device),
        ops.pointer_array([tk[l] for l in range(layers)], device),
        ops.pointer_array([tv[l] for l in range(layers)], device),
        num_kv_heads=hkv, head_dim=d, cache_head_stride=dk.stride(1),
        cache_token_stride=dk.stride(2), tree_row_stride=tk.stride(1),
        tree_head_stride=tk.stride(2),
        row_offset=torch.from_numpy(wl.row_offset).to(device),
        keep_rows=torch.from_numpy(keep).to(device),
        keep_len=torch.from_numpy(keep_len).to(device),
        prefix_start=torch.from_numpy(wl.prefix_start).to(device),
        lengths=lengths_dev, capacity=wl.capacity, status=status)
    torch.cuda.synchronize()

    ok = cache_k.view(torch.int16).numpy().copy()
    ov = cache_v.view(torch.int16).numpy().copy()
    olen = lengths.copy()
    oracle.kv_commit(ok, ov, olen, wl.capacity, range(n),
                     tree_k.view(torch.int16).numpy(), tree_v.view(torch.int16).numpy(),
                     wl.row_offset, wl.keep)
    return dk, dv, lengths_dev, status, ok, ov, olen


def test_commit_qwen3_8b_shape_bit_exact(device, oracle):
    wl = W.qwen3_8b_workload()
    dk, dv, lengths_dev, status, ok, ov, olen = _commit_case(device, oracle, wl, 2, 0)
    assert int(status.item()) == 0
    np.testing.assert_array_equal(lengths_dev.cpu().numpy(), olen)
    assert np.array_equal(dk.cpu().view(torch.int16).numpy(), ok)
    assert np.array_equal(dv.cpu().view(torch.int16).numpy(), ov)


def test_commit_tiny_many_layers_bit_exact(device, oracle):
    wl = W.tiny_attention_workload(seed=5)
    dk, dv, lengths_dev, status, ok, ov, olen = _commit_case(device, oracle, wl, 5, 1)
    assert int(status.item()) == 0
    np.testing.assert_array_equal(lengths_dev.cpu().numpy(), olen)
    assert np.array_equal(dk.cpu().view(torch.int16).numpy(), ok)
    assert np.array_equal(dv.cpu().view(torch.int16).numpy(), ov)


def test_commit_capacity_overflow_reports_erange(device, oracle):
    wl = W.tiny_attention_workload(seed=6)
    lengths = wl.prefix_len.astype(np.int32).copy()
    lengths[1] = wl.capacity - 1          # request 1 cannot take its kept rows
    gen = torch.Generator(device="cpu").manual_seed(3)
    n, hkv, d = wl.num_requests, wl.num_kv_heads, wl.head_dim
    cache = torch.randn((hkv, n * wl.capacity, d), generator=gen).to(torch.bfloat16).to(device)
    before = cache.clone()
    tree = torch.randn((wl.total_rows, hkv, d), generator=gen).to(torch.bfloat16).to(device)
    keep = np.full((n, 16), -1, np.int32)
    for i, k in enumerate(wl.keep):
        keep[i, :len(k)] = k
    keep_len = np.asarray([len(k) for k in wl.keep], np.int32)
    lengths_dev = torch.from_numpy(lengths.copy()).to(device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ptr = ops.pointer_array([cache], device)
    tptr = ops.pointer_array([tree], device)
    ops.kv_commit(ptr, ptr, tptr, tptr, num_kv_heads=hkv, head_dim=d,
                  cache_head_stride=cache.stride(0), cache_token_stride=cache.stride(1),
                  tree_row_stride=tree.stride(0), tree_head_stride=tree.stride(1),
                  row_offset=torch.from_numpy(wl.row_offset).to(device),
                  keep_rows=torch.from_numpy(keep).to(device),
                  keep_len=torch.from_numpy(keep_len).to(device),
                  prefix_start=torch.from_numpy(wl.prefix_start).to(device),
                  lengths=lengths_dev, capacity=wl.capacity, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == -2
    got = lengths_dev.cpu().numpy()
    assert got[1] == lengths[1]
    expected = lengths + keep_len
    expected[1] = lengths[1]
    np.testing.assert_array_equal(got, expected)
    region = slice(wl.capacity, 2 * wl.capacity)
    assert torch.equal(cache[:, region], before[:, region])
    with pytest.raises(RuntimeError, match="capacity exhausted"):
        oracle.kv_commit(np.zeros((1, hkv, n * wl.capacity, d)),
                         np.zeros((1, hkv, n * wl.capacity, d)), lengths.copy(),
                         wl.capacity, range(n), np.zeros((1, wl.total_rows, hkv, d)),
                         np.zeros((1, wl.total_rows, hkv, d)), wl.row_offset, wl.keep)


def _raw_commit(device, layers, rows, keep_lists, lengths, capacity, hkv, d, seed):
    """Commit through the C ABI on random data; returns device and host copies."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    n = len(rows)
    row_offset = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    cache_k = torch.randn((layers, hkv, n * capacity, d), generator=gen).to(torch.bfloat16)
    cache_v = torch.randn((layers, hkv, n * capacity, d), generator=gen).to(torch.bfloat16)
    tree_k = torch.randn((layers, int(row_offset[-1]), hkv, d), generator=gen).to(torch.bfloat16)
    tree_v = torch.randn((layers, int(row_offset[-1]), hkv, d), generator=gen).to(torch.bfloat16)
    keep_stride = max(len(k) for k in keep_lists)
    keep = np.full((n, keep_stride), -1, np.int32)
    for i, k in enumerate(keep_lists):
        keep[i, :len(k)] = k
    dk, dv = cache_k.to(device), cache_v.to(device)
    tk, tv = tree_k.to(device), tree_v.to(device)
    lengths_dev = torch.from_numpy(np.asarray(lengths, np.int32)).to(device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.kv_commit(
        ops.pointer_array([dk[l] for l in range(layers)], device),
        ops.pointer_array([dv[l] for l in range(layers)], device),
        ops.pointer_array([tk[l] for l in range(layers)], device),
        ops.pointer_array([tv[l] for l in range(layers)], device),
        num_kv_heads=hkv, head_dim=d, cache_head_stride=dk.stride(1),
        cache_token_stride=dk.stride(2), tree_row_stride=tk.stride(1),
        tree_head_stride=tk.stride(2), row_offset=torch.from_numpy(row_offset).to(device),
        keep_rows=torch.from_numpy(keep).to(device),
        keep_len=torch.from_numpy(np.asarray([len(k) for k in keep_lists], np.int32)).to(device),
        prefix_start=torch.from_numpy(np.arange(n, dtype=np.int64) * capacity).to(device),
        lengths=lengths_dev, capacity=capacity, status=status)
    torch.cuda.synchronize()
    return (dk, dv, lengths_dev, status, cache_k.view(torch.int16).numpy().copy(),
            cache_v.view(torch.int16).numpy().copy(), tree_k.view(torch.int16).numpy(),
            tree_v.view(torch.int16).numpy(), row_offset)


def test_commit_more_layers_and_kept_rows_than_staged(device, oracle):
    """130 layers (layer bases beyond the 128 staged in LDS) and a 300-row
    keep list (kept rows beyond the 256 staged) take the global-memory paths."""
    rng = np.random.default_rng(7)
    rows = [320, 5, 40]
    keep_lists = [[0] + sorted(rng.choice(np.arange(1, 320), 299, replace=False).tolist()),
                  [0, 3], [0, 1, 7, 30]]
    lengths = [10, 0, 33]
    capacity = 400
    dk, dv, lengths_dev, status, ok, ov, tk, tv, row_offset = _raw_commit(
        device, 130, rows, keep_lists, lengths, capacity, 1, 8, 11)
    olen = np.asarray(lengths, np.int32)
    oracle.kv_commit(ok, ov, olen, capacity, range(3), tk, tv, row_offset, keep_lists)
    assert int(status.item()) == 0
    np.testing.assert_array_equal(lengths_dev.cpu().numpy(), olen)
    assert np.array_equal(dk.cpu().view(torch.int16).numpy(), ok)
    assert np.array_equal(dv.cpu().view(torch.int16).numpy(), ov)


def test_commit_kept_row_outside_the_request_reports_einval(device, oracle):
    """A kept row past the request's packed rows leaves that request untouched
    (cache and length) and sets status to SG_EINVAL; the others commit."""
    rows = [16, 16, 16]
    keep_lists = [[0, 2, 5], [0, 16], [0, 1]]   # request 1: row 16 of 16 is out of range
    lengths = [4, 4, 4]
    capacity = 64
    dk, dv, lengths_dev, status, ok, ov, tk, tv, row_offset = _raw_commit(
        device, 2, rows, keep_lists, lengths, capacity, 2, 64, 12)
    olen = np.asarray(lengths, np.int32)
    # the oracle commits requests 0 and 2 only
    oracle.kv_commit(ok, ov, olen, capacity, range(3), tk, tv, row_offset,
                     [keep_lists[0], [], keep_lists[2]])
    assert int(status.item()) == -1
    np.testing.assert_array_equal(lengths_dev.cpu().numpy(), olen)
    assert np.array_equal(dk.cpu().view(torch.int16).numpy(), ok)
    assert np.array_equal(dv.cpu().view(torch.int16).numpy(), ov)


def test_commit_overflow_with_several_layers_reports_erange(device, oracle):
    """Several layers (copy launch + length launch): the request that would
    pass its capacity is left untouched in every layer and keeps its length;
    the others commit; status is SG_ERANGE."""
    rows = [8, 8, 8]
    keep_lists = [[0, 3], [0, 1], [0, 2, 5]]
    capacity = 32
    lengths = [4, capacity - 1, 20]
    dk, dv, lengths_dev, status, ok, ov, tk, tv, row_offset = _raw_commit(
        device, 3, rows, keep_lists, lengths, capacity, 2, 64, 13)
    olen = np.asarray(lengths, np.int32)
    oracle.kv_commit(ok, ov, olen, capacity, range(3), tk, tv, row_offset,
                     [keep_lists[0], [], keep_lists[2]])
    assert int(status.item()) == -2
    np.testing.assert_array_equal(lengths_dev.cpu().numpy(), olen)
    assert np.array_equal(dk.cpu().view(torch.int16).numpy(), ok)
    assert np.array_equal(dv.cpu().view(torch.int16).numpy(), ov)


def _split_case(device, oracle, wl, layers, seed, keep_lists, bad_row=False):
    """sg_kv_split over ``layers`` layers of the packed prefixes of ``wl``
    against oracle.kv_split, bit for bit (bf16 moved as 16-bit words)."""
    from specgrove_amd.ops import kv_split, pointer_array
    g = torch.Generator().manual_seed(seed)
    n, hkv, d = wl.num_requests, wl.num_kv_heads, wl.head_dim
    lengths = [int(v) for v in wl.prefix_len]
    P = sum(lengths)
    rows = wl.total_rows
    prefix_k = torch.randint(-30000, 30000, (layers, hkv, P, d), generator=g, dtype=torch.int16)
    prefix_v = torch.randint(-30000, 30000, (layers, hkv, P, d), generator=g, dtype=torch.int16)
    tree_k = torch.randint(-30000, 30000, (layers, rows, hkv, d), generator=g, dtype=torch.int16)
    tree_v = torch.randint(-30000, 30000, (layers, rows, hkv, d), generator=g, dtype=torch.int16)
    offsets = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    sizes = [L + len(k) for L, k in zip(lengths, keep_lists)]
    out_off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    T = int(sum(sizes))
    dev = [t.to(device) for t in (prefix_k, prefix_v, tree_k, tree_v)]
    out_k = torch.zeros((layers, hkv, T, d), dtype=torch.int16, device=device)
    out_v = torch.zeros_like(out_k)
    width = max(1, max(len(k) for k in keep_lists))
    keep = np.full((n, width), -1, np.int32)
    for i, k in enumerate(keep_lists):
        keep[i, :len(k)] = k
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ptr = lambda t: pointer_array([t[l] for l in range(layers)], device)  # noqa: E731
    kv_split(ptr(dev[0]), ptr(dev[1]), ptr(dev[2]), ptr(dev[3]), ptr(out_k), ptr(out_v),
             num_kv_heads=hkv, head_dim=d, prefix_head_stride=P * d, prefix_token_stride=d,
             tree_row_stride=hkv * d, tree_head_stride=d, out_head_stride=T * d,
             out_token_stride=d, cache_offset=torch.from_numpy(offsets).to(device),
             old_length=torch.tensor(lengths, dtype=torch.int32, device=device),
             row_offset=torch.from_numpy(wl.row_offset).to(device),
             keep_rows=torch.from_numpy(keep).to(device),
             keep_len=torch.tensor([len(k) for k in keep_lists], dtype=torch.int32,
                                   device=device),
             out_offset=torch.from_numpy(out_off).to(device), max_tokens=max(sizes),
             status=status)
    torch.cuda.synchronize()
    got_k, got_v = out_k.cpu().numpy(), out_v.cpu().numpy()
    if bad_row:
        return int(status.item()), got_k
    assert int(status.item()) == 0
    want = oracle.kv_split(prefix_k.numpy(), prefix_v.numpy(), tree_k.numpy(), tree_v.numpy(),
                           offsets, lengths, wl.row_offset, keep_lists)
    for i, (wk, wv) in enumerate(want):
        a, b = int(out_off[i]), int(out_off[i]) + sizes[i]
        assert np.array_equal(got_k[:, :, a:b], wk) and np.array_equal(got_v[:, :, a:b], wv), i


def test_split_qwen3_4b_shape_bit_exact(device, oracle):
    """The non-persistent split of the Qwen3-4B-shape wave (16 requests,
    prefixes U{256..2048}), 3 layers, kept paths of 1-9 rows."""
    wl = W.qwen3_4b_workload()
    _split_case(device, oracle, wl, 3, 5, wl.keep)


def test_split_fixture_and_edge_cases(device, oracle):
    """Empty keep lists, a request with an empty prefix, head dim 64, and a
    kept row outside its request (not copied, status EINVAL)."""
    wl = W.tiny_attention_workload(seed=4, num_q_heads=4, num_kv_heads=2, head_dim=64)
    wl.prefix_len[1] = 0
    keeps = [[0, 3, 5], [], [0], [0, 1, 2, 3, 4, 5, 6, 7, 8]]
    _split_case(device, oracle, wl, 2, 6, keeps)
    status, _ = _split_case(device, oracle, wl, 2, 6, [[0, 99], [0], [0], [0]], bad_row=True)
    assert status == -1
