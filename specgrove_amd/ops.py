"""Torch-facing wrappers of the HIP kernels (PyTorch is only the memory and
stream plumbing here: tensors are passed to the C ABI as raw device pointers,
and every call is enqueued on torch's current HIP stream).

Argument checks follow the reference's native-op conventions
(fused_tree_sampling.py:158-174, :472-509): contiguity/device/dtype problems
raise ValueError before anything is launched; launch errors raise RuntimeError.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib


# Raw handle of torch's current stream without building a Stream object
# (torch.cuda.current_stream() costs ~3 us per call, this ~0.1 us).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle() -> int:
    """torch's current HIP stream on the current device."""
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


class PreparedCall:
    """A validated C-ABI call whose argument struct is built once.

    Calling it only enqueues the kernels on torch's current stream, so a
    caller that repeats a call over the same buffers (a decode loop over
    persistent staging) pays the argument checks and the struct once.  It
    holds the tensors it points to: their contents may change between calls,
    their storage, shapes and strides may not.  Returns ``result``.
    """
    __slots__ = ("_fn", "_ref", "_args", "_keep", "_name", "result")

    def __init__(self, fn_name: str, args, keep, result=None):
        self._fn = getattr(_lib.load(), fn_name)
        self._args = args
        self._ref = ctypes.byref(args)
        self._keep = keep
        self._name = fn_name
        self.result = result

    def __call__(self):
        _lib.check(self._fn(self._ref, _stream_handle()), self._name)
        return self.result

    def set(self, **fields) -> "PreparedCall":
        """Update scalar fields of the bound argument struct (sizes and
        strides that change from call to call over the same buffers, e.g. a
        commit's request count); the library checks them on every call."""
        for name, value in fields.items():
            if not hasattr(self._args, name):
                raise ValueError(f"{self._name} has no argument {name}")
            setattr(self._args, name, value)
        return self


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise ValueError(message)


def _check_device_tensor(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == dtype:
        return
    _require(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _require(t.is_cuda, f"{name} must be a HIP device tensor")
    _require(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")


def _check_device_tensors(tensors: tuple, names: tuple, dtype: torch.dtype) -> None:
    """_check_device_tensor over several tensors of one dtype."""
    for t in tensors:
        if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == dtype):
            break
    else:
        return
    for t, name in zip(tensors, names):
        _check_device_tensor(t, name, dtype)


def _check_rows(t: torch.Tensor, name: str) -> None:
    """bf16 tensors whose last (head) dim is contiguous and 16-byte aligned."""
    _check_device_tensor(t, name, torch.bfloat16)
    st = t.stride()
    if st[-1] == 1 and t.data_ptr() % 16 == 0 and not any(s % 8 for s in st[:-1]):
        return
    _require(st[-1] == 1, f"{name} must have a contiguous last dimension")
    _require(t.data_ptr() % 16 == 0, f"{name} must be 16-byte aligned")
    _require(not any(s % 8 for s in st[:-1]), f"{name} strides must be multiples of 8 elements")


# --------------------------------------------------------------------------
# (A) attention
# --------------------------------------------------------------------------

@dataclass
class AttnPlan:
    """Host-built work list of the packed attention (one per wave, all layers)."""
    host: np.ndarray
    units: int
    merges: int
    workspace_bytes: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    device: torch.Tensor | None = None
    workspace: torch.Tensor | None = None

    @property
    def header(self) -> np.ndarray:
        """The plan header as int32 words (see decode_plan)."""
        return self.host[:64].view(np.int32)

    @property
    def num_requests(self) -> int:
        return int(self.header[8])

    @property
    def num_rows(self) -> int:
        return int(self.header[9])

    def to(self, device) -> "AttnPlan":
        """Copy the plan to the device and allocate its workspace (the fp32
        partial results of split units; every slot is written before the merge
        kernel reads it, so its initial contents do not matter)."""
        self.device = torch.from_numpy(self.host).to(device, non_blocking=False)
        self.workspace = torch.zeros(max(self.workspace_bytes, 16), dtype=torch.uint8,
                                     device=device)
        return self


def plan_attention(row_offset, prefix_len, num_q_heads: int, num_kv_heads: int,
                   head_dim: int, target_units: int = 0) -> AttnPlan:
    lib = _lib.load()
    ro = np.ascontiguousarray(np.asarray(row_offset, dtype=np.int32))
    pl = np.ascontiguousarray(np.asarray(prefix_len, dtype=np.int32))
    n = int(pl.size)
    _require(ro.size == n + 1, "row_offset must have num_requests + 1 entries")
    i32p = ctypes.POINTER(ctypes.c_int32)
    plan_bytes = ctypes.c_size_t()
    units = ctypes.c_int32()
    merges = ctypes.c_int32()
    ws = ctypes.c_size_t()
    args = (n, ro.ctypes.data_as(i32p), pl.ctypes.data_as(i32p), num_q_heads,
            num_kv_heads, head_dim, target_units)
    _lib.check(lib.sg_tree_attn_plan(*args, None, 0, ctypes.byref(plan_bytes),
                                     ctypes.byref(units), ctypes.byref(merges),
                                     ctypes.byref(ws)), "sg_tree_attn_plan")
    host = np.zeros(plan_bytes.value, dtype=np.uint8)
    _lib.check(lib.sg_tree_attn_plan(*args, host.ctypes.data_as(ctypes.c_void_p),
                                     host.nbytes, ctypes.byref(plan_bytes),
                                     ctypes.byref(units), ctypes.byref(merges),
                                     ctypes.byref(ws)), "sg_tree_attn_plan")
    return AttnPlan(host, units.value, merges.value, ws.value, num_q_heads,
                    num_kv_heads, head_dim)


def check_plan(plan: AttnPlan, row_offset_host, prefix_len_host) -> None:
    """Raise ValueError unless ``plan`` was built from exactly these row
    offsets and prefix lengths (plans are per wave: prefix lengths change
    after every commit)."""
    ro = np.ascontiguousarray(np.asarray(row_offset_host, dtype=np.int32))
    pl = np.ascontiguousarray(np.asarray(prefix_len_host, dtype=np.int32))
    _require(ro.size == pl.size + 1, "row_offset must have num_requests + 1 entries")
    i32p = ctypes.POINTER(ctypes.c_int32)
    _lib.check(_lib.load().sg_tree_attn_plan_check(
        plan.host.ctypes.data_as(ctypes.c_void_p), int(pl.size), ro.ctypes.data_as(i32p),
        pl.ctypes.data_as(i32p)), "sg_tree_attn_plan_check")


def check_plan_call(plan: AttnPlan, num_requests: int, num_rows: int, num_q_heads: int,
                    num_kv_heads: int, head_dim: int) -> None:
    """Host-side agreement of a plan with the call's shapes (no device access)."""
    _require((plan.num_q_heads, plan.num_kv_heads, plan.head_dim)
             == (num_q_heads, num_kv_heads, head_dim),
             "plan was built for another head configuration")
    _require(plan.num_requests == num_requests and plan.num_rows == num_rows,
             f"plan was built for another wave ({plan.num_requests} requests, "
             f"{plan.num_rows} rows; the call has {num_requests} and {num_rows})")


UNIT_FIELDS = ("req", "kv_head", "row_begin", "row_count", "key_begin", "key_end",
               "partial", "flags", "group", "num_splits", "first_partial", "pad")


MERGE_FIELDS = ("req", "kv_head", "row_begin", "row_count", "first_partial", "num_partials",
                "pad0", "pad1")


def decode_plan(plan: AttnPlan):
    """(header [16], units [U, 12], merges [M, 8], bin_offset [B+1]) int32 views
    of a host plan; unit columns are UNIT_FIELDS, merge-group columns
    MERGE_FIELDS.  Work list b (workgroup b of the attention kernel) runs
    units[bin_offset[b]:bin_offset[b+1]]."""
    words = plan.host.view(np.int32)
    header = words[:16]
    n_units, n_merges, n_bins = int(header[1]), int(header[2]), int(header[7])
    end = 16 + len(UNIT_FIELDS) * n_units
    units = words[16:end].reshape(n_units, len(UNIT_FIELDS))
    mend = end + len(MERGE_FIELDS) * n_merges
    merges = words[end:mend].reshape(n_merges, len(MERGE_FIELDS))
    bins = words[mend:mend + n_bins + 1]
    return header, units, merges, bins


def tree_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   k_tree: torch.Tensor, v_tree: torch.Tensor,
                   row_offset: torch.Tensor, prefix_start: torch.Tensor,
                   prefix_len: torch.Tensor, parent: torch.Tensor, plan: AttnPlan,
                   out: torch.Tensor | None = None, scale: float | None = None,
                   status: torch.Tensor | None = None) -> torch.Tensor:
    """Packed tree attention of one layer (see prepare_tree_attention)."""
    return prepare_tree_attention(q, k_cache, v_cache, k_tree, v_tree, row_offset,
                                  prefix_start, prefix_len, parent, plan, out=out,
                                  scale=scale, status=status)()


def prepare_tree_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           k_tree: torch.Tensor, v_tree: torch.Tensor,
                           row_offset: torch.Tensor, prefix_start: torch.Tensor,
                           prefix_len: torch.Tensor, parent: torch.Tensor, plan: AttnPlan,
                           out: torch.Tensor | None = None, scale: float | None = None,
                           status: torch.Tensor | None = None) -> PreparedCall:
    """Packed tree attention of one layer, validated and bound (call it to run).

    q [R, Hq, D], k/v_cache [Hkv, tokens, D] (the cache arena of this layer),
    k/v_tree [R, Hkv, D] (this wave's rows), row_offset [n+1] i32,
    prefix_start [n] i64, prefix_len [n] i32, parent [R] i32.  Returns
    out [R, Hq, D] bf16.  ``status`` (optional [1] i32 device word, never
    cleared here) is set to SG_EINVAL by any unit whose key range or rows
    disagree with prefix_len / row_offset (a plan of another wave), whose
    output rows are then NaN.
    """
    for t, name in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache"),
                    (k_tree, "k_tree"), (v_tree, "v_tree")):
        _check_rows(t, name)
    _check_device_tensors((row_offset, prefix_len, parent),
                          ("row_offset", "prefix_len", "parent"), torch.int32)
    _check_device_tensor(prefix_start, "prefix_start", torch.int64)
    _require(q.dim() == 3 and k_tree.dim() == 3 and k_cache.dim() == 3,
             "q/k_tree must be [R, H, D] and k_cache [Hkv, tokens, D]")
    rows, hq, dim = q.shape
    hkv = k_cache.shape[0]
    cache_strides = k_cache.stride()
    tree_strides = k_tree.stride()
    _require(k_cache.shape == v_cache.shape and cache_strides == v_cache.stride(),
             "k_cache and v_cache must share shape and strides")
    _require(k_tree.shape == (rows, hkv, dim) and v_tree.shape == k_tree.shape
             and tree_strides == v_tree.stride(),
             "k_tree/v_tree must be [R, Hkv, D] with equal strides")
    _require(k_cache.shape[2] == dim, "head dims disagree")
    n = prefix_len.numel()
    check_plan_call(plan, n, rows, hq, hkv, dim)
    _require(plan.device is not None and plan.device.is_cuda, "plan is not on the device")
    _require(parent.numel() >= rows, "parent must cover every packed row")
    _require(row_offset.numel() == n + 1 and prefix_start.numel() == n,
             "request metadata sizes disagree")
    if status is not None:
        _check_device_tensor(status, "status", torch.int32)
    if out is None:
        out = torch.empty((rows, hq, dim), dtype=torch.bfloat16, device=q.device)
    _check_rows(out, "out")
    _require(out.shape == (rows, hq, dim), "out must be [R, Hq, D]")
    q_strides = q.stride()
    out_strides = out.stride()
    workspace = plan.workspace
    # Positional, in the order of SgTreeAttnArgs' fields.
    a = _lib.SgTreeAttnArgs(
        n, rows, hq, hkv, dim, float(dim ** -0.5 if scale is None else scale),
        q.data_ptr(), q_strides[0], q_strides[1],
        k_cache.data_ptr(), v_cache.data_ptr(), cache_strides[0], cache_strides[1],
        k_tree.data_ptr(), v_tree.data_ptr(), tree_strides[0], tree_strides[1],
        row_offset.data_ptr(), prefix_start.data_ptr(), prefix_len.data_ptr(),
        parent.data_ptr(), out.data_ptr(), out_strides[0], out_strides[1],
        plan.device.data_ptr(), plan.host.ctypes.data, plan.units, plan.merges,
        workspace.data_ptr() if workspace is not None else 0,
        workspace.numel() if workspace is not None else 0,
        status.data_ptr() if status is not None else 0)
    keep = (q, k_cache, v_cache, k_tree, v_tree, row_offset, prefix_start, prefix_len, parent,
            plan, out, status)
    return PreparedCall("sg_tree_attn_fwd", a, keep, result=out)


# --------------------------------------------------------------------------
# (B) KV commit
# --------------------------------------------------------------------------

def pointer_array(tensors, device) -> torch.Tensor:
    """Device array of the tensors' base addresses (int64)."""
    return torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64, device=device)


def kv_commit(k_cache_ptrs: torch.Tensor, v_cache_ptrs: torch.Tensor,
              k_tree_ptrs: torch.Tensor, v_tree_ptrs: torch.Tensor, **kw) -> None:
    """Scatter the kept rows of every layer into the cache (one call; see
    prepare_kv_commit)."""
    prepare_kv_commit(k_cache_ptrs, v_cache_ptrs, k_tree_ptrs, v_tree_ptrs, **kw)()


def prepare_kv_commit(k_cache_ptrs: torch.Tensor, v_cache_ptrs: torch.Tensor,
                      k_tree_ptrs: torch.Tensor, v_tree_ptrs: torch.Tensor, *,
                      num_kv_heads: int, head_dim: int, cache_head_stride: int,
                      cache_token_stride: int, tree_row_stride: int, tree_head_stride: int,
                      row_offset: torch.Tensor, keep_rows: torch.Tensor, keep_len: torch.Tensor,
                      prefix_start: torch.Tensor, lengths: torch.Tensor, capacity: int,
                      status: torch.Tensor | None = None) -> PreparedCall:
    """Scatter the kept rows of every layer into the cache, validated and
    bound (call it to run; every run advances ``lengths`` again).

    ``*_ptrs`` are int64 device arrays of per-layer base addresses (see
    pointer_array); keep_rows [n, keep_stride] i32, keep_len [n] i32,
    prefix_start [n] i64, lengths [n] i32 (advanced in place).
    """
    _check_device_tensors((k_cache_ptrs, v_cache_ptrs, k_tree_ptrs, v_tree_ptrs, prefix_start),
                          ("k_cache_ptrs", "v_cache_ptrs", "k_tree_ptrs", "v_tree_ptrs",
                           "prefix_start"), torch.int64)
    _check_device_tensors((row_offset, keep_rows, keep_len, lengths),
                          ("row_offset", "keep_rows", "keep_len", "lengths"), torch.int32)
    layers = k_cache_ptrs.numel()
    _require(v_cache_ptrs.numel() == layers and k_tree_ptrs.numel() == layers
             and v_tree_ptrs.numel() == layers, "per-layer pointer arrays disagree")
    _require(keep_rows.dim() == 2 and keep_rows.is_contiguous(), "keep_rows must be [n, stride]")
    n, keep_stride = keep_rows.shape
    _require(keep_len.numel() == n and lengths.numel() == n and prefix_start.numel() == n
             and row_offset.numel() == n + 1, "request metadata sizes disagree")
    if status is not None:
        _check_device_tensor(status, "status", torch.int32)
    # Positional, in the order of SgKvCommitArgs' fields.
    a = _lib.SgKvCommitArgs(
        layers, n, num_kv_heads, head_dim,
        k_cache_ptrs.data_ptr(), v_cache_ptrs.data_ptr(), cache_head_stride, cache_token_stride,
        k_tree_ptrs.data_ptr(), v_tree_ptrs.data_ptr(), tree_row_stride, tree_head_stride,
        row_offset.data_ptr(), keep_rows.data_ptr(), keep_stride, keep_len.data_ptr(),
        prefix_start.data_ptr(), lengths.data_ptr(), capacity,
        status.data_ptr() if status is not None else 0)
    keep = (k_cache_ptrs, v_cache_ptrs, k_tree_ptrs, v_tree_ptrs, row_offset, keep_rows,
            keep_len, prefix_start, lengths, status)
    return PreparedCall("sg_kv_commit", a, keep)


def kv_split(k_prefix_ptrs: torch.Tensor, v_prefix_ptrs: torch.Tensor,
             k_tree_ptrs: torch.Tensor, v_tree_ptrs: torch.Tensor,
             k_out_ptrs: torch.Tensor, v_out_ptrs: torch.Tensor, *,
             num_kv_heads: int, head_dim: int, prefix_head_stride: int,
             prefix_token_stride: int, tree_row_stride: int, tree_head_stride: int,
             out_head_stride: int, out_token_stride: int, cache_offset: torch.Tensor,
             old_length: torch.Tensor, row_offset: torch.Tensor, keep_rows: torch.Tensor,
             keep_len: torch.Tensor, out_offset: torch.Tensor, max_tokens: int,
             status: torch.Tensor | None = None) -> None:
    """Rebuild every request's cache (old prefix + kept rows) from one packed
    wave, all layers in one call (the non-persistent split).

    ``*_ptrs`` are int64 device arrays of per-layer bases (see pointer_array);
    cache_offset/out_offset [n] i64, old_length/keep_len [n] i32, row_offset
    [n+1] i32, keep_rows [n, keep_stride] i32.
    """
    for t, name in ((k_prefix_ptrs, "k_prefix_ptrs"), (v_prefix_ptrs, "v_prefix_ptrs"),
                    (k_tree_ptrs, "k_tree_ptrs"), (v_tree_ptrs, "v_tree_ptrs"),
                    (k_out_ptrs, "k_out_ptrs"), (v_out_ptrs, "v_out_ptrs"),
                    (cache_offset, "cache_offset"), (out_offset, "out_offset")):
        _check_device_tensor(t, name, torch.int64)
    for t, name in ((old_length, "old_length"), (row_offset, "row_offset"),
                    (keep_rows, "keep_rows"), (keep_len, "keep_len")):
        _check_device_tensor(t, name, torch.int32)
    layers = k_prefix_ptrs.numel()
    _require(all(t.numel() == layers for t in (v_prefix_ptrs, k_tree_ptrs, v_tree_ptrs,
                                               k_out_ptrs, v_out_ptrs)),
             "per-layer pointer arrays disagree")
    _require(keep_rows.dim() == 2 and keep_rows.is_contiguous(), "keep_rows must be [n, stride]")
    n = keep_rows.shape[0]
    _require(cache_offset.numel() == n and out_offset.numel() == n and old_length.numel() == n
             and keep_len.numel() == n and row_offset.numel() == n + 1,
             "request metadata sizes disagree")
    if status is not None:
        _check_device_tensor(status, "status", torch.int32)
    a = _lib.SgKvSplitArgs()
    a.num_layers = layers
    a.num_requests = n
    a.num_kv_heads = num_kv_heads
    a.head_dim = head_dim
    a.max_tokens = max_tokens
    a.keep_stride = keep_rows.shape[1]
    a.k_prefix_layers_dev = k_prefix_ptrs.data_ptr()
    a.v_prefix_layers_dev = v_prefix_ptrs.data_ptr()
    a.prefix_head_stride, a.prefix_token_stride = prefix_head_stride, prefix_token_stride
    a.k_tree_layers_dev = k_tree_ptrs.data_ptr()
    a.v_tree_layers_dev = v_tree_ptrs.data_ptr()
    a.tree_row_stride, a.tree_head_stride = tree_row_stride, tree_head_stride
    a.k_out_layers_dev = k_out_ptrs.data_ptr()
    a.v_out_layers_dev = v_out_ptrs.data_ptr()
    a.out_head_stride, a.out_token_stride = out_head_stride, out_token_stride
    a.cache_offset_dev = cache_offset.data_ptr()
    a.old_length_dev = old_length.data_ptr()
    a.row_offset_dev = row_offset.data_ptr()
    a.keep_rows_dev = keep_rows.data_ptr()
    a.keep_len_dev = keep_len.data_ptr()
    a.out_offset_dev = out_offset.data_ptr()
    a.status_dev = status.data_ptr() if status is not None else 0
    _lib.check(_lib.load().sg_kv_split(ctypes.byref(a), _stream_handle()), "sg_kv_split")


# --------------------------------------------------------------------------
# (C) tree sampling
# --------------------------------------------------------------------------

@dataclass
class SampleResult:
    accept_nodes: torch.Tensor  # [n, max_depth] i32, -1 padded
    accept_len: torch.Tensor    # [n] i32
    bonus: torch.Tensor         # [n] i32
    keep_rows: torch.Tensor     # [n, max_depth + 1] i32 ([0] + nodes, -1 padded)
    row_max: torch.Tensor       # [R] f32
    row_sum: torch.Tensor       # [R] f32
    status: torch.Tensor        # [1] i32
    workspace: torch.Tensor | None = None  # per-slab complement totals of the exit rows


_LOGITS_DTYPES = {torch.float32: _lib.SG_DTYPE_F32, torch.bfloat16: _lib.SG_DTYPE_BF16,
                  torch.float16: _lib.SG_DTYPE_F16}


def _check_logits(logits: torch.Tensor) -> int:
    _require(isinstance(logits, torch.Tensor) and logits.is_cuda,
             "logits must be a HIP device tensor")
    _require(logits.dtype in _LOGITS_DTYPES,
             f"logits must be float32, bfloat16 or float16, got {logits.dtype}")
    _require(logits.dim() == 2 and logits.stride(1) == 1, "logits must be [R, V] row-contiguous")
    return _LOGITS_DTYPES[logits.dtype]


def _check_sample_out(out: "SampleResult", n: int, rows: int, max_depth: int) -> None:
    """Caller-supplied outputs must fit this call exactly (the kernels index
    them by n, R and max_depth)."""
    expect = {
        "accept_nodes": ((n, max(max_depth, 1)), torch.int32),
        "accept_len": ((n,), torch.int32),
        "bonus": ((n,), torch.int32),
        "keep_rows": ((n, max_depth + 1), torch.int32),
        "row_max": ((rows,), torch.float32),
        "row_sum": ((rows,), torch.float32),
        "status": ((1,), torch.int32),
    }
    for name, (shape, dtype) in expect.items():
        t = getattr(out, name)
        _check_device_tensor(t, f"out.{name}", dtype)
        _require(tuple(t.shape) == shape and t.is_contiguous(),
                 f"out.{name} must be a contiguous {list(shape)} tensor for this call, "
                 f"got {list(t.shape)}")


def _check_sample_inputs(logits, row_offset, parent, token, uniforms, max_depth):
    _check_logits(logits)
    for t, name in ((row_offset, "row_offset"), (parent, "parent"), (token, "token")):
        _check_device_tensor(t, name, torch.int32)
        _require(t.is_contiguous(), f"{name} must be contiguous")
    _check_device_tensor(uniforms, "uniforms", torch.float32)
    _require(uniforms.dim() == 2 and uniforms.is_contiguous(), "uniforms must be [n, U]")
    n = row_offset.numel() - 1
    rows = logits.shape[0]
    _require(uniforms.shape[0] == n, "one uniform row per request")
    _require(uniforms.shape[1] >= 2 * (max_depth + 1), "uniforms must cover 2*(max_depth+1)")
    _require(parent.numel() >= rows and token.numel() >= rows, "parent/token must cover R rows")
    return n, rows


def _sample_args(logits, row_offset, parent, token, uniforms, max_depth, out, n, rows,
                 workspace) -> "_lib.SgTreeSampleArgs":
    a = _lib.SgTreeSampleArgs()
    a.num_requests = n
    a.num_rows = rows
    a.vocab = logits.shape[1]
    a.max_depth = max_depth
    a.logits_dtype = _LOGITS_DTYPES[logits.dtype]
    a.logits_dev = logits.data_ptr()
    a.logits_row_stride = logits.stride(0)
    a.row_offset_dev = row_offset.data_ptr()
    a.parent_dev = parent.data_ptr()
    a.token_dev = token.data_ptr()
    a.uniforms_dev = uniforms.data_ptr()
    a.uniform_stride = uniforms.shape[1]
    a.row_max_dev = out.row_max.data_ptr() if hasattr(out, "row_max") else 0
    a.row_sum_dev = out.row_sum.data_ptr() if hasattr(out, "row_sum") else 0
    a.num_logits_rows = logits.shape[0]
    a.accept_nodes_dev = out.accept_nodes.data_ptr()
    a.accept_len_dev = out.accept_len.data_ptr()
    a.bonus_dev = out.bonus.data_ptr()
    a.keep_rows_dev = out.keep_rows.data_ptr()
    a.status_dev = out.status.data_ptr()
    a.workspace_dev = workspace.data_ptr() if workspace is not None else 0
    a.workspace_bytes = workspace.numel() if workspace is not None else 0
    return a


def tree_sample(logits: torch.Tensor, row_offset: torch.Tensor, parent: torch.Tensor,
                token: torch.Tensor, uniforms: torch.Tensor, max_depth: int,
                out: SampleResult | None = None) -> SampleResult:
    """Temperature-1 tree rejection sampling over all packed rows.

    logits [R, V] fp32, bf16 or f16 (row-contiguous; the 16-bit types widen to
    fp32 exactly), row_offset [n+1] i32 with row_offset[n] == R, parent/token
    [R] i32 (request-local parents, -1 for roots), uniforms [n, U] fp32 with
    U >= 2*(max_depth+1).  ``out`` (optional) must have been made for the same
    n, R and max_depth; its status word is cleared by the call.
    """
    n, rows = _check_sample_inputs(logits, row_offset, parent, token, uniforms, max_depth)
    dev = logits.device
    if out is None:
        depth_slots = max(max_depth, 1)
        out = SampleResult(
            accept_nodes=torch.empty((n, depth_slots), dtype=torch.int32, device=dev),
            accept_len=torch.empty(n, dtype=torch.int32, device=dev),
            bonus=torch.empty(n, dtype=torch.int32, device=dev),
            keep_rows=torch.empty((n, max_depth + 1), dtype=torch.int32, device=dev),
            row_max=torch.empty(rows, dtype=torch.float32, device=dev),
            row_sum=torch.empty(rows, dtype=torch.float32, device=dev),
            status=torch.zeros(1, dtype=torch.int32, device=dev),
        )
    else:
        _check_sample_out(out, n, rows, max_depth)
    # statistics of every logits row, with their slab pairs in the workspace
    ws_bytes = int(_lib.load().sg_tree_sample_workspace_bytes(n, logits.shape[0],
                                                              logits.shape[1]))
    if out.workspace is None or out.workspace.numel() < ws_bytes:
        out.workspace = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    a = _sample_args(logits, row_offset, parent, token, uniforms, max_depth, out, n, rows,
                     out.workspace)
    _lib.check(_lib.load().sg_tree_sample(ctypes.byref(a), _stream_handle()), "sg_tree_sample")
    return out


def tree_sample_noalloc(logits: torch.Tensor, row_offset: torch.Tensor, parent: torch.Tensor,
                        token: torch.Tensor, uniforms: torch.Tensor, max_depth: int,
                        out: SampleResult) -> SampleResult:
    """tree_sample through sg_tree_sample_noalloc: no device memory is
    allocated (the library's static per-GPU scratch replaces the workspace);
    the caller supplies every output in ``out`` (its ``workspace`` is unused)."""
    n, rows = _check_sample_inputs(logits, row_offset, parent, token, uniforms, max_depth)
    _require(isinstance(out, SampleResult), "sg_tree_sample_noalloc needs caller-owned outputs")
    _check_sample_out(out, n, rows, max_depth)
    a = _sample_args(logits, row_offset, parent, token, uniforms, max_depth, out, n, rows, None)
    _lib.check(_lib.load().sg_tree_sample_noalloc(ctypes.byref(a), _stream_handle()),
               "sg_tree_sample_noalloc")
    return out


@dataclass
class ProjectedSampleResult:
    accept_nodes: torch.Tensor   # [n, max_depth] i32, -1 padded
    accept_len: torch.Tensor     # [n] i32
    bonus: torch.Tensor          # [n] i32, -1 where the walk ended at an unprojected leaf
    keep_rows: torch.Tensor      # [n, max_depth + 1] i32
    terminal_leaf: torch.Tensor  # [n] i32: that leaf's local node id, else -1
    status: torch.Tensor         # [1] i32
    workspace: torch.Tensor


def tree_sample_projected(logits: torch.Tensor, row_offset: torch.Tensor, parent: torch.Tensor,
                          token: torch.Tensor, uniforms: torch.Tensor, max_depth: int, *,
                          row_max: torch.Tensor, row_sum: torch.Tensor,
                          row_map: torch.Tensor | None = None) -> ProjectedSampleResult:
    """The tree walk over LM-head logits whose statistics are already known
    (``lm_head`` wrote them): sg_tree_sample with SG_SAMPLE_STATS_READY.

    ``logits`` [Rp, V] holds the projected rows; ``row_map`` [R] i32 gives
    each packed node's logits row, -1 for a node that was not projected (only
    nodes without children; a walk that ends there reports it in
    ``terminal_leaf`` and leaves its bonus -1), None when row r is node r.
    ``row_max``/``row_sum`` [Rp] f32 are the LM head's row statistics.
    """
    _check_logits(logits)
    for t, name in ((row_offset, "row_offset"), (parent, "parent"), (token, "token")):
        _check_device_tensor(t, name, torch.int32)
        _require(t.is_contiguous(), f"{name} must be contiguous")
    _check_device_tensor(uniforms, "uniforms", torch.float32)
    _require(uniforms.dim() == 2 and uniforms.is_contiguous(), "uniforms must be [n, U]")
    n = row_offset.numel() - 1
    rows = parent.numel()
    logit_rows = logits.shape[0]
    _require(uniforms.shape[0] == n, "one uniform row per request")
    _require(uniforms.shape[1] >= 2 * (max_depth + 1), "uniforms must cover 2*(max_depth+1)")
    _require(token.numel() == rows, "parent and token must both cover the R packed rows")
    for t, name in ((row_max, "row_max"), (row_sum, "row_sum")):
        _check_device_tensor(t, name, torch.float32)
        _require(t.numel() == logit_rows and t.is_contiguous(), f"{name} must be [Rp]")
    if row_map is None:
        _require(logit_rows == rows, "without a row map the logits rows are the packed rows")
    else:
        _check_device_tensor(row_map, "row_map", torch.int32)
        _require(row_map.numel() == rows and row_map.is_contiguous(), "row_map must be [R]")
    dev = logits.device
    depth_slots = max(max_depth, 1)
    ws_bytes = int(_lib.load().sg_tree_sample_workspace_bytes(n, 0, logits.shape[1]))
    out = ProjectedSampleResult(
        accept_nodes=torch.empty((n, depth_slots), dtype=torch.int32, device=dev),
        accept_len=torch.empty(n, dtype=torch.int32, device=dev),
        bonus=torch.empty(n, dtype=torch.int32, device=dev),
        keep_rows=torch.empty((n, max_depth + 1), dtype=torch.int32, device=dev),
        terminal_leaf=torch.empty(n, dtype=torch.int32, device=dev),
        status=torch.zeros(1, dtype=torch.int32, device=dev),
        workspace=torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev))
    a = _sample_args(logits, row_offset, parent, token, uniforms, max_depth, out, n, rows,
                     out.workspace)
    a.row_max_dev = row_max.data_ptr()
    a.row_sum_dev = row_sum.data_ptr()
    a.logits_row_dev = row_map.data_ptr() if row_map is not None else 0
    a.num_logits_rows = logit_rows
    a.flags = _lib.SG_SAMPLE_STATS_READY
    a.terminal_leaf_dev = out.terminal_leaf.data_ptr()
    _lib.check(_lib.load().sg_tree_sample(ctypes.byref(a), _stream_handle()), "sg_tree_sample")
    return out


def row_stats(logits: torch.Tensor):
    dtype = _check_logits(logits)
    rows = logits.shape[0]
    m = torch.empty(rows, dtype=torch.float32, device=logits.device)
    z = torch.empty(rows, dtype=torch.float32, device=logits.device)
    _lib.check(_lib.load().sg_row_stats(logits.data_ptr(), dtype, logits.stride(0),
                                        logits.shape[1], rows, m.data_ptr(), z.data_ptr(),
                                        _stream_handle()),
               "sg_row_stats")
    return m, z


def exp_probe(x: torch.Tensor) -> torch.Tensor:
    _check_device_tensor(x, "x", torch.float32)
    x = x.contiguous()
    out = torch.empty_like(x)
    _lib.check(_lib.load().sg_exp_probe(x.data_ptr(), out.data_ptr(), x.numel(),
                                        _stream_handle()), "sg_exp_probe")
    return out


class ClockProbe:
    """Average shader clock over timed regions, per XCD.

    ``mark()`` enqueues ``sg_clock_probe`` on the current stream and returns
    the mark's index; after the stream has been synchronized, ``ghz(a, b)``
    gives {xcd: GHz} between marks ``a`` and ``b``.  The shader-cycle counters
    of different CUs are not aligned, so every CU that both marks saw gives
    its own clock (its counter's delta over the constant-rate counter's delta,
    times that counter's rate) and each XCD reports the median over its CUs.
    ``blocks`` workgroups per mark (1,024: every CU is seen by nearly every
    mark).  ``spread(a)`` is the largest difference of the shader-cycle
    counter between workgroups on one CU at one mark.
    """

    def __init__(self, device, capacity: int = 512, blocks: int = 1024):
        lib = _lib.load()
        index = torch.device(device).index or 0
        khz = int(lib.sg_wall_clock_khz(index))
        _require(khz > 0, "sg_wall_clock_khz failed: "
                 + lib.sg_last_error().decode(errors="replace"))
        self.wall_hz = khz * 1e3
        self.blocks, self.capacity, self.count = blocks, capacity, 0
        self._buf = torch.zeros((capacity, blocks, 4), dtype=torch.int64, device=device)

    def mark(self) -> int:
        _require(self.count < self.capacity, "clock probe capacity exhausted")
        _lib.check(_lib.load().sg_clock_probe(self._buf[self.count].data_ptr(), self.blocks,
                                              _stream_handle()), "sg_clock_probe")
        self.count += 1
        return self.count - 1

    def _per_cu(self, mark: int) -> dict:
        h = self._buf[mark].cpu().numpy()
        keys = h[:, 0] * 256 + ((h[:, 3] >> 8) & 0xFF)  # XCD, engine, array, CU
        return {int(k): (np.median(h[keys == k][:, 1]), np.median(h[keys == k][:, 2]),
                         int(np.ptp(h[keys == k][:, 1])))
                for k in np.unique(keys)}

    def ghz(self, a: int, b: int) -> dict:
        ra, rb = self._per_cu(a), self._per_cu(b)
        per_xcd: dict = {}
        for k in ra.keys() & rb.keys():
            ticks = rb[k][1] - ra[k][1]
            if ticks > 0:
                per_xcd.setdefault(k // 256, []).append(
                    (rb[k][0] - ra[k][0]) / ticks * self.wall_hz / 1e9)
        return {x: float(np.median(v)) for x, v in sorted(per_xcd.items())}

    def spread(self, a: int) -> int:
        return max(v[2] for v in self._per_cu(a).values())


# --------------------------------------------------------------------------
# (D) LM head with fused statistics
# --------------------------------------------------------------------------

@dataclass
class LmHeadResult:
    logits: torch.Tensor      # [Rp, V] bf16 (a view of rows padded to 8 elements)
    tile_stats: torch.Tensor  # [Rp, ceil(V/128), 2] f32: (max, sum of E(x - max)) per tile
    row_max: torch.Tensor     # [Rp] f32
    row_sum: torch.Tensor     # [Rp] f32
    status: torch.Tensor      # [1] i32: SG_EINVAL when a row index was out of range


class PackedLmHead:
    """``lm_head.weight`` re-laid out once for ``sg_lm_head_packed`` (every
    16 KiB weight stage of the kernel contiguous).  Holds the packed bytes
    beside the model's own weight; ``shape`` and ``dtype`` are the original
    weight's, so it stands in for it wherever ``lm_head`` takes a weight."""
    __slots__ = ("packed", "shape", "dtype", "device")

    def __init__(self, weight: torch.Tensor):
        _check_device_tensor(weight, "weight", torch.bfloat16)
        _require(weight.dim() == 2 and weight.stride(1) == 1,
                 "weight must be a row-contiguous matrix")
        vocab, hsize = weight.shape
        lib = _lib.load()
        nbytes = int(lib.sg_lm_head_packed_bytes(vocab, hsize))
        _require(nbytes > 0, "weight size unsupported (H a positive multiple of 64)")
        self.packed = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=weight.device)
        _lib.check(lib.sg_lm_head_pack_weight(weight.data_ptr(), weight.stride(0), vocab, hsize,
                                              self.packed.data_ptr(), _stream_handle()),
                   "sg_lm_head_pack_weight")
        self.shape = torch.Size((vocab, hsize))
        self.dtype = weight.dtype
        self.device = weight.device


def pack_lm_head(weight: torch.Tensor) -> PackedLmHead:
    """One-time packing of ``lm_head.weight`` for ``lm_head`` (enqueued on
    torch's current stream)."""
    return PackedLmHead(weight)


def lm_head(hidden: torch.Tensor, weight,
            row_index: torch.Tensor | None = None) -> LmHeadResult:
    """bf16 logits of the selected hidden rows and their softmax statistics
    (sg_lm_head, or sg_lm_head_packed for a PackedLmHead).

    ``hidden`` [N, H] bf16 (row-contiguous, H a multiple of 64), ``weight``
    [V, H] bf16 (``lm_head.weight``) or its ``PackedLmHead`` (same results,
    bit for bit), ``row_index`` [Rp] i32 selects the rows
    to project (None: all N).  Replaces ``lm_head(hidden)`` +
    ``probabilities(...)`` on the rows a tree walk can need
    (fused_tree_sampling.py:2899-2913, :2974-2984).
    """
    packed = isinstance(weight, PackedLmHead)
    checked = (hidden,) if packed else (hidden, weight)
    for t, name in zip(checked, ("hidden", "weight")):
        _check_device_tensor(t, name, torch.bfloat16)
        _require(t.dim() == 2 and t.stride(1) == 1, f"{name} must be a row-contiguous matrix")
    _require(hidden.shape[1] == weight.shape[1], "hidden and weight disagree on the hidden size")
    if row_index is not None:
        _check_device_tensor(row_index, "row_index", torch.int32)
        _require(row_index.dim() == 1 and row_index.is_contiguous(), "row_index must be [Rp]")
    rows = row_index.numel() if row_index is not None else hidden.shape[0]
    vocab, hsize = weight.shape
    dev = hidden.device
    pad = (vocab + 7) // 8 * 8
    tiles = int(_lib.load().sg_lm_head_tile_count(vocab))
    logits = torch.empty((rows, pad), dtype=torch.bfloat16, device=dev)
    res = LmHeadResult(
        logits=logits[:, :vocab],
        tile_stats=torch.empty((rows, tiles, 2), dtype=torch.float32, device=dev),
        row_max=torch.empty(rows, dtype=torch.float32, device=dev),
        row_sum=torch.empty(rows, dtype=torch.float32, device=dev),
        status=torch.zeros(1, dtype=torch.int32, device=dev))
    a = _lib.SgLmHeadArgs()
    a.num_rows = rows
    a.hidden_size = hsize
    a.vocab = vocab
    a.num_hidden_rows = hidden.shape[0]
    a.hidden_dev = hidden.data_ptr()
    a.hidden_row_stride = hidden.stride(0)
    a.row_index_dev = row_index.data_ptr() if row_index is not None else 0
    a.weight_dev = weight.packed.data_ptr() if packed else weight.data_ptr()
    a.weight_row_stride = hsize if packed else weight.stride(0)
    a.logits_dev = logits.data_ptr()
    a.logits_row_stride = pad
    a.tile_stats_dev = res.tile_stats.data_ptr()
    a.row_max_dev = res.row_max.data_ptr()
    a.row_sum_dev = res.row_sum.data_ptr()
    a.status_dev = res.status.data_ptr()
    name = "sg_lm_head_packed" if packed else "sg_lm_head"
    _lib.check(getattr(_lib.load(), name)(ctypes.byref(a), _stream_handle()), name)
    return res
