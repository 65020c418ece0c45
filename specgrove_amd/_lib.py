"""ctypes binding of libspecgrove_hip.so (the C ABI in include/specgrove_hip.h).

The library is built in-tree by ``specgrove_amd.build``.  Loading fails loudly
when it is missing: there is no CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libspecgrove_hip.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "specgrove_hip.h"

SG_OK = 0
SG_EINVAL = -1
SG_ERANGE = -2
SG_EHIP = -3

SG_ABI_VERSION = 5
SG_DTYPE_F32 = 0
SG_DTYPE_BF16 = 1
SG_DTYPE_F16 = 2
SG_SAMPLE_STATS_READY = 1

c_void_p = ctypes.c_void_p
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_size = ctypes.c_size_t


class SgTreeAttnArgs(ctypes.Structure):
    _fields_ = [
        ("num_requests", c_i32), ("num_rows", c_i32), ("num_q_heads", c_i32),
        ("num_kv_heads", c_i32), ("head_dim", c_i32), ("scale", c_f32),
        ("q_dev", c_void_p), ("q_row_stride", c_i64), ("q_head_stride", c_i64),
        ("k_cache_dev", c_void_p), ("v_cache_dev", c_void_p),
        ("cache_head_stride", c_i64), ("cache_token_stride", c_i64),
        ("k_tree_dev", c_void_p), ("v_tree_dev", c_void_p),
        ("tree_row_stride", c_i64), ("tree_head_stride", c_i64),
        ("row_offset_dev", c_void_p), ("prefix_start_dev", c_void_p),
        ("prefix_len_dev", c_void_p), ("parent_dev", c_void_p),
        ("out_dev", c_void_p), ("out_row_stride", c_i64), ("out_head_stride", c_i64),
        ("plan_dev", c_void_p), ("plan_host", c_void_p), ("plan_units", c_i32),
        ("plan_merges", c_i32), ("workspace_dev", c_void_p), ("workspace_bytes", c_size),
        ("status_dev", c_void_p),
    ]


class SgKvCommitArgs(ctypes.Structure):
    _fields_ = [
        ("num_layers", c_i32), ("num_requests", c_i32), ("num_kv_heads", c_i32),
        ("head_dim", c_i32),
        ("k_cache_layers_dev", c_void_p), ("v_cache_layers_dev", c_void_p),
        ("cache_head_stride", c_i64), ("cache_token_stride", c_i64),
        ("k_tree_layers_dev", c_void_p), ("v_tree_layers_dev", c_void_p),
        ("tree_row_stride", c_i64), ("tree_head_stride", c_i64),
        ("row_offset_dev", c_void_p), ("keep_rows_dev", c_void_p),
        ("keep_stride", c_i32), ("keep_len_dev", c_void_p),
        ("prefix_start_dev", c_void_p), ("lengths_dev", c_void_p),
        ("capacity", c_i32), ("status_dev", c_void_p),
    ]


class SgKvSplitArgs(ctypes.Structure):
    _fields_ = [
        ("num_layers", c_i32), ("num_requests", c_i32), ("num_kv_heads", c_i32),
        ("head_dim", c_i32), ("max_tokens", c_i32), ("keep_stride", c_i32),
        ("k_prefix_layers_dev", c_void_p), ("v_prefix_layers_dev", c_void_p),
        ("prefix_head_stride", c_i64), ("prefix_token_stride", c_i64),
        ("k_tree_layers_dev", c_void_p), ("v_tree_layers_dev", c_void_p),
        ("tree_row_stride", c_i64), ("tree_head_stride", c_i64),
        ("k_out_layers_dev", c_void_p), ("v_out_layers_dev", c_void_p),
        ("out_head_stride", c_i64), ("out_token_stride", c_i64),
        ("cache_offset_dev", c_void_p), ("old_length_dev", c_void_p),
        ("row_offset_dev", c_void_p), ("keep_rows_dev", c_void_p),
        ("keep_len_dev", c_void_p), ("out_offset_dev", c_void_p),
        ("status_dev", c_void_p),
    ]


class SgTreeSampleArgs(ctypes.Structure):
    _fields_ = [
        ("num_requests", c_i32), ("num_rows", c_i32), ("vocab", c_i32),
        ("max_depth", c_i32), ("logits_dtype", c_i32),
        ("logits_dev", c_void_p), ("logits_row_stride", c_i64),
        ("row_offset_dev", c_void_p), ("parent_dev", c_void_p),
        ("token_dev", c_void_p), ("uniforms_dev", c_void_p),
        ("uniform_stride", c_i32),
        ("row_max_dev", c_void_p), ("row_sum_dev", c_void_p),
        ("accept_nodes_dev", c_void_p), ("accept_len_dev", c_void_p),
        ("bonus_dev", c_void_p), ("keep_rows_dev", c_void_p),
        ("status_dev", c_void_p),
        ("workspace_dev", c_void_p), ("workspace_bytes", c_size),
        ("logits_row_dev", c_void_p), ("num_logits_rows", c_i32), ("flags", c_i32),
        ("terminal_leaf_dev", c_void_p),
    ]


class SgLmHeadArgs(ctypes.Structure):
    _fields_ = [
        ("num_rows", c_i32), ("hidden_size", c_i32), ("vocab", c_i32),
        ("num_hidden_rows", c_i32),
        ("hidden_dev", c_void_p), ("hidden_row_stride", c_i64),
        ("row_index_dev", c_void_p),
        ("weight_dev", c_void_p), ("weight_row_stride", c_i64),
        ("logits_dev", c_void_p), ("logits_row_stride", c_i64),
        ("tile_stats_dev", c_void_p), ("row_max_dev", c_void_p), ("row_sum_dev", c_void_p),
        ("status_dev", c_void_p),
    ]


class SgAddRmsNormArgs(ctypes.Structure):
    _fields_ = [
        ("num_rows", c_i32), ("hidden", c_i32), ("eps", c_f32), ("reserved", c_i32),
        ("x_dev", c_void_p), ("x_stride", c_i64),
        ("residual_dev", c_void_p), ("residual_stride", c_i64),
        ("weight_dev", c_void_p), ("out_dev", c_void_p), ("out_stride", c_i64),
        ("residual_out_dev", c_void_p), ("residual_out_stride", c_i64),
    ]


class SgQkNormRopeArgs(ctypes.Structure):
    _fields_ = [
        ("num_rows", c_i32), ("num_q_heads", c_i32), ("num_kv_heads", c_i32),
        ("head_dim", c_i32), ("eps", c_f32), ("reserved", c_i32),
        ("qkv_dev", c_void_p), ("qkv_row_stride", c_i64),
        ("q_norm_dev", c_void_p), ("k_norm_dev", c_void_p), ("inv_freq_dev", c_void_p),
        ("positions_dev", c_void_p), ("q_out_dev", c_void_p), ("q_row_stride", c_i64),
        ("k_out_dev", c_void_p), ("v_out_dev", c_void_p), ("kv_head_stride", c_i64),
    ]


EXPORTED_SYMBOLS = (
    "sg_abi_version", "sg_last_error", "sg_abi_struct_size",
    "sg_tree_attn_plan", "sg_tree_attn_fwd", "sg_kv_commit",
    "sg_tree_sample", "sg_tree_sample_workspace_bytes", "sg_row_stats", "sg_exp_probe",
    "sg_clock_probe", "sg_wall_clock_khz",
    "sg_tree_sample_noalloc", "sg_tree_attn_plan_check", "sg_kv_split",
    "sg_lm_head", "sg_lm_head_tile_count", "sg_lm_head_packed", "sg_lm_head_pack_weight",
    "sg_lm_head_packed_bytes",
    "sg_add_rmsnorm", "sg_qk_norm_rope", "sg_silu_mul", "sg_gather_rows",
)

# Static scratch of sg_tree_sample_noalloc (SG_TREE_SAMPLE_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 4 << 20

_lib = None


class HipLibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HipLibraryMissing(
            f"{LIB_PATH} is missing; build it with `python -m specgrove_amd.build`")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.sg_abi_version.restype = c_i32
    lib.sg_abi_version.argtypes = []
    lib.sg_last_error.restype = ctypes.c_char_p
    lib.sg_last_error.argtypes = []
    lib.sg_abi_struct_size.restype = c_i64
    lib.sg_abi_struct_size.argtypes = [c_i32]
    lib.sg_tree_attn_plan.restype = c_i32
    lib.sg_tree_attn_plan.argtypes = [
        c_i32, ctypes.POINTER(c_i32), ctypes.POINTER(c_i32), c_i32, c_i32, c_i32, c_i32,
        c_void_p, c_size, ctypes.POINTER(c_size), ctypes.POINTER(c_i32),
        ctypes.POINTER(c_i32), ctypes.POINTER(c_size),
    ]
    lib.sg_tree_attn_plan_check.restype = c_i32
    lib.sg_tree_attn_plan_check.argtypes = [c_void_p, c_i32, ctypes.POINTER(c_i32),
                                            ctypes.POINTER(c_i32)]
    lib.sg_tree_attn_fwd.restype = c_i32
    lib.sg_tree_attn_fwd.argtypes = [ctypes.POINTER(SgTreeAttnArgs), c_void_p]
    lib.sg_kv_commit.restype = c_i32
    lib.sg_kv_commit.argtypes = [ctypes.POINTER(SgKvCommitArgs), c_void_p]
    lib.sg_kv_split.restype = c_i32
    lib.sg_kv_split.argtypes = [ctypes.POINTER(SgKvSplitArgs), c_void_p]
    lib.sg_tree_sample.restype = c_i32
    lib.sg_tree_sample.argtypes = [ctypes.POINTER(SgTreeSampleArgs), c_void_p]
    lib.sg_tree_sample_noalloc.restype = c_i32
    lib.sg_tree_sample_noalloc.argtypes = [ctypes.POINTER(SgTreeSampleArgs), c_void_p]
    lib.sg_tree_sample_workspace_bytes.restype = c_i64
    lib.sg_tree_sample_workspace_bytes.argtypes = [c_i32, c_i32, c_i32]
    lib.sg_row_stats.restype = c_i32
    lib.sg_row_stats.argtypes = [c_void_p, c_i32, c_i64, c_i32, c_i32, c_void_p, c_void_p,
                                 c_void_p]
    lib.sg_lm_head.restype = c_i32
    lib.sg_lm_head.argtypes = [ctypes.POINTER(SgLmHeadArgs), c_void_p]
    lib.sg_lm_head_tile_count.restype = c_i64
    lib.sg_lm_head_tile_count.argtypes = [c_i32]
    lib.sg_lm_head_packed.restype = c_i32
    lib.sg_lm_head_packed.argtypes = [ctypes.POINTER(SgLmHeadArgs), c_void_p]
    lib.sg_lm_head_pack_weight.restype = c_i32
    lib.sg_lm_head_pack_weight.argtypes = [c_void_p, c_i64, c_i32, c_i32, c_void_p, c_void_p]
    lib.sg_lm_head_packed_bytes.restype = c_i64
    lib.sg_lm_head_packed_bytes.argtypes = [c_i32, c_i32]
    lib.sg_add_rmsnorm.restype = c_i32
    lib.sg_add_rmsnorm.argtypes = [ctypes.POINTER(SgAddRmsNormArgs), c_void_p]
    lib.sg_qk_norm_rope.restype = c_i32
    lib.sg_qk_norm_rope.argtypes = [ctypes.POINTER(SgQkNormRopeArgs), c_void_p]
    lib.sg_silu_mul.restype = c_i32
    lib.sg_silu_mul.argtypes = [c_void_p, c_i64, c_i32, c_i32, c_void_p, c_i64, c_void_p]
    lib.sg_gather_rows.restype = c_i32
    lib.sg_gather_rows.argtypes = [c_void_p, c_i32, c_i64, c_i32, c_i32, c_void_p, c_i32,
                                   c_void_p, c_i64, c_void_p, c_void_p]
    lib.sg_clock_probe.restype = c_i32
    lib.sg_clock_probe.argtypes = [c_void_p, c_i32, c_void_p]
    lib.sg_wall_clock_khz.restype = c_i64
    lib.sg_wall_clock_khz.argtypes = [c_i32]
    lib.sg_exp_probe.restype = c_i32
    lib.sg_exp_probe.argtypes = [c_void_p, c_void_p, c_i64, c_void_p]
    version = lib.sg_abi_version()
    if version != SG_ABI_VERSION:
        raise RuntimeError(f"ABI mismatch: the library is version {version}, the binding "
                           f"version {SG_ABI_VERSION}; rebuild with `python -m "
                           f"specgrove_amd.build`")
    expected = {0: SgTreeAttnArgs, 1: SgKvCommitArgs, 2: SgTreeSampleArgs, 3: SgKvSplitArgs,
                4: SgLmHeadArgs, 5: SgAddRmsNormArgs, 6: SgQkNormRopeArgs}
    for which, struct in expected.items():
        size = lib.sg_abi_struct_size(which)
        if size != ctypes.sizeof(struct):
            raise RuntimeError(
                f"ABI mismatch: {struct.__name__} is {size} bytes in the library, "
                f"{ctypes.sizeof(struct)} in the binding")
    _lib = lib
    return lib


def check(code: int, what: str) -> None:
    """Map SG_E* codes to the reference wrapper's exception classes."""
    if code == SG_OK:
        return
    message = load().sg_last_error().decode(errors="replace")
    if code == SG_EINVAL:
        raise ValueError(f"{what}: {message}")
    if code == SG_ERANGE:
        raise RuntimeError(f"{what}: Persistent request KV capacity exhausted ({message})")
    raise RuntimeError(f"{what}: {message} (code {code})")
