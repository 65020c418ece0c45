// Accepted-path KV commit: scatter the kept tree rows of every request into
// that request's cache region, for all layers in one launch.
//
// Semantics of the reference's persistent-arena append (reference
// continuous_tree_block_decode.py:215-261) with keep_i = [0] + accepted local
// nodes (:2108-2109):
//   cache[l][g, prefix_start_i + len_i + t] = tree[l][row_offset_i + keep_i[t], g]
// then len_i += keep_len_i.  A request whose rows would pass the capacity is
// left untouched and reported through status (reference :235-236 raises).
//
// Layout: one workgroup per request moves the request's kept rows of every
// layer (16-byte chunks per thread, coalesced), then advances the request's
// length; only that workgroup touches the length, so reading the old length
// and writing the new one cannot race across layers.
#include "sg_common.h"

namespace sg {
namespace {

constexpr int kCommitThreads = 512;

__global__ __launch_bounds__(kCommitThreads) void kv_commit_kernel(SgKvCommitArgs a) {
  const int req = blockIdx.x;
  const int keep_len = a.keep_len_dev[req];
  if (keep_len <= 0) return;
  const int len = a.lengths_dev[req];
  if (len < 0 || len + keep_len > a.capacity || keep_len > a.keep_stride) {
    if (threadIdx.x == 0 && a.status_dev) atomicExch(a.status_dev, SG_ERANGE);
    return;
  }
  const int r0 = a.row_offset_dev[req];
  const int rows = a.row_offset_dev[req + 1] - r0;
  const int64_t dst_token0 = a.prefix_start_dev[req] + len;
  const int32_t* keep = a.keep_rows_dev + static_cast<int64_t>(a.keep_stride) * req;
  for (int t = 0; t < keep_len; ++t) {
    if (keep[t] < 0 || keep[t] >= rows) {
      if (threadIdx.x == 0 && a.status_dev) atomicExch(a.status_dev, SG_EINVAL);
      return;
    }
  }
  const int chunks_per_head = a.head_dim / 8;  // 8 bf16 = 16 bytes
  const int chunks_per_row = a.num_kv_heads * chunks_per_head;
  const int per_layer = keep_len * 2 * chunks_per_row;
  const int64_t total = static_cast<int64_t>(per_layer) * a.num_layers;
  for (int64_t idx = threadIdx.x; idx < total; idx += kCommitThreads) {
    const int layer = static_cast<int>(idx / per_layer);
    const int in_layer = static_cast<int>(idx - static_cast<int64_t>(layer) * per_layer);
    const int t = in_layer / (2 * chunks_per_row);
    const int rem = in_layer - t * (2 * chunks_per_row);
    const bool is_v = rem >= chunks_per_row;
    const int c = is_v ? rem - chunks_per_row : rem;
    const int g = c / chunks_per_head;
    const int chunk = c - g * chunks_per_head;
    const uint16_t* src = static_cast<const uint16_t*>(
        is_v ? a.v_tree_layers_dev[layer] : a.k_tree_layers_dev[layer]);
    uint16_t* dst = static_cast<uint16_t*>(is_v ? a.v_cache_layers_dev[layer]
                                                : a.k_cache_layers_dev[layer]);
    const int64_t src_row = r0 + keep[t];
    const int64_t src_off = src_row * a.tree_row_stride + g * a.tree_head_stride + chunk * 8;
    const int64_t dst_off =
        g * a.cache_head_stride + (dst_token0 + t) * a.cache_token_stride + chunk * 8;
    *reinterpret_cast<uint4*>(dst + dst_off) = *reinterpret_cast<const uint4*>(src + src_off);
  }
  __syncthreads();
  if (threadIdx.x == 0) a.lengths_dev[req] = len + keep_len;
}

}  // namespace
}  // namespace sg

extern "C" int sg_kv_commit(const SgKvCommitArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null SgKvCommitArgs");
  const SgKvCommitArgs& a = *args;
  SG_REQUIRE(a.num_layers >= 0 && a.num_requests >= 0, "negative sizes");
  if (a.num_layers == 0 || a.num_requests == 0) return SG_OK;
  SG_REQUIRE(a.num_kv_heads >= 1 && a.head_dim >= 8 && a.head_dim % 8 == 0,
             "head_dim must be a positive multiple of 8");
  SG_REQUIRE(a.capacity >= 1 && a.keep_stride >= 1, "capacity and keep_stride must be positive");
  SG_REQUIRE(a.cache_head_stride % 8 == 0 && a.cache_token_stride % 8 == 0 &&
                 a.tree_row_stride % 8 == 0 && a.tree_head_stride % 8 == 0,
             "strides must be multiples of 8 elements (16-byte rows)");
  SG_REQUIRE(a.k_cache_layers_dev && a.v_cache_layers_dev && a.k_tree_layers_dev &&
                 a.v_tree_layers_dev && a.row_offset_dev && a.keep_rows_dev &&
                 a.keep_len_dev && a.prefix_start_dev && a.lengths_dev,
             "null device pointer");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(kv_commit_kernel, dim3(a.num_requests), dim3(kCommitThreads), 0, s, a);
  SG_LAUNCH_CHECK();
  return SG_OK;
}
