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
// Layout: one workgroup per (request, layer) moves that layer's kept rows
// (16-byte chunks per thread, coalesced, several loads in flight per
// thread).  With one layer the same workgroup then advances the request's
// length; with more, a second launch advances every length once all copies
// have read it, so no copy can see a length already advanced.  A kept row
// outside the request's packed rows leaves the request untouched and reports
// SG_EINVAL through status.
#include <type_traits>

#include "sg_common.h"

namespace sg {
namespace {

constexpr int kCommitThreads = 512;
constexpr int kCommitBatch = 4;      // 16-byte chunks a thread loads before it stores any
constexpr int kStagedRows = 256;     // kept rows staged in LDS (longer keep lists read global)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
using GlobalU4 = __attribute__((address_space(1))) u32x4;

// A request's commit metadata.  Every workgroup of the request checks it on
// the same inputs (capacity: SG_ERANGE; kept rows inside the request's packed
// rows: SG_EINVAL), so all of them skip the request or all of them copy it.
struct CommitRequest {
  int keep_len;
  int len;
  int r0;
  int rows;
  int64_t start;
};

__device__ __forceinline__ CommitRequest load_request(const SgKvCommitArgs& a, int req) {
  CommitRequest r;
  r.keep_len = a.keep_len_dev[req];
  r.len = a.lengths_dev[req];
  r.r0 = a.row_offset_dev[req];
  r.rows = a.row_offset_dev[req + 1] - r.r0;
  r.start = a.prefix_start_dev[req];
  return r;
}

__device__ __forceinline__ bool capacity_ok(const SgKvCommitArgs& a, const CommitRequest& r) {
  return r.len >= 0 && r.len + r.keep_len <= a.capacity && r.keep_len <= a.keep_stride;
}

// Copies the kept rows of layer blockIdx.y of request blockIdx.x.  kUpdate:
// the grid has one layer, and the workgroup also advances the request's
// length after its copy.
template <bool kUpdate>
__global__ __launch_bounds__(kCommitThreads) void kv_commit_kernel(SgKvCommitArgs a) {
  __shared__ int s_keep[kStagedRows];
  __shared__ int s_bad[kCommitThreads / 64];
  const int req = blockIdx.x;
  const int layer = blockIdx.y;
  // Everything the copy needs is loaded in one round trip: the request's
  // metadata, this thread's kept row (every thread below keep_stride reads
  // one; the keep array is [n, keep_stride]) and the layer's bases.
  const CommitRequest r = load_request(a, req);
  const int32_t* keep = a.keep_rows_dev + static_cast<int64_t>(a.keep_stride) * req;
  const int my_keep = static_cast<int>(threadIdx.x) < a.keep_stride ? keep[threadIdx.x] : -1;
  const uint16_t* k_src = static_cast<const uint16_t*>(a.k_tree_layers_dev[layer]);
  const uint16_t* v_src = static_cast<const uint16_t*>(a.v_tree_layers_dev[layer]);
  uint16_t* k_dst = static_cast<uint16_t*>(a.k_cache_layers_dev[layer]);
  uint16_t* v_dst = static_cast<uint16_t*>(a.v_cache_layers_dev[layer]);
  // An empty asm that reads every loaded value keeps the compiler from sinking
  // the loads behind the branches below (one wait for all of them).
  asm volatile("" ::"s"(r.keep_len), "s"(r.len), "s"(r.r0), "s"(r.rows), "s"(r.start),
               "s"(k_src), "s"(v_src), "s"(k_dst), "s"(v_dst), "v"(my_keep));
  const bool empty = r.keep_len <= 0;
  if (empty || !capacity_ok(a, r)) {
    if (!empty && threadIdx.x == 0 && blockIdx.y == 0 && a.status_dev)
      atomicExch(a.status_dev, SG_ERANGE);
    return;
  }
  // Every kept row is checked by one thread, in parallel, and staged in LDS;
  // each wave reports through its own LDS word.
  bool bad = false;
  for (int t = threadIdx.x; t < r.keep_len; t += kCommitThreads) {
    const int k = t == static_cast<int>(threadIdx.x) ? my_keep : keep[t];
    bad = bad || k < 0 || k >= r.rows;
    if (t < kStagedRows) s_keep[t] = k;
  }
  const bool wave_bad = __ballot(bad) != 0;
  if ((threadIdx.x & 63) == 0) s_bad[threadIdx.x / 64] = wave_bad ? 1 : 0;
  __syncthreads();
  int any_bad = 0;
#pragma unroll
  for (int w = 0; w < kCommitThreads / 64; ++w) any_bad |= s_bad[w];
  if (any_bad) {
    if (threadIdx.x == 0 && blockIdx.y == 0 && a.status_dev) atomicExch(a.status_dev, SG_EINVAL);
    return;
  }
  const int chunks_per_head = a.head_dim / 8;  // 8 bf16 = 16 bytes
  const int chunks_per_row = a.num_kv_heads * chunks_per_head;
  const int total = r.keep_len * 2 * chunks_per_row;  // the host bounds this below 2^31
  const int64_t dst_token0 = r.start + r.len;
  // Chunk idx -> (source, destination).  Lanes past the end load the pass's
  // first chunk again and store nothing.  The kept row comes from LDS when
  // the list is staged, else from global memory.
  auto locate = [&](auto staged, int raw, int base, const GlobalU4*& from, GlobalU4*& to) {
    const int idx = raw < total ? raw : base;
    const int t = idx / (2 * chunks_per_row);
    const int rem = idx - t * (2 * chunks_per_row);
    const bool is_v = rem >= chunks_per_row;
    const int c = is_v ? rem - chunks_per_row : rem;
    const int g = c / chunks_per_head;
    const int chunk = c - g * chunks_per_head;
    int k;
    if constexpr (decltype(staged)::value) {
      k = s_keep[t];
    } else {
      k = keep[t];
    }
    from = (const GlobalU4*)((is_v ? v_src : k_src) +
                             static_cast<int64_t>(r.r0 + k) * a.tree_row_stride +
                             g * a.tree_head_stride + chunk * 8);
    to = raw < total ? (GlobalU4*)((is_v ? v_dst : k_dst) + g * a.cache_head_stride +
                                   (dst_token0 + t) * a.cache_token_stride + chunk * 8)
                     : nullptr;
  };
  // Each pass loads four chunks per thread, then stores them: one memory
  // round trip per pass.
  static_assert(kCommitBatch == 4, "the pass below is written out for four chunks");
  auto copy = [&](auto staged) {
    for (int base = threadIdx.x; base < total; base += kCommitBatch * kCommitThreads) {
      const GlobalU4 *f0, *f1, *f2, *f3;
      GlobalU4 *t0, *t1, *t2, *t3;
      locate(staged, base, base, f0, t0);
      locate(staged, base + kCommitThreads, base, f1, t1);
      locate(staged, base + 2 * kCommitThreads, base, f2, t2);
      locate(staged, base + 3 * kCommitThreads, base, f3, t3);
      const u32x4 v0 = *f0, v1 = *f1, v2 = *f2, v3 = *f3;
      // All four loads complete here, before the conditional stores (the
      // compiler would otherwise sink each load into its store's branch).
      asm volatile("" ::"v"(v0), "v"(v1), "v"(v2), "v"(v3));
      if (t0 != nullptr) *t0 = v0;
      if (t1 != nullptr) *t1 = v1;
      if (t2 != nullptr) *t2 = v2;
      if (t3 != nullptr) *t3 = v3;
    }
  };
  if (r.keep_len <= kStagedRows) {
    copy(std::true_type{});
  } else {
    copy(std::false_type{});
  }
  if constexpr (kUpdate) {
    __syncthreads();
    if (threadIdx.x == 0) a.lengths_dev[req] = r.len + r.keep_len;
  }
}

// Advances the lengths after a copy launch with several workgroups per
// request: one wave per request repeats the copy's checks.
__global__ __launch_bounds__(64) void kv_commit_lengths_kernel(SgKvCommitArgs a) {
  const int req = blockIdx.x;
  const CommitRequest r = load_request(a, req);
  if (r.keep_len <= 0 || !capacity_ok(a, r)) return;
  const int32_t* keep = a.keep_rows_dev + static_cast<int64_t>(a.keep_stride) * req;
  bool bad = false;
  for (int t = threadIdx.x; t < r.keep_len; t += 64) {
    const int k = keep[t];
    bad = bad || k < 0 || k >= r.rows;
  }
  if (__ballot(bad) != 0) return;
  if (threadIdx.x == 0) a.lengths_dev[req] = r.len + r.keep_len;
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
  // Chunk indices of one workgroup are 32-bit: up to 2^31 / (2 * Hkv * D/8)
  // kept rows per request and layer.
  SG_REQUIRE(static_cast<int64_t>(a.keep_stride) * 2 * a.num_kv_heads * (a.head_dim / 8) <
                 (int64_t{1} << 31),
             "keep_stride * 2 * num_kv_heads * head_dim / 8 must stay below 2^31");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a.num_layers == 1) {
    // One workgroup per request copies and advances the length.
    hipLaunchKernelGGL(kv_commit_kernel<true>, dim3(a.num_requests), dim3(kCommitThreads), 0, s,
                       a);
    SG_LAUNCH_CHECK();
    return SG_OK;
  }
  // One workgroup per (request, layer); the lengths advance in a second launch,
  // after every copy has read them.
  hipLaunchKernelGGL(kv_commit_kernel<false>, dim3(a.num_requests, a.num_layers),
                     dim3(kCommitThreads), 0, s, a);
  SG_LAUNCH_CHECK();
  hipLaunchKernelGGL(kv_commit_lengths_kernel, dim3(a.num_requests), dim3(64), 0, s, a);
  SG_LAUNCH_CHECK();
  return SG_OK;
}
