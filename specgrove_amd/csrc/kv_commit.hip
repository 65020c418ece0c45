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
#include <algorithm>
#include <climits>
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

// ---------------------------------------------------------------------------
// Non-persistent split: rebuild every request's cache from one packed wave,
// all layers in one launch (reference _split_compacted_sequence_caches,
// continuous_tree_block_decode.py:409-450):
//   out[l][g, o_i + t]       = prefix[l][g, c_i + t]                 t < L_i
//   out[l][g, o_i + L_i + t] = tree[l][q_i + keep_i[t], g]           t < keep_len_i
// Grid (token block, request, layer); a workgroup moves the tokens of one
// block of one request's new cache for one layer (1024 16-byte chunks: 8
// tokens at 8 kv heads x D 128), four loads in flight per thread.  A kept row
// outside the request's packed rows is not copied and raises status
// (SG_EINVAL); so does a request longer than max_tokens.
// ---------------------------------------------------------------------------
namespace sg {
namespace {

constexpr int kSplitThreads = 256;
constexpr int kSplitChunksPerBlock = kSplitThreads * kCommitBatch;

__global__ __launch_bounds__(kSplitThreads) void kv_split_kernel(SgKvSplitArgs a,
                                                                 int tokens_per_block) {
  const int req = blockIdx.y;
  const int layer = blockIdx.z;
  const int L = a.old_length_dev[req];
  const int keep_len = a.keep_len_dev[req];
  const int r0 = a.row_offset_dev[req];
  const int rows = a.row_offset_dev[req + 1] - r0;
  const int64_t c0 = a.cache_offset_dev[req];
  const int64_t o0 = a.out_offset_dev[req];
  const int32_t* keep = a.keep_rows_dev + static_cast<int64_t>(a.keep_stride) * req;
  const int n_out = L + keep_len;
  if (blockIdx.x == 0 && layer == 0 && threadIdx.x == 0 && a.status_dev != nullptr &&
      (L < 0 || keep_len < 0 || keep_len > a.keep_stride || n_out > a.max_tokens))
    atomicExch(a.status_dev, SG_EINVAL);
  if (L < 0 || keep_len < 0 || keep_len > a.keep_stride || n_out > a.max_tokens) return;
  const int t_begin = blockIdx.x * tokens_per_block;
  const int t_end = min(n_out, t_begin + tokens_per_block);
  if (t_begin >= t_end) return;
  const uint16_t* k_pre = static_cast<const uint16_t*>(a.k_prefix_layers_dev[layer]);
  const uint16_t* v_pre = static_cast<const uint16_t*>(a.v_prefix_layers_dev[layer]);
  const uint16_t* k_tree = static_cast<const uint16_t*>(a.k_tree_layers_dev[layer]);
  const uint16_t* v_tree = static_cast<const uint16_t*>(a.v_tree_layers_dev[layer]);
  uint16_t* k_out = static_cast<uint16_t*>(a.k_out_layers_dev[layer]);
  uint16_t* v_out = static_cast<uint16_t*>(a.v_out_layers_dev[layer]);
  const int chunks_per_head = a.head_dim / 8;
  const int chunks_per_token = 2 * a.num_kv_heads * chunks_per_head;  // K then V
  const int total = (t_end - t_begin) * chunks_per_token;
  // Chunk idx -> (source, destination); nullptr destination: nothing to do.
  auto locate = [&](int idx, const GlobalU4*& from, GlobalU4*& to) {
    from = nullptr;
    to = nullptr;
    if (idx >= total) return;
    const int t = t_begin + idx / chunks_per_token;
    const int rem = idx % chunks_per_token;
    const bool is_v = rem >= chunks_per_token / 2;
    const int c = is_v ? rem - chunks_per_token / 2 : rem;
    const int g = c / chunks_per_head;
    const int chunk = c - g * chunks_per_head;
    if (t < L) {
      from = (const GlobalU4*)((is_v ? v_pre : k_pre) + g * a.prefix_head_stride +
                               (c0 + t) * a.prefix_token_stride + chunk * 8);
    } else {
      const int k = keep[t - L];
      if (k < 0 || k >= rows) {
        if (a.status_dev != nullptr) atomicExch(a.status_dev, SG_EINVAL);
        return;
      }
      from = (const GlobalU4*)((is_v ? v_tree : k_tree) +
                               static_cast<int64_t>(r0 + k) * a.tree_row_stride +
                               g * a.tree_head_stride + chunk * 8);
    }
    to = (GlobalU4*)((is_v ? v_out : k_out) + g * a.out_head_stride +
                     (o0 + t) * a.out_token_stride + chunk * 8);
  };
  for (int base = threadIdx.x; base < total; base += kSplitChunksPerBlock) {
    const GlobalU4* f[kCommitBatch];
    GlobalU4* d[kCommitBatch];
    u32x4 v[kCommitBatch];
#pragma unroll
    for (int j = 0; j < kCommitBatch; ++j) locate(base + j * kSplitThreads, f[j], d[j]);
#pragma unroll
    for (int j = 0; j < kCommitBatch; ++j) v[j] = d[j] != nullptr ? *f[j] : u32x4{0, 0, 0, 0};
    // All four loads complete here, before the conditional stores.
    asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]));
#pragma unroll
    for (int j = 0; j < kCommitBatch; ++j)
      if (d[j] != nullptr) *d[j] = v[j];
  }
}

}  // namespace
}  // namespace sg

extern "C" int sg_kv_split(const SgKvSplitArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null SgKvSplitArgs");
  const SgKvSplitArgs& a = *args;
  SG_REQUIRE(a.num_layers >= 0 && a.num_requests >= 0 && a.max_tokens >= 0, "negative sizes");
  if (a.num_layers == 0 || a.num_requests == 0 || a.max_tokens == 0) return SG_OK;
  SG_REQUIRE(a.num_kv_heads >= 1 && a.head_dim >= 8 && a.head_dim % 8 == 0,
             "head_dim must be a positive multiple of 8");
  SG_REQUIRE(a.keep_stride >= 1, "keep_stride must be positive");
  SG_REQUIRE(a.prefix_head_stride % 8 == 0 && a.prefix_token_stride % 8 == 0 &&
                 a.tree_row_stride % 8 == 0 && a.tree_head_stride % 8 == 0 &&
                 a.out_head_stride % 8 == 0 && a.out_token_stride % 8 == 0,
             "strides must be multiples of 8 elements (16-byte rows)");
  SG_REQUIRE(a.k_prefix_layers_dev && a.v_prefix_layers_dev && a.k_tree_layers_dev &&
                 a.v_tree_layers_dev && a.k_out_layers_dev && a.v_out_layers_dev &&
                 a.cache_offset_dev && a.old_length_dev && a.row_offset_dev &&
                 a.keep_rows_dev && a.keep_len_dev && a.out_offset_dev,
             "null device pointer");
  SG_REQUIRE(a.num_requests <= 65535 && a.num_layers <= 65535,
             "at most 65535 requests and layers per call");
  const int chunks_per_token = 2 * a.num_kv_heads * (a.head_dim / 8);
  SG_REQUIRE(chunks_per_token <= (1 << 20), "num_kv_heads * head_dim too large");
  const int tokens_per_block = std::max(1, kSplitChunksPerBlock / chunks_per_token);
  const int64_t blocks = (static_cast<int64_t>(a.max_tokens) + tokens_per_block - 1) /
                         tokens_per_block;
  SG_REQUIRE(blocks <= INT32_MAX, "max_tokens too large");
  hipLaunchKernelGGL(kv_split_kernel,
                     dim3(static_cast<unsigned>(blocks), a.num_requests, a.num_layers),
                     dim3(kSplitThreads), 0, reinterpret_cast<hipStream_t>(stream), a,
                     tokens_per_block);
  SG_LAUNCH_CHECK();
  return SG_OK;
}
