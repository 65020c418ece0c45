// Temperature-1 tree rejection sampling over a packed verification wave.
//
// Law: tree_verify_ancestral_batched (reference sampling.py:903-950) -- from a
// node's target row, a draw either follows an outgoing tree edge (the child is
// accepted and the walk continues there) or ends the walk as the bonus token.
// Uniform layout and fallbacks follow the reference's sparse-exit sampler
// (fused_tree_sampling.py:683-824): u[2d] routes over the children's
// cumulative mass in edge order, u[2d+1] draws from the complement of the
// children (the whole row at a leaf), and the fallback is the largest
// non-child token (:804-818).
//
// Arithmetic contract (bit-exact with the CPU restatement): binary32 only,
// no contraction except the explicit fmas of sg_exp, and the fixed reduction
// order below.  A row is addressed as token t = 2048*s + 256*j + 4*l + c
// (slab s, line j, lane l, component c); one wavefront owns a slab at a time
// and reads it as 8 coalesced 1 KiB float4 lines.
//
//   row stats: slab max; lane partials a_c = sum_j E(x - m_s); lane sum
//     (a0+a1)+(a2+a3); xor butterfly over the wave; slab (m, Z) merged into
//     lane s%64; final xor butterfly merge over the 64 lanes.
//   routing:  S += E(x[child token] - m) over children in node order; accept
//     the first child with u*Z < S.
//   exit, slab draw (statistics computed by this call, which keeps every
//     row's slab pairs (m_s, Z_s)): Z'_s = Z_s, or for a slab holding a child
//     token the same sums with the child terms left out; w_s = Z'_s *
//     E(m_s - M); sequential prefixes P_s, C = P_S; the first slab with
//     P_s + w_s > u*C; in it group sums of e = E(x - m_s), an inclusive
//     Kogge-Stone scan over the 64 lanes of each line and sequential line
//     prefixes; the bonus is the first non-child token whose running value
//     P_s + E(m_s - M) * r exceeds u*C, else the slab's last non-child token
//     with e > 0.
//   exit, complement draw (statistics given, SG_SAMPLE_STATS_READY): group
//     sums ((e0+e1)+e2)+e3 of e = E(x - M), inclusive Kogge-Stone scan over
//     the 64 lanes of a line, sequential line and slab prefixes; the bonus is
//     the first non-child token whose running value exceeds u*C.
//   Either way the fallback is the largest non-child token.
#pragma clang fp contract(off)

#include <limits.h>

#include <string>
#include <type_traits>

#include "sg_common.h"
#include "sg_math.h"

namespace sg {
namespace {

constexpr int kSlab = 2048;
constexpr int kLine = 256;
constexpr int kLinesPerSlab = 8;
constexpr int kMaxSlabs = 256;  // vocab <= 524288
constexpr int kStatsThreads = 512;
constexpr int kWalkThreads = 1024;
constexpr int kWalkWaves = kWalkThreads / kWave;
constexpr int kMaxTreeRows = 1024;
// Per-request record that the walk's part 1 leaves for part 2 in the
// workspace, after the slab and line totals: accept length (-1 for a broken
// walk), exit node, child count, exit logits row (-1: an unprojected leaf), then
// the exit node's child tokens.
constexpr int kRecordInts = 4 + kMaxTreeRows;
// Slab statistics of a statistics row: per slab (m_s, Z_s).
constexpr int kSlabStats = 2;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
  return v;
}

__device__ __forceinline__ float wave_butterfly_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = v + __shfl_xor(v, d);
  return v;
}

typedef __attribute__((ext_vector_type(4))) float floatx4;
typedef __attribute__((ext_vector_type(2))) unsigned int uintx2;

// Logits element types.  bf16 and f16 widen to fp32 exactly, so a row of
// either type gives the same statistics and decisions as its fp32 copy.
struct Bf16 {
  uint16_t bits;
};
struct F16 {
  _Float16 v;
};
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(Bf16 v) { return bf16_to_f32(v.bits); }
__device__ __forceinline__ float to_f32(F16 v) { return static_cast<float>(v.v); }

template <typename S>
__device__ __forceinline__ S half_at(uint32_t word, int hi) {
  return __builtin_bit_cast(S, static_cast<uint16_t>(hi ? (word >> 16) : (word & 0xffffu)));
}

// Four consecutive elements at p (16-byte aligned for fp32, 8-byte for the
// 16-bit types), widened to fp32.
template <typename S, bool kStream>
__device__ __forceinline__ void load4(const S* __restrict__ p, float out[4]) {
  if constexpr (sizeof(S) == 4) {
    const floatx4 q = kStream ? __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p))
                              : *reinterpret_cast<const floatx4*>(p);
    out[0] = q[0];
    out[1] = q[1];
    out[2] = q[2];
    out[3] = q[3];
  } else {
    const uintx2 q = kStream ? __builtin_nontemporal_load(reinterpret_cast<const uintx2*>(p))
                             : *reinterpret_cast<const uintx2*>(p);
    out[0] = to_f32(half_at<S>(q[0], 0));
    out[1] = to_f32(half_at<S>(q[0], 1));
    out[2] = to_f32(half_at<S>(q[1], 0));
    out[3] = to_f32(half_at<S>(q[1], 1));
  }
}

// Buffer resource over one logits row (vocab elements from x).  Third word:
// the gfx9 raw-buffer format (32-bit data, no swizzle, offset addressing).
template <typename S>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const S* x, int vocab) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(x), static_cast<short>(0),
                                           vocab * static_cast<int>(sizeof(S)), 0x00020000);
}

// load_slab<S, true, true> through a row's buffer resource, for slabs that
// may lie partly or wholly past the row: a load past the row's end returns
// zeros without a memory access, and the masking of tokens >= vocab is plain
// arithmetic.  With no branch around the loads a wave can prefetch its next
// slab unconditionally; a branch there makes the compiler wait for every
// outstanding load (the prefetch included) before the current slab's
// arithmetic.
constexpr int kBufNonTemporal = 2;  // the slc bit: `nt` on gfx950
template <typename S>
__device__ __forceinline__ void load_slab_rsrc(__amdgpu_buffer_rsrc_t rs, int vocab, int slab,
                                               int lane, float v[32]) {
  const int base = slab * kSlab + 4 * lane;
#pragma unroll
  for (int j = 0; j < kLinesPerSlab; ++j) {
    const int off = (base + kLine * j) * static_cast<int>(sizeof(S));
    if constexpr (sizeof(S) == 4) {
      const floatx4 q = __builtin_bit_cast(
          floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kBufNonTemporal));
      v[4 * j + 0] = q[0];
      v[4 * j + 1] = q[1];
      v[4 * j + 2] = q[2];
      v[4 * j + 3] = q[3];
    } else {
      const uintx2 q = __builtin_bit_cast(
          uintx2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kBufNonTemporal));
      v[4 * j + 0] = to_f32(half_at<S>(q[0], 0));
      v[4 * j + 1] = to_f32(half_at<S>(q[0], 1));
      v[4 * j + 2] = to_f32(half_at<S>(q[1], 0));
      v[4 * j + 3] = to_f32(half_at<S>(q[1], 1));
    }
  }
}

// Tokens >= vocab of slab s read as -inf (vocab is a multiple of 4 on the
// vector path, so each lane's 4-token chunk is wholly in or out).
__device__ __forceinline__ void mask_slab_tail(int vocab, int slab, int lane, float v[32]) {
  if ((slab + 1) * kSlab <= vocab) return;
  const int base = slab * kSlab + 4 * lane;
#pragma unroll
  for (int j = 0; j < kLinesPerSlab; ++j) {
    const bool out = base + kLine * j >= vocab;
#pragma unroll
    for (int c = 0; c < 4; ++c) v[4 * j + c] = out ? -__builtin_inff() : v[4 * j + c];
  }
}

// Lane l of the wave loads tokens 2048*s + 256*j + 4*l + c into v[4*j + c];
// tokens at or beyond vocab read as -inf (they contribute E = 0).
template <typename S, bool kVec, bool kStream = false>
__device__ __forceinline__ void load_slab(const S* __restrict__ x, int vocab,
                                          int slab, int lane, float v[32]) {
  const int base = slab * kSlab + 4 * lane;
  if (kVec && (slab + 1) * kSlab <= vocab) {  // full slab: no bounds checks
    // Non-temporal when asked: the statistics pass reads every row once.
#pragma unroll
    for (int j = 0; j < kLinesPerSlab; ++j) load4<S, kStream>(x + base + kLine * j, v + 4 * j);
  } else if (kVec) {
#pragma unroll
    for (int j = 0; j < kLinesPerSlab; ++j) {
      const int t = base + kLine * j;
      if (t < vocab) {
        load4<S, false>(x + t, v + 4 * j);
      } else {
        v[4 * j + 0] = v[4 * j + 1] = v[4 * j + 2] = v[4 * j + 3] = -__builtin_inff();
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kLinesPerSlab; ++j) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int t = base + kLine * j + c;
        v[4 * j + c] = (t < vocab) ? to_f32(x[t]) : -__builtin_inff();
      }
    }
  }
}

// (m, Z) of slab s from its 32 values per lane (identical in every lane).
__device__ __forceinline__ MZ slab_stats(const float v[32]) {
  float m = v[0];
#pragma unroll
  for (int k = 1; k < 32; ++k) m = fmaxf(m, v[k]);
  m = wave_max(m);
  MZ slab = {m, 0.0f};
  if (m != -__builtin_inff()) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
    for (int j = 0; j < kLinesPerSlab; ++j) {
      a0 = a0 + sg_exp_nonpos(v[4 * j + 0] - m);
      a1 = a1 + sg_exp_nonpos(v[4 * j + 1] - m);
      a2 = a2 + sg_exp_nonpos(v[4 * j + 2] - m);
      a3 = a3 + sg_exp_nonpos(v[4 * j + 3] - m);
    }
    slab.z = wave_butterfly_sum((a0 + a1) + (a2 + a3));
  }
  return slab;
}

// One row per workgroup: its eight waves compute the statistics of slabs
// s = wave, wave + 8, ... (the next slab's loads are issued before the
// current slab's arithmetic), then wave 0 merges the slabs in the canonical
// order -- slab s into lane s % 64 in increasing s, then the xor butterfly
// over the lanes -- which makes the result independent of how slabs were
// spread over waves.  Two workgroups per CU (4 waves per SIMD, 116 VGPRs):
// 512 rows in flight, so 2048 rows run in four equal rounds.  Measured 2 %
// faster over the whole sampling call than five 4-wave workgroups per CU
// (102 VGPRs), and equal to a grid that gives every workgroup the same
// number of (row, slab) tasks.
// Workgroup 0 also clears the caller's status word (when given): the later
// kernels of the call only ever raise it.
// With slab_out the row's slab pairs (m_s, Z_s) are also written there, once
// the slabs are done (600 bytes a row at vocab 151,936).
template <typename S, bool kVec>
__global__ __launch_bounds__(kStatsThreads, 2) void row_stats_kernel(
    const S* __restrict__ logits, int64_t row_stride, int vocab, int rows,
    float* __restrict__ row_max, float* __restrict__ row_sum, float* __restrict__ slab_out,
    int32_t* __restrict__ status) {
  __shared__ float s_m[kMaxSlabs];
  __shared__ float s_z[kMaxSlabs];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row = blockIdx.x;
  if (row == 0 && threadIdx.x == 0 && status != nullptr) *status = SG_OK;
  if (row >= rows) return;
  const S* __restrict__ x = logits + row_stride * row;
  const int slabs = (vocab + kSlab - 1) / kSlab;
  constexpr int kWavesPerRow = kStatsThreads / kWave;
  float v[32], w[32];
  int s = wave;
  if constexpr (kVec) {
    // Steady loop with an unconditional prefetch of the wave's next slab.
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(x, vocab);
    if (s < slabs) {
      load_slab_rsrc<S>(rs, vocab, s, lane, v);
      while (true) {
        load_slab_rsrc<S>(rs, vocab, s + kWavesPerRow, lane, w);
        mask_slab_tail(vocab, s, lane, v);
        const MZ a = slab_stats(v);
        if (lane == 0) {
          s_m[s] = a.m;
          s_z[s] = a.z;
        }
        s += kWavesPerRow;
        if (s >= slabs) break;
        load_slab_rsrc<S>(rs, vocab, s + kWavesPerRow, lane, v);
        mask_slab_tail(vocab, s, lane, w);
        const MZ b = slab_stats(w);
        if (lane == 0) {
          s_m[s] = b.m;
          s_z[s] = b.z;
        }
        s += kWavesPerRow;
        if (s >= slabs) break;
      }
    }
    s = slabs;  // the loop below is the unaligned path's
  }
  if (!kVec && s < slabs) load_slab<S, kVec, true>(x, vocab, s, lane, v);
  while (!kVec && s < slabs) {
    const int next = s + kWavesPerRow;
    if (next < slabs) load_slab<S, kVec, true>(x, vocab, next, lane, w);
    const MZ a = slab_stats(v);
    if (lane == 0) {
      s_m[s] = a.m;
      s_z[s] = a.z;
    }
    if (next >= slabs) break;
    const int next2 = next + kWavesPerRow;
    if (next2 < slabs) load_slab<S, kVec, true>(x, vocab, next2, lane, v);
    const MZ b = slab_stats(w);
    if (lane == 0) {
      s_m[next] = b.m;
      s_z[next] = b.z;
    }
    s = next2;
  }
  __syncthreads();
  if (slab_out != nullptr) {
    float2* __restrict__ out =
        reinterpret_cast<float2*>(slab_out) + static_cast<int64_t>(row) * slabs;
    for (int k = threadIdx.x; k < slabs; k += kStatsThreads) out[k] = make_float2(s_m[k], s_z[k]);
  }
  if (wave != 0) return;
  MZ acc = {-__builtin_inff(), 0.0f};
  for (int t = lane; t < slabs; t += kWave) {
    const MZ slab = {s_m[t], s_z[t]};
    acc = merge_mz(acc, slab);
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    MZ other;
    other.m = __shfl_xor(acc.m, d);
    other.z = __shfl_xor(acc.z, d);
    acc = merge_mz(acc, other);
  }
  if (lane == 0) {
    row_max[row] = acc.m;
    row_sum[row] = acc.z;
  }
}

// Child-token bitmask of this lane in slab s: bit 4*j+c marks token
// 2048*s + 256*j + 4*lane + c as a child token of the exit node.
__device__ __forceinline__ uint32_t child_bits(const int* child_tok, int count,
                                               int slab, int lane) {
  uint32_t bits = 0;
  for (int k = 0; k < count; ++k) {
    const int t = child_tok[k];
    const int local = t - slab * kSlab;
    if (local >= 0 && local < kSlab && ((local >> 2) & (kWave - 1)) == lane)
      bits |= 1u << (4 * (local >> 8) + (local & 3));
  }
  return bits;
}

// Exit-row values of one slab: e = 0 for child tokens and tokens >= vocab.
template <typename S, bool kVec>
__device__ __forceinline__ void exit_values(const S* __restrict__ x, int vocab,
                                            float m, int slab, int lane,
                                            uint32_t bits, float e[32]) {
  load_slab<S, kVec>(x, vocab, slab, lane, e);
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const float val = sg_exp_nonpos(e[k] - m);
    e[k] = ((bits >> k) & 1u) ? 0.0f : val;
  }
}

// Inclusive Kogge-Stone scan of the group sums of each line; returns the
// per-line inclusive values of this lane in incl[j] and the line totals.
__device__ __forceinline__ void line_scans(const float e[32], int lane,
                                           float incl[kLinesPerSlab],
                                           float total[kLinesPerSlab]) {
#pragma unroll
  for (int j = 0; j < kLinesPerSlab; ++j) {
    float g = ((e[4 * j + 0] + e[4 * j + 1]) + e[4 * j + 2]) + e[4 * j + 3];
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const float up = __shfl_up(g, d);
      g = (lane >= d) ? g + up : g;
    }
    incl[j] = g;
    total[j] = __shfl(g, kWave - 1);
  }
}

// Tree data of one request in LDS and the routing walk over it.
struct RouteShared {
  int parent[kMaxTreeRows];
  int token[kMaxTreeRows];
  float xchild[kMaxTreeRows];  // x_parent(c)[token(c)] of node c
  float rm[kMaxTreeRows];
  float rz[kMaxTreeRows];
  float u[2 * kMaxTreeRows + 2];
  int child_tok[kMaxTreeRows];  // children of the exit node, ascending node order
  int lrow[kMaxTreeRows];       // logits row of each node, -1 when not projected
  int child_count;
  int exit_node;
  int depth;
  int broken;
  int bad_rows;  // a node with children has no logits row, or a row is out of range
};

// Gathers everything the routing reads in one parallel round (the tree, the
// row statistics, the uniforms and each node's token logit in its parent's
// row -- the only logits routing touches), then walks on one wave: from v,
// the children in ascending node order accumulate S += E(x_v[token] - m_v) and
// the first child with u[2d] * Z_v < S is accepted.  Accepted nodes are
// written to nodes_out when write_nodes.  Ends with a barrier.
template <typename S>
__device__ void route_request(const SgTreeSampleArgs& a, int req, int r0, int n,
                              RouteShared& sh, bool write_nodes) {
  const S* __restrict__ logits = static_cast<const S*>(a.logits_dev);
  const int tid = threadIdx.x;
  const float* __restrict__ u = a.uniforms_dev + static_cast<int64_t>(a.uniform_stride) * req;
  const int n_u = min(a.uniform_stride, 2 * kMaxTreeRows + 2);
  const int n_logits = a.num_logits_rows > 0 ? a.num_logits_rows : a.num_rows;
  // First memory round trip: the tree, each node's logits row and the uniforms.
  if (tid == 0) sh.bad_rows = 0;
  for (int k = tid; k < n; k += blockDim.x) {
    sh.parent[k] = a.parent_dev[r0 + k];
    sh.token[k] = a.token_dev[r0 + k];
    sh.lrow[k] = a.logits_row_dev != nullptr ? a.logits_row_dev[r0 + k] : r0 + k;
  }
  for (int k = tid; k < n_u; k += blockDim.x) sh.u[k] = u[k];
  __syncthreads();
  // Second round trip: the row statistics and each node's token logit in its parent's
  // row (the only logits routing touches).  A node whose parent has no
  // logits row breaks the lazy-projection contract.
  for (int k = tid; k < n; k += blockDim.x) {
    const int lr = sh.lrow[k];
    const bool own = lr >= 0 && lr < n_logits;
    sh.rm[k] = own ? a.row_max_dev[lr] : -__builtin_inff();
    sh.rz[k] = own ? a.row_sum_dev[lr] : 0.0f;
    const int p = sh.parent[k];
    const int tok = sh.token[k];
    const bool edge = k > 0 && p >= 0 && p < k;
    const int pr = edge ? sh.lrow[p] : -1;
    const bool prow_ok = pr >= 0 && pr < n_logits;
    const bool readable = edge && prow_ok && tok >= 0 && tok < a.vocab;
    sh.xchild[k] = readable ? to_f32(logits[a.logits_row_stride * pr + tok]) : 0.0f;
    if (lr >= n_logits || (edge && !prow_ok)) sh.bad_rows = 1;
  }
  __syncthreads();
  // Wave 0 walks; every lane holds the same state.  The children of v, in
  // ascending node order, are the nodes c > v with parent v, found 64 at a
  // time by ballot and visited lowest bit first.
  if (tid < kWave) {
    const int lane = tid;
    int32_t* nodes_out = a.accept_nodes_dev + static_cast<int64_t>(a.max_depth) * req;
    int v = 0;
    int depth = 0;
    int broken = sh.bad_rows;
    for (;;) {
      if (broken) break;
      if (2 * depth + 1 >= a.uniform_stride || 2 * depth + 1 >= n_u) {
        broken = 1;
        break;
      }
      const float m = sh.rm[v];
      const float threshold = sh.u[2 * depth] * sh.rz[v];
      float cumulative = 0.0f;
      int accepted = -1;
      for (int base = v + 1; base < n && accepted == -1; base += kWave) {
        uint64_t mask = __ballot(base + lane < n && sh.parent[base + lane] == v);
        while (mask != 0) {
          const int c = base + __builtin_ctzll(mask);
          mask &= mask - 1;
          const int tok = sh.token[c];
          if (tok < 0 || tok >= a.vocab) {
            accepted = -2;  // draft token outside the vocabulary
            break;
          }
          cumulative = cumulative + sg_exp(sh.xchild[c] - m);
          if (threshold < cumulative) {
            accepted = c;
            break;
          }
        }
      }
      if (accepted >= 0 && depth >= a.max_depth) accepted = -2;
      if (accepted == -2) {
        broken = 1;
        break;
      }
      if (accepted < 0) break;
      if (write_nodes && lane == 0) nodes_out[depth] = accepted;
      v = accepted;
      ++depth;
    }
    int count = 0;
    for (int base = v + 1; base < n; base += kWave) {
      const bool is_child = base + lane < n && sh.parent[base + lane] == v;
      const uint64_t mask = __ballot(is_child);
      if (is_child)
        sh.child_tok[count + __popcll(mask & ((1ull << lane) - 1ull))] = sh.token[base + lane];
      count += __popcll(mask);
    }
    if (lane == 0) {
      sh.child_count = count;
      sh.exit_node = v;
      sh.depth = depth;
      sh.broken = broken;
    }
  }
  __syncthreads();
}

// Walk, part 1.  Grid (request, chunk of kWalkWaves slabs); every workgroup
// routes its request (cheap, LDS only), workgroup chunk 0 writes the accepted
// nodes, accept length and keep rows, and every wave computes the complement
// total of one slab of the exit row:
//   e = E(x - m) for non-child tokens below vocab, 0 otherwise; group sums
//   ((e0+e1)+e2)+e3; inclusive Kogge-Stone scan over the 64 lanes of a line;
//   slab total = sequential sum of the line totals.  The line totals are kept
//   too, for part 2.
template <typename S, bool kVec>
__global__ __launch_bounds__(kWalkThreads) void exit_totals_kernel(SgTreeSampleArgs a) {
  __shared__ RouteShared sh;
  const int req = blockIdx.x;
  const int chunk = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int r0 = a.row_offset_dev[req];
  const int n = a.row_offset_dev[req + 1] - r0;
  // A request must own 1 to kMaxTreeRows rows inside the num_rows rows whose
  // statistics were computed; the walk reports any other as a broken contract.
  if (n < 1 || n > kMaxTreeRows || r0 < 0 || r0 > a.num_rows - n) {
    if (chunk == 0 && tid == 0) {
      a.accept_len_dev[req] = -1;
      a.bonus_dev[req] = -1;
      if (a.terminal_leaf_dev) a.terminal_leaf_dev[req] = -1;
      if (a.status_dev) atomicExch(a.status_dev, SG_EINVAL);
    }
    return;
  }
  int32_t* nodes_out = a.accept_nodes_dev + static_cast<int64_t>(a.max_depth) * req;
  if (chunk == 0)
    for (int k = tid; k < a.max_depth; k += blockDim.x) nodes_out[k] = -1;
  __syncthreads();
  route_request<S>(a, req, r0, n, sh, chunk == 0);
  // The walk ended at a node whose row was not projected (a leaf): no exit
  // draw here; the caller projects that leaf and draws its bonus.
  const int exit_row = sh.broken ? -1 : sh.lrow[sh.exit_node];
  if (chunk == 0) {
    if (tid == 0) {
      a.accept_len_dev[req] = sh.broken ? -1 : sh.depth;
      if (a.terminal_leaf_dev)
        a.terminal_leaf_dev[req] = (!sh.broken && exit_row < 0) ? sh.exit_node : -1;
      if (sh.broken) {
        a.bonus_dev[req] = -1;
        if (a.status_dev) atomicExch(a.status_dev, SG_EINVAL);
      }
    }
    if (a.keep_rows_dev) {
      __syncthreads();  // nodes_out written by thread 0
      int32_t* keep = a.keep_rows_dev + static_cast<int64_t>(a.max_depth + 1) * req;
      for (int k = tid; k <= a.max_depth; k += blockDim.x)
        keep[k] = (k == 0) ? 0 : (!sh.broken && k <= sh.depth ? nodes_out[k - 1] : -1);
    }
    const int slabs_all = (a.vocab + kSlab - 1) / kSlab;
    int32_t* rec = reinterpret_cast<int32_t*>(static_cast<float*>(a.workspace_dev) +
                                              static_cast<int64_t>(a.num_requests) * slabs_all *
                                                  (1 + kLinesPerSlab)) +
                   static_cast<int64_t>(req) * kRecordInts;
    if (tid == 0) {
      rec[0] = sh.broken ? -1 : sh.depth;
      rec[1] = sh.exit_node;
      rec[2] = sh.child_count;
      rec[3] = exit_row;
    }
    for (int k = tid; k < sh.child_count; k += blockDim.x) rec[4 + k] = sh.child_tok[k];
  }
  if (sh.broken || exit_row < 0) return;
  const int slabs = (a.vocab + kSlab - 1) / kSlab;
  const int s = chunk * kWalkWaves + wave;
  if (s >= slabs) return;
  const S* __restrict__ x = static_cast<const S*>(a.logits_dev) + a.logits_row_stride * exit_row;
  const float m = sh.rm[sh.exit_node];
  float e[32], incl[kLinesPerSlab], total[kLinesPerSlab];
  exit_values<S, kVec>(x, a.vocab, m, s, lane, child_bits(sh.child_tok, sh.child_count, s, lane),
                     e);
  line_scans(e, lane, incl, total);
  float lp = 0.0f;
#pragma unroll
  for (int j = 0; j < kLinesPerSlab; ++j) lp = lp + total[j];
  if (lane == 0) {
    float* ws = static_cast<float*>(a.workspace_dev);
    ws[static_cast<int64_t>(req) * slabs + s] = lp;
    float* lines = ws + static_cast<int64_t>(a.num_requests) * slabs +
                   (static_cast<int64_t>(req) * slabs + s) * kLinesPerSlab;
#pragma unroll
    for (int j = 0; j < kLinesPerSlab; ++j) lines[j] = total[j];
  }
}

// Walk, part 2 (one wave per request): slab prefixes P_s (sequential),
// C = P_slabs, threshold u[2d+1] * C; the bonus is the first non-child token
// whose running value (P_s + line prefix + lane prefix + its group's
// elements) exceeds the threshold; fallback: the largest non-child token.
// The line prefix is the sequential sum of the slab's earlier line totals,
// which part 1 stored.  A line whose P_s + line prefix + line total lies below
// threshold - 1e-4 * C cannot hold that token (its running values differ from
// that sum by a few roundings), so only the lines from the first one that may
// are recomputed, one 256-token line at a time.
template <typename S, bool kVec>
__global__ __launch_bounds__(kWave) void exit_find_kernel(SgTreeSampleArgs a) {
  __shared__ int s_child_tok[kMaxTreeRows];
  __shared__ float s_total[kMaxSlabs];
  const int req = blockIdx.x;
  const int lane = threadIdx.x;
  const int slabs = (a.vocab + kSlab - 1) / kSlab;
  const float* __restrict__ totals =
      static_cast<const float*>(a.workspace_dev) + static_cast<int64_t>(req) * slabs;
  const float* __restrict__ line_totals = static_cast<const float*>(a.workspace_dev) +
                                          static_cast<int64_t>(a.num_requests) * slabs +
                                          static_cast<int64_t>(req) * slabs * kLinesPerSlab;
  const int32_t* rec = reinterpret_cast<const int32_t*>(
                           static_cast<const float*>(a.workspace_dev) +
                           static_cast<int64_t>(a.num_requests) * slabs * (1 + kLinesPerSlab)) +
                       static_cast<int64_t>(req) * kRecordInts;
  const float* __restrict__ u = a.uniforms_dev + static_cast<int64_t>(a.uniform_stride) * req;
  // One round trip: the row range, part 1's record (accept length, child
  // count, exit row), the first 64 child tokens and the slab totals.
  const int r0 = a.row_offset_dev[req];
  const int n = a.row_offset_dev[req + 1] - r0;
  const int depth = rec[0];
  const int count = rec[2];
  const int tok0 = rec[4 + lane];
  float tot[(kMaxSlabs + kWave - 1) / kWave];
#pragma unroll
  for (int q = 0; q < (kMaxSlabs + kWave - 1) / kWave; ++q)
    tot[q] = q * kWave + lane < slabs ? totals[q * kWave + lane] : 0.0f;
  // The record exists only for a valid tree; part 1 reported the others.
  if (n < 1 || n > kMaxTreeRows || r0 < 0 || r0 > a.num_rows - n) return;
  if (depth < 0) return;  // broken walk, reported by part 1
  const int exit_row = rec[3];
  if (exit_row < 0) {      // terminal leaf without a projected row
    if (lane == 0) a.bonus_dev[req] = -1;
    return;
  }
  if (lane < count) s_child_tok[lane] = tok0;
  for (int k = kWave + lane; k < count; k += kWave) s_child_tok[k] = rec[4 + k];
#pragma unroll
  for (int q = 0; q < (kMaxSlabs + kWave - 1) / kWave; ++q)
    if (q * kWave + lane < slabs) s_total[q * kWave + lane] = tot[q];
  // The exit draw's uniform and the exit row's max, in flight during the
  // sums below.
  const float u_exit = u[2 * depth + 1];
  const int64_t row = exit_row;
  const float m = a.row_max_dev[row];
  __builtin_amdgcn_wave_barrier();
  // C and the threshold (every lane runs the same sequential sums).
  float prefix = 0.0f;
  {
    int k = 0;
    for (; k + 8 <= slabs; k += 8) {
      float t[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = s_total[k + e];
#pragma unroll
      for (int e = 0; e < 8; ++e) prefix = prefix + t[e];
    }
    for (; k < slabs; ++k) prefix = prefix + s_total[k];
  }
  const float threshold = u_exit * prefix;
  const float bound = threshold - 1e-4f * prefix;
  // First line that may hold the bonus: slab s, line j, base = P_s + lp_j.
  int s = 0;
  float slab_prefix = 0.0f;
  {
    bool found = false;
    while (!found && s < slabs) {
      float t[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = s + e < slabs ? s_total[s + e] : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (found || s >= slabs) continue;
        if (slab_prefix + t[e] > bound) {
          found = true;
        } else {
          slab_prefix = slab_prefix + t[e];
          ++s;
        }
      }
    }
  }
  int j = 0;
  float lp = 0.0f;
  if (s < slabs) {
    // The slab's line totals in one round trip, then the same sequential scan.
    const float* lt = line_totals + static_cast<int64_t>(s) * kLinesPerSlab;
    float ltv[kLinesPerSlab];
#pragma unroll
    for (int e = 0; e < kLinesPerSlab; ++e) ltv[e] = lt[e];
#pragma unroll
    for (int e = 0; e < kLinesPerSlab - 1; ++e) {
      if (j == e && !((slab_prefix + lp) + ltv[e] > bound)) {
        lp = lp + ltv[e];
        j = e + 1;
      }
    }
  }
  const S* __restrict__ x = static_cast<const S*>(a.logits_dev) + a.logits_row_stride * row;
  int candidate = INT_MAX;
  while (s < slabs && candidate == INT_MAX) {
    // Line j of slab s: lane l holds tokens 2048*s + 256*j + 4*l + c.
    const int t0 = s * kSlab + kLine * j + 4 * lane;
    float e[4];
    if (kVec && t0 + 3 < a.vocab) {
      load4<S, false>(x + t0, e);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        e[c] = (t0 + c < a.vocab) ? to_f32(x[t0 + c]) : -__builtin_inff();
    }
    const uint32_t bits = child_bits(s_child_tok, count, s, lane) >> (4 * j);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float val = sg_exp_nonpos(e[c] - m);
      e[c] = ((bits >> c) & 1u) ? 0.0f : val;
    }
    // The same group sums and inclusive Kogge-Stone scan as part 1.
    float g = ((e[0] + e[1]) + e[2]) + e[3];
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const float up = __shfl_up(g, d);
      g = (lane >= d) ? g + up : g;
    }
    const float up = __shfl_up(g, 1);
    const float excl = (lane > 0) ? up : 0.0f;
    float run = (slab_prefix + lp) + excl;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      run = run + e[c];
      const bool hit = t0 + c < a.vocab && !((bits >> c) & 1u) && run > threshold;
      candidate = (hit && candidate == INT_MAX) ? t0 + c : candidate;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) candidate = min(candidate, __shfl_xor(candidate, d));
    // Next line: line prefixes restart at each slab.
    lp = lp + __shfl(g, kWave - 1);
    if (++j == kLinesPerSlab) {
      slab_prefix = slab_prefix + s_total[s];
      lp = 0.0f;
      j = 0;
      ++s;
    }
  }
  if (lane == 0) {
    int bonus = candidate;
    if (bonus == INT_MAX) {
      bonus = -1;
      for (int t = a.vocab - 1; t >= 0; --t) {
        bool child = false;
        for (int k = 0; k < count; ++k) child = child || s_child_tok[k] == t;
        if (!child) {
          bonus = t;
          break;
        }
      }
    }
    a.bonus_dev[req] = bonus;
  }
}

// Sum of E(x - m) over one slab in the statistics pass's order (lane
// partials over the lines, (a0+a1)+(a2+a3), butterfly), leaving out the
// child tokens of `bits` (bit 4j+c: token 2048s + 256j + 4*lane + c).
__device__ __forceinline__ float slab_sum_skip(const float v[32], float m, uint32_t bits) {
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  if (m != -__builtin_inff()) {
#pragma unroll
    for (int j = 0; j < kLinesPerSlab; ++j) {
      const float e0 = sg_exp_nonpos(v[4 * j + 0] - m);
      const float e1 = sg_exp_nonpos(v[4 * j + 1] - m);
      const float e2 = sg_exp_nonpos(v[4 * j + 2] - m);
      const float e3 = sg_exp_nonpos(v[4 * j + 3] - m);
      a0 = ((bits >> (4 * j + 0)) & 1u) ? a0 : a0 + e0;
      a1 = ((bits >> (4 * j + 1)) & 1u) ? a1 : a1 + e1;
      a2 = ((bits >> (4 * j + 2)) & 1u) ? a2 : a2 + e2;
      a3 = ((bits >> (4 * j + 3)) & 1u) ? a3 : a3 + e3;
    }
  }
  return wave_butterfly_sum((a0 + a1) + (a2 + a3));
}

// The walk with the slab draw, when the statistics pass of this call kept
// every row's slab pairs (no SG_SAMPLE_STATS_READY).  One workgroup per
// request: route (route_request), then from the exit row's slab pairs:
//   1. the slabs that hold a child token of the exit node are summed again
//      without those tokens (one wave per slab, the pass's order);
//   2. per slab w_s = Z'_s * E(m_s - M), then the sequential prefixes P_s
//      and C;
//   3. the first slab with P_s + w_s > u*C, and in it the first non-child
//      token whose running value (per line group sums, inclusive Kogge-Stone
//      scan over the 64 lanes, sequential line prefixes) exceeds u*C -- else
//      the slab's last non-child token with e > 0; no slab: the largest
//      non-child token.
// Four dependent memory round trips: the tree, the statistics and child
// logits, the exit row's slab pairs and child slabs, the crossing slab.
template <typename S, bool kVec>
__global__ __launch_bounds__(kWalkThreads) void slab_walk_kernel(
    SgTreeSampleArgs a, const float* __restrict__ slab_stats) {
  __shared__ RouteShared sh;
  __shared__ float s_m[kMaxSlabs];
  __shared__ float s_z[kMaxSlabs];   // Z_s, then Z'_s in place
  __shared__ float s_w[kMaxSlabs];
  __shared__ float s_es[kMaxSlabs];
  __shared__ float s_p[kMaxSlabs];
  __shared__ unsigned char s_child_slab[kMaxSlabs];
  __shared__ float s_thr;
  const int req = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int r0 = a.row_offset_dev[req];
  const int n = a.row_offset_dev[req + 1] - r0;
  if (n < 1 || n > kMaxTreeRows || r0 < 0 || r0 > a.num_rows - n) {
    if (tid == 0) {
      a.accept_len_dev[req] = -1;
      a.bonus_dev[req] = -1;
      if (a.terminal_leaf_dev) a.terminal_leaf_dev[req] = -1;
      if (a.status_dev) atomicExch(a.status_dev, SG_EINVAL);
    }
    return;
  }
  int32_t* nodes_out = a.accept_nodes_dev + static_cast<int64_t>(a.max_depth) * req;
  for (int k = tid; k < a.max_depth; k += blockDim.x) nodes_out[k] = -1;
  __syncthreads();
  route_request<S>(a, req, r0, n, sh, true);
  const int exit_row = sh.broken ? -1 : sh.lrow[sh.exit_node];
  if (tid == 0) {
    a.accept_len_dev[req] = sh.broken ? -1 : sh.depth;
    if (a.terminal_leaf_dev)
      a.terminal_leaf_dev[req] = (!sh.broken && exit_row < 0) ? sh.exit_node : -1;
    if (sh.broken || exit_row < 0) a.bonus_dev[req] = -1;
    if (sh.broken && a.status_dev) atomicExch(a.status_dev, SG_EINVAL);
  }
  if (a.keep_rows_dev) {
    __syncthreads();  // nodes_out written by thread 0
    int32_t* keep = a.keep_rows_dev + static_cast<int64_t>(a.max_depth + 1) * req;
    for (int k = tid; k <= a.max_depth; k += blockDim.x)
      keep[k] = (k == 0) ? 0 : (!sh.broken && k <= sh.depth ? nodes_out[k - 1] : -1);
  }
  if (sh.broken || exit_row < 0) return;
  const int slabs = (a.vocab + kSlab - 1) / kSlab;
  const float* __restrict__ src = slab_stats + static_cast<int64_t>(exit_row) * slabs * kSlabStats;
  for (int k = tid; k < slabs; k += blockDim.x) {
    s_m[k] = src[kSlabStats * k];
    s_z[k] = src[kSlabStats * k + 1];
    s_child_slab[k] = 0;
  }
  __syncthreads();
  for (int k = tid; k < sh.child_count; k += blockDim.x) {
    const int t = sh.child_tok[k];
    if (t >= 0 && t < a.vocab) s_child_slab[t / kSlab] = 1;
  }
  __syncthreads();
  const S* __restrict__ x = static_cast<const S*>(a.logits_dev) + a.logits_row_stride * exit_row;
  // 1. complement sums of the slabs with child tokens
  for (int s = wave; s < slabs; s += kWalkWaves) {
    if (!s_child_slab[s]) continue;
    float v[32];
    load_slab<S, kVec>(x, a.vocab, s, lane, v);
    const float z = slab_sum_skip(v, s_m[s], child_bits(sh.child_tok, sh.child_count, s, lane));
    if (lane == 0) s_z[s] = z;
  }
  __syncthreads();
  // 2. per-slab weights, then the sequential prefixes and the threshold
  const float m_row = sh.rm[sh.exit_node];
  for (int s = tid; s < slabs; s += blockDim.x) {
    const float es = sg_exp_nonpos(s_m[s] - m_row);
    s_es[s] = es;
    s_w[s] = s_z[s] * es;
  }
  __syncthreads();
  if (tid == 0) {
    float p = 0.0f;
    for (int s = 0; s < slabs; ++s) {
      s_p[s] = p;
      p = p + s_w[s];
    }
    s_thr = sh.u[2 * sh.depth + 1] * p;
  }
  __syncthreads();
  if (wave != 0) return;
  // 3. the crossing slab and token (every lane of wave 0 alike)
  const float thr = s_thr;
  int hit = -1;
  for (int base = 0; base < slabs && hit < 0; base += kWave) {
    const int s = base + lane;
    const uint64_t mask = __ballot(s < slabs && s_p[s] + s_w[s] > thr);
    if (mask != 0) hit = base + __builtin_ctzll(mask);
  }
  int bonus = -1;
  if (hit >= 0) {
    const float p = s_p[hit];
    const float es = s_es[hit];
    const float ms = s_m[hit];
    float v[32];
    load_slab<S, kVec>(x, a.vocab, hit, lane, v);
    const uint32_t bits = child_bits(sh.child_tok, sh.child_count, hit, lane);
    float q = 0.0f;
    int candidate = INT_MAX;
    int last = -1;
#pragma unroll
    for (int j = 0; j < kLinesPerSlab; ++j) {
      const int t0 = hit * kSlab + kLine * j + 4 * lane;
      float e[4];
      bool nonchild[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        nonchild[c] = t0 + c < a.vocab && !((bits >> (4 * j + c)) & 1u);
        e[c] = nonchild[c] ? sg_exp_nonpos(v[4 * j + c] - ms) : 0.0f;
      }
      float g = ((e[0] + e[1]) + e[2]) + e[3];
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const float up = __shfl_up(g, d);
        g = (lane >= d) ? g + up : g;
      }
      const float up = __shfl_up(g, 1);
      float r = q + ((lane > 0) ? up : 0.0f);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        r = r + e[c];
        if (nonchild[c] && candidate == INT_MAX && p + es * r > thr) candidate = t0 + c;
        if (nonchild[c] && e[c] > 0.0f) last = t0 + c;
      }
      q = q + __shfl(g, kWave - 1);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      candidate = min(candidate, __shfl_xor(candidate, d));
      last = max(last, __shfl_xor(last, d));
    }
    bonus = candidate != INT_MAX ? candidate : last;
  } else {
    // No slab crosses: the largest non-child token (every lane alike).
    for (int t = a.vocab - 1; t >= 0; --t) {
      bool child = false;
      for (int k = 0; k < sh.child_count; ++k) child = child || sh.child_tok[k] == t;
      if (!child) {
        bonus = t;
        break;
      }
    }
  }
  if (lane == 0) a.bonus_dev[req] = bonus;
}

__global__ void exp_probe_kernel(const float* __restrict__ x, float* __restrict__ out,
                                 int64_t count) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k < count) out[k] = sg_exp(x[k]);
}

size_t elem_bytes(int dtype) { return dtype == SG_DTYPE_F32 ? 4 : 2; }

// Whole 4-element groups (16 bytes of fp32, 8 bytes of bf16/f16) are aligned.
bool vec_ok(const void* p, int dtype, int64_t stride, int vocab) {
  return (reinterpret_cast<uintptr_t>(p) % (4 * elem_bytes(dtype)) == 0) && stride % 4 == 0 &&
         vocab % 4 == 0;
}

// Calls f(S{}, BoolTag) with the element type and vector flag of the logits.
template <typename F>
void dispatch_logits(const void* p, int dtype, int64_t stride, int vocab, F&& f) {
  const bool vec = vec_ok(p, dtype, stride, vocab);
  if (dtype == SG_DTYPE_BF16) {
    vec ? f(Bf16{}, std::true_type{}) : f(Bf16{}, std::false_type{});
  } else if (dtype == SG_DTYPE_F16) {
    vec ? f(F16{}, std::true_type{}) : f(F16{}, std::false_type{});
  } else {
    vec ? f(float{}, std::true_type{}) : f(float{}, std::false_type{});
  }
}

int launch_row_stats(const void* logits, int dtype, int64_t stride, int vocab, int rows,
                     float* row_max, float* row_sum, float* slab_out, int32_t* status,
                     hipStream_t stream) {
  if (rows == 0 && status == nullptr) return SG_OK;
  // One workgroup per row (one to clear the status when there are no rows).
  const dim3 grid(rows > 0 ? rows : 1);
  dispatch_logits(logits, dtype, stride, vocab, [&](auto elem, auto vec) {
    using S = decltype(elem);
    hipLaunchKernelGGL((row_stats_kernel<S, decltype(vec)::value>), grid, dim3(kStatsThreads),
                       0, stream, static_cast<const S*>(logits), stride, vocab, rows, row_max,
                       row_sum, slab_out, status);
  });
  SG_LAUNCH_CHECK();
  return SG_OK;
}

}  // namespace
}  // namespace sg

extern "C" int sg_row_stats(const void* logits_dev, int32_t logits_dtype, int64_t row_stride,
                            int32_t vocab, int32_t num_rows, float* row_max_dev,
                            float* row_sum_dev, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(logits_dtype == SG_DTYPE_F32 || logits_dtype == SG_DTYPE_BF16 ||
                 logits_dtype == SG_DTYPE_F16,
             "logits_dtype must be SG_DTYPE_F32, SG_DTYPE_BF16 or SG_DTYPE_F16");
  SG_REQUIRE(vocab >= 1 && vocab <= kMaxSlabs * kSlab, "vocab must be in [1, 524288]");
  SG_REQUIRE(num_rows >= 0, "num_rows must be non-negative");
  SG_REQUIRE(row_stride >= vocab, "logits row stride is below the vocabulary");
  SG_REQUIRE(num_rows == 0 || (logits_dev && row_max_dev && row_sum_dev),
             "null device pointer");
  return launch_row_stats(logits_dev, logits_dtype, row_stride, vocab, num_rows, row_max_dev,
                          row_sum_dev, nullptr, nullptr, reinterpret_cast<hipStream_t>(stream));
}

namespace sg {
namespace {

// Workspace layout: per request the complement draw's slab and line totals
// and the record its two kernels pass on (SG_SAMPLE_STATS_READY calls), then
// per statistics row its slab pairs (calls that compute statistics).
int64_t request_region_floats(int num_requests, int vocab) {
  return static_cast<int64_t>(num_requests) *
         (((vocab + kSlab - 1) / kSlab) * (1 + kLinesPerSlab) + kRecordInts);
}

}  // namespace
}  // namespace sg

extern "C" int64_t sg_tree_sample_workspace_bytes(int32_t num_requests, int32_t num_rows,
                                                  int32_t vocab) {
  using namespace sg;
  if (num_requests < 0 || num_rows < 0 || vocab < 1) return 0;
  return (request_region_floats(num_requests, vocab) +
          static_cast<int64_t>(num_rows) * ((vocab + kSlab - 1) / kSlab) * kSlabStats) *
         static_cast<int64_t>(sizeof(float));
}

namespace sg {
namespace {

// Checks every argument of sg_tree_sample except the workspace.
int check_sample_args(const SgTreeSampleArgs* args) {
  SG_REQUIRE(args != nullptr, "null SgTreeSampleArgs");
  const SgTreeSampleArgs& a = *args;
  SG_REQUIRE(a.num_requests >= 0 && a.num_rows >= 0, "negative sizes");
  SG_REQUIRE(a.logits_dtype == SG_DTYPE_F32 || a.logits_dtype == SG_DTYPE_BF16 ||
                 a.logits_dtype == SG_DTYPE_F16,
             "logits_dtype must be SG_DTYPE_F32, SG_DTYPE_BF16 or SG_DTYPE_F16");
  SG_REQUIRE(a.vocab >= 1 && a.vocab <= kMaxSlabs * kSlab, "vocab must be in [1, 524288]");
  SG_REQUIRE(a.logits_row_stride >= a.vocab, "logits row stride is below the vocabulary");
  SG_REQUIRE(a.max_depth >= 0, "max_depth must be non-negative");
  SG_REQUIRE(a.uniform_stride >= 2 * (a.max_depth + 1),
             "uniform_stride must cover 2*(max_depth+1) uniforms");
  SG_REQUIRE((a.flags & ~SG_SAMPLE_STATS_READY) == 0, "unknown sampler flags");
  SG_REQUIRE(a.num_logits_rows >= 0, "negative num_logits_rows");
  SG_REQUIRE(a.logits_row_dev != nullptr || a.num_logits_rows == 0 ||
                 a.num_logits_rows == a.num_rows,
             "without a logits row map the logits rows are the packed rows");
  SG_REQUIRE(a.logits_row_dev == nullptr || a.terminal_leaf_dev != nullptr,
             "a logits row map needs terminal_leaf_dev for walks that end at an unprojected leaf");
  if (a.num_requests == 0) return SG_OK;
  SG_REQUIRE(a.logits_dev && a.row_offset_dev && a.parent_dev && a.token_dev &&
                 a.uniforms_dev && a.row_max_dev && a.row_sum_dev && a.accept_len_dev &&
                 a.bonus_dev && (a.max_depth == 0 || a.accept_nodes_dev),
             "null device pointer");
  return SG_OK;
}

// Enqueues the three kernels of one sampling call; a.workspace_dev holds at
// least sg_tree_sample_workspace_bytes(num_requests, statistics rows, vocab) bytes.
int64_t stats_rows_of(const SgTreeSampleArgs& a) {
  return (a.flags & SG_SAMPLE_STATS_READY) ? 0
         : (a.num_logits_rows > 0 ? a.num_logits_rows : a.num_rows);
}

int launch_tree_sample(const SgTreeSampleArgs& a, hipStream_t s) {
  // With SG_SAMPLE_STATS_READY the statistics pass only clears the status and
  // the complement draw runs (exit_totals + exit_find); otherwise the pass
  // keeps every row's slab pairs and one kernel walks and draws.
  const bool ready = (a.flags & SG_SAMPLE_STATS_READY) != 0;
  const int stats_rows = static_cast<int>(stats_rows_of(a));
  float* slab_stats = static_cast<float*>(a.workspace_dev) +
                      request_region_floats(a.num_requests, a.vocab);
  int rc = launch_row_stats(a.logits_dev, a.logits_dtype, a.logits_row_stride, a.vocab,
                            stats_rows, a.row_max_dev, a.row_sum_dev,
                            ready ? nullptr : slab_stats, a.status_dev, s);
  if (rc != SG_OK) return rc;
  const int slabs = (a.vocab + kSlab - 1) / kSlab;
  const dim3 grid1(a.num_requests, (slabs + kWalkWaves - 1) / kWalkWaves);
  hipError_t err = hipSuccess;
  dispatch_logits(a.logits_dev, a.logits_dtype, a.logits_row_stride, a.vocab,
                  [&](auto elem, auto vec) {
                    using S = decltype(elem);
                    constexpr bool kVec = decltype(vec)::value;
                    if (!ready) {
                      hipLaunchKernelGGL((slab_walk_kernel<S, kVec>), dim3(a.num_requests),
                                         dim3(kWalkThreads), 0, s, a,
                                         static_cast<const float*>(slab_stats));
                      return;
                    }
                    hipLaunchKernelGGL((exit_totals_kernel<S, kVec>), grid1, dim3(kWalkThreads),
                                       0, s, a);
                    err = hipGetLastError();
                    if (err != hipSuccess) return;
                    hipLaunchKernelGGL((exit_find_kernel<S, kVec>), dim3(a.num_requests),
                                       dim3(kWave), 0, s, a);
                  });
  SG_HIP_CHECK(err);
  SG_LAUNCH_CHECK();
  return SG_OK;
}

}  // namespace
}  // namespace sg

extern "C" int sg_tree_sample(const SgTreeSampleArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  int rc = check_sample_args(args);
  if (rc != SG_OK || args->num_requests == 0) return rc;
  const SgTreeSampleArgs& a = *args;
  SG_REQUIRE(a.workspace_dev != nullptr &&
                 static_cast<int64_t>(a.workspace_bytes) >=
                     sg_tree_sample_workspace_bytes(a.num_requests,
                                                    static_cast<int32_t>(stats_rows_of(a)),
                                                    a.vocab),
             "workspace below sg_tree_sample_workspace_bytes");
  return launch_tree_sample(a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int sg_exp_probe(const float* x_dev, float* out_dev, int64_t count,
                            sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(count >= 0, "negative count");
  if (count == 0) return SG_OK;
  SG_REQUIRE(x_dev && out_dev, "null device pointer");
  const int threads = 256;
  const dim3 grid(static_cast<unsigned>((count + threads - 1) / threads));
  hipLaunchKernelGGL(exp_probe_kernel, grid, dim3(threads), 0,
                     reinterpret_cast<hipStream_t>(stream), x_dev, out_dev, count);
  SG_LAUNCH_CHECK();
  return SG_OK;
}

// ---------------------------------------------------------------------------
// sg_tree_sample_noalloc: sg_tree_sample with its workspace in a static device
// array, for callers that cannot allocate device memory.  Each GPU holds its
// own copy of `scratch` (kNoAllocScratchBytes) until the process ends; its
// device address is looked up once per device with hipGetSymbolAddress and
// only that address is handed to the kernels (the array's name is a host-side
// stand-in).  Every value the kernels read from it is written earlier in the
// same call, so it needs no clearing; calls that overlap on one GPU race on it.
// ---------------------------------------------------------------------------
#include <mutex>

static __device__ __align__(256) unsigned char scratch[SG_TREE_SAMPLE_NOALLOC_SCRATCH_BYTES];

namespace sg {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`.
int current_scratch(void** out) {
  int dev = -1;
  SG_HIP_CHECK(hipGetDevice(&dev));
  SG_REQUIRE(dev >= 0 && dev < kMaxDevices, "device index outside the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_dev[dev] == nullptr) {
    void* ptr = nullptr;
    SG_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    SG_REQUIRE(ptr != nullptr, "hipGetSymbolAddress returned no address for the scratch");
    g_scratch_dev[dev] = ptr;
  }
  *out = g_scratch_dev[dev];
  return SG_OK;
}

}  // namespace
}  // namespace sg

extern "C" int sg_tree_sample_noalloc(const SgTreeSampleArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  int rc = check_sample_args(args);
  if (rc != SG_OK || args->num_requests == 0) return rc;
  SG_REQUIRE(args->workspace_dev == nullptr && args->workspace_bytes == 0,
             "sg_tree_sample_noalloc uses its own scratch: workspace_dev must be NULL "
             "and workspace_bytes 0");
  const int64_t need = sg_tree_sample_workspace_bytes(
      args->num_requests, static_cast<int32_t>(stats_rows_of(*args)), args->vocab);
  if (need > static_cast<int64_t>(SG_TREE_SAMPLE_NOALLOC_SCRATCH_BYTES))
    return set_error(SG_EINVAL,
                     "sg_tree_sample_noalloc: " + std::to_string(args->num_requests) +
                         " requests over vocab " + std::to_string(args->vocab) + " need " +
                         std::to_string(need) + " scratch bytes, above the static maximum of " +
                         std::to_string(SG_TREE_SAMPLE_NOALLOC_SCRATCH_BYTES));
  void* ws = nullptr;
  rc = current_scratch(&ws);
  if (rc != SG_OK) return rc;
  SgTreeSampleArgs a = *args;
  a.workspace_dev = ws;
  a.workspace_bytes = SG_TREE_SAMPLE_NOALLOC_SCRATCH_BYTES;
  return launch_tree_sample(a, reinterpret_cast<hipStream_t>(stream));
}
