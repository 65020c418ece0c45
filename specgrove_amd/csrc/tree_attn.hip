// Request-isolated, tree-ancestor-masked GQA attention over a packed wave.
//
// Semantics: row k of request i (packed row row_offset[i]+k) attends, for each
// query head h with kv head g = h / (Hq/Hkv), to
//   * every key of request i's cached prefix (L_i tokens), and
//   * the request's own tree rows j that are ancestors of k or k itself,
// with softmax(q.k * scale) weights.  This is the visible set of the
// reference's dense packed mask (continuous_tree_block_decode.py:500-546 and
// tree.py:19-26) evaluated without materialising the mask or copying prefixes.
//
// Decomposition (MI355X, two 4-wave workgroups per CU):
//   unit      = (request, kv head, tile of up to 128/G query rows = 128 query
//               vectors = four 32-vector q-groups, range of prefix keys); the
//               unit that ends a request's key range also covers its tree rows;
//   work list = the units one workgroup runs in order; by default one unit,
//               largest first, so that the hardware dispatcher balances the
//               end of the launch;
//   window    = one barrier; consumes two 32-key K and V tiles, moved
//               HBM -> LDS by global_load_lds_dwordx4 (no register staging)
//               into 4-tile rings issued one window ahead;
//   wave      = one q-group over both tiles of every window (3-4 q-groups)
//               or one of two key streams of a q-group taking one tile of
//               each window (1-2 q-groups).  Every wave runs its own online
//               softmax; the key streams of a q-group are merged through LDS
//               at the end of the unit.
// Per 32-key block a wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16
// (A = K rows from LDS stored in the permuted order pi, so the result gives
// each lane 16 consecutive keys; B = Q in registers) and O^T += V^T P^T with
// the same MFMA (A = V read transposed from row-major LDS by ds_read_b64_tr_b16,
// B = P in registers).  LDS rows are unpadded; the 16-byte chunk c of row r is
// stored at chunk c ^ swz(r) so that both read patterns are bank-conflict free.
// Split key ranges (units far above a mean list, or waves with fewer units
// than lists) leave unnormalised partials that a second kernel combines.
#include <algorithm>
#include <climits>
#include <cstring>
#include <numeric>
#include <queue>
#include <type_traits>
#include <vector>

#include "sg_common.h"

namespace sg {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float floatx16;
typedef __attribute__((ext_vector_type(4))) short short4_t;
typedef __attribute__((ext_vector_type(8))) short short8_t;
typedef __attribute__((address_space(3))) short4_t lds_short4;

constexpr int kThreads = 256;
constexpr int kQPerUnit = 128;
constexpr int kTileKeys = 32;                   // keys per tile: one 32-key MFMA block
constexpr int kListsPerCU = 2;                  // resident workgroups per CU
constexpr int kStages = 4;
constexpr int kWaves = 4;
constexpr int kMaxTreeRows = 256;
constexpr int kAncWords = kMaxTreeRows / 32;
constexpr int kMergeThreads = 256;
constexpr int32_t kPlanMagic = 0x53475041;  // "SGPA"
constexpr int kMaxGroup = 16;               // query heads per kv head
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyLog2 = 8.0f;  // softmax reference point moves after a 2^8 growth
constexpr int kDefaultCUs = 256;
constexpr int64_t kSplitAbovePercent = 150;  // planner: split units above 1.5x a slot's share
constexpr int64_t kRowSplitAbovePercent = 150;  // planner: units split by rows instead

struct PlanHeader {
  int32_t magic;
  int32_t num_units;
  int32_t num_merges;
  int32_t rows_per_tile;
  int32_t head_dim;
  int32_t group;
  int32_t num_partials;
  int32_t num_bins;       // work lists = workgroups of the attention kernel
  int32_t num_requests;   // n and R = row_offset[n] of the wave the plan was built for
  int32_t num_rows;
  int32_t num_kv_heads;
  int32_t reserved0;
  uint64_t meta_hash;     // FNV-1a over row_offset[0..n] and prefix_len[0..n-1]
  int32_t reserved[2];
};
static_assert(sizeof(PlanHeader) == 64, "plan header is 64 bytes");

struct AttnUnit {
  int32_t req;
  int32_t kv_head;
  int32_t row_begin;
  int32_t row_count;
  int32_t key_begin;
  int32_t key_end;
  int32_t partial;        // partial slot of this unit, -1 when unsplit
  int32_t flags;          // bit 0: attend to the request's tree rows; bit 1: rows
                          // split, K/V shared with sibling units (no nt hint)
  int32_t group;          // split group (merge record index), -1 when unsplit
  int32_t num_splits;     // units in the group
  int32_t first_partial;  // partial slot of the group's first unit
  int32_t pad;
};
static_assert(sizeof(AttnUnit) == 48, "unit record is 48 bytes");

struct MergeGroup {
  int32_t req;
  int32_t kv_head;
  int32_t row_begin;
  int32_t row_count;
  int32_t first_partial;
  int32_t num_partials;
  int32_t pad0;
  int32_t pad1;
};

// 64-bit FNV-1a of the wave's row offsets and prefix lengths (host only).
uint64_t meta_hash(int n, const int32_t* row_offset, const int32_t* prefix_len) {
  uint64_t h = 1469598103934665603ull;
  auto mix = [&](int32_t v) {
    const uint32_t u = static_cast<uint32_t>(v);
    for (int b = 0; b < 4; ++b) {
      h ^= (u >> (8 * b)) & 0xffu;
      h *= 1099511628211ull;
    }
  };
  mix(n);
  for (int i = 0; i <= n; ++i) mix(row_offset[i]);
  for (int i = 0; i < n; ++i) mix(prefix_len[i]);
  return h;
}

__host__ __device__ constexpr size_t partial_floats(int head_dim) {
  return static_cast<size_t>(kQPerUnit) * (head_dim + 2);
}

__host__ __device__ constexpr int merge_blocks_per_group(int head_dim) {
  return (head_dim / 4) * kQPerUnit / kMergeThreads;
}

// LDS row of key k inside its 32-key block (inverse of pi).
__device__ __forceinline__ int key_slot(int k) {
  return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3);
}

// Key held by LDS row i of a 32-key K block (pi).
__device__ __forceinline__ int key_pi(int i) {
  return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3);
}

// XOR swizzles of the 16-byte chunks of LDS row r, chosen by exhaustive check
// of every read pattern of this kernel against both 32- and 64-bank LDS:
//   K rows (ds_read_b128, 16 consecutive rows at one chunk): r & 15 (D=128),
//     r & 7 (D=64, 8 chunks per row);
//   V rows (ds_read_b64_tr_b16, 4 consecutive rows at 2-4 adjacent chunks):
//     4*(r&3) + 2*((r>>1)&1) (D=128), 2*(r&3) (D=64).
template <int D>
__host__ __device__ constexpr int swz_k(int r) {
  return D == 128 ? (r & 15) : (r & 7);
}
template <int D>
__host__ __device__ constexpr int swz_v(int r) {
  return D == 128 ? 4 * (r & 3) + 2 * ((r >> 1) & 1) : 2 * (r & 3);
}

// 16-byte HBM -> LDS DMA of every lane: lane i's bytes at gbase + voff land at
// LDS byte lds + 16*i.  When a (request, kv head)'s K/V is read by one unit
// only, the loads carry the non-temporal hint (nt) and do not displace
// reusable lines in the caches (measured 3-7 % faster on the Qwen3-8B wave);
// the row tiles of a larger tree re-read the same K/V and keep it cached.  Issued as inline assembly so that the compiler does not
// model it: its automatic waits would otherwise stall the first LDS read of the
// other pipeline stage on this in-flight copy.  The kernel waits for the DMAs
// explicitly (s_waitcnt vmcnt(0)) before the barrier that publishes the tile.
// m0 (the LDS base of the copy) is written here and declared clobbered.
template <bool kStream>
__device__ __forceinline__ void dma16(const void* gbase, uint32_t voff, uint32_t lds) {
  if constexpr (kStream) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                 :
                 : "s"(lds), "v"(voff), "s"(gbase)
                 : "memory", "m0");
  } else {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(gbase)
                 : "memory", "m0");
  }
}
// Run-time choice for the unit's rare issue paths (prologue, partial and tree tiles).
__device__ __forceinline__ void dma16(const void* gbase, uint32_t voff, uint32_t lds,
                                      bool stream) {
  if (stream) {
    dma16<true>(gbase, voff, lds);
  } else {
    dma16<false>(gbase, voff, lds);
  }
}

// s_waitcnt immediate that waits for vmcnt <= n and leaves the other counters
// unconstrained (gfx9 layout: vmcnt bits [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8]).
constexpr int vmcnt_encoding(int n) {
  return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// max / sum of a value with the same lane of the other 32-lane half.
__device__ __forceinline__ float half_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

template <int N>
using IntTag = std::integral_constant<int, N>;
template <bool B>
using BoolTag = std::integral_constant<bool, B>;

// Per-wave attention state: one query column per lane pair.
template <int D>
struct WaveState {
  float m;  // running max of raw scores
  float l;  // running sum of exp2((s - m) * c2)
  floatx16 acc[D / 32];
};

// The unit's request, kv head and partial slot exist in this call (checked
// before any of them indexes memory).
template <int D>
__device__ __forceinline__ bool unit_indices_valid(const SgTreeAttnArgs& a, const AttnUnit& u) {
  return u.req >= 0 && u.req < a.num_requests && u.kv_head >= 0 &&
         u.kv_head < a.num_kv_heads &&
         (u.partial < 0 ||
          static_cast<size_t>(u.partial) < a.workspace_bytes / (sizeof(float) * partial_floats(D)));
}

// The unit's rows and key range lie inside request req's rows and cached
// prefix as the metadata of this call gives them, and the unit that covers
// the tree rows ends the key range exactly at the prefix length.
__device__ __forceinline__ bool unit_matches(const SgTreeAttnArgs& a, const AttnUnit& u, int r0,
                                             int n, int prefix_len) {
  return r0 >= 0 && n >= 1 && n <= kMaxTreeRows && r0 <= a.num_rows - n && u.row_begin >= 0 &&
         u.row_count >= 1 && u.row_begin + u.row_count <= n && u.key_begin >= 0 &&
         u.key_begin <= u.key_end && u.key_end <= prefix_len &&
         ((u.flags & 1) == 0 || u.key_end == prefix_len);
}

// Marks a mismatched unit: the status word, and NaN in its output rows (or in
// its split partial, which the merge then turns into NaN output).
template <int D>
__device__ void poison_unit(const SgTreeAttnArgs& a, const AttnUnit& u, int r0) {
  const int tid = threadIdx.x;
  if (tid == 0 && a.status_dev != nullptr) *a.status_dev = SG_EINVAL;
  const float qnan = __builtin_nanf("");
  if (u.partial >= 0) {
    float* part = static_cast<float*>(a.workspace_dev) + partial_floats(D) * u.partial;
    for (int k = tid; k < static_cast<int>(partial_floats(D)); k += kThreads)
      part[k] = (k >= kQPerUnit * D && k < kQPerUnit * (D + 1)) ? 0.0f : qnan;
    return;
  }
  const int G = a.num_q_heads / a.num_kv_heads;
  uint16_t* out = static_cast<uint16_t*>(a.out_dev);
  for (int k = tid; k < u.row_count * G * D; k += kThreads) {
    const int rr = k / (G * D);
    const int h = (k / D) % G;
    const int64_t row = static_cast<int64_t>(r0) + u.row_begin + rr;
    if (r0 < 0 || row < 0 || row >= a.num_rows) continue;
    out[row * a.out_row_stride + static_cast<int64_t>(u.kv_head * G + h) * a.out_head_stride +
        k % D] = 0x7fc0;  // bf16 quiet NaN
  }
}

// Attention of one work unit by the whole workgroup.
template <int D>
__device__ __forceinline__ void attn_unit(const SgTreeAttnArgs& a, const AttnUnit& u) {
  constexpr int KB = D / 16;                     // QK^T k-blocks of 16 head dims
  constexpr int DB = D / 32;                     // PV blocks of 32 head dims
  constexpr int ROWB = D * 2;                    // bytes per unpadded K/V row
  constexpr int STAGEB = kTileKeys * ROWB;       // bytes of one K (or V) tile
  constexpr int CHUNKS = ROWB / 16;              // 16-byte chunks per row
  constexpr int ROWS_PER_KB = 1024 / ROWB;       // rows covered by one wave DMA
  constexpr int DMAS = STAGEB / 1024 / kWaves;   // DMAs per wave per K (or V) tile
  constexpr int STATE = 2 + 16 * DB;             // floats per lane of a WaveState
  static_assert(DMAS >= 1, "tile too small for the workgroup");
  static_assert(kStages == 4, "the issue schedule assumes a 4-tile ring");
  static_assert(kStages * STAGEB <= 65536, "ring offsets must fit the LDS immediate");
  static_assert(2 * ((kStages * STAGEB) / (STATE * 64 * 4)) >= 2, "merge scratch");
  // Rings of kStages tiles of K and of V; reused as the merge scratch at the end.
  __shared__ __align__(1024) unsigned char s_k[kStages * STAGEB];
  __shared__ __align__(1024) unsigned char s_v[kStages * STAGEB];
  __shared__ uint32_t s_anc[kQPerUnit][kAncWords];
  __shared__ int s_parent[kMaxTreeRows];

  const int G = a.num_q_heads / a.num_kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int col = lane & 31;
  const int nq = (u.row_count * G + 31) / 32;   // q-groups in use, 1..4
  // Every window (one barrier) consumes two consecutive 32-key tiles.  With
  // 1-2 q-groups two waves share a q-group ("key streams") and take one tile
  // each; their results are merged at the end of the unit.  With 3-4 q-groups
  // every wave takes both tiles, one after the other.  Waves beyond
  // nq*streams repeat stream 0's work on the same LDS data and discard it.
  const int streams = nq <= 2 ? 2 : 1;
  const bool both = streams == 1;
  const int qg = wave % nq;
  const int ks = wave / nq;                     // key stream of this wave
  const bool active = ks < streams;
  const int my_tile = active ? ks : 0;          // tile of the window this wave takes first
  const int m = qg * 32 + col;                  // query vector inside the unit
  const int r_local = m / G;                    // query row inside the tile
  const int head = u.kv_head * G + (m - r_local * G);
  const bool q_valid = active && r_local < u.row_count;
  // A record whose request, kv head or partial slot this call does not have
  // (a plan of a larger wave, or not a plan) indexes nothing: it only marks
  // the status word.
  if (!unit_indices_valid<D>(a, u)) {
    if (tid == 0 && a.status_dev != nullptr) *a.status_dev = SG_EINVAL;
    return;
  }
  const int r0 = a.row_offset_dev[u.req];
  const int n = a.row_offset_dev[u.req + 1] - r0;
  // A unit of a plan built for another wave (other prefix lengths or rows)
  // reads nothing and marks its output instead.
  if (!unit_matches(a, u, r0, n, a.prefix_len_dev[u.req])) {
    poison_unit<D>(a, u, r0);
    return;
  }
  const int64_t row = static_cast<int64_t>(r0) + u.row_begin + r_local;
  const int g = u.kv_head;
  const bool do_tree = (u.flags & 1) != 0;
  // The request's K/V is read by this unit alone when its rows fit one row
  // tile and the planner did not split the rows (flags bit 1).
  const bool stream_kv = (u.flags & 2) == 0 && n * G <= kQPerUnit;

  // Ancestor-or-self bitsets of the tile's rows (request-local numbering).
  if (do_tree) {
    for (int k = tid; k < n; k += kThreads) s_parent[k] = a.parent_dev[r0 + k];
    for (int k = tid; k < kQPerUnit * kAncWords; k += kThreads) (&s_anc[0][0])[k] = 0u;
    __syncthreads();
    if (tid < u.row_count) {
      int node = u.row_begin + tid;
      uint32_t bits[kAncWords];
#pragma unroll
      for (int w = 0; w < kAncWords; ++w) bits[w] = 0u;
      for (int guard = 0; node >= 0 && guard < kMaxTreeRows; ++guard) {
#pragma unroll
        for (int w = 0; w < kAncWords; ++w)
          bits[w] |= (w == (node >> 5)) ? (1u << (node & 31)) : 0u;
        const int p = s_parent[node];
        node = (p < node) ? p : -1;
      }
#pragma unroll
      for (int w = 0; w < kAncWords; ++w) s_anc[tid][w] = bits[w];
    }
  }

  // Query operand: lane supplies Q[row, head, 16*kb + 8*half .. +7].
  bf16x8 qf[KB];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q_dev) + row * a.q_row_stride +
                         static_cast<int64_t>(head) * a.q_head_stride + 8 * half;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      qf[kb] = as_bf16x8(q_valid ? *reinterpret_cast<const uint4*>(qp + 16 * kb) : zero4());
  }

  const int prefix_keys = u.key_end - u.key_begin;
  const int tiles_prefix = (prefix_keys + kTileKeys - 1) / kTileKeys;
  const int tiles_full = prefix_keys / kTileKeys;
  const int tiles_tree = do_tree ? (n + kTileKeys - 1) / kTileKeys : 0;
  const int tiles = tiles_prefix + tiles_tree;
  const int64_t prefix0 = a.prefix_start_dev[u.req] + u.key_begin;
  const uint16_t* kc = static_cast<const uint16_t*>(a.k_cache_dev) + g * a.cache_head_stride +
                       prefix0 * a.cache_token_stride;
  const uint16_t* vc = static_cast<const uint16_t*>(a.v_cache_dev) + g * a.cache_head_stride +
                       prefix0 * a.cache_token_stride;
  const uint16_t* kt = static_cast<const uint16_t*>(a.k_tree_dev) + g * a.tree_head_stride +
                       static_cast<int64_t>(r0) * a.tree_row_stride;
  const uint16_t* vt = static_cast<const uint16_t*>(a.v_tree_dev) + g * a.tree_head_stride +
                       static_cast<int64_t>(r0) * a.tree_row_stride;

  // DMA slots of this lane: wave DMA i of a tile covers LDS rows
  // ROWS_PER_KB*(wave*DMAS + i) + lane / CHUNKS, physical chunk lane % CHUNKS;
  // the row holds key pi(row) for K and key row for V.  Full prefix tiles use
  // precomputed lane offsets; the last partial tile and tree tiles clamp the key.
  const int cstride = static_cast<int>(a.cache_token_stride);
  const int tstride = static_cast<int>(a.tree_row_stride);
  uint32_t k_dma[DMAS], v_dma[DMAS];
#pragma unroll
  for (int i = 0; i < DMAS; ++i) {
    const int lds_row = ROWS_PER_KB * (wave * DMAS + i) + lane / CHUNKS;
    const int phys = lane % CHUNKS;
    const int kk = (lds_row & ~31) + key_pi(lds_row & 31);
    k_dma[i] = static_cast<uint32_t>(2 * (kk * cstride + 8 * (phys ^ swz_k<D>(lds_row))));
    v_dma[i] = static_cast<uint32_t>(2 * (lds_row * cstride + 8 * (phys ^ swz_v<D>(lds_row))));
  }
  // K (is_v false) or V half of tile t into ring stage t % kStages.
  auto load_half = [&](int t, bool is_v) {
    unsigned char* ring = is_v ? s_v : s_k;
    const uint32_t dst = lds_addr(ring + (t % kStages) * STAGEB + wave * DMAS * 1024);
    if (t < tiles_full) {
      const unsigned char* base = reinterpret_cast<const unsigned char*>(
          (is_v ? vc : kc) + static_cast<int64_t>(t) * kTileKeys * cstride);
#pragma unroll
      for (int i = 0; i < DMAS; ++i)
        dma16(base, is_v ? v_dma[i] : k_dma[i], dst + 1024 * i, stream_kv);
      return;
    }
    const bool tree = t >= tiles_prefix;
    const int key0 = tree ? (t - tiles_prefix) * kTileKeys : t * kTileKeys;
    const int last = (tree ? n : prefix_keys) - key0 - 1;
    const int stride = tree ? tstride : cstride;
    const uint16_t* src = tree ? (is_v ? vt : kt) : (is_v ? vc : kc);
    const unsigned char* base =
        reinterpret_cast<const unsigned char*>(src + static_cast<int64_t>(key0) * stride);
#pragma unroll
    for (int i = 0; i < DMAS; ++i) {
      const int lds_row = ROWS_PER_KB * (wave * DMAS + i) + lane / CHUNKS;
      const int phys = lane % CHUNKS;
      // Keys past the range re-read the last valid key: finite data that the
      // score mask (K) or a zero probability (V) removes.
      const int key = is_v ? min(lds_row, last) : min((lds_row & ~31) + key_pi(lds_row & 31), last);
      const int sw = is_v ? swz_v<D>(lds_row) : swz_k<D>(lds_row);
      dma16(base, static_cast<uint32_t>(2 * (key * stride + 8 * (phys ^ sw))), dst + 1024 * i,
            stream_kv);
    }
  };

  // Issue schedule.  Window i = 0 .. groups-1 consumes tiles 2i and 2i+1:
  // the PV products of those tiles and the QK products one block ahead, so
  // that the QK MFMAs overlap the softmax VALU work.  The QK products of
  // window i read the next group's tiles 2i+2, 2i+3 (two key streams) or
  // tiles 2i+1, 2i+2 (one stream).  Window j issues V tiles 2j+2, 2j+3 and K
  // tiles 2j+koff, 2j+koff+1 (koff 4, or 3 for one stream) into the ring
  // slots that window j-1 finished reading; window i needs everything window
  // i-1 issued, so nothing is in flight at its barrier.
  const int groups = (tiles + 1) / 2;
  const int koff = both ? 3 : 4;
  auto issue = [&](int j) {
    for (int k = 0; k < 2; ++k) {
      const int t = 2 * j + 2 + k;
      if (t >= 0 && t < tiles) load_half(t, true);
    }
    for (int k = 0; k < 2; ++k) {
      const int t = 2 * j + koff + k;
      if (t >= 0 && t < tiles) load_half(t, false);
    }
  };
  // Wait until at most `newer` half tiles (the newest ones) are in flight.
  auto wait_halves = [&](int newer) {
    switch (newer) {
      case 0: __builtin_amdgcn_s_waitcnt(vmcnt_encoding(0)); break;
      case 1: __builtin_amdgcn_s_waitcnt(vmcnt_encoding(DMAS)); break;
      case 2: __builtin_amdgcn_s_waitcnt(vmcnt_encoding(2 * DMAS)); break;
      case 3: __builtin_amdgcn_s_waitcnt(vmcnt_encoding(3 * DMAS)); break;
      default: __builtin_amdgcn_s_waitcnt(vmcnt_encoding(4 * DMAS)); break;
    }
  };

  // Lane parts of the LDS read addresses (bytes), including this wave's tile
  // offset inside its window (my_tile stages); callers pass the ring stage of
  // the window's first tile.
  const int gq = lane >> 4;
  const int jj = lane & 15;
  const int rr = jj >> 2;
  const int cc = jj & 3;
  int k_off[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
    k_off[kb] = my_tile * STAGEB + col * ROWB + 16 * ((2 * kb + half) ^ swz_k<D>(col));
  int v_off[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int vrow = 16 * half + 4 * hi + rr;
      const int chunk = 4 * db + 2 * (gq & 1) + (cc >> 1);
      v_off[db][hi] = my_tile * STAGEB + vrow * ROWB +
                      16 * (chunk ^ swz_v<D>(vrow)) + 8 * (cc & 1);
    }

  const float c2 = a.scale * kLog2e;
  WaveState<D> st;
  st.m = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.acc[db][r] = 0.0f;

  // S^T of this wave's 32-key block of the group whose first tile is in ring
  // stage `stage`.
  auto qk = [&](int stage) {
    const unsigned char* sk = s_k + stage * STAGEB;
    floatx16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
    bf16x8 kf[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      kf[kb] = as_bf16x8(*reinterpret_cast<const uint4*>(sk + k_off[kb]));
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kb], qf[kb], s, 0, 0, 0);
    return s;
  };
  // Online softmax, step 1: running max of the scores x (masked already).
  // The reference point st.m moves only when some lane's max grew by more than
  // kLazyLog2 in exp2 units: until then the probabilities exp2((x - m) * c2)
  // may exceed 1 (at most 2^kLazyLog2, exact in fp32 and as bf16 MFMA
  // operands), and the final division by the sum normalises them all the
  // same.  With 32-key blocks the max of one of 32 queries grows in most
  // blocks, so rescaling at every growth would cost 64 multiplies in most
  // blocks.
  auto softmax_max = [&](const float (&x)[16]) {
    float tmax = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, x[r]);
    tmax = half_max(tmax);
    const float m_new = fmaxf(st.m, tmax);
    // st.m = -inf gives +inf here (rescale); both -inf gives NaN (keep).
    if (__ballot((m_new - st.m) * c2 > kLazyLog2)) {
      const float alpha = (st.m == -__builtin_inff()) ? 0.0f
                                                       : __builtin_amdgcn_exp2f((st.m - m_new) * c2);
      st.l *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.acc[db][r] *= alpha;
      st.m = m_new;
    }
  };
  // Step 2: probabilities exp2((x - m) * c2) and their sum.  Independent of
  // the accumulators, so it interleaves with the next block's QK MFMAs.
  auto softmax_exp = [&](float (&x)[16]) {
    const float mc = (st.m == -__builtin_inff()) ? 0.0f : st.m * c2;
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[r], c2, -mc));
      psum += x[r];
    }
    st.l += half_sum(psum);
  };
  // Step 3: bf16 probabilities, in the B-operand layout of the PV MFMA (two
  // 16-key halves).
  auto pack = [&](const float (&x)[16], bf16x8 (&pf)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[c][e] = static_cast<__bf16>(x[8 * c + e]);
  };
  // Step 4: O^T += V^T P^T from ring stage `stage`.
  auto pv = [&](const bf16x8 (&pf)[2], int stage) {
    const unsigned char* sv = s_v + stage * STAGEB;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const unsigned char* vrows = sv + 8 * c * ROWB;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const short4_t lo =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vrows + v_off[db][0]));
        const short4_t hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vrows + v_off[db][1]));
        const short8_t both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        st.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, both),
                                                             pf[c], st.acc[db], 0, 0, 0);
      }
    }
  };

  // Prologue: windows -2 and -1 of the issue schedule, then the first QK
  // products, which need the K tiles of window -2; V tiles 0, 1 and K tiles
  // koff-2, koff-1 of window -1 may still be in flight.
  issue(-2);
  issue(-1);
  wait_halves((0 < tiles) + (1 < tiles) + (koff - 2 < tiles) + (koff - 1 < tiles));
  __syncthreads();
  floatx16 s_next;
#pragma unroll
  for (int r = 0; r < 16; ++r) s_next[r] = 0.0f;
  if (my_tile < tiles) s_next = qk(0);

  // Windows whose issued tiles are all full prefix tiles (i < fast_end) need
  // none of the schedule arithmetic: the ring stages are compile-time and the
  // sources are one multiply away.
  const int fast_end = (tiles_full - koff) / 2;
  const int64_t tile_bytes = static_cast<int64_t>(kTileKeys) * cstride * 2;
  const uint32_t k_lds_wave = lds_addr(s_k) + wave * DMAS * 1024;
  const uint32_t v_lds_wave = lds_addr(s_v) + wave * DMAS * 1024;
  auto fast_issue = [&](int i, auto koff_tag, auto cur_tag, auto stream_tag) {
    constexpr int kK = decltype(koff_tag)::value;
    constexpr int kCur = decltype(cur_tag)::value;  // ring stage of tile 2i
    constexpr bool kStream = decltype(stream_tag)::value;
    const unsigned char* vb = reinterpret_cast<const unsigned char*>(vc) +
                              static_cast<int64_t>(2 * i + 2) * tile_bytes;
    const unsigned char* kb = reinterpret_cast<const unsigned char*>(kc) +
                              static_cast<int64_t>(2 * i + kK) * tile_bytes;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
#pragma unroll
      for (int d = 0; d < DMAS; ++d)
        dma16<kStream>(vb + k * tile_bytes, v_dma[d],
                       v_lds_wave + ((kCur + 2 + k) % kStages) * STAGEB + 1024 * d);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
#pragma unroll
      for (int d = 0; d < DMAS; ++d)
        dma16<kStream>(kb + k * tile_bytes, k_dma[d],
                       k_lds_wave + ((kCur + kK + k) % kStages) * STAGEB + 1024 * d);
    }
  };
  auto open_window = [&](int i, auto koff_tag, auto cur_tag, auto stream_tag) {
    wait_halves(0);
    __syncthreads();
    if (i < fast_end) {
      fast_issue(i, koff_tag, cur_tag, stream_tag);
    } else {
      issue(i);
    }
  };
  // Softmax of the current block interleaved with the next block's QK MFMAs;
  // leaves the probabilities in pf.
  auto softmax_qk = [&](int next_stage, bf16x8 (&pf)[2]) {
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = s_next[r];
    softmax_max(x);
    s_next = qk(next_stage);
    softmax_exp(x);
    __builtin_amdgcn_sched_group_barrier(0x100, KB, 0);
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
    pack(x, pf);
  };

  // Steady state: windows whose current tiles and the tiles of their QK
  // products are full prefix tiles need no mask, and the ring stages are
  // compile-time constants in loops unrolled by two windows (the ring size).
  // The last tile a window's QK products read is 2i+koff-1.
  const int steady_end = max(0, (tiles_full - koff + 2) / 2);
  int i = 0;
  bf16x8 pf[2];
  if (both) {
    auto step = [&](int w, auto cur_tag, auto stream_tag) {
      constexpr int kCur = decltype(cur_tag)::value;
      open_window(w, IntTag<3>{}, cur_tag, stream_tag);
      softmax_qk(kCur + 1, pf);
      pv(pf, kCur);
      softmax_qk((kCur + 2) % kStages, pf);
      pv(pf, kCur + 1);
    };
    if (stream_kv) {
      for (; i + 2 <= steady_end; i += 2) {
        step(i, IntTag<0>{}, BoolTag<true>{});
        step(i + 1, IntTag<2>{}, BoolTag<true>{});
      }
    } else {
      for (; i + 2 <= steady_end; i += 2) {
        step(i, IntTag<0>{}, BoolTag<false>{});
        step(i + 1, IntTag<2>{}, BoolTag<false>{});
      }
    }
  } else {
    // 1-2 q-groups: at most 64 query vectors, the request's rows fit one row
    // tile, so the unit is its K/V's only reader.
    auto step = [&](int w, auto cur_tag) {
      constexpr int kCur = decltype(cur_tag)::value;
      open_window(w, IntTag<4>{}, cur_tag, BoolTag<true>{});
      softmax_qk((kCur + 2) % kStages, pf);
      pv(pf, kCur);
    };
    for (; i + 2 <= steady_end; i += 2) {
      step(i, IntTag<0>{});
      step(i + 1, IntTag<2>{});
    }
  }
  // Remaining windows: runtime stages, masks from the key limit and the
  // ancestor bitsets.
  for (; i < groups; ++i) {
    wait_halves(0);
    __syncthreads();
    issue(i);
    for (int b = 0; b < (both ? 2 : 1); ++b) {
      const int t = 2 * i + my_tile + b;
      const int t_next = both ? t + 1 : t + 2;
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = s_next[r];
      if (t_next < tiles) s_next = qk((t_next - my_tile) % kStages);
      if (t < tiles) {
        const bool tree = t >= tiles_prefix;
        const int key0 = (tree ? t - tiles_prefix : t) * kTileKeys;
        const int limit = tree ? n : prefix_keys;
        const uint32_t bits = tree ? (s_anc[r_local][key0 >> 5] >> (16 * half)) : 0xffffffffu;
        const int first = key0 + 16 * half;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          x[r] = (first + r < limit && ((bits >> r) & 1u)) ? x[r] : -__builtin_inff();
        softmax_max(x);
        softmax_exp(x);
        pack(x, pf);
        pv(pf, (t - my_tile) % kStages);
      }
    }
  }
  __syncthreads();


  // Merge the key streams of each q-group through LDS (the ring is free now).
  // Slot k (k = (ks-1)*nq + qg < 6) lives at float offset k*STATE*64 of s_k|s_v.
  auto merge_slot = [&](int k) -> float* {
    constexpr int kPerBuf = (kStages * STAGEB) / (STATE * 64 * 4);
    unsigned char* buf = (k < kPerBuf) ? s_k : s_v;
    return reinterpret_cast<float*>(buf) + static_cast<size_t>(k % kPerBuf) * STATE * 64;
  };
  if (active && ks > 0) {
    float* slot = merge_slot((ks - 1) * nq + qg);
    slot[lane] = st.m;
    slot[64 + lane] = st.l;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) slot[(2 + 16 * db + r) * 64 + lane] = st.acc[db][r];
  }
  __syncthreads();
  if (!active || ks > 0) return;
  {
    float m_all = st.m;
    for (int s = 1; s < streams; ++s) m_all = fmaxf(m_all, merge_slot((s - 1) * nq + qg)[lane]);
    const float m_use = (m_all == -__builtin_inff()) ? 0.0f : m_all;
    const float w0 = (st.m == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((st.m - m_use) * c2);
    st.l *= w0;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[db][r] *= w0;
    for (int s = 1; s < streams; ++s) {
      const float* slot = merge_slot((s - 1) * nq + qg);
      const float ms = slot[lane];
      const float w = (ms == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((ms - m_use) * c2);
      st.l += w * slot[64 + lane];
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.acc[db][r] += w * slot[(2 + 16 * db + r) * 64 + lane];
    }
    st.m = m_all;
  }

  // st.acc[db][r] holds head dim 32*db + 8*(r/4) + 4*half + (r%4) of this lane's query.
  if (u.partial >= 0) {
    // Partial layout (floats): O as float4 chunks ((db*4 + q4)*2 + half)*128 + m,
    // then the running max (log2 units) and sum per query vector.
    float* part = static_cast<float*>(a.workspace_dev) + partial_floats(D) * u.partial;
    float4* o = reinterpret_cast<float4*>(part);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        o[((db * 4 + q4) * 2 + half) * kQPerUnit + m] =
            make_float4(st.acc[db][4 * q4], st.acc[db][4 * q4 + 1], st.acc[db][4 * q4 + 2],
                        st.acc[db][4 * q4 + 3]);
    if (half == 0) {
      part[static_cast<size_t>(kQPerUnit) * D + m] =
          (st.m == -__builtin_inff()) ? st.m : st.m * c2;
      part[static_cast<size_t>(kQPerUnit) * D + kQPerUnit + m] = st.l;
    }
    return;
  }
  // Output through a per-wave LDS staging tile: each lane holds 64 scattered
  // head dims of one query vector, while HBM wants each query vector's D
  // contiguous values written whole.  The tile (32 query vectors, rows padded
  // by 16 bytes against bank conflicts) lies in ring space this wave alone
  // uses now: with two key streams behind the stream-merge slot of its ring,
  // otherwise in one of the four quarters of the rings.
  constexpr int kRowBytes = 2 * D;
  constexpr int kPitch = kRowBytes + 16;
  constexpr int kSlotBytes = STATE * 64 * 4;
  static_assert(kSlotBytes + 32 * kPitch <= kStages * STAGEB &&
                    2 * 32 * kPitch <= kStages * STAGEB,
                "output staging must fit the rings");
  unsigned char* stage =
      ((qg & 1) ? s_v : s_k) + (streams > 1 ? kSlotBytes : (qg >> 1) * 32 * kPitch);
  const float inv = st.l > 0.0f ? 1.0f / st.l : 0.0f;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      uint2 packed;
      packed.x = pack_bf16x2(st.acc[db][4 * q4] * inv, st.acc[db][4 * q4 + 1] * inv);
      packed.y = pack_bf16x2(st.acc[db][4 * q4 + 2] * inv, st.acc[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(stage + col * kPitch + 2 * (32 * db + 8 * q4 + 4 * half)) =
          packed;
    }
  __builtin_amdgcn_wave_barrier();
  // Row-contiguous read-back (LDS keeps this wave's accesses in order): every
  // store instruction writes 1 KiB of whole query vectors, 16 bytes a lane when
  // the output strides allow it (multiples of 8 elements), else 8 bytes a lane.
  uint16_t* const out_base = static_cast<uint16_t*>(a.out_dev) +
                             (static_cast<int64_t>(r0) + u.row_begin) * a.out_row_stride +
                             static_cast<int64_t>(u.kv_head * G) * a.out_head_stride;
  auto dst_of = [&](int q, int within) {
    const int mq = qg * 32 + q;
    const int rq = mq / G;
    return rq < u.row_count
               ? out_base + static_cast<int64_t>(rq) * a.out_row_stride +
                     static_cast<int64_t>(mq - rq * G) * a.out_head_stride + within / 2
               : nullptr;
  };
  if (((a.out_row_stride | a.out_head_stride) & 7) == 0 &&
      (reinterpret_cast<uintptr_t>(a.out_dev) & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 32 * kRowBytes / 1024; ++i) {
      const int linear = i * 1024 + 16 * lane;
      const int q = linear / kRowBytes;  // query vector of this q-group
      const int within = linear - q * kRowBytes;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + q * kPitch + within);
      uint16_t* dst = dst_of(q, within);
      if (dst != nullptr) *reinterpret_cast<uint4*>(dst) = v;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32 * kRowBytes / 512; ++i) {
      const int linear = i * 512 + 8 * lane;
      const int q = linear / kRowBytes;
      const int within = linear - q * kRowBytes;
      const uint2 v = *reinterpret_cast<const uint2*>(stage + q * kPitch + within);
      uint16_t* dst = dst_of(q, within);
      if (dst != nullptr) *reinterpret_cast<uint2*>(dst) = v;
    }
  }
}

// One workgroup per work list (two resident per CU): the units of list b
// are units[bin_offset[b] .. bin_offset[b+1]), processed in order.
template <int D>
__global__ __launch_bounds__(kThreads, kListsPerCU) void tree_attn_kernel(SgTreeAttnArgs a) {
  const PlanHeader* hdr = static_cast<const PlanHeader*>(a.plan_dev);
  const AttnUnit* units = reinterpret_cast<const AttnUnit*>(hdr + 1);
  const int32_t* bin_offset = reinterpret_cast<const int32_t*>(
      reinterpret_cast<const MergeGroup*>(units + hdr->num_units) + hdr->num_merges);
  const int end = bin_offset[blockIdx.x + 1];
  for (int k = bin_offset[blockIdx.x]; k < end; ++k) {
    const AttnUnit u = units[k];
    attn_unit<D>(a, u);
    __syncthreads();  // LDS of this unit is free before the next one starts
  }
}

// Combines the partials of the split groups: merge_blocks_per_group(D)
// workgroups per group, thread -> one (query vector, float4 chunk).  groups:
// the plan's merge-group records on the device when the host knows where they
// are (saves the round trip through the plan header), else nullptr.
template <int D>
__global__ __launch_bounds__(kMergeThreads) void tree_attn_merge_kernel(
    SgTreeAttnArgs a, const MergeGroup* groups) {
  if (groups == nullptr) {
    const PlanHeader* hdr = static_cast<const PlanHeader*>(a.plan_dev);
    groups = reinterpret_cast<const MergeGroup*>(reinterpret_cast<const AttnUnit*>(hdr + 1) +
                                                 hdr->num_units);
  }
  const int sub = blockIdx.x % merge_blocks_per_group(D);
  const MergeGroup grp = groups[blockIdx.x / merge_blocks_per_group(D)];
  const int G = a.num_q_heads / a.num_kv_heads;
  // A record this call cannot hold (another wave's plan) indexes nothing.
  const size_t slots = a.workspace_bytes / (sizeof(float) * partial_floats(D));
  if (grp.req < 0 || grp.req >= a.num_requests || grp.kv_head < 0 ||
      grp.kv_head >= a.num_kv_heads || grp.row_count < 0 || grp.row_count * G > kQPerUnit ||
      grp.first_partial < 0 || grp.num_partials < 1 ||
      static_cast<size_t>(grp.first_partial) + grp.num_partials > slots) {
    if (threadIdx.x == 0 && a.status_dev != nullptr) *a.status_dev = SG_EINVAL;
    return;
  }
  const int r0 = a.row_offset_dev[grp.req];
  const float* ws = static_cast<const float*>(a.workspace_dev);
  const int vectors = grp.row_count * G;
  {
    const int item = sub * kMergeThreads + static_cast<int>(threadIdx.x);
    const int ch = item / kQPerUnit;  // chunk index ((db*4 + q4)*2 + half)
    const int m = item - ch * kQPerUnit;
    if (m >= vectors) return;
    // Every partial's (max, sum, O chunk) is loaded before any is used, so the
    // group costs one memory round trip (up to kMergeBatch partials at a time).
    constexpr int kMergeBatch = 4;
    const float* part0 = ws + partial_floats(D) * grp.first_partial;
    float mx = -__builtin_inff();
    float l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < grp.num_partials; s0 += kMergeBatch) {
      float ms[kMergeBatch], ls[kMergeBatch];
      float4 vs[kMergeBatch];
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) {
        ms[j] = -__builtin_inff();
        ls[j] = 0.0f;
        vs[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (s0 + j < grp.num_partials) {
          const float* part = part0 + partial_floats(D) * (s0 + j);
          ms[j] = part[static_cast<size_t>(kQPerUnit) * D + m];
          ls[j] = part[static_cast<size_t>(kQPerUnit) * D + kQPerUnit + m];
          vs[j] = reinterpret_cast<const float4*>(part)[ch * kQPerUnit + m];
        }
      }
      float bmx = mx;
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) bmx = fmaxf(bmx, ms[j]);
      const float m_use = (bmx == -__builtin_inff()) ? 0.0f : bmx;
      // Rescale what earlier batches accumulated to the new reference.
      const float w_old = (mx == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(mx - m_use);
      l *= w_old;
      o.x *= w_old;
      o.y *= w_old;
      o.z *= w_old;
      o.w *= w_old;
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) {
        const float w =
            (ms[j] == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(ms[j] - m_use);
        l += w * ls[j];
        o.x += w * vs[j].x;
        o.y += w * vs[j].y;
        o.z += w * vs[j].z;
        o.w += w * vs[j].w;
      }
      mx = bmx;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int r_local = m / G;
    const int head = grp.kv_head * G + (m - r_local * G);
    const int db = ch / 8;
    const int q4 = (ch / 2) & 3;
    const int hf = ch & 1;
    const int64_t row = static_cast<int64_t>(r0) + grp.row_begin + r_local;
    if (r0 < 0 || row >= a.num_rows) return;  // metadata of another wave
    uint16_t* dst = static_cast<uint16_t*>(a.out_dev) + row * a.out_row_stride +
                    static_cast<int64_t>(head) * a.out_head_stride + 32 * db + 8 * q4 + 4 * hf;
    uint2 packed;
    packed.x = pack_bf16x2(o.x * inv, o.y * inv);
    packed.y = pack_bf16x2(o.z * inv, o.w * inv);
    *reinterpret_cast<uint2*>(dst) = packed;
  }
}

}  // namespace
}  // namespace sg

extern "C" int sg_tree_attn_plan(int32_t num_requests, const int32_t* row_offset_host,
                                 const int32_t* prefix_len_host, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim,
                                 int32_t target_units_hint, void* plan_host,
                                 size_t plan_capacity_bytes, size_t* plan_bytes,
                                 int32_t* plan_units, int32_t* plan_merges,
                                 size_t* workspace_bytes) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(num_requests >= 0, "num_requests must be non-negative");
  SG_REQUIRE(num_requests == 0 || (row_offset_host && prefix_len_host), "null host array");
  SG_REQUIRE(num_kv_heads >= 1 && num_q_heads >= num_kv_heads &&
                 num_q_heads % num_kv_heads == 0,
             "num_q_heads must be a positive multiple of num_kv_heads");
  const int G = num_q_heads / num_kv_heads;
  SG_REQUIRE(G <= kMaxGroup && kQPerUnit % G == 0,
             "query heads per kv head must be 1, 2, 4, 8 or 16");
  SG_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128");
  SG_REQUIRE(plan_bytes && plan_units && plan_merges && workspace_bytes, "null output pointer");
  const int rows_per_tile = kQPerUnit / G;
  SG_REQUIRE(num_requests == 0 || row_offset_host[0] == 0, "row_offset[0] must be 0");

  // Units of one (request, kv head, row tile) are split over their prefix when
  // the wave has too few units to give every CU slot work, or when one would
  // dominate the end of the launch: each split costs a partial write and a
  // merge pass.  target_units_hint overrides the slot count.
  int64_t base_units = 0;
  for (int i = 0; i < num_requests; ++i) {
    const int rows = row_offset_host[i + 1] - row_offset_host[i];
    SG_REQUIRE(rows >= 0 && rows <= kMaxTreeRows,
               "every request must have between 0 and 256 packed rows");
    SG_REQUIRE(prefix_len_host[i] >= 0, "prefix lengths must be non-negative");
    const int tiles = (rows + rows_per_tile - 1) / rows_per_tile;
    base_units += static_cast<int64_t>(num_kv_heads) * tiles;
  }
  const int64_t target = target_units_hint > 0 ? target_units_hint : kDefaultCUs * kListsPerCU;
  auto unit_cost = [&](int row_count, int64_t tiles) -> int64_t {
    const int nq = (row_count * G + 31) / 32;
    return nq <= 2 ? 550 + 57 * tiles : 840 + 88 * tiles;
  };

  // Small waves (fewer (request, kv head, row tile) units than the GPU has
  // CUs) are latency-bound: every unit of request i is cut into
  // small_splits[i] key ranges, chosen greedily -- the request whose pieces
  // cost most gets one more piece -- while the wave stays within one unit
  // per CU (a lone workgroup streams at its CU's whole bandwidth, and fewer
  // pieces write fewer partials: 39 us against 44 us at two per CU on a
  // 16-request, 496-row Qwen3-4B wave) and pieces keep at least four tiles of
  // prefix.  No row splits: they would add units.
  const int64_t small_target = target_units_hint > 0 ? target_units_hint : kDefaultCUs;
  const bool small_wave = base_units > 0 && base_units < small_target;
  std::vector<int> small_splits(num_requests, 1);
  if (small_wave) {
    auto piece_cost = [&](int i, int pieces) -> int64_t {
      const int rows = row_offset_host[i + 1] - row_offset_host[i];
      const int64_t prefix_tiles = (prefix_len_host[i] + kTileKeys - 1) / kTileKeys;
      const int64_t tree_tiles = (rows + kTileKeys - 1) / kTileKeys;
      return unit_cost(std::min(rows, rows_per_tile),
                       (prefix_tiles + pieces - 1) / pieces + tree_tiles);
    };
    int64_t total = base_units;
    std::priority_queue<std::pair<int64_t, int>> heap;  // (piece cost, request)
    for (int i = 0; i < num_requests; ++i)
      if (row_offset_host[i + 1] > row_offset_host[i]) heap.push({piece_cost(i, 1), i});
    while (!heap.empty()) {
      const int i = heap.top().second;
      heap.pop();
      const int rows = row_offset_host[i + 1] - row_offset_host[i];
      const int next = small_splits[i] + 1;
      const int64_t add =
          static_cast<int64_t>(num_kv_heads) * ((rows + rows_per_tile - 1) / rows_per_tile);
      if (total + add > small_target || prefix_len_host[i] / next < 4 * kTileKeys) continue;
      small_splits[i] = next;
      total += add;
      heap.push({piece_cost(i, next), i});
    }
  }

  // Balance: a unit costing more than kSplitAbovePercent % of a CU slot's
  // mean share is split over its prefix into pieces below that bound, so that
  // no unit dominates the end of the launch (each piece costs a prologue, a
  // partial write and a merge, so the bound is high).
  std::vector<int> balance_splits(num_requests, 1);
  std::vector<char> split_rows(num_requests, 0);
  {
    int64_t total_cost = 0;
    std::vector<int64_t> req_cost(num_requests, 0);
    for (int i = 0; i < num_requests; ++i) {
      const int rows = row_offset_host[i + 1] - row_offset_host[i];
      const int64_t tiles = (prefix_len_host[i] + kTileKeys - 1) / kTileKeys +
                            (rows + kTileKeys - 1) / kTileKeys;
      for (int rb = 0; rb < rows; rb += rows_per_tile) {
        const int64_t c = unit_cost(std::min(rows_per_tile, rows - rb), tiles);
        total_cost += c * num_kv_heads;
        req_cost[i] = std::max(req_cost[i], c);
      }
    }
    const int64_t lists = std::max<int64_t>(1, std::min(target, base_units));
    const int64_t bound = std::max<int64_t>(1, total_cost * kSplitAbovePercent / (100 * lists));
    const int64_t row_bound =
        std::max<int64_t>(1, total_cost * kRowSplitAbovePercent / (100 * lists));
    for (int i = 0; i < num_requests; ++i) {
      if (req_cost[i] > bound) balance_splits[i] = static_cast<int>((req_cost[i] + bound - 1) / bound);
      const int rows = row_offset_host[i + 1] - row_offset_host[i];
      split_rows[i] = req_cost[i] > row_bound && rows * G > kQPerUnit / 2;
    }
  }
  std::vector<AttnUnit> units;
  std::vector<MergeGroup> merges;
  int32_t partials = 0;
  for (int i = 0; i < num_requests; ++i) {
    const int rows = row_offset_host[i + 1] - row_offset_host[i];
    if (rows == 0) continue;
    const int L = prefix_len_host[i];
    // A large unit with more than two q-groups is split by rows into units of
    // 64 query vectors (half a row tile), which read the same K/V on one XCD
    // (L2 serves the second read) and need no merge; only a unit of at most
    // 64 query vectors is split over its prefix.
    const bool row_split = !small_wave && split_rows[i] != 0;
    const int rpt = row_split ? rows_per_tile / 2 : rows_per_tile;
    // Pieces keep at least four full tiles of prefix.
    const int splits =
        small_wave ? small_splits[i]
                   : std::max(1, std::min(row_split ? 1 : balance_splits[i], L / (4 * kTileKeys)));
    const int tiles = (rows + rpt - 1) / rpt;
    for (int g = 0; g < num_kv_heads; ++g) {
      for (int tile = 0; tile < tiles; ++tile) {
        const int group = splits > 1 ? static_cast<int>(merges.size()) : -1;
        const int first = partials;
        for (int s = 0; s < splits; ++s) {
          AttnUnit u;
          u.req = i;
          u.kv_head = g;
          u.row_begin = tile * rpt;
          u.row_count = std::min(rpt, rows - u.row_begin);
          u.key_begin = static_cast<int32_t>(static_cast<int64_t>(L) * s / splits / kTileKeys *
                                             kTileKeys);
          u.key_end = s + 1 == splits ? L
                                      : static_cast<int32_t>(static_cast<int64_t>(L) * (s + 1) /
                                                             splits / kTileKeys * kTileKeys);
          u.partial = splits > 1 ? partials++ : -1;
          u.flags = ((s + 1 == splits) ? 1 : 0) | (row_split ? 2 : 0);
          u.group = group;
          u.num_splits = splits;
          u.first_partial = splits > 1 ? first : -1;
          u.pad = 0;
          units.push_back(u);
        }
        if (splits > 1) {
          MergeGroup mg;
          mg.req = i;
          mg.kv_head = g;
          mg.row_begin = tile * rpt;
          mg.row_count = std::min(rpt, rows - mg.row_begin);
          mg.first_partial = first;
          mg.num_partials = splits;
          mg.pad0 = mg.pad1 = 0;
          merges.push_back(mg);
        }
      }
    }
  }
  // Unit cost, the order of the lists and the packing of a hinted list count
  // (hundredths of a microsecond on MI355X at 32q/8kv, D=128): a fixed part
  // (prologue latency, epilogue) plus a part per 32-key tile; a unit with at
  // most two q-groups (64 query vectors) streams two tiles per window and
  // costs less per tile.
  std::vector<int64_t> cost(units.size());
  for (size_t k = 0; k < units.size(); ++k) {
    const int rows = row_offset_host[units[k].req + 1] - row_offset_host[units[k].req];
    const int64_t tiles =
        (units[k].key_end - units[k].key_begin + kTileKeys - 1) / kTileKeys +
        ((units[k].flags & 1) ? (rows + kTileKeys - 1) / kTileKeys : 0);
    cost[k] = unit_cost(units[k].row_count, tiles);
  }
  std::vector<size_t> order(units.size());
  std::iota(order.begin(), order.end(), size_t{0});
  std::stable_sort(order.begin(), order.end(),
                   [&](size_t x, size_t y) { return cost[x] > cost[y]; });
  // By default every unit is a work list of its own, in decreasing cost
  // order.  The first two per CU start at once, the largest on each CU's
  // first slot (which the CU's issue arbitration favours), and the hardware
  // dispatcher starts every further unit on the first slot that frees: greedy
  // list scheduling at the speed each slot actually achieves.  With a target
  // hint the units are packed onto that many lists instead.
  const int64_t bins = target_units_hint > 0
                           ? std::min<int64_t>(target, static_cast<int64_t>(units.size()))
                           : static_cast<int64_t>(units.size());
  constexpr int64_t kXcds = 8;
  std::vector<int64_t> load(bins, 0);
  std::vector<std::vector<size_t>> bin_units(bins);
  // Units that read the same (request, kv head) K/V (the row tiles of a tree
  // larger than one tile, and split pieces) go to lists of one XCD: the
  // dispatcher places workgroup b on XCD b % 8, whose L2 then serves the
  // re-reads.  (A placement heuristic only.)
  std::vector<int64_t> xcd_of(static_cast<size_t>(num_requests) * num_kv_heads, -1);
  for (size_t k : order) {
    const size_t key = static_cast<size_t>(units[k].req) * num_kv_heads + units[k].kv_head;
    int64_t b = -1;
    if (xcd_of[key] >= 0 && bins >= kXcds) {
      for (int64_t c = xcd_of[key]; c < bins; c += kXcds)
        if (b < 0 || load[c] < load[b]) b = c;
    } else {
      b = std::min_element(load.begin(), load.end()) - load.begin();
      xcd_of[key] = b % kXcds;
    }
    load[b] += cost[k];
    bin_units[b].push_back(k);
  }
  // Local search: move a unit out of the most loaded list, or swap it with a
  // smaller unit of the least loaded list, while that lowers the maximum.
  for (int round = 0; bins > 1 && round < 4096; ++round) {
    const int64_t hi = std::max_element(load.begin(), load.end()) - load.begin();
    const int64_t lo = std::min_element(load.begin(), load.end()) - load.begin();
    const int64_t gap = load[hi] - load[lo];
    int64_t best = 0;
    size_t bi = 0, bj = SIZE_MAX;
    for (size_t x = 0; x < bin_units[hi].size(); ++x) {
      const int64_t cx = cost[bin_units[hi][x]];
      if (cx < gap && cx > best) best = cx, bi = x, bj = SIZE_MAX;  // move
      for (size_t y = 0; y < bin_units[lo].size(); ++y) {
        const int64_t d = cx - cost[bin_units[lo][y]];
        if (d > 0 && d < gap && d > best) best = d, bi = x, bj = y;  // swap
      }
    }
    if (best == 0) break;
    const size_t ux = bin_units[hi][bi];
    if (bj == SIZE_MAX) {
      bin_units[hi].erase(bin_units[hi].begin() + bi);
      bin_units[lo].push_back(ux);
    } else {
      std::swap(bin_units[hi][bi], bin_units[lo][bj]);
    }
    load[hi] -= best;
    load[lo] += best;
  }
  // Lists left empty by the XCD placement are dropped.
  bin_units.erase(std::remove_if(bin_units.begin(), bin_units.end(),
                                 [](const std::vector<size_t>& b) { return b.empty(); }),
                  bin_units.end());
  const int64_t lists = static_cast<int64_t>(bin_units.size());

  const size_t bytes = sizeof(PlanHeader) + sizeof(AttnUnit) * units.size() +
                       sizeof(MergeGroup) * merges.size() + sizeof(int32_t) * (lists + 1);
  *plan_bytes = bytes;
  *plan_units = static_cast<int32_t>(lists);
  *plan_merges = static_cast<int32_t>(merges.size());
  *workspace_bytes = sizeof(float) * partial_floats(head_dim) * static_cast<size_t>(partials);
  if (plan_host == nullptr) return SG_OK;  // size query
  SG_REQUIRE(plan_capacity_bytes >= bytes, "plan buffer too small");
  PlanHeader hdr = {};
  hdr.magic = kPlanMagic;
  hdr.num_units = static_cast<int32_t>(units.size());
  hdr.num_merges = static_cast<int32_t>(merges.size());
  hdr.rows_per_tile = rows_per_tile;
  hdr.head_dim = head_dim;
  hdr.group = G;
  hdr.num_partials = partials;
  hdr.num_bins = static_cast<int32_t>(lists);
  hdr.num_requests = num_requests;
  hdr.num_rows = num_requests > 0 ? row_offset_host[num_requests] : 0;
  hdr.num_kv_heads = num_kv_heads;
  hdr.meta_hash = meta_hash(num_requests, row_offset_host, prefix_len_host);
  char* out = static_cast<char*>(plan_host);
  std::memcpy(out, &hdr, sizeof(hdr));
  AttnUnit* uo = reinterpret_cast<AttnUnit*>(out + sizeof(hdr));
  MergeGroup* mo = reinterpret_cast<MergeGroup*>(uo + units.size());
  int32_t* bo = reinterpret_cast<int32_t*>(mo + merges.size());
  size_t next = 0;
  for (int64_t b = 0; b < lists; ++b) {
    bo[b] = static_cast<int32_t>(next);
    for (size_t k : bin_units[b]) uo[next++] = units[k];
  }
  bo[lists] = static_cast<int32_t>(next);
  std::memcpy(mo, merges.data(), sizeof(MergeGroup) * merges.size());
  return SG_OK;
}

extern "C" int sg_tree_attn_plan_check(const void* plan_host, int32_t num_requests,
                                       const int32_t* row_offset_host,
                                       const int32_t* prefix_len_host) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(plan_host != nullptr, "null plan");
  SG_REQUIRE(num_requests >= 0, "num_requests must be non-negative");
  SG_REQUIRE(num_requests == 0 || (row_offset_host && prefix_len_host), "null host array");
  PlanHeader hdr;
  std::memcpy(&hdr, plan_host, sizeof(hdr));
  SG_REQUIRE(hdr.magic == kPlanMagic, "not a plan of sg_tree_attn_plan");
  SG_REQUIRE(hdr.num_requests == num_requests &&
                 hdr.meta_hash == meta_hash(num_requests, row_offset_host, prefix_len_host),
             "the plan was built for another wave (row offsets or prefix lengths differ)");
  return SG_OK;
}

extern "C" int sg_tree_attn_fwd(const SgTreeAttnArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null SgTreeAttnArgs");
  const SgTreeAttnArgs& a = *args;
  SG_REQUIRE(a.num_kv_heads >= 1 && a.num_q_heads >= a.num_kv_heads &&
                 a.num_q_heads % a.num_kv_heads == 0,
             "num_q_heads must be a positive multiple of num_kv_heads");
  const int G = a.num_q_heads / a.num_kv_heads;
  SG_REQUIRE(G <= kMaxGroup && kQPerUnit % G == 0,
             "query heads per kv head must be 1, 2, 4, 8 or 16");
  SG_REQUIRE(a.head_dim == 64 || a.head_dim == 128, "head_dim must be 64 or 128");
  SG_REQUIRE(a.num_requests >= 0 && a.num_rows >= 0, "negative sizes");
  SG_REQUIRE(a.plan_units >= 0 && a.plan_merges >= 0, "negative plan sizes");
  const MergeGroup* merge_groups = nullptr;
  if (a.plan_host != nullptr) {
    PlanHeader hdr;
    std::memcpy(&hdr, a.plan_host, sizeof(hdr));
    merge_groups = reinterpret_cast<const MergeGroup*>(
        static_cast<const char*>(a.plan_dev) + sizeof(PlanHeader) +
        sizeof(AttnUnit) * static_cast<size_t>(hdr.num_units));
    SG_REQUIRE(hdr.magic == kPlanMagic, "plan_host is not a plan of sg_tree_attn_plan");
    SG_REQUIRE(hdr.group == G && hdr.head_dim == a.head_dim &&
                   hdr.num_kv_heads == a.num_kv_heads,
               "the plan was built for another head configuration");
    SG_REQUIRE(hdr.num_requests == a.num_requests && hdr.num_rows == a.num_rows,
               "the plan was built for another wave (request or row count differs)");
    SG_REQUIRE(hdr.num_bins == a.plan_units && hdr.num_merges == a.plan_merges,
               "plan_units / plan_merges disagree with the plan");
    SG_REQUIRE(a.plan_merges == 0 ||
                   a.workspace_bytes >= sizeof(float) * partial_floats(a.head_dim) *
                                            static_cast<size_t>(hdr.num_partials),
               "workspace below the plan's split partials");
  }
  if (a.plan_units == 0) return SG_OK;
  SG_REQUIRE(a.q_dev && a.k_cache_dev && a.v_cache_dev && a.k_tree_dev && a.v_tree_dev &&
                 a.row_offset_dev && a.prefix_start_dev && a.prefix_len_dev && a.parent_dev &&
                 a.out_dev && a.plan_dev,
             "null device pointer");
  SG_REQUIRE(a.plan_merges == 0 || a.workspace_dev, "split plan needs a workspace");
  SG_REQUIRE(a.q_row_stride % 8 == 0 && a.q_head_stride % 8 == 0 &&
                 a.cache_head_stride % 8 == 0 && a.cache_token_stride % 8 == 0 &&
                 a.tree_row_stride % 8 == 0 && a.tree_head_stride % 8 == 0 &&
                 a.out_row_stride % 4 == 0 && a.out_head_stride % 4 == 0,
             "strides must be multiples of 8 elements (16-byte rows)");
  // Lane offsets inside one key tile are 32-bit byte offsets.
  SG_REQUIRE(a.cache_token_stride >= 0 && a.cache_token_stride < (int64_t{1} << 24) &&
                 a.tree_row_stride >= 0 && a.tree_row_stride < (int64_t{1} << 24),
             "cache_token_stride and tree_row_stride must lie in [0, 2^24) elements");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a.head_dim == 128) {
    hipLaunchKernelGGL(tree_attn_kernel<128>, dim3(a.plan_units), dim3(kThreads), 0, s, a);
    SG_LAUNCH_CHECK();
    if (a.plan_merges > 0) {
      hipLaunchKernelGGL(tree_attn_merge_kernel<128>,
                         dim3(a.plan_merges * merge_blocks_per_group(128)), dim3(kMergeThreads),
                         0, s, a, merge_groups);
      SG_LAUNCH_CHECK();
    }
  } else {
    hipLaunchKernelGGL(tree_attn_kernel<64>, dim3(a.plan_units), dim3(kThreads), 0, s, a);
    SG_LAUNCH_CHECK();
    if (a.plan_merges > 0) {
      hipLaunchKernelGGL(tree_attn_merge_kernel<64>,
                         dim3(a.plan_merges * merge_blocks_per_group(64)), dim3(kMergeThreads),
                         0, s, a, merge_groups);
      SG_LAUNCH_CHECK();
    }
  }
  return SG_OK;
}
