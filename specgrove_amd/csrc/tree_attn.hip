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
// Decomposition (MI355X): a work unit is (request, kv head, tile of up to
// 128/G query rows = 128 query vectors, range of prefix keys); the last unit
// of a request's key range also covers the tree rows.  A workgroup is four
// wavefronts; wavefront w owns 32 query vectors.  Per 64-key tile:
//   S^T[key, q] = K Q^T  with v_mfma_f32_32x32x16_bf16 (A = K rows from LDS,
//                        B = Q from registers),
//   online softmax per query column (one lane pair per query),
//   O^T[d, q] += V^T P^T with the same MFMA (A = V^T rows from LDS, B = P in
//                        registers).
// K rows are written to LDS in the permuted order pi (LDS row i of a 32-key
// block holds key pi(i) = 16*((i>>2)&1) + 4*(i>>3) + (i&3)) so that the MFMA
// result gives each lane 16 consecutive keys; V is stored transposed with the
// same permutation on head-dim rows so the output gives each lane 16
// consecutive head dims.  Tiles are double-buffered in LDS; rows of an unfinished
// key range are combined by a split-K merge kernel in log2 space.
#include <algorithm>
#include <cstring>
#include <numeric>
#include <vector>

#include "sg_common.h"

namespace sg {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float floatx16;

constexpr int kAttnThreads = 256;
constexpr int kQPerUnit = 128;
constexpr int kKeyTile = 64;
constexpr int kMaxTreeRows = 256;
constexpr int kAncWords = kMaxTreeRows / 32;
constexpr int32_t kPlanMagic = 0x53475041;  // "SGPA"
constexpr float kLog2e = 1.4426950408889634f;

struct PlanHeader {
  int32_t magic;
  int32_t num_units;
  int32_t num_merges;
  int32_t rows_per_tile;
  int32_t head_dim;
  int32_t group;
  int32_t num_partials;
  int32_t reserved[9];
};
static_assert(sizeof(PlanHeader) == 64, "plan header is 64 bytes");

struct AttnUnit {
  int32_t req;
  int32_t kv_head;
  int32_t row_begin;
  int32_t row_count;
  int32_t key_begin;
  int32_t key_end;
  int32_t partial;  // -1: write the final output
  int32_t flags;    // bit 0: attend to the request's tree rows
};

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

__host__ __device__ constexpr size_t partial_floats(int head_dim) {
  return static_cast<size_t>(kQPerUnit) * (head_dim + 2);
}

// LDS row of key k inside its 32-key block (inverse of pi).
__device__ __forceinline__ int key_slot(int k) {
  return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

template <int D>
struct TileRegs {
  uint4 k[D / 32];  // 64 keys * D/8 chunks / 256 threads
  uint4 v[4];       // 4 consecutive keys of one 8-wide head-dim chunk
};

template <int D>
__global__ __launch_bounds__(kAttnThreads, 2) void tree_attn_kernel(SgTreeAttnArgs a) {
  constexpr int KB = D / 16;       // QK^T k-blocks
  constexpr int DB = D / 32;       // PV d-blocks
  constexpr int DC = D / 8;        // 16-byte chunks per row
  constexpr int KS = D + 8;        // K row stride in LDS (bf16)
  constexpr int VS = kKeyTile + 8; // V^T row stride in LDS (bf16)
  constexpr int KLOADS = D / 32;
  __shared__ __align__(16) uint16_t s_k[2][kKeyTile * KS];
  __shared__ __align__(16) uint16_t s_v[2][D * VS];
  __shared__ uint32_t s_anc[kQPerUnit][kAncWords];
  __shared__ int s_parent[kMaxTreeRows];

  const PlanHeader* hdr = static_cast<const PlanHeader*>(a.plan_dev);
  const AttnUnit u = reinterpret_cast<const AttnUnit*>(hdr + 1)[blockIdx.x];
  const int G = a.num_q_heads / a.num_kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int col = lane & 31;
  const int m = wave * 32 + col;        // query vector inside the unit
  const int r_local = m / G;            // query row inside the tile
  const int head = u.kv_head * G + (m - r_local * G);
  const bool q_valid = r_local < u.row_count;
  const int r0 = a.row_offset_dev[u.req];
  const int n = a.row_offset_dev[u.req + 1] - r0;
  const int64_t row = static_cast<int64_t>(r0) + u.row_begin + r_local;
  const int g = u.kv_head;
  const bool do_tree = (u.flags & 1) != 0;

  // Ancestor-or-self bitsets of the tile's rows (request-local numbering).
  if (do_tree) {
    for (int k = tid; k < n; k += kAttnThreads) s_parent[k] = a.parent_dev[r0 + k];
    for (int k = tid; k < kQPerUnit * kAncWords; k += kAttnThreads) (&s_anc[0][0])[k] = 0u;
    __syncthreads();
    if (tid < u.row_count) {
      int node = u.row_begin + tid;
      uint32_t bits[kAncWords];
#pragma unroll
      for (int w = 0; w < kAncWords; ++w) bits[w] = 0u;
      for (int guard = 0; node >= 0 && guard < kMaxTreeRows; ++guard) {
        bits[node >> 5] |= 1u << (node & 31);
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
  const int tiles_prefix = (prefix_keys + kKeyTile - 1) / kKeyTile;
  const int tiles_tree = do_tree ? (n + kKeyTile - 1) / kKeyTile : 0;
  const int tiles = tiles_prefix + tiles_tree;
  const int64_t prefix_token0 = a.prefix_start_dev[u.req] + u.key_begin;
  const uint16_t* kc = static_cast<const uint16_t*>(a.k_cache_dev) + g * a.cache_head_stride;
  const uint16_t* vc = static_cast<const uint16_t*>(a.v_cache_dev) + g * a.cache_head_stride;
  const uint16_t* kt = static_cast<const uint16_t*>(a.k_tree_dev) + g * a.tree_head_stride;
  const uint16_t* vt = static_cast<const uint16_t*>(a.v_tree_dev) + g * a.tree_head_stride;

  auto key_address = [&](bool tree, int key, const uint16_t* cache, const uint16_t* tree_base,
                         int t) -> const uint16_t* {
    if (!tree) return cache + (prefix_token0 + static_cast<int64_t>(t) * kKeyTile + key) * a.cache_token_stride;
    return tree_base + (static_cast<int64_t>(r0) + (t - tiles_prefix) * kKeyTile + key) * a.tree_row_stride;
  };

  TileRegs<D> regs;
  auto load_tile = [&](int t) {
    const bool tree = t >= tiles_prefix;
    const int limit = tree ? n - (t - tiles_prefix) * kKeyTile : prefix_keys - t * kKeyTile;
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = tid + kAttnThreads * i;
      const int key = c / DC;
      const int dc = c - key * DC;
      regs.k[i] = key < limit
                      ? *reinterpret_cast<const uint4*>(key_address(tree, key, kc, kt, t) + 8 * dc)
                      : zero4();
    }
    if (tid < 16 * DC) {
      const int kg = tid / DC;
      const int dc = tid - kg * DC;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int key = 4 * kg + kk;
        regs.v[kk] = key < limit
                         ? *reinterpret_cast<const uint4*>(key_address(tree, key, vc, vt, t) + 8 * dc)
                         : zero4();
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = tid + kAttnThreads * i;
      const int key = c / DC;
      const int dc = c - key * DC;
      const int slot = (key & ~31) + key_slot(key & 31);
      *reinterpret_cast<uint4*>(&s_k[buf][slot * KS + 8 * dc]) = regs.k[i];
    }
    if (tid < 16 * DC) {
      const int kg = tid / DC;
      const int dc = tid - kg * DC;
      const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&regs.v[0]);
      const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&regs.v[1]);
      const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&regs.v[2]);
      const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&regs.v[3]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int sh = (e & 1) * 16;
        const uint32_t x0 = (w0[e >> 1] >> sh) & 0xffffu;
        const uint32_t x1 = (w1[e >> 1] >> sh) & 0xffffu;
        const uint32_t x2 = (w2[e >> 1] >> sh) & 0xffffu;
        const uint32_t x3 = (w3[e >> 1] >> sh) & 0xffffu;
        const int d = 8 * dc + e;
        const int vrow = (d & ~31) + key_slot(d & 31);
        uint2 packed;
        packed.x = x0 | (x1 << 16);
        packed.y = x2 | (x3 << 16);
        *reinterpret_cast<uint2*>(&s_v[buf][vrow * VS + 4 * kg]) = packed;
      }
    }
  };

  const float sl2 = a.scale * kLog2e;
  float m_run = -__builtin_inff();
  float l_run = 0.0f;
  floatx16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;

  if (tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  for (int t = 0; t < tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < tiles) load_tile(t + 1);
    const bool tree = t >= tiles_prefix;
    const int key0 = tree ? (t - tiles_prefix) * kKeyTile : t * kKeyTile;
    const int limit = tree ? n : prefix_keys;

    float x[2][16];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      floatx16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
      const uint16_t* krow = &s_k[buf][(32 * blk + col) * KS + 8 * half];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const bf16x8 kf = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 16 * kb));
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kb], s, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = key0 + 32 * blk + 16 * half + r;
        bool visible = key < limit;
        if (tree && visible) visible = (s_anc[r_local < kQPerUnit ? r_local : 0][key >> 5] >> (key & 31)) & 1u;
        x[blk][r] = visible ? s[r] * sl2 : -__builtin_inff();
      }
    }
    float tmax = x[0][0];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, x[blk][r]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.0f;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[blk][r] = __builtin_amdgcn_exp2f(x[blk][r] - m_use);
        psum += x[blk][r];
      }
    psum += __shfl_xor(psum, 32);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;

#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        bf16x8 pf;
#pragma unroll
        for (int e = 0; e < 8; ++e) pf[e] = static_cast<__bf16>(x[blk][8 * c + e]);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const uint16_t* vrow = &s_v[buf][(32 * db + col) * VS + 32 * blk + 16 * half + 8 * c];
          const bf16x8 vf = as_bf16x8(*reinterpret_cast<const uint4*>(vrow));
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc[db], 0, 0, 0);
        }
      }
    }
    if (t + 1 < tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (!q_valid) return;
  if (u.partial < 0) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    uint16_t* op = static_cast<uint16_t*>(a.out_dev) + row * a.out_row_stride +
                   static_cast<int64_t>(head) * a.out_head_stride;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      uint4 lo, hi;
      lo.x = pack_bf16x2(acc[db][0] * inv, acc[db][1] * inv);
      lo.y = pack_bf16x2(acc[db][2] * inv, acc[db][3] * inv);
      lo.z = pack_bf16x2(acc[db][4] * inv, acc[db][5] * inv);
      lo.w = pack_bf16x2(acc[db][6] * inv, acc[db][7] * inv);
      hi.x = pack_bf16x2(acc[db][8] * inv, acc[db][9] * inv);
      hi.y = pack_bf16x2(acc[db][10] * inv, acc[db][11] * inv);
      hi.z = pack_bf16x2(acc[db][12] * inv, acc[db][13] * inv);
      hi.w = pack_bf16x2(acc[db][14] * inv, acc[db][15] * inv);
      uint16_t* dst = op + 32 * db + 16 * half;
      *reinterpret_cast<uint4*>(dst) = lo;
      *reinterpret_cast<uint4*>(dst + 8) = hi;
    }
  } else {
    float* part = static_cast<float*>(a.workspace_dev) + partial_floats(D) * u.partial;
    float* o = part + static_cast<size_t>(m) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      float4* dst = reinterpret_cast<float4*>(o + 32 * db + 16 * half);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        dst[k] = make_float4(acc[db][4 * k], acc[db][4 * k + 1], acc[db][4 * k + 2],
                             acc[db][4 * k + 3]);
    }
    if (half == 0) {
      part[static_cast<size_t>(kQPerUnit) * D + m] = m_run;
      part[static_cast<size_t>(kQPerUnit) * D + kQPerUnit + m] = l_run;
    }
  }
}

// Combines the split-K partials of one (request, kv head, tile).
template <int D>
__global__ __launch_bounds__(kAttnThreads) void tree_attn_merge_kernel(SgTreeAttnArgs a) {
  const PlanHeader* hdr = static_cast<const PlanHeader*>(a.plan_dev);
  const MergeGroup grp = reinterpret_cast<const MergeGroup*>(
      reinterpret_cast<const AttnUnit*>(hdr + 1) + hdr->num_units)[blockIdx.x];
  const int G = a.num_q_heads / a.num_kv_heads;
  const int r0 = a.row_offset_dev[grp.req];
  const float* ws = static_cast<const float*>(a.workspace_dev);
  constexpr int DC4 = D / 4;
  for (int item = threadIdx.x; item < kQPerUnit * DC4; item += kAttnThreads) {
    const int m = item / DC4;
    const int c = item - m * DC4;
    const int r_local = m / G;
    if (r_local >= grp.row_count) continue;
    const int head = grp.kv_head * G + (m - r_local * G);
    float mx = -__builtin_inff();
    for (int s = 0; s < grp.num_partials; ++s) {
      const float* part = ws + partial_floats(D) * (grp.first_partial + s);
      mx = fmaxf(mx, part[static_cast<size_t>(kQPerUnit) * D + m]);
    }
    const float m_use = (mx == -__builtin_inff()) ? 0.0f : mx;
    float l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < grp.num_partials; ++s) {
      const float* part = ws + partial_floats(D) * (grp.first_partial + s);
      const float w = __builtin_amdgcn_exp2f(part[static_cast<size_t>(kQPerUnit) * D + m] - m_use);
      l += w * part[static_cast<size_t>(kQPerUnit) * D + kQPerUnit + m];
      const float4 v = reinterpret_cast<const float4*>(part + static_cast<size_t>(m) * D)[c];
      o.x += w * v.x;
      o.y += w * v.y;
      o.z += w * v.z;
      o.w += w * v.w;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int64_t row = static_cast<int64_t>(r0) + grp.row_begin + r_local;
    uint16_t* dst = static_cast<uint16_t*>(a.out_dev) + row * a.out_row_stride +
                    static_cast<int64_t>(head) * a.out_head_stride + 4 * c;
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
  SG_REQUIRE(kQPerUnit % G == 0, "query heads per kv head must divide 128");
  SG_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128");
  SG_REQUIRE(plan_bytes && plan_units && plan_merges && workspace_bytes, "null output pointer");
  const int rows_per_tile = kQPerUnit / G;
  SG_REQUIRE(num_requests == 0 || row_offset_host[0] == 0, "row_offset[0] must be 0");

  int64_t work = 0;
  for (int i = 0; i < num_requests; ++i) {
    const int rows = row_offset_host[i + 1] - row_offset_host[i];
    SG_REQUIRE(rows >= 0 && rows <= kMaxTreeRows,
               "every request must have between 0 and 256 packed rows");
    SG_REQUIRE(prefix_len_host[i] >= 0, "prefix lengths must be non-negative");
    const int tiles = (rows + rows_per_tile - 1) / rows_per_tile;
    work += static_cast<int64_t>(num_kv_heads) * tiles * (prefix_len_host[i] + rows);
  }
  const int64_t target = target_units_hint > 0 ? target_units_hint : 1024;
  int64_t chunk = (work + target - 1) / std::max<int64_t>(target, 1);
  chunk = std::max<int64_t>(chunk, 512);
  chunk = (chunk + kKeyTile - 1) / kKeyTile * kKeyTile;

  std::vector<AttnUnit> units;
  std::vector<MergeGroup> merges;
  int32_t partials = 0;
  for (int i = 0; i < num_requests; ++i) {
    const int rows = row_offset_host[i + 1] - row_offset_host[i];
    if (rows == 0) continue;
    const int L = prefix_len_host[i];
    const int splits = std::max<int64_t>(1, (L + chunk - 1) / chunk);
    const int tiles = (rows + rows_per_tile - 1) / rows_per_tile;
    for (int g = 0; g < num_kv_heads; ++g) {
      for (int tile = 0; tile < tiles; ++tile) {
        const int row_begin = tile * rows_per_tile;
        const int row_count = std::min(rows_per_tile, rows - row_begin);
        const int first = partials;
        for (int s = 0; s < splits; ++s) {
          AttnUnit u;
          u.req = i;
          u.kv_head = g;
          u.row_begin = row_begin;
          u.row_count = row_count;
          u.key_begin = static_cast<int32_t>(static_cast<int64_t>(L) * s / splits / kKeyTile * kKeyTile);
          u.key_end = s + 1 == splits
                          ? L
                          : static_cast<int32_t>(static_cast<int64_t>(L) * (s + 1) / splits /
                                                 kKeyTile * kKeyTile);
          u.partial = splits > 1 ? partials++ : -1;
          u.flags = (s + 1 == splits) ? 1 : 0;
          units.push_back(u);
        }
        if (splits > 1) {
          MergeGroup mg;
          mg.req = i;
          mg.kv_head = g;
          mg.row_begin = row_begin;
          mg.row_count = row_count;
          mg.first_partial = first;
          mg.num_partials = splits;
          mg.pad0 = mg.pad1 = 0;
          merges.push_back(mg);
        }
      }
    }
  }
  // Longest units first: the dispatcher hands out workgroups in order.
  std::vector<int64_t> cost(units.size());
  for (size_t k = 0; k < units.size(); ++k) {
    const int rows = row_offset_host[units[k].req + 1] - row_offset_host[units[k].req];
    cost[k] = (units[k].key_end - units[k].key_begin) + ((units[k].flags & 1) ? rows : 0);
  }
  std::vector<size_t> order(units.size());
  std::iota(order.begin(), order.end(), size_t{0});
  std::stable_sort(order.begin(), order.end(),
                   [&](size_t x, size_t y) { return cost[x] > cost[y]; });

  const size_t bytes = sizeof(PlanHeader) + sizeof(AttnUnit) * units.size() +
                       sizeof(MergeGroup) * merges.size();
  *plan_bytes = bytes;
  *plan_units = static_cast<int32_t>(units.size());
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
  char* out = static_cast<char*>(plan_host);
  std::memcpy(out, &hdr, sizeof(hdr));
  AttnUnit* uo = reinterpret_cast<AttnUnit*>(out + sizeof(hdr));
  for (size_t k = 0; k < order.size(); ++k) uo[k] = units[order[k]];
  std::memcpy(uo + units.size(), merges.data(), sizeof(MergeGroup) * merges.size());
  return SG_OK;
}

extern "C" int sg_tree_attn_fwd(const SgTreeAttnArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null SgTreeAttnArgs");
  const SgTreeAttnArgs& a = *args;
  SG_REQUIRE(a.num_kv_heads >= 1 && a.num_q_heads % a.num_kv_heads == 0 &&
                 kQPerUnit % (a.num_q_heads / a.num_kv_heads) == 0,
             "invalid head configuration");
  SG_REQUIRE(a.head_dim == 64 || a.head_dim == 128, "head_dim must be 64 or 128");
  SG_REQUIRE(a.plan_units >= 0 && a.plan_merges >= 0, "negative plan sizes");
  if (a.plan_units == 0) return SG_OK;
  SG_REQUIRE(a.q_dev && a.k_cache_dev && a.v_cache_dev && a.k_tree_dev && a.v_tree_dev &&
                 a.row_offset_dev && a.prefix_start_dev && a.parent_dev && a.out_dev &&
                 a.plan_dev,
             "null device pointer");
  SG_REQUIRE(a.plan_merges == 0 || a.workspace_dev, "split plan needs a workspace");
  SG_REQUIRE(a.q_row_stride % 8 == 0 && a.q_head_stride % 8 == 0 &&
                 a.cache_head_stride % 8 == 0 && a.cache_token_stride % 8 == 0 &&
                 a.tree_row_stride % 8 == 0 && a.tree_head_stride % 8 == 0 &&
                 a.out_row_stride % 8 == 0 && a.out_head_stride % 8 == 0,
             "strides must be multiples of 8 elements (16-byte rows)");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a.head_dim == 128) {
    hipLaunchKernelGGL(tree_attn_kernel<128>, dim3(a.plan_units), dim3(kAttnThreads), 0, s, a);
    SG_LAUNCH_CHECK();
    if (a.plan_merges > 0) {
      hipLaunchKernelGGL(tree_attn_merge_kernel<128>, dim3(a.plan_merges), dim3(kAttnThreads),
                         0, s, a);
      SG_LAUNCH_CHECK();
    }
  } else {
    hipLaunchKernelGGL(tree_attn_kernel<64>, dim3(a.plan_units), dim3(kAttnThreads), 0, s, a);
    SG_LAUNCH_CHECK();
    if (a.plan_merges > 0) {
      hipLaunchKernelGGL(tree_attn_merge_kernel<64>, dim3(a.plan_merges), dim3(kAttnThreads),
                         0, s, a);
      SG_LAUNCH_CHECK();
    }
  }
  return SG_OK;
}
