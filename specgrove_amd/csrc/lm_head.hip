// Vocabulary projection of a packed verification wave with fused row
// statistics (the "lazy projection" LM head).
//
// Replaces the reference's `lm_head(hidden)` followed by `probabilities(...)`
// on the rows the tree walk can need (fused_tree_sampling.py:2899-2913 for the
// internal rows of every request, :2974-2984 for the reached leaves;
// sampling.py:738-832 for the single-request law): the wave's hidden rows,
// gathered by index, are multiplied by the bf16 head weight; the kernel writes
// the bf16 logits and, from those rounded logits, the softmax statistics that
// the tree walk routes with, so no separate pass reads the logits to normalise
// them.
//
// Kernels: lm_head_pp_kernel for more than 128 projected rows (eight waves
// in two groups that alternate between the matrix pipe and the LDS/copy
// pipes, described at the kernel), lm_head_kernel<R> for up to 128 rows and
// for hidden sizes of 64 (one 4-wave workgroup per CU, 1 wave per SIMD):
//   tile      = 256 vocabulary tokens x 64 R projected rows; wave w owns the
//               128 x 32 R quarter (tokens 128*(w&1).., rows 32 R (w>>1)..);
//               the tiles of a last, partial round of workgroups run as
//               128-token halves (wave w: rows 16 R w ..) when R <= 2;
//   ring      = four stages of 32 hidden dims: the weight and hidden chunks
//               move HBM -> LDS with global_load_lds_dwordx4 (no register
//               staging), 64 contiguous bytes of each row per copy lane
//               group, three stages ahead of the MFMAs; a stage's copies,
//               its fragment reads for the next stage and its MFMAs are
//               interleaved in four parts, so that the four waves' LDS
//               traffic does not queue up right after the barrier;
//   product   = C^T = W X^T with v_mfma_f32_16x16x32_bf16 (A = weight rows,
//               B = hidden rows; one product per 16 x 16 block and 32-dim
//               stage), so each lane ends with 32 logits of one row per
//               16-row block (4 consecutive tokens of each 16), fp32-
//               accumulated over the stages in ascending order (the same
//               values, bit for bit, as 32x32x16 products over 16-dim
//               halves gave; the 16x16 shape draws less power, and the GPU
//               holds a higher clock under it);
//   epilogue  = round to bf16 (nearest even), per (row, 128-token tile) the
//               maximum m and z = sum of E(x - m) (the sampler's exp) in the
//               order below, and the bf16 logits written as whole 256-byte
//               row segments through LDS;
//   grid      = XCD-aware: the row tiles of one vocabulary tile run on one XCD
//               at the same time, so its L2 serves the weight tile to all of
//               them.
// A second small kernel merges each row's tile pairs into (max, sum).
//
// Statistics contract (bit-exact with the CPU restatement, fp32, contraction
// off).  Row r, tile t covers tokens 128*t .. 128*t+127 below V.  Token
// 128*t + 32*b + 8*q + 4*h + e (b, q, e in 0..3, h in 0..1) belongs to half
// h.  m_t = max of the tile; z_h = sequential sum, in increasing (b, q, e),
// of E(x - m_t) over the half's tokens below V; z_t = z_0 + z_1.  Row pair:
// tile t is merged into lane t % 64 in increasing t, then an xor butterfly
// (distances 32 .. 1) merges the 64 lanes; merge(a, b) = (M, a.z*E(a.m-M) +
// b.z*E(b.m-M)) with M = max(a.m, b.m).
#pragma clang fp contract(off)

#include <algorithm>
#include <climits>
#include <type_traits>

#include "sg_common.h"
#include "sg_math.h"

namespace sg {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float floatx16;
typedef __attribute__((ext_vector_type(4))) float floatx4;

constexpr int kLmThreads = 256;
constexpr int kTileV = 256;          // vocabulary tokens per workgroup tile
constexpr int kStepK = 32;           // hidden dims per ring stage
constexpr int kLmStages = 4;
constexpr int kWBytes = kTileV * kStepK * 2;  // weight bytes per stage (16 KiB)
constexpr int kStatTokens = 128;     // tokens per statistics tile
constexpr int kOutPitch = 2 * 128 + 16;  // LDS staging row: 128 bf16 + 16 bytes
constexpr int kLmXcds = 8;
constexpr int kMergeRowsPerBlock = 4;   // rows per 256-thread merge workgroup

// Row tile of 32R rows per wave (64R projected rows per workgroup):
// R = 2 up to 128 rows, 1 up to 64 (the leaf pass), so a small call does not
// multiply empty rows; R = 4 only where the ping-pong kernel cannot run (a
// hidden size of 64, two stages).
// kHalf (R = 1, 2): a workgroup takes one 128-token half of a tile and wave
// w rows 16 R w .. +16 R of the 64 R, for the tiles of the last, partial
// round of workgroups (each logit and each statistics tile is computed by one
// wave in the same order, so the results are the same bit for bit).
template <int R, bool kHalf = false>
struct RowTile {
  static constexpr int kTok = kHalf ? kTileV / 2 : kTileV;  // tokens per workgroup
  static constexpr int kWB = kTok * kStepK * 2;             // weight bytes per stage
  static constexpr int kWCopies = kTok / 64;                // weight copies per wave per stage
  static constexpr int kRows = 64 * R;
  static constexpr int kWaveRows = kHalf ? 16 * R : 32 * R;  // projected rows per wave
  static constexpr int kNB = kWaveRows / 16;                // 16-row blocks per wave
  static constexpr int kXBytes = kRows * kStepK * 2;        // hidden bytes per stage
  static constexpr int kStage = kWB + kXBytes;
  static constexpr int kDmas = kWCopies + R;                // copies per wave per stage
  static constexpr int kStaging = 4 * kWaveRows * kOutPitch;
  static constexpr int kLds = kLmStages * kStage > kStaging ? kLmStages * kStage : kStaging;
  static constexpr int kBlocksPerCU = R == 1 ? 2 : 1;
};
static_assert(RowTile<1, true>::kLds <= RowTile<1>::kLds &&
                  RowTile<2, true>::kLds <= RowTile<2>::kLds,
              "half tiles share the kernel's LDS");
// Workgroup slots of one round (256 CUs): tiles beyond the last whole round
// run as half tiles.
constexpr int kRoundCUs = 256;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// 16-byte HBM -> LDS copy of every lane: lane i's bytes at gbase + voff land
// at LDS byte lds + 16*i.  Inline assembly, so that the compiler neither
// models it nor inserts waits for it; the kernel waits explicitly (s_waitcnt
// vmcnt) before the barrier that publishes a stage.  m0 (the LDS base of the
// copy) is written here and declared clobbered.
__device__ __forceinline__ void dma16(const void* gbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(gbase)
               : "memory", "m0");
}
// The same copy with the non-temporal hint: the line is not kept for reuse.
__device__ __forceinline__ void dma16_nt(const void* gbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
               :
               : "s"(lds), "v"(voff), "s"(gbase)
               : "memory", "m0");
}
// Weight copies.  Calls of at most 128 rows have one row tile, so every
// weight byte is read once: with the packed layout (whole 1 KiB copies) they
// carry the non-temporal hint (64-row leaf pass 256 -> 239 us, 128 rows
// 319 -> 311 us).  Row-major copies read half of each 128-byte line per
// stage and need the line kept for the next stage's half (the hint made
// them 44 % slower); larger calls re-read each weight tile from L2.
template <int R, bool kPacked>
__device__ __forceinline__ void dma16_weight(const void* gbase, uint32_t voff, uint32_t lds) {
  if constexpr (kPacked && R <= 2) {
    dma16_nt(gbase, voff, lds);
  } else {
    dma16(gbase, voff, lds);
  }
}

// s_waitcnt immediate: vmcnt <= n, the other counters unconstrained.
constexpr int vmcnt_encoding(int n) {
  return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// max / sum of a value with the same lane of the other 32-lane half (the
// same bits in both lanes: both operations are symmetric).
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

// Two fp32 values to a packed bf16 pair (low half: lo), nearest-even
// rounding by v_cvt_pk_bf16_f32; for the finite values this library rounds
// it equals f32_to_bf16 bit for bit.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
  const f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// Epilogue of one 16-row block of a wave's 128-token statistics tile.  Lane
// (g, n) = (lane / 16, lane % 16) holds in acc[tb][rb][i] row n of the block
// at token tok0 + 16 tb + 4 g + i (the 16x16 MFMA output layout).  Rounds
// them to bf16, writes the bf16 logits into the lane's staging row (128
// tokens) and returns the tile's (m, z) of the statistics contract: m the
// maximum (every lane), z = z_0 + z_1 (lanes g < 2) with z_h the sum of
// E(x - m) over the half's tokens (bit 2 of the token = h) in increasing
// token order.  A half's tokens alternate between lanes g = h and g = h + 2
// in runs of four, so the lower lanes take the upper lanes' values and add
// them in that order.  kFull: every token of the tile is below V, so no
// token needs a mask (the masks are 64-bit lane masks per token, and 32 of
// them do not fit the scalar registers).
template <bool kFull, int NB>
__device__ __forceinline__ float2 block_epilogue(const floatx4 (&acc)[8][NB], int rb, int tok0,
                                                 int V, int g, unsigned char* stage_row) {
  float x[32];
#pragma unroll
  for (int tb = 0; tb < 8; ++tb)
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      const uint32_t pr = cvt_pk_bf16(acc[tb][rb][i], acc[tb][rb][i + 1]);
      x[4 * tb + i] = __uint_as_float(pr << 16);
      x[4 * tb + i + 1] = __uint_as_float(pr & 0xffff0000u);
    }
  auto live = [&](int tb, int i) { return kFull || tok0 + 16 * tb + 4 * g + i < V; };
  float m = -__builtin_inff();
#pragma unroll
  for (int tb = 0; tb < 8; ++tb)
#pragma unroll
    for (int i = 0; i < 4; ++i) m = live(tb, i) ? fmaxf(m, x[4 * tb + i]) : m;
  m = fmaxf(m, __shfl_xor(m, 16));
  m = half_max(m);
  // Tokens at or past V add exactly 0 (z stays a non-negative sum).
  const float mc = (m == -__builtin_inff()) ? 0.0f : m;
  float z = 0.0f;
#pragma unroll
  for (int tb = 0; tb < 8; ++tb) {
    float e[4], pe[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = sg_exp_nonpos(x[4 * tb + i] - mc);
      e[i] = live(tb, i) ? v : 0.0f;
    }
    // Lanes 0..31 receive lanes 32..63's values (the same tokens + 8).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(e[i]),
                                                      __float_as_uint(e[i]), false, false);
      pe[i] = __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) z = z + e[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) z = z + pe[i];
  }
  z = z + __shfl_xor(z, 16);  // z_0 + z_1 in lanes g = 0 and g = 1
  // bf16 logits into the staging row (LDS rows of 128 tokens); x is already
  // bf16, so packing keeps its upper halves.
  auto pack = [&](int i) {
    return __builtin_amdgcn_perm(__float_as_uint(x[i + 1]), __float_as_uint(x[i]), 0x07060302u);
  };
#pragma unroll
  for (int tb = 0; tb < 8; ++tb)
    *reinterpret_cast<uint2*>(stage_row + 2 * (16 * tb + 4 * g)) =
        make_uint2(pack(4 * tb), pack(4 * tb + 2));
  return make_float2(m, z);
}

// Workgroup b -> (vocabulary tile, row tile): the dispatcher places b on XCD
// b % 8, and the row tiles of one vocabulary tile take consecutive slots of
// one XCD.
__device__ __forceinline__ bool tile_of(int b, int v_tiles, int r_tiles, int& vt, int& rt) {
  const int xcd = b % kLmXcds;
  const int slot = b / kLmXcds;
  rt = slot % r_tiles;
  vt = (slot / r_tiles) * kLmXcds + xcd;
  return vt < v_tiles;
}

// kPacked: the weight is in the packed layout of sg_lm_head_pack_weight
// (tile, 32-dim stage, 256 rows x 32 dims): every stage of a tile is 16 KiB
// contiguous and every copy a contiguous 1 KiB.  Otherwise the weight is
// row-major [V, weight_row_stride] and a copy reads 64 bytes of each of 16
// rows.  The arithmetic is the same, so are the results.
// One workgroup's tile: vocabulary tile vt (its 128-token half `half` when
// kHalf), row tile rt.
template <int R, bool kPacked, bool kHalf>
__device__ __forceinline__ void lm_tile(const SgLmHeadArgs& a, unsigned char* smem, int vt, int rt,
                                        int half) {
  using T = RowTile<R, kHalf>;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int V = a.vocab;
  const int v0 = vt * kTileV + T::kTok * half;
  const int r0 = rt * T::kRows;
  // The second half of the last tile can lie wholly past the vocabulary: no
  // token, no copy (its weight offsets would start before the tile).
  if (kHalf && v0 >= V) return;

  // DMA slots.  Per stage the weight is 4 kWCopies copies of 1 KiB (wave w
  // issues kWCopies w .. +kWCopies-1: 16 for a whole tile, 8 for a half) and
  // the hidden rows 4R (wave w issues Rw .. Rw+R-1).  LDS
  // layout of an operand stage: rows of 64 bytes (the stage's 32 dims) whose
  // 16-byte chunk c sits at chunk c ^ swz(row), swz(row) = (row >> 1) & 3:
  // a fragment read (lane l: row l%16 of a 16-row block, chunk l/16) then
  // runs without LDS bank conflicts (measured with the bank-conflict counter:
  // (row >> 2) & 3, row & 3 and no swizzle each cost 4 conflict cycles per
  // read instruction of this pattern).  A copy lane reads 16 contiguous
  // bytes and four lanes one row's 64 bytes: every copy touches 16 cache
  // lines instead of 32.
  constexpr int kWc = T::kWCopies;
  uint32_t w_off[kWc], w_lds[kWc], x_off[R], x_lds[R];
  const int steps = a.hidden_size / kStepK;
  const unsigned char* wbase =
      static_cast<const unsigned char*>(a.weight_dev) +
      (kPacked ? static_cast<int64_t>(vt) * steps * kWBytes + T::kTok * kStepK * 2 * half
               : static_cast<int64_t>(v0) * a.weight_row_stride * 2);
  // Bytes between a tile's consecutive stages.
  constexpr int64_t kWStep = kPacked ? kWBytes : kStepK * 2;
  const unsigned char* xbase = static_cast<const unsigned char*>(a.hidden_dev);
  bool bad_index = false;
  // Copy q moves rows 16q .. 16q+15 of an operand, 64 bytes (the stage's 32
  // dims) of each: lane i reads row 16q + i/4, 16-byte chunk (i%4) ^ swz(row),
  // and lands at LDS chunk i%4 of that row.
  const int g_lane = (lane & 3) ^ ((lane >> 3) & 3);  // swz(row) = (row >> 1) & 3
#pragma unroll
  for (int i = 0; i < kWc; ++i) {
    const int q = wave * kWc + i;
    const int row = 16 * q + (lane >> 2);
    const int dim = 8 * g_lane;
    // Tokens past the vocabulary re-read the last token (finite data the
    // epilogue drops).
    const int tok = min(v0 + row, V - 1) - v0;
    w_off[i] = kPacked ? static_cast<uint32_t>(row * kStepK * 2 + dim * 2)
                       : static_cast<uint32_t>((static_cast<int64_t>(tok) * a.weight_row_stride +
                                                dim) * 2);
    w_lds[i] = static_cast<uint32_t>(1024 * q);
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int q = wave * R + i;
    const int row = 16 * q + (lane >> 2);
    const int dim = 8 * g_lane;
    // Rows past the projected rows re-read a valid row.
    const int prow = min(r0 + row, a.num_rows - 1);
    int src = a.row_index_dev != nullptr ? a.row_index_dev[prow] : prow;
    if (src < 0 || src >= a.num_hidden_rows) {
      bad_index = bad_index || (r0 + row < a.num_rows);
      src = 0;
    }
    x_off[i] = static_cast<uint32_t>((static_cast<int64_t>(src) * a.hidden_row_stride + dim) * 2);
    x_lds[i] = static_cast<uint32_t>(T::kWB + 1024 * q);
  }
  if (bad_index && a.status_dev != nullptr) atomicExch(a.status_dev, SG_EINVAL);

  const uint32_t ring = lds_addr(smem);
  auto issue = [&](int s) {
    const uint32_t stage = ring + (s % kLmStages) * T::kStage;
    const unsigned char* wk = wbase + static_cast<int64_t>(s) * kWStep;
    const unsigned char* xk = xbase + static_cast<int64_t>(s) * kStepK * 2;
#pragma unroll
    for (int i = 0; i < kWc; ++i) dma16_weight<R, kPacked>(wk, w_off[i], stage + w_lds[i]);
#pragma unroll
    for (int i = 0; i < R; ++i) dma16(xk, x_off[i], stage + x_lds[i]);
  };

  // Products: v_mfma_f32_16x16x32_bf16, one per (16-token block, 16-row
  // block) per stage (all 32 dims of the stage): acc[tb][rb][i] accumulates
  // token 16 tb + 4 g + i of this wave's 128 and row 16 rb + n of its
  // kWaveRows, g = lane / 16, n = lane % 16, over the stages in ascending
  // order.
  constexpr int NB = T::kNB;  // 16-row blocks of this wave
  floatx4 acc[8][NB];
#pragma unroll
  for (int tb = 0; tb < 8; ++tb)
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) acc[tb][rb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int wv = kHalf ? 0 : wave & 1;      // 128-token half of the tile
  const int wr = kHalf ? wave : wave >> 1;  // this wave's rows: kWaveRows wr ..
  const int g = lane >> 4;
  // Fragment of a 16-row block for lane l: row l%16 of the block, 16-byte
  // chunk l/16 (dims 8 (l/16) .. +7 of the stage), stored at LDS chunk
  // (l/16) ^ swz(l%16) of the 64-byte row (16-row blocks start at multiples
  // of 16 rows, so swz of the block row is swz(l%16)).
  const int lq = (lane & 15) * 64 + 16 * (g ^ (((lane & 15) >> 1) & 3));
  const int a_base = wv * 8 * 1024;        // this wave's 128 token rows
  const int b_base = T::kWB + wr * NB * 1024;  // this wave's hidden rows

  // Operand fragments of one stage, read from LDS one stage ahead of their
  // MFMAs.
  struct Frags {
    bf16x8 a[8];
    bf16x8 b[NB];
  };
  auto frag = [&](const unsigned char* st, int base, int blk) {
    return as_bf16x8(*reinterpret_cast<const uint4*>(st + base + blk * 1024 + lq));
  };
  auto load_frags = [&](int s, Frags& f) {
    const unsigned char* st = smem + (s % kLmStages) * T::kStage;
#pragma unroll
    for (int tb = 0; tb < 8; ++tb) f.a[tb] = frag(st, a_base, tb);
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) f.b[rb] = frag(st, b_base, rb);
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int tb = 0; tb < 8; ++tb)
#pragma unroll
      for (int rb = 0; rb < NB; ++rb)
        acc[tb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a[tb], f.b[rb], acc[tb][rb], 0, 0, 0);
  };
  for (int s = 0; s < kLmStages - 1 && s < steps; ++s) issue(s);
  // Stage s: wait for its copies (only the up to two later stages' remain in
  // flight) and publish it with the barrier, which also ends every wave's
  // reads of stage s-1.
  auto wait_stage = [&](int s) {
    const int newer = min(kLmStages - 2, steps - 1 - s);
    if (newer >= 2) {
      __builtin_amdgcn_s_waitcnt(vmcnt_encoding(2 * T::kDmas));
    } else if (newer == 1) {
      __builtin_amdgcn_s_waitcnt(vmcnt_encoding(T::kDmas));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_encoding(0));
    }
    __syncthreads();
  };
  // Stage s in four parts p (two 16-token weight blocks each): the MFMAs of
  // stage s-1's dims (fragments `cur`, read during stage s-1), a quarter of
  // the fragment reads of stage s (into `next`) placed one after each of the
  // part's first MFMAs, and a quarter of the copies that refill stage s-1's
  // slot with stage s+3.
  auto run_stage = [&](int s, Frags& next, const Frags& cur) {
    wait_stage(s);
    const bool refill = s + kLmStages - 1 < steps;
    const int t = s + kLmStages - 1;
    const uint32_t stage_t = ring + (t % kLmStages) * T::kStage;
    const unsigned char* wk = wbase + static_cast<int64_t>(t) * kWStep;
    const unsigned char* xk = xbase + static_cast<int64_t>(t) * kStepK * 2;
    const unsigned char* st = smem + (s % kLmStages) * T::kStage;
    constexpr int nd = kWc + R;
    auto part = [&](auto pc) {
      constexpr int p = decltype(pc)::value;
      // Reads: weight blocks 2p, 2p+1 and the hidden blocks j = p (mod 4).
      constexpr int kReads = 2 + (NB > p ? (NB - p + 3) / 4 : 0);
      constexpr int kMfmas = 2 * NB;
      constexpr int kPairs = kReads < kMfmas ? kReads : kMfmas;
      next.a[2 * p] = frag(st, a_base, 2 * p);
      next.a[2 * p + 1] = frag(st, a_base, 2 * p + 1);
#pragma unroll
      for (int j = p; j < NB; j += 4) next.b[j] = frag(st, b_base, j);
#pragma unroll
      for (int tb = 2 * p; tb < 2 * p + 2; ++tb)
#pragma unroll
        for (int rb = 0; rb < NB; ++rb)
          acc[tb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.a[tb], cur.b[rb], acc[tb][rb],
                                                                0, 0, 0);
#pragma unroll
      for (int k = 0; k < kPairs; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if constexpr (kMfmas > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfmas - kPairs, 0);
      if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPairs, 0);
      if (refill) {
#pragma unroll
        for (int d = p * nd / 4; d < (p + 1) * nd / 4; ++d) {
          if (d < kWc) {
            dma16_weight<R, kPacked>(wk, w_off[d], stage_t + w_lds[d]);
          } else {
            dma16(xk, x_off[d - kWc], stage_t + x_lds[d - kWc]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    part(std::integral_constant<int, 0>{});
    part(std::integral_constant<int, 1>{});
    part(std::integral_constant<int, 2>{});
    part(std::integral_constant<int, 3>{});
  };
  Frags f0, f1;
  wait_stage(0);
  if (kLmStages - 1 < steps) issue(kLmStages - 1);
  load_frags(0, f0);
  for (int s = 1; s + 1 < steps; s += 2) {
    run_stage(s, f1, f0);
    run_stage(s + 1, f0, f1);
  }
  wait_stage(steps - 1);
  load_frags(steps - 1, f1);
  mma(f0);
  mma(f1);
  __syncthreads();  // the ring is free: it becomes the output staging area

  // Epilogue, one 16-row block at a time.
  const int tok0 = v0 + 128 * wv;           // first token of this wave's statistics tile
  const bool tile_live = tok0 < V;
  const int n_tiles = (V + kStatTokens - 1) / kStatTokens;
  unsigned char* stage = smem + wave * T::kWaveRows * kOutPitch;
  auto epilogue = [&](auto full) {
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) {
      const int row_local = 16 * rb + (lane & 15);          // row inside this wave's rows
      const int row = r0 + T::kWaveRows * wr + row_local;  // projected row
      const float2 mz = block_epilogue<decltype(full)::value>(acc, rb, tok0, V, g,
                                                              stage + row_local * kOutPitch);
      if (g == 0 && tile_live && row < a.num_rows) {
        float* dst =
            a.tile_stats_dev + (static_cast<int64_t>(row) * n_tiles + tok0 / kStatTokens) * 2;
        *reinterpret_cast<float2*>(dst) = mz;
      }
      __builtin_amdgcn_sched_barrier(0);  // one 16-row block at a time (registers)
    }
  };
  if (tok0 + kStatTokens <= V) {
    epilogue(std::true_type{});
  } else {
    epilogue(std::false_type{});
  }
  __builtin_amdgcn_wave_barrier();
  // Row-contiguous read-back: every instruction moves four 256-byte row
  // segments (16 lanes x 16 bytes each).
  if (!tile_live) return;
  uint16_t* out = static_cast<uint16_t*>(a.logits_dev);
#pragma unroll 4
  for (int i = 0; i < T::kWaveRows / 4; ++i) {
    const int row_local = 4 * i + (lane >> 4);
    const int row = r0 + T::kWaveRows * wr + row_local;
    const int chunk = lane & 15;
    const int tok = tok0 + 8 * chunk;
    const uint4 v = *reinterpret_cast<const uint4*>(stage + row_local * kOutPitch + 16 * chunk);
    if (row >= a.num_rows || tok >= V) continue;
    uint16_t* dst = out + static_cast<int64_t>(row) * a.logits_row_stride + tok;
    if (tok + 8 <= V) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      for (int e = 0; tok + e < V; ++e) {
        const uint32_t w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
        dst[e] = static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
      }
    }
  }
}

// The 64- and 128-row kernels (R = 1, 2; one row tile) take the vocabulary
// tiles of every whole round of workgroups (256 CUs x kBlocksPerCU) as whole
// tiles (workgroup b: tile b) and split the tiles of the last, partial round
// into halves (workgroup full_blocks + 2k + h: half h of tile full_blocks +
// k), which would otherwise run one workgroup to a CU at the end of the
// launch (82 tiles of Qwen3-8B's 594 cost ~54 us of a 257 us leaf pass).
// full_blocks: every workgroup when no tile is split.
template <int R, bool kPacked>
__global__ __launch_bounds__(kLmThreads, RowTile<R>::kBlocksPerCU) void lm_head_kernel(
    SgLmHeadArgs a, int v_tiles, int r_tiles, int full_blocks) {
  __shared__ __align__(1024) unsigned char smem[RowTile<R>::kLds];
  if constexpr (R <= 2) {
    const int k = static_cast<int>(blockIdx.x) - full_blocks;
    if (k >= 0) {
      lm_tile<R, kPacked, true>(a, smem, full_blocks + k / 2, 0, k & 1);
      return;
    }
  }
  int vt, rt;
  if (!tile_of(blockIdx.x, v_tiles, r_tiles, vt, rt)) return;
  lm_tile<R, kPacked, false>(a, smem, vt, rt, 0);
}

// Ping-pong form of the 256-row tile (more than 128 projected rows): eight
// waves, two per SIMD, in two groups (waves 0-3 and 4-7) half a stage apart.
// Wave w owns tokens [128*(w&1), +128) and rows [64*(2*(w>>2) + ((w>>1)&1)),
// +64) of the 256 x 256 tile: 8 x 4 blocks of 16 x 16, 128 accumulators.  In
// phase 2t group A (waves 0-3) reads stage t's fragments from LDS and issues
// its share of the copies of stage t+3 while group B multiplies stage t-1; in
// phase 2t+1 the groups swap roles.  The two waves of a SIMD thus alternate
// between the matrix pipe and the LDS/copy pipes instead of meeting at the
// same barrier with the same work.  One barrier per phase; before it every
// wave waits for its own copies of the stage the next phase reads.  The
// products, their order per accumulator (ascending hidden dims) and the
// epilogue's statistics order are those of lm_head_kernel, so the logits and
// statistics are bit-identical.
constexpr int kPpThreads = 512;
struct PpTile {
  static constexpr int kRows = 256;
  static constexpr int kXBytes = kRows * kStepK * 2;  // hidden bytes per stage (16 KiB)
  static constexpr int kStage = kWBytes + kXBytes;     // 32 KiB
  static constexpr int kDmas = 4;                      // copies per wave per stage
  static constexpr int kStaging = 8 * 64 * kOutPitch;  // 64 rows x 128 tokens per wave
  static constexpr int kLds = kLmStages * kStage > kStaging ? kLmStages * kStage : kStaging;
};

template <bool kPacked>
__global__ __launch_bounds__(kPpThreads, 1) void lm_head_pp_kernel(SgLmHeadArgs a, int v_tiles,
                                                                    int r_tiles) {
  using T = PpTile;
  __shared__ __align__(1024) unsigned char smem[T::kLds];
  int vt, rt;
  if (!tile_of(blockIdx.x, v_tiles, r_tiles, vt, rt)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;               // 0: group A, 1: group B
  const int wv = wave & 1;                 // 128-token half of the tile
  const int wr = 2 * grp + ((wave >> 1) & 1);  // 64-row quarter of the tile
  const int g = lane >> 4;
  const int V = a.vocab;
  const int v0 = vt * kTileV;
  const int r0 = rt * T::kRows;

  // Copy slots, with the operand stage layout of lm_head_kernel: weight copy q
  // (rows 16q .. 16q+15, 64 bytes each) at LDS 1024 q, hidden copy q at
  // kWBytes + 1024 q; wave w issues weight and hidden copies 2w and 2w+1.
  uint32_t w_off[2], w_lds[2], x_off[2], x_lds[2];
  const int steps = a.hidden_size / kStepK;
  const unsigned char* wbase =
      static_cast<const unsigned char*>(a.weight_dev) +
      (kPacked ? static_cast<int64_t>(vt) * steps * kWBytes
               : static_cast<int64_t>(v0) * a.weight_row_stride * 2);
  constexpr int64_t kWStep = kPacked ? kWBytes : kStepK * 2;
  const unsigned char* xbase = static_cast<const unsigned char*>(a.hidden_dev);
  bool bad_index = false;
  const int g_lane = (lane & 3) ^ ((lane >> 3) & 3);  // swz(row) = (row >> 1) & 3
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = 2 * wave + i;
    const int row = 16 * q + (lane >> 2);
    const int dim = 8 * g_lane;
    const int tok = min(v0 + row, V - 1) - v0;
    w_off[i] = kPacked ? static_cast<uint32_t>(row * kStepK * 2 + dim * 2)
                       : static_cast<uint32_t>((static_cast<int64_t>(tok) * a.weight_row_stride +
                                                dim) * 2);
    w_lds[i] = static_cast<uint32_t>(1024 * q);
    const int prow = min(r0 + row, a.num_rows - 1);
    int src = a.row_index_dev != nullptr ? a.row_index_dev[prow] : prow;
    if (src < 0 || src >= a.num_hidden_rows) {
      bad_index = bad_index || (r0 + row < a.num_rows);
      src = 0;
    }
    x_off[i] = static_cast<uint32_t>((static_cast<int64_t>(src) * a.hidden_row_stride + dim) * 2);
    x_lds[i] = static_cast<uint32_t>(kWBytes + 1024 * q);
  }
  if (bad_index && a.status_dev != nullptr) atomicExch(a.status_dev, SG_EINVAL);

  const uint32_t ring = lds_addr(smem);
  auto issue = [&](int t) {
    const uint32_t stage = ring + (t % kLmStages) * T::kStage;
    const unsigned char* wk = wbase + static_cast<int64_t>(t) * kWStep;
    const unsigned char* xk = xbase + static_cast<int64_t>(t) * kStepK * 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(wk, w_off[i], stage + w_lds[i]);
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(xk, x_off[i], stage + x_lds[i]);
  };

  // Fragments as in lm_head_kernel: lane l reads row l%16 of a 16-row block,
  // chunk l/16, at LDS chunk (l/16) ^ swz(l%16).
  const int lq = (lane & 15) * 64 + 16 * (g ^ (((lane & 15) >> 1) & 3));
  const int a_base = wv * 8 * 1024;      // this wave's 128 token rows
  const int b_base = kWBytes + wr * 4 * 1024;  // this wave's 64 hidden rows
  // Waits until at most `newer` stages of this wave's copies are in flight.
  auto wait_newer = [&](int newer) {
    if (newer >= 2) {
      __builtin_amdgcn_s_waitcnt(vmcnt_encoding(2 * T::kDmas));
    } else if (newer == 1) {
      __builtin_amdgcn_s_waitcnt(vmcnt_encoding(T::kDmas));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_encoding(0));
    }
  };
  for (int t = 0; t < kLmStages - 1 && t < steps; ++t) issue(t);
  wait_newer(min(kLmStages - 2, steps - 1));  // stage 0 has landed
  __syncthreads();

  // The main loop and the epilogue, once per group (G known at compile time,
  // so each copy is straight-line code: no branch chooses between product
  // sites, which would make the compiler copy the accumulators).  A barrier
  // counts arrivals, not instructions: both copies pass 2 steps + 1 barriers.
  // Group A: phase 2t reads stage t and issues stage t+3, phase 2t+1
  // multiplies.  Group B: one idle phase, then phase 2t+1 reads stage t and
  // issues stage t+3, phase 2t+2 multiplies.  Before the barrier that ends
  // phase p every wave waits for its own copies of the stage read in phase
  // p+1, so that the barrier publishes the whole stage.
  auto body = [&](auto group) {
    constexpr int G = decltype(group)::value;
    // acc[tb][rb][i]: token 16 tb + 4 g + i of this wave's 128, row
    // 16 rb + n of its 64 (lm_head_kernel's products and order).
    floatx4 acc[8][4];
#pragma unroll
    for (int tb = 0; tb < 8; ++tb)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) acc[tb][rb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 fa[8], fb[4];
    auto read_frags = [&](int t) {
      const unsigned char* st = smem + (t % kLmStages) * T::kStage;
#pragma unroll
      for (int tb = 0; tb < 8; ++tb)
        fa[tb] = as_bf16x8(*reinterpret_cast<const uint4*>(st + a_base + tb * 1024 + lq));
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
        fb[rb] = as_bf16x8(*reinterpret_cast<const uint4*>(st + b_base + rb * 1024 + lq));
    };
    auto mma = [&]() {
#pragma unroll
      for (int tb = 0; tb < 8; ++tb)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
          acc[tb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[tb], fb[rb], acc[tb][rb], 0, 0,
                                                                0);
    };
    // One stage: read its fragments (and issue stage t+3 while steps remain),
    // multiply.  N is the number of this wave's stages newer than t+1 that
    // may stay in flight once stage t+1 must have landed (-1: t is the last
    // stage); a constant, so that the wait stays where it is written.
    auto stage_step = [&](int t, auto newer) {
      constexpr int N = decltype(newer)::value;
      auto wait_next = [&]() {
        if constexpr (N >= 2) {
          __builtin_amdgcn_s_waitcnt(vmcnt_encoding(2 * T::kDmas));
        } else if constexpr (N == 1) {
          __builtin_amdgcn_s_waitcnt(vmcnt_encoding(T::kDmas));
        } else if constexpr (N == 0) {
          __builtin_amdgcn_s_waitcnt(vmcnt_encoding(0));
        }
      };
      read_frags(t);
      if constexpr (N >= 2) issue(t + kLmStages - 1);
      // A: the next phase is B's read of stage t (landed).  B: the next phase
      // is A's read of stage t+1.
      if constexpr (G == 1) wait_next();
      // The scheduling fences keep every product inside its phase (the
      // compiler may otherwise move them across the barriers).
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      mma();
      __builtin_amdgcn_sched_barrier(0);
      // A: the next phase reads stage t+1.  B: the next phase is B's read of
      // stage t+1, landed before the barrier above.
      if constexpr (G == 0) wait_next();
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
    };
    static_assert(kLmStages == 4, "the tail below is written for a four-stage ring");
    if constexpr (G == 1) __syncthreads();  // phase 0: group A reads stage 0
    // steps >= 3 (the launcher's condition); stage t+3 exists for t < steps-3.
    for (int t = 0; t + kLmStages - 1 < steps; ++t) stage_step(t, std::integral_constant<int, 2>{});
    stage_step(steps - 3, std::integral_constant<int, 1>{});
    stage_step(steps - 2, std::integral_constant<int, 0>{});
    stage_step(steps - 1, std::integral_constant<int, -1>{});
    if constexpr (G == 0) __syncthreads();  // phase 2 steps: B's last products
    // The ring is free (every barrier above waited for the LDS reads): it
    // becomes the output staging area.

    // Epilogue (lm_head_kernel's, for the wave's four 16-row blocks).
    const int tok0 = v0 + 128 * wv;
    const bool tile_live = tok0 < V;
    const int n_tiles = (V + kStatTokens - 1) / kStatTokens;
    unsigned char* stage = smem + wave * 64 * kOutPitch;
    auto epilogue = [&](auto full) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const int row_local = 16 * rb + (lane & 15);
        const int row = r0 + 64 * wr + row_local;
        const float2 mz = block_epilogue<decltype(full)::value>(acc, rb, tok0, V, g,
                                                                stage + row_local * kOutPitch);
        if (g == 0 && tile_live && row < a.num_rows) {
          float* dst =
              a.tile_stats_dev + (static_cast<int64_t>(row) * n_tiles + tok0 / kStatTokens) * 2;
          *reinterpret_cast<float2*>(dst) = mz;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (tok0 + kStatTokens <= V) {
      epilogue(std::true_type{});
    } else {
      epilogue(std::false_type{});
    }
    __builtin_amdgcn_wave_barrier();
    if (!tile_live) return;
    uint16_t* out = static_cast<uint16_t*>(a.logits_dev);
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int row_local = 4 * i + (lane >> 4);
      const int row = r0 + 64 * wr + row_local;
      const int chunk = lane & 15;
      const int tok = tok0 + 8 * chunk;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + row_local * kOutPitch + 16 * chunk);
      if (row >= a.num_rows || tok >= V) continue;
      uint16_t* dst = out + static_cast<int64_t>(row) * a.logits_row_stride + tok;
      if (tok + 8 <= V) {
        *reinterpret_cast<uint4*>(dst) = v;
      } else {
        for (int e = 0; tok + e < V; ++e) {
          const uint32_t w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
          dst[e] = static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
        }
      }
    }
  };
  if (grp == 0) {
    body(std::integral_constant<int, 0>{});
  } else {
    body(std::integral_constant<int, 1>{});
  }
}

// Row (max, sum) from the tile pairs: one wave per row; lane l merges tiles
// l, l+64, ... in increasing order, then the xor butterfly merges the lanes.
__global__ __launch_bounds__(kMergeRowsPerBlock * kWave) void lm_head_rows_kernel(SgLmHeadArgs a) {
  const int row = blockIdx.x * kMergeRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= a.num_rows) return;
  const int n_tiles = (a.vocab + kStatTokens - 1) / kStatTokens;
  const float2* tiles =
      reinterpret_cast<const float2*>(a.tile_stats_dev) + static_cast<int64_t>(row) * n_tiles;
  MZ acc = {-__builtin_inff(), 0.0f};
  // The pairs are loaded 24 at a time before they are merged (the same
  // merges in the same order): up to 1,536 tiles (196,608 tokens) a row
  // costs one memory round trip instead of one per merge.
  constexpr int kBatch = 24;
  for (int t0 = lane; t0 < n_tiles; t0 += kWave * kBatch) {
    float2 p[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int t = t0 + kWave * j;
      p[j] = t < n_tiles ? tiles[t] : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (t0 + kWave * j < n_tiles) acc = merge_mz(acc, MZ{p[j].x, p[j].y});
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const MZ other = {__shfl_xor(acc.m, d), __shfl_xor(acc.z, d)};
    acc = merge_mz(acc, other);
  }
  if (lane == 0) {
    a.row_max_dev[row] = acc.m;
    a.row_sum_dev[row] = acc.z;
  }
}

// One 16 KiB stage of the packed weight per workgroup: packed stage
// (vt, s) row r dim d = weight[256 vt + r][32 s + d], zero for rows >= V.
// Thread t moves four 16-byte chunks: chunk c = t + 256 k is row c / 4,
// dims 8 (c % 4) .. +7.
__global__ __launch_bounds__(256) void lm_head_pack_kernel(const uint16_t* __restrict__ weight,
                                                           int64_t row_stride, int vocab,
                                                           int steps, uint16_t* __restrict__ packed) {
  const int vt = blockIdx.x / steps;
  const int s = blockIdx.x % steps;
  uint4* dst = reinterpret_cast<uint4*>(packed + static_cast<int64_t>(blockIdx.x) * kTileV * kStepK);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = threadIdx.x + 256 * k;
    const int row = kTileV * vt + c / 4;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < vocab)
      v = *reinterpret_cast<const uint4*>(weight + static_cast<int64_t>(row) * row_stride +
                                          kStepK * s + 8 * (c % 4));
    dst[c] = v;
  }
}

// Checks shared by both weight layouts; v_tiles and the launch follow.
int check_lm_head(const SgLmHeadArgs& a, bool packed) {
  SG_REQUIRE(a.num_hidden_rows >= 1, "num_hidden_rows must be positive");
  SG_REQUIRE(a.row_index_dev != nullptr || a.num_hidden_rows >= a.num_rows,
             "without a row index the hidden rows must cover every projected row");
  SG_REQUIRE(a.hidden_dev && a.weight_dev && a.logits_dev && a.tile_stats_dev &&
                 a.row_max_dev && a.row_sum_dev,
             "null device pointer");
  SG_REQUIRE(a.hidden_row_stride >= a.hidden_size &&
                 (packed || a.weight_row_stride >= a.hidden_size) &&
                 a.logits_row_stride >= a.vocab,
             "row strides must cover the rows");
  SG_REQUIRE((a.hidden_row_stride | (packed ? 0 : a.weight_row_stride) | a.logits_row_stride) %
                     8 == 0,
             "row strides must be multiples of 8 elements");
  SG_REQUIRE((reinterpret_cast<uintptr_t>(a.hidden_dev) | reinterpret_cast<uintptr_t>(a.weight_dev) |
              reinterpret_cast<uintptr_t>(a.logits_dev)) % 16 == 0,
             "hidden, weight and logits must be 16-byte aligned");
  // The per-lane copy offsets are 32-bit: a tile's weight rows and the whole
  // hidden matrix must each stay below 4 GiB.
  SG_REQUIRE(packed || static_cast<int64_t>(kTileV) * a.weight_row_stride * 2 < (int64_t{1} << 32),
             "weight rows too long");
  SG_REQUIRE(static_cast<int64_t>(a.num_hidden_rows) * a.hidden_row_stride * 2 < (int64_t{1} << 32),
             "hidden matrix above 4 GiB");
  return SG_OK;
}

int launch_lm_head(const SgLmHeadArgs& a, bool packed, hipStream_t s) {
  const int v_tiles = (a.vocab + kTileV - 1) / kTileV;
  auto launch = [&](auto tag) -> int {
    constexpr int R = decltype(tag)::value;
    const int r_tiles = (a.num_rows + RowTile<R>::kRows - 1) / RowTile<R>::kRows;
    int64_t blocks = static_cast<int64_t>((v_tiles + kLmXcds - 1) / kLmXcds) * kLmXcds * r_tiles;
    int full_blocks = static_cast<int>(std::min<int64_t>(blocks, INT32_MAX));
    constexpr int kSlots = kRoundCUs * RowTile<R>::kBlocksPerCU;
    if (R <= 2 && v_tiles > kSlots && v_tiles % kSlots != 0) {
      // Whole rounds as whole tiles, the last partial round as half tiles
      // (R <= 2: one row tile, so workgroup b of a whole round is tile b).
      full_blocks = v_tiles / kSlots * kSlots;
      blocks = full_blocks + 2 * static_cast<int64_t>(v_tiles - full_blocks);
    }
    SG_REQUIRE(blocks < INT32_MAX, "wave too large");
    if (packed) {
      lm_head_kernel<R, true><<<dim3(static_cast<unsigned>(blocks)), dim3(kLmThreads), 0, s>>>(
          a, v_tiles, r_tiles, full_blocks);
    } else {
      lm_head_kernel<R, false><<<dim3(static_cast<unsigned>(blocks)), dim3(kLmThreads), 0, s>>>(
          a, v_tiles, r_tiles, full_blocks);
    }
    SG_LAUNCH_CHECK();
    return SG_OK;
  };
  auto launch_pp = [&]() -> int {
    const int r_tiles = (a.num_rows + PpTile::kRows - 1) / PpTile::kRows;
    const int64_t blocks =
        static_cast<int64_t>((v_tiles + kLmXcds - 1) / kLmXcds) * kLmXcds * r_tiles;
    SG_REQUIRE(blocks < INT32_MAX, "wave too large");
    if (packed) {
      lm_head_pp_kernel<true><<<dim3(static_cast<unsigned>(blocks)), dim3(kPpThreads), 0, s>>>(
          a, v_tiles, r_tiles);
    } else {
      lm_head_pp_kernel<false><<<dim3(static_cast<unsigned>(blocks)), dim3(kPpThreads), 0, s>>>(
          a, v_tiles, r_tiles);
    }
    SG_LAUNCH_CHECK();
    return SG_OK;
  };
  // The ping-pong kernel's straight-line tail needs three stages or more.
  const bool pp = a.hidden_size / kStepK >= kLmStages - 1;
  const int rc = a.num_rows <= 64    ? launch(std::integral_constant<int, 1>{})
                 : a.num_rows <= 128 ? launch(std::integral_constant<int, 2>{})
                 : pp                ? launch_pp()
                                     : launch(std::integral_constant<int, 4>{});
  if (rc != SG_OK) return rc;
  const int merge_blocks = (a.num_rows + kMergeRowsPerBlock - 1) / kMergeRowsPerBlock;
  lm_head_rows_kernel<<<dim3(merge_blocks), dim3(kMergeRowsPerBlock * kWave), 0, s>>>(a);
  SG_LAUNCH_CHECK();
  return SG_OK;
}

}  // namespace
}  // namespace sg

extern "C" int64_t sg_lm_head_tile_count(int32_t vocab) {
  return vocab >= 1 ? (static_cast<int64_t>(vocab) + sg::kStatTokens - 1) / sg::kStatTokens : -1;
}

extern "C" int sg_lm_head(const SgLmHeadArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null args");
  const SgLmHeadArgs& a = *args;
  SG_REQUIRE(a.num_rows >= 0, "num_rows must be non-negative");
  SG_REQUIRE(a.vocab >= 1, "vocab must be positive");
  SG_REQUIRE(a.hidden_size >= 2 * kStepK && a.hidden_size % (2 * kStepK) == 0,
             "hidden_size must be a positive multiple of 64");
  if (a.num_rows == 0) return SG_OK;
  const int rc = check_lm_head(a, false);
  if (rc != SG_OK) return rc;
  return launch_lm_head(a, false, static_cast<hipStream_t>(stream));
}

extern "C" int64_t sg_lm_head_packed_bytes(int32_t vocab, int32_t hidden_size) {
  using namespace sg;
  if (vocab < 1 || hidden_size < 2 * kStepK || hidden_size % (2 * kStepK) != 0) return -1;
  return static_cast<int64_t>((vocab + kTileV - 1) / kTileV) * kTileV * hidden_size * 2;
}

extern "C" int sg_lm_head_pack_weight(const void* weight_dev, int64_t weight_row_stride,
                                      int32_t vocab, int32_t hidden_size, void* packed_dev,
                                      sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(vocab >= 1, "vocab must be positive");
  SG_REQUIRE(hidden_size >= 2 * kStepK && hidden_size % (2 * kStepK) == 0,
             "hidden_size must be a positive multiple of 64");
  SG_REQUIRE(weight_dev && packed_dev, "null device pointer");
  SG_REQUIRE(weight_row_stride >= hidden_size && weight_row_stride % 8 == 0,
             "weight_row_stride must cover the row and be a multiple of 8 elements");
  SG_REQUIRE((reinterpret_cast<uintptr_t>(weight_dev) | reinterpret_cast<uintptr_t>(packed_dev)) %
                     16 == 0,
             "weight and packed must be 16-byte aligned");
  const int steps = hidden_size / kStepK;
  const int64_t blocks = static_cast<int64_t>((vocab + kTileV - 1) / kTileV) * steps;
  SG_REQUIRE(blocks < INT32_MAX, "weight too large");
  lm_head_pack_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                        static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(weight_dev), weight_row_stride, vocab, steps,
      static_cast<uint16_t*>(packed_dev));
  SG_LAUNCH_CHECK();
  return SG_OK;
}

extern "C" int sg_lm_head_packed(const SgLmHeadArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null args");
  const SgLmHeadArgs& a = *args;
  SG_REQUIRE(a.num_rows >= 0, "num_rows must be non-negative");
  SG_REQUIRE(a.vocab >= 1, "vocab must be positive");
  SG_REQUIRE(a.hidden_size >= 2 * kStepK && a.hidden_size % (2 * kStepK) == 0,
             "hidden_size must be a positive multiple of 64");
  if (a.num_rows == 0) return SG_OK;
  const int rc = check_lm_head(a, true);
  if (rc != SG_OK) return rc;
  return launch_lm_head(a, true, static_cast<hipStream_t>(stream));
}
