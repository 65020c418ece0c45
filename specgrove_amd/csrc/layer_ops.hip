// Fused elementwise kernels of the target decoder layer stack (Qwen3 family)
// around the library projections, for the packed verification wave.
//
// The reference runs the Target's transformers decoder
// (engine.py:499-517 target_hidden_forward -> transformers' Qwen3 layers):
// per layer RMSNorm, q/k/v projections, per-head RMSNorm of q and k (QK-norm),
// rotary position embedding, attention, o projection, residual add, RMSNorm,
// gate/up projections, SiLU(gate) * up, down projection, residual add.  Here
// the projections are library GEMMs (hipBLASLt through torch.matmul) and every
// elementwise stage between them is one HBM pass:
//
//   sg_add_rmsnorm     residual add + RMSNorm (one read of each input, one
//                      write of each output);
//   sg_qk_norm_rope    QK-norm + RoPE of the merged q/k/v projection, writing
//                      q [R, Hq, D] for the attention and k/v [Hkv, R, D] as
//                      the wave's new cache rows;
//   sg_silu_mul        SiLU(gate) * up of the merged gate/up projection;
//   sg_gather_rows     the kept rows of several layers' hidden states side by
//                      side (the draft features, continuous_tree_block_decode.py
//                      :2144-2158).
//
// Arithmetic follows the transformers modules' rounding points: RMSNorm
// normalises in fp32, rounds to bf16, then multiplies by the bf16 weight and
// rounds again; RoPE uses bf16-rounded cos/sin of fp32 angles and rounds
// q*cos, rotate_half(q)*sin and their sum to bf16 in turn; SiLU rounds
// before the product with up.  Sums of squares run in fp32 in this kernel's
// own order, and 1/sqrt and sincos are the device's, so a normed or rotated
// value can still differ from transformers' by one bf16 ulp.
#include <cmath>

#include "sg_common.h"

namespace sg {
namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ __forceinline__ float block_sum(float v, float* scratch) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float t = 0.0f;
  const int waves = blockDim.x >> 6;
  for (int w = 0; w < waves; ++w) t += scratch[w];
  __syncthreads();
  return t;
}

// One row per workgroup; 8 bf16 (16 bytes) per thread per step.
// sum = x (+ residual); residual_out = bf16(sum) when requested;
// out = bf16(w * bf16(s * rsqrt(mean(s^2) + eps))), s = bf16(sum).
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ weight, uint16_t* __restrict__ out,
    uint16_t* __restrict__ residual_out, int hidden, int64_t x_stride, int64_t res_stride,
    int64_t out_stride, int64_t res_out_stride, float eps) {
  __shared__ float scratch[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * x_stride;
  const uint16_t* rr = residual != nullptr ? residual + row * res_stride : nullptr;
  constexpr int kMaxChunks = 4;  // hidden <= 8192
  uint4 s[kMaxChunks];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int e = 8 * (threadIdx.x + c * kNormThreads);
    s[c] = make_uint4(0u, 0u, 0u, 0u);
    if (e >= hidden) continue;
    uint4 a = *reinterpret_cast<const uint4*>(xr + e);
    if (rr != nullptr) {
      const uint4 b = *reinterpret_cast<const uint4*>(rr + e);
      const uint32_t av[4] = {a.x, a.y, a.z, a.w};
      const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = bf16_to_f32(av[k] & 0xffffu) + bf16_to_f32(bv[k] & 0xffffu);
        const float hi = bf16_to_f32(av[k] >> 16) + bf16_to_f32(bv[k] >> 16);
        o[k] = pack_bf16x2(lo, hi);
      }
      a = make_uint4(o[0], o[1], o[2], o[3]);
    }
    s[c] = a;
    const uint32_t v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float lo = bf16_to_f32(v[k] & 0xffffu);
      const float hi = bf16_to_f32(v[k] >> 16);
      ss += lo * lo + hi * hi;
    }
  }
  const float total = block_sum(ss, scratch);
  const float r = 1.0f / sqrtf(total / static_cast<float>(hidden) + eps);
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int e = 8 * (threadIdx.x + c * kNormThreads);
    if (e >= hidden) continue;
    if (residual_out != nullptr)
      *reinterpret_cast<uint4*>(residual_out + row * res_out_stride + e) = s[c];
    const uint4 w = *reinterpret_cast<const uint4*>(weight + e);
    const uint32_t v[4] = {s[c].x, s[c].y, s[c].z, s[c].w};
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float lo = bf16_to_f32(wv[k] & 0xffffu) * bf16r(bf16_to_f32(v[k] & 0xffffu) * r);
      const float hi = bf16_to_f32(wv[k] >> 16) * bf16r(bf16_to_f32(v[k] >> 16) * r);
      o[k] = pack_bf16x2(lo, hi);
    }
    *reinterpret_cast<uint4*>(out + row * out_stride + e) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// One row per workgroup.  A head's D dims are D/8 lanes of 16 bytes (lane j
// holds dims 8j .. 8j+7), so a wave takes 64/(D/8) heads at a time with
// 16-byte loads and stores; the rotary partner of dim i < D/2 (dim i + D/2)
// sits in lane j ^ (D/16) of the same head.  Heads 0..Hq-1 are q (normed,
// rotated, written to q_out[row, h]), Hq..Hq+Hkv-1 are k (normed, rotated,
// written to k_out[h, row]), the rest v (copied to v_out[h, row]).  The
// row's bf16 cos / sin of the fp32 angles position * inv_freq[p] are made once
// per workgroup (one pair per thread) and read from LDS.
template <int D>
__global__ __launch_bounds__(kNormThreads) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_stride, int hq, int hkv,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    const float* __restrict__ inv_freq, const int64_t* __restrict__ positions,
    uint16_t* __restrict__ q_out, int64_t q_row_stride, uint16_t* __restrict__ k_out,
    uint16_t* __restrict__ v_out, int64_t kv_head_stride, float eps) {
  constexpr int H2 = D / 2;
  constexpr int LPH = D / 8;        // lanes per head
  constexpr int HPW = kWave / LPH;  // heads per wave at a time
  __shared__ float s_cs[H2];
  __shared__ float s_sn[H2];
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const float pos = static_cast<float>(positions[row]);
  for (int p = threadIdx.x; p < H2; p += blockDim.x) {
    float sv, cv;
    sincosf(pos * inv_freq[p], &sv, &cv);
    s_cs[p] = bf16r(cv);
    s_sn[p] = bf16r(sv);
  }
  __syncthreads();
  const int j = lane % LPH;             // 16-byte chunk of the head
  const int slot = lane / LPH;          // head of the wave's group
  const bool lower = j < LPH / 2;       // dims below D/2
  const int pair0 = 8 * (j % (LPH / 2));
  float cs[8], sn[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    cs[k] = s_cs[pair0 + k];
    sn[k] = s_sn[pair0 + k];
  }
  const int heads = hq + 2 * hkv;
  for (int h0 = wave * HPW; h0 < heads; h0 += waves * HPW) {
    const int h = h0 + slot;
    const bool live = h < heads;
    const bool is_v = h >= hq + hkv;
    const uint16_t* src = qkv + row * qkv_stride + static_cast<int64_t>(h) * D + 8 * j;
    const uint4 raw = live ? *reinterpret_cast<const uint4*>(src) : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t rv[4] = {raw.x, raw.y, raw.z, raw.w};
    float x[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = bf16_to_f32(rv[k] & 0xffffu);
      x[2 * k + 1] = bf16_to_f32(rv[k] >> 16);
    }
    // RMS over the head's D dims: the lane's 8 squares, then the head's lanes.
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += x[k] * x[k];
#pragma unroll
    for (int d = LPH / 2; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
    const uint16_t* w = (h < hq ? q_norm : k_norm) + 8 * j;
    const uint4 wraw = (live && !is_v) ? *reinterpret_cast<const uint4*>(w)
                                       : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t wv[4] = {wraw.x, wraw.y, wraw.z, wraw.w};
    uint32_t nx[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float lo = bf16_to_f32(wv[k] & 0xffffu) * bf16r(x[2 * k] * r);
      const float hi = bf16_to_f32(wv[k] >> 16) * bf16r(x[2 * k + 1] * r);
      nx[k] = pack_bf16x2(lo, hi);
    }
    // The rotary partner's normed values (exact: bf16 pairs).
    uint32_t ny[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) ny[k] = __shfl_xor(nx[k], LPH / 2);
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float e[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float a = bf16_to_f32(t ? (nx[k] >> 16) : (nx[k] & 0xffffu));
        const float b = bf16_to_f32(t ? (ny[k] >> 16) : (ny[k] & 0xffffu));
        const int q = 2 * k + t;
        // x*cos + rotate_half(x)*sin, rotate_half(x) = (-x2, x1), with the
        // rounding points of transformers' bf16 tensors: each product is
        // rounded to bf16, then their sum (bf16r(-v) = -bf16r(v)).
        const float ac = bf16r(a * cs[q]);
        const float bs = bf16r(b * sn[q]);
        e[t] = lower ? ac - bs : ac + bs;
      }
      o[k] = pack_bf16x2(e[0], e[1]);
    }
    if (!live) continue;
    if (is_v) {
      *reinterpret_cast<uint4*>(v_out + static_cast<int64_t>(h - hq - hkv) * kv_head_stride +
                                row * D + 8 * j) = raw;
    } else {
      uint16_t* dst = h < hq ? q_out + row * q_row_stride + static_cast<int64_t>(h) * D
                             : k_out + static_cast<int64_t>(h - hq) * kv_head_stride + row * D;
      *reinterpret_cast<uint4*>(dst + 8 * j) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// out[r, i] = bf16(bf16(silu(gate[r, i])) * up[r, i]); gate = gu[r, :I],
// up = gu[r, I:2I].  8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                       int64_t gu_stride, int inter,
                                                       uint16_t* __restrict__ out,
                                                       int64_t out_stride, int64_t chunks) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k >= chunks) return;
  const int per_row = inter / 8;
  const int64_t row = k / per_row;
  const int e = 8 * static_cast<int>(k - row * per_row);
  const uint4 g = *reinterpret_cast<const uint4*>(gu + row * gu_stride + e);
  const uint4 u = *reinterpret_cast<const uint4*>(gu + row * gu_stride + inter + e);
  const uint32_t gv[4] = {g.x, g.y, g.z, g.w};
  const uint32_t uv[4] = {u.x, u.y, u.z, u.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float x = bf16_to_f32(h ? (gv[q] >> 16) : (gv[q] & 0xffffu));
      const float up = bf16_to_f32(h ? (uv[q] >> 16) : (uv[q] & 0xffffu));
      const float s = bf16r(x / (1.0f + expf(-x)));
      v[h] = s * up;
    }
    o[q] = pack_bf16x2(v[0], v[1]);
  }
  *reinterpret_cast<uint4*>(out + row * out_stride + e) = make_uint4(o[0], o[1], o[2], o[3]);
}

// out[k, l*width .. (l+1)*width) = src_l[index[k], :width]; one workgroup per
// output row, 16-byte chunks.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* const* __restrict__ srcs,
                                                          int num_src, int64_t src_stride,
                                                          int width, int num_src_rows,
                                                          const int32_t* __restrict__ index,
                                                          uint16_t* __restrict__ out,
                                                          int64_t out_stride,
                                                          int32_t* __restrict__ status) {
  const int k = blockIdx.x;
  const int r = index[k];
  const bool ok = r >= 0 && r < num_src_rows;
  if (!ok && threadIdx.x == 0 && status != nullptr) atomicExch(status, SG_EINVAL);
  const int chunks = width / 8;
  for (int c = threadIdx.x; c < num_src * chunks; c += blockDim.x) {
    const int l = c / chunks;
    const int e = 8 * (c - l * chunks);
    const uint4 v = ok ? *reinterpret_cast<const uint4*>(srcs[l] + static_cast<int64_t>(r) *
                                                                       src_stride + e)
                       : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(out + static_cast<int64_t>(k) * out_stride +
                              static_cast<int64_t>(l) * width + e) = v;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace sg

extern "C" int sg_add_rmsnorm(const SgAddRmsNormArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null args");
  const SgAddRmsNormArgs& a = *args;
  SG_REQUIRE(a.num_rows >= 0, "num_rows must be non-negative");
  SG_REQUIRE(a.hidden >= 8 && a.hidden % 8 == 0 && a.hidden <= 8 * 4 * kNormThreads,
             "hidden must be a multiple of 8 in [8, 8192]");
  if (a.num_rows == 0) return SG_OK;
  SG_REQUIRE(a.x_dev && a.weight_dev && a.out_dev, "null device pointer");
  SG_REQUIRE((a.x_stride | a.out_stride | (a.residual_dev ? a.residual_stride : 0) |
              (a.residual_out_dev ? a.residual_out_stride : 0)) % 8 == 0,
             "row strides must be multiples of 8 elements");
  SG_REQUIRE(aligned16(a.x_dev) && aligned16(a.weight_dev) && aligned16(a.out_dev) &&
                 (!a.residual_dev || aligned16(a.residual_dev)) &&
                 (!a.residual_out_dev || aligned16(a.residual_out_dev)),
             "tensors must be 16-byte aligned");
  add_rmsnorm_kernel<<<dim3(a.num_rows), dim3(kNormThreads), 0,
                       static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(a.x_dev), static_cast<const uint16_t*>(a.residual_dev),
      static_cast<const uint16_t*>(a.weight_dev), static_cast<uint16_t*>(a.out_dev),
      static_cast<uint16_t*>(a.residual_out_dev), a.hidden, a.x_stride, a.residual_stride,
      a.out_stride, a.residual_out_stride, a.eps);
  SG_LAUNCH_CHECK();
  return SG_OK;
}

extern "C" int sg_qk_norm_rope(const SgQkNormRopeArgs* args, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(args != nullptr, "null args");
  const SgQkNormRopeArgs& a = *args;
  SG_REQUIRE(a.num_rows >= 0, "num_rows must be non-negative");
  SG_REQUIRE(a.head_dim == 64 || a.head_dim == 128, "head_dim must be 64 or 128");
  SG_REQUIRE(a.num_q_heads >= 1 && a.num_kv_heads >= 1, "head counts must be positive");
  if (a.num_rows == 0) return SG_OK;
  SG_REQUIRE(a.qkv_dev && a.q_norm_dev && a.k_norm_dev && a.inv_freq_dev && a.positions_dev &&
                 a.q_out_dev && a.k_out_dev && a.v_out_dev,
             "null device pointer");
  SG_REQUIRE(a.qkv_row_stride >= static_cast<int64_t>(a.num_q_heads + 2 * a.num_kv_heads) *
                                     a.head_dim,
             "qkv row stride below the q/k/v width");
  SG_REQUIRE(a.q_row_stride >= static_cast<int64_t>(a.num_q_heads) * a.head_dim,
             "q row stride below Hq*D");
  SG_REQUIRE(a.kv_head_stride >= static_cast<int64_t>(a.num_rows) * a.head_dim,
             "k/v head stride below R*D");
  SG_REQUIRE((a.qkv_row_stride | a.q_row_stride | a.kv_head_stride) % 8 == 0,
             "row and head strides must be multiples of 8 elements");
  SG_REQUIRE(aligned16(a.qkv_dev) && aligned16(a.q_norm_dev) && aligned16(a.k_norm_dev) &&
                 aligned16(a.q_out_dev) && aligned16(a.k_out_dev) && aligned16(a.v_out_dev),
             "q/k/v, norm weights and outputs must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto go = [&](auto kernel) {
    kernel<<<dim3(a.num_rows), dim3(kNormThreads), 0, s>>>(
        static_cast<const uint16_t*>(a.qkv_dev), a.qkv_row_stride, a.num_q_heads,
        a.num_kv_heads, static_cast<const uint16_t*>(a.q_norm_dev),
        static_cast<const uint16_t*>(a.k_norm_dev), a.inv_freq_dev, a.positions_dev,
        static_cast<uint16_t*>(a.q_out_dev), a.q_row_stride, static_cast<uint16_t*>(a.k_out_dev),
        static_cast<uint16_t*>(a.v_out_dev), a.kv_head_stride, a.eps);
  };
  if (a.head_dim == 128) {
    go(qk_norm_rope_kernel<128>);
  } else {
    go(qk_norm_rope_kernel<64>);
  }
  SG_LAUNCH_CHECK();
  return SG_OK;
}

extern "C" int sg_silu_mul(const void* gate_up_dev, int64_t gate_up_row_stride,
                           int32_t num_rows, int32_t intermediate, void* out_dev,
                           int64_t out_row_stride, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(num_rows >= 0 && intermediate >= 8 && intermediate % 8 == 0,
             "intermediate must be a positive multiple of 8");
  if (num_rows == 0) return SG_OK;
  SG_REQUIRE(gate_up_dev && out_dev, "null device pointer");
  SG_REQUIRE(gate_up_row_stride >= 2 * static_cast<int64_t>(intermediate) &&
                 out_row_stride >= intermediate && (gate_up_row_stride | out_row_stride) % 8 == 0,
             "row strides must cover the rows and be multiples of 8");
  SG_REQUIRE(aligned16(gate_up_dev) && aligned16(out_dev), "tensors must be 16-byte aligned");
  const int64_t chunks = static_cast<int64_t>(num_rows) * (intermediate / 8);
  const int64_t blocks = (chunks + 255) / 256;
  SG_REQUIRE(blocks < INT32_MAX, "too many rows");
  silu_mul_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                    static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(gate_up_dev), gate_up_row_stride, intermediate,
      static_cast<uint16_t*>(out_dev), out_row_stride, chunks);
  SG_LAUNCH_CHECK();
  return SG_OK;
}

extern "C" int sg_gather_rows(const void* const* src_dev, int32_t num_src, int64_t src_row_stride,
                              int32_t width, int32_t num_src_rows, const int32_t* index_dev,
                              int32_t num_index, void* out_dev, int64_t out_row_stride,
                              int32_t* status_dev, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(num_src >= 1 && width >= 8 && width % 8 == 0 && num_index >= 0 &&
                 num_src_rows >= 1,
             "need at least one source of a positive multiple of 8 columns");
  if (num_index == 0) return SG_OK;
  SG_REQUIRE(src_dev && index_dev && out_dev, "null device pointer");
  SG_REQUIRE(src_row_stride >= width && out_row_stride >= static_cast<int64_t>(num_src) * width &&
                 (src_row_stride | out_row_stride) % 8 == 0,
             "row strides must cover the rows and be multiples of 8");
  SG_REQUIRE(aligned16(out_dev), "out must be 16-byte aligned");
  gather_rows_kernel<<<dim3(num_index), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint16_t* const*>(src_dev), num_src, src_row_stride, width,
      num_src_rows, index_dev, static_cast<uint16_t*>(out_dev), out_row_stride, status_dev);
  SG_LAUNCH_CHECK();
  return SG_OK;
}
