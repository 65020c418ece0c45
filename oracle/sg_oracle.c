/*
 * sg_oracle.c -- CPU restatement of the temperature-1 tree rejection sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP sampler in
 * specgrove_amd/csrc/tree_sample.hip.  Only tests/, __graft_entry__.smoke()
 * and bench.py's CPU-baseline leg may load the library built from it.  The
 * product path never calls it.
 *
 * What it restates (reference files, relative to the reference snapshot):
 *   - the ancestral acceptance law of tree_verify_ancestral_batched
 *     (code/natural/src/gbv_experiments/sampling.py:903-950): a draw from the
 *     node's target row either follows an outgoing tree edge (accept that
 *     child) or ends the walk and becomes the bonus token;
 *   - the explicit-uniform sparse-exit layout of the reference's CUDA sampler
 *     (code/natural/src/gbv_experiments/fused_tree_sampling.py:683-824):
 *     uniform u[2d] routes over the children's cumulative mass in edge order,
 *     u[2d+1] draws the exit token from the complement of the children, and the
 *     fallback is the largest non-child token (:804-818);
 *   - the inverse-CDF rule "first token whose running mass exceeds u * total"
 *     (fused_tree_sampling.py:2607-2612).
 *
 * The reference accumulates in fp64 with CUB's reduction order.  This build
 * computes in fp32 with its own exp and a fixed reduction order so that the
 * CPU and the GPU produce the same bits.  The order is:
 *
 *   exp:   x clamped to [-120, 88] (NaN and -inf to -120; above 88: +inf);
 *          Cody-Waite reduction x = n*ln2 + r (n = rint(x*log2e), ln2 split
 *          hi/lo, both by fma); a degree-5 polynomial for e^r (coefficients
 *          fitted for relative error) in Horner form with fma; p * 2^n with
 *          one rounding (exactly 0 below about -103.3, subnormal down from
 *          -87.3).
 *   token t of a row is addressed as t = 2048*s + 256*j + 4*l + c
 *          (slab s, line j in [0,8), lane l in [0,64), component c in [0,4)).
 *   row stats (m, Z):
 *          per slab: m_s = max; lane partial a_c = sum over j (ascending) of
 *          E(x - m_s); lane sum (a0+a1)+(a2+a3); slab sum Z_s by an xor
 *          butterfly over the 64 lanes (distances 32,16,8,4,2,1).  Slab
 *          (m_s, Z_s) pairs are merged into lane (s mod 64) in ascending s,
 *          then the 64 lane pairs are merged by the same xor butterfly;
 *          merge(a,b) = (M, a.z*E(a.m-M) + b.z*E(b.m-M)), M = max(a.m, b.m).
 *          The slab pairs of every row are kept.
 *   routing at node v: children in ascending node order; S += E(x[tok]-m_v);
 *          accept the first child with u[2d]*Z_v < S.
 *   exit at node v when the sampler computed the statistics (slab draw):
 *          Z'_s = Z_s, or for a slab holding a child token the same sums with
 *          the child terms 0; E_s = E(m_s - M) (M = m_v), w_s = Z'_s * E_s;
 *          P_0 = 0, P_(s+1) = P_s + w_s, C = P_S; threshold u[2d+1]*C; the
 *          slab is the first s with P_s + w_s > threshold; in it, per line,
 *          e_t = E(x_t - m_s) (0 for child tokens), group sums, an inclusive
 *          Kogge-Stone scan over the 64 lanes and sequential line prefixes
 *          Q_j; for token c of lane l in line j, r = (Q_j + EX_jl) + e_0 +
 *          ... + e_c; the bonus is the first non-child token with
 *          P_s + E_s*r > threshold, else the slab's last non-child token with
 *          e_t > 0; no slab crossing: the largest non-child token.
 *   exit at node v with given statistics (the LM head's; complement draw):
 *          e_t = 0 for child tokens, else E(x_t - m_v);
 *          group sum ((e0+e1)+e2)+e3 per (s,j,l); inclusive Kogge-Stone scan
 *          over the 64 lanes of a line (distances 1..32); line prefix and slab
 *          prefix sequential; complement total C = last slab prefix;
 *          threshold u[2d+1]*C; the bonus is the smallest non-child token t
 *          whose running value ((PX_s + LX_sj) + EX_sjl) + e_c0 + ... + e_c
 *          exceeds the threshold; fallback = largest non-child token.
 *
 * All arithmetic is IEEE binary32 with round-to-nearest-even; the build uses
 * -ffp-contract=off so that only the explicit fmaf calls fuse.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define SGO_LANES 64
#define SGO_SLAB 2048
#define SGO_LINE 256
#define SGO_LINES_PER_SLAB 8

#define SGO_LOG2E 0x1.715476p+0f
#define SGO_LN2_HI 0x1.62e4p-1f
#define SGO_LN2_LO 0x1.7f7d1cp-20f
#define SGO_C5 0x1.10625ap-7f
#define SGO_C4 0x1.5729eep-5f
#define SGO_C3 0x1.5557aep-3f
#define SGO_C2 0x1.fffdfcp-2f
#define SGO_EXP_LO (-120.0f)
#define SGO_EXP_HI 88.0f

/* Error codes shared with the product ABI. */
#define SGO_OK 0
#define SGO_EINVAL (-1)

/* 2^e for e in [-126, 127], from the exponent bits. */
static float sgo_pow2(int e) {
  int32_t bits = (e + 127) << 23;
  float v;
  memcpy(&v, &bits, sizeof(v));
  return v;
}

float sgo_exp(float x) {
  if (x > SGO_EXP_HI) return INFINITY;
  /* fmaxf returns the other operand for a NaN: NaN and -inf clamp to -120. */
  float xc = fmaxf(x, SGO_EXP_LO);
  float n = rintf(xc * SGO_LOG2E);
  float r = fmaf(-n, SGO_LN2_HI, xc);
  r = fmaf(-n, SGO_LN2_LO, r);
  float p = SGO_C5;
  p = fmaf(p, r, SGO_C4);
  p = fmaf(p, r, SGO_C3);
  p = fmaf(p, r, SGO_C2);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int e = (int)n;
  /* p * 2^n with one rounding: an exact scale into the normal range, then
     (below 2^-126) a second exact-operand product that rounds once. */
  if (e >= -126) return p * sgo_pow2(e);
  return (p * sgo_pow2(e + 64)) * sgo_pow2(-64);
}

typedef struct {
  float m;
  float z;
} sgo_mz;

static sgo_mz sgo_merge(sgo_mz a, sgo_mz b) {
  sgo_mz out;
  float mx = fmaxf(a.m, b.m);
  if (mx == -INFINITY) {
    out.m = -INFINITY;
    out.z = 0.0f;
    return out;
  }
  float left = a.z * sgo_exp(a.m - mx);
  float right = b.z * sgo_exp(b.m - mx);
  out.m = mx;
  out.z = left + right;
  return out;
}

static float sgo_butterfly_sum(float* v) {
  float t[SGO_LANES];
  for (int d = 32; d >= 1; d >>= 1) {
    for (int l = 0; l < SGO_LANES; ++l) t[l] = v[l] + v[l ^ d];
    memcpy(v, t, sizeof(t));
  }
  return v[0];
}

/* (m_s, Z_s) of slab s; with skip (child tokens, count) those tokens' terms
 * are 0 (the complement of one slab, same order). */
static sgo_mz sgo_slab_stats_skip(const float* x, int64_t vocab, int64_t slab,
                                  const int32_t* skip, int skip_count);

static sgo_mz sgo_slab_stats(const float* x, int64_t vocab, int64_t slab) {
  return sgo_slab_stats_skip(x, vocab, slab, 0, 0);
}

static int sgo_is_child_token(int64_t t, const int32_t* child_tokens, int child_count) {
  for (int k = 0; k < child_count; ++k)
    if (child_tokens[k] == t) return 1;
  return 0;
}

static sgo_mz sgo_slab_stats_skip(const float* x, int64_t vocab, int64_t slab,
                                  const int32_t* skip, int skip_count) {
  const int64_t base = slab * SGO_SLAB;
  float m = -INFINITY;
  for (int64_t t = base; t < base + SGO_SLAB && t < vocab; ++t) m = fmaxf(m, x[t]);
  sgo_mz out;
  if (m == -INFINITY) {
    out.m = -INFINITY;
    out.z = 0.0f;
    return out;
  }
  float lane[SGO_LANES];
  for (int l = 0; l < SGO_LANES; ++l) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < SGO_LINES_PER_SLAB; ++j) {
      for (int c = 0; c < 4; ++c) {
        int64_t t = base + (int64_t)SGO_LINE * j + 4 * l + c;
        if (t < vocab && !sgo_is_child_token(t, skip, skip_count))
          a[c] = a[c] + sgo_exp(x[t] - m);
      }
    }
    lane[l] = (a[0] + a[1]) + (a[2] + a[3]);
  }
  out.m = m;
  out.z = sgo_butterfly_sum(lane);
  return out;
}

/* Canonical (max, sum of exp) of one logits row; slab_stats (when not NULL,
 * [slabs][2]) receives each slab's (m_s, Z_s). */
void sgo_row_slab_stats(const float* x, int64_t vocab, float* out_m, float* out_z,
                        float* slab_stats) {
  sgo_mz lane[SGO_LANES];
  for (int l = 0; l < SGO_LANES; ++l) {
    lane[l].m = -INFINITY;
    lane[l].z = 0.0f;
  }
  const int64_t slabs = (vocab + SGO_SLAB - 1) / SGO_SLAB;
  for (int64_t s = 0; s < slabs; ++s) {
    int l = (int)(s % SGO_LANES);
    const sgo_mz slab = sgo_slab_stats(x, vocab, s);
    if (slab_stats) {
      slab_stats[2 * s] = slab.m;
      slab_stats[2 * s + 1] = slab.z;
    }
    lane[l] = sgo_merge(lane[l], slab);
  }
  sgo_mz t[SGO_LANES];
  for (int d = 32; d >= 1; d >>= 1) {
    for (int l = 0; l < SGO_LANES; ++l) t[l] = sgo_merge(lane[l], lane[l ^ d]);
    memcpy(lane, t, sizeof(t));
  }
  *out_m = lane[0].m;
  *out_z = lane[0].z;
}

void sgo_row_stats(const float* x, int64_t vocab, float* out_m, float* out_z) {
  sgo_row_slab_stats(x, vocab, out_m, out_z, 0);
}


/* Complement draw of one row: returns the bonus token and stores C. */
int32_t sgo_complement_draw(const float* x, int64_t vocab, float m,
                            const int32_t* child_tokens, int child_count,
                            float u, float* out_total) {
  const int64_t slabs = (vocab + SGO_SLAB - 1) / SGO_SLAB;
  /* Pass 1: per-line Kogge-Stone totals, line and slab prefixes. */
  float* slab_prefix = (float*)__builtin_alloca(sizeof(float) * (size_t)(slabs + 1));
  float lp[SGO_LINES_PER_SLAB + 1];
  slab_prefix[0] = 0.0f;
  for (int64_t s = 0; s < slabs; ++s) {
    lp[0] = 0.0f;
    for (int j = 0; j < SGO_LINES_PER_SLAB; ++j) {
      float v[SGO_LANES], w[SGO_LANES];
      for (int l = 0; l < SGO_LANES; ++l) {
        float g = 0.0f;
        float e[4];
        for (int c = 0; c < 4; ++c) {
          int64_t t = s * SGO_SLAB + (int64_t)SGO_LINE * j + 4 * l + c;
          e[c] = (t < vocab && !sgo_is_child_token(t, child_tokens, child_count))
                     ? sgo_exp(x[t] - m) : 0.0f;
        }
        g = ((e[0] + e[1]) + e[2]) + e[3];
        v[l] = g;
      }
      for (int d = 1; d < SGO_LANES; d <<= 1) {
        for (int l = 0; l < SGO_LANES; ++l) w[l] = (l >= d) ? v[l] + v[l - d] : v[l];
        memcpy(v, w, sizeof(w));
      }
      lp[j + 1] = lp[j] + v[SGO_LANES - 1];
    }
    slab_prefix[s + 1] = slab_prefix[s] + lp[SGO_LINES_PER_SLAB];
  }
  const float total = slab_prefix[slabs];
  if (out_total) *out_total = total;
  const float threshold = u * total;
  /* Pass 2: first token whose running value exceeds the threshold. */
  for (int64_t s = 0; s < slabs; ++s) {
    lp[0] = 0.0f;
    float lines_incl[SGO_LINES_PER_SLAB][SGO_LANES];
    float e_all[SGO_LINES_PER_SLAB][SGO_LANES][4];
    for (int j = 0; j < SGO_LINES_PER_SLAB; ++j) {
      float v[SGO_LANES], w[SGO_LANES];
      for (int l = 0; l < SGO_LANES; ++l) {
        for (int c = 0; c < 4; ++c) {
          int64_t t = s * SGO_SLAB + (int64_t)SGO_LINE * j + 4 * l + c;
          e_all[j][l][c] = (t < vocab && !sgo_is_child_token(t, child_tokens, child_count))
                               ? sgo_exp(x[t] - m) : 0.0f;
        }
        v[l] = ((e_all[j][l][0] + e_all[j][l][1]) + e_all[j][l][2]) + e_all[j][l][3];
      }
      for (int d = 1; d < SGO_LANES; d <<= 1) {
        for (int l = 0; l < SGO_LANES; ++l) w[l] = (l >= d) ? v[l] + v[l - d] : v[l];
        memcpy(v, w, sizeof(w));
      }
      memcpy(lines_incl[j], v, sizeof(v));
      lp[j + 1] = lp[j] + v[SGO_LANES - 1];
    }
    for (int j = 0; j < SGO_LINES_PER_SLAB; ++j) {
      for (int l = 0; l < SGO_LANES; ++l) {
        float excl = l ? lines_incl[j][l - 1] : 0.0f;
        float run = (slab_prefix[s] + lp[j]) + excl;
        for (int c = 0; c < 4; ++c) {
          int64_t t = s * SGO_SLAB + (int64_t)SGO_LINE * j + 4 * l + c;
          if (t >= vocab) break;
          run = run + e_all[j][l][c];
          if (!sgo_is_child_token(t, child_tokens, child_count) && run > threshold)
            return (int32_t)t;
        }
      }
    }
  }
  for (int64_t t = vocab - 1; t >= 0; --t)
    if (!sgo_is_child_token(t, child_tokens, child_count)) return (int32_t)t;
  return -1;
}

/* Slab draw of the exit row from its statistics-pass slab pairs (m_s, Z_s):
 * returns the bonus token and stores C. */
int32_t sgo_slab_draw(const float* x, int64_t vocab, float m_row, const float* slab_stats,
                      const int32_t* child_tokens, int child_count, float u,
                      float* out_total) {
  const int64_t slabs = (vocab + SGO_SLAB - 1) / SGO_SLAB;
  float* es = (float*)__builtin_alloca(sizeof(float) * (size_t)slabs);
  float* w = (float*)__builtin_alloca(sizeof(float) * (size_t)slabs);
  for (int64_t s = 0; s < slabs; ++s) {
    float zs = slab_stats[2 * s + 1];
    int has_child = 0;
    for (int k = 0; k < child_count; ++k)
      has_child |= child_tokens[k] >= s * SGO_SLAB && child_tokens[k] < (s + 1) * SGO_SLAB;
    if (has_child) zs = sgo_slab_stats_skip(x, vocab, s, child_tokens, child_count).z;
    es[s] = sgo_exp(slab_stats[2 * s] - m_row);
    w[s] = zs * es[s];
  }
  float total = 0.0f;
  for (int64_t s = 0; s < slabs; ++s) total = total + w[s];
  if (out_total) *out_total = total;
  const float threshold = u * total;
  float p = 0.0f;
  for (int64_t s = 0; s < slabs; ++s) {
    if (!(p + w[s] > threshold)) {
      p = p + w[s];
      continue;
    }
    /* The crossing slab: per line group sums, an inclusive Kogge-Stone scan
     * over the 64 lanes and sequential line prefixes; running values scaled
     * by E(m_s - M). */
    const float ms = slab_stats[2 * s];
    int32_t last = -1;
    float q = 0.0f;
    for (int j = 0; j < SGO_LINES_PER_SLAB; ++j) {
      float e[SGO_LANES][4], incl[SGO_LANES], tmp[SGO_LANES];
      const int64_t t0 = s * SGO_SLAB + (int64_t)SGO_LINE * j;
      for (int l = 0; l < SGO_LANES; ++l) {
        for (int c = 0; c < 4; ++c) {
          const int64_t t = t0 + 4 * l + c;
          e[l][c] = (t < vocab && !sgo_is_child_token(t, child_tokens, child_count))
                        ? sgo_exp(x[t] - ms) : 0.0f;
        }
        incl[l] = ((e[l][0] + e[l][1]) + e[l][2]) + e[l][3];
      }
      for (int d = 1; d < SGO_LANES; d <<= 1) {
        for (int l = 0; l < SGO_LANES; ++l) tmp[l] = (l >= d) ? incl[l] + incl[l - d] : incl[l];
        memcpy(incl, tmp, sizeof(tmp));
      }
      for (int l = 0; l < SGO_LANES; ++l) {
        float r = q + (l ? incl[l - 1] : 0.0f);
        for (int c = 0; c < 4; ++c) {
          const int64_t t = t0 + 4 * l + c;
          r = r + e[l][c];
          if (t >= vocab || sgo_is_child_token(t, child_tokens, child_count)) continue;
          if (p + es[s] * r > threshold) return (int32_t)t;
          if (e[l][c] > 0.0f) last = (int32_t)t;
        }
      }
      q = q + incl[SGO_LANES - 1];
    }
    return last;
  }
  for (int64_t t = vocab - 1; t >= 0; --t)
    if (!sgo_is_child_token(t, child_tokens, child_count)) return (int32_t)t;
  return -1;
}

/*
 * Sample every request of a packed wave.
 *   logits      [logits rows, row_stride] fp32 (only the first vocab entries used)
 *   row_offset  [n+1]   packed row range of request i
 *   parent      [rows]  request-local parent index, -1 for each request's root
 *   token       [rows]  draft token of each node (ignored for roots)
 *   uniforms    [n, uniform_stride] fp32, u[2d] routes and u[2d+1] exits at depth d
 *   max_depth   accept_nodes holds max_depth entries per request
 *   row_map     optional [rows]: logits row of each packed node, -1 when the node
 *               was not projected (then it must have no children); NULL: row r
 *   row_m_in, row_z_in  optional [logits rows]: given row statistics (the LM
 *               head's), with the complement draw at the exit; NULL: computed by
 *               sgo_row_slab_stats, with the slab draw at the exit
 * Outputs: accept_nodes [n, max_depth] (local node ids, -1 padded),
 *          accept_len [n], bonus [n] (-1 at an unprojected terminal leaf),
 *          terminal_leaf [n] (may be NULL: that leaf's local id, else -1).
 * Returns SGO_OK or SGO_EINVAL.
 */
int sgo_tree_sample_mapped(const float* logits, int64_t row_stride, int64_t vocab,
                           int32_t num_requests, const int32_t* row_offset,
                           const int32_t* parent, const int32_t* token,
                           const float* uniforms, int32_t uniform_stride,
                           int32_t max_depth, const int32_t* row_map,
                           const float* row_m_in, const float* row_z_in,
                           int32_t* accept_nodes, int32_t* accept_len, int32_t* bonus,
                           int32_t* terminal_leaf) {
  if (num_requests < 0 || vocab < 1 || max_depth < 0) return SGO_EINVAL;
  const int64_t slabs = (vocab + SGO_SLAB - 1) / SGO_SLAB;
  float* slab_stats = (float*)__builtin_alloca(sizeof(float) * (size_t)(2 * slabs));
  for (int32_t i = 0; i < num_requests; ++i) {
    const int32_t r0 = row_offset[i];
    const int32_t n = row_offset[i + 1] - r0;
    const float* u = uniforms + (int64_t)i * uniform_stride;
    for (int32_t k = 0; k < max_depth; ++k) accept_nodes[(int64_t)i * max_depth + k] = -1;
    if (terminal_leaf) terminal_leaf[i] = -1;
    int32_t v = 0, depth = 0;
    int32_t children[1024];
    int32_t child_tokens[1024];
    if (n < 1 || n > 1024) return SGO_EINVAL;
    for (;;) {
      if (2 * depth + 1 >= uniform_stride) return SGO_EINVAL;
      const int32_t lrow = row_map ? row_map[r0 + v] : r0 + v;
      int count = 0;
      for (int32_t w = v + 1; w < n; ++w) {
        if (parent[r0 + w] == v) {
          children[count] = w;
          child_tokens[count] = token[r0 + w];
          ++count;
        }
      }
      if (lrow < 0) {
        /* Unprojected node: only a leaf may be one; its bonus is drawn later. */
        if (count > 0) return SGO_EINVAL;
        accept_len[i] = depth;
        bonus[i] = -1;
        if (terminal_leaf) terminal_leaf[i] = v;
        break;
      }
      const float* x = logits + (int64_t)lrow * row_stride;
      float m, z;
      const int given = row_m_in && row_z_in;
      if (given) {
        m = row_m_in[lrow];
        z = row_z_in[lrow];
      } else {
        sgo_row_slab_stats(x, vocab, &m, &z, slab_stats);
      }
      const float route_threshold = u[2 * depth] * z;
      float cumulative = 0.0f;
      int32_t accepted = -1;
      for (int k = 0; k < count; ++k) {
        cumulative = cumulative + sgo_exp(x[child_tokens[k]] - m);
        if (route_threshold < cumulative) {
          accepted = children[k];
          break;
        }
      }
      if (accepted >= 0) {
        if (depth >= max_depth) return SGO_EINVAL;
        accept_nodes[(int64_t)i * max_depth + depth] = accepted;
        v = accepted;
        ++depth;
        continue;
      }
      accept_len[i] = depth;
      bonus[i] = given ? sgo_complement_draw(x, vocab, m, child_tokens, count,
                                             u[2 * depth + 1], 0)
                       : sgo_slab_draw(x, vocab, m, slab_stats, child_tokens, count,
                                       u[2 * depth + 1], 0);
      break;
    }
  }
  return SGO_OK;
}

/* The unmapped sampler: every packed row has logits, statistics computed here
 * (row_m / row_z, when given, receive them) and the slab draw at the exit. */
int sgo_tree_sample(const float* logits, int64_t row_stride, int64_t vocab,
                    int32_t num_requests, const int32_t* row_offset,
                    const int32_t* parent, const int32_t* token,
                    const float* uniforms, int32_t uniform_stride,
                    int32_t max_depth, int32_t* accept_nodes,
                    int32_t* accept_len, int32_t* bonus, float* row_m,
                    float* row_z) {
  if (num_requests < 0 || vocab < 1 || max_depth < 0) return SGO_EINVAL;
  const int32_t rows = row_offset[num_requests];
  if (row_m && row_z) {
    for (int32_t r = 0; r < rows; ++r)
      sgo_row_stats(logits + (int64_t)r * row_stride, vocab, &row_m[r], &row_z[r]);
  }
  return sgo_tree_sample_mapped(logits, row_stride, vocab, num_requests, row_offset, parent,
                                token, uniforms, uniform_stride, max_depth, 0, 0, 0,
                                accept_nodes, accept_len, bonus, 0);
}

/*
 * LM-head statistics (the fused epilogue of the HIP projection, restated).
 * Tile t of a row covers tokens 128t .. 128t+127 below vocab; token
 * 128t + 32b + 8q + 4h + e (b, q, e in 0..3; h in 0..1) is in half h.
 *   m_t = max of the tile (-inf for a tile with no token);
 *   z_h = sequential sum, increasing (b, q, e), of E(x - m_t) over half h;
 *   z_t = z_0 + z_1.
 * out_pairs receives (m_t, z_t) for t < ceil(vocab / 128).
 */
void sgo_lm_head_tile_stats(const float* x, int64_t vocab, float* out_pairs) {
  const int64_t tiles = (vocab + 127) / 128;
  for (int64_t t = 0; t < tiles; ++t) {
    float m = -INFINITY;
    for (int64_t k = 128 * t; k < 128 * t + 128 && k < vocab; ++k) m = fmaxf(m, x[k]);
    const float mc = (m == -INFINITY) ? 0.0f : m;
    float zh[2] = {0.0f, 0.0f};
    for (int h = 0; h < 2; ++h)
      for (int b = 0; b < 4; ++b)
        for (int q = 0; q < 4; ++q)
          for (int e = 0; e < 4; ++e) {
            const int64_t k = 128 * t + 32 * b + 8 * q + 4 * h + e;
            if (k < vocab) zh[h] = zh[h] + sgo_exp(x[k] - mc);
          }
    out_pairs[2 * t] = m;
    out_pairs[2 * t + 1] = zh[0] + zh[1];
  }
}

/* Row (max, sum) from its tile pairs: tile t merged into lane t % 64 in
 * increasing t, then the xor butterfly (32 .. 1) over the 64 lanes. */
void sgo_lm_head_row_stats(const float* pairs, int64_t tiles, float* out_m, float* out_z) {
  sgo_mz lane[SGO_LANES];
  for (int l = 0; l < SGO_LANES; ++l) {
    lane[l].m = -INFINITY;
    lane[l].z = 0.0f;
  }
  for (int64_t t = 0; t < tiles; ++t) {
    sgo_mz p;
    p.m = pairs[2 * t];
    p.z = pairs[2 * t + 1];
    lane[t % SGO_LANES] = sgo_merge(lane[t % SGO_LANES], p);
  }
  sgo_mz tmp[SGO_LANES];
  for (int d = 32; d >= 1; d >>= 1) {
    for (int l = 0; l < SGO_LANES; ++l) tmp[l] = sgo_merge(lane[l], lane[l ^ d]);
    memcpy(lane, tmp, sizeof(tmp));
  }
  *out_m = lane[0].m;
  *out_z = lane[0].z;
}

/* Slab statistics of many rows ([rows][slabs][2]), for tests of the GPU's. */
void sgo_rows_slab_stats(const float* logits, int64_t row_stride, int64_t vocab, int32_t rows,
                         float* row_m, float* row_z, float* slab_stats) {
  const int64_t slabs = (vocab + SGO_SLAB - 1) / SGO_SLAB;
  for (int32_t r = 0; r < rows; ++r)
    sgo_row_slab_stats(logits + (int64_t)r * row_stride, vocab, &row_m[r], &row_z[r],
                       slab_stats + (int64_t)r * 2 * slabs);
}

/* Vectorised E(x) for tests of the exp restatement. */
void sgo_exp_array(const float* x, float* out, int64_t count) {
  for (int64_t k = 0; k < count; ++k) out[k] = sgo_exp(x[k]);
}
