/*
 * specgrove_hip.h -- C ABI of libspecgrove_hip.so, the MI355X (gfx950) kernels
 * of SpecGrove's packed target-verification path.
 *
 * Conventions
 *   - Every pointer named *_dev is a device pointer owned by the caller; the
 *     library never allocates or frees device memory and never synchronises
 *     the device.  Work is enqueued on the given stream only.
 *   - Host pointers (named *_host) are read before the call returns.
 *   - Return 0 on success or a negative SG_E* code; sg_last_error() returns a
 *     thread-local message for the last failure on the calling thread.
 *   - bf16 tensors are passed as void* (raw 16-bit storage); the head
 *     dimension is contiguous, the other strides are given in elements.
 *
 * Reference interfaces replaced (paths relative to the reference snapshot;
 * CTBD = code/natural/src/gbv_experiments/continuous_tree_block_decode.py,
 * FTS = code/natural/src/gbv_experiments/fused_tree_sampling.py,
 * SMP = code/natural/src/gbv_experiments/sampling.py).
 */
#ifndef SPECGROVE_HIP_H
#define SPECGROVE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SG_ABI_VERSION 5

#define SG_OK 0
#define SG_EINVAL (-1)  /* shape or contract violation (Python: ValueError) */
#define SG_ERANGE (-2)  /* KV capacity exhausted (Python: RuntimeError) */
#define SG_EHIP (-3)    /* HIP launch/runtime error (Python: RuntimeError) */

typedef struct ihipStream_t* sg_stream_t; /* == hipStream_t */

/* Element types of the sampler's logits.  bf16 and f16 widen to fp32 exactly,
 * so their statistics and decisions equal those of the widened fp32 rows. */
#define SG_DTYPE_F32 0
#define SG_DTYPE_BF16 1
#define SG_DTYPE_F16 2

/* ABI version (SG_ABI_VERSION).  No reference counterpart. */
int sg_abi_version(void);

/* Message of the last error on this thread ("" if none).  Plays the role of
 * TORCH_CHECK's RuntimeError text in FTS:158-174. */
const char* sg_last_error(void);

/* ------------------------------------------------------------------------
 * (A) Request-isolated, tree-ancestor-masked GQA attention.
 *
 * Replaces the packed target wave's attention: _pack_cache_sequence
 * (CTBD:313-361) + the dense mask of _packed_block_inputs (CTBD:500-546) +
 * transformers' repeat_kv + F.scaled_dot_product_attention (called through
 * Engine.target_hidden_forward, code/natural/src/gbv_experiments/engine.py:499-517,
 * attention plug point engine.py:278-281).  Row q_i+k of request i attends to
 * the request's own cached prefix and to the tree rows that are ancestors of k
 * (or k itself), exactly the visible set of CTBD:535-545 / tree.py:19-26.
 * ---------------------------------------------------------------------- */
typedef struct SgTreeAttnArgs {
  int32_t num_requests;   /* n */
  int32_t num_rows;       /* R = row_offset[n]: rows of q, k/v_tree and out */
  int32_t num_q_heads;    /* Hq */
  int32_t num_kv_heads;   /* Hkv; Hq % Hkv == 0 and 1 <= Hq/Hkv <= 16 */
  int32_t head_dim;       /* D: 64 or 128 */
  float scale;            /* softmax scale, usually D^-0.5 */
  /* queries [R, Hq, D] bf16 */
  const void* q_dev;
  int64_t q_row_stride, q_head_stride;
  /* cached prefix K/V: element (head g, token t) at base + g*head_stride + t*token_stride */
  const void* k_cache_dev;
  const void* v_cache_dev;
  int64_t cache_head_stride, cache_token_stride;
  /* this wave's tree-row K/V [R, Hkv, D] bf16 (not yet in the cache) */
  const void* k_tree_dev;
  const void* v_tree_dev;
  int64_t tree_row_stride, tree_head_stride;
  /* request metadata (device, int32) */
  const int32_t* row_offset_dev;   /* [n+1] */
  const int64_t* prefix_start_dev; /* [n] first cache token of request i (slot*capacity) */
  const int32_t* prefix_len_dev;   /* [n] cached prefix length L_i; every unit checks its
                                      key range and rows against L_i and row_offset */
  const int32_t* parent_dev;       /* [R] request-local parent row, -1 for the root */
  /* output [R, Hq, D] bf16 */
  void* out_dev;
  int64_t out_row_stride, out_head_stride;
  /* work plan from sg_tree_attn_plan (device copy) and its scratch */
  const void* plan_dev;
  const void* plan_host; /* optional host copy of the same plan: its header is checked
                            against these arguments before anything is enqueued */
  int32_t plan_units;    /* work lists = workgroups of the first kernel */
  int32_t plan_merges;   /* split-K merge groups (second kernel's grid) */
  void* workspace_dev;
  size_t workspace_bytes;
  int32_t* status_dev;   /* optional [1] device word, never cleared by the library: set
                            to SG_EINVAL when a unit's key range or rows disagree with
                            prefix_len_dev / row_offset_dev (a plan of another wave); that
                            unit reads no K/V and writes NaN to its output rows.  A unit or
                            merge group naming a request, kv head or partial slot this
                            call does not have (a larger wave's plan passed without
                            plan_host) indexes nothing and only sets the word */
} SgTreeAttnArgs;

/* Host-side planner.  From host copies of row_offset [n+1] and prefix_len [n]
 * it writes the work list (plan_capacity_bytes of host memory) and reports its
 * size, its number of work lists (*plan_units: workgroups of the attention
 * kernel), its split-merge groups and the scratch bytes sg_tree_attn_fwd
 * needs.  Replaces the host index lists the reference builds per wave
 * (CTBD:327-350, :513-545).
 * target_units_hint <= 0: one unit per work list, in decreasing cost order,
 * with splits sized for 256 CUs; > 0: units packed onto at most that many
 * lists by estimated cost. */
int sg_tree_attn_plan(int32_t num_requests, const int32_t* row_offset_host,
                      const int32_t* prefix_len_host, int32_t num_q_heads,
                      int32_t num_kv_heads, int32_t head_dim,
                      int32_t target_units_hint, void* plan_host,
                      size_t plan_capacity_bytes, size_t* plan_bytes,
                      int32_t* plan_units, int32_t* plan_merges,
                      size_t* workspace_bytes);

/* SG_OK when plan_host was built by sg_tree_attn_plan from exactly these
 * row offsets and prefix lengths (the plan header keeps their count, the row
 * total and a 64-bit hash of both arrays), SG_EINVAL otherwise.  A plan is
 * per wave: prefix lengths change after every commit.  No reference
 * counterpart (the reference rebuilds its dense mask every wave). */
int sg_tree_attn_plan_check(const void* plan_host, int32_t num_requests,
                            const int32_t* row_offset_host, const int32_t* prefix_len_host);

/* Enqueue the attention of one layer. */
int sg_tree_attn_fwd(const SgTreeAttnArgs* args, sg_stream_t stream);

/* ------------------------------------------------------------------------
 * (B) Accepted-path KV commit.
 *
 * Replaces _PersistentRequestCachePool.append_packed_sequence (CTBD:215-261)
 * with the keep rule keep_i = [0] + accepted local nodes (CTBD:2108-2109):
 *   cache[l][g, prefix_start_i + len_i + t] = tree[l][row_offset_i + keep_i[t], g]
 * for every layer l, kv head g and t < keep_len_i.  If len_i + keep_len_i
 * exceeds capacity the request is not written and *status_dev is set to
 * SG_ERANGE (the reference raises "Persistent request KV capacity exhausted",
 * CTBD:235-236); callers check capacity on the host first.  A kept row
 * outside [0, row_offset_{i+1} - row_offset_i) likewise leaves the request
 * unwritten and sets *status_dev to SG_EINVAL.
 * ---------------------------------------------------------------------- */
typedef struct SgKvCommitArgs {
  int32_t num_layers;
  int32_t num_requests;
  int32_t num_kv_heads;
  int32_t head_dim;
  /* per-layer cache bases (device arrays of num_layers device pointers) */
  void* const* k_cache_layers_dev;
  void* const* v_cache_layers_dev;
  int64_t cache_head_stride, cache_token_stride;
  /* per-layer tree-row K/V bases [R, Hkv, D] (device arrays of pointers) */
  const void* const* k_tree_layers_dev;
  const void* const* v_tree_layers_dev;
  int64_t tree_row_stride, tree_head_stride;
  const int32_t* row_offset_dev;   /* [n+1] packed row range of request i */
  const int32_t* keep_rows_dev;    /* [n, keep_stride] local rows, ascending path order */
  int32_t keep_stride;
  const int32_t* keep_len_dev;     /* [n] */
  const int64_t* prefix_start_dev; /* [n] slot_i * capacity */
  int32_t* lengths_dev;            /* [n] cached length of request i; advanced in place */
  int32_t capacity;
  int32_t* status_dev;             /* optional [1]; SG_ERANGE on overflow */
} SgKvCommitArgs;

int sg_kv_commit(const SgKvCommitArgs* args, sg_stream_t stream);

/* ------------------------------------------------------------------------
 * (B') Non-persistent split: rebuild every request's cache from one packed
 * wave, all layers in one launch.
 *
 * Replaces _split_compacted_sequence_caches (CTBD:409-450), the path taken
 * without the persistent arena: request i's new cache is its old prefix
 * (L_i tokens at c_i of the packed prefix) followed by its kept tree rows,
 *   out[l][g, o_i + t]       = prefix[l][g, c_i + t]                t < L_i
 *   out[l][g, o_i + L_i + t] = tree[l][q_i + keep_i[t], g]          t < keep_len_i
 * with q_i = row_offset[i].  A kept row outside [0, row_offset[i+1] - q_i), or
 * L_i + keep_len_i above max_tokens, is not copied and sets *status_dev to
 * SG_EINVAL.
 * ---------------------------------------------------------------------- */
typedef struct SgKvSplitArgs {
  int32_t num_layers;
  int32_t num_requests;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t max_tokens;              /* >= max_i (L_i + keep_len_i) */
  int32_t keep_stride;
  /* packed prefix per layer: element (head g, token t) at base + g*head_stride + t*token_stride */
  const void* const* k_prefix_layers_dev;
  const void* const* v_prefix_layers_dev;
  int64_t prefix_head_stride, prefix_token_stride;
  /* this wave's tree-row K/V per layer [R, Hkv, D] */
  const void* const* k_tree_layers_dev;
  const void* const* v_tree_layers_dev;
  int64_t tree_row_stride, tree_head_stride;
  /* new caches per layer, same element addressing as the prefix */
  void* const* k_out_layers_dev;
  void* const* v_out_layers_dev;
  int64_t out_head_stride, out_token_stride;
  const int64_t* cache_offset_dev; /* [n] c_i */
  const int32_t* old_length_dev;   /* [n] L_i */
  const int32_t* row_offset_dev;   /* [n+1] */
  const int32_t* keep_rows_dev;    /* [n, keep_stride] local rows, ascending path order */
  const int32_t* keep_len_dev;     /* [n] */
  const int64_t* out_offset_dev;   /* [n] o_i, first token of request i's new cache */
  int32_t* status_dev;             /* optional [1]; SG_EINVAL, never cleared */
} SgKvSplitArgs;

int sg_kv_split(const SgKvSplitArgs* args, sg_stream_t stream);

/* ------------------------------------------------------------------------
 * (C) Temperature-1 tree rejection sampling over a packed wave.
 *
 * Replaces the fp32 softmax + ancestral verification of the formal path
 * (probabilities SMP:29-36 via CTBD:1821-1824, tree_verify_ancestral_batched
 * SMP:903-950) and the inline CUDA samplers (FTS:103-2058, sparse-exit layout
 * FTS:683-824): per request, starting at the root row, the route uniform
 * u[2d] accepts the first child (ascending node order) whose cumulative
 * target mass exceeds u[2d]*Z; otherwise u[2d+1] draws the bonus token from
 * the complement of the children (full row at a leaf), fallback = largest
 * non-child token (FTS:804-818).  fp32 throughout with a fixed reduction
 * order, so results are bit-reproducible.
 * ---------------------------------------------------------------------- */
typedef struct SgTreeSampleArgs {
  int32_t num_requests;
  int32_t num_rows;
  int32_t vocab;              /* V <= 524288 */
  int32_t max_depth;          /* accept_nodes slots per request */
  int32_t logits_dtype;       /* SG_DTYPE_F32, SG_DTYPE_BF16 or SG_DTYPE_F16 (the
                                 reference's logits kernels take f16/bf16/f32,
                                 FTS:941-1301) */
  const void* logits_dev;     /* [R, logits_row_stride] target logits (T = 1) */
  int64_t logits_row_stride;  /* elements */
  const int32_t* row_offset_dev; /* [n+1]; row_offset[n] <= num_rows (a request
                                    outside the num_rows rows is a broken walk) */
  const int32_t* parent_dev;     /* [R] local parent, -1 for roots */
  const int32_t* token_dev;      /* [R] draft token of each node (root entry unused) */
  const float* uniforms_dev;     /* [n, uniform_stride] fp32 in [0,1) */
  int32_t uniform_stride;        /* >= 2*(max_depth+1) */
  float* row_max_dev;            /* [R] scratch/output: row max */
  float* row_sum_dev;            /* [R] scratch/output: sum of exp(x - max) */
  int32_t* accept_nodes_dev;     /* [n, max_depth] local node ids, -1 padded */
  int32_t* accept_len_dev;       /* [n] */
  int32_t* bonus_dev;            /* [n] */
  int32_t* keep_rows_dev;        /* optional [n, max_depth+1]: [0] + nodes, -1 padded */
  int32_t* status_dev;           /* optional [1]: cleared to 0 by the call, then
                                    SG_EINVAL if a walk broke the contract */
  void* workspace_dev;           /* >= sg_tree_sample_workspace_bytes(): each
                                    statistics row's slab pairs (max and sum of
                                    exp per 2048-token slab), and for the
                                    complement draw per-slab and per-line totals
                                    of the exit rows and each request's exit node
                                    and children */
  size_t workspace_bytes;
  /* Lazy projection (FTS:2840-3019, SMP:738-832): only the rows a walk can
   * route from were projected (sg_lm_head below). */
  const int32_t* logits_row_dev; /* optional [num_rows]: logits row of each packed
                                    node, or -1 when the node was not projected,
                                    which only a node without children may be;
                                    NULL: node r reads logits row r */
  int32_t num_logits_rows;       /* rows of logits, row_max and row_sum; 0 means
                                    num_rows */
  int32_t flags;                 /* SG_SAMPLE_STATS_READY: row_max/row_sum already
                                    hold every logits row's statistics (as
                                    sg_lm_head writes them); no statistics pass */
  int32_t* terminal_leaf_dev;    /* optional [n]: the walk's last node when its row
                                    was not projected -- its bonus is then -1 and
                                    the caller projects that leaf and draws from it
                                    (FTS:2965-2989) -- else -1 */
} SgTreeSampleArgs;

#define SG_SAMPLE_STATS_READY 1

/* Row statistics of all packed rows followed by the per-request walk. */
int sg_tree_sample(const SgTreeSampleArgs* args, sg_stream_t stream);

/* Scratch bytes sg_tree_sample needs for num_requests requests over vocab,
 * with num_rows statistics rows: the rows whose statistics the call computes
 * (num_logits_rows, or num_rows without a row map), 0 with
 * SG_SAMPLE_STATS_READY.  Per 2048-token slab 8 bytes per statistics row and
 * 36 bytes per request, plus 4,112 bytes per request.  No reference
 * counterpart. */
int64_t sg_tree_sample_workspace_bytes(int32_t num_requests, int32_t num_rows, int32_t vocab);

/* Size of the static per-GPU scratch of sg_tree_sample_noalloc (4 MiB: e.g.
 * 128 requests and 4,096 statistics rows at vocab 151,936). */
#define SG_TREE_SAMPLE_NOALLOC_SCRATCH_BYTES (4u << 20)

/* sg_tree_sample without any device allocation: the workspace is a static
 * device array of SG_TREE_SAMPLE_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends.  args->workspace_dev must be NULL and workspace_bytes 0; calls
 * whose sg_tree_sample_workspace_bytes() exceeds the maximum return SG_EINVAL.
 * The caller still passes every input and output.  Calls that overlap on one
 * GPU (several streams or threads) race on the shared scratch.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int sg_tree_sample_noalloc(const SgTreeSampleArgs* args, sg_stream_t stream);

/* Row statistics only (max and sum of exp of each logits row). */
int sg_row_stats(const void* logits_dev, int32_t logits_dtype, int64_t row_stride,
                 int32_t vocab, int32_t num_rows, float* row_max_dev, float* row_sum_dev,
                 sg_stream_t stream);

/* ------------------------------------------------------------------------
 * (D) LM head with fused softmax statistics (lazy projection).
 *
 * Replaces lm_head(hidden) + probabilities(...) on the rows a tree walk can
 * need: the internal rows of every request (FTS:2899-2913) and, in a second
 * call, the leaves the walks reached (FTS:2974-2984); single-request law
 * SMP:738-832, call site CTBD:1807-1824.  logits[r] = weight . hidden[row_index[r]]
 * in fp32 over bf16 inputs, rounded to bf16 (nearest even).  From the rounded
 * logits: per 128-token tile t of row r, (max, sum of E(x - max)) in
 * tile_stats[r][t], and the row's (max, sum) in row_max/row_sum, which
 * sg_tree_sample takes with SG_SAMPLE_STATS_READY.  Summation order: tile
 * tokens 128t + 32b + 8q + 4h + e form half h, summed in increasing (b, q, e),
 * z = z_0 + z_1; tiles merge into lane t % 64 in increasing t, then an xor
 * butterfly over the 64 lanes.
 * ---------------------------------------------------------------------- */
typedef struct SgLmHeadArgs {
  int32_t num_rows;              /* Rp >= 0 rows to project */
  int32_t hidden_size;           /* H, a positive multiple of 64 */
  int32_t vocab;                 /* V >= 1 */
  int32_t num_hidden_rows;       /* rows of hidden_dev (row_index range) */
  const void* hidden_dev;        /* bf16 [num_hidden_rows, hidden_row_stride], < 4 GiB */
  int64_t hidden_row_stride;     /* elements, multiple of 8 */
  const int32_t* row_index_dev;  /* optional [Rp]: hidden row of projected row r;
                                    NULL: row r */
  const void* weight_dev;        /* bf16 [V, weight_row_stride] (lm_head.weight) */
  int64_t weight_row_stride;     /* elements, multiple of 8 */
  void* logits_dev;              /* bf16 [Rp, logits_row_stride] output */
  int64_t logits_row_stride;     /* elements, multiple of 8, >= V */
  float* tile_stats_dev;         /* [Rp, sg_lm_head_tile_count(V), 2] output */
  float* row_max_dev;            /* [Rp] output */
  float* row_sum_dev;            /* [Rp] output */
  int32_t* status_dev;           /* optional [1]: SG_EINVAL when a row index lies
                                    outside [0, num_hidden_rows); never cleared */
} SgLmHeadArgs;

int sg_lm_head(const SgLmHeadArgs* args, sg_stream_t stream);

/* 128-token statistics tiles per row: ceil(V / 128), or -1 for V < 1. */
int64_t sg_lm_head_tile_count(int32_t vocab);

/* Packed weight layout for sg_lm_head_packed (no reference counterpart: a
 * one-time re-layout of lm_head.weight at model load, kept beside it).
 * Tile t of 256 tokens, 32-dim stage s: 256 rows x 32 dims, row-major, at
 * element ((t * (H / 32) + s) * 256) * 32; rows past V are zero.  Every
 * 16 KiB stage the LM head copies is then contiguous.
 * sg_lm_head_packed_bytes: bytes of the packed weight (ceil(V/256) * 256 * H
 * * 2), or -1 for an invalid size.  sg_lm_head_pack_weight: writes it from
 * the bf16 [V, weight_row_stride] weight (stride a multiple of 8 elements,
 * both pointers 16-byte aligned), enqueued on `stream`. */
int64_t sg_lm_head_packed_bytes(int32_t vocab, int32_t hidden_size);
int sg_lm_head_pack_weight(const void* weight_dev, int64_t weight_row_stride, int32_t vocab,
                           int32_t hidden_size, void* packed_dev, sg_stream_t stream);

/* sg_lm_head with weight_dev pointing to the packed layout above
 * (weight_row_stride is ignored).  Same outputs, bit for bit; a call of up
 * to 64 rows runs about a fifth faster (every weight copy a contiguous
 * 1 KiB), larger calls about 5 % faster. */
int sg_lm_head_packed(const SgLmHeadArgs* args, sg_stream_t stream);

/* ------------------------------------------------------------------------
 * (E) Target decoder layer stack: the fused elementwise stages between the
 * library projections (Qwen3 family).
 *
 * Replace the transformers decoder layers the reference runs through
 * Engine.target_hidden_forward (engine.py:499-517; transformers==4.57.1 per
 * requirements-experiment.txt: Qwen3RMSNorm, Qwen3Attention's q_norm/k_norm
 * and apply_rotary_pos_emb, Qwen3MLP's act_fn(gate) * up) and the draft
 * feature gather of the kept rows (CTBD:2144-2158).  bf16 in and out, fp32
 * inside, with the modules' bf16 rounding points.
 * ---------------------------------------------------------------------- */
typedef struct SgAddRmsNormArgs {
  int32_t num_rows;
  int32_t hidden;                /* multiple of 8, at most 8192 */
  float eps;
  int32_t reserved;
  const void* x_dev;             /* bf16 [R, x_stride] */
  int64_t x_stride;
  const void* residual_dev;      /* optional bf16 [R, residual_stride], added to x first */
  int64_t residual_stride;
  const void* weight_dev;        /* bf16 [hidden] */
  void* out_dev;                 /* bf16 [R, out_stride]: RMSNorm(x + residual) */
  int64_t out_stride;
  void* residual_out_dev;        /* optional bf16 [R, residual_out_stride]: x + residual */
  int64_t residual_out_stride;
} SgAddRmsNormArgs;

/* out = weight * bf16((x + residual) * rsqrt(mean((x + residual)^2) + eps)),
 * with x + residual rounded to bf16 first (the decoder's residual stream). */
int sg_add_rmsnorm(const SgAddRmsNormArgs* args, sg_stream_t stream);

typedef struct SgQkNormRopeArgs {
  int32_t num_rows;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;              /* 64 or 128 */
  float eps;
  int32_t reserved;
  const void* qkv_dev;           /* bf16 [R, qkv_row_stride]: Hq q heads, Hkv k heads,
                                    Hkv v heads of D each (the merged projection) */
  int64_t qkv_row_stride;
  const void* q_norm_dev;        /* bf16 [D] */
  const void* k_norm_dev;        /* bf16 [D] */
  const float* inv_freq_dev;     /* [D/2] rotary inverse frequencies */
  const int64_t* positions_dev;  /* [R] */
  void* q_out_dev;               /* bf16 [R, q_row_stride] as [Hq, D] per row */
  int64_t q_row_stride;
  void* k_out_dev;               /* bf16 [Hkv, kv_head_stride] as [R, D] per head */
  void* v_out_dev;
  int64_t kv_head_stride;
} SgQkNormRopeArgs;

/* Per-head RMSNorm of q and k, rotary embedding of both (rotate-half form,
 * bf16 cos/sin of fp32 angles position * inv_freq), v copied.  The q/k/v rows,
 * norm weights and outputs are read and written 16 bytes at a time: their
 * pointers must be 16-byte aligned and qkv_row_stride, q_row_stride and
 * kv_head_stride multiples of 8 elements (else SG_EINVAL). */
int sg_qk_norm_rope(const SgQkNormRopeArgs* args, sg_stream_t stream);

/* out[r, :I] = bf16(bf16(silu(gate)) * up) with gate = gate_up[r, :I] and
 * up = gate_up[r, I:2I] (Qwen3MLP act_fn(gate_proj(x)) * up_proj(x)). */
int sg_silu_mul(const void* gate_up_dev, int64_t gate_up_row_stride, int32_t num_rows,
                int32_t intermediate, void* out_dev, int64_t out_row_stride,
                sg_stream_t stream);

/* Draft features of the kept rows (CTBD:2144-2158): out[k, l*width ..] =
 * src_dev[l][index_dev[k], :width] for l < num_src, i.e. the kept rows of
 * several layers' hidden states concatenated along the feature dimension.
 * src_dev is a device array of num_src device pointers; an index outside
 * [0, num_src_rows) writes zeros and sets *status_dev (optional) to SG_EINVAL. */
int sg_gather_rows(const void* const* src_dev, int32_t num_src, int64_t src_row_stride,
                   int32_t width, int32_t num_src_rows, const int32_t* index_dev,
                   int32_t num_index, void* out_dev, int64_t out_row_stride,
                   int32_t* status_dev, sg_stream_t stream);

/* sizeof() of the argument structs as compiled into the library, for binding
 * checks: which = 0 SgTreeAttnArgs, 1 SgKvCommitArgs, 2 SgTreeSampleArgs,
 * 3 SgKvSplitArgs, 4 SgLmHeadArgs, 5 SgAddRmsNormArgs, 6 SgQkNormRopeArgs.
 * Returns -1 for an unknown index.  No reference counterpart. */
int64_t sg_abi_struct_size(int32_t which);

/* Measurement helper, no reference counterpart: each of `blocks` workgroups
 * writes four int64 to out_dev[4*b ..]: the XCD it ran on, the shader-clock
 * counter, the constant-rate wall-clock counter, and its hardware id (CU,
 * array and engine).  Two probes bracketing a timed region give, per CU that
 * both saw, its average shader clock over the region. */
int sg_clock_probe(int64_t* out_dev, int32_t blocks, sg_stream_t stream);

/* Rate of the wall-clock counter sg_clock_probe samples, in kHz (-1 on error).
 * No reference counterpart. */
int64_t sg_wall_clock_khz(int32_t device);

/* Test hook: E(x) of the sampler's exp for count values (device arrays). */
int sg_exp_probe(const float* x_dev, float* out_dev, int64_t count,
                 sg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECGROVE_HIP_H */
