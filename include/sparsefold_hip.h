/*
 * sparsefold_hip.h -- C ABI of the MI355X (gfx950) gated pair-biased attention library.
 *
 * Every entry point takes plain device pointers, element strides and sizes, and a
 * hipStream_t (passed as void*; NULL = default stream).  Calls are asynchronous on that
 * stream.  The caller owns all memory: outputs and workspaces are allocated by the caller
 * (sizes from the *_workspace_bytes queries).  Return value 0 = success; non-zero = error,
 * with a message from sf_hip_last_error().  No entry point synchronises the device.
 *
 * Element types: "bf16" = IEEE bfloat16 bit patterns (uint16_t), "f32" = float,
 * "u8" = bool as one byte (0 = masked / invalid).
 *
 * Reference interfaces replaced (SparseFold, paths relative to src/sparsefold/):
 *   sf_hip_attention_fwd        backends/torch/attention/sdpa.py:22-121  dot_product_attention
 *   sf_hip_layer_norm_fwd       model/layers/primitives.py:471-497        LayerNorm.forward
 *                               model/diffusion/transformer.py:80-96      AdaptiveLayerNorm.forward
 *   sf_hip_linear_fwd           model/layers/primitives.py:328-372        Linear.forward (einsum,
 *                               bias, residual, sigmoid post-op)
 *   sf_hip_triangle_attn_fwd    model/trunk/blocks.py:293-366             GridSelfAttention.forward
 *                               (vecops op sparsefold_native::grid_self_attention,
 *                                backends/vecops/kernels/registry.py:1188-1233, dense form)
 *   sf_hip_pair_logits_fwd      model/trunk/blocks.py:745-749             SingleActUpdate pair logits
 *                               model/diffusion/transformer.py:430-447    Transformer pair-logit pack
 *                               model/diffusion/transformer.py:655-666    CrossAttTransformer pack
 *   sf_hip_window_gather_fwd    schema/atom_layout.py:61-83               convert (queries_to_keys,
 *                               CrossAttTransformer block key gather, transformer.py:671-673)
 *   sf_hip_self_attention_fwd   model/diffusion/transformer.py:306-345    SelfAttention.forward (+ AdaLN
 *                               :80-96, AdaLN-zero :138-154); SingleActUpdate attention,
 *                               model/trunk/blocks.py:750-763 (vecops ops evoformer_single_act_update,
 *                               diffusion_self_attention)
 *   sf_hip_cross_attention_fwd  model/diffusion/transformer.py:549-585    CrossAttention.forward, with the
 *                               key gather of :671-673 (vecops op diffusion_cross_attention, indexed form)
 *   sf_hip_transition_fwd       model/trunk/blocks.py:84-96                TransitionBlock.forward
 *                               model/diffusion/transformer.py:209-231     TransitionBlock.forward (diffusion)
 */
#ifndef SPARSEFOLD_HIP_H_
#define SPARSEFOLD_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SF_HIP_ABI_VERSION 11

/* ABI version of the loaded library (== SF_HIP_ABI_VERSION it was built with). */
int sf_hip_abi_version(void);

/* Copies the calling thread's last error message (NUL-terminated, truncated to n).
 * Returns the full message length. */
size_t sf_hip_last_error(char* buf, size_t n);

/* ---------------------------------------------------------------------------------------
 * Gated pair-biased attention (flash-style, bf16 MFMA, fp32 softmax / accumulation).
 *
 *   out[b,i,h,:] = softmax_j( scale * q[b,i,h,:].k[b,j,h,:] + bias[b,h,i,j] , masked ) v[b,j,h,:]
 *                  (* sigmoid(gate[b,i,h,:]) when gate != NULL)
 *
 * Batch is two-level, b = (b0, b1) with b0 < B0, b1 < B1; every tensor carries its own
 * element strides for b0 and b1 (0 = broadcast), so a bias shared by all rows / samples
 * costs nothing.  The last dimension of q, k, v, gate and out is contiguous (stride 1);
 * bias is contiguous along keys.  Masks: masked key j for query i <=> !mask_q[b,i] or
 * !mask_k[b,j]; a query whose every key is masked returns the mean of v over all K keys
 * (the reference's -finfo.max additive mask, sdpa.py:62-80).  D, Dv <= 64.
 * ------------------------------------------------------------------------------------- */
typedef struct sf_attention_args {
  int32_t B0, B1, Q, K, H, D, Dv;
  float scale;                                  /* logits scale (1/sqrt(D) if unspecified) */
  const void* q;    int64_t q_s[4];             /* bf16, strides [b0, b1, q, h]            */
  const void* k;    int64_t k_s[4];             /* bf16, strides [b0, b1, k, h]            */
  const void* v;    int64_t v_s[4];             /* bf16, strides [b0, b1, k, h]            */
  const void* bias; int64_t bias_s[4];          /* bf16 or NULL, strides [b0, b1, h, q]    */
  const uint8_t* mask_q; int64_t mq_s[3];       /* u8 or NULL, strides [b0, b1, q]         */
  const uint8_t* mask_k; int64_t mk_s[3];       /* u8 or NULL, strides [b0, b1, k]         */
  const void* gate; int64_t g_s[4];             /* bf16 or NULL (sigmoid gate logits)      */
  void* out;        int64_t o_s[4];             /* bf16, strides [b0, b1, q, h]            */
  /* Work decomposition: 0 = chosen from the sizes (normal use); 1 = query blocks of one
   * (batch, head) share their K/V tiles; 2 = every 32-query block is an independent task;
   * 3 = the shared-bias kernel: B0 = 5 samples, B1 = 1, D = Dv = 48, one bias for all samples
   * (bias_s[0] = 0), no query mask, a key mask shared by the samples, Q % 64 == 0,
   * K % 256 == 0, K <= 4096 (refused with an error otherwise; opt-in only, 0 never picks it).
   * All give the same result up to fp32 summation order; tests select each explicitly. */
  int32_t schedule;
  /* Key / value rows gathered by index (the key windows of CrossAttTransformer read from
   * per-atom K / V, DiffusionCrossAttentionIndexed.cpp:376-411): with kv_index (int32), key j of
   * batch (b0, b1) is row kv_index[b1 * kvi_s + j] of k / v at batch b0 (k_s[1] and v_s[1] are
   * not applied), or row kv_zero_row -- a row of zeros the caller provides -- where kv_mask
   * (u8 or NULL) is 0 or the index lies outside [0, kv_zero_row).  Needs 16-byte aligned q/k/v
   * rows (the direct-to-LDS route). */
  const int32_t* kv_index; const uint8_t* kv_mask; int64_t kvi_s; int32_t kv_zero_row;
} sf_attention_args;

int sf_hip_attention_fwd(const sf_attention_args* a, void* stream);

/* ---------------------------------------------------------------------------------------
 * Row LayerNorm, optionally adaptive (AdaLN):
 *   y[m,:] = LN(x[m,:]) * gamma + beta                       (gamma/beta f32 or NULL)
 *   y[m,:] = LN(x[m,:]) * scale[m % cond_rows,:] + shift[m % cond_rows,:]   (AdaLN)
 * x, y bf16 row-major with row strides; eps as given (reference 1e-5).  C <= 2048.
 * Optional row gather (the key windows of CrossAttTransformer, transformer.py:671-673): with
 * gather_idx, row m = s * gather_rows + r normalises x row s * gather_src_rows + gather_idx[r],
 * or a zero row where gather_mask[r] is 0 or the index is outside [0, gather_src_rows) -- the
 * rows sf_hip_window_gather_fwd would produce, without materialising them.
 * ------------------------------------------------------------------------------------- */
typedef struct sf_layer_norm_args {
  int64_t M; int32_t C; float eps;
  const void* x; int64_t x_rs;                  /* bf16 */
  const float* gamma; const float* beta;        /* f32 [C] or NULL */
  const void* scale; const void* shift;         /* bf16 [cond_rows, C] or NULL (AdaLN) */
  int64_t cond_rows; int64_t cond_rs;
  void* y; int64_t y_rs;                        /* bf16 */
  const int32_t* gather_idx; const uint8_t* gather_mask;   /* [gather_rows] or NULL */
  int64_t gather_rows, gather_src_rows;
} sf_layer_norm_args;

int sf_hip_layer_norm_fwd(const sf_layer_norm_args* a, void* stream);

/* ---------------------------------------------------------------------------------------
 * y[m,n] = post( sum_k x[m,k] * wt[n,k] + bias[n] ) * mul[m % mul_rows, n] + residual[m,n]
 * x bf16 [M,K] (row stride x_rs), wt bf16 [N,K] contiguous (weight pre-transposed so K is
 * contiguous), bias f32 [N] or NULL, residual bf16 or NULL, post = identity | sigmoid,
 * mul bf16 or NULL (multiplier applied after post, rows broadcast modulo mul_rows).
 * Only columns [0, ycols) go to y (ycols = 0 means all N).  Optional second output:
 * columns [tcol0, tcol0+tcols) are also written transposed, yt[n - tcol0, m] (bf16, row
 * stride yt_rs) -- used to emit [H, rows] bias planes.  K % 8 == 0.
 * Gated form (glu = 1, the SwiGLU of the transition blocks, primitives.py:586-631): the weight
 * rows are interleaved pairs, and y[m, j] = swish(v[2j]) * v[2j+1] with v = x wt^T (+ bias), so y
 * has N/2 columns; needs K % 64 == 0, N % 8 == 0 and no mul / residual / post_sigmoid / yt.
 * ------------------------------------------------------------------------------------- */
typedef struct sf_linear_args {
  int64_t M; int32_t N, K;
  const void* x; int64_t x_rs;
  const void* wt;
  const float* bias;
  const void* residual; int64_t r_rs;
  const void* mul; int64_t mul_rows, mul_rs;
  int32_t post_sigmoid;
  void* y; int64_t y_rs; int32_t ycols;        /* y may be NULL when only yt is wanted */
  int32_t tcol0, tcols; void* yt; int64_t yt_rs;
  int32_t glu;                                 /* 1: gated pairs (see above) */
  /* Batched form (batch > 1, K % 64 == 0, no mul / residual / yt): member b reads x + b*x_bs and
   * wt + b*w_bs and writes y + b*y_bs (element strides) -- the per-channel products of the
   * triangle multiplicative update.  batch 0 or 1 = one product. */
  int32_t batch; int64_t x_bs, w_bs, y_bs;
} sf_linear_args;

int sf_hip_linear_fwd(const sf_linear_args* a, void* stream);

/* ---------------------------------------------------------------------------------------
 * Triangle attention, starting (transpose = 0) or ending (transpose = 1) node, whole module:
 *   x = LN(z); bias[h,a,b] = (x W_b)[a,b,h] (untransposed); rows r of x (x^T for ending);
 *   per row: q,k,v,g projections, attention with mask_k = seq[r] & seq[k] and the shared
 *   bias, sigmoid gate, output projection; out = z + update (or update only).
 * z bf16 [N, N, C] contiguous; seq_mask u8 [N]; weights bf16 packed by the host:
 *   w_qkvgb [4*H*D + H, C]  rows: q (h,d), k (h,d), v (h,d), g (h,d), bias (h)
 *   w_o     [C, H*D]        (transposed output projection)
 * ln_w / ln_b f32 [C] (ln_b may be NULL).  Workspace from sf_hip_triangle_workspace_bytes.
 * out may not alias z.  Constraints: C % 8 == 0, H*D <= 1024, D <= 64.  Fast paths (operands in
 * the attention kernel's register layouts): C = 128, H = 4, D = 32 (the trunk) and C = 64, H = 4,
 * D = 16 (the template stack); other shapes run LN, a projection GEMM, strided attention and
 * an output GEMM.
 * ------------------------------------------------------------------------------------- */
typedef struct sf_triangle_args {
  int32_t N, C, H, D;
  int32_t transpose;                            /* 0 starting node, 1 ending node */
  int32_t add_residual;                         /* 1: out = z + update (module output) */
  const void* z;
  const uint8_t* seq_mask;
  const float* ln_w; const float* ln_b;
  const void* w_qkvgb;
  const void* w_o;
  void* out;
  /* Weight-sum limit of the fast paths' fixed-reference-point softmax: a (row, head)
   * whose sum of weights leaves [2^-100, limit] is recomputed by an exact two-pass softmax.
   * 0 = 2^100 (normal use); a smaller positive value sends more rows through the exact path, so
   * that tests can reach it with ordinary logits.  The result does not depend on it beyond
   * rounding. */
  float fixup_sum_limit;
} sf_triangle_args;

size_t sf_hip_triangle_workspace_bytes(int32_t N, int32_t C, int32_t H, int32_t D);
int sf_hip_triangle_attn_fwd(const sf_triangle_args* a, void* workspace, size_t workspace_bytes,
                             void* stream);

/* The same module as separate stages sharing one workspace (the fast paths: C = 128, H = 4,
 * D = 32 and C = 64, H = 4, D = 16), mirroring the
 * reference's projection / attention split of the row-sharded triangle attention
 * (backends/vecops/kernels/registry.py:1236-1309, grid_distributed_projection and
 * grid_distributed_attention):
 *   SF_TRI_STAGE_PROJECT  LN + q/k/v/bias projections into the workspace (also folds the LN
 *                         affine into the packed weight, which the output stage reuses)
 *   SF_TRI_STAGE_ATTEND   attention core (reads the projected operands)
 *   SF_TRI_STAGE_OUTPUT   sigmoid gate (recomputed from LN(z)), output projection (+ residual)
 * Stages run in that order when several bits are set; sf_hip_triangle_attn_fwd == all three.
 * A stage reads what the earlier stages left in the same workspace.
 *   SF_TRI_STAGE_FUSE     with ATTEND and OUTPUT: one attention kernel whose epilogue runs the
 *                         output stage per (row group, 256 queries) once its four heads are done
 *                         (results identical; measured slower on MI355X, so not the default;
 *                         head dim 32 only, ignored for head dim 16).
 *                         ATTEND needs a workspace a PROJECT stage has initialised. */
#define SF_TRI_STAGE_PROJECT 1
#define SF_TRI_STAGE_ATTEND 2
#define SF_TRI_STAGE_OUTPUT 4
#define SF_TRI_STAGE_ALL 7
#define SF_TRI_STAGE_FUSE 8
int sf_hip_triangle_stage_fwd(const sf_triangle_args* a, int32_t stages, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Block-sparse (IBS) form of the same module (head dim 32: C = 128, H = 4, D = 32), the
 * reference's native grid self-attention (vecops op grid_self_attention with index and weight
 * maps, backends/vecops/kernels/registry.py:2946-3040; GridSelfAttention.cpp:134-142,290-306;
 * parameters config.py:65-73): per (row r, head h, query tile t of 32 queries) num_samples slots
 * of (key block of 32 keys, weight) in index_map / weight_map, int32 / f32 [N, H, T, S],
 * T = ceil(N/32); a slot whose index lies outside [0, T) (-1 by convention) or whose weight is
 * <= 0 is unused, and a query tile with no used slot gets o = 0.  generate_maps = 1 samples them (this library's
 * importance sampler: static heaviest blocks to t_prob, num_rand_blocks draws up to tr_prob with
 * a u_prob floor, weight count / (R q); draws hashed from seed and (r, h, t)); 0 reuses the given
 * maps.  At most num_samples valid blocks per tile: all selected, weight 1, i.e. dense attention.
 * Masked rows follow the dense rule.  N <= 8192, num_samples <= 64.  Workspace from
 * sf_hip_triangle_ibs_workspace_bytes (0 = unsupported sizes). */
typedef struct sf_ibs_args {
  int32_t num_samples, num_rand_blocks;
  float t_prob, tr_prob, u_prob;
  int32_t generate_maps;
  uint64_t seed;
  int32_t* index_map;                           /* [N, H, T, S] */
  float* weight_map;                            /* [N, H, T, S] */
} sf_ibs_args;

size_t sf_hip_triangle_ibs_workspace_bytes(int32_t N, int32_t C, int32_t H, int32_t D);
int sf_hip_triangle_attn_ibs_fwd(const sf_triangle_args* a, const sf_ibs_args* p, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Pair logits: plane hp, position p holds (LN(z[p,:]) W)[hp]; z bf16 [P, C] contiguous
 * (C % 8 == 0, C <= 128), ln_w/ln_b f32 [C] (either may be NULL), w_t bf16 [H, C].
 * H <= 64 planes for any C; up to 1024 planes when C == 128 (one pass over z).
 *
 * Output layout (bf16):
 *   seg == 0: out[H, P]                       (plane-major, SingleActUpdate / Transformer pack:
 *                                              planes ordered (super-block, block, head))
 *   seg  > 0: out[H/group, P/seg, group, seg]  plane hp = blk*group + h, position p = u*seg + r
 *              -> element ((blk*(P/seg) + u)*group + h)*seg + r   (CrossAttTransformer pack
 *              "s q k b h -> b s h q k" with seg = Q*K, group = heads per block)
 *   seg > 0 needs P % seg == 0 and H % group == 0.
 * ------------------------------------------------------------------------------------- */
typedef struct sf_pair_logits_args {
  int64_t P; int32_t C, H;                      /* P = number of pair positions */
  const void* z;
  const float* ln_w; const float* ln_b;
  const void* w_t;
  void* out;
  int64_t seg;                                  /* 0 = plane-major output */
  int32_t group, reserved;                      /* heads per block when seg > 0; reserved = 0 */
} sf_pair_logits_args;

int sf_hip_pair_logits_fwd(const sf_pair_logits_args* a, void* stream);

/* ---------------------------------------------------------------------------------------
 * Key-window gather (atom_layout.convert with layout axes (-3,-2)):
 *   keys[s, u, j, :] = gather_mask[u,j] ? src[s, idx[u,j], :] : 0      (idx flat over U*Qw)
 * src bf16 [S, rows, C] contiguous, idx int32 [U*Kw], mask u8 [U*Kw], keys bf16 [S,U*Kw,C].
 * Indices are bounds-checked on the device: an index outside [0, rows) is treated as masked.
 * ------------------------------------------------------------------------------------- */
typedef struct sf_window_gather_args {
  int32_t S, rows, C, UK;
  const void* src; const int32_t* idx; const uint8_t* mask;
  void* keys;
} sf_window_gather_args;

int sf_hip_window_gather_fwd(const sf_window_gather_args* a, void* stream);

/* ---------------------------------------------------------------------------------------
 * Whole attention modules, one call each (every stage is one of the op entry points above, so
 * the numerics are those of the op-level path).  The caller provides the workspace; its size
 * comes from the *_workspace_bytes query for the same arguments.  Weights are the packed forms
 * the Python modules keep: f32 LayerNorm parameters, bf16 weights with K contiguous ([N, K]).
 *
 * Self attention, transformer.py:306-345 (single attention with pair bias, blocks.py:750-763;
 * diffusion token attention), with AdaLN (:80-96) and AdaLN-zero (:138-154):
 *   h = cond ? sigmoid(LN(c) W_scale^T + b_scale) * LN(x) + LN(c) W_shift^T : LN(x) * ln_w + ln_b
 *   [q|k|v|g] = h W_qkvg^T + b_qkvg;  o = attention(q, k, v; mask, bias) * sigmoid(g)
 *   out = (o W_t2^T) * (cond ? sigmoid(c W_zc^T + b_zc) : 1) + (add_residual ? x : 0)
 * x bf16 [S, N, C] contiguous; mask u8 [N] or NULL (key mask); bias bf16 pair logits or NULL,
 * strides [sample, head, query] (keys contiguous; sample stride 0 = shared); cond bf16 [N, Cs]
 * shared by the S samples, or NULL (Cs ignored).  H*D heads, D <= 64.
 * ------------------------------------------------------------------------------------- */
typedef struct sf_self_attention_args {
  int32_t S, N, C, H, D, Cs;
  float scale;                                  /* logits scale; 0 = 1/sqrt(D) */
  int32_t add_residual;
  const void* x;                                /* bf16 [S, N, C] */
  const uint8_t* mask;                          /* u8 [N] or NULL */
  const void* bias; int64_t bias_s[3];          /* bf16 or NULL, strides [sample, head, query] */
  const void* cond;                             /* bf16 [N, Cs] or NULL */
  const float* ln_w; const float* ln_b;         /* no condition: f32 [C] or NULL */
  const float* lnc_w; const float* lnc_b;       /* condition: LN of cond, f32 [Cs] or NULL */
  const void* w_scale; const float* b_scale;    /* bf16 [C, Cs], f32 [C] */
  const void* w_shift;                          /* bf16 [C, Cs] */
  const void* w_qkvg; const float* b_qkvg;      /* bf16 [4*H*D, C] rows q, k, v, g; f32 [4*H*D] or NULL */
  const void* w_t2;                             /* bf16 [C, H*D] */
  const void* w_zc; const float* b_zc;          /* bf16 [C, Cs], f32 [C] (condition only) */
  void* out;                                    /* bf16 [S, N, C] */
  /* Precomputed conditioning of this layer (one layer's columns of the
   * sf_hip_diffusion_conditioning_fwd outputs), or NULL: bf16 [N, C] each, row stride pre_rs.
   * When pre_scale is given, h = pre_scale * LN(x) + pre_shift and the output multiplier is
   * pre_zgate; cond, lnc_*, w_scale, b_scale, w_shift, w_zc and b_zc are not read. */
  const void* pre_scale; const void* pre_shift; const void* pre_zgate; int64_t pre_rs;
} sf_self_attention_args;

size_t sf_hip_self_attention_workspace_bytes(const sf_self_attention_args* a);
int sf_hip_self_attention_fwd(const sf_self_attention_args* a, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Allocation-free form of sf_hip_self_attention_fwd: no reference counterpart.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same kernels and result, with the module's scratch taken from a fixed
 * per-GPU device array of SF_HIP_NOALLOC_SCRATCH_BYTES (held by each GPU the library runs on
 * until the process ends) instead of a workspace.  Sizes whose
 * sf_hip_self_attention_workspace_bytes exceeds it are refused with an error (64 MiB covers
 * single attention up to N = 4096 at C = 384 and a 5 x 1024 x 768 diffusion block).  The call
 * allocates nothing.  All calls on one GPU share the array: calls that overlap in time on one
 * GPU (other streams, other threads) race and must be serialised by the caller. */
#define SF_HIP_NOALLOC_SCRATCH_BYTES (64u << 20)
int sf_hip_self_attention_fwd_noalloc(const sf_self_attention_args* a, void* stream);

/* Cross attention, transformer.py:549-585 (windowed atom attention), both sides conditioned:
 *   hq = AdaLN(xq, cond_q), hk = AdaLN(xk, cond_k) (as above, per side);
 *   [q|g] = hq W_qg^T + b_qg, [k|v] = hk W_kv^T;  o = attention(q, k, v; mask_q, mask_k, bias) * sigmoid(g)
 *   out = (o W_t2^T) * sigmoid(cond_q W_zc^T + b_zc) + (add_residual ? xq : 0)
 * Keys: xk bf16 [S, U, Kw, C], or (CrossAttTransformer, transformer.py:671-673) gathered from
 * the query rows: key row u*Kw + k of sample s = xq[s, gather_idx[u*Kw + k]] (flat index into the
 * U*Qw rows), zero where gather_mask is 0 or the index is out of range (atom_layout.py:78-82).
 * xq bf16 [S, U, Qw, C]; mask_q u8 [U, Qw], mask_k u8 [U, Kw] (NULL = all valid); bias bf16
 * [U, H, Qw, Kw] shared by the S samples or NULL; cond_q [U, Qw, C], cond_k [U, Kw, C]. */
typedef struct sf_cross_attention_args {
  int32_t S, U, Qw, Kw, C, H, D;
  float scale;                                  /* logits scale; 0 = 1/sqrt(D) */
  int32_t add_residual;
  const void* xq;                               /* bf16 [S, U, Qw, C] */
  const void* xk;                               /* bf16 [S, U, Kw, C] or NULL with gather_idx */
  const int32_t* gather_idx; const uint8_t* gather_mask;   /* [U*Kw] or NULL */
  const uint8_t* mask_q; const uint8_t* mask_k;
  const void* bias;                             /* bf16 [U, H, Qw, Kw] or NULL */
  const void* cond_q; const void* cond_k;       /* bf16 [U, Qw, C], [U, Kw, C] */
  const float* lnc_w_q; const float* lnc_b_q; const void* w_scale_q; const float* b_scale_q; const void* w_shift_q;
  const float* lnc_w_k; const float* lnc_b_k; const void* w_scale_k; const float* b_scale_k; const void* w_shift_k;
  const void* w_qg; const float* b_qg;          /* bf16 [2*H*D, C] rows q, g; f32 [2*H*D] or NULL */
  const void* w_kv;                             /* bf16 [2*H*D, C] rows k, v */
  const void* w_t2;                             /* bf16 [C, H*D] */
  const void* w_zc; const float* b_zc;          /* bf16 [C, C], f32 [C] */
  void* out;                                    /* bf16 [S, U, Qw, C] */
  /* Per-atom plan of the key windows (the native CrossAttTransformer's,
   * backends/vecops/modules.py:1302-1400): with gather_idx and pre_q_scale, the keys' condition
   * is the gathered queries' (keys_single_cond = convert(queries_to_keys, queries_single_cond),
   * atom.py:279-281), so both sides' AdaLN terms are per atom, computed once per example
   * (sf_hip_diffusion_conditioning_fwd) and given here: bf16 [U*Qw, C] each, row stride pre_rs.
   * K / V are then projected once per atom and the attention gathers their rows by gather_idx
   * (invalid keys: zero rows, as the gathered activations and conditions are zero there).
   * cond_q, cond_k and the conditioning weights are not read. */
  const void* pre_q_scale; const void* pre_q_shift; const void* pre_k_scale; const void* pre_k_shift;
  const void* pre_zgate; int64_t pre_rs;
} sf_cross_attention_args;

size_t sf_hip_cross_attention_workspace_bytes(const sf_cross_attention_args* a);
int sf_hip_cross_attention_fwd(const sf_cross_attention_args* a, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Transition blocks, whole module, one call:
 *   trunk transition (blocks.py:38-96, TransitionBlock.forward; vecops op transition_block,
 *   native_ops name "evoformer_transition_block"):            h = LN(x) * ln_w + ln_b
 *   diffusion transition (transformer.py:157-231; vecops op diffusion_transition_block,
 *   "diffusion_transition_block"): h = AdaLN(x, cond) as in sf_self_attention_args, or
 *                                   pre_scale * LN(x) + pre_shift (precomputed conditioning)
 *   c = swish(h W_a^T) * (h W_b^T)            (the GatedLinearUnit, primitives.py:586-631)
 *   out = (c W2^T) * (cond ? sigmoid(cond W_zc^T + b_zc) : 1) + (add_residual ? x : 0)
 * x bf16 [S, N, C] (the condition [N, Cs] is shared by the S samples); w1 bf16 [2I, C] with
 * interleaved rows: row 2i = column i of the reference's [C, 2I] weight (the swish half), row
 * 2i + 1 = column I + i; w2 bf16 [C, I].  C % 64 == 0.  Workspace from
 * sf_hip_transition_workspace_bytes. */
typedef struct sf_transition_args {
  int32_t S, N, C, I, Cs;
  int32_t add_residual;
  const void* x;                                /* bf16 [S, N, C] */
  const void* cond;                             /* bf16 [N, Cs] or NULL */
  const float* ln_w; const float* ln_b;         /* no condition: f32 [C] or NULL */
  const float* lnc_w; const float* lnc_b;       /* condition: LN of cond, f32 [Cs] or NULL */
  const void* w_scale; const float* b_scale;    /* bf16 [C, Cs], f32 [C] */
  const void* w_shift;                          /* bf16 [C, Cs] */
  const void* w1;                               /* bf16 [2I, C], interleaved */
  const void* w2;                               /* bf16 [C, I] */
  const void* w_zc; const float* b_zc;          /* bf16 [C, Cs], f32 [C] (condition only) */
  void* out;                                    /* bf16 [S, N, C] */
  const void* pre_scale; const void* pre_shift; const void* pre_zgate; int64_t pre_rs;
} sf_transition_args;

size_t sf_hip_transition_workspace_bytes(const sf_transition_args* a);
int sf_hip_transition_fwd(const sf_transition_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* Triangle multiplicative update, whole module (TriangleMultiplication.forward,
 * blocks.py:486-566, non-distributed), replacing the native triangle_multiplication op
 * (TriangleMultiplication.cpp; native_ops name "triangle_multiplication", config.py:30):
 *   x = LN(z) (left_norm_input); [a|b] = sigmoid(x W_g) * (x W_p), zero where
 *   mask[i] & mask[k] is false, a = projected channels 2c, b = 2c + 1;
 *   outgoing (incoming = 0, "...ikc,...jkc->...ijc"): t[i,j,c] = sum_k a[i,k,c] b[j,k,c]
 *   incoming (incoming = 1, "...kjc,...kic->...ijc"): t[i,j,c] = sum_k a[k,j,c] b[k,i,c]
 *   out = z + (LN(t) (center_norm) W_out) * sigmoid(x W_gate)      (add_residual = 0: no z)
 * z bf16 [N, N, C] contiguous, C = 128; mask u8 [N] or NULL; LN parameters f32 [C] (biases may
 * be NULL); weights bf16 with the input channel contiguous ([out, in]):
 *   w_glu  [4C, C] rows: gate of a (C), gate of b (C), projection of a (C), projection of b (C)
 *          (gate row c of a = gate_projection column 2c, of b = column 2c + 1; likewise the
 *          projection)
 *   w_out  [C, C] output_projection;  w_gate [C, C] gating_linear
 * Workspace from sf_hip_triangle_mult_workspace_bytes (0 = unsupported sizes).  out may not
 * alias z; z, out and the weights 16-byte aligned.  N <= 8192.  The per-channel products run as one
 * batched GEMM over zero-padded [128][Pn][Pn] planes (Pn = N rounded up to 64). */
typedef struct sf_triangle_mult_args {
  int32_t N, C;
  int32_t incoming;                             /* 0 outgoing, 1 incoming edges */
  int32_t add_residual;
  const void* z;                                /* bf16 [N, N, C] */
  const uint8_t* mask;                          /* u8 [N] or NULL */
  const float* ln_w; const float* ln_b;         /* left_norm_input */
  const void* w_glu;                            /* bf16 [4C, C] */
  const float* cn_w; const float* cn_b;         /* center_norm */
  const void* w_out;                            /* bf16 [C, C] */
  const void* w_gate;                           /* bf16 [C, C] */
  void* out;                                    /* bf16 [N, N, C] */
} sf_triangle_mult_args;

size_t sf_hip_triangle_mult_workspace_bytes(int32_t N, int32_t C);
int sf_hip_triangle_mult_fwd(const sf_triangle_mult_args* a, void* workspace, size_t workspace_bytes,
                             void* stream);

/* AdaLN conditioning of L conditioned layers in one call -- the diffusion Transformer's
 * per-layer scale, shift and zero-gate from one shared condition, computed once per Transformer
 * call instead of once per block.  Replaces diffusion_conditioning_packed
 * (backends/vecops/kernels/registry.py:720-760, DiffusionConditioning.cpp:78-222), which the
 * native Transformer calls once per super-block (backends/vecops/modules.py:1083-1092,1151);
 * Transformer.forward hands the same single_cond to every block (transformer.py:452-463).
 * For layer l (transformer.py:80-96 AdaLN, :138-154 AdaLN-zero):
 *   scale_l = sigmoid(LN(c) * lnc_w[l] W_scale,l^T + b_scale,l)
 *   shift_l = LN(c) * lnc_w[l] W_shift,l^T
 *   zgate_l = sigmoid(c W_zc,l^T + b_zc,l)
 * cond bf16 [rows, Cs]; lnc_w f32 [L, Cs] (the condition LayerNorm has no bias,
 * transformer.py:56-59); weights bf16 [L*C, Cs] (layer l = rows [l*C, (l+1)*C), each the
 * layer's [C, Cs] K-contiguous form); b_scale, b_zc f32 [L*C].  Outputs bf16 [rows, L*C] with
 * row stride out_rs >= L*C: layer l in columns [l*C, (l+1)*C).  scale and zgate hold values
 * after the sigmoid (the reference stores them before it and applies it in the block).
 * LN(c) is computed once and lnc_w is folded into the weights, (LN(c) * g) W^T = LN(c) (W * g)^T,
 * so each output is one GEMM of M = rows, N = L*C, K = Cs.  Cs % 8 == 0, Cs <= 2048. */
typedef struct sf_diffusion_conditioning_args {
  int64_t rows; int32_t L, C, Cs;
  const void* cond;                             /* bf16 [rows, Cs] */
  const float* lnc_w;                           /* f32 [L, Cs] */
  const void* w_scale; const float* b_scale;    /* bf16 [L*C, Cs], f32 [L*C] or NULL */
  const void* w_shift;                          /* bf16 [L*C, Cs] */
  const void* w_zc; const float* b_zc;          /* bf16 [L*C, Cs], f32 [L*C] or NULL */
  void* scale; void* shift; void* zgate;        /* bf16 [rows, L*C], row stride out_rs */
  int64_t out_rs;
} sf_diffusion_conditioning_args;

size_t sf_hip_diffusion_conditioning_workspace_bytes(const sf_diffusion_conditioning_args* a);
int sf_hip_diffusion_conditioning_fwd(const sf_diffusion_conditioning_args* a, void* workspace,
                                      size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSEFOLD_HIP_H_ */
