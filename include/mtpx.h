/*
 * mtpx -- MI355X (gfx950) single-stream MTP speculative-decode step for the
 * Qwen3.8-125B-A6B affine-4-bit MoE.  C ABI.
 *
 * Conventions (mirroring the mlx-c C ABI the reference's kernels bottom out in,
 * Vendor/mlx-swift/Source/Cmlx/mlx-c/mlx/c/fast.h:145-161, error.h:15-27):
 *   - every entry point returns int: 0 = MTPX_OK, nonzero = error; the message
 *     is in mtpx_last_error() (thread-local);
 *   - opaque handles are structs holding one `void* ctx`, created by *_new and
 *     released by *_free;
 *   - array arguments are plain device pointers to row-contiguous memory
 *     (bf16 as uint16_t bit patterns), sizes are explicit; outputs are written
 *     into caller-owned buffers;
 *   - work is enqueued on the context's HIP stream (mtpx_ctx_set_stream) and is
 *     asynchronous unless the function says otherwise.  One context is not
 *     re-entrant: calls on one context must not overlap.
 *
 * Weight format: MLX affine 4-bit (packed uint32 [N, K/8], element k at bits
 * 4*(k%8) of word k/8; bf16 scales and biases [N, K/gs]; gs in {32, 64}).
 */
#ifndef MTPX_H
#define MTPX_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTPX_OK 0
#define MTPX_ERR_ARG 1   /* invalid argument or unsupported shape */
#define MTPX_ERR_HIP 2   /* HIP runtime error */
#define MTPX_ERR_STATE 3 /* call out of sequence (round state machine) */
#define MTPX_ERR_OOM 4   /* device allocation failed */

/* Context limit of the dense verify/draft path: offset + window <= 2048 positions.  The
 * reference serves the same range on its fast path and hands longer contexts to the sparse
 * QSA indexer path (Runner/FastModel/TrackFastModel.swift:1292, TrackFastHead.swift:106;
 * indexer_budget in fixtures/qwen3_8_125b_a6b_config.json:49), which this library does not
 * build: mtpx_layer_forward, mtpx_head_forward and mtpx_target_verify refuse a window past it
 * with MTPX_ERR_ARG. */
#define MTPX_INDEXER_BUDGET 2048

typedef struct mtpx_ctx_ { void* ctx; } mtpx_ctx;
typedef struct mtpx_kv_ { void* ctx; } mtpx_kv;
typedef struct mtpx_layer_ { void* ctx; } mtpx_layer;
typedef struct mtpx_head_ { void* ctx; } mtpx_head;
typedef struct mtpx_drafter_ { void* ctx; } mtpx_drafter;

/* Thread-local text of the last error (replaces mlx-c's error handler,
 * mlx-c/mlx/c/error.h:15-27). */
const char* mtpx_last_error(void);
/* Library version string. */
const char* mtpx_version(void);

/* ---- context: device, stream and reusable workspace ------------------------
 * Replaces the implicit MLX default stream the reference's kernels run on
 * (Vendor/mlx-swift/Source/MLX/MLXFastKernel.swift:176-183 stream argument). */
int mtpx_ctx_new(mtpx_ctx* out, int device);
int mtpx_ctx_free(mtpx_ctx ctx);
/* Enqueue subsequent work on `hip_stream` (NULL = the legacy default stream). */
int mtpx_ctx_set_stream(mtpx_ctx ctx, void* hip_stream);
/* Return to the context's own non-blocking stream. */
int mtpx_ctx_use_own_stream(mtpx_ctx ctx);
int mtpx_ctx_synchronize(mtpx_ctx ctx);

/* ---- a1: MLX affine 4-bit quantisation on the device -----------------------
 * Replaces mlx::core::affine_quantize (MLX/ops.cpp:5036-5090; CPU semantics
 * MLX/backend/cpu/quantized.cpp:1158-1220). w bf16 [rows, K] -> wq, s, b. */
int mtpx_affine_quantize(mtpx_ctx ctx, const uint16_t* w, int64_t rows, int K, int gs,
                         uint32_t* wq, uint16_t* scales, uint16_t* biases);

/* Seeded N(0, sigma) bf16 fill (Philox4x32-10 + Box-Muller); `tensor` selects
 * an independent stream.  Random-init weights only (the reference loads a
 * checkpoint). */
int mtpx_randn_bf16(mtpx_ctx ctx, uint16_t* out, int64_t n, uint64_t seed, uint32_t tensor,
                    float sigma);

/* ---- packed scale/bias rows ---------------------------------------------------
 * Every q4 matrix may carry, next to its checkpoint-format bf16 scales and
 * biases [rows, K/gs], a packed copy: each (scale, bias) pair as one u32 (scale
 * in the low half) in the GEMV's lane order, mtpx_q4_sb_row_len(K, gs) u32 per
 * row.  The GEMVs then fetch a lane's pairs with one or two vector loads instead
 * of two 2-byte loads per 32-element block; values and results are identical.
 * This is a load-time layout of the MI355X build (no reference counterpart:
 * the reference reads scales and biases separately,
 * MLX/backend/metal/kernels/quantized.h:12-393). */
/* u32 entries per packed row; -1 for an unsupported (K, group_size). */
int mtpx_q4_sb_row_len(int K, int group_size);
/* out u32 [rows, mtpx_q4_sb_row_len(K, gs)] from scales and biases [rows, K/gs]. */
int mtpx_q4_pack_sb(mtpx_ctx ctx, const uint16_t* scales, const uint16_t* biases, int64_t rows,
                    int K, int gs, uint32_t* out);

/* ---- a2-a4, a12: q4 GEMV / small-M GEMM ------------------------------------
 * y[M, N] = x[M, K] . W[N, K]^T, M <= 4096, bf16 out (yf: optional f32 before
 * rounding); sb: packed scale/bias rows or NULL.  Every token's row is the
 * same whatever M (above 8 tokens: a prefill batch's GEMM on the matrix cores
 * where sb is given and the shape allows).  Replaces MLX quantizedMM's
 * qmv_fast / qmv / qmv_wide (MLX/backend/metal/kernels/quantized.h:758,825,989)
 * and the track's TrackQuantWeight.apply / TrackLUTGemv
 * (Runner/FastModel/TrackFastWeights.swift:40-49, Runner/FastModel/TrackAffineLUT.swift:121-368). */
int mtpx_qmv(mtpx_ctx ctx, const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
             const uint32_t* sb, int N, int K, int gs, const uint16_t* x, int M, uint16_t* y,
             float* yf);

/* ---- a5-a11: the MoE block -------------------------------------------------- */
typedef struct {
  int hidden;        /* H */
  int experts;       /* E */
  int top_k;         /* K */
  int expert_width;  /* F (routed and shared) */
  int group_size;    /* gs */
  const uint16_t* router;       /* bf16 [E, H] */
  const uint16_t* shared_gate;  /* bf16 [H]: the shared expert's sigmoid gate row */
  const uint32_t* gate_w; const uint16_t* gate_s; const uint16_t* gate_b; /* [E,F,H/8], [E,F,H/gs] */
  const uint32_t* up_w;   const uint16_t* up_s;   const uint16_t* up_b;
  const uint32_t* down_w; const uint16_t* down_s; const uint16_t* down_b; /* [E,H,F/8], [E,H,F/gs] */
  const uint32_t* sh_gate_w; const uint16_t* sh_gate_s; const uint16_t* sh_gate_b; /* [F,H/8] */
  const uint32_t* sh_up_w;   const uint16_t* sh_up_s;   const uint16_t* sh_up_b;
  const uint32_t* sh_down_w; const uint16_t* sh_down_s; const uint16_t* sh_down_b; /* [H,F/8] */
  /* packed scale/bias rows of the six matrices above (all six, or all NULL) */
  const uint32_t* gate_sb; const uint32_t* up_sb; const uint32_t* down_sb;
  const uint32_t* sh_gate_sb; const uint32_t* sh_up_sb; const uint32_t* sh_down_sb;
  /* The shared-expert gate as an affine-4-bit row [1, H] (the checkpoint's mlp.shared_expert_gate,
   * Sources/MLXFastTransform/Qwen4ExpCheckpointValidation.swift:383-385): when shared_gate_w is set
   * it replaces the bf16 row above (which may then be NULL) and the gate is the q4 GEMV of that row,
   * rounded to bf16 like any GEMV output (the route's gate of Runner/FastModel/TrackFastMoE.swift:780-800);
   * shared_gate_sb: its packed scale/bias row or NULL. */
  const uint32_t* shared_gate_w; const uint16_t* shared_gate_s; const uint16_t* shared_gate_b;
  const uint32_t* shared_gate_sb;
} mtpx_moe_weights;

/* y[M, H] = MoE(x[M, H]) for a decode/verify window of M <= 8 tokens: router
 * GEMV (bf16 weight, f32 activation; the shared-expert gate as one more bf16 row, or as the
 * q4 GEMV of shared_gate_w), top-k (value desc, index asc) + softmax,
 * expert-grouped gate|up + SwiGLU, down + rank-ordered combine + sigmoid-gated
 * shared expert.  Optional outputs (NULL to skip): idx int32 [M, K], w f32
 * [M, K], logits f32 [M, E], n_unique int32 [1] (distinct routed experts).
 * Replaces TrackQwen4ExpFastModel.moeForwardShared's decode branch
 * (Runner/FastModel/TrackFastModel.swift:867-954) and its kernels
 * TrackFastMoEKernels.routerGemv / route / gateUpAct / downCombine
 * (Runner/FastModel/TrackFastMoE.swift:2246-2310, 780-911, 1192-1404, 1412-1576). */
int mtpx_moe_forward(mtpx_ctx ctx, const mtpx_moe_weights* w, const uint16_t* x, int M,
                     uint16_t* y, int32_t* idx, float* wts, float* logits, int32_t* n_unique);

/* mtpx_moe_forward without any allocation: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the window's workspace (router logits, routing, dispatch table, prepared
 * activations, expert activations and outputs) lives in a static device scratch array of 2 MiB per
 * GPU, held until the process ends; windows that need more are refused (MTPX_ERR_ARG).  The
 * context must exist (mtpx_ctx_new looks the array up).  Same arguments, kernels and bits as
 * mtpx_moe_forward.  Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (two contexts or streams at once) race. */
int mtpx_moe_forward_noalloc(mtpx_ctx ctx, const mtpx_moe_weights* w, const uint16_t* x, int M, uint16_t* y,
                             int32_t* idx, float* wts, float* logits, int32_t* n_unique);

/* ---- a13-a15: attention pieces -----------------------------------------------
 * attn_prep: qkv rows [S, QW] = q(HQ*D) | gate(HQ*D) | k(HK*D) | v(HK*D) | ...
 * -> q [S, HQ, D]; k and v written into the cache (layout [HK, tmax, D]) at
 * positions pos0 .. pos0+S-1.  RMSNorm (eps) + rotate-half RoPE on the first
 * `rot` dims with bf16 tables cos/sin [positions, rot].
 * Replaces TrackFastKernels.attnPrep (Runner/FastModel/TrackFastKernels2.swift:381-476)
 * plus the cache append of Qwen4ExpAttentionCache.updateAndAttend
 * (called at Runner/FastModel/TrackFastModel.swift:790-792). */
int mtpx_attn_prep(mtpx_ctx ctx, const uint16_t* qkv, int S, int QW, int HQ, int HK, int D,
                   int rot, const uint16_t* qnorm, const uint16_t* knorm, float eps,
                   const uint16_t* cos_t, const uint16_t* sin_t, int pos0, uint16_t* q,
                   uint16_t* kcache, uint16_t* vcache, int64_t tmax);

/* Verify attention of S queries against T cached positions (key i visible to
 * query s iff i <= T - S + s), GQA HQ/HK, f32 online softmax.  out bf16
 * [S, HQ, D] (optional) and out_gated = out * sigmoid(gate) [S, HQ*D] with the
 * gate read from qkv[:, gate_off:] (optional).
 * Replaces the SDPA vector kernels (MLX/backend/metal/kernels/sdpa_vector.h:14-175,
 * MLX/backend/metal/scaled_dot_product_attention.cpp:364-452) and
 * TrackFastKernels.attnGate (Runner/FastModel/TrackFastKernels2.swift:478-510). */
int mtpx_attn_verify(mtpx_ctx ctx, const uint16_t* q, int S, int HQ, int HK, int D,
                     const uint16_t* kcache, const uint16_t* vcache, int64_t tmax, int T,
                     float scale, const uint16_t* qkv, int QW, int gate_off, uint16_t* out,
                     uint16_t* out_gated);

/* Row RMSNorm (H <= 4096); with resid != NULL the input is bf16(x + resid), also
 * written to sum_out when that is not NULL. */
int mtpx_rmsnorm(mtpx_ctx ctx, const uint16_t* x, const uint16_t* resid, int M, int H,
                 const uint16_t* w, float eps, uint16_t* sum_out, uint16_t* y);

/* ---- a16: KV cache with rollback ----------------------------------------------
 * Contiguous bf16 K and V [kv_heads, tmax, head_dim]; rollback = offset rewind
 * (Qwen4ExpAttentionCache.trim, used at Runner/Qwen4ExpMTPDrafter.swift:461-470
 * and Runner/Qwen4ExpRunner.swift:385-394). */
int mtpx_kv_new(mtpx_ctx ctx, int kv_heads, int head_dim, int64_t tmax, mtpx_kv* out);
int mtpx_kv_free(mtpx_kv kv);
int mtpx_kv_offset(mtpx_kv kv, int64_t* offset);
int mtpx_kv_set_offset(mtpx_kv kv, int64_t offset);
/* rewind by n positions; *trimmed receives the count actually removed */
int mtpx_kv_trim(mtpx_kv kv, int64_t n, int64_t* trimmed);
int mtpx_kv_buffers(mtpx_kv kv, uint16_t** k, uint16_t** v, int64_t* tmax);

/* ---- a18, a21: argmax and greedy acceptance ---------------------------------
 * argmax over V per row, lowest id on ties (Runner/Qwen4ExpMTPDrafter.swift:25-27).
 * A NaN ranks as -inf and never wins; a row of only -inf / NaN gives 0 (MLX's argmax,
 * MLX/backend/metal/kernels/arg_reduce.metal:42-62). */
int mtpx_argmax_rows(mtpx_ctx ctx, const float* x, int rows, int64_t V, int32_t* out);
/* The two best entries of each row: ids int32 [rows, 2] and values f32 [rows, 2] (exact copies of
 * the logits; a NaN ranks as -inf), in the argmax order: value descending, lowest id first among
 * equal values, so ids[r][0] is the row's argmax; V >= 2.  The MTP policy's top-two query
 * cbv2MTPTopTwo (Runner/FastModel/TrackFastModel.swift:1456-1460, CBv2MTPPolicyTopTwoProviding),
 * which the reference answers in the un-vendored engine core. */
int mtpx_top_two(mtpx_ctx ctx, const float* logits, int rows, int64_t V, int32_t* ids, float* values);
int mtpx_top_two_bf16(mtpx_ctx ctx, const uint16_t* logits, int rows, int64_t V, int32_t* ids, float* values);
/* logits f32 [k+1, V] (verify rows), drafts int32 [k] -> out3 int32 {n accepted,
 * bonus token, KV rollback index = kv_offset + n + 1}.  The engine-core accept
 * loop (docs/qwen38-125b-a6b-port-notes.md:313-343), decided on the device. */
int mtpx_accept_greedy(mtpx_ctx ctx, const float* logits, int k, int64_t V,
                       const int32_t* drafts, int32_t kv_offset, int32_t* out3);

/* The same decision on bf16 logits (the verify's output), with optional device outputs:
 * argmax_out int32 [k+1] (every row's argmax) and tokens_out int32 [k+1] (the committed
 * tokens: drafts[0..n-1], then the bonus), so a round needs no second argmax and no f32 copy. */
int mtpx_accept_greedy_bf16(mtpx_ctx ctx, const uint16_t* logits, int k, int64_t V, const int32_t* drafts,
                            int32_t kv_offset, int32_t* out3, int32_t* argmax_out, int32_t* tokens_out);

/* Benchmark forcing hook (the MTP head's output forced to the target's at rate
 * p through a seeded mask).  With probability p -- Philox4x32-10, key = seed, counter =
 * {pos lo, pos hi, 0x46524345, 0}, so the decision belongs to the position -- *token =
 * teacher[pos] (device int32).  No reference counterpart: a test hook on the drafter output. */
int mtpx_force_draft(mtpx_ctx ctx, int32_t* token, const int32_t* teacher, int64_t pos, float p, uint64_t seed);

/* ---- a22: temperature rejection sampling (no reference counterpart) ----------
 * Speculative sampling (Leviathan et al. 2023): draft i is accepted when u * p_d(d_i) < p_t(d_i),
 * the first rejection samples norm(max(0, p_t - p_d)) of its row, all accepted samples p_t of row
 * k; probabilities at the temperature.  tlogits f32 [k+1, V], dlogits f32 [k, V] (row i proposed
 * drafts[i]) or NULL: the draft distributions are one-hot at the drafts (a greedy drafter, as the
 * reference's MTP head: accept with probability p_t(d_i), a rejection samples p_t without d_i).
 * Philox4x32-10 key = seed, counter = {offset lo, offset hi, i, 0} for i = 1..k+1 (u = word 0,
 * the resampling draw = word 1).  out3 = {n, token, kv_offset + n + 1}. */
int mtpx_accept_sample(mtpx_ctx ctx, const float* tlogits, const float* dlogits, int k,
                       int64_t V, const int32_t* drafts, float temperature, uint64_t seed,
                       uint64_t offset, int32_t kv_offset, int32_t* out3);
/* The same on bf16 logits (the verify's output; dlogits bf16 [k, V] or NULL), with optional
 * tokens_out int32 [k+1]: the committed tokens, drafts[0..n-1] then the sampled token. */
int mtpx_accept_sample_bf16(mtpx_ctx ctx, const uint16_t* tlogits, const uint16_t* dlogits, int k, int64_t V,
                            const int32_t* drafts, float temperature, uint64_t seed, uint64_t offset,
                            int32_t kv_offset, int32_t* out3, int32_t* tokens_out);

/* ---- one full-shape decoder layer (attention + MoE) for verify windows -------
 * x -> h1 = rms(x); qkv = W_qkv h1; prep + KV append; verify attention with
 * output gate; o = W_o att; s = x + o; h2 = rms(s); y = s + MoE(h2).
 * Replaces the attention + MoE sublayers of the fast forward
 * (Runner/FastModel/TrackFastModel.swift:747-795, 867-954) without the
 * hyper-connection mixers. */
typedef struct {
  int hidden, experts, top_k, expert_width, group_size;
  int heads, kv_heads, head_dim, rot_dims, index_dim;
  float rope_theta, eps;
  int64_t max_positions;
} mtpx_layer_config;

typedef struct {
  const uint16_t* attn_norm; const uint16_t* post_norm; /* bf16 [H] */
  const uint32_t* qkv_w; const uint16_t* qkv_s; const uint16_t* qkv_b; /* [QW, H] */
  const uint16_t* q_norm; const uint16_t* k_norm; /* bf16 [D] */
  const uint32_t* o_w; const uint16_t* o_s; const uint16_t* o_b; /* [H, HQ*D] */
  const uint16_t* rope_cos; const uint16_t* rope_sin; /* bf16 [max_positions, rot] */
  mtpx_moe_weights moe;
  int qkv_rows;
  const uint32_t* qkv_sb; const uint32_t* o_sb; /* packed scale/bias rows (or NULL) */
} mtpx_layer_weights;

int mtpx_layer_new_random(mtpx_ctx ctx, const mtpx_layer_config* cfg, uint64_t seed,
                          mtpx_layer* out);
int mtpx_layer_free(mtpx_layer layer);
int mtpx_layer_weights_get(mtpx_layer layer, mtpx_layer_weights* out);
/* y[M, H] for M tokens at the cache's offset; advances the offset by M. */
int mtpx_layer_forward(mtpx_ctx ctx, mtpx_layer layer, mtpx_kv kv, const uint16_t* x, int M,
                       uint16_t* y);
/* ---- a18: shortlist draft argmax ----------------------------------------------
 * The drafter's headStep tail (Runner/Qwen4ExpMTPDrafter.swift:68-75, 91-108,
 * 122-153): logits = bf16(W_sl x) over the shortlist rows of lm_head (q4
 * [rows, H]), argmax over the bf16 logits (lowest position on ties), mapped
 * through ids (ascending) -> out[0].  x is one bf16 row [H] on the device. */
int mtpx_shortlist_argmax(mtpx_ctx ctx, const uint16_t* x, int H, const uint32_t* w,
                          const uint16_t* s, const uint16_t* b, const uint32_t* sb,
                          int group_size, int rows, const int32_t* ids, int32_t* out);

/* ---- a17: the MTP head (one draft step) ------------------------------------------
 * TrackQwen4ExpMTPModule.callAsFunction (Runner/Qwen4ExpMTP.swift:101-130) over
 * the fast kernels of TrackFastHead.forward (Runner/FastModel/TrackFastHead.swift:101-153):
 *   e = fc_embedding(rms(embed(ids)));  h = fc_hidden(rms_W(multi)) per stream
 *   hyper = e (every stream) + h
 *   attention block : (st, n) = hc_norm(hyper); (x, j) = mix(attn_hc, n); a = attn(x)
 *   MoE block       : (st, n) = hc_norm(st + a*j); (x, j) = mix(mlp_hc, n); m = MoE(x)
 *   multi_next, n   = hc_norm(st + m*j);  sample = mix(final_hc, n)
 *   draft           = shortlist argmax of the last row's sample
 * mix(hc, n): lo = down n, inj = inject n, w = up silu(lo),
 *   x = sum over streams of sigmoid(w) * n, j = 2 * sigmoid(inj). */
typedef struct {
  const uint32_t* w; const uint16_t* s; const uint16_t* b; /* q4 matrix; w == NULL: absent */
  const uint32_t* sb;                                      /* packed scale/bias rows or NULL */
} mtpx_q4;

/* One hyper-connection mixer (TrackHC, Runner/FastModel/TrackFastModel.swift:182-195,
 * bound at :374-402). */
typedef struct {
  const uint16_t* norm_scale; /* bf16 [hc*H]: hc_norm weight / hc_count */
  mtpx_q4 down;               /* [lowrank, hc*H] input_mix_weight_down */
  mtpx_q4 inject;             /* [hc, hc*H] block_inject_weight (w == NULL: none) */
  mtpx_q4 up;                 /* [hc*H, lowrank] input_mix_weight_up */
} mtpx_hc_weights;

typedef struct {
  mtpx_layer_config layer;     /* the head's decoder layer (attention + MoE) */
  int hc;                      /* hc_count (4) */
  int lowrank;                 /* hc_lowrank (320) */
  int64_t vocab;               /* rows of embed_tokens / lm_head (248320) */
  int shortlist_low;           /* shortlist ids 0..low-1 (98304; padded so the count % 8 == 0) */
  int64_t shortlist_special_from; /* plus ids special_from..vocab-1 (248044) */
} mtpx_head_config;

typedef struct {
  mtpx_q4 embed;                       /* [vocab, H] the target's embed_tokens */
  const uint16_t* pre_norm_embedding;  /* bf16 [H] */
  const uint16_t* pre_norm_hidden;     /* bf16 [hc*H]: one statistic over the flat row */
  mtpx_q4 fc_embedding;                /* [H, H] */
  mtpx_q4 fc_hidden;                   /* [H, H], applied to each stream */
  mtpx_hc_weights attn_hc, mlp_hc, final_hc; /* final_hc has no inject */
  mtpx_layer_weights layer;            /* attn_norm / post_norm unused */
  mtpx_q4 shortlist;                   /* [shortlist_rows, H] lm_head rows */
  const int32_t* shortlist_ids;        /* int32 [shortlist_rows], ascending */
  int shortlist_rows;
} mtpx_head_weights;

int mtpx_head_new_random(mtpx_ctx ctx, const mtpx_head_config* cfg, uint64_t seed, mtpx_head* out);
/* Adopt a checkpoint's MTP head (adoptMTPHead, Runner/Qwen4ExpRunner.swift:324-342) from caller-owned
 * device tensors, as mtpx_target_adopt: embed is the target's embed_tokens (the head has none),
 * shortlist the lm_head rows of shortlist_ids (ascending, shortlist_rows a multiple of 8). */
int mtpx_head_adopt(mtpx_ctx ctx, const mtpx_head_config* cfg, const mtpx_head_weights* weights, int pack_sb,
                    mtpx_head* out);
int mtpx_head_free(mtpx_head head);
int mtpx_head_weights_get(mtpx_head head, mtpx_head_weights* out);
/* One head application over S inputs at the cache's offset (advances it by S): a draft step
 * (S <= 8) or a batch of up to 256 backlog positions (the drafter's flush after a prompt; every
 * output equals that of windows of 8 in turn): ids int32 [S] and multi bf16 [S, hc*H] on the
 * device -> multi_next bf16 [S, hc*H], sample bf16 [S, H] (may be NULL), draft int32 [1] (the
 * last row's shortlist argmax; may be NULL).  An id outside [0, vocab) embeds as a zero row. */
int mtpx_head_forward(mtpx_ctx ctx, mtpx_head head, mtpx_kv kv, const int32_t* ids, int S,
                      const uint16_t* multi, uint16_t* multi_next, uint16_t* sample,
                      int32_t* draft);

/* ---- a19: the drafter's per-request round state ---------------------------------
 * CBv2MTPRequestStatefulDrafter as TrackQwen4ExpInlineMTPAssistant implements it
 * (Runner/Qwen4ExpMTPDrafter.swift:162-475).  A drafter owns the head's KV cache
 * for one request and the trusted target transitions (multi[t], token[t+1]) not
 * yet in it.  Tokens and multi streams are device pointers (int32, bf16 [n, hc*H]);
 * the state copies what it keeps.  Out-of-sequence calls (the reference's
 * preconditions) return MTPX_ERR_STATE and leave the state unchanged. */
#define MTPX_MAX_DRAFT_DEPTH 6 /* maximumDraftTokens */

typedef struct {
  int64_t cache_offset;      /* head cache positions */
  int64_t committed_inputs;  /* trusted inputs: in the cache or in the backlog */
  int64_t staged_inputs;     /* speculative inputs of the round in flight */
  int64_t backlog_inputs;
  int64_t round_base_offset, round_valid_offset;
  int round_in_flight, round_draft_steps, has_frontier, released;
} mtpx_drafter_info;

/* makeRequestState (:277-279): a fresh state with an empty head cache. */
int mtpx_drafter_new(mtpx_ctx ctx, mtpx_head head, mtpx_drafter* out);
int mtpx_drafter_free(mtpx_drafter d);
/* observeCommittedTarget (:288-316): n committed target inputs and their multi streams. */
int mtpx_drafter_observe(mtpx_drafter d, const int32_t* tokens, const uint16_t* multi, int n);
/* draftStep (:328-366): the first step of a round flushes the backlog plus this
 * carry through the head; later steps feed back the previous draft and multi.
 * -> draft int32 [1], multi bf16 [1, hc*H]. */
int mtpx_drafter_step(mtpx_drafter d, const int32_t* token, const uint16_t* multi, int32_t* draft,
                      uint16_t* multi_out);
/* finalizeRound (:410-441): confirmed verify inputs; n committed drafts with the
 * target's multi streams at their positions. */
int mtpx_drafter_finalize(mtpx_drafter d, int confirmed_inputs, const int32_t* tokens,
                          const uint16_t* multi, int n);
/* discardRound (:443-454). */
int mtpx_drafter_discard(mtpx_drafter d);
/* releaseRequestState (:472-475): the state refuses every later call. */
int mtpx_drafter_release(mtpx_drafter d);
int mtpx_drafter_info_get(mtpx_drafter d, mtpx_drafter_info* out);
/* requestStateBytesPerToken (:267-275). */
int mtpx_drafter_bytes_per_token(mtpx_head head, int64_t* out);

/* ---- a20 (part): the gated-deltanet sublayer of the target's linear-attention layers ----
 * TrackQwen4ExpFastModel.gdnForward (Runner/FastModel/TrackFastModel.swift:655-737):
 *   proj = in_proj(x)  (rows qkv | z | b | a, TrackFastModel.swift:404-432)
 *   per position: causal depthwise conv (kc taps) + SiLU; q/k RMS norm and 1/dk, 1/sqrt(dk)
 *   scales; beta = sigmoid(b); decay = exp(-exp(A_log) * softplus(a + dt_bias))
 *   (TrackFastKernels.swift:48-117); the delta rule with a Kahan key product (:486-605);
 *   gated RMS norm (TrackFastKernels2.swift:325-352);  y = out_proj(gated).
 * Head dims are 128.  Window state: a forward over S positions leaves the committed
 * recurrent state unchanged and keeps a journal of the window; mtpx_gdn_commit(n) makes
 * its first n positions committed (the capture-and-stage of TrackFastModel.swift:726-731,
 * as an offset).  The next forward (or mtpx_gdn_state_store) applies them first. */
typedef struct mtpx_gdn_ { void* ctx; } mtpx_gdn;
typedef struct mtpx_gdn_state_ { void* ctx; } mtpx_gdn_state;

typedef struct {
  int hidden;        /* 2560 */
  int key_heads;     /* linear_num_key_heads (16) */
  int value_heads;   /* linear_num_value_heads (48), a multiple of key_heads */
  int conv_kernel;   /* linear_conv_kernel_dim (4) */
  int group_size;    /* 32 or 64 */
  float eps;         /* gated RMS epsilon (1e-6) */
} mtpx_gdn_config;

typedef struct {
  mtpx_q4 in_proj;              /* [conv_dim + value_heads*128 + 2*value_heads, hidden] */
  const uint16_t* conv_w;       /* bf16 [conv_dim, conv_kernel], conv_dim = (2*key_heads + value_heads)*128 */
  const float* neg_exp_alog;    /* f32 [value_heads]: -exp(A_log) */
  const uint16_t* dt_bias;      /* bf16 [value_heads] */
  const uint16_t* norm_w;       /* bf16 [128] */
  mtpx_q4 out_proj;             /* [hidden, value_heads*128] */
} mtpx_gdn_weights;

int mtpx_gdn_new_random(mtpx_ctx ctx, const mtpx_gdn_config* cfg, uint64_t seed, mtpx_gdn* out);
int mtpx_gdn_free(mtpx_gdn gdn);
int mtpx_gdn_weights_get(mtpx_gdn gdn, mtpx_gdn_weights* out);
/* Per-request recurrent state (Qwen4ExpCacheEvaluation's conv + ssm entries for one layer):
 * zero conv rows and zero state. */
int mtpx_gdn_state_new(mtpx_ctx ctx, const mtpx_gdn_config* cfg, mtpx_gdn_state* out);
int mtpx_gdn_state_free(mtpx_gdn_state st);
/* Committed state in/out (device pointers): conv bf16 [conv_kernel-1, conv_dim], ssm f32
 * [value_heads, 128, 128].  load drops any window; store does not modify the state. */
int mtpx_gdn_state_load(mtpx_ctx ctx, mtpx_gdn_state st, const uint16_t* conv, const float* ssm);
int mtpx_gdn_state_store(mtpx_ctx ctx, mtpx_gdn_state st, uint16_t* conv, float* ssm);
/* The first n (0..window) positions of the last window become committed. */
int mtpx_gdn_commit(mtpx_gdn_state st, int n);
int mtpx_gdn_state_info(mtpx_gdn_state st, int* window, int* committed);
/* The core on given projections: proj bf16 [S, proj_w] -> gated bf16 [S, value_heads*128]. */
int mtpx_gdn_core(mtpx_ctx ctx, mtpx_gdn gdn, mtpx_gdn_state st, const uint16_t* proj, int S,
                  uint16_t* gated);
/* The sublayer: x bf16 [S, hidden] -> y bf16 [S, hidden] (gated may be NULL). */
int mtpx_gdn_forward(mtpx_ctx ctx, mtpx_gdn gdn, mtpx_gdn_state st, const uint16_t* x, int S,
                     uint16_t* y, uint16_t* gated);

/* ---- a20 (part): the PLE n-gram block of the target's layer index 1 -------------------------
 * pleForward (Runner/FastModel/TrackFastModel.swift:1011-1144) with the three-launch kernels of
 * Runner/FastModel/TrackFastPLE.swift:
 *   history = context (the last ctx_len tokens) ++ ids;  per position and head: a row id of the
 *   n-gram table (docs/ngram-cache-design.md:47-96: shifted copies that never cross an eos,
 *   mix = XOR of copy_p * multiplier_p over widths 2..ngram_size, id = mix % vocab[h] + offset[h]);
 *   e = the rows, dequantized ([S, embed_dim]);  key = key_proj(e) [S, hc*H], value = value_proj(e)
 *   [S, H];  per stream c: dot = sum(norm_key(key_c) * norm_query(stream_c)) in bf16;
 *   g = sqrt(max(|dot / sqrt(H)|, 1e-6)) * sign;  gated_c = sigmoid(g) * value;
 *   normed = norm_conv(gated);  out = gated + silu(conv1d_dilated(state ++ normed)).
 * The table (100-byte rows at the model's geometry) is resident in device memory: the row gather
 * of the host row source (Qwen4ExpNGramHostRowSource, TrackFastModel.swift:1033-1067) becomes a
 * device read.  Window state as for the GDN sublayer: a forward leaves the committed conv rows
 * and context alone; mtpx_ple_commit(n) keeps the window's first n positions (the stage /
 * stageCaptured of :1097-1140, as an offset). */
#define MTPX_PLE_MAX_NGRAM 8
#define MTPX_PLE_MAX_HEADS 32
typedef struct mtpx_ple_ { void* ctx; } mtpx_ple;
typedef struct mtpx_ple_state_ { void* ctx; } mtpx_ple_state;

typedef struct {
  int hidden, hc;          /* the stream is hc*hidden wide (hidden % 256 == 0, <= 4096) */
  int embed_dim;           /* ple_embed_dim (2560) = heads * row width */
  int ngram_size;          /* 3: widths 2..ngram_size; also the conv dilation */
  int heads_per_ngram;     /* 8 */
  int conv_kernel;         /* ple_conv_kernel_size (4) */
  int group_size;          /* key/value projections: 32 or 64 */
  int row_group_size;      /* n-gram table rows: 32 */
  int32_t eos;             /* eos_token_id (248044) */
  int64_t vocab_base;      /* ngram_vocab_size_base (20000000): head vocabularies are the primes above it */
  int64_t token_vocab;     /* vocab_size (248320): bounds the multipliers */
  float eps;               /* RMS epsilon (1e-6) */
} mtpx_ple_config;

typedef struct {
  const uint32_t* w; const uint16_t* s; const uint16_t* b; /* [rows, row_dim/8], [rows, row_dim/row_gs] x2 */
  int64_t rows;                                            /* sum of the head vocabularies */
  int64_t multiplier[MTPX_PLE_MAX_NGRAM];                  /* layer_multipliers */
  int64_t vocab[MTPX_PLE_MAX_HEADS];                       /* ngram_heads_vocab_sizes */
  int64_t offset[MTPX_PLE_MAX_HEADS];                      /* ngram_heads_offsets */
} mtpx_ngram_table;

typedef struct {
  mtpx_q4 key_proj;              /* [hc*hidden, embed_dim] */
  mtpx_q4 value_proj;            /* [hidden, embed_dim] */
  const uint16_t* norm_key;      /* bf16 [hc*hidden] */
  const uint16_t* norm_query;    /* bf16 [hc*hidden] */
  const uint16_t* norm_conv;     /* bf16 [hc*hidden] */
  const uint16_t* conv_w;        /* bf16 [hc*hidden, conv_kernel] */
  mtpx_ngram_table table;
} mtpx_ple_weights;

/* Random init: q4 projections, norm weights near 1, conv taps ~ N(0, 0.3), a table of
 * sum(head vocabularies) random rows and multipliers of the documented form (odd, below
 * (2^63-1) / token_vocab / 2) from a splitmix64 stream of the seed. */
int mtpx_ple_new_random(mtpx_ctx ctx, const mtpx_ple_config* cfg, uint64_t seed, mtpx_ple* out);
int mtpx_ple_free(mtpx_ple ple);
int mtpx_ple_weights_get(mtpx_ple ple, mtpx_ple_weights* out);
/* Per-request state: conv rows bf16 [(conv_kernel-1)*ngram_size, hc*hidden] (zero) and the
 * context int32 [max(1, ngram_size-1)] (eos), the reference's fresh-state defaults (:1019-1028). */
int mtpx_ple_state_new(mtpx_ctx ctx, const mtpx_ple_config* cfg, mtpx_ple_state* out);
int mtpx_ple_state_free(mtpx_ple_state st);
/* Committed state in/out (device pointers).  load drops any window; store does not modify it. */
int mtpx_ple_state_load(mtpx_ctx ctx, mtpx_ple_state st, const uint16_t* conv, const int32_t* context);
int mtpx_ple_state_store(mtpx_ctx ctx, mtpx_ple_state st, uint16_t* conv, int32_t* context);
int mtpx_ple_commit(mtpx_ple_state st, int n);
int mtpx_ple_state_info(mtpx_ple_state st, int* window, int* committed);
/* Row ids of the last S positions of a history (device int32 [ctx_len + S]) ->
 * int32 [S, (ngram_size-1)*heads_per_ngram] (-1 where an id falls outside the table):
 * hostRowIds(history:newCount:) (TrackFastModel.swift:1060). */
int mtpx_ngram_row_ids(mtpx_ctx ctx, mtpx_ple ple, const int32_t* history, int S, int32_t* out);
/* One window: ids (device int32 [S], S <= 8), stream bf16 [S, hc*hidden] -> out bf16
 * [S, hc*hidden] (the block's output, gated + silu(conv)) and/or sum = stream + out (either may
 * be NULL; embedded bf16 [S, embed_dim] may be NULL). */
int mtpx_ple_forward(mtpx_ctx ctx, mtpx_ple ple, mtpx_ple_state st, const int32_t* ids, int S,
                     const uint16_t* stream, uint16_t* out, uint16_t* sum, uint16_t* embedded);

/* ---- a20: the target's verify forward ------------------------------------------------------
 * cbv2ForwardWithHiddenCaptured (Runner/FastModel/TrackFastModel.swift:1463-1475) over
 * fastStreams (:1165-1265):  residual = embed(ids);  per layer
 *   (stream, n) = hc_norm(residual + out * inject)   (the first layer: the embedding tiled)
 *   (x, j) = mix(attn_hc, n);   a = gdn(x), or attention(x) on every interval-th layer
 *   (stream, n) = hc_norm(stream + a * j);   (x, j) = mix(mlp_hc, n);   out = MoE(x)
 * then (multi, n) = hc_norm(residual + out * inject) with the final mixer, mixed = mix(final, n)
 * and logits = lm_head(mixed) (:1330-1333).  A verify leaves the committed state alone:
 * attention caches rewind to it and GDN states keep a journal; mtpx_target_commit(n) keeps the
 * window's first n positions.  On the PLE layer (:1188-1200) the first norm's stream goes
 * through the PLE block (mtpx_ple_forward) and is normed again before the attention mixer:
 *   stream = hc_norm(residual + out * inject).stream;  stream += ple(stream, ids);
 *   (stream, n) = hc_norm(stream)   (no inject). */
#define MTPX_LAYER_GDN 0
#define MTPX_LAYER_ATTENTION 1
typedef struct mtpx_target_ { void* ctx; } mtpx_target;
typedef struct mtpx_target_state_ { void* ctx; } mtpx_target_state;

typedef struct {
  mtpx_layer_config layer;       /* attention and MoE dims, group size, eps, max_positions */
  int key_heads, value_heads;    /* GDN heads (dims 128) */
  int conv_kernel;               /* GDN conv taps */
  int num_layers;                /* 48 */
  int full_attention_interval;   /* 4: layer i is attention iff (i + 1) % interval == 0 */
  int hc, lowrank;               /* hyper-connection streams (4), mixer rank (320) */
  int64_t vocab;                 /* 248320 */
  int ple_layer;                 /* the layer with the PLE block (1; -1: none) */
  mtpx_ple_config ple;           /* its geometry (hidden, hc, group_size, eps: the target's) */
} mtpx_target_config;

typedef struct {
  int kind;                      /* MTPX_LAYER_GDN or MTPX_LAYER_ATTENTION */
  mtpx_layer_weights attn;       /* attention weights (attention layers) and the layer's MoE */
  mtpx_gdn_weights gdn;          /* GDN layers */
  mtpx_hc_weights attn_hc, mlp_hc;
  mtpx_ple_weights ple;          /* the PLE layer */
} mtpx_target_layer_weights;

typedef struct {
  mtpx_q4 embed;                 /* [vocab, hidden] */
  mtpx_hc_weights final_hc;      /* no inject */
  mtpx_q4 lm_head;               /* [vocab, hidden] */
} mtpx_target_weights;

int mtpx_target_new_random(mtpx_ctx ctx, const mtpx_target_config* cfg, uint64_t seed, mtpx_target* out);
/* Adopt caller-owned device weights in the checkpoint's MLX layout (runner adoption,
 * Runner/Qwen4ExpRunner.swift:135-229: the serving model holds the SAME loaded tensors, no copy):
 * every q4 matrix and vector is used in place and must outlive the target.  layers [num_layers]
 * in the config's schedule (a GDN layer's MoE in attn.moe, the PLE layer's block in ple; attention
 * norms attn_norm/post_norm unused).  The library adds only: packed scale/bias rows when pack_sb != 0
 * and the caller gave none (else the kernels read the checkpoint's scales/biases), RoPE tables when
 * rope_cos/rope_sin are NULL (rows max_positions), and the n-gram table's head sizes and offsets,
 * which follow from the config (the table must hold at least their sum of rows -- a checkpoint pads it to
 * whole shards, and rows past the sum are never read; the multipliers are the
 * caller's).  gdn.neg_exp_alog is -exp(A_log) as f32.  A missing tensor: MTPX_ERR_ARG. */
int mtpx_target_adopt(mtpx_ctx ctx, const mtpx_target_config* cfg, const mtpx_target_weights* weights,
                      const mtpx_target_layer_weights* layers, int pack_sb, mtpx_target* out);
int mtpx_target_free(mtpx_target t);
int mtpx_target_weights_get(mtpx_target t, mtpx_target_weights* out);
int mtpx_target_layer_weights_get(mtpx_target t, int layer, mtpx_target_layer_weights* out);
/* Per-request caches (Qwen4ExpCBv2LayerCache per attention layer, recurrent state per GDN
 * layer): empty attention caches of max_positions, zero GDN states. */
int mtpx_target_state_new(mtpx_ctx ctx, mtpx_target t, mtpx_target_state* out);
int mtpx_target_state_free(mtpx_target_state st);
/* The cache of attention layer `layer` / the state of GDN layer `layer` (owned by st). */
int mtpx_target_state_kv(mtpx_target_state st, int layer, mtpx_kv* out);
int mtpx_target_state_gdn(mtpx_target_state st, int layer, mtpx_gdn_state* out);
/* The PLE block's state of the PLE layer (owned by st). */
int mtpx_target_state_ple(mtpx_target_state st, mtpx_ple_state* out);
/* Committed positions of every attention cache (a prefix written through mtpx_kv_buffers). */
int mtpx_target_state_set_offset(mtpx_target_state st, int64_t offset);
int mtpx_target_state_info(mtpx_target_state st, int64_t* offset, int* window);
/* Back to a fresh request: every cache empty (offset 0), GDN and PLE states zero / default.
 * A verify that fails after its first launch leaves the state refusing mtpx_target_verify and
 * mtpx_target_commit (MTPX_ERR_STATE) until this call: some layers may already hold the failed
 * window.  (Qwen4ExpCBv2LayerCache / recurrent state re-creation, Runner/Qwen4ExpRunner.swift:385-394.) */
int mtpx_target_state_reset(mtpx_ctx ctx, mtpx_target_state st);
/* S <= 8 tokens (device int32) at the committed offset -> logits bf16 [S, vocab], multi bf16
 * [S, hc*hidden], mixed bf16 [S, hidden] (each may be NULL).  ids in plain host memory: MTPX_ERR_ARG
 * before anything runs. */
int mtpx_target_verify(mtpx_ctx ctx, mtpx_target t, mtpx_target_state st, const int32_t* ids, int S,
                       uint16_t* logits, uint16_t* multi, uint16_t* mixed);
/* The first n (0..window) positions of the last verify become committed. */
int mtpx_target_commit(mtpx_target_state st, int n);
/* Prefill: S >= 1 prompt tokens (device int32) at the committed offset, processed and committed
 * (an open verify window is discarded first) -> logits bf16 [vocab] of the LAST position and multi
 * bf16 [S, hc*hidden] of every position (each may be NULL).  Every output and the state it leaves
 * equal those of verifying and committing the tokens in windows of 8 in turn; the work runs over
 * batches of up to 512 positions at once: one launch per kernel for the whole batch where each
 * position's result is its own (the dense projections as GEMMs on the matrix cores, norms, mixers,
 * attention -- every query attends to the keys up to its own position --, the MoE routed as windows
 * of 8 and its experts over the batch's slots sorted by expert, the GDN recurrence over the batch),
 * the PLE recurrence window by window.  Replaces the runner's prompt prefill windows (Runner/FastModel/TrackP12Prefill.swift:1-237,
 * TrackPrefillSort.swift:1-201, TrackPrefillIndirect.swift:5-227), with the decode path's arithmetic
 * instead of MLX's steel GEMM: the prompt's positions get the bits the verify path gives them.
 * ids (device int32 [S]) in plain host memory: MTPX_ERR_ARG before anything runs. */
int mtpx_target_prefill(mtpx_ctx ctx, mtpx_target t, mtpx_target_state st, const int32_t* ids, int S,
                        uint16_t* logits, uint16_t* multi);
/* Distinct routed experts of each layer's MoE in the last verify (host int32 [num_layers];
 * synchronises), for the algorithmic byte count of the expert GEMVs. */
int mtpx_target_moe_unique(mtpx_ctx ctx, mtpx_target_state st, int32_t* out);

/* ---- the speculative round, device-resident ------------------------------------------------
 * A session = one request: the target's caches, the drafter's request state and the carry (the
 * next input token with the target multi stream of the position before it).  mtpx_round runs
 * k drafter steps, the verify of the carry + k drafts, the greedy accept on the device, ONE
 * readback of its integers (accepted count, bonus, committed tokens), the target commit of
 * n + 1 positions, the drafter finalize with the target's own multi streams, and moves the
 * carry on the device.  k = 0 is a serial decode step.  Replaces the engine core's accept loop
 * (docs/qwen38-125b-a6b-port-notes.md:313-343, the un-vendored mlx-swift-lm) around
 * CBv2MTPRequestStatefulDrafter (Runner/Qwen4ExpMTPDrafter.swift:328-454) and
 * cbv2ForwardWithHiddenCaptured (Runner/FastModel/TrackFastModel.swift:1463-1475). */
typedef struct mtpx_session_ { void* ctx; } mtpx_session;

typedef struct {
  const int32_t* teacher;  /* device int32 [teacher_len]: the token at each absolute position; NULL: no forcing */
  int64_t teacher_len;
  float rate;              /* forcing probability per position */
  uint64_t seed;
} mtpx_force_params;

/* head may be {NULL}: serial decode only (k = 0). */
int mtpx_session_new(mtpx_ctx ctx, mtpx_target target, mtpx_head head, mtpx_session* out);
int mtpx_session_free(mtpx_session s);
/* Back to an empty request (caches reset, a fresh drafter state). */
int mtpx_session_reset(mtpx_session s);
/* The prompt (device int32 [n], offset + n <= MTPX_INDEXER_BUDGET): mtpx_target_prefill in batches
 * of up to 512 positions, each committed and its multi streams observed by the drafter;
 * *first_token (host) = the argmax of the last position, which becomes the carry.  Synchronises
 * once.  ids in plain host memory: MTPX_ERR_ARG, the session unchanged. */
int mtpx_session_prefill(mtpx_session s, const int32_t* ids, int n, int32_t* first_token);
/* One round of draft depth k (0..MTPX_MAX_DRAFT_DEPTH); force may be NULL.  tokens (host, k+1
 * entries) receives the n + 1 committed tokens, *n_tokens = n + 1.  A prefill or round that fails
 * after it began (e.g. a prompt longer than the caches: its first windows are committed) leaves the
 * session refusing every prefill and round with MTPX_ERR_STATE until mtpx_session_reset. */
int mtpx_round(mtpx_session s, int k, const mtpx_force_params* force, int32_t* tokens, int* n_tokens);
/* A round at temperature > 0: the same steps with the greedy accept replaced by speculative
 * sampling over the verify's bf16 logits with one-hot draft distributions (mtpx_accept_sample_bf16
 * with dlogits NULL): key = seed, offset = the session's committed position before the round, so
 * every round draws from its own counters and a round's draws belong to its position.  The output
 * is distributed as sampling the target at that temperature token by token.  temperature == 0 is
 * mtpx_round.  No reference counterpart (the reference decodes greedily). */
int mtpx_round_sampled(mtpx_session s, int k, const mtpx_force_params* force, float temperature, uint64_t seed,
                       int32_t* tokens, int* n_tokens);
/* Committed offset; the session's target state and drafter (owned by the session). */
int mtpx_session_info(mtpx_session s, int64_t* offset, mtpx_target_state* state, mtpx_drafter* drafter);

/* ---- safetensors checkpoints -------------------------------------------------------------------
 * The header reader of Sources/MLXFastCore/Safetensors.swift:75-176 (Safetensors.readHeader): an
 * 8-byte little-endian header length (0 and lengths above 100,000,000 bytes or past the file refused),
 * a JSON object of tensors {dtype, shape, data_offsets} and an optional "__metadata__" string map;
 * offsets within the data section.  Entries are listed in name order; the data is read from a
 * read-only mapping of the file.  Malformed files are refused with MTPX_ERR_ARG and the reference's
 * messages. */
typedef struct mtpx_st_ { void* ctx; } mtpx_st;
int mtpx_st_open(const char* path, mtpx_st* out);
int mtpx_st_free(mtpx_st st);
int mtpx_st_count(mtpx_st st, int64_t* n);
/* Entry i (name order): name, dtype ("BF16", "U32", "I64", ...), shape [ndim] and byte count (pointers
 * valid until mtpx_st_free; any may be NULL). */
int mtpx_st_tensor(mtpx_st st, int64_t i, const char** name, const char** dtype, int* ndim, const int64_t** shape,
                   int64_t* nbytes);
/* The entry index of `name` (MTPX_ERR_ARG and -1 if absent). */
int mtpx_st_find(mtpx_st st, const char* name, int64_t* i);
/* A metadata value, or *value = NULL if the key is absent. */
int mtpx_st_metadata(mtpx_st st, const char* key, const char** value);
/* Copy entry i's bytes to host memory (nbytes must equal its byte count). */
int mtpx_st_read(mtpx_st st, int64_t i, void* dst, int64_t nbytes);

/* A checkpoint: the given safetensors files (a directory stands for every *.safetensors file in it), one
 * tensor name space (a name in two files is refused). */
typedef struct mtpx_checkpoint_ { void* ctx; } mtpx_checkpoint;
int mtpx_checkpoint_open(const char* const* paths, int n, mtpx_checkpoint* out);
int mtpx_checkpoint_free(mtpx_checkpoint ck);
int mtpx_checkpoint_count(mtpx_checkpoint ck, int64_t* n);
/* A target from an MLX affine-4-bit checkpoint of this family (the tensor inventory of
 * Sources/MLXFastTransform/Qwen4ExpCheckpointValidation.swift:312-510; names under `prefix`, NULL =
 * "language_model."): every tensor's dtype and shape is checked against cfg, copied to the device and
 * transformed as the reference's binding does (Runner/FastModel/TrackFastModel.swift:365-575: norm scale
 * = bf16(hc_norm.weight * 1/hc); GDN in-projection rows in_proj_qkv | z | b | a; neg_exp_alog =
 * -exp(float(A_log)); q_proj rows regrouped as every head's query, then every head's gate, followed by
 * k_proj, v_proj and the last index_dim rows of indexer.index_qk_proj; the shared-expert gate as its q4
 * row; the PLE table as its shards' rows in order, with the checkpoint's layer_multipliers, and its
 * ngram_heads_vocab_sizes / offsets checked against the config's), then mtpx_target_adopt (pack_sb as
 * there).  The target owns the device copies.  Replaces the runner's module adoption
 * (Runner/Qwen4ExpRunner.swift:135-229) over mlx-swift-lm's loader. */
int mtpx_target_load(mtpx_ctx ctx, const mtpx_target_config* cfg, mtpx_checkpoint ck, const char* prefix,
                     int pack_sb, mtpx_target* out);
/* The checkpoint's embedded MTP head (prefix + "mtp.": pre_fc_norm_embedding/hidden, fc_embedding/hidden,
 * the final mixer, layers.0 attention + MoE with its two mixers; adoptMTPHead,
 * Runner/Qwen4ExpRunner.swift:324-342) over `target`: the head embeds with the target's embed_tokens and
 * its shortlist rows are copies of the target's lm_head rows; the target must outlive the head. */
int mtpx_head_load(mtpx_ctx ctx, const mtpx_head_config* cfg, mtpx_checkpoint ck, mtpx_target target,
                   const char* prefix, int pack_sb, mtpx_head* out);

/* ---- per-kernel timing (replaces TrackFastProfile, Runner/FastModel/TrackFastWeights.swift:81-98) ----
 * With profiling on, every launch the library issues is bracketed by HIP events
 * on the context stream.  mtpx_profile_dump synchronises and writes one line per
 * kernel name: "<name> <launches> <total ms>\n". */
int mtpx_profile_enable(mtpx_ctx ctx, int on);
int mtpx_profile_reset(mtpx_ctx ctx);
int mtpx_profile_dump(mtpx_ctx ctx, char* buf, size_t n);

/* Algorithmic HBM bytes of the last mtpx_moe_forward / layer forward's MoE on
 * this context (distinct experts read back from the device; synchronises). */
int mtpx_last_moe_bytes(mtpx_ctx ctx, int64_t* bytes, int32_t* n_unique);

#ifdef __cplusplus
}
#endif
#endif
