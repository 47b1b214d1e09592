/*
 * mtpx CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the arithmetic of the single-stream MTP speculative
 * decode step (affine 4-bit expert GEMV, router, MoE combine, verify attention,
 * greedy and sampled acceptance).  It exists to check the HIP kernels; nothing
 * in the product library links, loads or calls it.  Only tests/, the
 * __graft_entry__.smoke() check and bench.py's cpu_baseline leg use it.
 *
 * Every function fixes one evaluation order (documented at the function) and
 * the HIP kernels reproduce that order, so GPU and oracle agree bit for bit.
 * The orders are pinned independently of the GPU by the tests in
 * tests/test_oracle_*.py (float64 brute force, closed forms, known answers).
 *
 * Parity unpinned: o_rope_table -- the fork's rotary table construction
 * (Qwen4ExpRotary.cosSin) is in an absent submodule; this table is the
 * standard rotate-half theta^(-2i/rot) one, which the tests pin only against
 * float64 RoPE of that same definition.
 *
 * Build: compile with -ffp-contract=off (no implicit FMA contraction).
 */
#ifndef MTPX_ORACLE_H
#define MTPX_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t o_bf16;

/* ---- scalar numerics ---------------------------------------------------- */
float o_bf2f(o_bf16 h);
o_bf16 o_f2bf(float f);              /* round to nearest even; NaN -> 0x7fc0 */
float o_round_bf(float f);           /* f32 -> bf16 -> f32 */
float o_expf(float x);               /* the build's own exp (see mtpx_oracle.c) */
float o_sigmoid_bf16(float x);       /* MLX Sigmoid functor in bf16 arithmetic */
float o_silu_bf16(float x);          /* x * sigmoid(x), bf16 arithmetic */
int o_lanes_for_blocks(int nblocks); /* lanes-per-row rule of the q4 GEMV */

/* ---- a1: MLX affine 4-bit quantization ---------------------------------- */
void o_affine_quantize(const o_bf16* w, int64_t rows, int K, int gs,
                       uint32_t* wq, o_bf16* scales, o_bf16* biases);

/* ---- a2-a4, a12: q4 GEMV  y[M,N] = x[M,K] . W[N,K]^T -------------------- */
void o_qmv(const uint32_t* wq, const o_bf16* scales, const o_bf16* biases,
           int64_t N, int K, int gs, const o_bf16* x, int M, o_bf16* y, float* yf);
/* the 32-element activation block transform the GEMV uses (exposed for tests) */
void o_xblock(const o_bf16* x32, int32_t* m_out, int32_t* E_out);

/* ---- a6/a9: bf16-weight router GEMV over f32 activations ---------------- */
void o_router_gemv(const o_bf16* W, int rows, int H, const float* x, int M, float* out);

/* ---- a8: top-k (value desc, index asc) + softmax over the selected ------ */
void o_topk_softmax(const float* logits, int M, int E, int K, int32_t* idx, float* w);

/* ---- a5, a10, a11: the MoE block ---------------------------------------- */
typedef struct {
  int H, E, K, F, gs;
  const o_bf16* router;       /* [E, H] bf16 */
  const o_bf16* shared_gate;  /* [H] bf16 (the shared-expert sigmoid gate row) */
  const uint32_t* gate_w; const o_bf16* gate_s; const o_bf16* gate_b; /* [E,F,H/8], [E,F,H/gs] */
  const uint32_t* up_w;   const o_bf16* up_s;   const o_bf16* up_b;
  const uint32_t* down_w; const o_bf16* down_s; const o_bf16* down_b; /* [E,H,F/8], [E,H,F/gs] */
  const uint32_t* sh_gate_w; const o_bf16* sh_gate_s; const o_bf16* sh_gate_b; /* [F,H/8] */
  const uint32_t* sh_up_w;   const o_bf16* sh_up_s;   const o_bf16* sh_up_b;
  const uint32_t* sh_down_w; const o_bf16* sh_down_s; const o_bf16* sh_down_b; /* [H,F/8] */
  /* the shared-expert gate as a q4 row [1, H] (NULL: the bf16 row shared_gate) */
  const uint32_t* sg_w; const o_bf16* sg_s; const o_bf16* sg_b;
} o_moe_weights;

void o_moe_block(const o_moe_weights* mw, const o_bf16* x, int M, o_bf16* y,
                 int32_t* idx, float* w, float* logits, o_bf16* gate,
                 o_bf16* act /* [M*(K+1), F] or NULL */);

/* ---- a13-a15: attention --------------------------------------------------- */
void o_rope_table(int positions, int rot, double theta, o_bf16* cos_t, o_bf16* sin_t);
void o_attn_prep(const o_bf16* qkv, int S, int QW, int HQ, int HK, int D, int ROT,
                 const o_bf16* qnorm, const o_bf16* knorm, float eps,
                 const o_bf16* cos_t, const o_bf16* sin_t, int pos0,
                 o_bf16* q, o_bf16* k, o_bf16* v);
void o_attn_verify(const o_bf16* q, int S, int HQ, int HK, int D,
                   const o_bf16* kc, const o_bf16* vc, int64_t tmax, int T,
                   float scale, int chunk, o_bf16* out);
void o_attn_gate(const o_bf16* att, const o_bf16* qkv, int S, int QW, int gate_off,
                 int width, o_bf16* out);
void o_rmsnorm(const o_bf16* x, int M, int H, const o_bf16* w, float eps, o_bf16* y);

/* ---- a17: MTP head pieces (embedding, hyper-connection mixer) ------------ */
void o_embed_rows(const uint32_t* wq, const o_bf16* scales, const o_bf16* biases, int H, int gs,
                  const int32_t* ids, int S, o_bf16* out);
void o_hc_norm(const o_bf16* residual, const o_bf16* out, const o_bf16* inject, int S, int hc,
               int H, int tile, const o_bf16* scale, float eps, o_bf16* stream, o_bf16* normed);
void o_silu_rows(const o_bf16* x, int64_t n, o_bf16* y);
void o_hc_mix(const o_bf16* w, const o_bf16* normed, const o_bf16* inj, int S, int hc, int H,
              o_bf16* input, o_bf16* inject_out);

/* ---- a20: the gated-deltanet sublayer (head dims 128) -------------------- */
typedef struct {
  int hk, hv, dk, dv, kc, conv_dim; /* key heads, value heads, 128, 128, conv taps, (2hk+hv)*128 */
  int proj_w, z_off, b_off, a_off;  /* projection row: qkv | z | b | a */
} o_gdn_geom;
float o_log1p_det(float y);        /* y in [0, 1] */
float o_logaddexp0_bf16(float x);  /* MLX logaddexp(x, 0) in bf16 arithmetic */
float o_sigmoid_f32(float x);      /* MLX Sigmoid in f32 */
void o_gdn_prep(const o_gdn_geom* g, const o_bf16* conv_state, const o_bf16* prow, const o_bf16* conv_w,
                const float* neg_exp_alog, const o_bf16* dt_bias, o_bf16* q, o_bf16* k, o_bf16* v,
                float* decay, float* beta);
void o_gdn_step(const o_gdn_geom* g, float* ssm, const o_bf16* q, const o_bf16* k, const o_bf16* v,
                const float* decay, const float* beta, o_bf16* y, float* delta_out);
void o_gdn_gated_rms(const o_gdn_geom* g, const o_bf16* y, const o_bf16* z, const o_bf16* w, float eps,
                     o_bf16* out);
void o_gdn_core(const o_gdn_geom* g, const o_bf16* proj, int S, o_bf16* conv_state, float* ssm,
                const o_bf16* conv_w, const float* neg_exp_alog, const o_bf16* dt_bias, const o_bf16* norm_w,
                float eps, o_bf16* gated, o_bf16* q_out, o_bf16* k_out, o_bf16* v_out, o_bf16* y_out,
                float* decay_out, float* beta_out, float* delta_out);

/* ---- a18, a21, a22: argmax and acceptance ------------------------------- */
void o_argmax_rows(const float* x, int rows, int64_t V, int32_t* out);
void o_top2_rows(const float* x, int rows, int64_t V, int32_t* ids, float* vals);
void o_accept_greedy(const float* logits, int k, int64_t V, const int32_t* drafts,
                     int32_t kv_offset, int32_t* out3);
void o_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float o_uniform(uint32_t r);
void o_accept_sample(const float* tlogits, const float* dlogits, int k, int64_t V,
                     const int32_t* drafts, float temperature, uint64_t seed,
                     uint64_t offset, int32_t kv_offset, int32_t* out3);
float o_softmax_row_sum(const float* e, int64_t V);

/* PLE n-gram block (layer index 1): row ids, gate, conv. */
void o_ngram_row_ids(const int32_t* history, int ctx_len, int S, int ngram_size, int heads_per_ngram,
                     const int64_t* mult, const int64_t* vocab, const int64_t* offs, int64_t rows, int32_t eos,
                     int32_t* out);
float o_ple_gate(const o_bf16* key, const o_bf16* stream, const o_bf16* value, const o_bf16* kscale,
                 const o_bf16* qscale, const o_bf16* cscale, int H, float eps, o_bf16* gated, o_bf16* normed);
void o_ple_conv(const o_bf16* full, const o_bf16* conv_w, const o_bf16* gated, int S, int64_t W, int kc, int dil,
                o_bf16* out);

/* Thread count of the row-parallel loops (results do not depend on it). */
void o_set_threads(int n);
int o_get_threads(void);
/* mlx_cpu mode: MLX's CPU _qmm_t with bf16 accumulation (timing baseline only). */
void o_qmm_t_bf16(const o_bf16* x, const uint32_t* wq, const o_bf16* scales, const o_bf16* biases,
                  int M, int64_t N, int K, int gs, o_bf16* y);

#ifdef __cplusplus
}
#endif
#endif
