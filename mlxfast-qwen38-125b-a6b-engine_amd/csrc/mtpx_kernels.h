// Kernel launchers shared by the C-ABI layer (host side) and the .hip files.
#pragma once
#include <stddef.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mtpx_device.h"

namespace mtpx {

constexpr int QMV_IT = 8;        // max blocks per lane: K <= 8 * 32 * lanes_for_blocks(K/32)
constexpr int MAX_TOKENS = 8;    // verify width ceiling (draft depth <= 7)
constexpr int HEAD_BATCH = 256;  // MTP head positions per call (the drafter's backlog flush)
constexpr int QMV_MAX_TOKENS = 4096;  // tokens per mtpx_qmv call
constexpr int MAX_TOPK = 16;
constexpr int ATTN_CHUNK = 32;   // keys per split-KV partial

// Raise a kernel's dynamic-LDS limit to `bytes` (only when above what it has;
// `cur` caches the value already set for that kernel).
template <typename Kern>
inline hipError_t ensure_lds(Kern* kernel, size_t bytes, size_t& cur) {
  if (bytes <= cur || bytes <= 64 * 1024) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) cur = bytes;
  return e;
}

// Compute units of the current device (cached per device).
inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) ? n : 256;
  }
  return cus[dev];
}

// Agent-coherent stores/loads of ticket-published data.
__device__ __forceinline__ void st_pub(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_pub(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Last-arriver ticket: every thread waits until its published stores are
// complete, the workgroup synchronises, one thread takes the ticket; the
// workgroup that draws `last` resets the counter and returns true.
__device__ __forceinline__ bool ticket_last(uint32_t* ctr, uint32_t last) {
  __shared__ int is_last;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t t = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (t == last);
    if (t == last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return is_last != 0;
}

// --- dense q4 GEMV and friends (qmv.hip)
hipError_t launch_xprep(const bf16* x, int M, int K, uint32_t* xp, hipStream_t st);
// sb: packed scale/bias rows (sb_row_len(K, gs) u32 per row) or null
// Two few-row matrices (N1, N2 rows; w2 may be null) over one batch of M > MAX_TOKENS prepared
// tokens, through xmb [M][K/32][XMB_DW] (workspace), where qmv_pair_ok holds (else launch_qmv per
// matrix).
constexpr int XMB_DW = 36;
bool qmv_pair_ok(const uint32_t* sb1, const uint32_t* w2, const uint32_t* sb2, int K, int M);
hipError_t launch_qmv_pair(const uint32_t* w1, const uint32_t* sb1, int N1, bf16* y1, const uint32_t* w2,
                           const uint32_t* sb2, int N2, bf16* y2, int K, int gs, const uint32_t* xp, uint32_t* xmb,
                           int M, hipStream_t st);
hipError_t launch_qmv(const uint32_t* wq, const bf16* s, const bf16* b, const uint32_t* sb, int N, int K, int gs,
                      const uint32_t* xp, int M, bf16* y, float* yf, hipStream_t st);
hipError_t launch_pack_sb(const bf16* s, const bf16* b, int64_t N, int K, int gs, uint32_t* out, hipStream_t st);
hipError_t launch_quantize(const bf16* w, int64_t rows, int K, int gs, uint32_t* wq, bf16* s, bf16* b,
                           hipStream_t st);
hipError_t launch_randn_bf16(bf16* out, int64_t n, uint64_t seed, uint32_t tensor, float sigma,
                             hipStream_t st);
hipError_t launch_fill_bf16(bf16* out, int64_t n, bf16 v, hipStream_t st);

// --- scratch of the allocation-free MoE entry point (noalloc.hip)
size_t moe_scratch_bytes();
hipError_t moe_scratch_address(int device, void** ptr);
bool moe_scratch_claim(int device, const void* owner);
void moe_scratch_release(int device, const void* owner);

// --- MoE (moe.hip)
// Expert-grouped dispatch of one MoE window, indexed by the expert kernels'
// grid row y: y = 0 the shared expert (expert -1, every token), y = 1..n_unique
// the routed experts selected by at least one token, expert -2 beyond.
struct MoeDispatch {
  int n_unique;  // routed experts selected by at least one token
  int pad[3];
  int expert[MAX_TOKENS * MAX_TOPK + 1];
  int count[MAX_TOKENS * MAX_TOPK + 1];
  int16_t slot[MAX_TOKENS * MAX_TOPK + 1][MAX_TOKENS];  // m*K + k (routed) or M*K + m (shared)
  // every slot once, in dispatch order: the M shared slots, then each selected expert's slots
  // (so the slots of one expert are adjacent); entry = slot | (expert + 1) << 16, expert -1
  // the shared one, so a workgroup finds its weight rows with one load
  int32_t order[MAX_TOKENS * (MAX_TOPK + 1)];
};
static_assert(offsetof(MoeDispatch, slot) % 8 == 0 && sizeof(MoeDispatch::slot[0]) == 16,
              "slot rows are read as two 8-byte words");

struct MoeArgs {
  int H, E, K, F, gs, M;
  const bf16* router;       // [E, H]
  const bf16* shared_gate;  // [H]
  const uint32_t *gate_w, *up_w, *down_w;
  const bf16 *gate_s, *gate_b, *up_s, *up_b, *down_s, *down_b;
  const uint32_t *sh_gate_w, *sh_up_w, *sh_down_w;
  const bf16 *sh_gate_s, *sh_gate_b, *sh_up_s, *sh_up_b, *sh_down_s, *sh_down_b;
  // packed scale/bias rows (all six or none)
  const uint32_t *gate_sb, *up_sb, *down_sb, *sh_gate_sb, *sh_up_sb, *sh_down_sb;
  // the shared-expert gate as a q4 row [1, H] (null: the bf16 row shared_gate)
  const uint32_t* sg_w = nullptr;
  const bf16 *sg_s = nullptr, *sg_b = nullptr;
  const uint32_t* sg_sb = nullptr;
  // activations and workspace
  const bf16* x;       // [M, H]
  bf16* y;             // [M, H]
  float* logits;       // [M, E]
  float* gate_logit;   // [M]
  int32_t* idx;        // [M, K]
  float* w;            // [M, K]
  MoeDispatch* disp;
  uint32_t* xp_x;      // [M, H/32, XP_DW]
  int xp_ready;        // xp_x already holds the prepared x (the router skips its preparation)
  bf16* act;           // [M*(K+1), F]
  bf16* r;             // [M*(K+1), H]
  const bf16* resid;   // [M, H] or null: y2 = bf16(resid + y)
  bf16* y2;            // [M, H] or null
  uint32_t* ticket;    // router+route ticket, zero at rest
  // one window: the router logits' publish buffer [MAX_TOKENS, MAX_EXPERTS], every word
  // ROUTE_SENTINEL at rest (the route puts it back), polled by the route; null: the ticket
  float* pub = nullptr;
  int32_t* nu_out;     // if set: the route also writes the distinct routed expert count here
  // windows of M tokens in one launch (a prefill batch): window w's tokens, slots, dispatch table,
  // ticket and count follow window w-1's, each window routed and computed as its own launch would
  int nwin = 1;
  // with nwin > 1: all windows' slots in one order grouped by expert (entry = global slot
  // w * M * (K + 1) + slot | (expert + 1) << 16), walked by the expert kernels in one 1-D grid, so
  // an expert's weight rows are fetched once for the whole batch; null: each window's own table
  int32_t* gorder = nullptr;
  // with gorder: the order cut into chunks of at most MQ_CHUNK slots of one expert (k_moe_sort):
  // chunks[c] = (gorder position, count | (expert + 1) << 16, 0 the shared expert), *chunk_n of
  // them, at most max_chunks; xp_act [slots][F/32][XP_DW]: the gate|up rows prepared for down
  int32_t* chunks = nullptr;
  int32_t* chunk_n = nullptr;
  int max_chunks = 0;
  uint32_t* xp_act = nullptr;
};
constexpr int MQ_CHUNK = 8;
inline int moe_max_chunks(int T, int E, int K) {
  return (T + MQ_CHUNK - 1) / MQ_CHUNK + E + (T * K + MQ_CHUNK - 1) / MQ_CHUNK;
}
bool moe_qmm_supported(const MoeArgs& a);
hipError_t launch_moe_qmm_down(const MoeArgs& a, hipStream_t st);

constexpr int MOE_TICKETS = 64;
constexpr int MAX_EXPERTS = 1024;
// A logit never has these bits: a NaN the GEMV makes carries the payload of a bf16 operand (low 16
// bits zero) or the default NaN's.
constexpr uint32_t ROUTE_SENTINEL = 0xffffffffu;
constexpr int ROUTE_SPIN = 1 << 20;  // polls of the publish buffer before the route goes on regardless
hipError_t launch_moe_router_route(const MoeArgs& a, hipStream_t st);
hipError_t launch_moe_gate_up(const MoeArgs& a, hipStream_t st);
hipError_t launch_moe_down(const MoeArgs& a, hipStream_t st);
// one workgroup per (slot, row block) in dispatch order (the slots of one expert side by side on
// one XCD, so its weight rows are fetched from HBM once and served to the others by that L2)
bool moe_dd_supported(int H, int F, int K);
hipError_t launch_moe_sort(const MoeArgs& a, hipStream_t st);  // a.gorder from the windows' routes
hipError_t launch_moe_gate_up_dd(const MoeArgs& a, hipStream_t st);
hipError_t launch_moe_down_dd(const MoeArgs& a, hipStream_t st);
hipError_t launch_moe_combine(const MoeArgs& a, hipStream_t st);

// --- attention (attn.hip)
hipError_t launch_attn_prep(const bf16* qkv, int S, int QW, int HQ, int HK, int D, int ROT,
                            const bf16* qnorm, const bf16* knorm, float eps, const bf16* cos_t,
                            const bf16* sin_t, int pos0, bf16* q, bf16* kcache, bf16* vcache,
                            int64_t tmax, hipStream_t st);
hipError_t launch_attn_verify(const bf16* q, int S, int HQ, int HK, int D, const bf16* kc,
                              const bf16* vc, int64_t tmax, int T, float scale, float* part,
                              const bf16* qkv, int QW, int gate_off, bf16* out, bf16* out_gated,
                              uint32_t* xp_gated, hipStream_t st);
size_t attn_partial_lds(int G, int D);
// The verify window's prep folded into the partial launch (q/k norms, rotation, the KV append), for
// S <= MAX_TOKENS and head dim 256.
bool attn_prep_fused_ok(int S, int HQ, int HK, int D, int QW);
hipError_t launch_attn_partial_prep(const bf16* qkv, int QW, int S, int HQ, int HK, int D, int ROT, const bf16* qnorm,
                                    const bf16* knorm, float eps, const bf16* cos_t, const bf16* sin_t, bf16* kcache,
                                    bf16* vcache, int64_t tmax, int T, float scale, float* part, hipStream_t st);
hipError_t launch_attn_partial(const bf16* q, int S, int HQ, int HK, int D, const bf16* kc, const bf16* vc,
                               int64_t tmax, int T, float scale, float* part, hipStream_t st);
hipError_t launch_attn_combine(int S, int HQ, int HK, int D, int T, const float* part, const bf16* qkv, int QW,
                               int gate_off, bf16* out, bf16* out_gated, uint32_t* xp_gated, hipStream_t st);
hipError_t launch_rmsnorm(const bf16* x, const bf16* resid, int M, int H, const bf16* w, float eps,
                          bf16* sum_out, bf16* y, uint32_t* xp, hipStream_t st);
hipError_t launch_add(const bf16* a, const bf16* b, int64_t n, bf16* out, hipStream_t st);
size_t attn_partial_floats(int S, int HQ, int D, int T);

// --- acceptance (accept.hip)
hipError_t launch_argmax_rows(const float* x, int rows, int64_t V, float* pval, int32_t* pidx,
                              int32_t* out, hipStream_t st);
hipError_t launch_accept_greedy(const float* logits, int k, int64_t V, const int32_t* drafts,
                                int32_t kv_offset, float* pval, int32_t* pidx, int32_t* out3,
                                hipStream_t st);
// bf16 logits (the verify's output); amax [k+1] and tokens [k+1] optional (see k_accept_greedy)
hipError_t launch_accept_greedy_bf16(const bf16* logits, int k, int64_t V, const int32_t* drafts, int32_t kv_offset,
                                     float* pval, int32_t* pidx, int32_t* out3, int32_t* amax, int32_t* tokens,
                                     hipStream_t st);
hipError_t launch_force_draft(int32_t* token, const int32_t* teacher, int64_t pos, float p, uint64_t seed,
                              hipStream_t st);
hipError_t launch_accept_sample(const float* tlogits, const float* dlogits, int k, int64_t V,
                                const int32_t* drafts, float temperature, uint64_t seed, uint64_t offset,
                                int32_t kv_offset, float* work, int32_t* out3, hipStream_t st);
// bf16 logits (the verify's output); dlogits null = one-hot draft rows at drafts (a greedy drafter);
// tokens [k+1] optional: the committed tokens (drafts[0..n-1], then the sampled token)
hipError_t launch_accept_sample_bf16(const bf16* tlogits, const bf16* dlogits, int k, int64_t V,
                                     const int32_t* drafts, float temperature, uint64_t seed, uint64_t offset,
                                     int32_t kv_offset, float* work, int32_t* out3, int32_t* tokens, hipStream_t st);
size_t accept_sample_work_floats(int k, int64_t V);
// top two of each row (x f32 or, when x is null, xb bf16): p2 = 4 * argmax_work_items(rows, V) floats
hipError_t launch_top2(const float* x, const bf16* xb, int rows, int64_t V, float* p2, int32_t* ids, float* vals,
                       hipStream_t st);
size_t argmax_work_items(int rows, int64_t V);
hipError_t launch_argmax_rows_bf16(const bf16* x, int rows, int64_t V, float* pval, int32_t* pidx,
                                   const int32_t* ids, int32_t* out, hipStream_t st);

// --- MTP head pieces (head.hip)
hipError_t launch_embed_rows(const uint32_t* wq, const bf16* s, const bf16* b, int H, int gs, int64_t V,
                             const int32_t* ids, int S, bf16* out, hipStream_t st);
hipError_t launch_hc_norm(const bf16* residual, const bf16* out, const bf16* inject, int S, int hc, int H,
                          int tile, const bf16* scale, float eps, bf16* stream, bf16* normed, uint32_t* xp,
                          hipStream_t st);
hipError_t launch_silu_xprep(const bf16* lo, int S, int LW, bf16* act, uint32_t* xp, hipStream_t st);
hipError_t launch_hc_mix(const bf16* w, const bf16* normed, const bf16* inj, int S, int hc, int H, bf16* input,
                         bf16* inject_out, uint32_t* xp, hipStream_t st);

// --- hyper-connection mixer in two launches (mixer.hip)
struct MixArgs {
  int H, hc, LW, gs, S;
  const uint32_t* dw; const bf16 *ds, *db; const uint32_t* dsb;  // down [LW, hc*H]
  const uint32_t* iw; const bf16 *is, *ib; const uint32_t* isb;  // inject [hc, hc*H] or iw == null
  const uint32_t* uw; const bf16 *us, *ub; const uint32_t* usb;  // up [hc*H, LW]
  const uint32_t* xpW;                                           // [S, hc*H/32] prepared normed streams
  const bf16* normed;                                            // [S, hc*H]
  float* part;                                                   // [Q, S, LW + hc] class partials
  bf16* x;                                                       // [S, H] block input
  bf16* j;                                                       // [S, hc] 2*sigmoid(inject) or null
  uint32_t* xpH;                                                 // [S, H/32] prepared x or null
};
int mix_classes(int W);
bool mix_supported(int H, int hc, int LW, int S);
hipError_t launch_mixer(const MixArgs& a, hipStream_t st);

// --- gated-deltanet sublayer core (gdn.hip); head dims 128
struct GdnArgs {
  int hk, hv, kc, cd, pw, z_off, b_off, a_off;  // key/value heads, conv taps, conv channels, projection row layout
  int S, P;                                     // window positions; committed steps of the previous window
  float eps;                                    // gated RMS epsilon
  const bf16* proj;                             // [S, pw]: qkv | z | b | a
  const bf16* conv_w;                           // [cd, kc]
  const float* neg_exp_alog;                    // [hv]: -exp(A_log)
  const bf16* dt_bias;                          // [hv]
  const bf16* norm_w;                           // [128]
  const bf16* conv_cur;                         // [kc-1, cd] conv base of the previous window
  const bf16* win_cur;                          // [*, cd]  previous window's conv input rows
  const bf16* key_cur;                          // [*, hk, 128]
  const float* delta_cur;                       // [*, hv, 128]
  const float* decay_cur;                       // [*, hv]
  bf16 *conv_nxt, *win_nxt, *key_nxt;           // this window's journal (same shapes)
  float *delta_nxt, *decay_nxt;
  float* ssm;                                   // [hv, 128, 128] committed recurrent state (in place)
  bf16* gated;                                  // [S, hv*128] or null
  uint32_t* xp;                                 // [S, hv*4, XP_DW] prepared gated rows or null
  uint32_t* tickets;                            // [hv] per-head last-arriver counters, zero at rest
  float* ypub;                                  // [S, hv, 128] recurrence outputs published for the gated norm
};
hipError_t launch_gdn_step(const GdnArgs& a, hipStream_t st);
// a prefill batch of a.S positions (any count), every one committed; a.ypub holds a.S positions
struct GdnBatch {
  float* vecs;   // [S, 2*hk + hv, 128] the positions' q (per key head), k (per key head), v (per value head)
  float* gates;  // [S, hv, 2] decay, beta
};
hipError_t launch_gdn_batch(const GdnArgs& a, const GdnBatch& b, hipStream_t st);
hipError_t launch_gdn_replay(const GdnArgs& a, float* ssm_dst, bf16* conv_dst, hipStream_t st);

// --- PLE n-gram block (ple.hip)
constexpr int PLE_MAX_NGRAM = 8;
constexpr int PLE_MAX_HEADS = 32;  // (ngram - 1) * heads_per_ngram
constexpr int PLE_MAX_CTX = 8;     // carried context tokens

struct PleRowArgs {
  int S, ctx_len, ngram, hpn, row_dim, rgs, P;  // window, context, hash geometry, row width and groups, committed
  int32_t eos;
  int64_t rows;                  // table rows
  const int64_t* hash;           // device [ngram + 2*heads]: multipliers | head vocab sizes | head offsets
  const int32_t* ctx_cur;        // [ctx_len] base context of the previous window
  const int32_t* ids_prev;       // [*] previous window's tokens
  const int32_t* ids;            // [S] this window's tokens
  int32_t *ctx_nxt, *ids_nxt;    // this window's base context and tokens (or null)
  int32_t* row_ids;              // [S, heads] or null
  const uint32_t* tw;            // table [rows, row_dim/8]
  const bf16 *ts, *tb;           // [rows, row_dim/rgs]
  bf16* emb;                     // [S, heads*row_dim] or null
  uint32_t* xp;                  // prepared blocks of emb or null
};
hipError_t launch_ple_rows(const PleRowArgs& a, hipStream_t st);
hipError_t launch_ple_gate(const bf16* key, const bf16* stream, const bf16* value, const bf16* kscale,
                           const bf16* qscale, const bf16* cscale, int S, int hc, int H, float eps, bf16* gated,
                           bf16* normed, hipStream_t st);
struct PleConvArgs {
  int S, kc, dil, P;
  int64_t W;
  const bf16* conv_cur;  // [nb, W] base rows of the previous window
  const bf16* win_cur;   // [*, W] previous window's normed rows
  const bf16* win_nxt;   // [S, W] this window's normed rows
  const bf16* conv_w;    // [W, kc]
  const bf16* gated;     // [S, W]
  const bf16* stream;    // [S, W] (for sum)
  bf16* out;             // [S, W] gated + silu(conv) or null
  bf16* sum;             // [S, W] stream + out or null
  bf16* conv_nxt;        // [nb, W] this window's base rows or null
};
hipError_t launch_ple_conv(const PleConvArgs& a, hipStream_t st);

}  // namespace mtpx
