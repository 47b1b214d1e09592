// C-ABI layer of libmtpx: argument checks, contexts, workspace, handles.
// No torch types, no host fallbacks: every compute entry point enqueues HIP
// kernels and fails with an error code when it cannot.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/mtpx.h"
#include "abi_internal.h"
#include "drafter.h"
#include "mtpx_kernels.h"

using namespace mtpx;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_OK(expr)                                                                              \
  do {                                                                                            \
    hipError_t e_ = (expr);                                                                       \
    if (e_ != hipSuccess) return fail(MTPX_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));      \
  } while (0)

#define ARG(cond, ...)                                 \
  do {                                                 \
    if (!(cond)) return fail(MTPX_ERR_ARG, __VA_ARGS__); \
  } while (0)

struct Ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  void* ws = nullptr;
  size_t ws_size = 0;
  size_t ws_used = 0;
  bool ws_over = false;              // a take ran past the reservation (see ws_take)
  MoeDispatch* last_disp = nullptr;  // inside the workspace of the last MoE call
  uint32_t* tickets = nullptr;       // MOE_TICKETS counters, zero at rest
  float* route_pub = nullptr;        // [MAX_TOKENS, MAX_EXPERTS] router logits publish buffer, ROUTE_SENTINEL at rest
  void* scratch = nullptr;           // this device's MoE scratch array (noalloc.hip), looked up at set-up
  int last_H = 0, last_E = 0, last_F = 0, last_gs = 0;
  // per-kernel timing with events on the launch stream (off by default)
  bool prof = false;
  struct Rec {
    const char* name;
    hipEvent_t a, b;
  };
  std::vector<hipEvent_t> ev_free;
  std::vector<Rec> pending;
  std::map<std::string, std::pair<int64_t, double>> stats;  // launches, total ms
};

hipEvent_t ev_get(Ctx* c) {
  if (!c->ev_free.empty()) {
    hipEvent_t e = c->ev_free.back();
    c->ev_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Launch `expr`; with profiling on, bracket it with events on the context stream.
#define LAUNCH(c, name, expr)                                        \
  do {                                                               \
    if ((c)->ws_over)                                                \
      return fail(MTPX_ERR_STATE, "internal workspace accounting error before %s", name); \
    (void)hipGetLastError(); /* an earlier call's error (already returned to its caller) is not this launch's */ \
    hipEvent_t a_ = nullptr;                                         \
    if ((c)->prof && (a_ = ev_get(c))) hipEventRecord(a_, (c)->stream); \
    HIP_OK(expr);                                                    \
    if (a_) {                                                        \
      hipEvent_t b_ = ev_get(c);                                     \
      if (b_) {                                                      \
        hipEventRecord(b_, (c)->stream);                             \
        (c)->pending.push_back({name, a_, b_});                      \
      } else {                                                       \
        (c)->ev_free.push_back(a_);                                  \
      }                                                              \
    }                                                                \
  } while (0)

int prof_fold(Ctx* c) {
  if (c->pending.empty()) return MTPX_OK;
  HIP_OK(hipStreamSynchronize(c->stream));
  for (auto& r : c->pending) {
    float ms = 0.0f;
    HIP_OK(hipEventElapsedTime(&ms, r.a, r.b));
    auto& st = c->stats[r.name];
    st.first += 1;
    st.second += ms;
    c->ev_free.push_back(r.a);
    c->ev_free.push_back(r.b);
  }
  c->pending.clear();
  return MTPX_OK;
}

// Workspace bump allocation.  Calls on one context are serialised on its
// stream, so every call may reuse the whole workspace from offset 0.
int ws_reserve(Ctx* c, size_t bytes) {
  if (bytes <= c->ws_size) return MTPX_OK;
  if (c->ws) {
    HIP_OK(hipStreamSynchronize(c->stream));
    HIP_OK(hipFree(c->ws));
    c->ws = nullptr;
    c->last_disp = nullptr;
  }
  size_t sz = bytes < ((size_t)64 << 20) ? ((size_t)64 << 20) : bytes + (bytes >> 2);
  if (hipMalloc(&c->ws, sz) != hipSuccess) {
    c->ws = nullptr;
    c->ws_size = 0;
    return fail(MTPX_ERR_OOM, "workspace allocation of %zu bytes failed", sz);
  }
  c->ws_size = sz;
  return MTPX_OK;
}

// Every entry point reserves its whole need before the first take; running
// past the reservation is an internal accounting error.  The take then marks
// the context (ws_over) and returns the workspace base; LAUNCH refuses every
// launch while the mark is set, so no kernel sees memory outside the
// allocation and the entry point returns MTPX_ERR_STATE.
template <typename T>
T* ws_take(Ctx* c, size_t count) {
  const size_t off = (c->ws_used + 255) & ~(size_t)255;
  c->ws_used = off + count * sizeof(T);
  if (c->ws_used > c->ws_size) {
    c->ws_over = true;
    return reinterpret_cast<T*>(c->ws);
  }
  return reinterpret_cast<T*>(static_cast<char*>(c->ws) + off);
}

// Start of an entry point's workspace use.
void ws_begin(Ctx* c) {
  c->ws_used = 0;
  c->ws_over = false;
}

size_t al(size_t b) { return (b + 255) & ~(size_t)255; }

Ctx* C(mtpx_ctx h) { return static_cast<Ctx*>(h.ctx); }

int set_device(Ctx* c) {
  HIP_OK(hipSetDevice(c->device));
  return MTPX_OK;
}

bool gs_ok(int gs) { return gs == 32 || gs == 64; }

// K limits of the GEMV: multiple of 32 and of gs, at most QMV_IT blocks per lane.
bool k_ok(int K, int gs) {
  if (K <= 0 || K % 32 || K % gs) return false;
  const int nb = K / 32;
  return nb <= QMV_IT * lanes_for_blocks(nb);
}

struct Kv {
  Ctx* ctx;
  int heads, dim;
  int64_t tmax, offset = 0;
  uint16_t *k = nullptr, *v = nullptr;
};

struct Layer {
  mtpx_layer_config cfg;
  mtpx_layer_weights w;
  std::vector<void*> allocs;
  int QW;
};

int moe_check(const mtpx_moe_weights* w, int M) {
  ARG(w, "moe weights is NULL");
  ARG(M >= 1 && M <= MAX_TOKENS, "M=%d outside 1..%d", M, MAX_TOKENS);
  ARG(gs_ok(w->group_size), "group size %d not in {32, 64}", w->group_size);
  ARG(w->top_k >= 1 && w->top_k <= MAX_TOPK && w->top_k <= w->experts, "top_k=%d", w->top_k);
  ARG(w->experts >= 1 && w->experts <= 1024, "experts=%d outside 1..1024", w->experts);
  ARG(w->hidden % 8 == 0 && w->hidden <= 4096, "hidden=%d", w->hidden);
  ARG(k_ok(w->hidden, w->group_size), "hidden=%d not a supported GEMV depth", w->hidden);
  ARG(k_ok(w->expert_width, w->group_size), "expert_width=%d not a supported GEMV depth", w->expert_width);
  ARG(w->router && (w->shared_gate || w->shared_gate_w) && w->gate_w && w->up_w && w->down_w && w->sh_gate_w &&
          w->sh_up_w && w->sh_down_w,
      "missing MoE weight pointer");
  ARG(!w->shared_gate_w || w->shared_gate_sb || (w->shared_gate_s && w->shared_gate_b),
      "the q4 shared-expert gate needs its scales and biases (or packed row)");
  const int nsb = !!w->gate_sb + !!w->up_sb + !!w->down_sb + !!w->sh_gate_sb + !!w->sh_up_sb + !!w->sh_down_sb;
  ARG(nsb == 0 || nsb == 6, "packed scale/bias rows: give all six matrices or none");
  return MTPX_OK;
}

size_t moe_ws_bytes(const mtpx_moe_weights* w, int M, int nwin = 1) {
  const int H = w->hidden, E = w->experts, K = w->top_k, F = w->expert_width;
  const size_t T = (size_t)M * nwin, slots = T * (K + 1);
  return al(4 * T * E) + al(4 * T) + al(4 * T * K) * 2 + al(sizeof(MoeDispatch) * (size_t)nwin) +
         al(4 * T * (H / 32) * XP_DW) + al(2 * slots * F) + al(2 * slots * H) +
         (nwin > 1 ? al(4 * slots) + al(8 * (size_t)moe_max_chunks((int)T, E, K)) + al(4) +
                         al(4 * slots * (F / 32) * XP_DW)
                   : 0) +
         4096;
}

// Workspace of S tokens through moe_enqueue_windows (its launches reuse one region in turn).
size_t moe_windows_ws_bytes(const mtpx_moe_weights* w, int S) {
  const int full = S / MAX_TOKENS < MOE_TICKETS ? S / MAX_TOKENS : MOE_TICKETS, tail = S % MAX_TOKENS;
  return std::max(full ? moe_ws_bytes(w, MAX_TOKENS, full) : (size_t)0, tail ? moe_ws_bytes(w, tail) : (size_t)0);
}


// Enqueue the MoE block; workspace already reserved.
int moe_enqueue(Ctx* c, const mtpx_moe_weights* w, const uint16_t* x, int M, uint16_t* y, int32_t* idx,
                float* wts, float* logits, const uint16_t* resid = nullptr, uint16_t* y2 = nullptr,
                uint32_t* xp_ready = nullptr, int32_t* nu_out = nullptr, int nwin = 1) {
  MoeArgs a;
  a.H = w->hidden;
  a.E = w->experts;
  a.K = w->top_k;
  a.F = w->expert_width;
  a.gs = w->group_size;
  a.M = M;
  a.router = w->router;
  a.shared_gate = w->shared_gate;
  a.sg_w = w->shared_gate_w;
  a.sg_s = reinterpret_cast<const bf16*>(w->shared_gate_s);
  a.sg_b = reinterpret_cast<const bf16*>(w->shared_gate_b);
  a.sg_sb = w->shared_gate_sb;
  a.gate_w = w->gate_w; a.gate_s = w->gate_s; a.gate_b = w->gate_b;
  a.up_w = w->up_w; a.up_s = w->up_s; a.up_b = w->up_b;
  a.down_w = w->down_w; a.down_s = w->down_s; a.down_b = w->down_b;
  a.sh_gate_w = w->sh_gate_w; a.sh_gate_s = w->sh_gate_s; a.sh_gate_b = w->sh_gate_b;
  a.sh_up_w = w->sh_up_w; a.sh_up_s = w->sh_up_s; a.sh_up_b = w->sh_up_b;
  a.sh_down_w = w->sh_down_w; a.sh_down_s = w->sh_down_s; a.sh_down_b = w->sh_down_b;
  a.gate_sb = w->gate_sb; a.up_sb = w->up_sb; a.down_sb = w->down_sb;
  a.sh_gate_sb = w->sh_gate_sb; a.sh_up_sb = w->sh_up_sb; a.sh_down_sb = w->sh_down_sb;
  a.x = x;
  a.y = y;
  a.nwin = nwin;
  const size_t T = (size_t)M * nwin, slots = T * (a.K + 1);
  a.logits = logits ? logits : ws_take<float>(c, T * a.E);
  a.gate_logit = ws_take<float>(c, T);
  a.idx = idx ? idx : ws_take<int32_t>(c, T * a.K);
  a.w = wts ? wts : ws_take<float>(c, T * a.K);
  a.disp = ws_take<MoeDispatch>(c, nwin);
  a.xp_x = xp_ready ? xp_ready : ws_take<uint32_t>(c, T * (a.H / 32) * XP_DW);
  a.xp_ready = xp_ready != nullptr;
  a.act = ws_take<uint16_t>(c, slots * a.F);
  a.r = ws_take<uint16_t>(c, slots * a.H);
  a.resid = resid;
  a.y2 = y2;
  a.ticket = c->tickets;
  a.pub = nwin == 1 ? c->route_pub : nullptr;
  a.nu_out = nu_out;
  c->last_disp = a.disp;
  c->last_H = a.H;
  c->last_E = a.E;
  c->last_F = a.F;
  c->last_gs = a.gs;
  LAUNCH(c, "moe_router_route", launch_moe_router_route(a, c->stream));
  if (moe_dd_supported(a.H, a.F, a.K)) {  // one workgroup per (slot, row block), slots in dispatch order
    if (nwin > 1) {  // a batch of windows: one order of all their slots, grouped by expert
      a.gorder = ws_take<int32_t>(c, slots);
      a.chunks = ws_take<int32_t>(c, 2 * (size_t)moe_max_chunks((int)T, a.E, a.K));
      a.chunk_n = ws_take<int32_t>(c, 1);
      a.max_chunks = moe_max_chunks((int)T, a.E, a.K);
      a.xp_act = ws_take<uint32_t>(c, slots * (a.F / 32) * XP_DW);
      LAUNCH(c, "moe_sort", launch_moe_sort(a, c->stream));
      if (moe_qmm_supported(a)) {  // down over the experts' chunks on the matrix cores
        LAUNCH(c, "moe_gate_up", launch_moe_gate_up_dd(a, c->stream));
        LAUNCH(c, "moe_act_prep", launch_xprep(reinterpret_cast<const bf16*>(a.act), (int)slots, a.F, a.xp_act, c->stream));
        LAUNCH(c, "moe_down", launch_moe_qmm_down(a, c->stream));
        LAUNCH(c, "moe_combine", launch_moe_combine(a, c->stream));
        return MTPX_OK;
      }
    }
    LAUNCH(c, "moe_gate_up", launch_moe_gate_up_dd(a, c->stream));
    LAUNCH(c, "moe_down", launch_moe_down_dd(a, c->stream));
    LAUNCH(c, "moe_combine", launch_moe_combine(a, c->stream));
    return MTPX_OK;
  }
  LAUNCH(c, "moe_gate_up", launch_moe_gate_up(a, c->stream));
  LAUNCH(c, "moe_down", launch_moe_down(a, c->stream));
  LAUNCH(c, "moe_combine", launch_moe_combine(a, c->stream));
  return MTPX_OK;
}

// S tokens of a prefill batch through the MoE block as windows of MAX_TOKENS tokens, routed and
// computed as separate windows would be (each token's output is the window's): the full windows
// in one batched launch per kernel, the remaining tokens as one more window.
int moe_enqueue_windows(Ctx* c, const mtpx_moe_weights* w, const uint16_t* x, int S, uint16_t* y,
                        uint32_t* xp_ready) {
  const int full = S / MAX_TOKENS, tail = S % MAX_TOKENS, H = w->hidden;
  const size_t mark = c->ws_used;
  int rc;
  for (int w0 = 0; w0 < full; w0 += MOE_TICKETS) {  // a ticket per window of a launch
    const int nw = full - w0 < MOE_TICKETS ? full - w0 : MOE_TICKETS;
    const size_t t0 = (size_t)w0 * MAX_TOKENS;
    c->ws_used = mark;  // the previous launches' workspace is free again in stream order
    if ((rc = moe_enqueue(c, w, x + t0 * H, MAX_TOKENS, y + t0 * H, nullptr, nullptr, nullptr, nullptr, nullptr,
                          xp_ready ? xp_ready + t0 * (H / 32) * XP_DW : nullptr, nullptr, nw)))
      return rc;
  }
  if (tail) {
    const size_t t0 = (size_t)full * MAX_TOKENS;
    c->ws_used = mark;
    if ((rc = moe_enqueue(c, w, x + t0 * H, tail, y + t0 * H, nullptr, nullptr, nullptr, nullptr, nullptr,
                          xp_ready ? xp_ready + t0 * (H / 32) * XP_DW : nullptr)))
      return rc;
  }
  return MTPX_OK;
}

// Random-init weights on the device: N(0, sigma) bf16 from the counter-based
// generator (stream = seed, tensor id), q4 matrices quantised with MLX's
// affine_quantize, through one bf16 staging buffer.
struct RandInit {
  Ctx* c;
  uint64_t seed;
  int gs;
  std::vector<void*>* allocs;
  uint32_t tensor = 1;
  bool ok = true;
  uint16_t* tmp = nullptr;

  void* alloc(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
      ok = false;
      return nullptr;
    }
    allocs->push_back(p);
    return p;
  }
  void qmat(int64_t rows, int K, const uint32_t** w, const uint16_t** s, const uint16_t** b) {
    uint32_t* pw = (uint32_t*)alloc((size_t)rows * K / 2);
    uint16_t* ps = (uint16_t*)alloc((size_t)rows * (K / gs) * 2);
    uint16_t* pb = (uint16_t*)alloc((size_t)rows * (K / gs) * 2);
    *w = pw;
    *s = ps;
    *b = pb;
    if (!pw || !ps || !pb) return;
    const int64_t slice = (int64_t)1 << 24;  // staging elements
    const int64_t rows_per = slice / K > 0 ? slice / K : 1;
    if (!tmp && hipMalloc(&tmp, (size_t)(rows_per * K > slice ? rows_per * K : slice) * 2) != hipSuccess) {
      tmp = nullptr;
      ok = false;
      return;
    }
    for (int64_t r0 = 0; r0 < rows && ok; r0 += rows_per) {
      const int64_t nr = rows - r0 < rows_per ? rows - r0 : rows_per;
      if (launch_randn_bf16(tmp, nr * K, seed, tensor * 65536u + (uint32_t)(r0 / rows_per), 0.02f, c->stream) ||
          launch_quantize(tmp, nr, K, gs, pw + r0 * (K / 8), ps + r0 * (K / gs), pb + r0 * (K / gs), c->stream))
        ok = false;
    }
    ++tensor;
  }
  // the same, plus the packed scale/bias rows
  void qmat(int64_t rows, int K, const uint32_t** w, const uint16_t** s, const uint16_t** b, const uint32_t** sb) {
    qmat(rows, K, w, s, b);
    uint32_t* p = (uint32_t*)alloc((size_t)rows * sb_row_len(K, gs) * 4);
    *sb = p;
    if (p && *s && *b && launch_pack_sb(*s, *b, rows, K, gs, p, c->stream)) ok = false;
  }
  void qmat(int64_t rows, int K, mtpx_q4* q) { qmat(rows, K, &q->w, &q->s, &q->b, &q->sb); }
  // sigma > 0: N(0, sigma); sigma == 0: filled with the bf16 pattern `ones`
  const uint16_t* dense(int64_t n, float sigma, uint16_t ones = 0x3f80) {
    uint16_t* p = (uint16_t*)alloc((size_t)n * 2);
    if (!p) return nullptr;
    if (sigma > 0.0f) {
      if (launch_randn_bf16(p, n, seed, tensor * 65536u, sigma, c->stream)) ok = false;
    } else if (launch_fill_bf16(p, n, ones, c->stream)) {
      ok = false;
    }
    ++tensor;
    return p;
  }
  // synchronise, release the staging buffer; MTPX_OK or an error (allocations stay listed)
  int finish(const char* what) {
    const hipError_t se = hipStreamSynchronize(c->stream);
    if (tmp) hipFree(tmp);
    tmp = nullptr;
    if (!ok || se != hipSuccess) return fail(ok ? MTPX_ERR_HIP : MTPX_ERR_OOM, "%s initialisation failed", what);
    return MTPX_OK;
  }
};

uint16_t bf16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

int layer_check(const mtpx_layer_config* cfg) {
  const int H = cfg->hidden, F = cfg->expert_width, gs = cfg->group_size;
  const int HQ = cfg->heads, HK = cfg->kv_heads, D = cfg->head_dim;
  ARG(gs_ok(gs) && k_ok(H, gs) && k_ok(F, gs) && k_ok(HQ * D, gs), "unsupported GEMV depths");
  ARG(HK >= 1 && HQ % HK == 0 && HQ / HK <= 32 && D <= 256 && cfg->rot_dims <= D && cfg->max_positions >= 1 &&
          cfg->max_positions <= 65536,
      "attention dims (max_positions <= 65536)");
  return MTPX_OK;
}

// MoE weights of one layer (random init): bf16 router and shared gate row, q4 experts.
void moe_random(RandInit& ri, const mtpx_layer_config* cfg, mtpx_moe_weights* mw) {
  const int H = cfg->hidden, E = cfg->experts, F = cfg->expert_width;
  mtpx_moe_weights& m = *mw;
  m.hidden = H;
  m.experts = E;
  m.top_k = cfg->top_k;
  m.expert_width = F;
  m.group_size = cfg->group_size;
  m.router = ri.dense((int64_t)E * H, 0.02f);
  m.shared_gate = ri.dense(H, 0.02f);
  ri.qmat((int64_t)E * F, H, &m.gate_w, &m.gate_s, &m.gate_b, &m.gate_sb);
  ri.qmat((int64_t)E * F, H, &m.up_w, &m.up_s, &m.up_b, &m.up_sb);
  ri.qmat((int64_t)E * H, F, &m.down_w, &m.down_s, &m.down_b, &m.down_sb);
  ri.qmat(F, H, &m.sh_gate_w, &m.sh_gate_s, &m.sh_gate_b, &m.sh_gate_sb);
  ri.qmat(F, H, &m.sh_up_w, &m.sh_up_s, &m.sh_up_b, &m.sh_up_sb);
  ri.qmat(H, F, &m.sh_down_w, &m.sh_down_s, &m.sh_down_b, &m.sh_down_sb);
}

// Rotate-half RoPE tables [max_positions, rot] (bf16): entry d uses theta^(-2*(d mod rot/2)/rot);
// angles and cos/sin in double.  Synchronises (the host vectors go out of scope).
bool rope_tables(Ctx* c, const mtpx_layer_config* cfg, std::vector<void*>* allocs, const uint16_t** cos_out,
                 const uint16_t** sin_out) {
  const int rot = cfg->rot_dims;
  std::vector<uint16_t> ct((size_t)cfg->max_positions * rot), st((size_t)cfg->max_positions * rot);
  for (int64_t p = 0; p < cfg->max_positions; ++p)
    for (int d = 0; d < rot; ++d) {
      const int i = d % (rot / 2);
      const double inv = std::pow((double)cfg->rope_theta, -2.0 * (double)i / (double)rot);
      const double a = (double)p * inv;
      ct[(size_t)p * rot + d] = bf16_bits((float)std::cos(a));
      st[(size_t)p * rot + d] = bf16_bits((float)std::sin(a));
    }
  void *dc = nullptr, *ds = nullptr;
  if (hipMalloc(&dc, ct.size() * 2) != hipSuccess) return false;
  allocs->push_back(dc);
  if (hipMalloc(&ds, st.size() * 2) != hipSuccess) return false;
  allocs->push_back(ds);
  if (hipMemcpyAsync(dc, ct.data(), ct.size() * 2, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
      hipMemcpyAsync(ds, st.data(), st.size() * 2, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return false;
  *cos_out = static_cast<const uint16_t*>(dc);
  *sin_out = static_cast<const uint16_t*>(ds);
  return true;
}

// Attention + MoE weights of one decoder layer (random init), RoPE tables from the host.
int layer_create(Ctx* c, const mtpx_layer_config* cfg, uint64_t seed, Layer** out) {
  int rc = layer_check(cfg);
  if (rc) return rc;
  const int H = cfg->hidden, E = cfg->experts, F = cfg->expert_width, gs = cfg->group_size;
  const int HQ = cfg->heads, HK = cfg->kv_heads, D = cfg->head_dim;
  Layer* L = new Layer();
  L->cfg = *cfg;
  memset(&L->w, 0, sizeof(L->w));
  const int QW = 2 * HQ * D + 2 * HK * D + cfg->index_dim;
  L->QW = QW;
  L->w.qkv_rows = QW;
  RandInit ri{c, seed, gs, &L->allocs};
  L->w.attn_norm = ri.dense(H, 0.0f);
  L->w.post_norm = ri.dense(H, 0.0f);
  L->w.q_norm = ri.dense(D, 0.0f);
  L->w.k_norm = ri.dense(D, 0.0f);
  ri.qmat(QW, H, &L->w.qkv_w, &L->w.qkv_s, &L->w.qkv_b, &L->w.qkv_sb);
  ri.qmat(H, HQ * D, &L->w.o_w, &L->w.o_s, &L->w.o_b, &L->w.o_sb);
  moe_random(ri, cfg, &L->w.moe);
  if (!rope_tables(c, cfg, &L->allocs, &L->w.rope_cos, &L->w.rope_sin)) ri.ok = false;
  if ((rc = ri.finish("layer"))) {
    for (void* p : L->allocs) hipFree(p);
    delete L;
    return rc;
  }
  *out = L;
  return MTPX_OK;
}

// Attention sublayer for M tokens whose prepared input blocks are in xp:
// qkv GEMV, q/k norm + RoPE + KV append, verify attention with the output gate,
// o_proj GEMV -> o [M, H].  xp is reused for the gated attention output, so it
// holds max(H, HQ*D)/32 blocks per token.  Workspace already reserved.
int attn_enqueue(Ctx* c, const Layer* L, Kv* kv, uint32_t* xp, int M, uint16_t* o) {
  const mtpx_layer_config& g = L->cfg;
  const int H = g.hidden, HQ = g.heads, HK = g.kv_heads, D = g.head_dim, QW = L->QW, gs = g.group_size;
  const int T = (int)(kv->offset + M);
  uint16_t* qkv = ws_take<uint16_t>(c, (size_t)M * QW);
  uint16_t* q = ws_take<uint16_t>(c, (size_t)M * HQ * D);
  uint16_t* att = ws_take<uint16_t>(c, (size_t)M * HQ * D);
  float* part = ws_take<float>(c, attn_partial_floats(M, HQ, D, T));
  hipStream_t st = c->stream;
  LAUNCH(c, "qmv_qkv", launch_qmv(L->w.qkv_w, L->w.qkv_s, L->w.qkv_b, L->w.qkv_sb, QW, H, gs, xp, M, qkv, nullptr, st));
  if (attn_prep_fused_ok(M, HQ, HK, D, QW)) {  // a verify window: the prep inside the partial launch
    LAUNCH(c, "attn_partial", launch_attn_partial_prep(qkv, QW, M, HQ, HK, D, g.rot_dims, L->w.q_norm, L->w.k_norm,
                                                       g.eps, L->w.rope_cos, L->w.rope_sin, kv->k, kv->v, kv->tmax, T,
                                                       1.0f / std::sqrt((float)D), part, st));
  } else {
    LAUNCH(c, "attn_prep", launch_attn_prep(qkv, M, QW, HQ, HK, D, g.rot_dims, L->w.q_norm, L->w.k_norm, g.eps,
                                            L->w.rope_cos, L->w.rope_sin, (int)kv->offset, q, kv->k, kv->v,
                                            kv->tmax, st));
    LAUNCH(c, "attn_partial", launch_attn_partial(q, M, HQ, HK, D, kv->k, kv->v, kv->tmax, T,
                                                  1.0f / std::sqrt((float)D), part, st));
  }
  LAUNCH(c, "attn_combine", launch_attn_combine(M, HQ, HK, D, T, part, qkv, QW, HQ * D, nullptr, att, xp, st));
  LAUNCH(c, "qmv_o", launch_qmv(L->w.o_w, L->w.o_s, L->w.o_b, L->w.o_sb, H, HQ * D, gs, xp, M, o, nullptr, st));
  return MTPX_OK;
}

size_t attn_ws_bytes(const Layer* L, int M, int T) {
  const mtpx_layer_config& g = L->cfg;
  const int HQ = g.heads, D = g.head_dim;
  return al(2 * (size_t)M * L->QW) + al(2 * (size_t)M * HQ * D) * 2 + al(4 * attn_partial_floats(M, HQ, D, T));
}

// ---------------------------------------------------------------------------
// MTP head
struct Head {
  mtpx_head_config cfg;
  Layer* layer = nullptr;
  mtpx_head_weights w;
  std::vector<void*> allocs;
};

int head_check(const mtpx_head_config* cfg) {
  int rc = layer_check(&cfg->layer);
  if (rc) return rc;
  const int H = cfg->layer.hidden, gs = cfg->layer.group_size;
  ARG(cfg->hc >= 1 && cfg->hc <= 8 && cfg->lowrank >= 32 && cfg->lowrank % 32 == 0, "hc=%d lowrank=%d", cfg->hc,
      cfg->lowrank);
  ARG(k_ok(cfg->hc * H, gs) && k_ok(cfg->lowrank, gs), "unsupported mixer GEMV depths");
  ARG(cfg->hc * H <= 256 * 48, "hc*hidden=%d above 12288", cfg->hc * H);
  ARG(cfg->vocab >= 1 && cfg->vocab < ((int64_t)1 << 31) && cfg->shortlist_low >= 0, "vocab=%lld",
      (long long)cfg->vocab);
  return MTPX_OK;
}

// The drafter's shortlist (Runner/Qwen4ExpMTPDrafter.swift:91-108): ids 0..low-1
// with low padded so the count is a multiple of 8, then special_from..vocab-1.
std::vector<int32_t> shortlist_ids(const mtpx_head_config* cfg) {
  const int64_t n = cfg->vocab;
  const int64_t sf = cfg->shortlist_special_from;
  const int64_t specials = (sf > cfg->shortlist_low && sf < n) ? n - sf : 0;
  int64_t low = cfg->shortlist_low < n ? cfg->shortlist_low : n;
  low += (8 - (low + specials) % 8) % 8;
  std::vector<int32_t> ids;
  for (int64_t i = 0; i < (low < n ? low : n); ++i) ids.push_back((int32_t)i);
  for (int64_t i = 0; i < specials; ++i) ids.push_back((int32_t)(sf + i));
  return ids;
}

size_t head_ws_bytes(const Head* hd, int S, int T) {
  const mtpx_head_config& g = hd->cfg;
  const int H = g.layer.hidden, W = g.hc * H, LW = g.lowrank, HQ = g.layer.heads, D = g.layer.head_dim;
  const int XB = (H > HQ * D ? H : HQ * D) / 32;
  // per mixer call (three per step): lo, act [S, LW]; inj [S, hc]; xpL; w [S, W]
  const size_t mix = al(2 * (size_t)S * LW) * 2 + al(2 * (size_t)S * g.hc) + al(4 * (size_t)S * (LW / 32) * XP_DW) +
                     al(2 * (size_t)S * W) + (S > MAX_TOKENS ? al(4 * (size_t)S * (W / 32) * XMB_DW) : 0);
  const size_t moe = S > MAX_TOKENS ? moe_windows_ws_bytes(&hd->w.layer.moe, S) : moe_ws_bytes(&hd->w.layer.moe, S);
  return moe + attn_ws_bytes(hd->layer, S, T) + 3 * mix + al(2 * (size_t)S * H) * 6 +
         al(2 * (size_t)S * W) * 5 + al(2 * (size_t)S * g.hc) + al(4 * (size_t)S * XB * XP_DW) +
         al(4 * (size_t)S * (W / 32) * XP_DW) + al(2 * (size_t)hd->w.shortlist_rows) +
         al(4 * argmax_work_items(1, hd->w.shortlist_rows)) * 2 + 8192;
}

// One hyper-connection mixer over the normed rows (prepared blocks in xpW):
// lo = down n, inj = inject n, act = silu(lo), w = up act,
// x = sum_c sigmoid(w) * n (+ its prepared blocks in xpH), j = 2 * sigmoid(inj).
struct HcGeom {
  int H, hc, LW, gs;  // hidden, streams, low rank, group size
};

int hc_mix_enqueue(Ctx* c, const HcGeom& g, const mtpx_hc_weights* hw, const uint16_t* normed, const uint32_t* xpW,
                   int S, uint16_t* x, uint16_t* j, uint32_t* xpH) {
  const int H = g.H, W = g.hc * H, LW = g.LW, gs = g.gs;
  hipStream_t st = c->stream;
  if (mix_supported(H, g.hc, LW, S)) {
    MixArgs a;
    a.H = H;
    a.hc = g.hc;
    a.LW = LW;
    a.gs = gs;
    a.S = S;
    a.dw = hw->down.w; a.ds = hw->down.s; a.db = hw->down.b; a.dsb = hw->down.sb;
    a.iw = hw->inject.w; a.is = hw->inject.s; a.ib = hw->inject.b; a.isb = hw->inject.sb;
    a.uw = hw->up.w; a.us = hw->up.s; a.ub = hw->up.b; a.usb = hw->up.sb;
    a.xpW = xpW;
    a.normed = reinterpret_cast<const bf16*>(normed);
    a.part = ws_take<float>(c, (size_t)mix_classes(W) * S * (LW + g.hc));
    a.x = reinterpret_cast<bf16*>(x);
    a.j = reinterpret_cast<bf16*>(j);
    a.xpH = xpH;
    LAUNCH(c, "mixer", launch_mixer(a, st));
    return MTPX_OK;
  }
  uint16_t* lo = ws_take<uint16_t>(c, (size_t)S * LW);
  uint16_t* act = ws_take<uint16_t>(c, (size_t)S * LW);
  uint16_t* inj = ws_take<uint16_t>(c, (size_t)S * g.hc);
  uint32_t* xpL = ws_take<uint32_t>(c, (size_t)S * (LW / 32) * XP_DW);
  uint16_t* wm = ws_take<uint16_t>(c, (size_t)S * W);
  if (qmv_pair_ok(hw->down.sb, hw->inject.w, hw->inject.sb, W, S)) {  // a batch: down and inject rows in one launch
    uint32_t* xmb = ws_take<uint32_t>(c, (size_t)S * (W / 32) * XMB_DW);
    LAUNCH(c, "hc_down_inject", launch_qmv_pair(hw->down.w, hw->down.sb, LW, reinterpret_cast<bf16*>(lo), hw->inject.w,
                                                hw->inject.sb, g.hc, reinterpret_cast<bf16*>(inj), W, gs, xpW, xmb, S, st));
  } else {
    LAUNCH(c, "hc_down", launch_qmv(hw->down.w, hw->down.s, hw->down.b, hw->down.sb, LW, W, gs, xpW, S, lo, nullptr, st));
    if (hw->inject.w)
      LAUNCH(c, "hc_inject", launch_qmv(hw->inject.w, hw->inject.s, hw->inject.b, hw->inject.sb, g.hc, W, gs, xpW, S, inj, nullptr, st));
  }
  LAUNCH(c, "hc_silu", launch_silu_xprep(lo, S, LW, act, xpL, st));
  LAUNCH(c, "hc_up", launch_qmv(hw->up.w, hw->up.s, hw->up.b, hw->up.sb, W, LW, gs, xpL, S, wm, nullptr, st));
  LAUNCH(c, "hc_mix", launch_hc_mix(wm, normed, hw->inject.w ? inj : nullptr, S, g.hc, H, x, j, xpH, st));
  return MTPX_OK;
}

int hc_mix_enqueue(Ctx* c, const Head* hd, const mtpx_hc_weights* hw, const uint16_t* normed, const uint32_t* xpW,
                   int S, uint16_t* x, uint16_t* j, uint32_t* xpH) {
  const HcGeom g{hd->cfg.layer.hidden, hd->cfg.hc, hd->cfg.lowrank, hd->cfg.layer.group_size};
  return hc_mix_enqueue(c, g, hw, normed, xpW, S, x, j, xpH);
}

// One hyper-connection mixer's weights (random init): hc_norm weight 1/hc (a
// power of two for hc in {1, 2, 4, 8}), q4 down/inject/up.
void hc_random(RandInit& ri, int H, int hc, int LW, bool inject, mtpx_hc_weights* m) {
  const int W = hc * H;
  m->norm_scale = ri.dense(W, 0.0f, bf16_bits(1.0f / (float)hc));
  ri.qmat(LW, W, &m->down);
  if (inject) ri.qmat(hc, W, &m->inject);
  ri.qmat(W, LW, &m->up);
}

int head_create(Ctx* c, const mtpx_head_config* cfg, uint64_t seed, Head** out) {
  int rc = head_check(cfg);
  if (rc) return rc;
  Head* hd = new Head();
  hd->cfg = *cfg;
  memset(&hd->w, 0, sizeof(hd->w));
  if ((rc = layer_create(c, &cfg->layer, seed, &hd->layer))) {
    delete hd;
    return rc;
  }
  hd->w.layer = hd->layer->w;
  const int H = cfg->layer.hidden, W = cfg->hc * H, LW = cfg->lowrank;
  RandInit ri{c, seed ^ 0x9E3779B97F4A7C15ull, cfg->layer.group_size, &hd->allocs};
  mtpx_head_weights& w = hd->w;
  ri.qmat(cfg->vocab, H, &w.embed);
  w.pre_norm_embedding = ri.dense(H, 0.0f);
  w.pre_norm_hidden = ri.dense(W, 0.0f);
  ri.qmat(H, H, &w.fc_embedding);
  ri.qmat(H, H, &w.fc_hidden);
  mtpx_hc_weights* hcs[3] = {&w.attn_hc, &w.mlp_hc, &w.final_hc};
  for (int i = 0; i < 3; ++i) hc_random(ri, H, cfg->hc, LW, i < 2, hcs[i]);
  const std::vector<int32_t> ids = shortlist_ids(cfg);
  w.shortlist_rows = (int)ids.size();
  ri.qmat((int64_t)ids.size(), H, &w.shortlist);
  int32_t* dids = (int32_t*)ri.alloc(ids.size() * 4);
  if (dids && hipMemcpyAsync(dids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess)
    ri.ok = false;
  w.shortlist_ids = dids;
  if ((rc = ri.finish("head"))) {
    for (void* p : hd->allocs) hipFree(p);
    for (void* p : hd->layer->allocs) hipFree(p);
    delete hd->layer;
    delete hd;
    return rc;
  }
  *out = hd;
  return MTPX_OK;
}

// ---------------------------------------------------------------------------
// Drafter backend: rows in pooled device buffers (token ids, then bf16 rows of
// width W), the head run in windows of at most MAX_TOKENS inputs.  Buffers go
// back to the pool when their Rows die; reuse is ordered behind earlier reads by
// the one context stream.
struct RowPool {
  std::vector<std::pair<int, void*>> free_;  // (capacity rows, buffer)
  std::vector<void*> all_;
  void* get(int n, int W, int* cap) {
    int c = 1;
    while (c < n) c *= 2;
    for (size_t i = 0; i < free_.size(); ++i)
      if (free_[i].first == c) {
        void* p = free_[i].second;
        free_.erase(free_.begin() + i);
        *cap = c;
        return p;
      }
    void* p = nullptr;
    if (hipMalloc(&p, al(4 * (size_t)c) + 2 * (size_t)c * W) != hipSuccess) return nullptr;
    all_.push_back(p);
    *cap = c;
    return p;
  }
  void put(int cap, void* p) { free_.push_back({cap, p}); }
  ~RowPool() {
    for (void* p : all_) hipFree(p);
  }
};

struct DevBackend {
  struct Rows {
    RowPool* pool = nullptr;
    void* buf = nullptr;
    int n = 0, cap = 0, W = 0;
    Rows() = default;
    Rows(const Rows&) = delete;
    Rows& operator=(const Rows&) = delete;
    Rows(Rows&& o) noexcept { *this = std::move(o); }
    Rows& operator=(Rows&& o) noexcept {
      if (this != &o) {
        release();
        pool = o.pool; buf = o.buf; n = o.n; cap = o.cap; W = o.W;
        o.buf = nullptr; o.n = 0;
      }
      return *this;
    }
    ~Rows() { release(); }
    void release() {
      if (buf && pool) pool->put(cap, buf);
      buf = nullptr;
    }
  };

  Ctx* c = nullptr;
  mtpx_head hh{nullptr};
  Kv* kv = nullptr;
  int W = 0;
  RowPool pool;
  uint16_t* multi_scratch = nullptr;  // [MAX_TOKENS, W]

  static int count(const Rows& r) { return r.n; }
  static int32_t* tok(const Rows& r) { return static_cast<int32_t*>(r.buf); }
  static uint16_t* hid(const Rows& r) {
    return reinterpret_cast<uint16_t*>(static_cast<char*>(r.buf) + al(4 * (size_t)r.cap));
  }
  bool ok(const Rows& r) const { return r.buf != nullptr; }

  Rows make(const int32_t* t, const uint16_t* h, int n) {
    Rows r;
    r.pool = &pool;
    r.W = W;
    r.n = n;
    r.buf = pool.get(n, W, &r.cap);
    if (!r.buf) return r;
    if ((t && hipMemcpyAsync(tok(r), t, 4 * (size_t)n, hipMemcpyDeviceToDevice, c->stream) != hipSuccess) ||
        hipMemcpyAsync(hid(r), h, 2 * (size_t)n * W, hipMemcpyDeviceToDevice, c->stream) != hipSuccess)
      r.release();
    return r;
  }

  int head_run(const std::vector<const Rows*>& segs, int32_t* draft, uint16_t* multi) {
    int S = 0;
    for (const Rows* r : segs) S += r->n;
    const int32_t* t = nullptr;
    const uint16_t* h = nullptr;
    Rows staged;
    if (segs.size() == 1) {
      t = tok(*segs[0]);
      h = hid(*segs[0]);
    } else {
      staged.pool = &pool;
      staged.W = W;
      staged.n = S;
      staged.buf = pool.get(S, W, &staged.cap);
      if (!staged.buf) return MTPX_ERR_OOM;
      int off = 0;
      for (const Rows* r : segs) {
        HIP_OK(hipMemcpyAsync(tok(staged) + off, tok(*r), 4 * (size_t)r->n, hipMemcpyDeviceToDevice, c->stream));
        HIP_OK(hipMemcpyAsync(hid(staged) + (size_t)off * W, hid(*r), 2 * (size_t)r->n * W,
                              hipMemcpyDeviceToDevice, c->stream));
        off += r->n;
      }
      t = tok(staged);
      h = hid(staged);
    }
    mtpx_ctx ch{c};
    mtpx_kv kh{kv};
    int rc = MTPX_OK, last = 0;
    for (int off = 0; off < S; off += HEAD_BATCH) {  // the backlog in batches (the same bits as windows of 8)
      last = S - off < HEAD_BATCH ? S - off : HEAD_BATCH;
      const bool end = off + last == S;
      rc = mtpx_head_forward(ch, hh, kh, t + off, last, h + (size_t)off * W, multi_scratch, nullptr,
                             end ? draft : nullptr);
      if (rc) return rc;
    }
    HIP_OK(hipMemcpyAsync(multi, multi_scratch + (size_t)(last - 1) * W, 2 * (size_t)W, hipMemcpyDeviceToDevice,
                          c->stream));
    return MTPX_OK;
  }
  int head(const std::vector<const Rows*>& segs, int32_t* draft, uint16_t* multi) {
    return head_run(segs, draft, multi);
  }
  int64_t offset() { return kv->offset; }
  int64_t trim(int64_t n) {
    const int64_t t = n < kv->offset ? n : kv->offset;
    kv->offset -= t;
    return t;
  }
};

struct DrafterObj {
  DevBackend be;
  Drafter<DevBackend>* d = nullptr;
};

}  // namespace

// ---------------------------------------------------------------------------
// Gated-deltanet sublayer (gdn.hip).
namespace {

struct GdnGeom {
  int hk, hv, kc, cd, pw, z_off, b_off, a_off;
};

GdnGeom gdn_geom(const mtpx_gdn_config& g) {
  GdnGeom r;
  r.hk = g.key_heads;
  r.hv = g.value_heads;
  r.kc = g.conv_kernel;
  r.cd = (2 * g.key_heads + g.value_heads) * 128;
  r.z_off = r.cd;
  r.b_off = r.cd + g.value_heads * 128;
  r.a_off = r.b_off + g.value_heads;
  r.pw = r.a_off + g.value_heads;
  return r;
}

int gdn_check(const mtpx_gdn_config* g) {
  ARG(g, "null config");
  ARG(gs_ok(g->group_size), "group_size=%d", g->group_size);
  ARG(g->hidden >= 32 && k_ok(g->hidden, g->group_size), "hidden=%d unsupported", g->hidden);
  ARG(g->key_heads >= 1 && g->value_heads >= g->key_heads && g->value_heads % g->key_heads == 0 &&
          g->value_heads <= 256,
      "key_heads=%d value_heads=%d", g->key_heads, g->value_heads);
  ARG(k_ok(g->value_heads * 128, g->group_size), "value_heads*128=%d unsupported GEMV depth", g->value_heads * 128);
  ARG(g->conv_kernel >= 2 && g->conv_kernel <= 8, "conv_kernel=%d", g->conv_kernel);
  ARG(g->eps > 0.0f, "eps must be positive");
  return MTPX_OK;
}

struct GdnLayer {
  mtpx_gdn_config cfg;
  mtpx_gdn_weights w;
  std::vector<void*> allocs;
};

struct GdnState {
  mtpx_gdn_config cfg;
  uint16_t* conv[2] = {nullptr, nullptr};  // conv base per slot [kc-1, cd]
  uint16_t* win[2] = {nullptr, nullptr};   // window conv input rows [MAX_TOKENS, cd]
  uint16_t* key[2] = {nullptr, nullptr};   // [MAX_TOKENS, hk, 128]
  float* delta[2] = {nullptr, nullptr};    // [MAX_TOKENS, hv, 128]
  float* decay[2] = {nullptr, nullptr};    // [MAX_TOKENS, hv]
  float* ssm = nullptr;                    // [hv, 128, 128]
  uint32_t* tickets = nullptr;             // [hv] per-head last-arriver counters of the step, zero at rest
  float* ypub = nullptr;                   // [MAX_TOKENS, hv, 128] the step's published recurrence outputs
  int cur = 0, window = 0, committed = 0;
  std::vector<void*> allocs;
};

// splitmix64 -> uniform [0, 1): host-side values of the small per-head vectors
double host_uniform(uint64_t& s) {
  uint64_t z = (s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  z ^= z >> 31;
  return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

// Weights of one GDN sublayer (random init): q4 projections, conv taps ~ N(0, 0.3);
// A_log = log U(1, 16); dt = U(0.001, 0.1) with dt_bias its softplus inverse; norm
// weight U(0.9, 1.1).
void gdn_random(RandInit& ri, const mtpx_gdn_config& cfg, uint64_t seed, mtpx_gdn_weights* w) {
  const GdnGeom g = gdn_geom(cfg);
  ri.qmat(g.pw, cfg.hidden, &w->in_proj);
  ri.qmat(cfg.hidden, g.hv * 128, &w->out_proj);
  w->conv_w = ri.dense((int64_t)g.cd * g.kc, 0.3f);
  uint64_t hs = seed ^ 0x6a09e667f3bcc908ull;
  std::vector<float> nea(g.hv);
  std::vector<uint16_t> dtb(g.hv), nw(128);
  for (int i = 0; i < g.hv; ++i) {
    nea[i] = (float)(-(1.0 + 15.0 * host_uniform(hs)));
    const double dt = 0.001 + 0.099 * host_uniform(hs);
    dtb[i] = bf16_bits((float)std::log(std::expm1(dt)));
  }
  for (int i = 0; i < 128; ++i) nw[i] = bf16_bits((float)(0.9 + 0.2 * host_uniform(hs)));
  float* pn = (float*)ri.alloc(4 * (size_t)g.hv);
  uint16_t* pd = (uint16_t*)ri.alloc(2 * (size_t)g.hv);
  uint16_t* pw = (uint16_t*)ri.alloc(2 * 128);
  if (pn && pd && pw &&
      (hipMemcpy(pn, nea.data(), 4 * (size_t)g.hv, hipMemcpyHostToDevice) != hipSuccess ||
       hipMemcpy(pd, dtb.data(), 2 * (size_t)g.hv, hipMemcpyHostToDevice) != hipSuccess ||
       hipMemcpy(pw, nw.data(), 2 * 128, hipMemcpyHostToDevice) != hipSuccess))
    ri.ok = false;
  w->neg_exp_alog = pn;
  w->dt_bias = pd;
  w->norm_w = pw;
}

GdnArgs gdn_args(GdnState* st, const GdnLayer* L, const uint16_t* proj, int S, uint16_t* gated, uint32_t* xp) {
  const GdnGeom g = gdn_geom(st->cfg);
  GdnArgs a;
  a.hk = g.hk;
  a.hv = g.hv;
  a.kc = g.kc;
  a.cd = g.cd;
  a.pw = g.pw;
  a.z_off = g.z_off;
  a.b_off = g.b_off;
  a.a_off = g.a_off;
  a.S = S;
  a.P = st->committed;
  a.eps = st->cfg.eps;
  a.proj = reinterpret_cast<const bf16*>(proj);
  a.conv_w = L ? reinterpret_cast<const bf16*>(L->w.conv_w) : nullptr;
  a.neg_exp_alog = L ? L->w.neg_exp_alog : nullptr;
  a.dt_bias = L ? reinterpret_cast<const bf16*>(L->w.dt_bias) : nullptr;
  a.norm_w = L ? reinterpret_cast<const bf16*>(L->w.norm_w) : nullptr;
  const int c = st->cur, n = st->cur ^ 1;
  a.conv_cur = reinterpret_cast<const bf16*>(st->conv[c]);
  a.win_cur = reinterpret_cast<const bf16*>(st->win[c]);
  a.key_cur = reinterpret_cast<const bf16*>(st->key[c]);
  a.delta_cur = st->delta[c];
  a.decay_cur = st->decay[c];
  a.conv_nxt = reinterpret_cast<bf16*>(st->conv[n]);
  a.win_nxt = reinterpret_cast<bf16*>(st->win[n]);
  a.key_nxt = reinterpret_cast<bf16*>(st->key[n]);
  a.delta_nxt = st->delta[n];
  a.decay_nxt = st->decay[n];
  a.ssm = st->ssm;
  a.tickets = st->tickets;
  a.ypub = st->ypub;
  a.gated = reinterpret_cast<bf16*>(gated);
  a.xp = xp;
  return a;
}

bool gdn_same(const mtpx_gdn_config& a, const mtpx_gdn_config& b) {
  return a.key_heads == b.key_heads && a.value_heads == b.value_heads && a.conv_kernel == b.conv_kernel;
}

// one window through the core; the state's slots advance
int gdn_enqueue(Ctx* c, const GdnLayer* L, GdnState* st, const uint16_t* proj, int S, uint16_t* gated, uint32_t* xp) {
  const GdnArgs a = gdn_args(st, L, proj, S, gated, xp);
  LAUNCH(c, "gdn_step", launch_gdn_step(a, c->stream));
  st->cur ^= 1;
  st->window = S;
  st->committed = 0;
  return MTPX_OK;
}

// A prefill batch of S positions through the core in one launch, every position committed: the
// state holds them all, the conv base is in the other slot, nothing is left to replay.
// Workspace: S * (hv * 128 + (2 hk + hv) * 128 + 2 hv) floats (recurrence outputs, prepped vectors, gates).
int gdn_enqueue_batch(Ctx* c, const GdnLayer* L, GdnState* st, const uint16_t* proj, int S, uint16_t* gated,
                      uint32_t* xp) {
  GdnArgs a = gdn_args(st, L, proj, S, gated, xp);
  a.ypub = ws_take<float>(c, (size_t)S * a.hv * 128);
  GdnBatch b;
  b.vecs = ws_take<float>(c, (size_t)S * (2 * a.hk + a.hv) * 128);
  b.gates = ws_take<float>(c, (size_t)S * a.hv * 2);
  LAUNCH(c, "gdn_batch", launch_gdn_batch(a, b, c->stream));
  st->cur ^= 1;
  st->window = 0;
  st->committed = 0;
  return MTPX_OK;
}

}  // namespace


// ---------------------------------------------------------------------------
// The PLE n-gram block (layer index 1 of the target).
namespace {

struct PleGeom {
  int W, nh, row_dim, ctx_len, nb;  // stream width, heads, row width, carried tokens, carried conv rows
};

PleGeom ple_geom(const mtpx_ple_config& g) {
  PleGeom r;
  r.W = g.hc * g.hidden;
  r.nh = (g.ngram_size - 1) * g.heads_per_ngram;
  r.row_dim = r.nh > 0 ? g.embed_dim / r.nh : 0;
  r.ctx_len = g.ngram_size - 1 > 1 ? g.ngram_size - 1 : 1;
  r.nb = (g.conv_kernel - 1) * g.ngram_size;
  return r;
}

int ple_check(const mtpx_ple_config* g) {
  ARG(g, "null config");
  ARG(gs_ok(g->group_size), "group_size=%d", g->group_size);
  ARG(g->hidden >= 256 && g->hidden % 256 == 0 && g->hidden <= 4096, "hidden=%d (a multiple of 256, <= 4096)",
      g->hidden);
  ARG(g->hc >= 1 && g->hc <= 8, "hc=%d", g->hc);
  ARG(g->ngram_size >= 2 && g->ngram_size <= MTPX_PLE_MAX_NGRAM && g->ngram_size - 1 <= PLE_MAX_CTX, "ngram_size=%d",
      g->ngram_size);
  const PleGeom pg = ple_geom(*g);
  ARG(g->heads_per_ngram >= 1 && pg.nh <= MTPX_PLE_MAX_HEADS, "heads_per_ngram=%d", g->heads_per_ngram);
  ARG(g->row_group_size == 32 || g->row_group_size == 64, "row_group_size=%d", g->row_group_size);
  ARG(g->embed_dim % 256 == 0 && g->embed_dim % pg.nh == 0 && pg.row_dim % g->row_group_size == 0 &&
          k_ok(g->embed_dim, g->group_size),
      "embed_dim=%d (a multiple of 256 and of the %d heads; row width %d a multiple of row_group_size)", g->embed_dim,
      pg.nh, pg.row_dim);
  ARG(g->conv_kernel >= 1 && g->conv_kernel <= 8, "conv_kernel=%d", g->conv_kernel);
  ARG(g->vocab_base >= 1 && g->vocab_base < ((int64_t)1 << 30), "vocab_base=%lld", (long long)g->vocab_base);
  ARG(g->token_vocab >= 2 && g->token_vocab < ((int64_t)1 << 31) && g->eos >= 0 && g->eos < g->token_vocab,
      "token_vocab=%lld eos=%d", (long long)g->token_vocab, g->eos);
  ARG(g->eps > 0.0f, "eps must be positive");
  return MTPX_OK;
}

bool is_prime(int64_t v) {
  if (v < 2) return false;
  for (int64_t d = 2; d * d <= v; ++d)
    if (v % d == 0) return false;
  return true;
}

// Head vocabularies (consecutive primes above the base), their offsets (running
// sum) and the table's row count: docs/ngram-cache-design.md:62-64, 84-89.
int64_t ngram_heads(const mtpx_ple_config& g, mtpx_ngram_table* t) {
  const int nh = ple_geom(g).nh;
  int64_t v = g.vocab_base, off = 0;
  for (int h = 0; h < nh; ++h) {
    do ++v;
    while (!is_prime(v));
    t->vocab[h] = v;
    t->offset[h] = off;
    off += v;
  }
  t->rows = off;
  return off;
}

struct PleLayer {
  mtpx_ple_config cfg;
  mtpx_ple_weights w;
  int64_t* hash = nullptr;  // device [ngram + 2*heads]: multipliers | vocab sizes | offsets
  std::vector<void*> allocs;
};

struct PleState {
  mtpx_ple_config cfg;
  uint16_t* conv[2] = {nullptr, nullptr};  // base conv rows per slot [nb, W]
  uint16_t* win[2] = {nullptr, nullptr};   // window normed rows [MAX_TOKENS, W]
  int32_t* ctx[2] = {nullptr, nullptr};    // base context [ctx_len]
  int32_t* ids[2] = {nullptr, nullptr};    // window tokens [MAX_TOKENS]
  int cur = 0, window = 0, committed = 0;
  std::vector<void*> allocs;
};

bool ple_same(const mtpx_ple_config& a, const mtpx_ple_config& b) {
  return a.hidden == b.hidden && a.hc == b.hc && a.ngram_size == b.ngram_size && a.conv_kernel == b.conv_kernel;
}

// Random PLE weights; the multipliers are odd and below (2^63-1) / token_vocab / 2, so every
// product token * multiplier stays non-negative (docs/ngram-cache-design.md:71-79).
int ple_random(Ctx* c, const mtpx_ple_config& cfg, uint64_t seed, PleLayer* L) {
  const PleGeom pg = ple_geom(cfg);
  const int H = cfg.hidden, W = pg.W;
  RandInit ri{c, seed, cfg.group_size, &L->allocs};
  mtpx_ple_weights& w = L->w;
  memset(&w, 0, sizeof(w));
  ri.qmat(W, cfg.embed_dim, &w.key_proj);
  ri.qmat(H, cfg.embed_dim, &w.value_proj);
  w.conv_w = ri.dense((int64_t)W * cfg.conv_kernel, 0.3f);
  uint64_t hs = seed ^ 0x510e527fade682d1ull;
  std::vector<uint16_t> nrm(3 * (size_t)W);
  for (auto& v : nrm) v = bf16_bits((float)(0.8 + 0.4 * host_uniform(hs)));
  uint16_t* pn = (uint16_t*)ri.alloc(2 * nrm.size());
  if (pn && hipMemcpy(pn, nrm.data(), 2 * nrm.size(), hipMemcpyHostToDevice) != hipSuccess) ri.ok = false;
  w.norm_key = pn;
  w.norm_query = pn ? pn + W : nullptr;
  w.norm_conv = pn ? pn + 2 * (size_t)W : nullptr;
  mtpx_ngram_table& t = w.table;
  const int64_t rows = ngram_heads(cfg, &t);
  const uint64_t bound = 0x7fffffffffffffffull / (uint64_t)cfg.token_vocab / 2;
  for (int p = 0; p < cfg.ngram_size; ++p)
    t.multiplier[p] = (int64_t)(((uint64_t)(host_uniform(hs) * 9007199254740992.0) % (bound / 2)) * 2 + 1);
  const int rgs = cfg.row_group_size;
  uint32_t* tw = (uint32_t*)ri.alloc((size_t)rows * pg.row_dim / 2);
  uint16_t* ts = (uint16_t*)ri.alloc((size_t)rows * (pg.row_dim / rgs) * 2);
  uint16_t* tb = (uint16_t*)ri.alloc((size_t)rows * (pg.row_dim / rgs) * 2);
  t.w = tw;
  t.s = ts;
  t.b = tb;
  if (tw && ts && tb) {
    // random nibbles (bf16 normal bit patterns), scales and biases ~ N(0, 0.02)
    if (launch_randn_bf16(reinterpret_cast<bf16*>(tw), rows * pg.row_dim / 4, seed, 0x7e000001u, 1.0f, c->stream) ||
        launch_randn_bf16(reinterpret_cast<bf16*>(ts), rows * (pg.row_dim / rgs), seed, 0x7e000002u, 0.02f,
                          c->stream) ||
        launch_randn_bf16(reinterpret_cast<bf16*>(tb), rows * (pg.row_dim / rgs), seed, 0x7e000003u, 0.02f,
                          c->stream))
      ri.ok = false;
  }
  const int nh = pg.nh, n = cfg.ngram_size;
  std::vector<int64_t> hv(n + 2 * (size_t)nh);
  for (int p = 0; p < n; ++p) hv[p] = t.multiplier[p];
  for (int h = 0; h < nh; ++h) {
    hv[n + h] = t.vocab[h];
    hv[n + nh + h] = t.offset[h];
  }
  L->hash = (int64_t*)ri.alloc(8 * hv.size());
  if (L->hash && hipMemcpy(L->hash, hv.data(), 8 * hv.size(), hipMemcpyHostToDevice) != hipSuccess) ri.ok = false;
  return ri.finish("ple");
}

PleRowArgs ple_row_args(const PleLayer* L, const int32_t* ids, int S) {
  const PleGeom pg = ple_geom(L->cfg);
  PleRowArgs a;
  memset(&a, 0, sizeof(a));
  a.S = S;
  a.ctx_len = pg.ctx_len;
  a.ngram = L->cfg.ngram_size;
  a.hpn = L->cfg.heads_per_ngram;
  a.row_dim = pg.row_dim;
  a.rgs = L->cfg.row_group_size;
  a.eos = L->cfg.eos;
  a.rows = L->w.table.rows;
  a.hash = L->hash;
  a.ids = ids;
  a.tw = L->w.table.w;
  a.ts = reinterpret_cast<const bf16*>(L->w.table.s);
  a.tb = reinterpret_cast<const bf16*>(L->w.table.b);
  return a;
}

size_t ple_ws_bytes(const mtpx_ple_config& g, int S) {
  const PleGeom pg = ple_geom(g);
  return al(2 * (size_t)S * g.embed_dim) + al(4 * (size_t)S * (g.embed_dim / 32) * XP_DW) +
         al(2 * (size_t)S * pg.W) * 2 + al(2 * (size_t)S * g.hidden) + 4096;
}

// One window through the block (workspace from the context); the state's slots advance.
int ple_enqueue(Ctx* c, const PleLayer* L, PleState* st, const int32_t* ids, int S, const uint16_t* stream,
                uint16_t* out, uint16_t* sum, uint16_t* embedded) {
  const mtpx_ple_config& g = L->cfg;
  const PleGeom pg = ple_geom(g);
  const int H = g.hidden, E = g.embed_dim, gs = g.group_size;
  uint16_t* emb = embedded ? embedded : ws_take<uint16_t>(c, (size_t)S * E);
  uint32_t* xp = ws_take<uint32_t>(c, (size_t)S * (E / 32) * XP_DW);
  uint16_t* key = ws_take<uint16_t>(c, (size_t)S * pg.W);
  uint16_t* gated = ws_take<uint16_t>(c, (size_t)S * pg.W);
  uint16_t* value = ws_take<uint16_t>(c, (size_t)S * H);
  const int cs = st->cur, ns = st->cur ^ 1;
  PleRowArgs ra = ple_row_args(L, ids, S);
  ra.P = st->committed;
  ra.ctx_cur = st->ctx[cs];
  ra.ids_prev = st->ids[cs];
  ra.ctx_nxt = st->ctx[ns];
  ra.ids_nxt = st->ids[ns];
  ra.emb = reinterpret_cast<bf16*>(emb);
  ra.xp = xp;
  hipStream_t s = c->stream;
  LAUNCH(c, "ple_rows", launch_ple_rows(ra, s));
  const mtpx_q4& kp = L->w.key_proj;
  const mtpx_q4& vp = L->w.value_proj;
  LAUNCH(c, "qmv_ple_key", launch_qmv(kp.w, kp.s, kp.b, kp.sb, pg.W, E, gs, xp, S, key, nullptr, s));
  LAUNCH(c, "qmv_ple_value", launch_qmv(vp.w, vp.s, vp.b, vp.sb, H, E, gs, xp, S, value, nullptr, s));
  LAUNCH(c, "ple_gate", launch_ple_gate(key, stream, value, L->w.norm_key, L->w.norm_query, L->w.norm_conv, S, g.hc, H,
                                        g.eps, gated, st->win[ns], s));
  PleConvArgs ca;
  ca.S = S;
  ca.kc = g.conv_kernel;
  ca.dil = g.ngram_size;
  ca.P = st->committed;
  ca.W = pg.W;
  ca.conv_cur = st->conv[cs];
  ca.win_cur = st->win[cs];
  ca.win_nxt = st->win[ns];
  ca.conv_w = L->w.conv_w;
  ca.gated = gated;
  ca.stream = stream;
  ca.out = out;
  ca.sum = sum;
  ca.conv_nxt = st->conv[ns];
  LAUNCH(c, "ple_conv", launch_ple_conv(ca, s));
  st->cur = ns;
  st->window = S;
  st->committed = 0;
  return MTPX_OK;
}

int ple_state_create(Ctx* c, const mtpx_ple_config& cfg, PleState** out) {
  const PleGeom pg = ple_geom(cfg);
  PleState* st = new PleState();
  st->cfg = cfg;
  bool ok = true;
  auto take = [&](size_t bytes) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
      ok = false;
      return nullptr;
    }
    st->allocs.push_back(p);
    return p;
  };
  for (int s = 0; s < 2; ++s) {
    st->conv[s] = (uint16_t*)take(2 * (size_t)(pg.nb > 0 ? pg.nb : 1) * pg.W);
    st->win[s] = (uint16_t*)take(2 * (size_t)MAX_TOKENS * pg.W);
    st->ctx[s] = (int32_t*)take(4 * (size_t)PLE_MAX_CTX);
    st->ids[s] = (int32_t*)take(4 * (size_t)MAX_TOKENS);
  }
  if (ok) {
    std::vector<int32_t> eos(PLE_MAX_CTX, cfg.eos);
    if (hipMemsetAsync(st->conv[0], 0, 2 * (size_t)(pg.nb > 0 ? pg.nb : 1) * pg.W, c->stream) != hipSuccess ||
        hipMemcpyAsync(st->ctx[0], eos.data(), 4 * eos.size(), hipMemcpyHostToDevice, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
      ok = false;
  }
  if (!ok) {
    for (void* p : st->allocs) hipFree(p);
    delete st;
    return fail(MTPX_ERR_OOM, "ple state allocation failed");
  }
  *out = st;
  return MTPX_OK;
}

void ple_state_release(PleState* st) {
  for (void* p : st->allocs) hipFree(p);
  delete st;
}

}  // namespace

// ---------------------------------------------------------------------------
// The target model's verify forward.
namespace {

struct TargetLayer {
  int kind = MTPX_LAYER_GDN;
  Layer* attn = nullptr;     // attention layers: attention + MoE weights
  GdnLayer* gdn = nullptr;   // GDN layers
  mtpx_moe_weights moe;      // this layer's MoE
  mtpx_hc_weights attn_hc, mlp_hc;
};

struct Target {
  mtpx_target_config cfg;
  std::vector<TargetLayer> layers;
  mtpx_q4 embed, lm_head;
  mtpx_hc_weights final_hc;
  PleLayer* ple = nullptr;  // the PLE layer's block (ple_layer >= 0)
  std::vector<void*> allocs;
};

struct TargetState {
  Target* t = nullptr;
  std::vector<Kv*> kv;          // per layer (attention layers), else null
  std::vector<GdnState*> gdn;   // per layer (GDN layers), else null
  PleState* ple = nullptr;      // the PLE layer's state
  std::vector<void*> allocs;
  int32_t* moe_unique = nullptr;  // device [num_layers]: distinct routed experts of the last verify
  int64_t offset = 0;           // committed positions
  int window = 0;
  // A verify that failed after its first launch may have advanced some layers' window state
  // (GDN slots flipped, K/V rows written at the committed offset): the state refuses verify and
  // commit until mtpx_target_state_reset.
  bool broken = false;
};

// Committed GDN state back to zero (conv rows, recurrent state, tickets); no window.
int gdn_state_zero(Ctx* c, GdnState* st) {
  const GdnGeom g = gdn_geom(st->cfg);
  st->cur = 0;
  st->window = 0;
  st->committed = 0;
  HIP_OK(hipMemsetAsync(st->tickets, 0, 4 * (size_t)g.hv, c->stream));
  HIP_OK(hipMemsetAsync(st->conv[0], 0, 2 * (size_t)(g.kc - 1) * g.cd, c->stream));
  HIP_OK(hipMemsetAsync(st->ssm, 0, 4 * (size_t)g.hv * 128 * 128, c->stream));
  return MTPX_OK;
}

// PLE state back to its fresh defaults: zero conv rows, an eos context; no window.
int ple_state_zero(Ctx* c, PleState* st) {
  const PleGeom pg = ple_geom(st->cfg);
  st->cur = 0;
  st->window = 0;
  st->committed = 0;
  std::vector<int32_t> eos(PLE_MAX_CTX, st->cfg.eos);
  HIP_OK(hipMemsetAsync(st->conv[0], 0, 2 * (size_t)(pg.nb > 0 ? pg.nb : 1) * pg.W, c->stream));
  HIP_OK(hipMemcpyAsync(st->ctx[0], eos.data(), 4 * eos.size(), hipMemcpyHostToDevice, c->stream));
  HIP_OK(hipStreamSynchronize(c->stream));  // the host vector goes out of scope
  return MTPX_OK;
}

mtpx_gdn_config target_gdn_cfg(const mtpx_target_config& g) {
  mtpx_gdn_config r;
  r.hidden = g.layer.hidden;
  r.key_heads = g.key_heads;
  r.value_heads = g.value_heads;
  r.conv_kernel = g.conv_kernel;
  r.group_size = g.layer.group_size;
  r.eps = g.layer.eps;
  return r;
}

int target_check(const mtpx_target_config* g) {
  ARG(g, "null config");
  int rc = layer_check(&g->layer);
  if (rc) return rc;
  const mtpx_gdn_config gc = target_gdn_cfg(*g);
  if ((rc = gdn_check(&gc))) return rc;
  const int H = g->layer.hidden, gs = g->layer.group_size;
  ARG(g->num_layers >= 1 && g->num_layers <= 256 && g->full_attention_interval >= 1, "num_layers=%d interval=%d",
      g->num_layers, g->full_attention_interval);
  ARG(g->hc >= 1 && g->hc <= 8 && g->lowrank >= 32 && g->lowrank % 32 == 0, "hc=%d lowrank=%d", g->hc, g->lowrank);
  ARG(k_ok(g->hc * H, gs) && k_ok(g->lowrank, gs) && g->hc * H <= 256 * 48, "unsupported mixer GEMV depths");
  ARG(g->vocab >= 1 && g->vocab < ((int64_t)1 << 31), "vocab=%lld", (long long)g->vocab);
  ARG(g->ple_layer >= -1 && g->ple_layer < g->num_layers, "ple_layer=%d of %d layers", g->ple_layer, g->num_layers);
  if (g->ple_layer >= 0) {
    ARG(g->ple.hidden == H && g->ple.hc == g->hc && g->ple.group_size == gs,
        "ple geometry (hidden %d, hc %d, group_size %d) differs from the target's", g->ple.hidden, g->ple.hc,
        g->ple.group_size);
    if ((rc = ple_check(&g->ple))) return rc;
  }
  return MTPX_OK;
}

void target_release(Target* t) {
  for (TargetLayer& L : t->layers) {
    if (L.attn) {
      for (void* p : L.attn->allocs) hipFree(p);
      delete L.attn;
    }
    if (L.gdn) {
      for (void* p : L.gdn->allocs) hipFree(p);
      delete L.gdn;
    }
  }
  if (t->ple) {
    for (void* p : t->ple->allocs) hipFree(p);
    delete t->ple;
  }
  for (void* p : t->allocs) hipFree(p);
  delete t;
}

void target_state_release(TargetState* s) {
  if (s->moe_unique) hipFree(s->moe_unique);
  for (Kv* kv : s->kv)
    if (kv) {
      hipFree(kv->k);
      hipFree(kv->v);
      delete kv;
    }
  for (GdnState* g : s->gdn)
    if (g) {
      for (void* p : g->allocs) hipFree(p);
      delete g;
    }
  if (s->ple) ple_state_release(s->ple);
  delete s;
}

}  // namespace

namespace mtpx {
hipStream_t ctx_stream(mtpx_ctx h) { return C(h)->stream; }
int ctx_device(mtpx_ctx h) { return C(h)->device; }
int set_error(int code, const char* msg) { return fail(code, "%s", msg); }
void target_dims(mtpx_target th, int64_t* vocab, int* width) {
  const Target* t = static_cast<const Target*>(th.ctx);
  *vocab = t->cfg.vocab;
  *width = t->cfg.hc * t->cfg.layer.hidden;
}
int head_width(mtpx_head hh) {
  const Head* hd = static_cast<const Head*>(hh.ctx);
  return hd->cfg.hc * hd->cfg.layer.hidden;
}
void target_own(mtpx_target th, void* p) { static_cast<Target*>(th.ctx)->allocs.push_back(p); }
void head_own(mtpx_head hh, void* p) { static_cast<Head*>(hh.ctx)->allocs.push_back(p); }
std::vector<int32_t> head_shortlist_ids(const mtpx_head_config* cfg) { return shortlist_ids(cfg); }
}  // namespace mtpx

extern "C" {

const char* mtpx_last_error(void) { return g_err.c_str(); }
const char* mtpx_version(void) { return "mtpx 0.1 gfx950"; }

int mtpx_ctx_new(mtpx_ctx* out, int device) {
  ARG(out, "out is NULL");
  int n = 0;
  HIP_OK(hipGetDeviceCount(&n));
  ARG(device >= 0 && device < n, "device %d of %d", device, n);
  Ctx* c = new Ctx();
  c->device = device;
  if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(MTPX_ERR_HIP, "stream creation failed on device %d", device);
  }
  c->stream = c->own;
  // ticket counters of the fused MoE launches, zeroed once (every launch leaves them at zero), and the
  // router logits' publish buffer, all sentinel once (every route puts it back)
  const size_t pub_bytes = (size_t)MAX_TOKENS * MAX_EXPERTS * 4;
  if (hipMalloc((void**)&c->tickets, MOE_TICKETS * 4 + pub_bytes) != hipSuccess ||
      hipMemset(c->tickets, 0, MOE_TICKETS * 4) != hipSuccess ||
      hipMemset(c->tickets + MOE_TICKETS, 0xff, pub_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    if (c->tickets) hipFree(c->tickets);
    hipStreamDestroy(c->own);
    delete c;
    return fail(MTPX_ERR_HIP, "ticket allocation failed on device %d", device);
  }
  static_assert(ROUTE_SENTINEL == 0xffffffffu, "the publish buffer is filled with 0xff bytes");
  c->route_pub = reinterpret_cast<float*>(c->tickets + MOE_TICKETS);
  const hipError_t se = moe_scratch_address(device, &c->scratch);
  if (se != hipSuccess) {
    hipFree(c->tickets);
    hipStreamDestroy(c->own);
    delete c;
    return fail(MTPX_ERR_HIP, "scratch lookup failed on device %d: %s", device, hipGetErrorString(se));
  }
  out->ctx = c;
  return MTPX_OK;
}

int mtpx_ctx_free(mtpx_ctx h) {
  Ctx* c = C(h);
  if (!c) return MTPX_OK;
  hipSetDevice(c->device);
  hipStreamSynchronize(c->stream);
  moe_scratch_release(c->device, c);
  if (c->ws) hipFree(c->ws);
  if (c->tickets) hipFree(c->tickets);
  for (auto& r : c->pending) {
    hipEventDestroy(r.a);
    hipEventDestroy(r.b);
  }
  for (hipEvent_t e : c->ev_free) hipEventDestroy(e);
  if (c->own) hipStreamDestroy(c->own);
  delete c;
  return MTPX_OK;
}

int mtpx_ctx_set_stream(mtpx_ctx h, void* s) {
  Ctx* c = C(h);
  ARG(c, "null context");
  c->stream = static_cast<hipStream_t>(s);
  return MTPX_OK;
}

int mtpx_ctx_use_own_stream(mtpx_ctx h) {
  Ctx* c = C(h);
  ARG(c, "null context");
  c->stream = c->own;
  return MTPX_OK;
}

int mtpx_ctx_synchronize(mtpx_ctx h) {
  Ctx* c = C(h);
  ARG(c, "null context");
  HIP_OK(hipStreamSynchronize(c->stream));
  return MTPX_OK;
}

int mtpx_affine_quantize(mtpx_ctx h, const uint16_t* w, int64_t rows, int K, int gs, uint32_t* wq, uint16_t* s,
                         uint16_t* b) {
  Ctx* c = C(h);
  ARG(c && w && wq && s && b, "null argument");
  ARG(gs_ok(gs) && K > 0 && K % gs == 0 && rows >= 0, "K=%d gs=%d rows=%lld", K, gs, (long long)rows);
  if (set_device(c)) return MTPX_ERR_HIP;
  LAUNCH(c, "quantize", launch_quantize(w, rows, K, gs, wq, s, b, c->stream));
  return MTPX_OK;
}

int mtpx_randn_bf16(mtpx_ctx h, uint16_t* out, int64_t n, uint64_t seed, uint32_t tensor, float sigma) {
  Ctx* c = C(h);
  ARG(c && out && n >= 0, "bad argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  LAUNCH(c, "randn_bf16", launch_randn_bf16(out, n, seed, tensor, sigma, c->stream));
  return MTPX_OK;
}

int mtpx_q4_sb_row_len(int K, int gs) {
  if (!gs_ok(gs) || !k_ok(K, gs)) {
    fail(MTPX_ERR_ARG, "K=%d gs=%d unsupported", K, gs);
    return -1;
  }
  return sb_row_len(K, gs);
}

int mtpx_q4_pack_sb(mtpx_ctx h, const uint16_t* s, const uint16_t* b, int64_t rows, int K, int gs, uint32_t* out) {
  Ctx* c = C(h);
  ARG(c && s && b && out && rows >= 0, "bad argument");
  ARG(gs_ok(gs) && k_ok(K, gs), "K=%d gs=%d", K, gs);
  if (set_device(c)) return MTPX_ERR_HIP;
  LAUNCH(c, "pack_sb", launch_pack_sb(s, b, rows, K, gs, out, c->stream));
  return MTPX_OK;
}

int mtpx_qmv(mtpx_ctx h, const uint32_t* wq, const uint16_t* s, const uint16_t* b, const uint32_t* sb, int N, int K, int gs,
             const uint16_t* x, int M, uint16_t* y, float* yf) {
  Ctx* c = C(h);
  ARG(c && wq && s && b && x && y, "null argument");
  ARG(N >= 1 && M >= 1 && M <= QMV_MAX_TOKENS, "N=%d M=%d", N, M);
  ARG(gs_ok(gs) && k_ok(K, gs), "K=%d gs=%d unsupported", K, gs);
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t xpn = (size_t)M * (K / 32) * XP_DW;
  int rc = ws_reserve(c, al(xpn * 4) + 256);
  if (rc) return rc;
  ws_begin(c);
  uint32_t* xp = ws_take<uint32_t>(c, xpn);
  LAUNCH(c, "xprep", launch_xprep(x, M, K, xp, c->stream));
  LAUNCH(c, "qmv", launch_qmv(wq, s, b, sb, N, K, gs, xp, M, y, yf, c->stream));
  return MTPX_OK;
}

int mtpx_moe_forward(mtpx_ctx h, const mtpx_moe_weights* w, const uint16_t* x, int M, uint16_t* y, int32_t* idx,
                     float* wts, float* logits, int32_t* n_unique) {
  Ctx* c = C(h);
  ARG(c && x && y, "null argument");
  int rc = moe_check(w, M);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  if ((rc = ws_reserve(c, moe_ws_bytes(w, M)))) return rc;
  ws_begin(c);
  if ((rc = moe_enqueue(c, w, x, M, y, idx, wts, logits))) return rc;
  if (n_unique) HIP_OK(hipMemcpyAsync(n_unique, &c->last_disp->n_unique, 4, hipMemcpyDeviceToDevice, c->stream));
  return MTPX_OK;
}

int mtpx_moe_forward_noalloc(mtpx_ctx h, const mtpx_moe_weights* w, const uint16_t* x, int M, uint16_t* y,
                             int32_t* idx, float* wts, float* logits, int32_t* n_unique) {
  Ctx* c = C(h);
  ARG(c && x && y, "null argument");
  int rc = moe_check(w, M);
  if (rc) return rc;
  const size_t need = moe_ws_bytes(w, M);
  ARG(need <= moe_scratch_bytes(), "the MoE window needs %zu bytes of scratch; the maximum is %zu", need,
      moe_scratch_bytes());
  ARG(c->scratch, "no scratch on device %d", c->device);
  if (!moe_scratch_claim(c->device, c))
    return fail(MTPX_ERR_STATE, "the allocation-free MoE scratch of device %d belongs to another context", c->device);
  if (set_device(c)) return MTPX_ERR_HIP;
  // The same launches as mtpx_moe_forward, with the device scratch standing in for the workspace for
  // this call (nothing is allocated: the context's own workspace is put back afterwards).  No part of
  // the scratch has to start at zero: the route writes every dispatch entry the expert kernels read.
  void* ws0 = c->ws;
  const size_t sz0 = c->ws_size;
  c->ws = c->scratch;
  c->ws_size = moe_scratch_bytes();
  ws_begin(c);
  rc = moe_enqueue(c, w, x, M, y, idx, wts, logits);
  c->ws = ws0;
  c->ws_size = sz0;
  c->ws_used = 0;
  const MoeDispatch* disp = c->last_disp;
  c->last_disp = nullptr;  // inside the shared scratch: mtpx_last_moe_bytes does not cover this call
  if (rc) return rc;
  if (n_unique) HIP_OK(hipMemcpyAsync(n_unique, &disp->n_unique, 4, hipMemcpyDeviceToDevice, c->stream));
  return MTPX_OK;
}

int mtpx_attn_prep(mtpx_ctx h, const uint16_t* qkv, int S, int QW, int HQ, int HK, int D, int rot,
                   const uint16_t* qnorm, const uint16_t* knorm, float eps, const uint16_t* cos_t,
                   const uint16_t* sin_t, int pos0, uint16_t* q, uint16_t* kc, uint16_t* vc, int64_t tmax) {
  Ctx* c = C(h);
  ARG(c && qkv && qnorm && knorm && cos_t && sin_t && q && kc && vc, "null argument");
  ARG(S >= 1 && S <= MAX_TOKENS, "S=%d", S);
  ARG(D >= 8 && D <= 256 && (D & (D - 1)) == 0, "head_dim=%d must be a power of two in 8..256", D);
  ARG(HK >= 1 && HQ % HK == 0, "heads %d / kv heads %d", HQ, HK);
  ARG(rot >= 2 && rot <= D && rot % 2 == 0, "rot=%d", rot);
  ARG(QW >= 2 * HQ * D + 2 * HK * D, "QW=%d too small", QW);
  ARG(pos0 >= 0 && pos0 + S <= tmax, "positions %d..%d beyond cache %lld", pos0, pos0 + S, (long long)tmax);
  if (set_device(c)) return MTPX_ERR_HIP;
  LAUNCH(c, "attn_prep", launch_attn_prep(qkv, S, QW, HQ, HK, D, rot, qnorm, knorm, eps, cos_t, sin_t, pos0, q, kc, vc, tmax,
                          c->stream));
  return MTPX_OK;
}

int mtpx_attn_verify(mtpx_ctx h, const uint16_t* q, int S, int HQ, int HK, int D, const uint16_t* kc,
                     const uint16_t* vc, int64_t tmax, int T, float scale, const uint16_t* qkv, int QW,
                     int gate_off, uint16_t* out, uint16_t* out_gated) {
  Ctx* c = C(h);
  ARG(c && q && kc && vc, "null argument");
  ARG(out || out_gated, "no output requested");
  ARG(!out_gated || qkv, "out_gated needs qkv");
  ARG(S >= 1 && S <= MAX_TOKENS && T >= S && T <= tmax && T <= 65536, "S=%d T=%d tmax=%lld (T <= 65536)", S, T,
      (long long)tmax);
  ARG(D >= 8 && D <= 256 && (D & (D - 1)) == 0, "head_dim=%d", D);
  ARG(HK >= 1 && HQ % HK == 0, "heads %d / kv heads %d", HQ, HK);
  ARG(D % 32 == 0, "head_dim=%d must be a multiple of 32", D);
  ARG(HQ / HK <= 32 && attn_partial_lds(HQ / HK, D) <= 160 * 1024, "GQA group of %d heads unsupported (<= 32)",
      HQ / HK);
  ARG(!out_gated || (gate_off >= 0 && gate_off + HQ * D <= QW), "gate columns outside qkv rows");
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t pf = attn_partial_floats(S, HQ, D, T);
  int rc = ws_reserve(c, al(pf * 4) + 256);
  if (rc) return rc;
  ws_begin(c);
  float* part = ws_take<float>(c, pf);
  LAUNCH(c, "attn_partial", launch_attn_partial(q, S, HQ, HK, D, kc, vc, tmax, T, scale, part, c->stream));
  LAUNCH(c, "attn_combine", launch_attn_combine(S, HQ, HK, D, T, part, qkv, QW, gate_off, out, out_gated, nullptr,
                                                c->stream));
  return MTPX_OK;
}

int mtpx_rmsnorm(mtpx_ctx h, const uint16_t* x, const uint16_t* resid, int M, int H, const uint16_t* w, float eps,
                 uint16_t* sum_out, uint16_t* y) {
  Ctx* c = C(h);
  ARG(c && x && w && y, "null argument");
  ARG(M >= 1 && H >= 1 && H <= 4096, "M=%d H=%d (H <= 4096)", M, H);
  if (set_device(c)) return MTPX_ERR_HIP;
  LAUNCH(c, "rmsnorm", launch_rmsnorm(x, resid, M, H, w, eps, sum_out, y, nullptr, c->stream));
  return MTPX_OK;
}

int mtpx_kv_new(mtpx_ctx h, int kv_heads, int head_dim, int64_t tmax, mtpx_kv* out) {
  Ctx* c = C(h);
  ARG(c && out && kv_heads >= 1 && head_dim >= 1 && tmax >= 1, "bad argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  Kv* kv = new Kv();
  kv->ctx = c;
  kv->heads = kv_heads;
  kv->dim = head_dim;
  kv->tmax = tmax;
  const size_t bytes = (size_t)kv_heads * tmax * head_dim * 2;
  if (hipMalloc(&kv->k, bytes) != hipSuccess || hipMalloc(&kv->v, bytes) != hipSuccess) {
    if (kv->k) hipFree(kv->k);
    delete kv;
    return fail(MTPX_ERR_OOM, "kv cache of 2 x %zu bytes", bytes);
  }
  hipMemsetAsync(kv->k, 0, bytes, c->stream);
  hipMemsetAsync(kv->v, 0, bytes, c->stream);
  out->ctx = kv;
  return MTPX_OK;
}

int mtpx_kv_free(mtpx_kv h) {
  Kv* kv = static_cast<Kv*>(h.ctx);
  if (!kv) return MTPX_OK;
  hipStreamSynchronize(kv->ctx->stream);
  hipFree(kv->k);
  hipFree(kv->v);
  delete kv;
  return MTPX_OK;
}

int mtpx_kv_offset(mtpx_kv h, int64_t* off) {
  Kv* kv = static_cast<Kv*>(h.ctx);
  ARG(kv && off, "null argument");
  *off = kv->offset;
  return MTPX_OK;
}

int mtpx_kv_set_offset(mtpx_kv h, int64_t off) {
  Kv* kv = static_cast<Kv*>(h.ctx);
  ARG(kv && off >= 0 && off <= kv->tmax, "offset %lld outside 0..tmax", (long long)off);
  kv->offset = off;
  return MTPX_OK;
}

int mtpx_kv_trim(mtpx_kv h, int64_t n, int64_t* trimmed) {
  Kv* kv = static_cast<Kv*>(h.ctx);
  ARG(kv && n >= 0, "bad argument");
  const int64_t t = n < kv->offset ? n : kv->offset;
  kv->offset -= t;
  if (trimmed) *trimmed = t;
  return MTPX_OK;
}

int mtpx_kv_buffers(mtpx_kv h, uint16_t** k, uint16_t** v, int64_t* tmax) {
  Kv* kv = static_cast<Kv*>(h.ctx);
  ARG(kv, "null kv");
  if (k) *k = kv->k;
  if (v) *v = kv->v;
  if (tmax) *tmax = kv->tmax;
  return MTPX_OK;
}

int mtpx_argmax_rows(mtpx_ctx h, const float* x, int rows, int64_t V, int32_t* out) {
  Ctx* c = C(h);
  ARG(c && x && out && rows >= 1 && V >= 1 && V < (int64_t)1 << 31, "bad argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t n = argmax_work_items(rows, V);
  int rc = ws_reserve(c, al(n * 4) * 2 + 256);
  if (rc) return rc;
  ws_begin(c);
  float* pv = ws_take<float>(c, n);
  int32_t* pi = ws_take<int32_t>(c, n);
  LAUNCH(c, "argmax_rows", launch_argmax_rows(x, rows, V, pv, pi, out, c->stream));
  return MTPX_OK;
}

int mtpx_accept_greedy(mtpx_ctx h, const float* logits, int k, int64_t V, const int32_t* drafts, int32_t kv_offset,
                       int32_t* out3) {
  Ctx* c = C(h);
  ARG(c && logits && out3 && (drafts || k == 0), "null argument");
  ARG(k >= 0 && k + 1 <= MAX_TOKENS && V >= 1 && V < (int64_t)1 << 31, "k=%d V=%lld", k, (long long)V);
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t n = argmax_work_items(k + 1, V);
  int rc = ws_reserve(c, al(n * 4) * 2 + 256);
  if (rc) return rc;
  ws_begin(c);
  float* pv = ws_take<float>(c, n);
  int32_t* pi = ws_take<int32_t>(c, n);
  LAUNCH(c, "accept_greedy", launch_accept_greedy(logits, k, V, drafts, kv_offset, pv, pi, out3, c->stream));
  return MTPX_OK;
}

int mtpx_accept_greedy_bf16(mtpx_ctx h, const uint16_t* logits, int k, int64_t V, const int32_t* drafts,
                            int32_t kv_offset, int32_t* out3, int32_t* argmax_out, int32_t* tokens_out) {
  Ctx* c = C(h);
  ARG(c && logits && out3 && (k == 0 || drafts), "null argument");
  ARG(k >= 0 && k + 1 <= MAX_TOKENS && V >= 1 && V < (int64_t)1 << 31, "k=%d V=%lld", k, (long long)V);
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t n = argmax_work_items(k + 1, V);
  int rc = ws_reserve(c, al(n * 4) * 2 + 256);
  if (rc) return rc;
  ws_begin(c);
  float* pv = ws_take<float>(c, n);
  int32_t* pi = ws_take<int32_t>(c, n);
  LAUNCH(c, "accept_greedy", launch_accept_greedy_bf16(reinterpret_cast<const bf16*>(logits), k, V, drafts, kv_offset,
                                                       pv, pi, out3, argmax_out, tokens_out, c->stream));
  return MTPX_OK;
}

static int top_two(Ctx* c, const float* x, const uint16_t* xb, int rows, int64_t V, int32_t* ids, float* vals) {
  ARG(c && (x || xb) && ids && vals, "null argument");
  ARG(rows >= 1 && V >= 2 && V < (int64_t)1 << 31, "rows=%d V=%lld", rows, (long long)V);
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t n = 4 * argmax_work_items(rows, V);
  int rc = ws_reserve(c, al(n * 4) + 256);
  if (rc) return rc;
  ws_begin(c);
  float* p2 = ws_take<float>(c, n);
  LAUNCH(c, "top_two", launch_top2(x, reinterpret_cast<const bf16*>(xb), rows, V, p2, ids, vals, c->stream));
  return MTPX_OK;
}

int mtpx_top_two(mtpx_ctx h, const float* logits, int rows, int64_t V, int32_t* ids, float* values) {
  return top_two(C(h), logits, nullptr, rows, V, ids, values);
}

int mtpx_top_two_bf16(mtpx_ctx h, const uint16_t* logits, int rows, int64_t V, int32_t* ids, float* values) {
  return top_two(C(h), nullptr, logits, rows, V, ids, values);
}

int mtpx_force_draft(mtpx_ctx h, int32_t* token, const int32_t* teacher, int64_t pos, float p, uint64_t seed) {
  Ctx* c = C(h);
  ARG(c && token && teacher && pos >= 0, "bad argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  LAUNCH(c, "force_draft", launch_force_draft(token, teacher, pos, p, seed, c->stream));
  return MTPX_OK;
}

int mtpx_accept_sample(mtpx_ctx h, const float* tlogits, const float* dlogits, int k, int64_t V,
                       const int32_t* drafts, float temperature, uint64_t seed, uint64_t offset, int32_t kv_offset,
                       int32_t* out3) {
  Ctx* c = C(h);
  ARG(c && tlogits && out3 && (k == 0 || drafts), "null argument");
  ARG(k >= 0 && k + 1 <= MAX_TOKENS && V >= 1 && V < (int64_t)1 << 31, "k=%d V=%lld", k, (long long)V);
  ARG(temperature > 0.0f && std::isfinite(temperature), "temperature must be > 0");
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t n = accept_sample_work_floats(k, V);
  int rc = ws_reserve(c, al(n * 4) + 256);
  if (rc) return rc;
  ws_begin(c);
  float* work = ws_take<float>(c, n);
  LAUNCH(c, "accept_sample", launch_accept_sample(tlogits, dlogits, k, V, drafts, temperature, seed, offset,
                                                  kv_offset, work, out3, c->stream));
  return MTPX_OK;
}

int mtpx_accept_sample_bf16(mtpx_ctx h, const uint16_t* tlogits, const uint16_t* dlogits, int k, int64_t V,
                            const int32_t* drafts, float temperature, uint64_t seed, uint64_t offset,
                            int32_t kv_offset, int32_t* out3, int32_t* tokens_out) {
  Ctx* c = C(h);
  ARG(c && tlogits && out3 && (k == 0 || drafts), "null argument");
  ARG(k >= 0 && k + 1 <= MAX_TOKENS && V >= 1 && V < (int64_t)1 << 31, "k=%d V=%lld", k, (long long)V);
  ARG(temperature > 0.0f && std::isfinite(temperature), "temperature must be > 0");
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t n = accept_sample_work_floats(k, V);
  int rc = ws_reserve(c, al(n * 4) + 256);
  if (rc) return rc;
  ws_begin(c);
  float* work = ws_take<float>(c, n);
  LAUNCH(c, "accept_sample",
         launch_accept_sample_bf16(reinterpret_cast<const bf16*>(tlogits), reinterpret_cast<const bf16*>(dlogits), k,
                                   V, drafts, temperature, seed, offset, kv_offset, work, out3, tokens_out,
                                   c->stream));
  return MTPX_OK;
}

// ---------------------------------------------------------------------------
// decoder layer

int mtpx_layer_new_random(mtpx_ctx h, const mtpx_layer_config* cfg, uint64_t seed, mtpx_layer* out) {
  Ctx* c = C(h);
  ARG(c && cfg && out, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  Layer* L = nullptr;
  int rc = layer_create(c, cfg, seed, &L);
  if (rc) return rc;
  out->ctx = L;
  return MTPX_OK;
}

int mtpx_layer_free(mtpx_layer h) {
  Layer* L = static_cast<Layer*>(h.ctx);
  if (!L) return MTPX_OK;
  for (void* p : L->allocs) hipFree(p);
  delete L;
  return MTPX_OK;
}

int mtpx_layer_weights_get(mtpx_layer h, mtpx_layer_weights* out) {
  Layer* L = static_cast<Layer*>(h.ctx);
  ARG(L && out, "null argument");
  *out = L->w;
  return MTPX_OK;
}

int mtpx_layer_forward(mtpx_ctx h, mtpx_layer lh, mtpx_kv kvh, const uint16_t* x, int M, uint16_t* y) {
  Ctx* c = C(h);
  Layer* L = static_cast<Layer*>(lh.ctx);
  Kv* kv = static_cast<Kv*>(kvh.ctx);
  ARG(c && L && kv && x && y, "null argument");
  const mtpx_layer_config& g = L->cfg;
  ARG(M >= 1 && M <= MAX_TOKENS, "M=%d", M);
  ARG(kv->heads == g.kv_heads && kv->dim == g.head_dim, "kv cache geometry does not match the layer");
  ARG(kv->offset + M <= kv->tmax && kv->offset + M <= g.max_positions, "cache full (offset %lld + %d)",
      (long long)kv->offset, M);
  ARG(kv->offset + M <= MTPX_INDEXER_BUDGET, "offset %lld + %d tokens is past the indexer budget %d",
      (long long)kv->offset, M, MTPX_INDEXER_BUDGET);
  int rc = moe_check(&L->w.moe, M);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  const int H = g.hidden, HQ = g.heads, D = g.head_dim;
  const int T = (int)(kv->offset + M);
  const int XB = (H > HQ * D ? H : HQ * D) / 32;
  const size_t need = moe_ws_bytes(&L->w.moe, M) + attn_ws_bytes(L, M, T) + al(2 * (size_t)M * H) * 4 +
                      al(4 * (size_t)M * XB * XP_DW) + al(4 * (size_t)M * (H / 32) * XP_DW) + 4096;
  if ((rc = ws_reserve(c, need))) return rc;
  ws_begin(c);
  uint16_t* h1 = ws_take<uint16_t>(c, (size_t)M * H);
  uint16_t* o = ws_take<uint16_t>(c, (size_t)M * H);
  uint16_t* s = ws_take<uint16_t>(c, (size_t)M * H);
  uint16_t* h2 = ws_take<uint16_t>(c, (size_t)M * H);
  uint32_t* xp = ws_take<uint32_t>(c, (size_t)M * XB * XP_DW);
  uint32_t* xp2 = ws_take<uint32_t>(c, (size_t)M * (H / 32) * XP_DW);
  hipStream_t st = c->stream;
  LAUNCH(c, "rmsnorm", launch_rmsnorm(x, nullptr, M, H, L->w.attn_norm, g.eps, nullptr, h1, xp, st));
  if ((rc = attn_enqueue(c, L, kv, xp, M, o))) return rc;
  LAUNCH(c, "rmsnorm", launch_rmsnorm(x, o, M, H, L->w.post_norm, g.eps, s, h2, xp2, st));
  if ((rc = moe_enqueue(c, &L->w.moe, h2, M, h1, nullptr, nullptr, nullptr, s, y, xp2))) return rc;
  kv->offset += M;
  return MTPX_OK;
}


int mtpx_gdn_new_random(mtpx_ctx h, const mtpx_gdn_config* cfg, uint64_t seed, mtpx_gdn* out) {
  Ctx* c = C(h);
  ARG(c && cfg && out, "null argument");
  int rc = gdn_check(cfg);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  GdnLayer* L = new GdnLayer();
  L->cfg = *cfg;
  RandInit ri{c, seed, cfg->group_size, &L->allocs};
  gdn_random(ri, *cfg, seed, &L->w);
  if ((rc = ri.finish("gdn"))) {
    for (void* p : L->allocs) hipFree(p);
    delete L;
    return rc;
  }
  out->ctx = L;
  return MTPX_OK;
}

int mtpx_gdn_free(mtpx_gdn gh) {
  GdnLayer* L = static_cast<GdnLayer*>(gh.ctx);
  if (!L) return MTPX_OK;
  for (void* p : L->allocs) hipFree(p);
  delete L;
  return MTPX_OK;
}

int mtpx_gdn_weights_get(mtpx_gdn gh, mtpx_gdn_weights* out) {
  GdnLayer* L = static_cast<GdnLayer*>(gh.ctx);
  ARG(L && out, "null argument");
  *out = L->w;
  return MTPX_OK;
}

int mtpx_gdn_state_new(mtpx_ctx h, const mtpx_gdn_config* cfg, mtpx_gdn_state* out) {
  Ctx* c = C(h);
  ARG(c && cfg && out, "null argument");
  int rc = gdn_check(cfg);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  const GdnGeom g = gdn_geom(*cfg);
  GdnState* st = new GdnState();
  st->cfg = *cfg;
  bool ok = true;
  auto take = [&](size_t bytes) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
      ok = false;
      return nullptr;
    }
    st->allocs.push_back(p);
    return p;
  };
  for (int s = 0; s < 2; ++s) {
    st->conv[s] = (uint16_t*)take(2 * (size_t)(g.kc - 1) * g.cd);
    st->win[s] = (uint16_t*)take(2 * (size_t)MAX_TOKENS * g.cd);
    st->key[s] = (uint16_t*)take(2 * (size_t)MAX_TOKENS * g.hk * 128);
    st->delta[s] = (float*)take(4 * (size_t)MAX_TOKENS * g.hv * 128);
    st->decay[s] = (float*)take(4 * (size_t)MAX_TOKENS * g.hv);
  }
  st->ssm = (float*)take(4 * (size_t)g.hv * 128 * 128);
  st->tickets = (uint32_t*)take(4 * (size_t)g.hv);
  st->ypub = (float*)take(4 * (size_t)MAX_TOKENS * g.hv * 128);
  if (ok) {
    if (hipMemsetAsync(st->tickets, 0, 4 * (size_t)g.hv, c->stream) != hipSuccess) ok = false;
    for (int s = 0; s < 2; ++s)
      if (hipMemsetAsync(st->conv[s], 0, 2 * (size_t)(g.kc - 1) * g.cd, c->stream) != hipSuccess) ok = false;
    if (hipMemsetAsync(st->ssm, 0, 4 * (size_t)g.hv * 128 * 128, c->stream) != hipSuccess) ok = false;
    if (hipStreamSynchronize(c->stream) != hipSuccess) ok = false;
  }
  if (!ok) {
    for (void* p : st->allocs) hipFree(p);
    delete st;
    return fail(MTPX_ERR_OOM, "gdn state allocation failed");
  }
  out->ctx = st;
  return MTPX_OK;
}

int mtpx_gdn_state_free(mtpx_gdn_state sh) {
  GdnState* st = static_cast<GdnState*>(sh.ctx);
  if (!st) return MTPX_OK;
  for (void* p : st->allocs) hipFree(p);
  delete st;
  return MTPX_OK;
}

int mtpx_gdn_state_load(mtpx_ctx h, mtpx_gdn_state sh, const uint16_t* conv, const float* ssm) {
  Ctx* c = C(h);
  GdnState* st = static_cast<GdnState*>(sh.ctx);
  ARG(c && st && conv && ssm, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  const GdnGeom g = gdn_geom(st->cfg);
  HIP_OK(hipMemcpyAsync(st->conv[st->cur], conv, 2 * (size_t)(g.kc - 1) * g.cd, hipMemcpyDeviceToDevice, c->stream));
  HIP_OK(hipMemcpyAsync(st->ssm, ssm, 4 * (size_t)g.hv * 128 * 128, hipMemcpyDeviceToDevice, c->stream));
  st->window = 0;
  st->committed = 0;
  return MTPX_OK;
}

int mtpx_gdn_state_store(mtpx_ctx h, mtpx_gdn_state sh, uint16_t* conv, float* ssm) {
  Ctx* c = C(h);
  GdnState* st = static_cast<GdnState*>(sh.ctx);
  ARG(c && st && conv && ssm, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  const GdnArgs a = gdn_args(st, nullptr, nullptr, 0, nullptr, nullptr);
  LAUNCH(c, "gdn_replay", launch_gdn_replay(a, ssm, reinterpret_cast<bf16*>(conv), c->stream));
  return MTPX_OK;
}

int mtpx_gdn_commit(mtpx_gdn_state sh, int n) {
  GdnState* st = static_cast<GdnState*>(sh.ctx);
  ARG(st, "null state");
  if (n < 0 || n > st->window)
    return fail(MTPX_ERR_STATE, "commit of %d positions; the last window has %d", n, st->window);
  st->committed = n;
  return MTPX_OK;
}

int mtpx_gdn_state_info(mtpx_gdn_state sh, int* window, int* committed) {
  GdnState* st = static_cast<GdnState*>(sh.ctx);
  ARG(st, "null state");
  if (window) *window = st->window;
  if (committed) *committed = st->committed;
  return MTPX_OK;
}

int mtpx_gdn_core(mtpx_ctx h, mtpx_gdn gh, mtpx_gdn_state sh, const uint16_t* proj, int S, uint16_t* gated) {
  Ctx* c = C(h);
  GdnLayer* L = static_cast<GdnLayer*>(gh.ctx);
  GdnState* st = static_cast<GdnState*>(sh.ctx);
  ARG(c && L && st && proj && gated, "null argument");
  ARG(S >= 1 && S <= MAX_TOKENS, "S=%d", S);
  ARG(gdn_same(L->cfg, st->cfg), "state geometry does not match the layer");
  if (set_device(c)) return MTPX_ERR_HIP;
  return gdn_enqueue(c, L, st, proj, S, gated, nullptr);
}

int mtpx_gdn_forward(mtpx_ctx h, mtpx_gdn gh, mtpx_gdn_state sh, const uint16_t* x, int S, uint16_t* y,
                     uint16_t* gated) {
  Ctx* c = C(h);
  GdnLayer* L = static_cast<GdnLayer*>(gh.ctx);
  GdnState* st = static_cast<GdnState*>(sh.ctx);
  ARG(c && L && st && x && y, "null argument");
  ARG(S >= 1 && S <= MAX_TOKENS, "S=%d", S);
  ARG(gdn_same(L->cfg, st->cfg), "state geometry does not match the layer");
  if (set_device(c)) return MTPX_ERR_HIP;
  const mtpx_gdn_config& cfg = L->cfg;
  const GdnGeom g = gdn_geom(cfg);
  const int H = cfg.hidden, VD = g.hv * 128, gs = cfg.group_size;
  const size_t xin = (size_t)S * (H / 32) * XP_DW, xout = (size_t)S * (VD / 32) * XP_DW;
  int rc = ws_reserve(c, al(xin * 4) + al(2 * (size_t)S * g.pw) + al(xout * 4) + 1024);
  if (rc) return rc;
  ws_begin(c);
  uint32_t* xp = ws_take<uint32_t>(c, xin);
  uint16_t* proj = ws_take<uint16_t>(c, (size_t)S * g.pw);
  uint32_t* xp2 = ws_take<uint32_t>(c, xout);
  const mtpx_q4& ip = L->w.in_proj;
  const mtpx_q4& op = L->w.out_proj;
  LAUNCH(c, "xprep", launch_xprep(reinterpret_cast<const bf16*>(x), S, H, xp, c->stream));
  LAUNCH(c, "qmv_gdn_in", launch_qmv(ip.w, reinterpret_cast<const bf16*>(ip.s), reinterpret_cast<const bf16*>(ip.b), ip.sb,
                                      g.pw, H, gs, xp, S, reinterpret_cast<bf16*>(proj), nullptr, c->stream));
  if ((rc = gdn_enqueue(c, L, st, proj, S, gated, xp2))) return rc;
  LAUNCH(c, "qmv_gdn_out", launch_qmv(op.w, reinterpret_cast<const bf16*>(op.s), reinterpret_cast<const bf16*>(op.b),
                                       op.sb, H, VD, gs, xp2, S, reinterpret_cast<bf16*>(y), nullptr, c->stream));
  return MTPX_OK;
}


int mtpx_ple_new_random(mtpx_ctx h, const mtpx_ple_config* cfg, uint64_t seed, mtpx_ple* out) {
  Ctx* c = C(h);
  ARG(c && cfg && out, "null argument");
  int rc = ple_check(cfg);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  PleLayer* L = new PleLayer();
  L->cfg = *cfg;
  if ((rc = ple_random(c, *cfg, seed, L))) {
    for (void* p : L->allocs) hipFree(p);
    delete L;
    return rc;
  }
  out->ctx = L;
  return MTPX_OK;
}

int mtpx_ple_free(mtpx_ple ph) {
  PleLayer* L = static_cast<PleLayer*>(ph.ctx);
  if (!L) return MTPX_OK;
  for (void* p : L->allocs) hipFree(p);
  delete L;
  return MTPX_OK;
}

int mtpx_ple_weights_get(mtpx_ple ph, mtpx_ple_weights* out) {
  PleLayer* L = static_cast<PleLayer*>(ph.ctx);
  ARG(L && out, "null argument");
  *out = L->w;
  return MTPX_OK;
}

int mtpx_ple_state_new(mtpx_ctx h, const mtpx_ple_config* cfg, mtpx_ple_state* out) {
  Ctx* c = C(h);
  ARG(c && cfg && out, "null argument");
  int rc = ple_check(cfg);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  PleState* st = nullptr;
  if ((rc = ple_state_create(c, *cfg, &st))) return rc;
  out->ctx = st;
  return MTPX_OK;
}

int mtpx_ple_state_free(mtpx_ple_state sh) {
  PleState* st = static_cast<PleState*>(sh.ctx);
  if (st) ple_state_release(st);
  return MTPX_OK;
}

int mtpx_ple_state_load(mtpx_ctx h, mtpx_ple_state sh, const uint16_t* conv, const int32_t* context) {
  Ctx* c = C(h);
  PleState* st = static_cast<PleState*>(sh.ctx);
  ARG(c && st && conv && context, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  const PleGeom pg = ple_geom(st->cfg);
  if (pg.nb > 0)
    HIP_OK(hipMemcpyAsync(st->conv[st->cur], conv, 2 * (size_t)pg.nb * pg.W, hipMemcpyDeviceToDevice, c->stream));
  HIP_OK(hipMemcpyAsync(st->ctx[st->cur], context, 4 * (size_t)pg.ctx_len, hipMemcpyDeviceToDevice, c->stream));
  st->window = 0;
  st->committed = 0;
  return MTPX_OK;
}

// The committed state: rows P.. of the base, then the window's first P rows (and the same for the context).
int mtpx_ple_state_store(mtpx_ctx h, mtpx_ple_state sh, uint16_t* conv, int32_t* context) {
  Ctx* c = C(h);
  PleState* st = static_cast<PleState*>(sh.ctx);
  ARG(c && st && conv && context, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  const PleGeom pg = ple_geom(st->cfg);
  const int P = st->committed, cs = st->cur;
  const size_t row = 2 * (size_t)pg.W;
  const int keep = pg.nb - P > 0 ? pg.nb - P : 0;  // base rows that stay
  if (keep > 0) HIP_OK(hipMemcpyAsync(conv, st->conv[cs] + (size_t)P * pg.W, keep * row, hipMemcpyDeviceToDevice, c->stream));
  if (pg.nb - keep > 0)
    HIP_OK(hipMemcpyAsync(conv + (size_t)keep * pg.W, st->win[cs] + (size_t)(P - (pg.nb - keep)) * pg.W,
                          (pg.nb - keep) * row, hipMemcpyDeviceToDevice, c->stream));
  const int ck = pg.ctx_len - P > 0 ? pg.ctx_len - P : 0;
  if (ck > 0) HIP_OK(hipMemcpyAsync(context, st->ctx[cs] + P, 4 * (size_t)ck, hipMemcpyDeviceToDevice, c->stream));
  if (pg.ctx_len - ck > 0)
    HIP_OK(hipMemcpyAsync(context + ck, st->ids[cs] + (P - (pg.ctx_len - ck)), 4 * (size_t)(pg.ctx_len - ck),
                          hipMemcpyDeviceToDevice, c->stream));
  return MTPX_OK;
}

int mtpx_ple_commit(mtpx_ple_state sh, int n) {
  PleState* st = static_cast<PleState*>(sh.ctx);
  ARG(st, "null state");
  if (n < 0 || n > st->window)
    return fail(MTPX_ERR_STATE, "commit of %d positions; the last window has %d", n, st->window);
  st->committed = n;
  return MTPX_OK;
}

int mtpx_ple_state_info(mtpx_ple_state sh, int* window, int* committed) {
  PleState* st = static_cast<PleState*>(sh.ctx);
  ARG(st, "null state");
  if (window) *window = st->window;
  if (committed) *committed = st->committed;
  return MTPX_OK;
}

int mtpx_ngram_row_ids(mtpx_ctx h, mtpx_ple ph, const int32_t* history, int S, int32_t* out) {
  Ctx* c = C(h);
  PleLayer* L = static_cast<PleLayer*>(ph.ctx);
  ARG(c && L && history && out, "null argument");
  ARG(S >= 1 && S <= MAX_TOKENS, "S=%d", S);
  if (set_device(c)) return MTPX_ERR_HIP;
  const PleGeom pg = ple_geom(L->cfg);
  PleRowArgs a = ple_row_args(L, history + pg.ctx_len, S);
  a.ctx_cur = history;
  a.ids_prev = history;  // P = 0: not read
  a.row_ids = out;
  LAUNCH(c, "ngram_row_ids", launch_ple_rows(a, c->stream));
  return MTPX_OK;
}

int mtpx_ple_forward(mtpx_ctx h, mtpx_ple ph, mtpx_ple_state sh, const int32_t* ids, int S, const uint16_t* stream,
                     uint16_t* out, uint16_t* sum, uint16_t* embedded) {
  Ctx* c = C(h);
  PleLayer* L = static_cast<PleLayer*>(ph.ctx);
  PleState* st = static_cast<PleState*>(sh.ctx);
  ARG(c && L && st && ids && stream, "null argument");
  ARG(out || sum, "neither out nor sum given");
  ARG(S >= 1 && S <= MAX_TOKENS, "S=%d", S);
  ARG(ple_same(L->cfg, st->cfg), "state geometry does not match the block");
  if (set_device(c)) return MTPX_ERR_HIP;
  int rc = ws_reserve(c, ple_ws_bytes(L->cfg, S));
  if (rc) return rc;
  ws_begin(c);
  return ple_enqueue(c, L, st, ids, S, stream, out, sum, embedded);
}

int mtpx_target_new_random(mtpx_ctx h, const mtpx_target_config* cfg, uint64_t seed, mtpx_target* out) {
  Ctx* c = C(h);
  ARG(c && cfg && out, "null argument");
  int rc = target_check(cfg);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  const mtpx_layer_config& lc = cfg->layer;
  const mtpx_gdn_config gc = target_gdn_cfg(*cfg);
  Target* t = new Target();
  t->cfg = *cfg;
  t->layers.resize(cfg->num_layers);
  RandInit ri{c, seed, lc.group_size, &t->allocs};
  ri.qmat(cfg->vocab, lc.hidden, &t->embed);
  ri.qmat(cfg->vocab, lc.hidden, &t->lm_head);
  hc_random(ri, lc.hidden, cfg->hc, cfg->lowrank, false, &t->final_hc);
  for (int i = 0; i < cfg->num_layers && rc == MTPX_OK && ri.ok; ++i) {
    TargetLayer& L = t->layers[i];
    const uint64_t ls = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(i + 1);
    hc_random(ri, lc.hidden, cfg->hc, cfg->lowrank, true, &L.attn_hc);
    hc_random(ri, lc.hidden, cfg->hc, cfg->lowrank, true, &L.mlp_hc);
    if ((i + 1) % cfg->full_attention_interval == 0) {
      L.kind = MTPX_LAYER_ATTENTION;
      rc = layer_create(c, &lc, ls, &L.attn);
      if (rc == MTPX_OK) L.moe = L.attn->w.moe;
    } else {
      L.kind = MTPX_LAYER_GDN;
      L.gdn = new GdnLayer();
      L.gdn->cfg = gc;
      RandInit gi{c, ls, lc.group_size, &L.gdn->allocs};
      gdn_random(gi, gc, ls, &L.gdn->w);
      moe_random(gi, &lc, &L.moe);
      rc = gi.finish("target gdn layer");
    }
  }
  if (rc == MTPX_OK && ri.ok && cfg->ple_layer >= 0) {
    t->ple = new PleLayer();
    t->ple->cfg = cfg->ple;
    rc = ple_random(c, cfg->ple, seed ^ 0x5be0cd19137e2179ull, t->ple);
  }
  const int rc2 = ri.finish("target");
  if (rc || rc2) {
    target_release(t);
    return rc ? rc : rc2;
  }
  out->ctx = t;
  return MTPX_OK;
}

namespace {

// Adoption of caller-owned weights (MLX layout): every q4 matrix and dense vector is used in place;
// the library adds only packed scale/bias rows (when asked and the caller gave none), RoPE tables
// (when the caller gave none) and the n-gram table's device hash parameters.
struct Adopt {
  Ctx* c;
  int gs;
  bool pack;
  std::vector<void*>* allocs;
  bool ok = true;
  std::string missing;

  bool need(const void* p, const char* what) {
    if (!p && missing.empty()) missing = what;
    return p != nullptr;
  }
  void sb_rows(int64_t rows, int K, const uint16_t* s, const uint16_t* b, const uint32_t** sb) {
    if (*sb || !pack || !s || !b) return;
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)rows * sb_row_len(K, gs) * 4) != hipSuccess) {
      ok = false;
      return;
    }
    allocs->push_back(p);
    (void)hipGetLastError();  // only this launch's error counts
    if (launch_pack_sb(reinterpret_cast<const bf16*>(s), reinterpret_cast<const bf16*>(b), rows, K, gs,
                       static_cast<uint32_t*>(p), c->stream) != hipSuccess)
      ok = false;
    *sb = static_cast<uint32_t*>(p);
  }
  void q4(mtpx_q4* q, int64_t rows, int K, const char* what, bool optional = false) {
    if (optional && !q->w) return;
    if (need(q->w, what) & need(q->s, what) & need(q->b, what)) sb_rows(rows, K, q->s, q->b, &q->sb);
  }
  void moe(mtpx_moe_weights* m, const mtpx_layer_config& lc) {
    const int H = lc.hidden, E = lc.experts, F = lc.expert_width;
    m->hidden = H;
    m->experts = E;
    m->top_k = lc.top_k;
    m->expert_width = F;
    m->group_size = lc.group_size;
    need(m->router, "moe router");
    if (m->shared_gate_w) {  // the q4 gate row: its packed pair row when the caller gave none
      if (need(m->shared_gate_s, "moe shared gate scales") & need(m->shared_gate_b, "moe shared gate biases"))
        sb_rows(1, H, m->shared_gate_s, m->shared_gate_b, &m->shared_gate_sb);
    } else {
      need(m->shared_gate, "moe shared gate");
    }
    const int nsb = !!m->gate_sb + !!m->up_sb + !!m->down_sb + !!m->sh_gate_sb + !!m->sh_up_sb + !!m->sh_down_sb;
    if (nsb != 0 && nsb != 6 && missing.empty()) missing = "moe packed scale/bias rows (all six or none)";
    struct {
      const uint32_t* w; const uint16_t* s; const uint16_t* b; const uint32_t** sb; int64_t rows; int K;
    } mats[6] = {{m->gate_w, m->gate_s, m->gate_b, &m->gate_sb, (int64_t)E * F, H},
                 {m->up_w, m->up_s, m->up_b, &m->up_sb, (int64_t)E * F, H},
                 {m->down_w, m->down_s, m->down_b, &m->down_sb, (int64_t)E * H, F},
                 {m->sh_gate_w, m->sh_gate_s, m->sh_gate_b, &m->sh_gate_sb, F, H},
                 {m->sh_up_w, m->sh_up_s, m->sh_up_b, &m->sh_up_sb, F, H},
                 {m->sh_down_w, m->sh_down_s, m->sh_down_b, &m->sh_down_sb, H, F}};
    for (auto& x : mats)
      if (need(x.w, "moe expert matrix") & need(x.s, "moe expert scales") & need(x.b, "moe expert biases") &&
          nsb == 0)
        sb_rows(x.rows, x.K, x.s, x.b, x.sb);
  }
  void hc(mtpx_hc_weights* m, int H, int hc_, int LW, bool inject) {
    const int W = hc_ * H;
    need(m->norm_scale, "hyper-connection norm scale");
    q4(&m->down, LW, W, "hyper-connection down");
    if (inject) q4(&m->inject, hc_, W, "hyper-connection inject");
    q4(&m->up, W, LW, "hyper-connection up");
  }
  int finish(const char* what) {
    if (!missing.empty()) return fail(MTPX_ERR_ARG, "%s: missing %s", what, missing.c_str());
    if (!ok || hipStreamSynchronize(c->stream) != hipSuccess) return fail(MTPX_ERR_OOM, "%s: adoption failed", what);
    return MTPX_OK;
  }
};

}  // namespace

int mtpx_target_adopt(mtpx_ctx h, const mtpx_target_config* cfg, const mtpx_target_weights* tw,
                      const mtpx_target_layer_weights* layers, int pack_sb, mtpx_target* out) {
  Ctx* c = C(h);
  ARG(c && cfg && tw && layers && out, "null argument");
  int rc = target_check(cfg);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  const mtpx_layer_config& lc = cfg->layer;
  const int H = lc.hidden;
  for (int i = 0; i < cfg->num_layers; ++i) {
    const int want = (i + 1) % cfg->full_attention_interval == 0 ? MTPX_LAYER_ATTENTION : MTPX_LAYER_GDN;
    ARG(layers[i].kind == want, "layer %d: kind %d, the schedule has %d", i, layers[i].kind, want);
  }
  Target* t = new Target();
  t->cfg = *cfg;
  t->layers.resize(cfg->num_layers);
  Adopt ad{c, lc.group_size, pack_sb != 0, &t->allocs};
  t->embed = tw->embed;
  t->lm_head = tw->lm_head;
  t->final_hc = tw->final_hc;
  ad.q4(&t->embed, cfg->vocab, H, "embed");
  ad.q4(&t->lm_head, cfg->vocab, H, "lm_head");
  ad.hc(&t->final_hc, H, cfg->hc, cfg->lowrank, false);
  const mtpx_gdn_config gc = target_gdn_cfg(*cfg);
  const GdnGeom gg = gdn_geom(gc);
  for (int i = 0; i < cfg->num_layers; ++i) {
    TargetLayer& L = t->layers[i];
    const mtpx_target_layer_weights& in = layers[i];
    L.kind = in.kind;
    L.attn_hc = in.attn_hc;
    L.mlp_hc = in.mlp_hc;
    ad.hc(&L.attn_hc, H, cfg->hc, cfg->lowrank, true);
    ad.hc(&L.mlp_hc, H, cfg->hc, cfg->lowrank, true);
    if (in.kind == MTPX_LAYER_ATTENTION) {
      L.attn = new Layer();
      L.attn->cfg = lc;
      L.attn->w = in.attn;
      L.attn->QW = 2 * lc.heads * lc.head_dim + 2 * lc.kv_heads * lc.head_dim + lc.index_dim;
      mtpx_layer_weights& w = L.attn->w;
      w.qkv_rows = L.attn->QW;
      ad.need(w.q_norm, "attention q_norm");
      ad.need(w.k_norm, "attention k_norm");
      Adopt la{c, lc.group_size, pack_sb != 0, &L.attn->allocs};
      mtpx_q4 qkv{w.qkv_w, w.qkv_s, w.qkv_b, w.qkv_sb}, o{w.o_w, w.o_s, w.o_b, w.o_sb};
      la.q4(&qkv, L.attn->QW, H, "attention qkv");
      la.q4(&o, H, lc.heads * lc.head_dim, "attention o_proj");
      w.qkv_sb = qkv.sb;
      w.o_sb = o.sb;
      la.moe(&w.moe, lc);
      if ((!w.rope_cos || !w.rope_sin) && !rope_tables(c, &lc, &L.attn->allocs, &w.rope_cos, &w.rope_sin))
        la.ok = false;
      if ((rc = la.finish("target attention layer"))) break;
      L.moe = w.moe;
    } else {
      L.gdn = new GdnLayer();
      L.gdn->cfg = gc;
      L.gdn->w = in.gdn;
      mtpx_gdn_weights& g = L.gdn->w;
      Adopt la{c, lc.group_size, pack_sb != 0, &L.gdn->allocs};
      la.q4(&g.in_proj, gg.pw, H, "gdn in_proj");
      la.q4(&g.out_proj, H, gg.hv * 128, "gdn out_proj");
      la.need(g.conv_w, "gdn conv_w");
      la.need(g.neg_exp_alog, "gdn neg_exp_alog");
      la.need(g.dt_bias, "gdn dt_bias");
      la.need(g.norm_w, "gdn norm_w");
      L.moe = in.attn.moe;  // a GDN layer's MoE travels in the attention slot
      la.moe(&L.moe, lc);
      if ((rc = la.finish("target gdn layer"))) break;
    }
  }
  if (rc == MTPX_OK && cfg->ple_layer >= 0) {
    t->ple = new PleLayer();
    t->ple->cfg = cfg->ple;
    t->ple->w = layers[cfg->ple_layer].ple;
    mtpx_ple_weights& w = t->ple->w;
    Adopt la{c, cfg->ple.group_size, pack_sb != 0, &t->ple->allocs};
    const PleGeom pg = ple_geom(cfg->ple);
    la.q4(&w.key_proj, pg.W, cfg->ple.embed_dim, "ple key_proj");
    la.q4(&w.value_proj, H, cfg->ple.embed_dim, "ple value_proj");
    la.need(w.norm_key, "ple norm_key");
    la.need(w.norm_query, "ple norm_query");
    la.need(w.norm_conv, "ple norm_conv");
    la.need(w.conv_w, "ple conv_w");
    la.need(w.table.w, "ngram table");
    la.need(w.table.s, "ngram table scales");
    la.need(w.table.b, "ngram table biases");
    // the head vocabularies and offsets follow from the config; the multipliers are the caller's
    mtpx_ngram_table expect;
    const int64_t rows = ngram_heads(cfg->ple, &expect);
    // a checkpoint pads the table to whole shards: rows past the heads' sum are never addressed
    if (w.table.rows < rows && la.missing.empty()) la.missing = "an n-gram table of at least the config's row count";
    for (int hh = 0; hh < pg.nh; ++hh) {
      w.table.vocab[hh] = expect.vocab[hh];
      w.table.offset[hh] = expect.offset[hh];
    }
    std::vector<int64_t> hv(cfg->ple.ngram_size + 2 * (size_t)pg.nh);
    for (int p = 0; p < cfg->ple.ngram_size; ++p) hv[p] = w.table.multiplier[p];
    for (int hh = 0; hh < pg.nh; ++hh) {
      hv[cfg->ple.ngram_size + hh] = w.table.vocab[hh];
      hv[cfg->ple.ngram_size + pg.nh + hh] = w.table.offset[hh];
    }
    void* hp = nullptr;
    if (hipMalloc(&hp, 8 * hv.size()) != hipSuccess ||
        hipMemcpy(hp, hv.data(), 8 * hv.size(), hipMemcpyHostToDevice) != hipSuccess)
      la.ok = false;
    if (hp) t->ple->allocs.push_back(hp);
    t->ple->hash = static_cast<int64_t*>(hp);
    rc = la.finish("target ple block");
  }
  const int rc2 = rc ? rc : ad.finish("target");
  if (rc2) {
    target_release(t);
    return rc2;
  }
  out->ctx = t;
  return MTPX_OK;
}

int mtpx_target_free(mtpx_target th) {
  Target* t = static_cast<Target*>(th.ctx);
  if (t) target_release(t);
  return MTPX_OK;
}

int mtpx_target_weights_get(mtpx_target th, mtpx_target_weights* out) {
  Target* t = static_cast<Target*>(th.ctx);
  ARG(t && out, "null argument");
  out->embed = t->embed;
  out->final_hc = t->final_hc;
  out->lm_head = t->lm_head;
  return MTPX_OK;
}

int mtpx_target_layer_weights_get(mtpx_target th, int i, mtpx_target_layer_weights* out) {
  Target* t = static_cast<Target*>(th.ctx);
  ARG(t && out, "null argument");
  ARG(i >= 0 && i < (int)t->layers.size(), "layer %d of %d", i, (int)t->layers.size());
  const TargetLayer& L = t->layers[i];
  memset(out, 0, sizeof(*out));
  out->kind = L.kind;
  if (L.attn) out->attn = L.attn->w;
  out->attn.moe = L.moe;
  if (L.gdn) out->gdn = L.gdn->w;
  out->attn_hc = L.attn_hc;
  out->mlp_hc = L.mlp_hc;
  if (i == t->cfg.ple_layer && t->ple) out->ple = t->ple->w;
  return MTPX_OK;
}

int mtpx_target_state_new(mtpx_ctx h, mtpx_target th, mtpx_target_state* out) {
  Ctx* c = C(h);
  Target* t = static_cast<Target*>(th.ctx);
  ARG(c && t && out, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  const mtpx_layer_config& lc = t->cfg.layer;
  const mtpx_gdn_config gc = target_gdn_cfg(t->cfg);
  TargetState* s = new TargetState();
  s->t = t;
  const int n = (int)t->layers.size();
  s->kv.assign(n, nullptr);
  s->gdn.assign(n, nullptr);
  int rc = MTPX_OK;
  if (hipMalloc((void**)&s->moe_unique, 4 * (size_t)n) != hipSuccess) {
    s->moe_unique = nullptr;
    rc = fail(MTPX_ERR_OOM, "target state");
  } else if (hipMemsetAsync(s->moe_unique, 0, 4 * (size_t)n, c->stream) != hipSuccess) {
    rc = fail(MTPX_ERR_HIP, "target state");
  }
  for (int i = 0; i < n && rc == MTPX_OK; ++i) {
    if (t->layers[i].kind == MTPX_LAYER_ATTENTION) {
      mtpx_kv k{nullptr};
      rc = mtpx_kv_new(h, lc.kv_heads, lc.head_dim, lc.max_positions, &k);
      s->kv[i] = static_cast<Kv*>(k.ctx);
    } else {
      mtpx_gdn_state g{nullptr};
      rc = mtpx_gdn_state_new(h, &gc, &g);
      s->gdn[i] = static_cast<GdnState*>(g.ctx);
    }
  }
  if (rc == MTPX_OK && t->ple) rc = ple_state_create(c, t->cfg.ple, &s->ple);
  if (rc) {
    target_state_release(s);
    return rc;
  }
  out->ctx = s;
  return MTPX_OK;
}

int mtpx_target_state_free(mtpx_target_state sh) {
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  if (!s) return MTPX_OK;
  for (Kv* kv : s->kv)
    if (kv) hipStreamSynchronize(kv->ctx->stream);
  target_state_release(s);
  return MTPX_OK;
}

int mtpx_target_state_kv(mtpx_target_state sh, int i, mtpx_kv* out) {
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(s && out, "null argument");
  ARG(i >= 0 && i < (int)s->kv.size() && s->kv[i], "layer %d is not an attention layer", i);
  out->ctx = s->kv[i];
  return MTPX_OK;
}

int mtpx_target_state_gdn(mtpx_target_state sh, int i, mtpx_gdn_state* out) {
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(s && out, "null argument");
  ARG(i >= 0 && i < (int)s->gdn.size() && s->gdn[i], "layer %d is not a GDN layer", i);
  out->ctx = s->gdn[i];
  return MTPX_OK;
}

int mtpx_target_state_ple(mtpx_target_state sh, mtpx_ple_state* out) {
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(s && out, "null argument");
  ARG(s->ple, "the target has no PLE layer");
  out->ctx = s->ple;
  return MTPX_OK;
}

int mtpx_target_state_set_offset(mtpx_target_state sh, int64_t offset) {
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(s, "null state");
  ARG(offset >= 0 && offset <= s->t->cfg.layer.max_positions, "offset %lld", (long long)offset);
  s->offset = offset;
  s->window = 0;
  for (Kv* kv : s->kv)
    if (kv) kv->offset = offset;
  return MTPX_OK;
}

int mtpx_target_state_reset(mtpx_ctx h, mtpx_target_state sh) {
  Ctx* c = C(h);
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(c && s, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  int rc;
  for (GdnState* g : s->gdn)
    if (g && (rc = gdn_state_zero(c, g))) return rc;
  if (s->ple && (rc = ple_state_zero(c, s->ple))) return rc;
  s->offset = 0;
  s->window = 0;
  for (Kv* kv : s->kv)
    if (kv) kv->offset = 0;
  s->broken = false;
  return MTPX_OK;
}

int mtpx_target_state_info(mtpx_target_state sh, int64_t* offset, int* window) {
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(s, "null state");
  if (offset) *offset = s->offset;
  if (window) *window = s->window;
  return MTPX_OK;
}

int mtpx_target_moe_unique(mtpx_ctx h, mtpx_target_state sh, int32_t* out) {
  Ctx* c = C(h);
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(c && s && out, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  HIP_OK(hipMemcpyAsync(out, s->moe_unique, 4 * s->kv.size(), hipMemcpyDeviceToHost, c->stream));
  HIP_OK(hipStreamSynchronize(c->stream));
  return MTPX_OK;
}

int mtpx_target_commit(mtpx_target_state sh, int n) {
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(s, "null state");
  if (s->broken) return fail(MTPX_ERR_STATE, "state left inconsistent by a failed verify; reset it first");
  if (n < 0 || n > s->window)
    return fail(MTPX_ERR_STATE, "commit of %d positions; the last verify had %d", n, s->window);
  if (s->window == 0) return MTPX_OK;  // nothing open: committing nothing again changes nothing
  for (GdnState* g : s->gdn)
    if (g) g->committed = n;
  if (s->ple) s->ple->committed = n;
  s->offset += n;
  s->window = 0;
  for (Kv* kv : s->kv)
    if (kv) kv->offset = s->offset;
  return MTPX_OK;
}

namespace {
int target_verify_enqueue(Ctx* c, Target* t, TargetState* s, const int32_t* ids, int S, uint16_t* logits,
                          uint16_t* multi, uint16_t* mixed, bool* launched, bool prefill = false);
}

int mtpx_target_verify(mtpx_ctx h, mtpx_target th, mtpx_target_state sh, const int32_t* ids, int S, uint16_t* logits,
                       uint16_t* multi, uint16_t* mixed) {
  Ctx* c = C(h);
  Target* t = static_cast<Target*>(th.ctx);
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(c && t && s && ids, "null argument");
  ARG(device_readable(ids), "ids: not memory the device can read (device or pinned host memory)");
  ARG(s->t == t, "state of another target");
  if (s->broken) return fail(MTPX_ERR_STATE, "state left inconsistent by a failed verify; reset it first");
  ARG(S >= 1 && S <= MAX_TOKENS, "S=%d", S);
  const mtpx_layer_config& lc = t->cfg.layer;
  ARG(s->offset + S <= lc.max_positions, "cache full (offset %lld + %d)", (long long)s->offset, S);
  ARG(s->offset + S <= MTPX_INDEXER_BUDGET,
      "offset %lld + %d tokens is past the indexer budget %d (the sparse-indexer path is not built)",
      (long long)s->offset, S, MTPX_INDEXER_BUDGET);
  if (set_device(c)) return MTPX_ERR_HIP;
  bool launched = false;
  const int rc = target_verify_enqueue(c, t, s, ids, S, logits, multi, mixed, &launched);
  if (rc && launched) {
    s->window = 0;
    s->broken = true;
  }
  return rc;
}

constexpr int PREFILL_PASS = 512;  // positions per prefill batch (workspace: attention partials grow with it)

int mtpx_target_prefill(mtpx_ctx h, mtpx_target th, mtpx_target_state sh, const int32_t* ids, int S,
                        uint16_t* logits, uint16_t* multi) {
  Ctx* c = C(h);
  Target* t = static_cast<Target*>(th.ctx);
  TargetState* s = static_cast<TargetState*>(sh.ctx);
  ARG(c && t && s && ids, "null argument");
  ARG(device_readable(ids), "ids: not memory the device can read (device or pinned host memory)");
  ARG(s->t == t, "state of another target");
  if (s->broken) return fail(MTPX_ERR_STATE, "state left inconsistent by a failed verify; reset it first");
  ARG(S >= 1, "S=%d", S);
  const mtpx_layer_config& lc = t->cfg.layer;
  ARG(s->offset + S <= lc.max_positions, "cache full (offset %lld + %d)", (long long)s->offset, S);
  ARG(s->offset + S <= MTPX_INDEXER_BUDGET,
      "offset %lld + %d tokens is past the indexer budget %d (the sparse-indexer path is not built)",
      (long long)s->offset, S, MTPX_INDEXER_BUDGET);
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t W = (size_t)t->cfg.hc * lc.hidden;
  for (int p0 = 0; p0 < S; p0 += PREFILL_PASS) {
    const int n = S - p0 < PREFILL_PASS ? S - p0 : PREFILL_PASS;
    bool launched = false;
    const int rc = target_verify_enqueue(c, t, s, ids + p0, n, p0 + n == S ? logits : nullptr,
                                         multi ? multi + (size_t)p0 * W : nullptr, nullptr, &launched, true);
    if (rc) {
      if (launched || p0 > 0) {  // some layers hold part of the batch
        s->window = 0;
        s->broken = true;
      }
      return rc;
    }
  }
  return MTPX_OK;
}

namespace {
// One window of S <= MAX_TOKENS positions (verify), or a prefill batch of S positions: the same
// kernels over all S tokens where every token's output is its own (GEMVs, norms, mixers,
// attention -- each query sees the keys up to its own position --, the MoE as windows of
// MAX_TOKENS), the recurrent cores (GDN, PLE) window by window of MAX_TOKENS with each window
// committed before the next, and the logits of the last position only.  Every output equals that
// of the windows of MAX_TOKENS verified and committed in turn.
int target_verify_enqueue(Ctx* c, Target* t, TargetState* s, const int32_t* ids, int S, uint16_t* logits,
                          uint16_t* multi, uint16_t* mixed, bool* launched, bool prefill) {
  const mtpx_target_config& g = t->cfg;
  const mtpx_layer_config& lc = g.layer;
  const int H = lc.hidden, hc = g.hc, W = hc * H, gs = lc.group_size, HQ = lc.heads, D = lc.head_dim;
  const GdnGeom gg = gdn_geom(target_gdn_cfg(g));
  const int VD = gg.hv * 128;
  const int XB = std::max(H, HQ * D) / 32;
  const HcGeom hg{H, hc, g.lowrank, gs};
  const float eps = lc.eps;
  // an uncommitted window is discarded: caches rewind to the committed offset
  for (Kv* kv : s->kv)
    if (kv) kv->offset = s->offset;
  const int T = (int)s->offset + S;
  const size_t mix = al(2 * (size_t)S * g.lowrank) * 2 + al(2 * (size_t)S * hc) +
                     al(4 * (size_t)S * (g.lowrank / 32) * XP_DW) + al(2 * (size_t)S * W) +
                     (S > MAX_TOKENS ? al(4 * (size_t)S * (W / 32) * XMB_DW) : 0);
  const Layer* any_attn = nullptr;
  for (const TargetLayer& L : t->layers)
    if (L.attn) any_attn = L.attn;
  const int SW = S < MAX_TOKENS ? S : MAX_TOKENS;  // positions of one recurrent window
  const size_t moe_ws = prefill ? moe_windows_ws_bytes(&t->layers[0].moe, S) : moe_ws_bytes(&t->layers[0].moe, S);
  const size_t gdn_ws = prefill ? al(4 * (size_t)S * gg.hv * 128) + al(4 * (size_t)S * (2 * gg.hk + gg.hv) * 128) +
                                      al(8 * (size_t)S * gg.hv)
                                : 0;  // the batch's recurrence outputs, prepped vectors and gates
  const size_t per_layer = std::max(std::max(std::max(mix + moe_ws, mix + (any_attn ? attn_ws_bytes(any_attn, S, T) : 0)),
                                             mix + gdn_ws),
                                    t->ple ? ple_ws_bytes(t->ple->cfg, SW) + al(2 * (size_t)S * W) : 0) + 4096;
  const size_t fixed = al(2 * (size_t)S * H) * 5 + al(2 * (size_t)S * W) * 4 + al(2 * (size_t)S * hc) * 2 +
                       al(4 * (size_t)S * (W / 32) * XP_DW) + al(4 * (size_t)S * XB * XP_DW) +
                       al(4 * (size_t)S * (VD / 32) * XP_DW) + al(2 * (size_t)S * gg.pw) + 4096;
  int rc = ws_reserve(c, fixed + per_layer);
  if (rc) return rc;
  ws_begin(c);
  uint16_t* e = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* x = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* ao = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* mo = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* mx = mixed ? mixed : ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* sA = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* sM = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* nrm = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* mt = multi ? multi : ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* jA = ws_take<uint16_t>(c, (size_t)S * hc);
  uint16_t* jM = ws_take<uint16_t>(c, (size_t)S * hc);
  uint32_t* xpW = ws_take<uint32_t>(c, (size_t)S * (W / 32) * XP_DW);
  uint32_t* xpH = ws_take<uint32_t>(c, (size_t)S * XB * XP_DW);
  uint32_t* xpG = ws_take<uint32_t>(c, (size_t)S * (VD / 32) * XP_DW);
  uint16_t* proj = ws_take<uint16_t>(c, (size_t)S * gg.pw);
  const size_t mark = c->ws_used;
  hipStream_t st = c->stream;
  *launched = true;
  LAUNCH(c, "embed", launch_embed_rows(t->embed.w, t->embed.s, t->embed.b, H, gs, g.vocab, ids, S, e, st));
  for (int i = 0; i < (int)t->layers.size(); ++i) {
    const TargetLayer& L = t->layers[i];
    const bool first = i == 0;
    c->ws_used = mark;
    if (i == g.ple_layer && t->ple) {
      // the stream of the first inject-norm goes through the PLE block, then is normed again
      LAUNCH(c, "hc_norm", launch_hc_norm(first ? e : sM, first ? nullptr : mo, first ? nullptr : jM, S, hc, H,
                                          first ? 1 : 0, L.attn_hc.norm_scale, eps, sA, nrm, nullptr, st));
      uint16_t* sp = ws_take<uint16_t>(c, (size_t)S * W);
      const size_t mark2 = c->ws_used;
      for (int w0 = 0; w0 < S; w0 += MAX_TOKENS) {  // window by window (one window when verifying)
        const int n = S - w0 < MAX_TOKENS ? S - w0 : MAX_TOKENS;
        c->ws_used = mark2;
        if ((rc = ple_enqueue(c, t->ple, s->ple, ids + w0, n, sA + (size_t)w0 * W, nullptr, sp + (size_t)w0 * W,
                              nullptr)))
          return rc;
        if (prefill) s->ple->committed = n;
      }
      LAUNCH(c, "hc_norm", launch_hc_norm(sp, nullptr, nullptr, S, hc, H, 0, L.attn_hc.norm_scale, eps, sA, nrm, xpW,
                                          st));
    } else {
      LAUNCH(c, "hc_norm", launch_hc_norm(first ? e : sM, first ? nullptr : mo, first ? nullptr : jM, S, hc, H,
                                          first ? 1 : 0, L.attn_hc.norm_scale, eps, sA, nrm, xpW, st));
    }
    c->ws_used = mark;
    if ((rc = hc_mix_enqueue(c, hg, &L.attn_hc, nrm, xpW, S, x, jA, xpH))) return rc;
    if (L.kind == MTPX_LAYER_GDN) {
      const mtpx_q4& ip = L.gdn->w.in_proj;
      const mtpx_q4& op = L.gdn->w.out_proj;
      LAUNCH(c, "qmv_gdn_in", launch_qmv(ip.w, ip.s, ip.b, ip.sb, gg.pw, H, gs, xpH, S, proj, nullptr, st));
      if (prefill) {  // the batch in one launch, committed
        const size_t mark3 = c->ws_used;
        if ((rc = gdn_enqueue_batch(c, L.gdn, s->gdn[i], proj, S, nullptr, xpG))) return rc;
        c->ws_used = mark3;
      } else if ((rc = gdn_enqueue(c, L.gdn, s->gdn[i], proj, S, nullptr, xpG))) {
        return rc;
      }
      LAUNCH(c, "qmv_gdn_out", launch_qmv(op.w, op.s, op.b, op.sb, H, VD, gs, xpG, S, ao, nullptr, st));
    } else {
      if ((rc = attn_enqueue(c, L.attn, s->kv[i], xpH, S, ao))) return rc;
    }
    LAUNCH(c, "hc_norm", launch_hc_norm(sA, ao, jA, S, hc, H, 0, L.mlp_hc.norm_scale, eps, sM, nrm, xpW, st));
    c->ws_used = mark;
    if ((rc = hc_mix_enqueue(c, hg, &L.mlp_hc, nrm, xpW, S, x, jM, xpH))) return rc;
    if (prefill) {
      if ((rc = moe_enqueue_windows(c, &L.moe, x, S, mo, xpH))) return rc;
    } else if ((rc = moe_enqueue(c, &L.moe, x, S, mo, nullptr, nullptr, nullptr, nullptr, nullptr, xpH,
                                 s->moe_unique + i))) {
      return rc;
    }
  }
  LAUNCH(c, "hc_norm", launch_hc_norm(sM, mo, jM, S, hc, H, 0, t->final_hc.norm_scale, eps, mt, nrm, xpW, st));
  c->ws_used = mark;
  if ((rc = hc_mix_enqueue(c, hg, &t->final_hc, nrm, xpW, S, mx, nullptr, xpH))) return rc;
  if (logits) {
    const int r0 = prefill ? S - 1 : 0;  // prefill: the last position's row only
    LAUNCH(c, "qmv_lm_head", launch_qmv(t->lm_head.w, t->lm_head.s, t->lm_head.b, t->lm_head.sb, (int)g.vocab, H, gs,
                                        xpH + (size_t)r0 * (H / 32) * XP_DW, S - r0, logits, nullptr, st));
  }
  for (Kv* kv : s->kv)
    if (kv) kv->offset = s->offset + S;
  if (prefill) {  // every window committed (the recurrent states' last window in full)
    s->offset += S;
    s->window = 0;
    return MTPX_OK;
  }
  s->window = S;
  return MTPX_OK;
}
}  // namespace

int mtpx_profile_enable(mtpx_ctx h, int on) {
  Ctx* c = C(h);
  ARG(c, "null context");
  c->prof = on != 0;
  return MTPX_OK;
}

int mtpx_profile_reset(mtpx_ctx h) {
  Ctx* c = C(h);
  ARG(c, "null context");
  int rc = prof_fold(c);
  if (rc) return rc;
  c->stats.clear();
  return MTPX_OK;
}

int mtpx_profile_dump(mtpx_ctx h, char* buf, size_t n) {
  Ctx* c = C(h);
  ARG(c && buf && n > 0, "bad argument");
  int rc = prof_fold(c);
  if (rc) return rc;
  std::string out;
  for (auto& kv : c->stats) {
    char line[160];
    snprintf(line, sizeof(line), "%s %lld %.6f\n", kv.first.c_str(), (long long)kv.second.first, kv.second.second);
    out += line;
  }
  ARG(out.size() < n, "buffer of %zu bytes too small", n);
  memcpy(buf, out.c_str(), out.size() + 1);
  return MTPX_OK;
}

int mtpx_last_moe_bytes(mtpx_ctx h, int64_t* bytes, int32_t* n_unique) {
  Ctx* c = C(h);
  ARG(c && bytes, "null argument");
  ARG(c->last_disp, "no MoE call with this context's workspace yet (the allocation-free entry keeps no count)");
  if (set_device(c)) return MTPX_ERR_HIP;
  int nu = 0;
  HIP_OK(hipMemcpyAsync(&nu, &c->last_disp->n_unique, 4, hipMemcpyDeviceToHost, c->stream));
  HIP_OK(hipStreamSynchronize(c->stream));
  const int64_t H = c->last_H, E = c->last_E, F = c->last_F, gs = c->last_gs;
  auto B = [&](int64_t N, int64_t K) { return N * K / 2 + 4 * N * K / gs; };
  *bytes = (int64_t)(nu + 1) * (2 * B(F, H) + B(H, F)) + 2 * E * H + 2 * H;
  if (n_unique) *n_unique = nu;
  return MTPX_OK;
}

int mtpx_shortlist_argmax(mtpx_ctx h, const uint16_t* x, int H, const uint32_t* w, const uint16_t* s,
                          const uint16_t* b, const uint32_t* sb, int gs, int rows, const int32_t* ids, int32_t* out) {
  Ctx* c = C(h);
  ARG(c && x && w && s && b && out, "null argument");
  ARG(gs_ok(gs) && k_ok(H, gs), "H=%d gs=%d", H, gs);
  ARG(rows >= 1, "rows=%d", rows);
  if (set_device(c)) return MTPX_ERR_HIP;
  const size_t n = argmax_work_items(1, rows);
  int rc = ws_reserve(c, al(4 * (size_t)(H / 32) * XP_DW) + al(2 * (size_t)rows) + al(n * 4) * 2 + 1024);
  if (rc) return rc;
  ws_begin(c);
  uint32_t* xp = ws_take<uint32_t>(c, (size_t)(H / 32) * XP_DW);
  uint16_t* y = ws_take<uint16_t>(c, (size_t)rows);
  float* pv = ws_take<float>(c, n);
  int32_t* pi = ws_take<int32_t>(c, n);
  hipStream_t st = c->stream;
  LAUNCH(c, "xprep", launch_xprep(x, 1, H, xp, st));
  LAUNCH(c, "qmv_shortlist", launch_qmv(w, s, b, sb, rows, H, gs, xp, 1, y, nullptr, st));
  LAUNCH(c, "shortlist_argmax", launch_argmax_rows_bf16(y, 1, rows, pv, pi, ids, out, st));
  return MTPX_OK;
}

int mtpx_head_new_random(mtpx_ctx h, const mtpx_head_config* cfg, uint64_t seed, mtpx_head* out) {
  Ctx* c = C(h);
  ARG(c && cfg && out, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  Head* hd = nullptr;
  int rc = head_create(c, cfg, seed, &hd);
  if (rc) return rc;
  out->ctx = hd;
  return MTPX_OK;
}

int mtpx_head_adopt(mtpx_ctx h, const mtpx_head_config* cfg, const mtpx_head_weights* win, int pack_sb,
                    mtpx_head* out) {
  Ctx* c = C(h);
  ARG(c && cfg && win && out, "null argument");
  int rc = head_check(cfg);
  if (rc) return rc;
  ARG(win->shortlist_rows >= 1 && win->shortlist_rows % 8 == 0, "shortlist_rows=%d (a positive multiple of 8)",
      win->shortlist_rows);
  if (set_device(c)) return MTPX_ERR_HIP;
  const mtpx_layer_config& lc = cfg->layer;
  const int H = lc.hidden, W = cfg->hc * H;
  Head* hd = new Head();
  hd->cfg = *cfg;
  hd->w = *win;
  hd->layer = new Layer();
  hd->layer->cfg = lc;
  hd->layer->w = win->layer;
  hd->layer->QW = 2 * lc.heads * lc.head_dim + 2 * lc.kv_heads * lc.head_dim + lc.index_dim;
  mtpx_layer_weights& lw = hd->layer->w;
  lw.qkv_rows = hd->layer->QW;
  Adopt ad{c, lc.group_size, pack_sb != 0, &hd->allocs};
  Adopt la{c, lc.group_size, pack_sb != 0, &hd->layer->allocs};
  mtpx_q4 qkv{lw.qkv_w, lw.qkv_s, lw.qkv_b, lw.qkv_sb}, o{lw.o_w, lw.o_s, lw.o_b, lw.o_sb};
  la.q4(&qkv, hd->layer->QW, H, "head qkv");
  la.q4(&o, H, lc.heads * lc.head_dim, "head o_proj");
  lw.qkv_sb = qkv.sb;
  lw.o_sb = o.sb;
  la.need(lw.q_norm, "head q_norm");
  la.need(lw.k_norm, "head k_norm");
  la.moe(&lw.moe, lc);
  if ((!lw.rope_cos || !lw.rope_sin) && !rope_tables(c, &lc, &hd->layer->allocs, &lw.rope_cos, &lw.rope_sin))
    la.ok = false;
  mtpx_head_weights& w = hd->w;
  ad.q4(&w.embed, cfg->vocab, H, "head embed (the target's embed_tokens)");
  ad.need(w.pre_norm_embedding, "pre_norm_embedding");
  ad.need(w.pre_norm_hidden, "pre_norm_hidden");
  ad.q4(&w.fc_embedding, H, H, "fc_embedding");
  ad.q4(&w.fc_hidden, H, H, "fc_hidden");
  ad.hc(&w.attn_hc, H, cfg->hc, cfg->lowrank, true);
  ad.hc(&w.mlp_hc, H, cfg->hc, cfg->lowrank, true);
  ad.hc(&w.final_hc, H, cfg->hc, cfg->lowrank, false);
  ad.q4(&w.shortlist, w.shortlist_rows, H, "shortlist rows");
  ad.need(w.shortlist_ids, "shortlist ids");
  (void)W;
  rc = la.finish("head layer");
  if (!rc) rc = ad.finish("head");
  if (rc) {
    for (void* p : hd->allocs) hipFree(p);
    for (void* p : hd->layer->allocs) hipFree(p);
    delete hd->layer;
    delete hd;
    return rc;
  }
  w.layer = lw;
  out->ctx = hd;
  return MTPX_OK;
}

int mtpx_head_free(mtpx_head h) {
  Head* hd = static_cast<Head*>(h.ctx);
  if (!hd) return MTPX_OK;
  for (void* p : hd->allocs) hipFree(p);
  if (hd->layer) {
    for (void* p : hd->layer->allocs) hipFree(p);
    delete hd->layer;
  }
  delete hd;
  return MTPX_OK;
}

int mtpx_head_weights_get(mtpx_head h, mtpx_head_weights* out) {
  Head* hd = static_cast<Head*>(h.ctx);
  ARG(hd && out, "null argument");
  *out = hd->w;
  return MTPX_OK;
}

int mtpx_head_forward(mtpx_ctx h, mtpx_head hh, mtpx_kv kvh, const int32_t* ids, int S, const uint16_t* multi,
                      uint16_t* multi_next, uint16_t* sample, int32_t* draft) {
  Ctx* c = C(h);
  Head* hd = static_cast<Head*>(hh.ctx);
  Kv* kv = static_cast<Kv*>(kvh.ctx);
  ARG(c && hd && kv && ids && multi && multi_next, "null argument");
  const mtpx_head_config& g = hd->cfg;
  const mtpx_layer_config& lg = g.layer;
  ARG(S >= 1 && S <= HEAD_BATCH, "S=%d", S);
  ARG(kv->heads == lg.kv_heads && kv->dim == lg.head_dim, "kv cache geometry does not match the head");
  ARG(kv->offset + S <= kv->tmax && kv->offset + S <= lg.max_positions, "cache full (offset %lld + %d)",
      (long long)kv->offset, S);
  ARG(kv->offset + S <= MTPX_INDEXER_BUDGET, "offset %lld + %d tokens is past the indexer budget %d",
      (long long)kv->offset, S, MTPX_INDEXER_BUDGET);
  int rc = moe_check(&hd->w.layer.moe, S < MAX_TOKENS ? S : MAX_TOKENS);
  if (rc) return rc;
  if (set_device(c)) return MTPX_ERR_HIP;
  const int H = lg.hidden, hc = g.hc, W = hc * H, gs = lg.group_size, HQ = lg.heads, D = lg.head_dim;
  const int XB = (H > HQ * D ? H : HQ * D) / 32;
  const float eps = lg.eps;
  const mtpx_head_weights& w = hd->w;
  if ((rc = ws_reserve(c, head_ws_bytes(hd, S, (int)kv->offset + S)))) return rc;
  ws_begin(c);
  uint16_t* e = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* en = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* emb = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* x = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* ao = ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* samp = sample ? sample : ws_take<uint16_t>(c, (size_t)S * H);
  uint16_t* mn = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* hs = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* st0 = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* st1 = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* nrm = ws_take<uint16_t>(c, (size_t)S * W);
  uint16_t* j = ws_take<uint16_t>(c, (size_t)S * hc);
  uint32_t* xpH = ws_take<uint32_t>(c, (size_t)S * XB * XP_DW);
  uint32_t* xpW = ws_take<uint32_t>(c, (size_t)S * (W / 32) * XP_DW);
  hipStream_t st = c->stream;
  // e = fc_embedding(rms(embed(ids))); h = fc_hidden(rms_W(multi)) per stream
  LAUNCH(c, "embed", launch_embed_rows(w.embed.w, w.embed.s, w.embed.b, H, gs, g.vocab, ids, S, e, st));
  LAUNCH(c, "hc_norm", launch_hc_norm(e, nullptr, nullptr, S, 1, H, 0, w.pre_norm_embedding, eps, nullptr, en, xpH,
                                      st));
  LAUNCH(c, "qmv_fc", launch_qmv(w.fc_embedding.w, w.fc_embedding.s, w.fc_embedding.b, w.fc_embedding.sb, H, H, gs, xpH, S, emb,
                                 nullptr, st));
  LAUNCH(c, "hc_norm", launch_hc_norm(multi, nullptr, nullptr, S, 1, W, 0, w.pre_norm_hidden, eps, nullptr, mn, xpW,
                                      st));
  LAUNCH(c, "qmv_fc", launch_qmv(w.fc_hidden.w, w.fc_hidden.s, w.fc_hidden.b, w.fc_hidden.sb, H, H, gs, xpW, S * hc, hs, nullptr,
                                 st));
  // attention block: hyper = e + h; (st0, n) = hc_norm(hyper); (x, j) = mix(attn_hc, n); ao = attn(x)
  LAUNCH(c, "hc_norm", launch_hc_norm(hs, emb, nullptr, S, hc, H, 0, w.attn_hc.norm_scale, eps, st0, nrm, xpW, st));
  if ((rc = hc_mix_enqueue(c, hd, &w.attn_hc, nrm, xpW, S, x, j, xpH))) return rc;
  if ((rc = attn_enqueue(c, hd->layer, kv, xpH, S, ao))) return rc;
  // MoE block
  LAUNCH(c, "hc_norm", launch_hc_norm(st0, ao, j, S, hc, H, 0, w.mlp_hc.norm_scale, eps, st1, nrm, xpW, st));
  if ((rc = hc_mix_enqueue(c, hd, &w.mlp_hc, nrm, xpW, S, x, j, xpH))) return rc;
  if (S > MAX_TOKENS) {  // a batch of the drafter's backlog: the MoE as windows of MAX_TOKENS
    if ((rc = moe_enqueue_windows(c, &w.layer.moe, x, S, ao, xpH))) return rc;
  } else if ((rc = moe_enqueue(c, &w.layer.moe, x, S, ao, nullptr, nullptr, nullptr, nullptr, nullptr, xpH))) {
    return rc;
  }
  // final mixer: multi_next = st1 + m*j; sample = mix(final_hc, hc_norm(multi_next))
  LAUNCH(c, "hc_norm", launch_hc_norm(st1, ao, j, S, hc, H, 0, w.final_hc.norm_scale, eps, multi_next, nrm, xpW,
                                      st));
  if ((rc = hc_mix_enqueue(c, hd, &w.final_hc, nrm, xpW, S, samp, nullptr, xpH))) return rc;
  if (draft) {
    const int NS = w.shortlist_rows;
    const size_t n = argmax_work_items(1, NS);
    uint16_t* yl = ws_take<uint16_t>(c, (size_t)NS);
    float* pv = ws_take<float>(c, n);
    int32_t* pi = ws_take<int32_t>(c, n);
    LAUNCH(c, "qmv_shortlist", launch_qmv(w.shortlist.w, w.shortlist.s, w.shortlist.b, w.shortlist.sb, NS, H, gs,
                                          xpH + (size_t)(S - 1) * (H / 32) * XP_DW, 1, yl, nullptr, st));
    LAUNCH(c, "shortlist_argmax", launch_argmax_rows_bf16(yl, 1, NS, pv, pi, w.shortlist_ids, draft, st));
  }
  kv->offset += S;
  return MTPX_OK;
}

static int dr_status(DrafterObj* o, int rc) {
  if (rc == DR_OK) return MTPX_OK;
  if (rc == DR_ERR_BACKEND) return g_err.empty() ? fail(MTPX_ERR_HIP, "%s", o->d->error().c_str()) : MTPX_ERR_HIP;
  return fail(rc == DR_ERR_ARG ? MTPX_ERR_ARG : MTPX_ERR_STATE, "%s", o->d->error().c_str());
}

int mtpx_drafter_new(mtpx_ctx h, mtpx_head hh, mtpx_drafter* out) {
  Ctx* c = C(h);
  Head* hd = static_cast<Head*>(hh.ctx);
  ARG(c && hd && out, "null argument");
  if (set_device(c)) return MTPX_ERR_HIP;
  const mtpx_layer_config& lg = hd->cfg.layer;
  mtpx_kv kv{nullptr};
  int rc = mtpx_kv_new(h, lg.kv_heads, lg.head_dim, lg.max_positions, &kv);
  if (rc) return rc;
  DrafterObj* o = new DrafterObj();
  o->be.c = c;
  o->be.hh = hh;
  o->be.kv = static_cast<Kv*>(kv.ctx);
  o->be.W = hd->cfg.hc * lg.hidden;
  if (hipMalloc((void**)&o->be.multi_scratch, 2 * (size_t)HEAD_BATCH * o->be.W) != hipSuccess) {
    mtpx_kv_free(kv);
    delete o;
    return fail(MTPX_ERR_OOM, "drafter scratch");
  }
  o->d = new Drafter<DevBackend>(o->be);
  out->ctx = o;
  return MTPX_OK;
}

int mtpx_drafter_free(mtpx_drafter dh) {
  DrafterObj* o = static_cast<DrafterObj*>(dh.ctx);
  if (!o) return MTPX_OK;
  hipSetDevice(o->be.c->device);
  hipStreamSynchronize(o->be.c->stream);
  delete o->d;  // rows go back to the pool first
  if (o->be.multi_scratch) hipFree(o->be.multi_scratch);
  mtpx_kv_free(mtpx_kv{o->be.kv});
  delete o;
  return MTPX_OK;
}

int mtpx_drafter_observe(mtpx_drafter dh, const int32_t* tokens, const uint16_t* multi, int n) {
  DrafterObj* o = static_cast<DrafterObj*>(dh.ctx);
  ARG(o, "null drafter");
  if (set_device(o->be.c)) return MTPX_ERR_HIP;
  g_err.clear();
  return dr_status(o, o->d->observe(tokens, multi, n, o->be.W));
}

int mtpx_drafter_step(mtpx_drafter dh, const int32_t* token, const uint16_t* multi, int32_t* draft,
                      uint16_t* multi_out) {
  DrafterObj* o = static_cast<DrafterObj*>(dh.ctx);
  ARG(o && draft && multi_out, "null argument");
  if (set_device(o->be.c)) return MTPX_ERR_HIP;
  g_err.clear();
  return dr_status(o, o->d->step(token, multi, draft, multi_out));
}

int mtpx_drafter_finalize(mtpx_drafter dh, int confirmed_inputs, const int32_t* tokens, const uint16_t* multi,
                          int n) {
  DrafterObj* o = static_cast<DrafterObj*>(dh.ctx);
  ARG(o, "null drafter");
  if (set_device(o->be.c)) return MTPX_ERR_HIP;
  g_err.clear();
  return dr_status(o, o->d->finalize(confirmed_inputs, tokens, multi, n));
}

int mtpx_drafter_discard(mtpx_drafter dh) {
  DrafterObj* o = static_cast<DrafterObj*>(dh.ctx);
  ARG(o, "null drafter");
  g_err.clear();
  return dr_status(o, o->d->discard());
}

int mtpx_drafter_release(mtpx_drafter dh) {
  DrafterObj* o = static_cast<DrafterObj*>(dh.ctx);
  ARG(o, "null drafter");
  o->d->release();
  return MTPX_OK;
}

int mtpx_drafter_info_get(mtpx_drafter dh, mtpx_drafter_info* out) {
  DrafterObj* o = static_cast<DrafterObj*>(dh.ctx);
  ARG(o && out, "null argument");
  Drafter<DevBackend>& d = *o->d;
  out->cache_offset = d.cache_offset();
  out->committed_inputs = d.committed_inputs();
  out->staged_inputs = d.staged_inputs();
  out->backlog_inputs = d.backlog_inputs();
  out->round_base_offset = d.round_base_offset();
  out->round_valid_offset = d.round_valid_offset();
  out->round_in_flight = d.in_flight();
  out->round_draft_steps = d.draft_steps();
  out->has_frontier = d.has_frontier();
  out->released = d.released();
  return MTPX_OK;
}

int mtpx_drafter_bytes_per_token(mtpx_head hh, int64_t* out) {
  Head* hd = static_cast<Head*>(hh.ctx);
  ARG(hd && out, "null argument");
  const mtpx_layer_config& lg = hd->cfg.layer;
  const int64_t per_layer = 2 * (int64_t)lg.kv_heads * lg.head_dim + lg.index_dim;
  *out = per_layer * 1 * 2 + (int64_t)hd->cfg.hc * lg.hidden * 2 + 4;  // one head layer, bf16 rows, one int32 id
  return MTPX_OK;
}

}  // extern "C"
