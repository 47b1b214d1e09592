// One request's single-stream MTP speculative decode, device-resident: the round of the
// engine core the reference's runner drives (the accept loop of the un-vendored engine core,
// semantics docs/qwen38-125b-a6b-port-notes.md:313-343; drafter calls
// Runner/Qwen4ExpMTPDrafter.swift:328-454; target verify + commit
// Runner/FastModel/TrackFastModel.swift:1463-1475, :726-731).
//
// A session holds the target's per-request caches, the drafter's request state and the carry
// (the token at the committed offset that the next round feeds first, with the target's multi
// stream of the position before it).  A round with draft depth k:
//   k drafter steps (the first flushes the drafter's backlog), each draft optionally replaced by
//   the forcing hook; a verify of the carry and the k drafts; the greedy accept on the device
//   (row argmaxes, accepted prefix n, bonus token, committed tokens) -- or, at a temperature,
//   speculative sampling with one-hot draft distributions --; ONE readback of those
//   integers; the target commit of n + 1 positions and the drafter finalize with the target's
//   own multi streams; the next carry is copied on the device (bonus token, multi row n).
// k = 0 is a plain serial decode step (verify of the carry alone, commit, observe).
// Built on the public C ABI only; every call of a session runs on its context's stream.
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/mtpx.h"
#include "abi_internal.h"

namespace {

using namespace mtpx;

constexpr int OUT_WORDS = 24;  // out3 at 0, argmax rows at 4.., committed tokens at 12..
constexpr int PROMPT_BATCH = 512;  // prompt positions per target prefill call (their multi streams are observed)

struct Session {
  mtpx_ctx ctx{nullptr};
  mtpx_target target{nullptr};
  mtpx_head head{nullptr};
  mtpx_target_state state{nullptr};
  mtpx_drafter drafter{nullptr};
  int64_t vocab = 0;
  int W = 0;
  int32_t* ids = nullptr;      // [MTPX_MAX_DRAFT_DEPTH + 2]: carry, drafts
  uint16_t* logits = nullptr;  // bf16 [8, vocab]
  uint16_t* multi = nullptr;   // bf16 [8, W]: the verify's multi streams
  uint16_t* mo = nullptr;      // bf16 [MTPX_MAX_DRAFT_DEPTH, W]: the drafter's multi streams
  uint16_t* carry = nullptr;   // bf16 [W]: multi stream paired with the carry token
  uint16_t* pmulti = nullptr;  // bf16 [PROMPT_BATCH, W]: a prompt batch's multi streams
  int32_t* out = nullptr;      // device [OUT_WORDS]
  int32_t* host = nullptr;     // pinned [OUT_WORDS]
  int64_t offset = 0;          // committed positions (mirrors the target state)
  bool primed = false;         // a carry exists (after prefill)
  bool broken = false;         // a prefill or round failed part way: refused until mtpx_session_reset
};

#define RC(expr)             \
  do {                       \
    const int rc_ = (expr);  \
    if (rc_) return rc_;     \
  } while (0)

#define HIPRC(expr)                                                              \
  do {                                                                           \
    if ((expr) != hipSuccess) return set_error(MTPX_ERR_HIP, #expr " failed"); \
  } while (0)

void release(Session* s) {
  if (s->drafter.ctx) mtpx_drafter_free(s->drafter);
  if (s->state.ctx) mtpx_target_state_free(s->state);
  for (void* p : {(void*)s->ids, (void*)s->logits, (void*)s->multi, (void*)s->mo, (void*)s->carry, (void*)s->out,
                  (void*)s->pmulti})
    if (p) hipFree(p);
  if (s->host) hipHostFree(s->host);
  delete s;
}

// Read the round's integers back (the one host synchronisation of a round).
int readback(Session* s) {
  hipStream_t st = ctx_stream(s->ctx);
  HIPRC(hipMemcpyAsync(s->host, s->out, 4 * OUT_WORDS, hipMemcpyDeviceToHost, st));
  HIPRC(hipStreamSynchronize(st));
  return MTPX_OK;
}

// Next carry on the device: token tokens[n] -> ids[0], row n of the multi streams -> carry.
int next_carry(Session* s, const uint16_t* multi, int n) {
  hipStream_t st = ctx_stream(s->ctx);
  HIPRC(hipMemcpyAsync(s->ids, s->out + 1, 4, hipMemcpyDeviceToDevice, st));
  HIPRC(hipMemcpyAsync(s->carry, multi + (size_t)n * s->W, 2 * (size_t)s->W, hipMemcpyDeviceToDevice, st));
  return MTPX_OK;
}

}  // namespace

extern "C" {

int mtpx_session_new(mtpx_ctx ctx, mtpx_target target, mtpx_head head, mtpx_session* out) {
  if (!ctx.ctx || !target.ctx || !out) return set_error(MTPX_ERR_ARG, "session: null argument");
  Session* s = new Session();
  s->ctx = ctx;
  s->target = target;
  s->head = head;
  target_dims(target, &s->vocab, &s->W);
  if (head.ctx && head_width(head) != s->W) {
    delete s;
    return set_error(MTPX_ERR_ARG, "session: the head's multi stream width differs from the target's");
  }
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) {
    delete s;
    return set_error(MTPX_ERR_HIP, "session: hipSetDevice");
  }
  int rc = mtpx_target_state_new(ctx, target, &s->state);
  if (!rc && head.ctx) rc = mtpx_drafter_new(ctx, head, &s->drafter);
  bool ok = rc == MTPX_OK;
  ok = ok && hipMalloc((void**)&s->ids, 4 * (MTPX_MAX_DRAFT_DEPTH + 2)) == hipSuccess;
  ok = ok && hipMalloc((void**)&s->logits, 2 * (size_t)8 * s->vocab) == hipSuccess;
  ok = ok && hipMalloc((void**)&s->multi, 2 * (size_t)8 * s->W) == hipSuccess;
  ok = ok && hipMalloc((void**)&s->mo, 2 * (size_t)MTPX_MAX_DRAFT_DEPTH * s->W) == hipSuccess;
  ok = ok && hipMalloc((void**)&s->carry, 2 * (size_t)s->W) == hipSuccess;
  ok = ok && hipMalloc((void**)&s->pmulti, 2 * (size_t)PROMPT_BATCH * s->W) == hipSuccess;
  ok = ok && hipMalloc((void**)&s->out, 4 * OUT_WORDS) == hipSuccess;
  ok = ok && hipHostMalloc((void**)&s->host, 4 * OUT_WORDS, hipHostMallocDefault) == hipSuccess;
  if (!ok) {
    release(s);
    return rc ? rc : set_error(MTPX_ERR_OOM, "session buffers");
  }
  out->ctx = s;
  return MTPX_OK;
}

int mtpx_session_free(mtpx_session sh) {
  Session* s = static_cast<Session*>(sh.ctx);
  if (!s) return MTPX_OK;
  mtpx_ctx_synchronize(s->ctx);
  release(s);
  return MTPX_OK;
}

int mtpx_session_reset(mtpx_session sh) {
  Session* s = static_cast<Session*>(sh.ctx);
  if (!s) return set_error(MTPX_ERR_ARG, "session: null");
  RC(mtpx_target_state_reset(s->ctx, s->state));
  if (s->drafter.ctx) {
    RC(mtpx_ctx_synchronize(s->ctx));
    mtpx_drafter_free(s->drafter);
    s->drafter.ctx = nullptr;
    RC(mtpx_drafter_new(s->ctx, s->head, &s->drafter));
  }
  s->offset = 0;
  s->primed = false;
  s->broken = false;
  return MTPX_OK;
}

static int prefill_batches(Session* s, const int32_t* ids, int n, int32_t* first_token);
static int round_steps(Session* s, int k, const mtpx_force_params* force, float temperature, uint64_t seed,
                       int32_t* tokens, int* n_tokens);

int mtpx_session_prefill(mtpx_session sh, const int32_t* ids, int n, int32_t* first_token) {
  Session* s = static_cast<Session*>(sh.ctx);
  if (!s || !ids || n < 1) return set_error(MTPX_ERR_ARG, "session prefill: bad argument");
  if (!device_readable(ids))
    return set_error(MTPX_ERR_ARG, "session prefill: ids are not memory the device can read (device or pinned host)");
  if (s->broken) return set_error(MTPX_ERR_STATE, "session: a previous call failed part way (reset it)");
  if (s->primed) return set_error(MTPX_ERR_STATE, "session prefill: the session already holds a context");
  if (s->offset + n > MTPX_INDEXER_BUDGET) return set_error(MTPX_ERR_ARG, "session prefill: past the indexer budget");
  const int rc = prefill_batches(s, ids, n, first_token);
  if (rc) s->broken = true;  // batches may have been committed: the caches no longer match the offset
  return rc;
}

// The prompt through the target prefill in batches (each committed), the drafter observing every
// batch's multi streams; the first generated token is the argmax of the last position's logits.
static int prefill_batches(Session* s, const int32_t* ids, int n, int32_t* first_token) {
  for (int off = 0; off < n; off += PROMPT_BATCH) {
    const int S = n - off < PROMPT_BATCH ? n - off : PROMPT_BATCH;
    const bool last = off + S == n;
    RC(mtpx_target_prefill(s->ctx, s->target, s->state, ids + off, S, last ? s->logits : nullptr, s->pmulti));
    if (s->drafter.ctx) RC(mtpx_drafter_observe(s->drafter, ids + off, s->pmulti, S));
    if (last) {
      // out3[1] of a depth-0 accept on the last row
      RC(mtpx_accept_greedy_bf16(s->ctx, s->logits, 0, s->vocab, nullptr, (int32_t)(s->offset + off + S - 1), s->out,
                                 nullptr, nullptr));
      RC(next_carry(s, s->pmulti, S - 1));
    }
  }
  RC(readback(s));
  s->offset += n;
  s->primed = true;
  if (first_token) *first_token = s->host[1];
  return MTPX_OK;
}

int mtpx_round(mtpx_session sh, int k, const mtpx_force_params* force, int32_t* tokens, int* n_tokens) {
  return mtpx_round_sampled(sh, k, force, 0.0f, 0, tokens, n_tokens);
}

int mtpx_round_sampled(mtpx_session sh, int k, const mtpx_force_params* force, float temperature, uint64_t seed,
                       int32_t* tokens, int* n_tokens) {
  Session* s = static_cast<Session*>(sh.ctx);
  if (!s || !tokens || !n_tokens) return set_error(MTPX_ERR_ARG, "round: null argument");
  if (!(temperature >= 0.0f) || !(temperature < 3.4e38f)) return set_error(MTPX_ERR_ARG, "round: temperature");
  if (s->broken) return set_error(MTPX_ERR_STATE, "session: a previous call failed part way (reset it)");
  if (!s->primed) return set_error(MTPX_ERR_STATE, "round: no context (prefill first)");
  if (k < 0 || k > MTPX_MAX_DRAFT_DEPTH || (k > 0 && !s->drafter.ctx))
    return set_error(MTPX_ERR_ARG, "round: draft depth out of range (or no drafter)");
  if (s->offset + k + 1 > MTPX_INDEXER_BUDGET) return set_error(MTPX_ERR_ARG, "round: past the indexer budget");
  if (force && force->teacher && (force->rate < 0.0f || force->rate > 1.0f))
    return set_error(MTPX_ERR_ARG, "round: forcing rate outside [0, 1]");
  const int rc = round_steps(s, k, force, temperature, seed, tokens, n_tokens);
  if (rc) s->broken = true;  // drafter and target may have advanced apart
  return rc;
}

static int round_steps(Session* s, int k, const mtpx_force_params* force, float temperature, uint64_t seed,
                       int32_t* tokens, int* n_tokens) {
  const int64_t o = s->offset;
  for (int i = 0; i < k; ++i) {
    RC(mtpx_drafter_step(s->drafter, s->ids + i, i == 0 ? s->carry : s->mo + (size_t)(i - 1) * s->W, s->ids + i + 1,
                         s->mo + (size_t)i * s->W));
    if (force && force->teacher && o + i + 1 < force->teacher_len)
      RC(mtpx_force_draft(s->ctx, s->ids + i + 1, force->teacher, o + i + 1, force->rate, force->seed));
  }
  RC(mtpx_target_verify(s->ctx, s->target, s->state, s->ids, k + 1, s->logits, s->multi, nullptr));
  if (temperature > 0.0f)
    RC(mtpx_accept_sample_bf16(s->ctx, s->logits, nullptr, k, s->vocab, s->ids + 1, temperature, seed, (uint64_t)o,
                               (int32_t)o, s->out, s->out + 12));
  else
    RC(mtpx_accept_greedy_bf16(s->ctx, s->logits, k, s->vocab, s->ids + 1, (int32_t)o, s->out, s->out + 4,
                               s->out + 12));
  RC(readback(s));
  const int n = s->host[0];
  if (n < 0 || n > k) return set_error(MTPX_ERR_STATE, "round: accept count out of range");
  RC(mtpx_target_commit(s->state, n + 1));
  if (s->drafter.ctx) {
    if (k > 0) {
      RC(mtpx_drafter_finalize(s->drafter, n + 1, n ? s->ids + 1 : nullptr, n ? s->multi : nullptr, n));
    } else {
      // A drafted round leaves no frontier: its carry (the multi stream before the carry token)
      // is paired with the token only by the next round's first draft step.  A serial step
      // observes the carry token instead, so the carry's stream becomes the frontier first;
      // otherwise the transition (carry stream, carry token) would never reach the head.
      mtpx_drafter_info di;
      RC(mtpx_drafter_info_get(s->drafter, &di));
      if (!di.has_frontier) RC(mtpx_drafter_observe(s->drafter, s->ids, s->carry, 1));
      RC(mtpx_drafter_observe(s->drafter, s->ids, s->multi, 1));
    }
  }
  RC(next_carry(s, s->multi, n));
  s->offset += n + 1;
  std::memcpy(tokens, s->host + 12, 4 * (size_t)(n + 1));
  *n_tokens = n + 1;
  return MTPX_OK;
}

int mtpx_session_info(mtpx_session sh, int64_t* offset, mtpx_target_state* state, mtpx_drafter* drafter) {
  Session* s = static_cast<Session*>(sh.ctx);
  if (!s) return set_error(MTPX_ERR_ARG, "session: null");
  if (offset) *offset = s->offset;
  if (state) *state = s->state;
  if (drafter) *drafter = s->drafter;
  return MTPX_OK;
}

}  // extern "C"
