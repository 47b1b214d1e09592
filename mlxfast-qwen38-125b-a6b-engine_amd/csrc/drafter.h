// Request state of the MTP drafter: the trusted target transitions not yet in
// the head's cache (backlog), the round in flight, and the head cache geometry
// around it.  One instance per request; not re-entrant.
//
// A transition pairs the target's multi stream at position t with the token at
// t+1.  A round begins with the first draft step, which flushes the backlog
// plus the current target carry through the head (trusted history); every
// later step of the round is speculative and is trimmed when the round ends.
// finalize keeps the committed drafts as new trusted transitions (paired with
// the target's own multi streams, never the head's); discard restores every
// trusted transition the round consumed, in order.
//
// Backend (the storage and the head; device memory for the library, host
// memory for the CPU test):
//   using Rows = ...;   movable: n token ids + n hidden rows
//   Rows make(const int32_t* tok, const uint16_t* hid, int n);   // copies n rows
//                                                                 // (tok may be null)
//   static int count(const Rows&); const int32_t* tok(const Rows&);
//   const uint16_t* hid(const Rows&);
//   int head(const std::vector<const Rows*>& segs, int32_t* draft, uint16_t* multi);
//       runs the head over the rows of segs in order at the cache offset; the
//       last row's draft id and multi stream go to draft / multi
//   int64_t offset();  int64_t trim(int64_t n);  // head cache
//   bool ok(const Rows&);                           // allocation succeeded
//
// Reference: Runner/Qwen4ExpMTPDrafter.swift:162-249 (RequestState), :277-279
// (makeRequestState), :288-316 (observeCommittedTarget), :328-366 (draftStep),
// :368-397 (beginRound), :410-441 (finalizeRound), :443-454 (discardRound),
// :461-470 (trim), :472-475 (releaseRequestState).
#pragma once
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace mtpx {

constexpr int DRAFT_MAX_DEPTH = 6;  // TrackQwen4ExpInlineMTPAssistant.maximumDepth

enum DrafterStatus { DR_OK = 0, DR_ERR_ARG = 1, DR_ERR_BACKEND = 2, DR_ERR_STATE = 3 };

template <class Backend>
class Drafter {
 public:
  using Rows = typename Backend::Rows;

  explicit Drafter(Backend& be) : be_(be) { clear_round(); }

  const std::string& error() const { return err_; }

  // ---- introspection (RequestState's derived counts)
  int64_t cache_offset() { return be_.offset(); }
  int64_t backlog_inputs() const {
    int64_t n = 0;
    for (const Rows& r : backlog_) n += Backend::count(r);
    return n;
  }
  int64_t committed_inputs() { return (in_flight_ ? valid_offset_ : cache_offset()) + backlog_inputs(); }
  int64_t staged_inputs() {
    if (!in_flight_) return 0;
    const int64_t d = cache_offset() - valid_offset_;
    return d > 0 ? d : 0;
  }
  bool in_flight() const { return in_flight_; }
  int draft_steps() const { return steps_; }
  int64_t round_base_offset() const { return base_offset_; }
  int64_t round_valid_offset() const { return valid_offset_; }
  bool has_frontier() const { return has_frontier_; }
  bool released() const { return released_; }

  // ---- observeCommittedTarget: n target inputs (tokens) with their multi streams
  int observe(const int32_t* tok, const uint16_t* hid, int n, int W) {
    if (released_) return fail(DR_ERR_STATE, "observed released request state");
    if (in_flight_) return fail(DR_ERR_STATE, "observed target during a round");
    if (n < 0 || (n > 0 && (!tok || !hid))) return fail(DR_ERR_ARG, "target observation shape mismatch");
    if (n == 0) return DR_OK;
    // cross-chunk transition: the previous chunk's last multi pairs with this chunk's first token
    if (has_frontier_) {
      Rows r = be_.make(tok, Backend::hid(frontier_), 1);
      if (!be_.ok(r)) return fail(DR_ERR_BACKEND, "row storage");
      backlog_.push_back(std::move(r));
    }
    // intra-chunk transitions: multi[t] conditions token[t+1]
    if (n > 1) {
      Rows r = be_.make(tok + 1, hid, n - 1);
      if (!be_.ok(r)) return fail(DR_ERR_BACKEND, "row storage");
      backlog_.push_back(std::move(r));
    }
    frontier_ = be_.make(nullptr, hid + (size_t)(n - 1) * W, 1);
    if (!be_.ok(frontier_)) return fail(DR_ERR_BACKEND, "row storage");
    has_frontier_ = true;
    return DR_OK;
  }

  // ---- draftStep: one token and its multi stream -> the draft id and the head's multi stream
  int step(const int32_t* tok, const uint16_t* hid, int32_t* draft, uint16_t* multi) {
    if (released_) return fail(DR_ERR_STATE, "drafted with released request state");
    if (!tok || !hid) return fail(DR_ERR_ARG, "draft input shape mismatch");
    const bool first = !in_flight_;
    int rc;
    if (first) {
      if ((rc = begin_round(tok, hid))) return rc;
      std::vector<const Rows*> segs;
      for (const Rows& r : trusted_) segs.push_back(&r);
      if ((rc = be_.head(segs, draft, multi))) return fail(DR_ERR_BACKEND, "head step failed");
    } else {
      if (steps_ >= DRAFT_MAX_DEPTH) return fail(DR_ERR_STATE, "exceeded the draft chain depth");
      Rows r = be_.make(tok, hid, 1);
      if (!be_.ok(r)) return fail(DR_ERR_BACKEND, "row storage");
      std::vector<const Rows*> segs{&r};
      if ((rc = be_.head(segs, draft, multi))) return fail(DR_ERR_BACKEND, "head step failed");
    }
    steps_ += 1;
    // the trusted flush ends with the first step; later inputs are speculative
    if (first) valid_offset_ = cache_offset();
    return DR_OK;
  }

  // ---- finalizeRound
  int finalize(int confirmed, const int32_t* tok, const uint16_t* hid, int n) {
    if (released_) return fail(DR_ERR_STATE, "finalized released request state");
    if (!in_flight_) return fail(DR_ERR_STATE, "finalized without a round");
    if (confirmed < 0 || confirmed > steps_ + 1) return fail(DR_ERR_STATE, "confirmed prefix exceeds the draft round");
    if (n < 0 || (n > 0 && (!tok || !hid))) return fail(DR_ERR_ARG, "committed target rows mismatch");
    const int lim = confirmed - 1 > 0 ? confirmed - 1 : 0;
    if (n > steps_ || n > lim) return fail(DR_ERR_STATE, "committed drafts exceed confirmed target inputs");
    int rc = trim_to(valid_offset_);
    if (rc) return rc;
    if (n > 0) {
      // target verify multi streams, never speculative head outputs; they flush with the next carry
      Rows r = be_.make(tok, hid, n);
      if (!be_.ok(r)) return fail(DR_ERR_BACKEND, "row storage");
      backlog_.push_back(std::move(r));
    }
    clear_round();
    return DR_OK;
  }

  // ---- discardRound (no round in flight, or released: nothing to do)
  int discard() {
    if (released_ || !in_flight_) return DR_OK;
    int rc = trim_to(base_offset_);
    if (rc) return rc;
    // restore every trusted transition the abandoned round consumed, in original order
    std::vector<Rows> restored;
    for (Rows& r : trusted_) restored.push_back(std::move(r));
    for (Rows& r : backlog_) restored.push_back(std::move(r));
    backlog_ = std::move(restored);
    clear_round();
    return DR_OK;
  }

  // ---- releaseRequestState
  void release() {
    backlog_.clear();
    trusted_.clear();
    frontier_ = Rows();
    has_frontier_ = false;
    base_offset_ = valid_offset_ = 0;
    steps_ = 0;
    in_flight_ = false;
    released_ = true;
  }

 private:
  int begin_round(const int32_t* tok, const uint16_t* hid) {
    base_offset_ = cache_offset();
    valid_offset_ = base_offset_;
    steps_ = 0;
    in_flight_ = true;
    trusted_ = std::move(backlog_);
    backlog_.clear();
    // the current target carry is trusted and completes the frontier transition
    Rows r = be_.make(tok, hid, 1);
    if (!be_.ok(r)) {
      in_flight_ = false;
      backlog_ = std::move(trusted_);
      trusted_.clear();
      return fail(DR_ERR_BACKEND, "row storage");
    }
    trusted_.push_back(std::move(r));
    frontier_ = Rows();
    has_frontier_ = false;
    return DR_OK;
  }

  int trim_to(int64_t off) {
    const int64_t rollback = cache_offset() - off;
    if (rollback < 0) return fail(DR_ERR_STATE, "cache checkpoint moved forward");
    if (rollback == 0) return DR_OK;
    if (be_.trim(rollback) != rollback) return fail(DR_ERR_STATE, "head cache refused the rollback");
    return DR_OK;
  }

  void clear_round() {
    base_offset_ = cache_offset();
    valid_offset_ = base_offset_;
    steps_ = 0;
    in_flight_ = false;
    trusted_.clear();
  }

  int fail(int code, const char* msg) {
    err_ = std::string("MTP drafter: ") + msg;
    return code;
  }

  Backend& be_;
  std::vector<Rows> backlog_;
  std::vector<Rows> trusted_;
  Rows frontier_{};
  bool has_frontier_ = false;
  int64_t base_offset_ = 0, valid_offset_ = 0;
  int steps_ = 0;
  bool in_flight_ = false;
  bool released_ = false;
  std::string err_;
};

}  // namespace mtpx
