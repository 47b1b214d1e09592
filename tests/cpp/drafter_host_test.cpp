// CPU test of the drafter's round state machine (csrc/drafter.h) with a host
// backend whose "head" records every input row it is given.  Built and run by
// tests/test_drafter_cpu.py; exits non-zero with a message on the first failure.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "drafter.h"

using namespace mtpx;

static const int W = 4;

struct HostBackend {
  struct Rows {
    std::vector<int32_t> t;
    std::vector<uint16_t> h;
    int n = 0;
  };
  int64_t off = 0;
  std::vector<std::vector<int32_t>> calls_tok;   // tokens of every head call
  std::vector<std::vector<uint16_t>> calls_hid;  // hidden[row][0] of every head call

  Rows make(const int32_t* tok, const uint16_t* hid, int n) {
    Rows r;
    r.n = n;
    if (tok)
      r.t.assign(tok, tok + n);
    else
      r.t.assign(n, -1);
    r.h.assign(hid, hid + (size_t)n * W);
    return r;
  }
  static int count(const Rows& r) { return r.n; }
  static const int32_t* tok(const Rows& r) { return r.t.data(); }
  static const uint16_t* hid(const Rows& r) { return r.h.data(); }
  bool ok(const Rows&) const { return true; }
  int head(const std::vector<const Rows*>& segs, int32_t* draft, uint16_t* multi) {
    std::vector<int32_t> ts;
    std::vector<uint16_t> hs;
    for (const Rows* r : segs)
      for (int i = 0; i < r->n; ++i) {
        ts.push_back(r->t[i]);
        hs.push_back(r->h[(size_t)i * W]);
      }
    off += (int64_t)ts.size();
    *draft = 1000 + ts.back();
    for (int k = 0; k < W; ++k) multi[k] = (uint16_t)(hs.back() + 500);
    calls_tok.push_back(ts);
    calls_hid.push_back(hs);
    return 0;
  }
  int64_t offset() { return off; }
  int64_t trim(int64_t n) {
    const int64_t t = n < off ? n : off;
    off -= t;
    return t;
  }
};

static int fails = 0;
#define EXPECT(c)                                                   \
  do {                                                              \
    if (!(c)) {                                                     \
      fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #c); \
      ++fails;                                                      \
    }                                                               \
  } while (0)

// n rows whose first element is v0, v0+1, ...
static std::vector<uint16_t> rows(int n, int v0) {
  std::vector<uint16_t> h((size_t)n * W);
  for (int i = 0; i < n; ++i)
    for (int k = 0; k < W; ++k) h[(size_t)i * W + k] = (uint16_t)(v0 + i);
  return h;
}

static bool eq(const std::vector<int32_t>& a, std::vector<int32_t> b) { return a == b; }
static bool eqh(const std::vector<uint16_t>& a, std::vector<uint16_t> b) { return a == b; }

int main() {
  HostBackend be;
  Drafter<HostBackend> d(be);
  int32_t draft = 0;
  uint16_t multi[W];

  // observe one chunk: transitions (h0,11) (h1,12) (h2,13); frontier h3
  {
    int32_t t[4] = {10, 11, 12, 13};
    auto h = rows(4, 100);
    EXPECT(d.observe(t, h.data(), 4, W) == DR_OK);
  }
  EXPECT(d.backlog_inputs() == 3 && d.has_frontier() && d.committed_inputs() == 3 && d.cache_offset() == 0);
  // cross-chunk: the frontier h3 pairs with the next chunk's first token 14
  {
    int32_t t[2] = {14, 15};
    auto h = rows(2, 200);
    EXPECT(d.observe(t, h.data(), 2, W) == DR_OK);
  }
  EXPECT(d.backlog_inputs() == 5 && d.committed_inputs() == 5);
  EXPECT(d.observe(nullptr, nullptr, 0, W) == DR_OK);  // empty observation: no change
  EXPECT(d.backlog_inputs() == 5);

  // round 1, first step: backlog + carry (16, h=300) flushed through the head
  {
    int32_t t = 16;
    auto h = rows(1, 300);
    EXPECT(d.step(&t, h.data(), &draft, multi) == DR_OK);
  }
  EXPECT(be.calls_tok.size() == 1);
  EXPECT(eq(be.calls_tok[0], {11, 12, 13, 14, 15, 16}));
  EXPECT(eqh(be.calls_hid[0], {100, 101, 102, 103, 200, 300}));
  EXPECT(draft == 1016 && multi[0] == 800);
  EXPECT(d.in_flight() && d.draft_steps() == 1 && d.cache_offset() == 6 && d.round_base_offset() == 0 &&
         d.round_valid_offset() == 6 && d.backlog_inputs() == 0 && !d.has_frontier());
  EXPECT(d.staged_inputs() == 0 && d.committed_inputs() == 6);
  // observing during a round is refused
  {
    int32_t t = 1;
    auto h = rows(1, 1);
    EXPECT(d.observe(&t, h.data(), 1, W) == DR_ERR_STATE);
  }
  // chained speculative steps
  for (int i = 0; i < 2; ++i) {
    int32_t t = draft;
    EXPECT(d.step(&t, multi, &draft, multi) == DR_OK);
  }
  EXPECT(eq(be.calls_tok[1], {1016}) && eq(be.calls_tok[2], {2016}));
  EXPECT(d.draft_steps() == 3 && d.cache_offset() == 8 && d.staged_inputs() == 2 && d.committed_inputs() == 6);
  // finalize argument checks (the state stays as it was)
  {
    int32_t t[3] = {1016, 2016, 3016};
    auto h = rows(3, 400);
    EXPECT(d.finalize(5, t, h.data(), 1) == DR_ERR_STATE);  // confirmed > steps + 1
    EXPECT(d.finalize(2, t, h.data(), 2) == DR_ERR_STATE);  // committed > confirmed - 1
    EXPECT(d.finalize(4, t, h.data(), 4) == DR_ERR_STATE);  // committed > steps
    EXPECT(d.in_flight() && d.cache_offset() == 8);
    // accept one draft: the head cache rolls back to the trusted flush, the
    // committed draft joins the backlog with the target's multi stream
    EXPECT(d.finalize(2, t, h.data(), 1) == DR_OK);
  }
  EXPECT(!d.in_flight() && d.cache_offset() == 6 && d.backlog_inputs() == 1 && d.committed_inputs() == 7);
  EXPECT(d.round_base_offset() == 6 && d.round_valid_offset() == 6 && d.draft_steps() == 0);
  EXPECT(d.finalize(1, nullptr, nullptr, 0) == DR_ERR_STATE);  // no round in flight

  // round 2: flush = committed draft (1016, h400) + carry (17, h500); then discard
  {
    int32_t t = 17;
    auto h = rows(1, 500);
    EXPECT(d.step(&t, h.data(), &draft, multi) == DR_OK);
  }
  EXPECT(eq(be.calls_tok[3], {1016, 17}) && eqh(be.calls_hid[3], {400, 500}));
  EXPECT(d.cache_offset() == 8);
  {
    int32_t t = draft;
    EXPECT(d.step(&t, multi, &draft, multi) == DR_OK);
  }
  EXPECT(d.cache_offset() == 9);
  EXPECT(d.discard() == DR_OK);
  // every trusted transition of the abandoned round is back, in order
  EXPECT(!d.in_flight() && d.cache_offset() == 6 && d.backlog_inputs() == 2 && d.committed_inputs() == 8);
  EXPECT(d.discard() == DR_OK);  // nothing in flight: no-op
  {
    int32_t t = 18;
    auto h = rows(1, 600);
    EXPECT(d.step(&t, h.data(), &draft, multi) == DR_OK);
  }
  EXPECT(eq(be.calls_tok[5], {1016, 17, 18}) && eqh(be.calls_hid[5], {400, 500, 600}));
  // depth ceiling: steps 2..6 fine, the 7th refused
  for (int i = 2; i <= DRAFT_MAX_DEPTH; ++i) {
    int32_t t = draft;
    EXPECT(d.step(&t, multi, &draft, multi) == DR_OK);
  }
  {
    int32_t t = draft;
    EXPECT(d.step(&t, multi, &draft, multi) == DR_ERR_STATE);
  }
  EXPECT(d.draft_steps() == DRAFT_MAX_DEPTH);
  // reject everything: confirmed 1 (only the carry), nothing committed
  EXPECT(d.finalize(1, nullptr, nullptr, 0) == DR_OK);
  EXPECT(d.cache_offset() == 9 && d.backlog_inputs() == 0 && d.committed_inputs() == 9);

  // serial steps after a drafted round, as the session's depth-0 round drives them: the round left
  // no frontier, so the carry (19, its stream 700) is observed first to make 700 the frontier,
  // then the carry token with the verify's stream 710 pairs (700, 19) into the backlog
  EXPECT(!d.has_frontier());
  {
    int32_t t = 19;
    auto carry = rows(1, 700);
    auto verify = rows(1, 710);
    EXPECT(d.observe(&t, carry.data(), 1, W) == DR_OK);
    EXPECT(d.backlog_inputs() == 0 && d.has_frontier());
    EXPECT(d.observe(&t, verify.data(), 1, W) == DR_OK);
  }
  EXPECT(d.backlog_inputs() == 1 && d.committed_inputs() == 10);
  {
    int32_t t = 20;  // the next serial step: the frontier exists, one observation
    auto verify = rows(1, 720);
    EXPECT(d.observe(&t, verify.data(), 1, W) == DR_OK);
  }
  EXPECT(d.backlog_inputs() == 2 && d.committed_inputs() == 11);
  {
    int32_t t = 21;  // a drafted round again: its flush holds every serial transition and the carry
    auto h = rows(1, 720);
    EXPECT(d.step(&t, h.data(), &draft, multi) == DR_OK);
  }
  EXPECT(eq(be.calls_tok.back(), {19, 20, 21}) && eqh(be.calls_hid.back(), {700, 710, 720}));
  EXPECT(d.finalize(1, nullptr, nullptr, 0) == DR_OK);
  EXPECT(d.cache_offset() == 12 && d.committed_inputs() == 12);

  // release: every later call is refused, discard stays a no-op
  d.release();
  {
    int32_t t = 1;
    auto h = rows(1, 1);
    EXPECT(d.observe(&t, h.data(), 1, W) == DR_ERR_STATE);
    EXPECT(d.step(&t, h.data(), &draft, multi) == DR_ERR_STATE);
    EXPECT(d.finalize(1, nullptr, nullptr, 0) == DR_ERR_STATE);
    EXPECT(d.discard() == DR_OK);
  }
  if (fails) {
    fprintf(stderr, "%d failure(s)\n", fails);
    return 1;
  }
  printf("drafter host test: ok\n");
  return 0;
}
