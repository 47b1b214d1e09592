// The MoE block of the decode/verify window (M <= 8 tokens), three launches:
//   router+route: bf16 router GEMV (+ shared-expert gate row) over f32(x) and
//            the activation block preparation of x; the last row workgroup to
//            finish (ticket) runs the route: top-k (value desc, index asc) +
//            softmax, and the expert-grouped dispatch table (each selected
//            expert once, with its tokens)
//   gate_up: one workgroup per CU over the (slot, 32-row block of F) items,
//            slot = the shared expert of one token or one routed (token,
//            rank) pair: gate and up rows against that token, SwiGLU -> bf16
//            activations per slot
//   down   : the same layout over (slot, block of H) items: block preparation
//            of the slot's activations, down rows against them -> routed/
//            shared outputs per slot
// The expert kernels stream the weights with the next item's loads in flight
// while the current item is computed; the distinct-expert count of the
// dispatch table is what the window reads from HBM (an expert chosen by two
// tokens is read twice, the second time from cache).
//   combine: per (token, 256 rows of H): fold the routed outputs in rank order,
//            add the sigmoid-gated shared expert (MLX col_reduce_small
//            association), optionally add the residual stream
// The ticket is a u32 counter that is zero at rest: the last arriver of a
// launch puts it back to zero.  What it publishes (the router logits) is
// written and read with agent-scope atomic stores/loads, which go
// to the device-coherent level; each thread waits for its stores to complete
// before the workgroup barrier that precedes the ticket, so no cache-wide
// writeback or invalidate is needed.
// Reference: FM/TrackFastModel.swift:867-954 (orchestration),
// FM/TrackFastMoE.swift:2490-2638 (router + route in one launch with a
// last-arriver ticket), :780-911 (route), :1192-1404 (gate|up+act),
// :1412-1576 (down+combine), :2246-2310 (router GEMV),
// FM/TrackFastKernels2.swift:21-58,512-544 (sigmoid, colsum fold, combine).
#include <algorithm>

#include "qrows.h"

namespace mtpx {

// ---------------------------------------------------------------------------
// route (run by one workgroup of RR_THREADS threads): wave m selects token m's
// top-k (a threshold search over order-preserving integer keys, wave ballots
// counting the keys above each candidate) and its softmax; then the dispatch table is built in LDS by
// the threads of the M*K slots: each expert once (ordered by its first (token,
// rank) slot), with its slots ordered by token.  No serial loop over slots or
// experts: leaders by an LDS minimum, expert offsets by a wave scan.

// Window w of a batched launch (grid dimension w, a.nwin windows of a.M tokens): the pointers of
// its tokens and slots, its dispatch table and its ticket.
__device__ __forceinline__ MoeArgs moe_window(MoeArgs a, int w) {
  if (w == 0) return a;
  const size_t t = (size_t)w * a.M, sl = t * (a.K + 1);
  a.x += t * a.H;
  if (a.y) a.y += t * a.H;
  a.logits += t * a.E;
  a.gate_logit += t;
  a.idx += t * a.K;
  a.w += t * a.K;
  a.disp += w;
  a.xp_x += t * (a.H / 32) * XP_DW;
  a.act += sl * a.F;
  a.r += sl * a.H;
  if (a.resid) a.resid += t * a.H;
  if (a.y2) a.y2 += t * a.H;
  a.ticket += w;
  if (a.nu_out) a.nu_out += w;
  return a;
}
constexpr int RR_THREADS = 512;
static_assert(MAX_TOKENS * MAX_TOPK <= 128, "the slots fit the first two waves");

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Order-preserving key of a router logit: key(a) > key(b) exactly when a > b as floats, -0 and +0
// share a key, and a NaN logit ranks as -inf.  Key 0, below every logit, marks the lanes past E.
__device__ __forceinline__ uint32_t route_key(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u << 1) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// lanes below this one set in m
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// keys >= t over the wave's EPER key registers: one ballot and popcount per register
template <int EPER>
__device__ __forceinline__ int route_count_ge(const uint32_t (&key)[EPER], uint32_t t) {
  int n = 0;
#pragma unroll
  for (int j = 0; j < EPER; ++j) n += __popcll(__ballot(key[j] >= t));
  return n;
}

// EPER = ceil(E / 64) rounded up to 8 or 16: the logits per lane (expert lane + 64 j in register j).
// POLL: the logits come from the publish buffer a.pub, each token's wave loading them until none is
// the sentinel (at most ROUTE_SPIN polls), then copying them to a.logits and putting the sentinel
// back for the next launch; else from a.logits, complete (the ticket).
template <int EPER, bool POLL>
__device__ void route_body(const MoeArgs& a) {
  const int E = a.E, K = a.K, M = a.M;
  const int MK = M * K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ int sel[MAX_TOKENS * MAX_TOPK];
  __shared__ int first[1024];
  __shared__ uint32_t tokbits[MAX_TOKENS][32];  // expert membership per token
  __shared__ uint64_t leadmask[2];
  __shared__ int wtot[2];
  __shared__ int uid[MAX_TOKENS * MAX_TOPK];
  __shared__ int pre[MAX_TOKENS * MAX_TOPK];
  __shared__ uint32_t ckey[MAX_TOKENS][MAX_TOPK];  // the selected of each token, in expert order
  __shared__ int cidx[MAX_TOKENS][MAX_TOPK];
  __shared__ float cval[MAX_TOKENS][MAX_TOPK];
  for (int i = threadIdx.x; i < E; i += blockDim.x) first[i] = 0x7fffffff;
  for (int i = threadIdx.x; i < MAX_TOKENS * 32; i += blockDim.x) (&tokbits[0][0])[i] = 0u;
  if (wave < M) {
    float x[EPER];
    if constexpr (POLL) {
      float* pr = a.pub + (size_t)wave * E;
      for (int spin = 0; spin < ROUTE_SPIN; ++spin) {
        bool ready = true;
#pragma unroll
        for (int j = 0; j < EPER; ++j) {
          const int e = lane + 64 * j;
          x[j] = (e < E) ? ld_pub(pr + e) : 0.0f;
          ready = ready && (e >= E || __float_as_uint(x[j]) != ROUTE_SENTINEL);
        }
        if (__all(ready)) break;
      }
#pragma unroll
      for (int j = 0; j < EPER; ++j) {
        const int e = lane + 64 * j;
        if (e < E) {
          a.logits[(size_t)wave * E + e] = x[j];
          pr[e] = __uint_as_float(ROUTE_SENTINEL);
        }
      }
    } else {
      const float* lr = a.logits + (size_t)wave * E;
#pragma unroll
      for (int j = 0; j < EPER; ++j) {
        const int e = lane + 64 * j;
        x[j] = (e < E) ? ld_pub(lr + e) : 0.0f;
      }
    }
    float v[EPER];
    uint32_t key[EPER];
#pragma unroll
    for (int j = 0; j < EPER; ++j) {
      const int e = lane + 64 * j;
      v[j] = (e < E && x[j] == x[j]) ? x[j] : -__uint_as_float(0x7f800000u);  // a NaN logit ranks as -inf
      key[j] = e < E ? route_key(v[j]) : 0u;
    }
    // T: the K-th largest key, the largest t with at least K keys >= t, found bit by bit from the
    // top.  A count of exactly K ends the search early: t then parts the K largest from the rest.
    // T >= key(-inf) > 0 (K <= E), so no lane past E is selected.
    uint32_t T = 0u;
    for (int b = 31; b >= 0; --b) {
      const uint32_t c = T | (1u << b);
      const int n = route_count_ge<EPER>(key, c);
      if (n >= K) {
        T = c;
        if (n == K) break;
      }
    }
    // selected: every key above T, and of the keys equal to T the lowest experts, K in all
    // (value descending, expert ascending); compacted into LDS in expert order
    const int need = K - route_count_ge<EPER>(key, T + 1u);
    int ties = 0, before = 0;
#pragma unroll
    for (int j = 0; j < EPER; ++j) {
      const uint64_t eq = __ballot(key[j] == T);
      const bool s = key[j] > T || (key[j] == T && ties + lanes_below(eq) < need);
      const uint64_t sm = __ballot(s);
      if (s) {
        const int p = before + lanes_below(sm);
        ckey[wave][p] = key[j];
        cidx[wave][p] = lane + 64 * j;
        cval[wave][p] = v[j];
      }
      ties += __popcll(eq);
      before += __popcll(sm);
    }
    // the wave reads what it wrote (LDS operations of one wave complete in order)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // lane p < K: entry p's rank among the K, then each entry pushed to the lane of its rank
    int rank = lane;
    float pv = 0.0f;
    int pe = 0;
    if (lane < K) {
      const uint32_t kp = ckey[wave][lane];
      rank = 0;
      for (int q = 0; q < K; ++q) {
        const uint32_t kq = ckey[wave][q];
        rank += (kq > kp || (kq == kp && q < lane)) ? 1 : 0;
      }
      pv = cval[wave][lane];
      pe = cidx[wave][lane];
    }
    // lane k < K: the k-th selected logit and expert
    const float myv = __int_as_float(__builtin_amdgcn_ds_permute(rank * 4, __float_as_int(pv)));
    const int mys = __builtin_amdgcn_ds_permute(rank * 4, pe);
    // softmax over the K selected: exp per lane, sum in rank order (lane values read uniformly)
    const float ev = expf_det(myv - readlane_f(myv, 0));
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum = sum + readlane_f(ev, k);
    sum = 1.0f / sum;
    if (lane < K) {
      sel[wave * K + lane] = mys;
      a.idx[wave * K + lane] = mys;
      a.w[wave * K + lane] = ev * sum;
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  int e = 0;
  if (t < MK) {
    e = sel[t];
    atomicMin(&first[e], t);
    atomicOr(&tokbits[t / K][e >> 5], 1u << (e & 31));
  }
  __syncthreads();
  // leaders (first slot of an expert) in slot order = experts in dispatch order; each leader's
  // token count, and the exclusive scan of the counts over the slots (waves 0 and 1)
  const bool leader = t < MK && first[e] == t;
  int count = 0;
  if (leader)
    for (int m = 0; m < M; ++m) count += (tokbits[m][e >> 5] >> (e & 31)) & 1u;
  int incl = count;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  const uint64_t bal = __ballot(leader);
  if (wave < 2) {
    if (lane == 0) leadmask[wave] = bal;
    if (lane == 63) wtot[wave] = incl;
  }
  __syncthreads();
  MoeDispatch* d = a.disp;
  const int n = __popcll(leadmask[0]) + (MK > 64 ? __popcll(leadmask[1]) : 0);
  if (leader) {
    const uint64_t below = (t & 63) ? (leadmask[t >> 6] & ((~0ull) >> (64 - (t & 63)))) : 0ull;
    const int u = __popcll(below) + (t >= 64 ? __popcll(leadmask[0]) : 0);
    uid[t] = u;
    pre[u] = M + incl - count + (t >= 64 ? wtot[0] : 0);  // slots before expert u, shared ones first
    d->expert[u + 1] = e;
    d->count[u + 1] = count;
  }
  __syncthreads();
  if (t < MK) {
    const int u = uid[first[e]];
    int pos = 0;
    for (int m = 0; m < t / K; ++m) pos += (tokbits[m][e >> 5] >> (e & 31)) & 1u;
    d->slot[u + 1][pos] = (int16_t)t;
    d->order[pre[u] + pos] = t | ((e + 1) << 16);
    if (t + 1 > n) d->expert[t + 1] = -2;  // grid rows past the routed experts: no work
  }
  if (t == 0) {
    d->n_unique = n;
    if (a.nu_out) *a.nu_out = n;
    d->expert[0] = -1;
    d->count[0] = M;
    for (int m = 0; m < M; ++m) {
      d->slot[0][m] = (int16_t)(MK + m);
      d->order[m] = MK + m;
    }
  }
}

// ---------------------------------------------------------------------------
// router + route: workgroups [0, row_wgs) hold one wave per router row (rows
// 0..E-1 router, row E the shared-expert gate); lane l walks 8-element chunks
// l, l+64, ...: acc = fmaf(w, x, acc) in element order, then an xor butterfly
// over the wave.  The window's activations are staged into LDS first, their
// loads in flight together with the weight rows' (read from global inside the
// token loop, each chunk would wait for its own round trip).  The remaining
// workgroups prepare x's activation blocks for the expert GEMVs (32 lanes per
// block) and take no ticket.
constexpr int ROUTER_IT = 8;  // H <= 8 * 64 * 8

// The shared-expert gate as a q4 row (GL lanes per token, the q4 GEMV's lane rule for K = H): the
// workgroup after the row and preparation workgroups issues the row's loads, prepares the window's
// activation blocks into LDS (32 lanes per block), then each group of GL lanes walks the row against
// one token and folds its lanes (the GEMV's chains and butterfly).  The value before the bf16
// rounding goes to gate_logit, which the combine rounds like the bf16 row's.  No ticket: the gate is
// first read by the combine launch.
template <int GL, int GIT>
__device__ __forceinline__ void shared_gate_q4(const MoeArgs& a, uint32_t* __restrict__ xpl) {
  const int H = a.H, M = a.M, nb = H / 32;
  const int grp = (int)threadIdx.x / GL, sub = (int)threadIdx.x % GL;
  QRow<GL, GIT> R;
  R.load(a.sg_w, a.sg_s, a.sg_b, a.sg_sb, nb, a.gs, sub, grp < M);
  asm volatile("" ::: "memory");
  const int i = threadIdx.x & 31;
  for (int blk = (int)(threadIdx.x >> 5); blk < M * nb; blk += RR_THREADS / 32)
    xprep_lanes_direct(a.x[(size_t)(blk / nb) * H + (size_t)(blk % nb) * 32 + i], i, xpl + (size_t)blk * XP_DW);
  __syncthreads();
  float v = R.dot(xpl + (size_t)(grp < M ? grp : 0) * nb * XP_DW, nb, sub);
  v = lane_fold<GL>(v);
  if (sub == 0 && grp < M) a.gate_logit[grp] = v;
}

// GL = 0: the gate is router row E (bf16); GL > 0: the q4 row, computed by the workgroup after the
// row and preparation workgroups.  route_wg >= 0 (one window): the grid's last workgroup routes,
// polling the publish buffer (dispatched last, every row workgroup is resident or done before it
// starts, so its wait ends); route_wg < 0: the last row workgroup to take the ticket routes.
template <int GL, int GIT>
__global__ __launch_bounds__(RR_THREADS) void k_moe_router_route(MoeArgs a0, int row_wgs, int route_wg) {
  const MoeArgs a = moe_window(a0, blockIdx.y);
  const int H = a.H, E = a.E, M = a.M;
  extern __shared__ uint4 xs[];  // [M, H/8] (the router rows); the gate workgroup: [M][H/32][XP_DW]
  if ((int)blockIdx.x == route_wg) {
    if (E <= 512)
      route_body<8, true>(a);
    else
      route_body<16, true>(a);
    return;
  }
  if constexpr (GL > 0) {
    if ((int)blockIdx.x == (route_wg >= 0 ? route_wg : (int)gridDim.x) - 1) {
      shared_gate_q4<GL, GIT>(a, reinterpret_cast<uint32_t*>(xs));
      return;
    }
  }
  if ((int)blockIdx.x >= row_wgs) {
    const int nb = H / 32;
    const int i = threadIdx.x & 31;
    const int blk = ((int)blockIdx.x - row_wgs) * (RR_THREADS / 32) + (int)(threadIdx.x >> 5);
    if (blk < M * nb)
      xprep_lanes_direct(a.x[(size_t)(blk / nb) * H + (size_t)(blk % nb) * 32 + i], i, a.xp_x + (size_t)blk * XP_DW);
    return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = blockIdx.x * (RR_THREADS / 64) + wave;
  const int nc = H / 8;
  const bool row_ok = GL > 0 ? r < E : r <= E;
  const bf16* wrow = (r < E) ? a.router + (size_t)r * H : a.shared_gate;
  uint4 wv[ROUTER_IT];
#pragma unroll
  for (int i = 0; i < ROUTER_IT; ++i) {
    const int c = lane + 64 * i;
    wv[i] = (row_ok && c < nc) ? *reinterpret_cast<const uint4*>(wrow + (size_t)c * 8) : make_uint4(0, 0, 0, 0);
  }
  // LDS-direct copies: no register round trip, one wait for all of them
  stage16(reinterpret_cast<uint32_t*>(xs), reinterpret_cast<const uint32_t*>(a.x), M * H / 2);
  stage_sync();
  if (row_ok) {
    for (int m = 0; m < M; ++m) {
      uint4 xr[ROUTER_IT];
#pragma unroll
      for (int i = 0; i < ROUTER_IT; ++i) {  // every chunk of the token read before the first use
        const int c = lane + 64 * i;
        xr[i] = xs[m * nc + (c < nc ? c : nc - 1)];
      }
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < ROUTER_IT; ++i) {
        const int c = lane + 64 * i;
        if (c < nc) {
          const uint4 xv = xr[i];
          const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
          const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            acc = __builtin_fmaf(__uint_as_float(ww[t] << 16), __uint_as_float(xx[t] << 16), acc);
            acc = __builtin_fmaf(__uint_as_float(ww[t] & 0xffff0000u), __uint_as_float(xx[t] & 0xffff0000u), acc);
          }
        }
      }
      acc = wave_fold64(acc);
      if (lane == 0) {
        if (r < E)
          st_pub((route_wg >= 0 ? a.pub : a.logits) + (size_t)m * E + r, acc);
        else
          a.gate_logit[m] = acc;
      }
    }
  }
  if (route_wg >= 0) return;
  if (!ticket_last(a.ticket, (uint32_t)row_wgs - 1u)) return;
  if (E <= 512)
    route_body<8, false>(a);
  else
    route_body<16, false>(a);
}


// ---------------------------------------------------------------------------
// gate|up + SwiGLU, one workgroup of GU_THREADS = 512 threads per CU over the
// work items of the window.  An item is (slot row r, 32-row block b of F),
// i = r * (F/32) + b, with slot rows 0..M-1 the shared expert for token r and
// rows M.. the routed slots t = m*K + k (expert idx[t], token m) -- one token
// per item, so every item is the same work (an expert chosen by two tokens is
// read twice, the second time from cache).  Workgroup w takes the contiguous
// items [w*n/G, (w+1)*n/G): at most F/32 of them, so at most two slot rows
// and two tokens.  Every wave owns RW = 64/L f rows of an item (gate and up).
// Order: the loads of the two tokens' activation blocks are issued first,
// then the weight loads of the first items, then the activation blocks are
// written to LDS (the memory counter retires loads in order, so this waits
// for the activations only).  Each wave then walks its items in straight-line
// code with GU_DEPTH register sets: the next item's loads are in flight while
// item k is computed.  Items past the range re-load the first one (loads are
// unconditional, so no register version merges) and are not computed.  The
// expert ids come through a restrict pointer: scalar loads, off the vector
// memory counter.  The output is the bf16 activation act[slot][F]; the down
// projection prepares its blocks.
constexpr int GU_THREADS = 512;
constexpr int GU_DEPTH = 2;  // register sets: the next item's loads are in flight
constexpr int GU_STAGE = 4;  // 16-byte staging loads per thread: 2 tokens x H/32 blocks x 7 <= 4 * 512

template <int L, int IT>
struct GateUpItem {
  QRow<L, IT> G, U;
  int slot, tok, f0;
};

// The gate and up matrices of the routed experts or of the shared expert.
struct GateUpMats {
  const uint32_t *gw, *uw, *gsb, *usb;
  const bf16 *gs, *gb, *us, *ub;
};

__device__ __forceinline__ int gu_token(int r, int M, int K) { return r < M ? r : (r - M) / K; }

// Issue the loads of item i into `it` (PK: packed scale/bias rows).  The
// pointer pairs are selected as values with a uniform condition.
template <int L, int IT, bool PK>
__device__ __forceinline__ void gate_up_load(const GateUpMats rm, const GateUpMats sm, int H, int F, int gs, int M,
                                             int K, const int32_t* __restrict__ ids, GateUpItem<L, IT>& it, int i,
                                             int nfb, int fi, bool valid, int sub) {
  const int nb = H / 32, ng = H / gs, P = sb_row_len(H, gs);
  const int r = i / nfb;
  it.f0 = (i % nfb) * 32;
  const bool shared = r < M;
  const int t = r - M;
  it.slot = shared ? M * K + r : t;
  it.tok = gu_token(r, M, K);
  const int e = shared ? 0 : ids[t];
  const int f = it.f0 + (valid ? fi : 0);
  const size_t row = shared ? (size_t)f : (size_t)e * F + f;
  const uint32_t* gw = shared ? sm.gw : rm.gw;
  const uint32_t* uw = shared ? sm.uw : rm.uw;
  const uint32_t* gsb = shared ? sm.gsb : rm.gsb;
  const uint32_t* usb = shared ? sm.usb : rm.usb;
  const bf16* gsc = shared ? sm.gs : rm.gs;
  const bf16* gbi = shared ? sm.gb : rm.gb;
  const bf16* usc = shared ? sm.us : rm.us;
  const bf16* ubi = shared ? sm.ub : rm.ub;
  it.G.template load_as<PK>(gw + row * (H / 8), gsc + row * ng, gbi + row * ng, PK ? gsb + row * P : nullptr, nb,
                            gs, sub, valid);
  it.U.template load_as<PK>(uw + row * (H / 8), usc + row * ng, ubi + row * ng, PK ? usb + row * P : nullptr, nb,
                            gs, sub, valid);
}

// gate and up of the item's rows against its token (LDS slot ts); SwiGLU.
template <int L, int IT>
__device__ __forceinline__ void gate_up_compute(const MoeArgs& a, GateUpItem<L, IT>& it,
                                                const uint32_t* __restrict__ xl, int ts, int fi, bool valid, int sub) {
  const int nb = a.H / 32;
  float g, up;
  dot2<L, IT, false>(it.G, it.U, xl + (size_t)ts * nb * XP_DW, nb, sub, g, up);
  g = lane_fold<L>(g);
  up = lane_fold<L>(up);
  if (sub == 0 && valid) a.act[(size_t)it.slot * a.F + it.f0 + fi] = f2bf(silu_bf16(round_bf(g)) * round_bf(up));
}

template <int L, int IT, bool PK, int NIT>
__global__ __launch_bounds__(GU_THREADS) void k_moe_gate_up(MoeArgs a0, const int32_t* __restrict__ ids) {
  const MoeArgs a = moe_window(a0, blockIdx.y);
  ids += (size_t)blockIdx.y * a0.M * a0.K;
  extern __shared__ uint32_t lds[];  // [2][H/32][XP_DW]
  constexpr int RW = 64 / L;         // f rows per wave
  constexpr int WAVES = GU_THREADS / 64;
  constexpr int NP = (32 + WAVES * RW - 1) / (WAVES * RW);  // passes over the 32 rows (L > 16: more than one)
  constexpr int D = NIT < GU_DEPTH ? NIT : GU_DEPTH;         // items in flight
  const int H = a.H, F = a.F, gs = a.gs, M = a.M, K = a.K;
  const int nb = H / 32, nfb = F / 32;
  const int n_items = (M + M * K) * nfb;
  const int G = gridDim.x;
  const int i0 = (int)(((int64_t)blockIdx.x * n_items) / G);
  const int n = (int)(((int64_t)(blockIdx.x + 1) * n_items) / G) - i0;  // 1 <= n <= NIT
  const int t0 = gu_token(i0 / nfb, M, K), t1 = gu_token((i0 + n - 1) / nfb, M, K);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const GateUpMats rm{a.gate_w, a.up_w, a.gate_sb, a.up_sb, a.gate_s, a.gate_b, a.up_s, a.up_b};
  const GateUpMats sm{a.sh_gate_w, a.sh_up_w, a.sh_gate_sb, a.sh_up_sb, a.sh_gate_s, a.sh_gate_b, a.sh_up_s, a.sh_up_b};
  auto item = [&](int k) { return k < n ? i0 + k : i0; };  // past the range: re-load the first item
  // activation loads of tokens t0 (LDS slot 0) and t1 (slot 1)
  const int n4 = nb * (XP_DW / 4);
  uint4 st[GU_STAGE];
#pragma unroll
  for (int q = 0; q < GU_STAGE; ++q) {
    const int u = threadIdx.x + q * GU_THREADS;
    const int tk = u < n4 ? t0 : t1, w = u < n4 ? u : u - n4;
    st[q] = u < 2 * n4 ? reinterpret_cast<const uint4*>(a.xp_x + (size_t)tk * nb * XP_DW)[w] : make_uint4(0, 0, 0, 0);
  }
  asm volatile("" ::: "memory");  // keep the activation loads ahead of the weight loads
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int fi = (wave + p * WAVES) * RW + grp;  // row of the 32-row block
    const bool live = (wave + p * WAVES) * RW < 32;  // uniform per wave: waves past the block have no rows
    const bool valid = fi < 32;
    GateUpItem<L, IT> S[D];
    // unconditional, also in waves without rows (they load a real row and never use it): a load
    // under a branch would merge register versions, and the copy would wait for the loads
#pragma unroll
    for (int k = 0; k + 1 < D; ++k)
      gate_up_load<L, IT, PK>(rm, sm, H, F, gs, M, K, ids, S[k], item(k), nfb, fi, valid, sub);
    asm volatile("" ::: "memory");  // and the first weight loads ahead of the barrier
    if (p == 0) {
#pragma unroll
      for (int q = 0; q < GU_STAGE; ++q) {
        const int u = threadIdx.x + q * GU_THREADS;
        if (u < 2 * n4) reinterpret_cast<uint4*>(lds)[u] = st[q];
      }
      __syncthreads();
    }
    if (!live) continue;
#pragma unroll
    for (int k = 0; k < NIT; ++k) {
      if (k + D - 1 < NIT)
        gate_up_load<L, IT, PK>(rm, sm, H, F, gs, M, K, ids, S[(k + D - 1) % D], item(k + D - 1), nfb, fi, valid, sub);
      S[k % D].G.opaque();  // retire this item's loads here, computed or not
      S[k % D].U.opaque();
      if (k < n) gate_up_compute(a, S[k % D], lds, S[k % D].tok == t0 ? 0 : 1, fi, valid, sub);
    }
  }
}

// ---------------------------------------------------------------------------
// combine: grid (ceil(H/256), M).  out = bf16(fold_k r_k*w_k) + bf16(sig(g)*shared);
// y = bf16(out) and, with a residual, y2 = bf16(resid + out).
__device__ __forceinline__ float colsum_small(const float* r, int K) {
  const int TY = K < 8 ? K : 8;
  float t[8];
  for (int y = 0; y < TY; ++y) {
    float acc = 0.0f;
    for (int rr = y; rr < K; rr += TY) acc = r[rr] + acc;
    t[y] = acc;
  }
  float total = t[0];
  for (int j = 1; j < TY; ++j) total = t[j] + total;
  return total;
}

// K is a template parameter so the K + 1 row loads are issued together and the
// fold is unrolled (a runtime-K loop waits for each load in turn).
template <int K>
__global__ __launch_bounds__(256) void k_moe_combine(MoeArgs a0) {
  const MoeArgs a = moe_window(a0, blockIdx.z);
  const int m = blockIdx.y, h = blockIdx.x * 256 + threadIdx.x;
  if (h >= a.H) return;
  const int H = a.H, M = a.M;
  float rv[K];
#pragma unroll
  for (int k = 0; k < K; ++k) rv[k] = bf2f(a.r[(size_t)(m * K + k) * H + h]);
  const float shv = bf2f(a.r[(size_t)(M * K + m) * H + h]);
  // the residual row with the others (unconditional: without one, an expert row is read and unused)
  const bf16 resb = (a.resid ? a.resid : a.r)[(size_t)m * H + h];
  asm volatile("" ::: "memory");
  float prod[K];
#pragma unroll
  for (int k = 0; k < K; ++k) prod[k] = rv[k] * a.w[m * K + k];
  const float rr = round_bf(colsum_small(prod, K));
  const float sg = sigmoid_bf16(round_bf(a.gate_logit[m]));
  const float sh = round_bf(sg * shv);
  const bf16 out = f2bf(rr + sh);
  if (a.y) a.y[(size_t)m * H + h] = out;
  if (a.y2) a.y2[(size_t)m * H + h] = f2bf(bf2f(resb) + bf2f(out));
}

// ---------------------------------------------------------------------------
// down, laid out like gate|up: one workgroup of DN_THREADS = 512 threads per
// CU over the items (slot row r, block of DR = WAVES * 2 * 64/L rows of H),
// slot rows as in gate|up (0..M-1 the shared expert of token r, then the
// routed slots); workgroup w takes a contiguous range of at most two slot
// rows.  Every lane-group owns two rows (each LDS read of an activation block
// feeds both).  Order: the bf16 activation loads of the (at most two) slots,
// then the first item's weight loads, then each 32-lane group prepares one
// activation block into LDS (waiting for the activations only), a barrier,
// and the straight-line walk with two register sets.
constexpr int DN_THREADS = 512;
constexpr int DN_STAGE = 8;  // activation elements per thread: 2 slots x F <= 8 * 512

template <int L, int IT>
struct DownItem {
  QRow<L, IT> A, B;
  int slot, h0;
};

struct DownMats {
  const uint32_t *w, *sb;
  const bf16 *s, *b;
};

__device__ __forceinline__ int dn_slot(int r, int M, int K) { return r < M ? M * K + r : r - M; }

template <int L, int IT, bool PK>
__device__ __forceinline__ void down_load(const DownMats rm, const DownMats sm, int H, int F, int gs, int M, int K,
                                          const int32_t* __restrict__ ids, DownItem<L, IT>& it, int i, int nhb, int hi,
                                          int sub) {
  constexpr int DR = (DN_THREADS / 64) * 2 * (64 / L);
  const int nb = F / 32, ng = F / gs, P = sb_row_len(F, gs);
  const int r = i / nhb;
  it.h0 = (i % nhb) * DR;
  const bool shared = r < M;
  it.slot = dn_slot(r, M, K);
  const int e = shared ? 0 : ids[r - M];
  const bool va = it.h0 + hi < H, vb = it.h0 + hi + 1 < H;
  const size_t base = shared ? 0 : (size_t)e * H;
  const size_t ra = base + (size_t)(va ? it.h0 + hi : it.h0), rb = base + (size_t)(vb ? it.h0 + hi + 1 : it.h0);
  const uint32_t* w = shared ? sm.w : rm.w;
  const uint32_t* sb = shared ? sm.sb : rm.sb;
  const bf16* sc = shared ? sm.s : rm.s;
  const bf16* bi = shared ? sm.b : rm.b;
  it.A.template load_as<PK>(w + ra * (F / 8), sc + ra * ng, bi + ra * ng, PK ? sb + ra * P : nullptr, nb, gs, sub, va);
  it.B.template load_as<PK>(w + rb * (F / 8), sc + rb * ng, bi + rb * ng, PK ? sb + rb * P : nullptr, nb, gs, sub, vb);
}

template <int L, int IT, bool PK, int NIT>
__global__ __launch_bounds__(DN_THREADS) void k_moe_down(MoeArgs a0, const int32_t* __restrict__ ids) {
  const MoeArgs a = moe_window(a0, blockIdx.y);
  ids += (size_t)blockIdx.y * a0.M * a0.K;
  extern __shared__ uint32_t lds[];  // [2][F/32][XP_DW]
  constexpr int RW = 64 / L;
  constexpr int DR = (DN_THREADS / 64) * 2 * RW;
  constexpr int D = NIT < 2 ? NIT : 2;  // items in flight
  const int H = a.H, F = a.F, gs = a.gs, M = a.M, K = a.K;
  const int nb = F / 32, nhb = (H + DR - 1) / DR;
  const int n_items = (M + M * K) * nhb;
  const int G = gridDim.x;
  const int i0 = (int)(((int64_t)blockIdx.x * n_items) / G);
  const int n = (int)(((int64_t)(blockIdx.x + 1) * n_items) / G) - i0;  // 1 <= n <= NIT
  const int s0 = dn_slot(i0 / nhb, M, K), s1 = dn_slot((i0 + n - 1) / nhb, M, K);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int hi = wave * 2 * RW + 2 * grp;  // first of this lane-group's two rows within the block
  const DownMats rm{a.down_w, a.down_sb, a.down_s, a.down_b};
  const DownMats sm{a.sh_down_w, a.sh_down_sb, a.sh_down_s, a.sh_down_b};
  auto item = [&](int k) { return k < n ? i0 + k : i0; };
  // activation element u = q * 512 + t: block u / 32 of slot s0 (blocks 0..nb-1) or s1 (nb..2nb-1)
  uint32_t hv[DN_STAGE];
#pragma unroll
  for (int q = 0; q < DN_STAGE; ++q) {
    const int u = (int)threadIdx.x + q * DN_THREADS, bq = u >> 5;
    const int sl = bq < nb ? s0 : s1, b = bq < nb ? bq : bq - nb;
    hv[q] = bq < 2 * nb ? a.act[(size_t)sl * F + b * 32 + (u & 31)] : 0u;
  }
  asm volatile("" ::: "memory");  // activation loads ahead of the weight loads
  DownItem<L, IT> S[D];
#pragma unroll
  for (int k = 0; k + 1 < D; ++k) down_load<L, IT, PK>(rm, sm, H, F, gs, M, K, ids, S[k], item(k), nhb, hi, sub);
  asm volatile("" ::: "memory");  // and the first weight loads ahead of the preparation
#pragma unroll
  for (int q = 0; q < DN_STAGE; ++q) {
    const int bq = ((int)threadIdx.x + q * DN_THREADS) >> 5;  // uniform per 32-lane group
    if (bq < 2 * nb) xprep_lanes_direct(hv[q], threadIdx.x & 31, lds + (size_t)bq * XP_DW);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NIT; ++k) {
    if (k + D - 1 < NIT) down_load<L, IT, PK>(rm, sm, H, F, gs, M, K, ids, S[(k + D - 1) % D], item(k + D - 1), nhb, hi, sub);
    DownItem<L, IT>& it = S[k % D];
    it.A.opaque();  // retire this item's loads here, computed or not
    it.B.opaque();
    if (k < n) {
      float ra, rb;
      dot2<L, IT, false>(it.A, it.B, lds + (size_t)(it.slot == s0 ? 0 : nb) * XP_DW, nb, sub, ra, rb);
      ra = lane_fold<L>(ra);
      rb = lane_fold<L>(rb);
      // rows hi, hi+1 (hi even, H a multiple of 8): one 4-byte store of both
      if (sub == 0 && it.h0 + hi < H) {
        bf16* dst = a.r + (size_t)it.slot * H + it.h0 + hi;
        *reinterpret_cast<uint32_t*>(dst) = (uint32_t)f2bf(ra) | ((uint32_t)f2bf(rb) << 16);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Expert kernels, one workgroup per (slot, row block) unit: the M*(K+1) slots are walked in
// the route's dispatch order (the shared expert's M slots, then each selected expert's slots
// side by side), and workgroup b takes unit (b % 8) * ceil(n/8) + b / 8: every XCD (workgroups
// go round-robin over the 8 XCDs) walks a contiguous run of units, so the slots of one expert
// run on one XCD at about the same time and its weight rows come from HBM once, the repeats from
// that XCD's L2.  Every workgroup does the same work (one token, the same rows), issues its
// weight loads first (after the one scalar read of its slot), and computes the per-slot
// kernels' dot products (same lanes, blocks, folds), so the bits are the same.
constexpr int DD_THREADS = 256;

__device__ __forceinline__ int dd_unit(int n_units) {
  const int per = (n_units + 7) / 8;
  return (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
}

// gate|up: a unit = dd_gate_up_rows<L>() rows of F (gate and up rows side by side): 16, or one
// pass of the 4 waves when that is more (64/L rows a wave); NP passes.  Units of 16 rows keep a
// workgroup's registers low enough for six per CU, so the launch runs in about one round
// (measured: 23.5 -> 19.1 us per launch at M = 4 against units of 32 rows).
template <int L>
constexpr int dd_gate_up_rows() { return 4 * (64 / L) > 16 ? 4 * (64 / L) : 16; }

template <int L, int IT, bool PK, bool CB>
__global__ __launch_bounds__(DD_THREADS) void k_moe_gate_up_dd(MoeArgs a0) {
  const MoeArgs a = a0.gorder ? a0 : moe_window(a0, blockIdx.y);
  extern __shared__ uint32_t lds[];  // [H/32][XP_DW]: the slot's token
  constexpr int RW = 64 / L;
  constexpr int UR = dd_gate_up_rows<L>();
  constexpr int NP = UR / (4 * RW);
  static_assert(4 * RW * NP == UR, "four waves cover the rows of a unit");
  const int H = a.H, F = a.F, gs = a.gs, M = a.M, K = a.K;
  const int nb = H / 32, ng = H / gs, P = sb_row_len(H, gs), nfb = F / UR;
  const int wslots = M * (K + 1), slots = a.gorder ? a.nwin * wslots : wslots;
  const int n_units = slots * nfb;
  const int w = dd_unit(n_units);
  if (w >= n_units) return;
  const int o = w / nfb, f0 = (w % nfb) * UR;
  const int ov = a.gorder ? a.gorder[o] : a.disp->order[o];
  const int sl = min(ov & 0xffff, slots - 1);  // (clamps: never out of the weights, whatever the table holds)
  const int win = sl / wslots, ls = sl - win * wslots;  // window and its slot (window 0 without gorder)
  const bool shared = ls >= M * K;
  const int m = win * M + (shared ? ls - M * K : ls / K);
  const int e = shared ? 0 : min(max((ov >> 16) - 1, 0), a.E - 1);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const uint32_t* gw = shared ? a.sh_gate_w : a.gate_w;
  const uint32_t* uw = shared ? a.sh_up_w : a.up_w;
  const uint32_t* gsb = shared ? a.sh_gate_sb : a.gate_sb;
  const uint32_t* usb = shared ? a.sh_up_sb : a.up_sb;
  const bf16* gsc = shared ? a.sh_gate_s : a.gate_s;
  const bf16* gbi = shared ? a.sh_gate_b : a.gate_b;
  const bf16* usc = shared ? a.sh_up_s : a.up_s;
  const bf16* ubi = shared ? a.sh_up_b : a.up_b;
  const size_t rbase = shared ? 0 : (size_t)e * F;
  QRow<L, IT> G[NP], U[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const size_t row = rbase + f0 + (p * 4 + wave) * RW + grp;
    G[p].template load_as<PK, CB>(gw + row * (H / 8), gsc + row * ng, gbi + row * ng, PK ? gsb + row * P : nullptr, nb,
                                  gs, sub, true);
    U[p].template load_as<PK, CB>(uw + row * (H / 8), usc + row * ng, ubi + row * ng, PK ? usb + row * P : nullptr, nb,
                                  gs, sub, true);
  }
  // the token's prepared activation blocks -> LDS (LDS-direct, one wait)
  stage16(lds, a.xp_x + (size_t)m * nb * XP_DW, nb * XP_DW);
  stage_sync();
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float g, up;
    dot2<L, IT, false>(G[p], U[p], lds, nb, sub, g, up);
    g = lane_fold<L>(g);
    up = lane_fold<L>(up);
    if (sub == 0)
      a.act[(size_t)sl * F + f0 + (p * 4 + wave) * RW + grp] = f2bf(silu_bf16(round_bf(g)) * round_bf(up));
  }
}

// down: a unit = NW * 64/L rows of H (one row per lane group) of one slot (two rows per lane
// group measured 15.3 against 13.6 us per launch at M = 4); the combine launch folds the slots'
// outputs.  (Combining in this launch -- agent-scope stores of the outputs, a per-row-block
// ticket and the last arriver folding the block -- was measured slower: the coherent stores, the
// wait for them and the serial tail cost more than the combine launch.)
// NW waves a unit (8 for a window's slots: the slot's activation load and block preparation shared by
// twice the rows; 4 in the prefill's global order).
template <int L, int NW = 4>
constexpr int dd_down_rows() { return NW * (64 / L); }

template <int L, int IT, bool PK, int NW>
__global__ __launch_bounds__(64 * NW) void k_moe_down_dd(MoeArgs a0) {
  const MoeArgs a = a0.gorder ? a0 : moe_window(a0, blockIdx.y);
  extern __shared__ uint32_t lds[];  // [F/32][XP_DW]
  constexpr int RW = 64 / L;
  constexpr int DR = dd_down_rows<L, NW>();
  constexpr int NT = 64 * NW;
  const int H = a.H, F = a.F, gs = a.gs, M = a.M, K = a.K;
  const int nb = F / 32, ng = F / gs, P = sb_row_len(F, gs), nhb = (H + DR - 1) / DR;
  const int wslots = M * (K + 1), slots = a.gorder ? a.nwin * wslots : wslots;
  const int n_units = slots * nhb;
  const int wu = dd_unit(n_units);
  if (wu >= n_units) return;
  const int o = wu / nhb, hb = wu % nhb, h0 = hb * DR;
  const int ov = a.gorder ? a.gorder[o] : a.disp->order[o];
  const int sl = min(ov & 0xffff, slots - 1);  // (clamps: never out of the weights, whatever the table holds)
  const bool shared = sl % wslots >= M * K;
  const int e = shared ? 0 : min(max((ov >> 16) - 1, 0), a.E - 1);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int hi = h0 + wave * RW + grp;  // this lane group's row
  const bool va = hi < H;
  const uint32_t* w = shared ? a.sh_down_w : a.down_w;
  const uint32_t* sb = shared ? a.sh_down_sb : a.down_sb;
  const bf16* sc = shared ? a.sh_down_s : a.down_s;
  const bf16* bi = shared ? a.sh_down_b : a.down_b;
  const size_t base = shared ? 0 : (size_t)e * H;
  const size_t ra = base + (va ? hi : h0);
  // the slot's bf16 activations first (element q * NT + t), then the weights
  constexpr int NA = 8 * DD_THREADS / NT;  // F <= 8 * 256
  bf16 av[NA];
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    const int i = q * NT + threadIdx.x;
    av[q] = i < F ? a.act[(size_t)sl * F + i] : (bf16)0;
  }
  asm volatile("" ::: "memory");
  QRow<L, IT> A;
  A.template load_as<PK>(w + ra * (F / 8), sc + ra * ng, bi + ra * ng, PK ? sb + ra * P : nullptr, nb, gs, sub, va);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    const int blk = (q * NT + (int)threadIdx.x) >> 5;  // uniform per 32-lane group
    if (blk < nb) xprep_lanes_direct(av[q], threadIdx.x & 31, lds + (size_t)blk * XP_DW);
  }
  __syncthreads();
  float x0 = A.dot(lds, nb, sub);
  x0 = lane_fold<L>(x0);
  if (sub == 0 && va) a.r[(size_t)sl * H + hi] = f2bf(x0);
}

// ---------------------------------------------------------------------------
template <int GL, int GIT>
static hipError_t router_route_go(const MoeArgs& a, hipStream_t st) {
  const int rows = GL > 0 ? a.E : a.E + 1;  // the bf16 gate row rides as router row E
  const int row_wgs = (rows + RR_THREADS / 64 - 1) / (RR_THREADS / 64);
  const int prep_wgs = a.xp_ready ? 0 : (a.M * (a.H / 32) + RR_THREADS / 32 - 1) / (RR_THREADS / 32);
  const int gx = row_wgs + prep_wgs + (GL > 0 ? 1 : 0);
  const bool poll = a.pub && a.nwin == 1;
  size_t lds = (size_t)a.M * a.H * 2;  // the staged activations
  if (GL > 0) lds = std::max(lds, (size_t)a.M * (a.H / 32) * XP_DW * 4);  // the gate's prepared blocks
  static size_t cur = 0;
  const hipError_t e = ensure_lds(k_moe_router_route<GL, GIT>, lds + 16 * 1024, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_moe_router_route<GL, GIT>), dim3(gx + (poll ? 1 : 0), a.nwin), dim3(RR_THREADS), lds, st, a,
                     row_wgs, poll ? gx : -1);
  return hipGetLastError();
}

hipError_t launch_moe_router_route(const MoeArgs& a, hipStream_t st) {
  if (a.M < 1 || a.M > MAX_TOKENS || a.H % 8 != 0 || a.H / 8 > ROUTER_IT * 64) return hipErrorInvalidValue;
  if (a.nwin < 1 || a.nwin > MOE_TICKETS) return hipErrorInvalidValue;  // a ticket per window
  if (!a.sg_w) return router_route_go<0, 0>(a, st);
  // the q4 gate row: the model's K = H = 2560 and 2048 tiled exactly, other widths by the predicated walker
  const int nb = a.H / 32, L = lanes_for_blocks(nb);
  if (a.H % 32 != 0 || nb > L * QMV_IT) return hipErrorInvalidValue;
  if (L == 16 && nb == 80) return router_route_go<16, 5>(a, st);
  if (L == 16 && nb == 64) return router_route_go<16, 4>(a, st);
  switch (L) {
    case 1: return router_route_go<1, 0>(a, st);
    case 2: return router_route_go<2, 0>(a, st);
    case 4: return router_route_go<4, 0>(a, st);
    case 8: return router_route_go<8, 0>(a, st);
    case 16: return router_route_go<16, 0>(a, st);
    case 32: return router_route_go<32, 0>(a, st);
    default: return router_route_go<64, 0>(a, st);
  }
}

template <int L, int IT, bool PK, int NIT>
static hipError_t gate_up_nit(const MoeArgs& a, int grid, hipStream_t st) {
  const size_t lds = (size_t)2 * (a.H / 32) * XP_DW * 4;
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_moe_gate_up<L, IT, PK, NIT>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_moe_gate_up<L, IT, PK, NIT>), dim3(grid, a.nwin), dim3(GU_THREADS), lds, st, a,
                     (const int32_t*)a.idx);
  return hipGetLastError();
}

// One workgroup per CU (more when a workgroup's range would exceed F/32 items,
// fewer for small windows); NIT = the most items a workgroup walks, rounded up
// to 1, 2, 4 or 8.
template <int L, int IT, bool PK>
static hipError_t gate_up_pk(const MoeArgs& a, hipStream_t st) {
  const int nfb = a.F / 32;
  const int items = (a.M + a.M * a.K) * nfb;
  int grid = items < device_cus() ? items : device_cus();
  const int lim = nfb < 8 ? nfb : 8;  // items per workgroup: at most two slot rows, at most 8
  if ((items + grid - 1) / grid > lim) grid = (items + lim - 1) / lim;
  const int per = (items + grid - 1) / grid;
  const int nit = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
  switch (nit) {
    case 1: return gate_up_nit<L, IT, PK, 1>(a, grid, st);
    case 2: return gate_up_nit<L, IT, PK, 2>(a, grid, st);
    case 4: return gate_up_nit<L, IT, PK, 4>(a, grid, st);
    default: return gate_up_nit<L, IT, PK, 8>(a, grid, st);
  }
}

template <int L, int IT>
static hipError_t gate_up_li(const MoeArgs& a, hipStream_t st) {
  return a.gate_sb ? gate_up_pk<L, IT, true>(a, st) : gate_up_pk<L, IT, false>(a, st);
}

template <int L, int IT, bool PK, int NIT>
static hipError_t down_nit(const MoeArgs& a, int grid, hipStream_t st) {
  const size_t lds = (size_t)2 * (a.F / 32) * XP_DW * 4;
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_moe_down<L, IT, PK, NIT>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_moe_down<L, IT, PK, NIT>), dim3(grid, a.nwin), dim3(DN_THREADS), lds, st, a,
                     (const int32_t*)a.idx);
  return hipGetLastError();
}

template <int L, int IT, bool PK>
static hipError_t down_pk(const MoeArgs& a, hipStream_t st) {
  constexpr int DR = (DN_THREADS / 64) * 2 * (64 / L);
  if (2 * a.F > DN_STAGE * DN_THREADS) return hipErrorInvalidValue;
  const int nhb = (a.H + DR - 1) / DR;
  const int items = (a.M + a.M * a.K) * nhb;
  int grid = items < device_cus() ? items : device_cus();
  const int lim = nhb < 8 ? nhb : 8;  // items per workgroup: at most two slot rows, at most 8
  if ((items + grid - 1) / grid > lim) grid = (items + lim - 1) / lim;
  const int per = (items + grid - 1) / grid;
  const int nit = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
  switch (nit) {
    case 1: return down_nit<L, IT, PK, 1>(a, grid, st);
    case 2: return down_nit<L, IT, PK, 2>(a, grid, st);
    case 4: return down_nit<L, IT, PK, 4>(a, grid, st);
    default: return down_nit<L, IT, PK, 8>(a, grid, st);
  }
}

template <int L, int IT>
static hipError_t down_li(const MoeArgs& a, hipStream_t st) {
  return a.down_sb ? down_pk<L, IT, true>(a, st) : down_pk<L, IT, false>(a, st);
}

hipError_t launch_moe_gate_up(const MoeArgs& a, hipStream_t st) { MTPX_QROW_DISPATCH(a.H / 32, gate_up_li, a, st); }

hipError_t launch_moe_down(const MoeArgs& a, hipStream_t st) { MTPX_QROW_DISPATCH(a.F / 32, down_li, a, st); }

template <int K>
static hipError_t combine_k(const MoeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_moe_combine<K>, dim3((a.H + 255) / 256, a.M, a.nwin), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const MoeArgs& a, hipStream_t st) {
  switch (a.K) {
    case 1: return combine_k<1>(a, st);
    case 2: return combine_k<2>(a, st);
    case 3: return combine_k<3>(a, st);
    case 4: return combine_k<4>(a, st);
    case 5: return combine_k<5>(a, st);
    case 6: return combine_k<6>(a, st);
    case 7: return combine_k<7>(a, st);
    case 8: return combine_k<8>(a, st);
    case 9: return combine_k<9>(a, st);
    case 10: return combine_k<10>(a, st);
    case 11: return combine_k<11>(a, st);
    case 12: return combine_k<12>(a, st);
    case 13: return combine_k<13>(a, st);
    case 14: return combine_k<14>(a, st);
    case 15: return combine_k<15>(a, st);
    case 16: return combine_k<16>(a, st);
    default: return hipErrorInvalidValue;
  }
}


// ---------------------------------------------------------------------------
// The batch's expert order (one workgroup): every window's slots grouped by expert -- the
// shared expert's slots first, then each routed expert's -- by a counting sort over the routes'
// expert ids (a.idx of all windows, consecutive).  The order inside an expert's group follows the
// atomics and is free: every slot's outputs are its own.
constexpr int SORT_THREADS = 1024;

__global__ __launch_bounds__(SORT_THREADS) void k_moe_sort(MoeArgs a) {
  __shared__ int cnt[1024], base[1024], cbase[1024];
  const int E = a.E, K = a.K, M = a.M, T = a.nwin * M, wslots = M * (K + 1);
  for (int e = threadIdx.x; e < E; e += SORT_THREADS) cnt[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < T * K; i += SORT_THREADS) atomicAdd(&cnt[min(max(a.idx[i], 0), E - 1)], 1);
  __syncthreads();
  const int sh_chunks = (T + MQ_CHUNK - 1) / MQ_CHUNK;
  if (threadIdx.x < 64) {  // exclusive scans of the counts and chunk counts by one wave, 64 experts per step
    int run = T;  // the shared expert's T slots come first
    int crun = sh_chunks;  // and its chunks
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + (int)threadIdx.x;
      const int c = e < E ? cnt[e] : 0, cc = (c + MQ_CHUNK - 1) / MQ_CHUNK;
      int incl = c, cincl = cc;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64), cy = __shfl_up(cincl, off, 64);
        if ((int)threadIdx.x >= off) {
          incl += y;
          cincl += cy;
        }
      }
      if (e < E) {
        base[e] = run + incl - c;
        cbase[e] = crun + cincl - cc;
      }
      run += __shfl(incl, 63, 64);
      crun += __shfl(cincl, 63, 64);
    }
    if (threadIdx.x == 0 && a.chunk_n) *a.chunk_n = crun;
  }
  __syncthreads();
  if (a.chunks) {  // chunks of at most MQ_CHUNK slots of one expert: (order position, count | (expert + 1) << 16)
    for (int c = threadIdx.x; c < sh_chunks; c += SORT_THREADS) {
      a.chunks[2 * c] = c * MQ_CHUNK;
      a.chunks[2 * c + 1] = min(MQ_CHUNK, T - c * MQ_CHUNK);
    }
    for (int e = threadIdx.x; e < E; e += SORT_THREADS)
      for (int k = 0; k * MQ_CHUNK < cnt[e]; ++k) {
        a.chunks[2 * (cbase[e] + k)] = base[e] + k * MQ_CHUNK;
        a.chunks[2 * (cbase[e] + k) + 1] = min(MQ_CHUNK, cnt[e] - k * MQ_CHUNK) | ((e + 1) << 16);
      }
    __syncthreads();  // base[] is the scatter's cursor below
  }
  for (int t = threadIdx.x; t < T; t += SORT_THREADS)  // shared slots: window t / M, slot M*K + t % M
    a.gorder[t] = (t / M) * wslots + M * K + t % M;
  for (int i = threadIdx.x; i < T * K; i += SORT_THREADS) {
    const int e = min(max(a.idx[i], 0), E - 1);
    const int t = i / K, k = i % K;
    const int pos = atomicAdd(&base[e], 1);
    a.gorder[pos] = ((t / M) * wslots + (t % M) * K + k) | ((e + 1) << 16);
  }
}

hipError_t launch_moe_sort(const MoeArgs& a, hipStream_t st) {
  if (!a.gorder || a.E > 1024 || (size_t)a.nwin * a.M * (a.K + 1) > 0xffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(SORT_THREADS), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// expert-grouped launches: grid = (M*K + 1 dispatch rows) x row blocks
template <int L, int IT, bool PK>
static hipError_t gate_up_dd_pk(const MoeArgs& a, hipStream_t st) {
  if constexpr (L < 4) {
    return hipErrorNotSupported;
  } else {
    const size_t lds = (size_t)(a.H / 32) * XP_DW * 4;
    static size_t cur = 0, cur_b = 0;
    hipError_t e = a.gorder ? ensure_lds(k_moe_gate_up_dd<L, IT, PK, true>, lds, cur_b)
                            : ensure_lds(k_moe_gate_up_dd<L, IT, PK, false>, lds, cur);
    if (e != hipSuccess) return e;
    if (a.F % dd_gate_up_rows<L>() != 0) return hipErrorInvalidValue;
    const int nw = a.gorder ? 1 : a.nwin;  // the global order: every window's units in one row of the grid
    const int units = a.M * (a.K + 1) * (a.gorder ? a.nwin : 1) * (a.F / dd_gate_up_rows<L>());
    // the global order reads an expert's rows once per slot of the batch, side by side on one XCD: cached loads
    if (a.gorder)
      hipLaunchKernelGGL((k_moe_gate_up_dd<L, IT, PK, true>), dim3((units + 7) / 8 * 8, nw), dim3(DD_THREADS), lds, st, a);
    else
      hipLaunchKernelGGL((k_moe_gate_up_dd<L, IT, PK, false>), dim3((units + 7) / 8 * 8, nw), dim3(DD_THREADS), lds, st, a);
    return hipGetLastError();
  }
}

template <int L, int IT>
static hipError_t gate_up_dd_li(const MoeArgs& a, hipStream_t st) {
  return a.gate_sb ? gate_up_dd_pk<L, IT, true>(a, st) : gate_up_dd_pk<L, IT, false>(a, st);
}

template <int L, int IT, bool PK>
static hipError_t down_dd_pk(const MoeArgs& a, hipStream_t st) {
  const size_t lds = (size_t)(a.F / 32) * XP_DW * 4;
  const int nw = a.gorder ? 1 : a.nwin;
  const int slots = a.M * (a.K + 1) * (a.gorder ? a.nwin : 1);
  auto go = [&](auto kern, size_t& cur, int dr, int nthr) {
    hipError_t e = ensure_lds(kern, lds, cur);
    if (e != hipSuccess) return e;
    const int units = slots * ((a.H + dr - 1) / dr);
    hipLaunchKernelGGL(kern, dim3((units + 7) / 8 * 8, nw), dim3(nthr), lds, st, a);
    return hipGetLastError();
  };
  static size_t c4 = 0, c8 = 0;
  // eight-wave units for a window (the slot's activation load and block preparation shared by twice the
  // rows: 9.2 -> 8.4 us per launch at one token, 11.3 -> 10.2 at two, 13.2 -> 12.1 at three, 17.9 -> 17.2 at
  // six); the prefill's global order keeps four
  constexpr int D4 = dd_down_rows<L, 4>(), D8 = dd_down_rows<L, 8>();
  if (!a.gorder) return go(k_moe_down_dd<L, IT, PK, 8>, c8, D8, 512);
  return go(k_moe_down_dd<L, IT, PK, 4>, c4, D4, 256);
}

template <int L, int IT>
static hipError_t down_dd_li(const MoeArgs& a, hipStream_t st) {
  return a.down_sb ? down_dd_pk<L, IT, true>(a, st) : down_dd_pk<L, IT, false>(a, st);
}

hipError_t launch_moe_gate_up_dd(const MoeArgs& a, hipStream_t st) {
  MTPX_QROW_DISPATCH(a.H / 32, gate_up_dd_li, a, st);
}

hipError_t launch_moe_down_dd(const MoeArgs& a, hipStream_t st) { MTPX_QROW_DISPATCH(a.F / 32, down_dd_li, a, st); }

bool moe_dd_supported(int H, int F, int K) {
  const int Lg = lanes_for_blocks(H / 32);
  const int ur = 4 * (64 / Lg) > 16 ? 4 * (64 / Lg) : 16;  // dd_gate_up_rows
  return Lg >= 4 && F % ur == 0 && H % 8 == 0 && F <= 8 * DD_THREADS && K >= 1;
}

}  // namespace mtpx
