// The hyper-connection mixer of one sublayer in two launches:
//   k_mix_down : lo = down . n and inj = inject . n (n = the normed streams,
//                K = hc*H), split over the lane rule's classes: the L lanes of
//                a row's walk are grouped by lane mod Q (Q = min(L, 4)); each
//                workgroup computes one class of a row block for one part of
//                the window's tokens from that class's activation blocks only
//                and folds the class's lanes (the butterfly levels L/2 .. Q),
//                leaving Q partials per row and token
//   k_mix_up   : per (32 hidden positions, part of the tokens): every
//                workgroup finishes the butterfly for its tokens' low-rank rows
//                ((v0 + v2) + (v1 + v3) for Q = 4: the remaining levels Q/2 .. 1
//                in the same order), rounds, applies SiLU and prepares the
//                activation blocks; then the up rows of its 32 hidden
//                positions in every stream (w), the mix
//                x = bf16 running sum over streams of bf16(sigmoid(w) * n), the
//                prepared blocks of x, and j = 2 * sigmoid(inj)
// The float order of every row is the one of the single-launch GEMV (same
// lanes, same blocks per lane, same butterfly), so the outputs are those of
// down/inject GEMV -> SiLU -> up GEMV -> mix.
// Reference: Runner/FastModel/TrackFastMixer.swift:14-224 (downInject, upMix),
// Runner/FastModel/TrackFastMixerSplitK.swift (the split-K down projection),
// Runner/FastModel/TrackFastKernels2.swift:160-280 (hcMix).
#include "qrows.h"

namespace mtpx {

constexpr int MIX_THREADS = 256;

// SBM, the scale/bias layout the launch reads: 1 the packed pair rows (every matrix of the launch has
// them), 0 the checkpoint's scale and bias rows (always present; the same values).  One load path per
// launch, so no load waits at a join of the two.
template <int SBM, int L, int IT>
__device__ __forceinline__ void mix_row_load(QRow<L, IT>& R, const uint32_t* wrow, const bf16* srow, const bf16* brow,
                                             const uint32_t* sbrow, int nb, int gs, int sub, bool valid) {
  R.template load_as<SBM == 1>(wrow, srow, brow, sbrow, nb, gs, sub, valid);
}

template <int SBM, int L, int IT>
__global__ __launch_bounds__(MIX_THREADS) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_mix_down(MixArgs a,
                                                                                                    int tsplit) {
  static_assert(IT > 0, "exact lane tiling");
  extern __shared__ uint32_t lds[];  // this class's activation blocks [tokens of this workgroup][nb/Q]
  constexpr int Q = L < 4 ? L : 4;
  constexpr int LC = L / Q;       // lanes of one row within a class
  constexpr int RPW = 64 / LC;    // rows per wave
  const int W = a.hc * a.H, nb = W / 32, ncb = nb / Q;
  const int NR = a.LW + (a.iw ? a.hc : 0);
  // Workgroup w -> (row block, class, token part): the Q classes of a row block read the interleaved
  // 16-byte blocks of the same cache lines, and its token parts the same rows, so they get ids 8
  // apart -- the same XCD (ids go round-robin over the 8 XCDs) and one L2.  The window's tokens are
  // cut into tsplit parts (one workgroup each: more workgroups on the chip for a wide window).
  const int wg = blockIdx.x;
  const int g = (wg / 8) % Q;
  const int tp = (wg / (8 * Q)) % tsplit;
  const int rb = (wg / (8 * Q * tsplit)) * 8 + wg % 8;
  const int per = (a.S + tsplit - 1) / tsplit, s0 = tp * per, s1 = min(a.S, s0 + per), S = s1 - s0;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int subc = lane % LC, grp = lane / LC;
  const int sub = g + Q * subc;  // the lane of the single-launch walk this lane stands in for
  const int row = rb * (4 * RPW) + wave * RPW + grp;
  if (rb * (4 * RPW) >= NR) return;
  const bool valid = row < NR;
  const int r = valid ? row : 0;
  const bool inj = r >= a.LW;
  const int rr = inj ? r - a.LW : r;
  const int ng = W / a.gs, P = sb_row_len(W, a.gs);
  const uint32_t* wq = inj ? a.iw : a.dw;
  const bf16* sc = inj ? a.is : a.ds;
  const bf16* bi = inj ? a.ib : a.db;
  const uint32_t* sb = inj ? a.isb : a.dsb;
  // stage the class's blocks with LDS-direct loads: compact block c = subc' + LC * it holds
  // block g + Q * subc' + L * it; unit i = (s * ncb + c) * 7 + q
  QRow<L, IT> R;
  mix_row_load<SBM>(R, wq + (size_t)rr * (W / 8), sc + (size_t)rr * ng, bi + (size_t)rr * ng, sb ? sb + (size_t)rr * P : nullptr,
         nb, a.gs, sub, valid);
  asm volatile("" ::: "memory");
  const int n4 = S * ncb * (XP_DW / 4);
  for (int i = threadIdx.x; i < n4; i += MIX_THREADS) {
    const int q = i % (XP_DW / 4), c = (i / (XP_DW / 4)) % ncb, s = s0 + i / (XP_DW / 4) / ncb;
    const int j = g + Q * (c % LC) + L * (c / LC);
    lds_dma16(reinterpret_cast<uint4*>(lds) + (i - lane), a.xpW + ((size_t)s * nb + j) * XP_DW + 4 * q);
  }
  lds_dma_wait();
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const uint32_t* xl = lds + ((size_t)s * ncb + subc + LC * it) * XP_DW;
      acc = block_accum(acc, block_dot(R.w[it], xl), __uint_as_float(R.sb[it] << 16),
                        __uint_as_float(R.sb[it] & 0xffff0000u), xl);
    }
    acc = lane_fold<LC>(acc);
    if (subc == 0 && valid) a.part[((size_t)g * a.S + s0 + s) * NR + row] = acc;
  }
}

// Butterfly levels Q/2 .. 1 over the class partials of one row.
template <int Q>
__device__ __forceinline__ float class_fold_v(const float* v) {
  if constexpr (Q == 4) return (v[0] + v[2]) + (v[1] + v[3]);
  if constexpr (Q == 2) return v[0] + v[1];
  return v[0];
}

// grid (H/32 position blocks x tsplit token parts, rounded to whole groups of 8), UP_THREADS threads.
// Up rows of the block: local row lr = c*32 + i is global row c*H + d0 + i.  A workgroup takes one
// part of the window's tokens; the two halves of the workgroup (waves 0-3 and 4-7) walk the same up
// rows for the part's even and odd tokens.  The parts of a position block get ids 8 apart (one XCD:
// the second reads the up rows from that L2).  FB and MR size the loads issued up front to the part's
// tokens: FB batches of class partials (S * LW <= FB * UP_THREADS) and MR rounds of normed values
// (S * hc * 32 <= MR * UP_THREADS), so no clamped duplicate load queues ahead of the up rows.
constexpr int UP_THREADS = 512;
constexpr int UP_FB_MAX = 8, UP_MR_MAX = MAX_TOKENS * 8 * 32 / UP_THREADS;  // any window: hc <= 8

template <int QD, int SBM, int L, int IT, int FB, int MR>
__global__ __launch_bounds__(UP_THREADS) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_mix_up(MixArgs a,
                                                                                                  int tsplit) {
  constexpr int RW = 64 / L;
  constexpr int MAXROWS = 8 * 32;  // hc <= 8
  constexpr int NP = (MAXROWS + 4 * RW - 1) / (4 * RW);
  constexpr int FOLD_BATCH = FB;  // S * LW <= FOLD_BATCH * UP_THREADS: one round of partial loads
  __shared__ uint32_t xpa[MAX_TOKENS * 12 * XP_DW];  // [S][LW/32][XP_DW], S * LW / 32 <= 96
  __shared__ bf16 wl[MAX_TOKENS][MAXROWS];
  constexpr int MIX_ROUNDS = MR;                    // (token, stream, position) terms per thread
  __shared__ float term[MAX_TOKENS * MAXROWS];      // [S][hc][32] bf16(sigmoid(w) * n)
  const int H = a.H, hc = a.hc, LW = a.LW, W = hc * H;
  const int NR = LW + (a.iw ? hc : 0);
  const int nbA = LW / 32, ng = LW / a.gs, P = sb_row_len(LW, a.gs);
  const int pb = ((int)blockIdx.x / (8 * tsplit)) * 8 + (int)blockIdx.x % 8, tp = ((int)blockIdx.x / 8) % tsplit;
  if (pb * 32 >= H) return;
  const int per = (a.S + tsplit - 1) / tsplit, s0 = tp * per, S = min(a.S, s0 + per) - s0;  // this part's tokens
  const int d0 = pb * 32;
  const int wave = (threadIdx.x >> 6) & 3, half = threadIdx.x >> 8, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int nrows = hc * 32;
  // Loads in the order they are needed (the memory counter retires them in
  // order): the class partials of the low-rank rows (S * LW <= FOLD_BATCH *
  // UP_THREADS: one round), the normed streams for the mix, then the up rows,
  // which stream in during the fold, SiLU and activation preparation.
  float pp[FOLD_BATCH][QD];
#pragma unroll
  for (int u = 0; u < FOLD_BATCH; ++u) {
    const int i0 = threadIdx.x + u * UP_THREADS, i = i0 < S * LW ? i0 : S * LW - 1;
    const float* p = a.part + (size_t)(s0 + i / LW) * NR + i % LW;
#pragma unroll
    for (int q = 0; q < QD; ++q) pp[u][q] = p[(size_t)q * a.S * NR];
  }
  // inject gate (s, c) of this thread: the first workgroup, for every token of the window
  const bool jt = blockIdx.x == 0 && a.iw && a.j && (int)threadIdx.x < a.S * hc;
  float jp[QD];
#pragma unroll
  for (int q = 0; q < QD; ++q)
    jp[q] = jt ? a.part[(size_t)q * a.S * NR + (size_t)(threadIdx.x / hc) * NR + LW + threadIdx.x % hc] : 0.0f;
  // the mix's terms: thread i of round r takes (token, stream, position) u = r * UP_THREADS + i,
  // u = (s * hc + c) * 32 + position; unconditional loads (clamped), used only for u < S * hc * 32
  const int nterm = S * hc * 32;
  float nv[MIX_ROUNDS];
#pragma unroll
  for (int r = 0; r < MIX_ROUNDS; ++r) {
    const int u0 = r * UP_THREADS + (int)threadIdx.x, u = u0 < nterm ? u0 : nterm - 1;
    const int sc = u >> 5;  // s * hc + c
    nv[r] = bf2f(a.normed[(size_t)(s0 + sc / hc) * W + (size_t)(sc % hc) * H + d0 + (u & 31)]);
  }
  QRow<L, IT> U[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    if (p * 4 * RW >= nrows) break;  // uniform
    const int lr = p * 4 * RW + wave * RW + grp;
    const bool v = lr < nrows;
    const int gr = v ? (lr / 32) * H + d0 + (lr % 32) : 0;
    mix_row_load<SBM>(U[p], a.uw + (size_t)gr * (LW / 8), a.us + (size_t)gr * ng, a.ub + (size_t)gr * ng,
                      a.usb ? a.usb + (size_t)gr * P : nullptr, nbA, a.gs, sub, v);
  }
  // low-rank rows: finish the fold, round, SiLU, and the prepared blocks straight from the registers:
  // item i = t + u * UP_THREADS is element i % 32 of block i / 32, and the 32 lanes of a block are 32
  // consecutive threads (UP_THREADS and S * LW are multiples of 32, so a block is all in or all out)
#pragma unroll
  for (int u = 0; u < FOLD_BATCH; ++u) {
    if (u * UP_THREADS >= S * LW) break;  // uniform: only the batches that hold rows
    const int i = threadIdx.x + u * UP_THREADS;
    const bf16 v = f2bf(silu_bf16(round_bf(class_fold_v<QD>(pp[u]))));
    if (i < S * LW) xprep_lanes_direct(v, threadIdx.x & 31, xpa + (size_t)(i >> 5) * XP_DW);
  }
  if (jt) a.j[threadIdx.x] = f2bf(2.0f * sigmoid_bf16(round_bf(class_fold_v<QD>(jp))));  // [s * hc + c]
  __syncthreads();
  // up rows of the block: this half's tokens
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int lr = p * 4 * RW + wave * RW + grp;
    if (p * 4 * RW >= nrows) break;  // uniform
    for (int s = half; s < S; s += 2) {
      float v = U[p].dot(xpa + (size_t)s * nbA * XP_DW, nbA, sub);
      v = lane_fold<L>(v);
      if (sub == 0 && lr < nrows) wl[s][lr] = f2bf(v);
    }
  }
  __syncthreads();
  // mix: every term bf16(sigmoid(w) * n) by its own thread, then the running sum over the streams
  // (in stream order) by 32 lanes per token, and the prepared block of x
#pragma unroll
  for (int r = 0; r < MIX_ROUNDS; ++r) {
    if (r * UP_THREADS >= nterm) break;  // uniform
    const int u = r * UP_THREADS + (int)threadIdx.x, uc = u < nterm ? u : nterm - 1;
    const float tv = round_bf(sigmoid_bf16(bf2f(wl[(uc >> 5) / hc][((uc >> 5) % hc) * 32 + (uc & 31)])) * nv[r]);
    if (u < nterm) term[u] = tv;
  }
  __syncthreads();
  const int ms = threadIdx.x >> 5, mi = threadIdx.x & 31;
  if (ms < S) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c)
      if (c < hc) acc = round_bf(acc + term[(ms * hc + c) * 32 + mi]);
    const bf16 y = f2bf(acc);
    a.x[(size_t)(s0 + ms) * H + d0 + mi] = y;
    if (a.xpH) xprep_lanes_direct(y, mi, a.xpH + ((size_t)(s0 + ms) * (H / 32) + pb) * XP_DW);
  }
}

template <int L, int IT>
static hipError_t mix_down_li(const MixArgs& a, hipStream_t st) {
  if constexpr (IT == 0) {
    return hipErrorInvalidValue;  // exact tiling only (checked by the caller)
  } else {
    constexpr int Q = L < 4 ? L : 4;
    constexpr int RPB = 4 * (64 / (L / Q));
    const int W = a.hc * a.H, NR = a.LW + (a.iw ? a.hc : 0);
    // two or more tokens in two parts: twice the workgroups, half the tokens each (measured against one
    // part: 17.8 -> 16.1 us for the mixer pair at 2 tokens, 20.7 -> 17.5 at 4; three or four parts were
    // slower)
    const int tsplit = a.S >= 2 ? 2 : 1;
    const int per = (a.S + tsplit - 1) / tsplit;
    const size_t lds = (size_t)per * (W / 32 / Q) * XP_DW * 4;
    const int nrb = (NR + RPB - 1) / RPB;
    const dim3 grid((nrb + 7) / 8 * 8 * Q * tsplit);
    auto go = [&](auto kern, size_t& cur) {
      hipError_t e = ensure_lds(kern, lds, cur);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, grid, dim3(MIX_THREADS), lds, st, a, tsplit);
      return hipGetLastError();
    };
    static size_t cur0 = 0, cur1 = 0;
    if (a.dsb && (!a.iw || a.isb)) return go(k_mix_down<1, L, IT>, cur1);
    return go(k_mix_down<0, L, IT>, cur0);
  }
}

template <int QD, int SBM, int L, int IT>
static hipError_t mix_up_go(const MixArgs& a, hipStream_t st) {
  // (as the down launch: two parts from two tokens on; four parts need two rounds of these workgroups)
  const int tsplit = a.S >= 2 ? 2 : 1;
  const dim3 grid((a.H / 32 + 7) / 8 * 8 * tsplit);
  // the up-front loads sized to the part's tokens (the model's four classes, exact walkers)
  const int per = (a.S + tsplit - 1) / tsplit;
  const int fb = (per * a.LW + UP_THREADS - 1) / UP_THREADS, mr = (per * a.hc * 32 + UP_THREADS - 1) / UP_THREADS;
  if constexpr (QD == 4 && IT > 0) {
    if (fb <= 1 && mr <= 1) {
      hipLaunchKernelGGL((k_mix_up<QD, SBM, L, IT, 1, 1>), grid, dim3(UP_THREADS), 0, st, a, tsplit);
      return hipGetLastError();
    }
    if (fb <= 2 && mr <= 1) {
      hipLaunchKernelGGL((k_mix_up<QD, SBM, L, IT, 2, 1>), grid, dim3(UP_THREADS), 0, st, a, tsplit);
      return hipGetLastError();
    }
    if (fb <= 3 && mr <= 1) {
      hipLaunchKernelGGL((k_mix_up<QD, SBM, L, IT, 3, 1>), grid, dim3(UP_THREADS), 0, st, a, tsplit);
      return hipGetLastError();
    }
  }
  if (fb > UP_FB_MAX || mr > UP_MR_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_mix_up<QD, SBM, L, IT, UP_FB_MAX, UP_MR_MAX>), grid, dim3(UP_THREADS), 0, st, a, tsplit);
  return hipGetLastError();
}

// The up rows' lane rule over K = LW: at most 4 lanes a row (mix_supported), so only those walkers.
template <int QD, int SBM>
static hipError_t mix_up_lw(const MixArgs& a, hipStream_t st) {
  const int nb = a.LW / 32, L = lanes_for_blocks(nb), IT = nb % L == 0 ? nb / L : 0;
  switch (L * 16 + (IT >= 4 && IT <= 7 ? IT : 0)) {
    case 2 * 16 + 4: return mix_up_go<QD, SBM, 2, 4>(a, st);
    case 2 * 16 + 5: return mix_up_go<QD, SBM, 2, 5>(a, st);
    case 4 * 16 + 4: return mix_up_go<QD, SBM, 4, 4>(a, st);
    case 4 * 16 + 5: return mix_up_go<QD, SBM, 4, 5>(a, st);
    case 4 * 16 + 6: return mix_up_go<QD, SBM, 4, 6>(a, st);
    default: break;
  }
  switch (L) {
    case 1: return mix_up_go<QD, SBM, 1, 0>(a, st);
    case 2: return mix_up_go<QD, SBM, 2, 0>(a, st);
    default: return mix_up_go<QD, SBM, 4, 0>(a, st);
  }
}

template <int QD>
static hipError_t mix_up_q(const MixArgs& a, hipStream_t st) {
  return a.usb ? mix_up_lw<QD, 1>(a, st) : mix_up_lw<QD, 0>(a, st);
}

static hipError_t mix_down(const MixArgs& a, hipStream_t st) { MTPX_QROW_DISPATCH(a.hc * a.H / 32, mix_down_li, a, st); }

int mix_classes(int W) {
  const int L = lanes_for_blocks(W / 32);
  return L < 4 ? L : 4;
}

// Fused path: exact lane tiling of the down rows (4..7 blocks per lane), up rows
// walked by at most 4 lanes (their registers hold a workgroup's rows without
// spilling), the low-rank activations and their prepared blocks within LDS.
bool mix_supported(int H, int hc, int LW, int S) {
  const int nb = hc * H / 32, L = lanes_for_blocks(nb);
  return S >= 1 && S <= MAX_TOKENS && nb % L == 0 && nb / L >= 4 && nb / L <= 7 && hc <= 8 && LW % 32 == 0 &&
         lanes_for_blocks(LW / 32) <= 4 && S * LW <= MAX_TOKENS * 512 &&
         S * (LW / 32) <= MAX_TOKENS * 12 && H % 32 == 0;
}

hipError_t launch_mixer(const MixArgs& a, hipStream_t st) {
  hipError_t e = mix_down(a, st);
  if (e != hipSuccess) return e;
  switch (mix_classes(a.hc * a.H)) {
    case 4: return mix_up_q<4>(a, st);
    case 2: return mix_up_q<2>(a, st);
    default: return mix_up_q<1>(a, st);
  }
}

}  // namespace mtpx
