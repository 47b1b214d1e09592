// The MoE block of the decode/verify window (M <= 8 tokens), three launches:
//   router+route: bf16 router GEMV (+ shared-expert gate row) over f32(x) and
//            the activation block preparation of x; the last row workgroup to
//            finish (ticket) runs the route: top-k (value desc, index asc) +
//            softmax, and the expert-grouped dispatch table (each selected
//            expert once, with its tokens)
//   gate_up: per (32-row block of F, selected expert): gate and up rows of the
//            expert against every token routed to it, SwiGLU, and the block
//            preparation of the activation for the down projection
//   down   : per (128-row block of H, selected expert): down rows against the
//            expert's activations -> routed/shared outputs per slot
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
#include "qrows.h"

namespace mtpx {

// ---------------------------------------------------------------------------
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

// ---------------------------------------------------------------------------
// route (run by one workgroup of RR_THREADS threads): wave m selects token m's
// top-k; then the dispatch table is built in LDS by all threads: each expert
// once (ordered by its first (token, rank) slot), with its slots ordered by
// token.
constexpr int ROUTE_EPER = 16;  // E <= 1024
constexpr int RR_THREADS = 512;

__device__ void route_body(const MoeArgs& a) {
  const int E = a.E, K = a.K, M = a.M;
  const int MK = M * K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ int sel[MAX_TOKENS * MAX_TOPK];
  __shared__ float selv[MAX_TOKENS][MAX_TOPK];
  __shared__ int first[1024];
  __shared__ uint32_t tokbits[MAX_TOKENS][32];  // expert membership per token
  __shared__ uint64_t leadmask[2];
  __shared__ int uid[MAX_TOKENS * MAX_TOPK];
  for (int i = threadIdx.x; i < E; i += blockDim.x) first[i] = 0x7fffffff;
  for (int i = threadIdx.x; i < MAX_TOKENS * 32; i += blockDim.x) (&tokbits[0][0])[i] = 0u;
  __syncthreads();
  if (wave < M) {
    const float* lr = a.logits + (size_t)wave * E;
    float v[ROUTE_EPER];
    uint32_t taken = 0;  // bit j: expert lane + 64*j already selected (or absent)
#pragma unroll
    for (int j = 0; j < ROUTE_EPER; ++j) {
      const int e = lane + 64 * j;
      v[j] = (e < E) ? ld_pub(lr + e) : -__uint_as_float(0x7f800000u);
      if (e >= E) taken |= 1u << j;
    }
    for (int k = 0; k < K; ++k) {
      float bv = -__uint_as_float(0x7f800000u);
      int bj = -1;
#pragma unroll
      for (int j = 0; j < ROUTE_EPER; ++j)
        if (!((taken >> j) & 1u) && (bj < 0 || v[j] > bv)) {
          bv = v[j];
          bj = j;
        }
      float gmax = bv;
      gmax = fmaxf(gmax, lane_xor_f<32>(gmax));
      gmax = fmaxf(gmax, lane_xor_f<16>(gmax));
      gmax = fmaxf(gmax, lane_xor_f<8>(gmax));
      gmax = fmaxf(gmax, lane_xor_f<4>(gmax));
      gmax = fmaxf(gmax, lane_xor_f<2>(gmax));
      gmax = fmaxf(gmax, lane_xor_f<1>(gmax));
      int cand = (bj >= 0 && bv == gmax) ? lane + 64 * bj : 0x7fffffff;
      cand = min(cand, lane_xor_i<32>(cand));
      cand = min(cand, lane_xor_i<16>(cand));
      cand = min(cand, lane_xor_i<8>(cand));
      cand = min(cand, lane_xor_i<4>(cand));
      cand = min(cand, lane_xor_i<2>(cand));
      cand = min(cand, lane_xor_i<1>(cand));
      if (bj >= 0 && cand == lane + 64 * bj) taken |= 1u << bj;
      // only NaN logits leave no candidate; keep the index addressable
      if (cand >= E) cand = 0;
      if (lane == 0) {
        sel[wave * K + k] = cand;
        selv[wave][k] = gmax;
      }
    }
    // softmax over the K selected: exp per lane, sum in rank order on lane 0
    const float mx = selv[wave][0];
    if (lane < K) selv[wave][lane] = expf_det(selv[wave][lane] - mx);
    if (lane == 0) {
      float sum = 0.0f;
      for (int k = 0; k < K; ++k) sum = sum + selv[wave][k];
      sum = 1.0f / sum;
      for (int k = 0; k < K; ++k) selv[wave][k] = selv[wave][k] * sum;
    }
    if (lane < K) {
      a.idx[wave * K + lane] = sel[wave * K + lane];
      a.w[wave * K + lane] = selv[wave][lane];
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
  const bool leader = t < MK && first[e] == t;
  const uint64_t bal = __ballot(leader);
  if (lane == 0 && wave < 2) leadmask[wave] = bal;
  __syncthreads();
  MoeDispatch* d = a.disp;
  if (leader) {
    const uint64_t below = (t & 63) ? (leadmask[t >> 6] & ((~0ull) >> (64 - (t & 63)))) : 0ull;
    const int u = __popcll(below) + (t >= 64 ? __popcll(leadmask[0]) : 0);
    uid[t] = u;
    int count = 0;
    for (int m = 0; m < M; ++m) count += (tokbits[m][e >> 5] >> (e & 31)) & 1u;
    d->expert[u] = e;
    d->count[u] = count;
  }
  __syncthreads();
  if (t < MK) {
    const int u = uid[first[e]];
    int pos = 0;
    for (int m = 0; m < t / K; ++m) pos += (tokbits[m][e >> 5] >> (e & 31)) & 1u;
    d->slot[u][pos] = (int16_t)t;
  }
  if (t == 0) {
    const int n = __popcll(leadmask[0]) + (MK > 64 ? __popcll(leadmask[1]) : 0);
    d->n_unique = n;
    if (a.nu_out) *a.nu_out = n;
    d->expert[n] = -1;
    d->count[n] = M;
    for (int m = 0; m < M; ++m) d->slot[n][m] = (int16_t)(MK + m);
  }
}

// ---------------------------------------------------------------------------
// router + route: workgroups [0, row_wgs) hold one wave per router row (rows
// 0..E-1 router, row E the shared-expert gate); lane l walks 8-element chunks
// l, l+64, ...: acc = fmaf(w, x, acc) in element order, then an xor butterfly
// over the wave.  The remaining workgroups prepare x's activation blocks for
// the expert GEMVs (32 lanes per block) and take no ticket.
constexpr int ROUTER_IT = 8;  // H <= 8 * 64 * 8

__global__ __launch_bounds__(RR_THREADS) void k_moe_router_route(MoeArgs a, int row_wgs) {
  const int H = a.H, E = a.E, M = a.M;
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
  if (r <= E) {
    const bf16* wrow = (r < E) ? a.router + (size_t)r * H : a.shared_gate;
    const int nc = H / 8;
    uint4 wv[ROUTER_IT];
#pragma unroll
    for (int i = 0; i < ROUTER_IT; ++i) {
      const int c = lane + 64 * i;
      wv[i] = (c < nc) ? *reinterpret_cast<const uint4*>(wrow + (size_t)c * 8) : make_uint4(0, 0, 0, 0);
    }
    for (int m = 0; m < M; ++m) {
      const bf16* xm = a.x + (size_t)m * H;
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < ROUTER_IT; ++i) {
        const int c = lane + 64 * i;
        if (c < nc) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xm + (size_t)c * 8);
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
          st_pub(a.logits + (size_t)m * E + r, acc);
        else
          a.gate_logit[m] = acc;
      }
    }
  }
  if (!ticket_last(a.ticket, (uint32_t)row_wgs - 1u)) return;
  route_body(a);
}

// Dispatch entry of grid row y: row 0 is the shared expert (every token, the
// most work per workgroup, so it is dispatched first), rows 1..nu the routed
// experts in dispatch order; -1 for the rows beyond.
__device__ __forceinline__ int expert_slot(int y, int nu) {
  if (y == 0) return nu;
  return y - 1 < nu ? y - 1 : -1;
}

__device__ __forceinline__ int slot_token(int slot, int M, int K) {
  return slot < M * K ? slot / K : slot - M * K;
}

// ---------------------------------------------------------------------------
// gate|up + SwiGLU.  grid (F/32, M*K+1), GU_THREADS threads.  Every lane-group
// owns one f of the block and walks its gate row and up row; the weight loads
// are issued before the activations are staged into LDS.
// GU_THREADS threads: 512 (eight waves, one pass each) for a one-token window,
// where only parallelism matters; 256 (four waves, two passes each: the second
// pass's loads are in flight while the first is computed) for wider windows.
template <int L, int IT, int GU_THREADS>
__global__ __launch_bounds__(GU_THREADS) void k_moe_gate_up(MoeArgs a) {
  extern __shared__ uint32_t lds[];
  __shared__ bf16 actb[MAX_TOKENS][32];
  constexpr int WAVES = GU_THREADS / 64;
  constexpr int RW = 64 / L;                                  // f rows per wave pass
  constexpr int NI = (32 + WAVES * RW - 1) / (WAVES * RW);     // passes for 32 rows
  const int H = a.H, F = a.F, M = a.M, K = a.K, gs = a.gs;
  const int nb = H / 32, ng = H / gs;
  const int nu = a.disp->n_unique;
  const int u = expert_slot(blockIdx.y, nu);
  if (u < 0) return;
  const bool shared = (u == nu);
  const int e = a.disp->expert[u];
  const int cnt = a.disp->count[u];
  const uint32_t* gw = shared ? a.sh_gate_w : a.gate_w + (size_t)e * F * (H / 8);
  const bf16* gsc = shared ? a.sh_gate_s : a.gate_s + (size_t)e * F * ng;
  const bf16* gbi = shared ? a.sh_gate_b : a.gate_b + (size_t)e * F * ng;
  const uint32_t* uw = shared ? a.sh_up_w : a.up_w + (size_t)e * F * (H / 8);
  const bf16* usc = shared ? a.sh_up_s : a.up_s + (size_t)e * F * ng;
  const bf16* ubi = shared ? a.sh_up_b : a.up_b + (size_t)e * F * ng;
  const int P = sb_row_len(H, gs);
  const uint32_t* gsb = a.gate_sb ? (shared ? a.sh_gate_sb : a.gate_sb + (size_t)e * F * P) : nullptr;
  const uint32_t* usb = a.gate_sb ? (shared ? a.sh_up_sb : a.up_sb + (size_t)e * F * P) : nullptr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int f0 = blockIdx.x * 32;
  QRow<L, IT> G[NI], U[NI];
#pragma unroll
  for (int p = 0; p < NI; ++p) {
    const int fi = (wave + p * WAVES) * RW + grp;
    const bool valid = fi < 32;
    const int f = f0 + (valid ? fi : 0);
    G[p].load(gw + (size_t)f * (H / 8), gsc + (size_t)f * ng, gbi + (size_t)f * ng, gsb ? gsb + (size_t)f * P : nullptr,
              nb, gs, sub, valid);
    U[p].load(uw + (size_t)f * (H / 8), usc + (size_t)f * ng, ubi + (size_t)f * ng, usb ? usb + (size_t)f * P : nullptr,
              nb, gs, sub, valid);
  }
  for (int tk = 0; tk < cnt; ++tk) {
    const int m = slot_token(a.disp->slot[u][tk], M, K);
    stage16(lds + (size_t)tk * nb * XP_DW, a.xp_x + (size_t)m * nb * XP_DW, nb * XP_DW);
  }
  stage_sync();
#pragma unroll
  for (int p = 0; p < NI; ++p) {
    const int fi = (wave + p * WAVES) * RW + grp;
    if ((wave + p * WAVES) * RW >= 32) break;  // uniform per wave
    for (int tk = 0; tk < cnt; ++tk) {
      float g, up;
      dot2(G[p], U[p], lds + (size_t)tk * nb * XP_DW, nb, sub, g, up);
      g = lane_fold<L>(g);
      up = lane_fold<L>(up);
      if (sub == 0 && fi < 32) {
        const bf16 act = f2bf(silu_bf16(round_bf(g)) * round_bf(up));
        actb[tk][fi] = act;
        a.act[(size_t)a.disp->slot[u][tk] * F + f0 + fi] = act;
      }
    }
  }
  __syncthreads();
  // prepared activation block of this f-block for every slot: 32 lanes per slot
  {
    const int tk = threadIdx.x >> 5, i = threadIdx.x & 31;
    if (tk < cnt)
      xprep_lanes_direct(actb[tk][i], i, a.xp_act + ((size_t)a.disp->slot[u][tk] * (F / 32) + blockIdx.x) * XP_DW);
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

__global__ __launch_bounds__(256) void k_moe_combine(MoeArgs a) {
  const int m = blockIdx.y, h = blockIdx.x * 256 + threadIdx.x;
  if (h >= a.H) return;
  const int H = a.H, M = a.M, K = a.K;
  float prod[MAX_TOPK];
  for (int k = 0; k < K; ++k) prod[k] = bf2f(a.r[(size_t)(m * K + k) * H + h]) * a.w[m * K + k];
  const float rr = round_bf(colsum_small(prod, K));
  const float sg = sigmoid_bf16(round_bf(a.gate_logit[m]));
  const float sh = round_bf(sg * bf2f(a.r[(size_t)(M * K + m) * H + h]));
  const bf16 out = f2bf(rr + sh);
  if (a.y) a.y[(size_t)m * H + h] = out;
  if (a.y2) a.y2[(size_t)m * H + h] = f2bf(bf2f(a.resid[(size_t)m * H + h]) + bf2f(out));
}

// ---------------------------------------------------------------------------
// down: grid (H/DOWN_ROWS, M*K+1), 256 threads; each lane-group owns two rows
// (RPL = 2) so each LDS read of an activation block feeds two rows.
template <int L, int IT>
__global__ __launch_bounds__(256) void k_moe_down(MoeArgs a) {
  extern __shared__ uint32_t lds[];
  constexpr int RW = 64 / L;
  constexpr int NI = (DOWN_ROWS + 8 * RW - 1) / (8 * RW);  // passes of 2*RW rows per wave
  const int H = a.H, F = a.F, K = a.K, gs = a.gs;
  const int nb = F / 32, ng = F / gs;
  const int nu = a.disp->n_unique;
  const int u = expert_slot(blockIdx.y, nu);
  if (u < 0) return;
  const bool shared = (u == nu);
  const int e = a.disp->expert[u];
  const int cnt = a.disp->count[u];
  const uint32_t* dw = shared ? a.sh_down_w : a.down_w + (size_t)e * H * (F / 8);
  const bf16* dsc = shared ? a.sh_down_s : a.down_s + (size_t)e * H * ng;
  const bf16* dbi = shared ? a.sh_down_b : a.down_b + (size_t)e * H * ng;
  const int P = sb_row_len(F, gs);
  const uint32_t* dsb = a.down_sb ? (shared ? a.sh_down_sb : a.down_sb + (size_t)e * H * P) : nullptr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int h0 = blockIdx.x * DOWN_ROWS;
  QRow<L, IT> A[NI], B[NI];
#pragma unroll
  for (int p = 0; p < NI; ++p) {
    const int hi = (wave + 4 * p) * 2 * RW + 2 * grp;
    const bool va = hi < DOWN_ROWS && h0 + hi < H, vb = hi + 1 < DOWN_ROWS && h0 + hi + 1 < H;
    const int ha = va ? h0 + hi : h0, hb = vb ? h0 + hi + 1 : h0;
    A[p].load(dw + (size_t)ha * (F / 8), dsc + (size_t)ha * ng, dbi + (size_t)ha * ng,
              dsb ? dsb + (size_t)ha * P : nullptr, nb, gs, sub, va);
    B[p].load(dw + (size_t)hb * (F / 8), dsc + (size_t)hb * ng, dbi + (size_t)hb * ng,
              dsb ? dsb + (size_t)hb * P : nullptr, nb, gs, sub, vb);
  }
  for (int tk = 0; tk < cnt; ++tk)
    stage16(lds + (size_t)tk * nb * XP_DW, a.xp_act + (size_t)a.disp->slot[u][tk] * nb * XP_DW, nb * XP_DW);
  stage_sync();
#pragma unroll
  for (int p = 0; p < NI; ++p) {
    if ((wave + 4 * p) * 2 * RW >= DOWN_ROWS) break;  // uniform per wave
    const int hi = (wave + 4 * p) * 2 * RW + 2 * grp;
    for (int tk = 0; tk < cnt; ++tk) {
      float ra, rb;
      dot2(A[p], B[p], lds + (size_t)tk * nb * XP_DW, nb, sub, ra, rb);
      ra = lane_fold<L>(ra);
      rb = lane_fold<L>(rb);
      // rows hi, hi+1 (hi even, H a multiple of 8): one 4-byte store of both
      if (sub == 0 && hi < DOWN_ROWS && h0 + hi < H) {
        bf16* dst = a.r + (size_t)a.disp->slot[u][tk] * H + h0 + hi;
        *reinterpret_cast<uint32_t*>(dst) = (uint32_t)f2bf(ra) | ((uint32_t)f2bf(rb) << 16);
      }
    }
  }
}

// ---------------------------------------------------------------------------
hipError_t launch_moe_router_route(const MoeArgs& a, hipStream_t st) {
  const int row_wgs = (a.E + 1 + RR_THREADS / 64 - 1) / (RR_THREADS / 64);
  const int prep_wgs = a.xp_ready ? 0 : (a.M * (a.H / 32) + RR_THREADS / 32 - 1) / (RR_THREADS / 32);
  hipLaunchKernelGGL(k_moe_router_route, dim3(row_wgs + prep_wgs), dim3(RR_THREADS), 0, st, a, row_wgs);
  return hipGetLastError();
}

template <int L, int IT, int THREADS>
static hipError_t gate_up_launch(const MoeArgs& a, hipStream_t st) {
  const dim3 grid(a.F / 32, a.M * a.K + 1);
  const size_t lds = (size_t)a.M * (a.H / 32) * XP_DW * 4;
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_moe_gate_up<L, IT, THREADS>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_moe_gate_up<L, IT, THREADS>), grid, dim3(THREADS), lds, st, a);
  return hipGetLastError();
}

template <int L, int IT>
static hipError_t gate_up_li(const MoeArgs& a, hipStream_t st) {
  return a.M == 1 ? gate_up_launch<L, IT, 512>(a, st) : gate_up_launch<L, IT, 256>(a, st);
}

template <int L, int IT>
static hipError_t down_li(const MoeArgs& a, hipStream_t st) {
  const dim3 grid((a.H + DOWN_ROWS - 1) / DOWN_ROWS, a.M * a.K + 1);
  const size_t lds = (size_t)a.M * (a.F / 32) * XP_DW * 4;
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_moe_down<L, IT>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_moe_down<L, IT>), grid, dim3(256), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_moe_gate_up(const MoeArgs& a, hipStream_t st) { MTPX_QROW_DISPATCH(a.H / 32, gate_up_li, a, st); }

hipError_t launch_moe_down(const MoeArgs& a, hipStream_t st) { MTPX_QROW_DISPATCH(a.F / 32, down_li, a, st); }

hipError_t launch_moe_combine(const MoeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_moe_combine, dim3((a.H + 255) / 256, a.M), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace mtpx
