// The MoE block of the decode/verify window (M <= 8 tokens), four launches:
//   router : bf16 router GEMV (+ shared-expert gate row) over f32(x), and the
//            activation block preparation of x
//   route  : top-k (value desc, index asc) + softmax, and the expert-grouped
//            dispatch table (each selected expert once, with its tokens)
//   gate_up: per (32-row block of F, selected expert): gate and up rows of the
//            expert against every token routed to it, SwiGLU, and the block
//            preparation of the activation for the down projection
//   down   : per (64-row block of H, selected expert): down rows against the
//            expert's activations; the last workgroup to finish a row block
//            folds the routed outputs in rank order and adds the gated shared
//            expert (MLX col_reduce_small association)
// Reference: FM/TrackFastModel.swift:867-954 (orchestration),
// FM/TrackFastMoE.swift:780-911 (route), :1192-1404 (gate|up+act),
// :1412-1576 (down+combine), :2246-2310 (router GEMV),
// FM/TrackFastKernels2.swift:21-58,512-544 (sigmoid, colsum fold, combine).
#include "mtpx_kernels.h"

namespace mtpx {

// ---------------------------------------------------------------------------
// router: one wave per row (rows 0..E-1 router, row E the shared-expert gate).
// Lane l walks 8-element chunks l, l+64, ...: acc = fmaf(w, x, acc) in element
// order, then an xor butterfly over the wave.
constexpr int ROUTER_IT = 8;  // H <= 8 * 64 * 8

__global__ __launch_bounds__(256) void k_moe_router(MoeArgs a, int row_wgs) {
  const int H = a.H, E = a.E, M = a.M;
  if ((int)blockIdx.x >= row_wgs) {
    // activation block preparation of x for the expert GEMVs
    const int nb = H / 32;
    const int i = ((int)blockIdx.x - row_wgs) * blockDim.x + threadIdx.x;
    if (i < M * nb) xprep_block(a.x + (size_t)(i / nb) * H + (size_t)(i % nb) * 32, a.xp_x + (size_t)i * XP_DW);
    return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + wave;
  if (r > E) return;
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
        a.logits[(size_t)m * E + r] = acc;
      else
        a.gate_logit[m] = acc;
    }
  }
}

// ---------------------------------------------------------------------------
// route: wave m selects token m's top-k; then thread 0 builds the dispatch.
constexpr int ROUTE_EPER = 16;  // E <= 1024

__global__ __launch_bounds__(512) void k_moe_route(MoeArgs a) {
  const int E = a.E, K = a.K, M = a.M;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ int sel[MAX_TOKENS][MAX_TOPK];
  __shared__ float selv[MAX_TOKENS][MAX_TOPK];
  if (wave < M) {
    const float* lr = a.logits + (size_t)wave * E;
    float v[ROUTE_EPER];
#pragma unroll
    for (int j = 0; j < ROUTE_EPER; ++j) {
      const int e = lane + 64 * j;
      v[j] = (e < E) ? lr[e] : -__uint_as_float(0x7f800000u);
    }
    bool taken[ROUTE_EPER];
#pragma unroll
    for (int j = 0; j < ROUTE_EPER; ++j) taken[j] = (lane + 64 * j) >= E;
    for (int k = 0; k < K; ++k) {
      float bv = -__uint_as_float(0x7f800000u);
      int bj = -1;
#pragma unroll
      for (int j = 0; j < ROUTE_EPER; ++j)
        if (!taken[j] && (bj < 0 || v[j] > bv)) {
          bv = v[j];
          bj = j;
        }
      float gmax = bv;
#pragma unroll
      for (int off = 32; off >= 1; off /= 2) gmax = fmaxf(gmax, __shfl_xor(gmax, off, 64));
      int cand = (bj >= 0 && bv == gmax) ? lane + 64 * bj : 0x7fffffff;
#pragma unroll
      for (int off = 32; off >= 1; off /= 2) cand = min(cand, __shfl_xor(cand, off, 64));
      if (bj >= 0 && cand == lane + 64 * bj) taken[bj] = true;
      // only NaN logits leave no candidate; keep the index addressable
      if (cand >= E) cand = 0;
      if (lane == 0) {
        sel[wave][k] = cand;
        selv[wave][k] = gmax;
      }
    }
    if (lane == 0) {
      const float mx = selv[wave][0];
      float e[MAX_TOPK];
      float sum = 0.0f;
      for (int k = 0; k < K; ++k) {
        e[k] = expf_det(selv[wave][k] - mx);
        sum = sum + e[k];
      }
      const float inv = 1.0f / sum;
      for (int k = 0; k < K; ++k) {
        a.idx[wave * K + k] = sel[wave][k];
        a.w[wave * K + k] = e[k] * inv;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    MoeDispatch* d = a.disp;
    int n = 0;
    for (int m = 0; m < M; ++m)
      for (int k = 0; k < K; ++k) {
        const int e = sel[m][k];
        int u = 0;
        while (u < n && d->expert[u] != e) ++u;
        if (u == n) {
          d->expert[n] = e;
          d->count[n] = 0;
          ++n;
        }
        if (d->count[u] < MAX_TOKENS) d->slot[u][d->count[u]++] = (int16_t)(m * K + k);
      }
    d->n_unique = n;
    d->expert[n] = -1;
    d->count[n] = M;
    for (int m = 0; m < M; ++m) d->slot[n][m] = (int16_t)(M * K + m);
  }
}

// ---------------------------------------------------------------------------
// gate|up + SwiGLU.  grid (F/32, M*K+1).  Lanes: L per row, each lane-group
// owns one f and walks its gate row and its up row (the two RowLoads).
template <int L>
struct RowLoad1 {
  uint32_t w[QMV_IT][4];
  float s[QMV_IT], b[QMV_IT];
  __device__ __forceinline__ void load(const uint32_t* __restrict__ wrow, const bf16* __restrict__ srow,
                                       const bf16* __restrict__ brow, int nb, int gs, int sub, bool valid) {
#pragma unroll
    for (int it = 0; it < QMV_IT; ++it) {
      const int j = sub + it * L;
      if (valid && j < nb) {
        const uint4 v = ldg16(wrow + (size_t)j * 4);
        w[it][0] = v.x; w[it][1] = v.y; w[it][2] = v.z; w[it][3] = v.w;
        const int g = (j * 32) / gs;
        s[it] = bf2f(srow[g]);
        b[it] = bf2f(brow[g]);
      } else {
        w[it][0] = w[it][1] = w[it][2] = w[it][3] = 0u;
        s[it] = b[it] = 0.0f;
      }
    }
  }
  __device__ __forceinline__ float dot(const uint32_t* __restrict__ xpv, int nb, int sub) const {
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < QMV_IT; ++it) {
      const int j = sub + it * L;
      if (j < nb) {
        const uint32_t* xl = xpv + (size_t)j * XP_DW;
        acc = block_accum(acc, block_dot(w[it], xl), s[it], b[it], xl);
      }
    }
    return acc;
  }
};

__device__ __forceinline__ int slot_token(int slot, int M, int K) {
  return slot < M * K ? slot / K : slot - M * K;
}

template <int L>
__global__ __launch_bounds__(256) void k_moe_gate_up(MoeArgs a) {
  extern __shared__ uint32_t lds[];
  __shared__ bf16 actb[MAX_TOKENS][32];
  const int H = a.H, F = a.F, M = a.M, K = a.K, gs = a.gs;
  const int nb = H / 32, ng = H / gs;
  const int u = blockIdx.y;
  const int nu = a.disp->n_unique;
  if (u > nu) return;
  const bool shared = (u == nu);
  const int e = a.disp->expert[u];
  const int cnt = a.disp->count[u];
  for (int i = threadIdx.x; i < cnt * nb * XP_DW; i += blockDim.x) {
    const int t = i / (nb * XP_DW), rem = i % (nb * XP_DW);
    const int m = slot_token(a.disp->slot[u][t], M, K);
    lds[i] = a.xp_x[(size_t)m * nb * XP_DW + rem];
  }
  __syncthreads();
  const uint32_t* gw = shared ? a.sh_gate_w : a.gate_w + (size_t)e * F * (H / 8);
  const bf16* gsc = shared ? a.sh_gate_s : a.gate_s + (size_t)e * F * ng;
  const bf16* gbi = shared ? a.sh_gate_b : a.gate_b + (size_t)e * F * ng;
  const uint32_t* uw = shared ? a.sh_up_w : a.up_w + (size_t)e * F * (H / 8);
  const bf16* usc = shared ? a.sh_up_s : a.up_s + (size_t)e * F * ng;
  const bf16* ubi = shared ? a.sh_up_b : a.up_b + (size_t)e * F * ng;
  constexpr int RW = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int f0 = blockIdx.x * 32;
  for (int fi0 = wave * RW; fi0 < 32; fi0 += 4 * RW) {  // uniform per wave (shuffles below)
    const int fi = fi0 + grp;
    const bool valid = fi < 32;
    const int f = f0 + (valid ? fi : 0);
    RowLoad1<L> G, U;
    G.load(gw + (size_t)f * (H / 8), gsc + (size_t)f * ng, gbi + (size_t)f * ng, nb, gs, sub, valid);
    U.load(uw + (size_t)f * (H / 8), usc + (size_t)f * ng, ubi + (size_t)f * ng, nb, gs, sub, valid);
    for (int t = 0; t < cnt; ++t) {
      const uint32_t* xm = lds + (size_t)t * nb * XP_DW;
      const float g = lane_fold<L>(G.dot(xm, nb, sub));
      const float up = lane_fold<L>(U.dot(xm, nb, sub));
      if (sub == 0 && valid) {
        const bf16 act = f2bf(silu_bf16(round_bf(g)) * round_bf(up));
        actb[t][fi] = act;
        a.act[(size_t)a.disp->slot[u][t] * F + f] = act;
      }
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < cnt) {
    const int slot = a.disp->slot[u][threadIdx.x];
    xprep_block(actb[threadIdx.x], a.xp_act + ((size_t)slot * (F / 32) + blockIdx.x) * XP_DW);
  }
}

// ---------------------------------------------------------------------------
// down + combine.  grid (H/64, M*K+1).
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

template <int L>
__global__ __launch_bounds__(256) void k_moe_down(MoeArgs a) {
  extern __shared__ uint32_t lds[];
  __shared__ int is_last;
  const int H = a.H, F = a.F, M = a.M, K = a.K, gs = a.gs;
  const int nb = F / 32, ng = F / gs;
  const int u = blockIdx.y;
  const int nu = a.disp->n_unique;
  if (u > nu) return;
  const bool shared = (u == nu);
  const int e = a.disp->expert[u];
  const int cnt = a.disp->count[u];
  for (int i = threadIdx.x; i < cnt * nb * XP_DW; i += blockDim.x) {
    const int t = i / (nb * XP_DW), rem = i % (nb * XP_DW);
    lds[i] = a.xp_act[(size_t)a.disp->slot[u][t] * nb * XP_DW + rem];
  }
  __syncthreads();
  const uint32_t* dw = shared ? a.sh_down_w : a.down_w + (size_t)e * H * (F / 8);
  const bf16* dsc = shared ? a.sh_down_s : a.down_s + (size_t)e * H * ng;
  const bf16* dbi = shared ? a.sh_down_b : a.down_b + (size_t)e * H * ng;
  constexpr int RW = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int h0 = blockIdx.x * DOWN_ROWS;
  for (int hi0 = wave * RW; hi0 < DOWN_ROWS; hi0 += 4 * RW) {
    const int hi = hi0 + grp;
    const bool valid = hi < DOWN_ROWS && h0 + hi < H;
    const int h = valid ? h0 + hi : h0;
    RowLoad1<L> D;
    D.load(dw + (size_t)h * (F / 8), dsc + (size_t)h * ng, dbi + (size_t)h * ng, nb, gs, sub, valid);
    for (int t = 0; t < cnt; ++t) {
      const float r = lane_fold<L>(D.dot(lds + (size_t)t * nb * XP_DW, nb, sub));
      if (sub == 0 && valid) a.r[(size_t)a.disp->slot[u][t] * H + h] = f2bf(r);
    }
  }
  // the last workgroup of this row block folds every expert's rows
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(&a.counters[blockIdx.x], 1u);
    is_last = (old == (uint32_t)nu);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int i = threadIdx.x; i < M * DOWN_ROWS; i += blockDim.x) {
    const int m = i / DOWN_ROWS, h = h0 + i % DOWN_ROWS;
    if (h >= H) continue;
    float prod[MAX_TOPK];
    for (int k = 0; k < K; ++k)
      prod[k] = bf2f(a.r[(size_t)(m * K + k) * H + h]) * a.w[m * K + k];
    const float rr = round_bf(colsum_small(prod, K));
    const float sg = sigmoid_bf16(round_bf(a.gate_logit[m]));
    const float sh = round_bf(sg * bf2f(a.r[(size_t)(M * K + m) * H + h]));
    a.y[(size_t)m * H + h] = f2bf(rr + sh);
  }
  if (threadIdx.x == 0) a.counters[blockIdx.x] = 0u;
}

// ---------------------------------------------------------------------------
hipError_t launch_moe_router(const MoeArgs& a, hipStream_t st) {
  const int row_wgs = (a.E + 1 + 3) / 4;
  const int prep_wgs = (a.M * (a.H / 32) + 255) / 256;
  hipLaunchKernelGGL(k_moe_router, dim3(row_wgs + prep_wgs), dim3(256), 0, st, a, row_wgs);
  return hipGetLastError();
}

hipError_t launch_moe_route(const MoeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(64 * a.M), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_moe_gate_up(const MoeArgs& a, hipStream_t st) {
  const dim3 grid(a.F / 32, a.M * a.K + 1);
  const size_t lds = (size_t)a.M * (a.H / 32) * XP_DW * 4;
  switch (lanes_for_blocks(a.H / 32)) {
#define GU(Lv)                                                            \
  case Lv: {                                                              \
    static size_t cur = 0;                                                \
    hipError_t e = ensure_lds(k_moe_gate_up<Lv>, lds, cur);                   \
    if (e != hipSuccess) return e;                                        \
    hipLaunchKernelGGL(k_moe_gate_up<Lv>, grid, dim3(256), lds, st, a);       \
  } break;
    GU(1) GU(2) GU(4) GU(8) GU(16) GU(32) GU(64)
#undef GU
  }
  return hipGetLastError();
}

hipError_t launch_moe_down(const MoeArgs& a, hipStream_t st) {
  const dim3 grid((a.H + DOWN_ROWS - 1) / DOWN_ROWS, a.M * a.K + 1);
  const size_t lds = (size_t)a.M * (a.F / 32) * XP_DW * 4;
  switch (lanes_for_blocks(a.F / 32)) {
#define DN(Lv)                                                            \
  case Lv: {                                                              \
    static size_t cur = 0;                                                \
    hipError_t e = ensure_lds(k_moe_down<Lv>, lds, cur);                   \
    if (e != hipSuccess) return e;                                        \
    hipLaunchKernelGGL(k_moe_down<Lv>, grid, dim3(256), lds, st, a);       \
  } break;
    DN(1) DN(2) DN(4) DN(8) DN(16) DN(32) DN(64)
#undef DN
  }
  return hipGetLastError();
}

hipError_t launch_moe_block(const MoeArgs& a, hipStream_t st) {
  hipError_t e;
  if ((e = launch_moe_router(a, st)) != hipSuccess) return e;
  if ((e = launch_moe_route(a, st)) != hipSuccess) return e;
  if ((e = launch_moe_gate_up(a, st)) != hipSuccess) return e;
  return launch_moe_down(a, st);
}

}  // namespace mtpx
