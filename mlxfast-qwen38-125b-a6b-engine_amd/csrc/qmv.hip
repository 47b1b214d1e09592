// Dense affine-4-bit GEMV (y[M,N] = x[M,K] . W[N,K]^T), activation block
// preparation, device-side MLX affine quantisation and seeded weight init.
//
// Weight format (MLX affine 4-bit, unchanged from the reference checkpoint):
// packed uint32 [N, K/8], element k at bits 4*(k%8) of word k/8; bf16 scale
// and bias [N, K/gs].  Arithmetic: see mtpx_device.h.
#include <algorithm>

#include "qrows.h"

namespace mtpx {

// Activation block preparation of x [M, K] -> xp [M, K/32, XP_DW]: a 32-lane
// group per block, eight blocks per 256-thread workgroup.
__global__ __launch_bounds__(256) void k_xprep(const bf16* __restrict__ x, int M, int K, uint32_t* __restrict__ xp) {
  const int nb = K / 32;
  const int i = threadIdx.x & 31;
  const int blk = blockIdx.x * 8 + (int)(threadIdx.x >> 5);
  if (blk < M * nb) xprep_lanes_direct(x[(size_t)(blk / nb) * K + (size_t)(blk % nb) * 32 + i], i, xp + (size_t)blk * XP_DW);
}

// Dense GEMV.  NWV waves (4, or 5 where that fits a launch's workgroups to the CUs); every lane-group
// owns two rows (RPL = 2) so each LDS read of a prepared activation block feeds two weight rows.  A wave's
// rows are loaded before the activations are staged.  Grid Y batches windows
// of `win` tokens (window w: tokens w * win .. of the M in all), each computed
// as its own launch would.  PK: the scale/bias pairs from the packed rows (sbp),
// else from the checkpoint's rows -- one load path, so no load waits at a join.
template <int L, int IT, bool CB, bool PK, int NWV>
__global__ __launch_bounds__(64 * NWV) void k_qmv(const uint32_t* __restrict__ wq, const bf16* __restrict__ sc,
                                             const bf16* __restrict__ bi, const uint32_t* __restrict__ sbp,
                                             int N, int K, int gs,
                                             const uint32_t* __restrict__ xp, int M, bf16* __restrict__ y,
                                             float* __restrict__ yf, int rows_per_wg, int win) {
  extern __shared__ uint32_t lds[];
  constexpr int RW = 64 / L;
  constexpr int RPW = 2 * RW;  // rows per wave pass
  const int nb = K / 32, ng = K / gs, P = sb_row_len(K, gs);
  {
    const int t0 = (int)blockIdx.y * win;
    xp += (size_t)t0 * nb * XP_DW;
    y += (size_t)t0 * N;
    if (yf) yf += (size_t)t0 * N;
    M = min(M - t0, win);
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int row0 = blockIdx.x * rows_per_wg;
  const int row_end = min(row0 + rows_per_wg, N);
  QRow<L, IT> A, B;
  int base = row0 + wave * RPW;
  auto load2 = [&](int b0) {
    const int rA = b0 + grp * 2, rB = rA + 1;
    const bool vA = rA < row_end, vB = rB < row_end;
    const int ra = vA ? rA : row0, rb = vB ? rB : row0;
    A.template load_as<PK, CB>(wq + (size_t)ra * (K / 8), sc + (size_t)ra * ng, bi + (size_t)ra * ng,
                               PK ? sbp + (size_t)ra * P : nullptr, nb, gs, sub, vA);
    B.template load_as<PK, CB>(wq + (size_t)rb * (K / 8), sc + (size_t)rb * ng, bi + (size_t)rb * ng,
                               PK ? sbp + (size_t)rb * P : nullptr, nb, gs, sub, vB);
  };
  if (base < row_end) load2(base);  // first rows in flight before the staging
  stage16(lds, xp, M * nb * XP_DW);
  stage_sync();
  for (bool first = true; base < row_end; base += NWV * RPW, first = false) {  // uniform per wave
    if (!first) load2(base);
    const int rA = base + grp * 2, rB = rA + 1;
    for (int m = 0; m < M; ++m) {
      float a, b;
      dot2(A, B, lds + (size_t)m * nb * XP_DW, nb, sub, a, b);
      a = lane_fold<L>(a);
      b = lane_fold<L>(b);
      if (sub == 0) {
        if (rA < row_end) {
          y[(size_t)m * N + rA] = f2bf(a);
          if (yf) yf[(size_t)m * N + rA] = a;
        }
        if (rB < row_end) {
          y[(size_t)m * N + rB] = f2bf(b);
          if (yf) yf[(size_t)m * N + rB] = b;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Dense GEMV on the matrix cores for 2..4 tokens (y = x . W^T, same bits as
// k_qmv).  The exact integer block sums come from v_mfma_i32_16x16x32_i8 with
//   A (16 x 32): row 4t + l = limb l of token t's 24-bit fixed-point block,
//                limbs l = bits 0-6, 7-13, 14-15 (unsigned) and 16-23 (signed)
//                of m, so every byte fits a signed i8 and four tokens fill
//                the 16 rows;
//   B (32 x 16): the 32 nibbles of one block of 16 weight rows;
// lane (token t = lane / 16, row n = lane % 16) then holds the four limb sums
// Da..Dd, and low = Da + 128 Db + 16384 Dc, D2 = Dd are the integers the
// dot-product path forms from its byte limbs (low = sum w * (m & 0xffff),
// D2 = sum w * (m >> 16)), so dxraw = fmaf(D2, 65536, low) and the block
// combine are the same float operations.  The K order inside a block is the
// prepared layout's (even elements of a word, then odd), for A and B alike.
// Chains: block j joins chain j % L (L = lanes_for_blocks(K/32)), chains fold
// in the lane walk's butterfly order.  A wave owns one tile of 16 rows and one
// class c of C chain classes (chains = c mod C): its blocks j = c, c + C, ...
// in order; the classes of a tile are waves of one workgroup and their
// partials meet in LDS for the last log2(C) butterfly levels.  Weights stream
// as one 16-byte load per lane per four blocks (lane group g loads block g of
// the four), turned by a 4x4 transpose across the lane groups (two
// permlane32 and two permlane16 swaps) into lane group g = word g of each
// block; the next four blocks' loads are in flight while these are computed.
constexpr int MMA_TOK = 4;   // tokens per tile (4 tokens x 4 limbs = 16 A rows)
constexpr int MB_DW = 36;    // LDS block: [limb][word g][even, odd] (32 dwords), p, SX, pad
static_assert(MB_DW == XMB_DW, "the four-limb block in memory");
constexpr int MMA_THREADS = 512;

typedef int v4i_t __attribute__((ext_vector_type(4)));

// Prepared blocks of M tokens (xp [M][NB][XP_DW]) -> the four-limb layout in
// LDS [MMA_TOK * TG][NB][MB_DW] (TG groups of four tokens); tokens M.. are zero
// (their sums are 0, p = SX = 0).
// Unit u = (token, block, word g, even/odd) converts three limb words into
// four; the loads (all units of this thread, then its p/SX pairs) are issued
// by mma_stage_load, so the caller can put its own loads behind them and
// mma_stage_store waits for these only.
template <int NB, int TG, int NTH>
struct MmaStage {
  static constexpr int NT = MMA_TOK * TG;                      // tokens staged
  static constexpr int NU = (NT * NB * 8 + NTH - 1) / NTH;     // units per thread (NTH threads)
  static constexpr int NP = (NT * NB + NTH - 1) / NTH;         // p/SX pairs per thread
  uint32_t w[NU][3];
  uint32_t ps[NP][2];

  __device__ __forceinline__ void load(const uint32_t* __restrict__ xp, int M) {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = threadIdx.x + k * NTH;
      const int t = u / (NB * 8), rem = u - t * (NB * 8), blk = rem >> 3, ge = rem & 7;
      const bool in = u < NT * NB * 8 && t < M;
      const uint32_t* src = xp + ((size_t)(in ? t : 0) * NB + (in ? blk : 0)) * XP_DW + ((ge & 1) ? 4 : 0) + (ge >> 1);
      w[k][0] = in ? src[0] : 0u;
      w[k][1] = in ? src[8] : 0u;
      w[k][2] = in ? src[16] : 0u;
    }
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int u = threadIdx.x + k * NTH;
      const int t = u / NB, blk = u - t * NB;
      const bool in = u < NT * NB && t < M;
      const uint32_t* src = xp + ((size_t)(in ? t : 0) * NB + (in ? blk : 0)) * XP_DW + 24;
      ps[k][0] = in ? src[0] : 0u;
      ps[k][1] = in ? src[1] : 0u;
    }
  }

  __device__ __forceinline__ void store(uint32_t* __restrict__ lds) const {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = threadIdx.x + k * NTH;
      if (u < NT * NB * 8) {
        const int t = u / (NB * 8), rem = u - t * (NB * 8), blk = rem >> 3, ge = rem & 7;
        const uint32_t w0 = w[k][0], w1 = w[k][1];
        uint32_t* dst = lds + ((size_t)t * NB + blk) * MB_DW + 2 * (ge >> 1) + (ge & 1);
        dst[0] = w0 & 0x7f7f7f7fu;                                          // bits 0-6
        dst[8] = ((w0 >> 7) & 0x01010101u) | ((w1 << 1) & 0x7e7e7e7eu);    // bits 7-13
        dst[16] = (w1 >> 6) & 0x03030303u;                                  // bits 14-15
        dst[24] = w[k][2];                                                  // bits 16-23 (signed)
      }
    }
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int u = threadIdx.x + k * NTH;
      if (u < NT * NB) {
        uint32_t* dst = lds + (size_t)u * MB_DW + 32;  // u = t * NB + blk
        dst[0] = ps[k][0];
        dst[1] = ps[k][1];
      }
    }
  }
};

// butterfly levels S, S/2, .., 1 over v[0..2S-1]: v[u] = v[u] + v[u + S] (u < S); result v[0]
template <int S, int NV>
__device__ __forceinline__ void fold_levels(float (&v)[NV]) {
  if constexpr (S >= 1) {
#pragma unroll
    for (int u = 0; u < S; ++u) v[u] = v[u] + v[u + S];
    fold_levels<S / 2>(v);
  }
}

// Chunks per loop body: half of the class's chunks when a class has at most 12 (two bodies: the
// walk waits for HBM about twice), else LC/4 (at least 2); in both, 8 * BC is a multiple of LC, so
// every body repeats the chain order.
template <int L, int IT, int C>
constexpr int mma_body_chunks() {
  constexpr int LC = L / C, NCH = L * IT / C / 4, B0 = LC / 4 > 2 ? LC / 4 : 2;
  if (LC < 1 || NCH < 2) return B0;  // no valid tiling (rejected by mma_c_ok)
  return (NCH <= 12 && NCH % 2 == 0 && (8 * (NCH / 2)) % LC == 0 && NCH / 2 >= B0) ? NCH / 2 : B0;
}

template <int L, int IT, int C, int TG, bool XPF, int NWV>
__global__ __launch_bounds__(64 * NWV) void k_qmv_mma(const uint32_t* __restrict__ wq, const uint32_t* __restrict__ sbp,
                                                        int N, int K, int gs, const uint32_t* __restrict__ xp, int M,
                                                        bf16* __restrict__ y, float* __restrict__ yf) {
  constexpr int NB = L * IT;   // blocks per row
  constexpr int LC = L / C;    // chains per class
  constexpr int NQ = NB / C;   // blocks per class
  constexpr int NCH = NQ / 4;  // four-block chunks per class
  constexpr int BC = mma_body_chunks<L, IT, C>();  // chunks per loop body
  constexpr int TPG = NWV / C;                 // tiles per workgroup pass (NWV waves)
  static_assert(NB % (4 * C) == 0 && NCH % BC == 0 && C <= L && C <= 8 && LC <= 16 && NWV % C == 0,
                "whole bodies of four-block chunks, whole tiles per workgroup");
  // LDS: activations [MMA_TOK * TG][NB][MB_DW]; per wave the (scale, bias) pairs of its tile and class
  // [16][NQ]; class partials [2][NWV waves][TG][64].  Token group tq (tokens 4 tq .. 4 tq + 3) takes its own
  // MFMA on the same weight operand, so a launch serves up to 4 TG tokens with one read of the weights.
  constexpr size_t TGO = (size_t)MMA_TOK * NB * MB_DW;  // one token group's activations
  extern __shared__ uint32_t lds[];
  {  // grid Y batches windows of 4 TG tokens (window w: tokens 4 TG w .. of the M in all)
    const int t0 = (int)blockIdx.y * (MMA_TOK * TG);
    xp += (size_t)t0 * NB * XP_DW;
    y += (size_t)t0 * N;
    if (yf) yf += (size_t)t0 * N;
    M = min(M - t0, MMA_TOK * TG);
  }
  uint32_t* sbl = lds + TG * TGO;
  float* part = reinterpret_cast<float*>(sbl + NWV * 16 * NQ);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = wave % C, tl = wave / C;
  const int n = lane & 15, g = lane >> 4;
  const int r = gs / 32, P = sb_row_len(K, gs);
  const int ntiles = (N + 15) / 16, ngroups = (ntiles + TPG - 1) / TPG;
  uint32_t* mysb = sbl + wave * 16 * NQ;
  // A operand of lane (A row = token (lane & 15) >> 2, limb lane & 3; word g); p, SX of token g
  const uint32_t* xa = lds + (size_t)((lane & 15) >> 2) * NB * MB_DW + (lane & 3) * 8 + 2 * g;
  const uint32_t* xps = lds + (size_t)g * NB * MB_DW + 32;
  // activations once per workgroup
  {
    MmaStage<NB, TG, 64 * NWV> stg;
    stg.load(xp, M);
    stg.store(lds);
  }
  __syncthreads();
  // this tile's (scale, bias) pairs of the class's blocks q = 0..NQ-1 (block c + C q), gathered into
  // this wave's LDS region [16][NQ] (pair q of row rr at rr * NQ + q), all at once (gather_all) or
  // body by body (gather_body, QB blocks each, one body ahead); the weights in bodies of BC
  // four-block chunks (lane group g: block g of each chunk), one body ahead
  constexpr int NG = (16 * NQ + 63) / 64;
  auto gather_all = [&](int tile, uint32_t (&gv)[NG]) {
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      const int e = lane + 64 * k, rr = e / NQ, q = e - rr * NQ, j = c + C * q;
      const int rw = tile * 16 + rr;
      gv[k] = e < 16 * NQ ? sbp[(size_t)(rw < N ? rw : N - 1) * P + ((j % L) / r) * IT + j / L] : 0u;
    }
  };
  constexpr int QB = 4 * BC;
  constexpr int NGB = (16 * QB + 63) / 64;
  auto gather_body = [&](int tile, int body, uint32_t (&gv)[NGB]) {
#pragma unroll
    for (int k = 0; k < NGB; ++k) {
      const int e = lane + 64 * k, rr = e / QB, q = body * QB + (e - rr * QB), j = c + C * q;
      const int rw = tile * 16 + rr;
      gv[k] = e < 16 * QB ? sbp[(size_t)(rw < N ? rw : N - 1) * P + ((j % L) / r) * IT + j / L] : 0u;
    }
  };
  auto put_body = [&](int body, const uint32_t (&gv)[NGB]) {
#pragma unroll
    for (int k = 0; k < NGB; ++k) {
      const int e = lane + 64 * k, rr = e / QB, q = body * QB + (e - rr * QB);
      if (e < 16 * QB) mysb[rr * NQ + q] = gv[k];  // this wave's region: read back by this wave only
    }
  };
  auto row_ptr = [&](int tile) {
    const int rw = tile * 16 + n;
    return wq + (size_t)(rw < N ? rw : N - 1) * (K / 8);
  };
  uint4 wv[2][BC];
  auto load_body = [&](const uint32_t* wrow, int ch0, int buf) {
#pragma unroll
    for (int cb = 0; cb < BC; ++cb) wv[buf][cb] = ldg16(wrow + (size_t)(c + C * (4 * (ch0 + cb) + g)) * 4);
  };
  // XPF (a launch whose workgroups walk several tile groups) with an even number of bodies per
  // tile: the pairs go body by body, and the last body computes buffer 1 while the next tile
  // group's first body (buffer 0) is loaded, so a workgroup waits for HBM once, not once per
  // group.  After its last group a workgroup loads rows 0..15 there instead (no branch around the
  // loads; cache hits, unused).  Taken with two token groups only: with one, the registers it
  // needs cost the second workgroup per CU, which hides more (measured).
  constexpr bool XP = XPF && (NCH / BC) % 2 == 0;
  uint32_t gvb[NGB];
  bool pref = false;  // this group's first body in flight from the previous group
  int iter = 0;
  for (int grp = blockIdx.x; grp < ngroups; grp += gridDim.x, ++iter) {
    const int tile = grp * TPG + tl;
    const int row = tile * 16 + n;
    const uint32_t* wrow = row_ptr(tile);
    if constexpr (XP) {
      if (!pref) {
        gather_body(tile, 0, gvb);
        asm volatile("" ::: "memory");  // the pair gathers ahead of the weight loads
        load_body(wrow, 0, 0);
        asm volatile("" ::: "memory");
      }
    } else {
      uint32_t gv[NG];
      gather_all(tile, gv);
      asm volatile("" ::: "memory");  // the pair gathers ahead of the weight loads
      load_body(wrow, 0, 0);
      asm volatile("" ::: "memory");
#pragma unroll
      for (int k = 0; k < NG; ++k)
        if (lane + 64 * k < 16 * NQ) mysb[lane + 64 * k] = gv[k];  // this wave's region: read back by this wave only
    }
    const int ngrp = grp + (int)gridDim.x;
    const bool next = XP && ngrp < ngroups;
    float acc[TG][LC];
#pragma unroll
    for (int tq = 0; tq < TG; ++tq)
#pragma unroll
      for (int u = 0; u < LC; ++u) acc[tq][u] = 0.0f;
#pragma unroll 1
    for (int ch0 = 0; ch0 < NCH; ch0 += 2 * BC) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int cbase = ch0 + half * BC;
        if (cbase >= NCH) break;  // uniform
        if constexpr (XP) {
          put_body(cbase / BC, gvb);  // this body's pairs
          if (cbase + BC < NCH) {
            gather_body(tile, cbase / BC + 1, gvb);
            asm volatile("" ::: "memory");
            load_body(wrow, cbase + BC, half ^ 1);
          } else if (half == 1) {
            const int nt = next ? ngrp * TPG + tl : 0;
            gather_body(nt, 0, gvb);
            asm volatile("" ::: "memory");
            load_body(row_ptr(nt), 0, 0);
          }
        } else {
          if (cbase + BC < NCH) load_body(wrow, cbase + BC, half ^ 1);
        }
#pragma unroll
        for (int cb = 0; cb < BC; ++cb) {
          const int ch = cbase + cb;
          const uint4 w = wv[half][cb];
          // 4x4 transpose across the lane groups: T[b] at lane group g = word g of block b of the chunk
          const auto p0 = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
          const auto p1 = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
          const auto q0 = __builtin_amdgcn_permlane16_swap(p0[0], p1[0], false, false);
          const auto q1 = __builtin_amdgcn_permlane16_swap(p0[1], p1[1], false, false);
          const uint32_t T[4] = {q0[0], q0[1], q1[0], q1[1]};
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int q = 4 * ch + b, j = c + C * q;
            const long bop = (long)(T[b] & 0x0f0f0f0fu) | ((long)((T[b] >> 4) & 0x0f0f0f0fu) << 32);
            const uint32_t sb = mysb[n * NQ + q];
#pragma unroll
            for (int tq = 0; tq < TG; ++tq) {
              long aop;
              __builtin_memcpy(&aop, xa + tq * TGO + (size_t)j * MB_DW, 8);
              v4i_t d = {0, 0, 0, 0};
              d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, d, 0, 0, 0);
              const int low = d[0] + 128 * d[1] + 16384 * d[2];
              const float dx = __builtin_fmaf((float)d[3], 65536.0f, (float)low);
              uint2 ps;
              __builtin_memcpy(&ps, xps + tq * TGO + (size_t)j * MB_DW, 8);
              float& a = acc[tq][(4 * cb + b + 4 * BC * half) % LC];  // chain (j % L) / C, in block order
              a = __builtin_fmaf(__uint_as_float(sb << 16), dx * __uint_as_float(ps.x), a);
              a = __builtin_fmaf(__uint_as_float(sb & 0xffff0000u), __uint_as_float(ps.y), a);
            }
          }
        }
        asm volatile("" ::: "memory");  // one body's operands live at a time (no LDS reads hoisted across)
      }
    }
    pref = next;
    float v[TG];
#pragma unroll
    for (int tq = 0; tq < TG; ++tq) {
      fold_levels<LC / 2>(acc[tq]);  // butterfly levels L/2 .. C: this class's chains
      v[tq] = acc[tq][0];
    }
    if constexpr (C > 1) {
      float* pb = part + (iter & 1) * NWV * TG * 64;  // by parity: the next write to it is two barriers away
#pragma unroll
      for (int tq = 0; tq < TG; ++tq) pb[(wave * TG + tq) * 64 + lane] = v[tq];
      __syncthreads();
#pragma unroll
      for (int tq = 0; tq < TG; ++tq) {
        float pc[C];
#pragma unroll
        for (int q = 0; q < C; ++q) pc[q] = pb[((tl * C + q) * TG + tq) * 64 + lane];
        fold_levels<C / 2>(pc);  // levels C/2 .. 1 across the classes
        v[tq] = pc[0];
      }
    }
#pragma unroll
    for (int tq = 0; tq < TG; ++tq) {
      const int tok = tq * MMA_TOK + g;
      if (c == 0 && tok < M && row < N) {
        y[(size_t)tok * N + row] = f2bf(v[tq]);
        if (yf) yf[(size_t)tok * N + row] = v[tq];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Dense GEMM on the matrix cores for a batch of many tokens (a prefill batch), with the same bits
// as k_qmv and k_qmv_mma: one weight operand serves 4 QT tokens.  A workgroup owns 128 rows (eight
// waves of 16) and 4 QT tokens, and walks K chain by chain.  The butterfly that folds the lane
// rule's L chains (level S = L/2 .. 1: v[u] += v[u + S]) is a perfect binary tree over the chains
// taken in bit-reversed order (L = 8: ((c0 + c4) + (c2 + c6)) + ((c1 + c5) + (c3 + c7))), so the
// chains are finished in that order, four per group (leaves 4q .. 4q + 3, folded as ((a + b) +
// (c + d))), and the groups fold by a binary counter over a stack of log2(L/4) subtrees: 4 QT
// (token, row) sums per chain of the group and one per stack level live at a time, whatever L.
// Step (q, it) stages block u + L it of each of the group's four chains u for the workgroup's
// tokens in LDS (the four-limb layout of k_qmv_mma, double buffered); each lane group loads one of
// the four blocks' 16-byte rows and the 4x4 transpose gives every lane group word g of all four.
// The next step's weights, (scale, bias) pairs and activation words are in flight while a step is
// computed.  Every chain adds its blocks in K order from 0 with the block combine of k_qmv_mma.
constexpr int QMM_THREADS = 512;
constexpr int QMM_ROWS = 128;     // eight waves x 16 rows
constexpr int QMM_MIN_ROWS = 1024;  // smallest matrix the batch GEMM takes (fewer rows: too few workgroups)

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

template <int L, int IT, int QT>
__global__ __launch_bounds__(QMM_THREADS) void k_qmm(const uint32_t* __restrict__ wq, const uint32_t* __restrict__ sbp,
                                                    int N, int K, int gs, const uint32_t* __restrict__ xp, int M,
                                                    bf16* __restrict__ y, float* __restrict__ yf, int tiles,
                                                    int tblocks) {
  constexpr int NB = L * IT;
  constexpr int QTOK = MMA_TOK * QT;                // tokens per workgroup
  constexpr int LOGL = ilog2(L), LOGQ = LOGL - 2;   // stack levels: subtrees of 4, 8, .. L/2 chains
  constexpr int STEPS = (L / 4) * IT;
  constexpr int SDW = QTOK * 4 * MB_DW;             // one stage: [token][block of the group][MB_DW]
  constexpr int NU = QTOK * 4 * 8 / QMM_THREADS;    // activation units (token, block, word, even/odd)
  static_assert(L >= 4 && (1 << LOGL) == L && NU >= 1 && NU * QMM_THREADS == QTOK * 32,
                "four chains per group, whole units per thread");
  extern __shared__ uint32_t lds[];
  // workgroup id -> (XCD id % 8, k = id / 8): the token blocks of a row tile are consecutive
  // workgroups of one XCD, so they read the tile's weights through one L2
  const int xcd = (int)blockIdx.x & 7, kk = (int)blockIdx.x >> 3;
  const int tile = (kk / tblocks) * 8 + xcd, tb = kk - (kk / tblocks) * tblocks;
  if (tile >= tiles) return;  // whole workgroup, before any barrier
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int row = tile * QMM_ROWS + wave * 16 + n;
  const int rc = row < N ? row : N - 1;
  const int rs = gs == 32 ? 0 : gs == 64 ? 1 : 2;  // log2 of the blocks per scale group
  const uint32_t* wrow = wq + (size_t)rc * (K / 8);
  const uint32_t* srow = sbp + (size_t)rc * sb_row_len(K, gs);
  const int m0 = tb * QTOK, Mt = min(M - m0, QTOK);
  xp += (size_t)m0 * NB * XP_DW;
  // chain of leaf position i (bit reversal over log2 L bits)
  auto chain = [](int i) { return (int)(__builtin_bitreverse32((uint32_t)i) >> (32 - LOGL)); };
  // activation words of step s: unit (token t, block b, word ge >> 1, even/odd ge & 1); units with
  // ge < 2 also carry word ge of the block's (p, SX) pair, the others a copy into the block's pad
  // dwords, so every thread runs the same loads and stores (no branch inside a step)
  uint32_t aw[NU][4];
  auto load_act = [&](int s) {
    const int q = s / IT, it = s - q * IT;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = threadIdx.x + k * QMM_THREADS;
      const int t = u >> 5, b = (u >> 3) & 3, ge = u & 7;
      const int j = chain(4 * q + b) + L * it;  // < NB for every step index
      const bool in = t < Mt;
      const uint32_t* src = xp + ((size_t)(in ? t : 0) * NB + j) * XP_DW;
      const uint32_t* sw = src + ((ge & 1) ? 4 : 0) + (ge >> 1);
      const uint32_t v0 = sw[0], v1 = sw[8], v2 = sw[16], v3 = src[24 + (ge & 1)];
      aw[k][0] = in ? v0 : 0u;
      aw[k][1] = in ? v1 : 0u;
      aw[k][2] = in ? v2 : 0u;
      aw[k][3] = in ? v3 : 0u;
    }
  };
  auto store_act = [&](uint32_t* st) {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = threadIdx.x + k * QMM_THREADS;
      const int t = u >> 5, b = (u >> 3) & 3, ge = u & 7;
      const uint32_t w0 = aw[k][0], w1 = aw[k][1];
      uint32_t* blk = st + (t * 4 + b) * MB_DW;
      uint32_t* dst = blk + 2 * (ge >> 1) + (ge & 1);
      dst[0] = w0 & 0x7f7f7f7fu;                                          // bits 0-6
      dst[8] = ((w0 >> 7) & 0x01010101u) | ((w1 << 1) & 0x7e7e7e7eu);    // bits 7-13
      dst[16] = (w1 >> 6) & 0x03030303u;                                  // bits 14-15
      dst[24] = aw[k][2];                                                 // bits 16-23 (signed)
      blk[(ge < 2 ? 32 : 34) + (ge & 1)] = aw[k][3];                      // p, SX (or the pad)
    }
  };
  // weights and (scale, bias) pairs of step s for this lane's row
  uint4 wc, wn;
  uint32_t pc[4], pn[4];
  auto load_w = [&](int s, uint4& w, uint32_t (&p)[4]) {  // cached: the row tile's other token blocks reread it
    const int q = s / IT, it = s - q * IT;
    w = *reinterpret_cast<const uint4*>(wrow + (size_t)(chain(4 * q + g) + L * it) * 4);
#pragma unroll
    for (int b = 0; b < 4; ++b) p[b] = srow[(chain(4 * q + b) >> rs) * IT + it];
  };
  load_act(0);
  store_act(lds);
  load_w(0, wc, pc);
  load_act(1);  // past the last step the loads still address blocks of the matrix (unused)
  __syncthreads();
  float ch[4][QT], stk[LOGQ > 0 ? LOGQ : 1][QT], res[QT];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int tq = 0; tq < QT; ++tq) ch[b][tq] = 0.0f;
  // A operand of lane: token 4 tq + (lane & 15) / 4, limb lane & 3, word g; (p, SX) of token 4 tq + g
  const int aoff2 = ((((lane & 15) >> 2) * 4) * MB_DW + (lane & 3) * 8 + 2 * g) / 2;  // in uint2
  const int poff2 = ((g * 4) * MB_DW + 32) / 2;
#pragma unroll 1
  for (int s = 0; s < STEPS; ++s) {
    const int q = s / IT, it = s - q * IT;
    load_w(s + 1, wn, pn);
    const uint2* st2 = reinterpret_cast<const uint2*>(lds + (s & 1) * SDW);  // 8-byte LDS reads
    const auto p0 = __builtin_amdgcn_permlane32_swap(wc.x, wc.z, false, false);
    const auto p1 = __builtin_amdgcn_permlane32_swap(wc.y, wc.w, false, false);
    const auto q0 = __builtin_amdgcn_permlane16_swap(p0[0], p1[0], false, false);
    const auto q1 = __builtin_amdgcn_permlane16_swap(p0[1], p1[1], false, false);
    const uint32_t T[4] = {q0[0], q0[1], q1[0], q1[1]};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const long bop = (long)(T[b] & 0x0f0f0f0fu) | ((long)((T[b] >> 4) & 0x0f0f0f0fu) << 32);
      const uint32_t sb = pc[b];
      // the block's QT products first (independent), then their combines in token-group order
      v4i_t d[QT];
#pragma unroll
      for (int tq = 0; tq < QT; ++tq) {
        const long aop = *reinterpret_cast<const long*>(st2 + aoff2 + (tq * 16 + b) * (MB_DW / 2));
        const v4i_t z = {0, 0, 0, 0};
        d[tq] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, z, 0, 0, 0);
      }
#pragma unroll
      for (int tq = 0; tq < QT; ++tq) {
        const int low = d[tq][0] + 128 * d[tq][1] + 16384 * d[tq][2];
        const float dx = __builtin_fmaf((float)d[tq][3], 65536.0f, (float)low);
        const uint2 ps = st2[poff2 + (tq * 16 + b) * (MB_DW / 2)];
        float& a = ch[b][tq];
        a = __builtin_fmaf(__uint_as_float(sb << 16), dx * __uint_as_float(ps.x), a);
        a = __builtin_fmaf(__uint_as_float(sb & 0xffff0000u), __uint_as_float(ps.y), a);
      }
      __builtin_amdgcn_sched_barrier(0);  // one block's products and operands live at a time
    }
    store_act(lds + ((s + 1) & 1) * SDW);
    load_act(s + 2);
    __syncthreads();
    wc = wn;
#pragma unroll
    for (int b = 0; b < 4; ++b) pc[b] = pn[b];
    if (it == IT - 1) {  // the group's subtree ((a + b) + (c + d)), then the binary counter over the groups
#pragma unroll
      for (int tq = 0; tq < QT; ++tq) {
        float x = (ch[0][tq] + ch[1][tq]) + (ch[2][tq] + ch[3][tq]);
        bool open = true;
#pragma unroll
        for (int k = 0; k < LOGQ; ++k) {
          if (open) {
            if ((q >> k) & 1) {
              x = stk[k][tq] + x;
            } else {
              stk[k][tq] = x;
              open = false;
            }
          }
        }
        if (open) res[tq] = x;  // the last group (every bit of q set): the whole tree
#pragma unroll
        for (int b = 0; b < 4; ++b) ch[b][tq] = 0.0f;
      }
    }
  }
#pragma unroll
  for (int tq = 0; tq < QT; ++tq) {
    const int t = tq * MMA_TOK + g;
    if (t < Mt && row < N) {
      y[(size_t)(m0 + t) * N + row] = f2bf(res[tq]);
      if (yf) yf[(size_t)(m0 + t) * N + row] = res[tq];
    }
  }
}

// ---------------------------------------------------------------------------
// The MoE down projection of a prefill batch on the matrix cores (same bits as the slot-per-
// workgroup kernel): the batch's slots sorted by expert are cut into chunks of at most MQ_CHUNK
// slots of one expert (k_moe_sort), and a workgroup owns one chunk and 128 rows of H of the expert's
// down matrix, against the slots' prepared activation rows, into the slots' output rows.  The K
// walk is k_qmm's: chains in the butterfly's bit-reversed leaf order, groups of four folded by a
// binary counter, each weight operand serving every token group of the chunk that holds a slot.  A phase is one group of four chains: all IT blocks of each for
// the chunk's tokens are staged in LDS (double buffered, the next phase's activation words loaded
// during this one), and the weight rows stream one phase ahead (a ring of IT register buffers: an
// expert's rows are read once per chunk, so the walk waits on HBM unless many loads are in flight).
template <int L, int IT>
__global__ __launch_bounds__(QMM_THREADS) void k_moe_qmm(MoeArgs a, int tiles) {
  constexpr int QT = MQ_CHUNK / MMA_TOK, QTOK = MQ_CHUNK, NB = L * IT;
  constexpr int LOGL = ilog2(L), LOGQ = LOGL - 2, NPH = L / 4, NBP = 4 * IT;
  constexpr int TR = 128;                                  // rows of the tile
  constexpr int PDW = QTOK * NBP * MB_DW;                   // one phase's staging buffer
  constexpr int NU = (QTOK * NBP * 8 + QMM_THREADS - 1) / QMM_THREADS;  // staging units per thread
  static_assert(L >= 4 && (1 << LOGL) == L, "groups of four chains");
  extern __shared__ uint32_t lds[];  // [NPH > 1 ? 2 : 1][QTOK][NBP][MB_DW]
  __shared__ int slot_l[QTOK];
  const int ck = (int)blockIdx.x / tiles, tile = (int)blockIdx.x - ck * tiles;
  if (ck >= *a.chunk_n) return;  // whole workgroup, before any barrier
  const int2 cv = reinterpret_cast<const int2*>(a.chunks)[ck];
  const int cnt = min(cv.y & 0xffff, QTOK), ev = cv.y >> 16;  // ev: expert + 1, 0 the shared expert
  const bool shared = ev == 0;
  const int e = shared ? 0 : min(ev - 1, a.E - 1);
  const int H = a.H, F = a.F, gs = a.gs;
  const int slots = a.nwin * a.M * (a.K + 1);
  const int K = F, N = H;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int row = tile * TR + wave * 16 + n, rc = row < N ? row : N - 1;
  const int rs = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  const int P = sb_row_len(K, gs);
  const size_t rbase = shared ? 0 : (size_t)e * N;
  const uint32_t* wm = shared ? a.sh_down_w : a.down_w;
  const uint32_t* sm = shared ? a.sh_down_sb : a.down_sb;
  const uint32_t* wrow = wm + (rbase + rc) * (size_t)(K / 8);
  const uint32_t* srow = sm + (rbase + rc) * (size_t)P;
  auto chain = [](int i) { return (int)(__builtin_bitreverse32((uint32_t)i) >> (32 - LOGL)); };
  uint4 wr[IT];
  uint32_t pr[IT][4];
  auto load_w = [&](int q, int it, uint4& w, uint32_t (&p)[4]) {  // any q: the blocks stay inside the matrix
    w = *reinterpret_cast<const uint4*>(wrow + (size_t)(chain(4 * q + g) + L * it) * 4);  // cached: an expert's chunks
#pragma unroll
    for (int b = 0; b < 4; ++b) p[b] = srow[(chain(4 * q + b) >> rs) * IT + it];
  };
#pragma unroll
  for (int it = 0; it < IT; ++it) load_w(0, it, wr[it], pr[it]);  // the weights first: they come from HBM
  if (threadIdx.x < QTOK)
    slot_l[threadIdx.x] = (int)threadIdx.x < cnt ? min(a.gorder[min(cv.x + (int)threadIdx.x, slots - 1)] & 0xffff, slots - 1)
                                                 : -1;
  __syncthreads();
  // staging units (token t, phase block pb = b * IT + it, word/half ge) of this thread, their rows
  const uint32_t* urow[NU];
  int uoff[NU];
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    const int u = threadIdx.x + k * QMM_THREADS;
    const int t = u / (NBP * 8), sl = t < QTOK ? slot_l[t] : -1;
    uoff[k] = sl >= 0 ? u - t * (NBP * 8) : -1;  // -1: a zero unit (no slot) or past the stage
    urow[k] = a.xp_act + (size_t)(sl >= 0 ? sl : 0) * NB * XP_DW;
  }
  uint32_t aw[NU][4];
  auto load_act = [&](int q) {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int o = uoff[k] < 0 ? 0 : uoff[k], pb = o >> 3, ge = o & 7, bb = pb / IT, it = pb - bb * IT;
      const uint32_t* src = urow[k] + (size_t)(chain(4 * q + bb) + L * it) * XP_DW;
      const uint32_t* sw = src + ((ge & 1) ? 4 : 0) + (ge >> 1);
      const uint32_t v0 = sw[0], v1 = sw[8], v2 = sw[16], v3 = src[24 + (ge & 1)];
      const bool in = uoff[k] >= 0;
      aw[k][0] = in ? v0 : 0u;
      aw[k][1] = in ? v1 : 0u;
      aw[k][2] = in ? v2 : 0u;
      aw[k][3] = in ? v3 : 0u;
    }
  };
  auto store_act = [&](uint32_t* st) {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = threadIdx.x + k * QMM_THREADS;
      if (u < QTOK * NBP * 8) {
        const int t = u / (NBP * 8), o = u - t * (NBP * 8), pb = o >> 3, ge = o & 7;
        uint32_t* blk = st + (t * NBP + pb) * MB_DW;
        uint32_t* dst = blk + 2 * (ge >> 1) + (ge & 1);
        dst[0] = aw[k][0] & 0x7f7f7f7fu;
        dst[8] = ((aw[k][0] >> 7) & 0x01010101u) | ((aw[k][1] << 1) & 0x7e7e7e7eu);
        dst[16] = (aw[k][1] >> 6) & 0x03030303u;
        dst[24] = aw[k][2];
        blk[(ge < 2 ? 32 : 34) + (ge & 1)] = aw[k][3];
      }
    }
  };
  load_act(0);
  store_act(lds);
  if (NPH > 1) load_act(1);
  __syncthreads();
  const int qte = (cnt + MMA_TOK - 1) / MMA_TOK;  // token groups holding a slot (uniform)
  float ch[4][QT], stk[LOGQ > 0 ? LOGQ : 1][QT], res[QT];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int tq = 0; tq < QT; ++tq) ch[b][tq] = 0.0f;
  // A operand of lane: token 4 tq + (lane & 15) / 4, limb lane & 3, word g; (p, SX) of token 4 tq + g
  const int aoff2 = ((((lane & 15) >> 2) * NBP) * MB_DW + (lane & 3) * 8 + 2 * g) / 2;
  const int poff2 = ((g * NBP) * MB_DW + 32) / 2;
  constexpr int TGS = MMA_TOK * NBP * MB_DW / 2;  // one token group, in uint2
#pragma unroll 1
  for (int q = 0; q < NPH; ++q) {
    const uint2* st2 = reinterpret_cast<const uint2*>(lds + (NPH > 1 ? (q & 1) * PDW : 0));
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const auto p0 = __builtin_amdgcn_permlane32_swap(wr[it].x, wr[it].z, false, false);
      const auto p1 = __builtin_amdgcn_permlane32_swap(wr[it].y, wr[it].w, false, false);
      const auto q0 = __builtin_amdgcn_permlane16_swap(p0[0], p1[0], false, false);
      const auto q1 = __builtin_amdgcn_permlane16_swap(p0[1], p1[1], false, false);
      const uint32_t T[4] = {q0[0], q0[1], q1[0], q1[1]};
      uint32_t sbv[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) sbv[b] = pr[it][b];
      load_w(q + 1, it, wr[it], pr[it]);  // the ring slot's block of the next phase
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int pb = b * IT + it;
        const long bop = (long)(T[b] & 0x0f0f0f0fu) | ((long)((T[b] >> 4) & 0x0f0f0f0fu) << 32);
        const uint32_t sb = sbv[b];
        v4i_t d[QT];
#pragma unroll
        for (int tq = 0; tq < QT; ++tq) {
          if (tq < qte) {
            const long aop = *reinterpret_cast<const long*>(st2 + aoff2 + tq * TGS + pb * (MB_DW / 2));
            const v4i_t z = {0, 0, 0, 0};
            d[tq] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, z, 0, 0, 0);
          }
        }
#pragma unroll
        for (int tq = 0; tq < QT; ++tq) {
          if (tq < qte) {
            const int low = d[tq][0] + 128 * d[tq][1] + 16384 * d[tq][2];
            const float dx = __builtin_fmaf((float)d[tq][3], 65536.0f, (float)low);
            const uint2 ps = st2[poff2 + tq * TGS + pb * (MB_DW / 2)];
            float& acc = ch[b][tq];
            acc = __builtin_fmaf(__uint_as_float(sb << 16), dx * __uint_as_float(ps.x), acc);
            acc = __builtin_fmaf(__uint_as_float(sb & 0xffff0000u), __uint_as_float(ps.y), acc);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // the group's subtree ((a + b) + (c + d)), then the binary counter over the groups
#pragma unroll
    for (int tq = 0; tq < QT; ++tq) {
      float x = (ch[0][tq] + ch[1][tq]) + (ch[2][tq] + ch[3][tq]);
      bool open = true;
#pragma unroll
      for (int k = 0; k < LOGQ; ++k) {
        if (open) {
          if ((q >> k) & 1) {
            x = stk[k][tq] + x;
          } else {
            stk[k][tq] = x;
            open = false;
          }
        }
      }
      if (open) res[tq] = x;
#pragma unroll
      for (int b = 0; b < 4; ++b) ch[b][tq] = 0.0f;
    }
    if (NPH > 1 && q + 1 < NPH) {  // the next phase's words -> the other buffer, then the one after into registers
      store_act(lds + ((q + 1) & 1) * PDW);
      load_act(q + 2 < NPH ? q + 2 : q + 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int tq = 0; tq < QT; ++tq) {
    const int t = tq * MMA_TOK + g;
    const int sl = slot_l[t];
    if (sl >= 0 && row < N) a.r[(size_t)sl * H + row] = f2bf(res[tq]);
  }
}

// ---------------------------------------------------------------------------
// Prepared blocks xp [M][NB][XP_DW] -> the matrix cores' four-limb layout in memory, xmb
// [M][NB][MB_DW] (limbs at dwords 0..31, p and SX at 32, 33): one thread per (token, block, word,
// even/odd) unit, as the GEMMs' LDS staging converts them.
__global__ __launch_bounds__(256) void k_xmb(const uint32_t* __restrict__ xp, int units, uint32_t* __restrict__ xmb) {
  const int u = blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const int blk = u >> 3, ge = u & 7;  // blk = token * NB + block
  const uint32_t* src = xp + (size_t)blk * XP_DW;
  const uint32_t* sw = src + ((ge & 1) ? 4 : 0) + (ge >> 1);
  const uint32_t w0 = sw[0], w1 = sw[8];
  uint32_t* dst = xmb + (size_t)blk * MB_DW + 2 * (ge >> 1) + (ge & 1);
  dst[0] = w0 & 0x7f7f7f7fu;                                          // bits 0-6
  dst[8] = ((w0 >> 7) & 0x01010101u) | ((w1 << 1) & 0x7e7e7e7eu);    // bits 7-13
  dst[16] = (w1 >> 6) & 0x03030303u;                                  // bits 14-15
  dst[24] = sw[16];                                                   // bits 16-23 (signed)
  if (ge < 2) xmb[(size_t)blk * MB_DW + 32 + ge] = src[24 + ge];      // p, SX
}

// Batch GEMM for matrices of few rows and long K (the hyper-connection mixer's down and inject
// projections over a prefill batch), same bits as k_qmv: a workgroup owns one 16-row tile of one
// of two matrices and 4 QT tokens; its four waves take a quarter of the chain groups each (a
// subtree of L/4 chains of the butterfly's bit-reversed leaf order, folded as in k_qmm), and the
// quarters meet in LDS as ((n0 + n1) + (n2 + n3)).  A operands and (p, SX) pairs come straight
// from the four-limb layout in memory (k_xmb), each step's loads in flight during the previous one.
constexpr int QMN_THREADS = 256;

template <int L, int IT, int QT>
__global__ __launch_bounds__(QMN_THREADS) void k_qmn(const uint32_t* __restrict__ wq1, const uint32_t* __restrict__ sb1,
                                                    int N1, bf16* __restrict__ y1, const uint32_t* __restrict__ wq2,
                                                    const uint32_t* __restrict__ sb2, int N2, bf16* __restrict__ y2,
                                                    int K, int gs, const uint32_t* __restrict__ xmb, int M, int tiles1,
                                                    int tiles) {
  constexpr int NB = L * IT, P = 4, G = L / 4 / P, LOGG = ilog2(G), STEPS = G * IT, LOGL = ilog2(L);
  static_assert(L >= 16 && (1 << LOGL) == L && (1 << LOGG) == G, "four quarters of whole chain groups");
  __shared__ float part[P][QT][64];
  // workgroup id -> (XCD id % 8, k = id / 8): every tile of a token block on one XCD, so its L2 holds
  // the block's activations for all of them
  const int xcd = (int)blockIdx.x & 7, kk = (int)blockIdx.x >> 3;
  const int tb = (kk / tiles) * 8 + xcd, tile = kk - (kk / tiles) * tiles;
  if (tb * MMA_TOK * QT >= M) return;  // whole workgroup, before the barrier
  const int p = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const bool second = tile >= tiles1;
  const uint32_t* wq = second ? wq2 : wq1;
  const uint32_t* sbp = second ? sb2 : sb1;
  const int N = second ? N2 : N1;
  const int row = (second ? tile - tiles1 : tile) * 16 + n, rc = row < N ? row : N - 1;
  const int rs = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  const uint32_t* wrow = wq + (size_t)rc * (K / 8);
  const uint32_t* srow = sbp + (size_t)rc * sb_row_len(K, gs);
  const int m0 = tb * MMA_TOK * QT;
  // this lane's A rows (token 4 tq + (lane & 15) / 4, limb lane & 3, word g) and (p, SX) rows (token
  // 4 tq + g), tokens past M clamped (their sums are not stored)
  const uint2* xa[QT];
  const uint2* xs[QT];
#pragma unroll
  for (int tq = 0; tq < QT; ++tq) {
    const int ta = min(m0 + 4 * tq + ((lane & 15) >> 2), M - 1), ts = min(m0 + 4 * tq + g, M - 1);
    xa[tq] = reinterpret_cast<const uint2*>(xmb + (size_t)ta * NB * MB_DW + (lane & 3) * 8 + 2 * g);
    xs[tq] = reinterpret_cast<const uint2*>(xmb + (size_t)ts * NB * MB_DW + 32);
  }
  auto chain = [](int i) { return (int)(__builtin_bitreverse32((uint32_t)i) >> (32 - LOGL)); };
  struct Step {
    uint4 w;
    uint32_t pr[4];
    uint2 a[4][QT], ps[4][QT];
  };
  auto load = [&](int s, Step& d) {
    const int q = p * G + s / IT, it = s - (s / IT) * IT;
    d.w = *reinterpret_cast<const uint4*>(wrow + (size_t)(chain(4 * q + g) + L * it) * 4);  // cached: reread per token block
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int u = chain(4 * q + b), j = u + L * it;
      d.pr[b] = srow[(u >> rs) * IT + it];
#pragma unroll
      for (int tq = 0; tq < QT; ++tq) {
        d.a[b][tq] = xa[tq][(size_t)j * (MB_DW / 2)];
        d.ps[b][tq] = xs[tq][(size_t)j * (MB_DW / 2)];
      }
    }
  };
  float ch[4][QT], stk[LOGG > 0 ? LOGG : 1][QT], res[QT];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int tq = 0; tq < QT; ++tq) ch[b][tq] = 0.0f;
  auto compute = [&](int s, const Step& d) {
    const auto p0 = __builtin_amdgcn_permlane32_swap(d.w.x, d.w.z, false, false);
    const auto p1 = __builtin_amdgcn_permlane32_swap(d.w.y, d.w.w, false, false);
    const auto q0 = __builtin_amdgcn_permlane16_swap(p0[0], p1[0], false, false);
    const auto q1 = __builtin_amdgcn_permlane16_swap(p0[1], p1[1], false, false);
    const uint32_t T[4] = {q0[0], q0[1], q1[0], q1[1]};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const long bop = (long)(T[b] & 0x0f0f0f0fu) | ((long)((T[b] >> 4) & 0x0f0f0f0fu) << 32);
      const uint32_t sb = d.pr[b];
      v4i_t dd[QT];
#pragma unroll
      for (int tq = 0; tq < QT; ++tq) {
        long aop;
        __builtin_memcpy(&aop, &d.a[b][tq], 8);
        const v4i_t z = {0, 0, 0, 0};
        dd[tq] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, z, 0, 0, 0);
      }
#pragma unroll
      for (int tq = 0; tq < QT; ++tq) {
        const int low = dd[tq][0] + 128 * dd[tq][1] + 16384 * dd[tq][2];
        const float dx = __builtin_fmaf((float)dd[tq][3], 65536.0f, (float)low);
        float& a = ch[b][tq];
        a = __builtin_fmaf(__uint_as_float(sb << 16), dx * __uint_as_float(d.ps[b][tq].x), a);
        a = __builtin_fmaf(__uint_as_float(sb & 0xffff0000u), __uint_as_float(d.ps[b][tq].y), a);
      }
    }
    const int ql = s / IT;
    if (s - ql * IT == IT - 1) {  // the group's subtree, then the binary counter over this quarter's groups
#pragma unroll
      for (int tq = 0; tq < QT; ++tq) {
        float x = (ch[0][tq] + ch[1][tq]) + (ch[2][tq] + ch[3][tq]);
        bool open = true;
#pragma unroll
        for (int k = 0; k < LOGG; ++k) {
          if (open) {
            if ((ql >> k) & 1) {
              x = stk[k][tq] + x;
            } else {
              stk[k][tq] = x;
              open = false;
            }
          }
        }
        if (open) res[tq] = x;  // the quarter's last group: its whole subtree
#pragma unroll
        for (int b = 0; b < 4; ++b) ch[b][tq] = 0.0f;
      }
    }
  };
  Step d0, d1;
  load(0, d0);
#pragma unroll 1
  for (int s = 0; s < STEPS; s += 2) {
    load(s + 1 < STEPS ? s + 1 : s, d1);  // in range either way (unused past the end)
    compute(s, d0);
    load(s + 2 < STEPS ? s + 2 : s, d0);
    if (s + 1 < STEPS) compute(s + 1, d1);
  }
#pragma unroll
  for (int tq = 0; tq < QT; ++tq) part[p][tq][lane] = res[tq];
  __syncthreads();
  if (p == 0) {
#pragma unroll
    for (int tq = 0; tq < QT; ++tq) {
      const float v = (part[0][tq][lane] + part[1][tq][lane]) + (part[2][tq][lane] + part[3][tq][lane]);
      const int t = m0 + 4 * tq + g;
      if (t < M && row < N) (second ? y2 : y1)[(size_t)t * N + row] = f2bf(v);
    }
  }
}

// MLX affine quantisation of bf16 rows; one thread per group
// (MLX/backend/cpu/quantized.cpp:1158-1220).
__global__ void k_quantize(const bf16* __restrict__ w, int64_t groups, int gs, uint32_t* __restrict__ wq,
                           bf16* __restrict__ scales, bf16* __restrict__ biases) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const bf16* wg = w + gi * gs;
  float wmin = __uint_as_float(0x7f800000u), wmax = -wmin;
  for (int j = 0; j < gs; ++j) {
    const float v = bf2f(wg[j]);
    wmax = fmaxf(wmax, v);
    wmin = fminf(wmin, v);
  }
  const bool mask = fabsf(wmin) > fabsf(wmax);
  float scale = fmaxf((wmax - wmin) / 15.0f, 1e-7f);
  scale = mask ? scale : -scale;
  const float edge = mask ? wmin : wmax;
  const float q0 = __builtin_rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  for (int j = 0; j < gs / 8; ++j) {
    uint32_t word = 0;
    for (int t = 0; t < 8; ++t) {
      float v = __builtin_rintf((bf2f(wg[j * 8 + t]) - bias) / scale);
      v = fminf(fmaxf(v, 0.0f), 15.0f);
      word |= (uint32_t)v << (4 * t);
    }
    wq[gi * (gs / 8) + j] = word;
  }
  scales[gi] = f2bf(scale);
  biases[gi] = f2bf(bias);
}

// Philox4x32-10 (Salmon et al., SC'11).
__device__ __forceinline__ uint4 philox(uint4 c, uint2 k) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k.x += 0x9E3779B9u;
      k.y += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c.x), lo0 = 0xD2511F53u * c.x;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c.z), lo1 = 0xCD9E8D57u * c.z;
    c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
  }
  return c;
}

// Seeded N(0, sigma) bf16 values (Box-Muller over Philox); element i uses
// counter (i/4, tensor, 0, 0), so the values do not depend on the launch shape.
__global__ void k_randn_bf16(bf16* __restrict__ out, int64_t n, uint64_t seed, uint32_t tensor, float sigma) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i0 = q * 4;
  if (i0 >= n) return;
  const uint4 r = philox(make_uint4((uint32_t)q, (uint32_t)(q >> 32), tensor, 0u),
                         make_uint2((uint32_t)seed, (uint32_t)(seed >> 32)));
  const float u0 = ((r.x >> 8) + 0.5f) * 5.9604644775390625e-08f;
  const float u1 = (r.y >> 8) * 5.9604644775390625e-08f;
  const float u2 = ((r.z >> 8) + 0.5f) * 5.9604644775390625e-08f;
  const float u3 = (r.w >> 8) * 5.9604644775390625e-08f;
  const float r0 = sqrtf(-2.0f * __logf(u0)), r1 = sqrtf(-2.0f * __logf(u2));
  float s0, c0, s1, c1;
  __sincosf(6.2831853f * u1, &s0, &c0);
  __sincosf(6.2831853f * u3, &s1, &c1);
  const float v[4] = {r0 * c0, r0 * s0, r1 * c1, r1 * s1};
  for (int t = 0; t < 4 && i0 + t < n; ++t) out[i0 + t] = f2bf(v[t] * sigma);
}

__global__ void k_fill_bf16(bf16* __restrict__ out, int64_t n, bf16 v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = v;
}

// Packed (scale, bias) pairs of a q4 matrix in the walker's lane order: one
// thread per entry [row][q][it] = pair of the group of block q*r + L*it.
__global__ void k_pack_sb(const bf16* __restrict__ s, const bf16* __restrict__ b, int64_t N, int K, int gs,
                          uint32_t* __restrict__ out) {
  const int P = sb_row_len(K, gs), nbv = sb_entries_per_class(K), L = lanes_for_blocks(K / 32);
  const int r = gs / 32, nb = K / 32, ng = K / gs;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * P) return;
  const int64_t row = idx / P;
  const int e = (int)(idx % P), q = e / nbv, it = e % nbv;
  const int j = q * r + L * it;
  uint32_t v = 0;
  if (j < nb) {
    const int g = j / r;
    v = (uint32_t)s[row * ng + g] | ((uint32_t)b[row * ng + g] << 16);
  }
  out[idx] = v;
}

// ---------------------------------------------------------------------------
// host launchers

hipError_t launch_pack_sb(const bf16* s, const bf16* b, int64_t N, int K, int gs, uint32_t* out, hipStream_t st) {
  const int64_t n = N * sb_row_len(K, gs);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_pack_sb, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, b, N, K, gs, out);
  return hipGetLastError();
}

hipError_t launch_xprep(const bf16* x, int M, int K, uint32_t* xp, hipStream_t st) {
  const int n = M * (K / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_xprep, dim3((n + 7) / 8), dim3(256), 0, st, x, M, K, xp);
  return hipGetLastError();
}

// M tokens in windows of `win` (one window: a plain launch; more: grid Y, the row grid rounded
// up to whole XCD rounds so every window of a row range runs on the same XCD and L2).  win = 0
// (a prefill batch): windows and rows per workgroup chosen for about four workgroups per CU in
// all -- short windows where the rows are few, several row passes per workgroup where the
// windows are many -- with at most `cap` tokens per window (50 KB of LDS: three per CU).
template <int L, int IT>
static hipError_t qmv_li(const uint32_t* wq, const bf16* s, const bf16* b, const uint32_t* sb, int N, int K, int gs,
                         const uint32_t* xp, int M, bf16* y, float* yf, int win, hipStream_t st) {
  constexpr int rows_pass = 4 * (64 / L) * 2;
  const int passes = (N + rows_pass - 1) / rows_pass;
  int per = (passes + 511) / 512;  // about two workgroups per CU, at least one pass each
  const bool batch = win <= 0;     // a prefill batch: its windows reread the rows, so cached loads
  if (batch) {
    int cap = (int)((50 * 1024) / ((size_t)(K / 32) * XP_DW * 4));  // three workgroups' LDS per CU
    cap = cap < 1 ? 1 : cap;
    const int want = 4 * device_cus();
    int nw = (want + passes - 1) / passes;
    nw = std::max((M + cap - 1) / cap, std::min(M, nw));
    win = (M + nw - 1) / nw;
    nw = (M + win - 1) / win;
    const int g = std::max(1, std::min(passes, (want + nw - 1) / nw));
    per = (passes + g - 1) / g;
  }
  const int nwin = (M + win - 1) / win;
  const size_t lds = (size_t)(M < win ? M : win) * (K / 32) * XP_DW * 4;
  auto go = [&](auto kern, size_t& cur, int rows_per_wg, int nthr) {
    int grid = (N + rows_per_wg - 1) / rows_per_wg;
    if (nwin > 1) grid = (grid + 7) / 8 * 8;
    hipError_t e = ensure_lds(kern, lds, cur);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(grid, nwin), dim3(nthr), lds, st, wq, s, b, sb, N, K, gs, xp, M, y, yf, rows_per_wg,
                       win);
    return hipGetLastError();
  };
  static size_t c00 = 0, c01 = 0, c10 = 0, c11 = 0, c5 = 0;
  if (batch) return sb ? go(k_qmv<L, IT, true, true, 4>, c11, per * rows_pass, 256)
                       : go(k_qmv<L, IT, true, false, 4>, c10, per * rows_pass, 256);
  // Equal windows whose workgroups a five-wave launch (a fifth more rows a pass) spreads with a quarter
  // fewer rows on the busiest CU (launch workgroups spread evenly): the K = 6144 output projections at
  // four and six tokens, two windows of 2 x 160 four-wave workgroups on 256 CUs, the 64 CUs with two
  // finishing last (12.35 -> 11.58 us at 4 tokens).  Not taken: a shorter last window (three tokens:
  // 2 + 1) leaves those CUs less loaded and the larger workgroups cost more (11.10 -> 11.55 us); one
  // window (GDN in-projection at one and two tokens, 258 two-pass four-wave workgroups against 412
  // one-pass five-wave ones: 12.6 -> 14.4 us, 16.3 -> 17.8).
  if (sb && nwin > 1 && M % win == 0) {
    const int cus = device_cus();
    constexpr int r5 = 5 * (64 / L) * 2;
    const int per5 = ((N + r5 - 1) / r5 + 511) / 512;
    auto busiest = [&](int rpw) {
      const int g = (N + rpw - 1) / rpw, w = (nwin > 1 ? (g + 7) / 8 * 8 : g) * nwin;
      return (int64_t)((w + cus - 1) / cus) * rpw;
    };
    if (4 * busiest(per5 * r5) <= 3 * busiest(per * rows_pass))
      return go(k_qmv<L, IT, false, true, 5>, c5, per5 * r5, 320);
  }
  return sb ? go(k_qmv<L, IT, false, true, 4>, c01, per * rows_pass, 256)
            : go(k_qmv<L, IT, false, false, 4>, c00, per * rows_pass, 256);
}

static hipError_t qmv_tokens(const uint32_t* wq, const bf16* s, const bf16* b, const uint32_t* sb, int N, int K,
                             int gs, const uint32_t* xp, int M, bf16* y, float* yf, int win, hipStream_t st) {
  MTPX_QROW_DISPATCH(K / 32, qmv_li, wq, s, b, sb, N, K, gs, xp, M, y, yf, win, st);
}

template <int L, int IT, int C, int TG, int NWV = 8>
constexpr size_t mma_lds_bytes() {
  return (size_t)MMA_TOK * TG * L * IT * MB_DW * 4 + (size_t)NWV * 16 * (L * IT / C) * 4 + (size_t)2 * NWV * TG * 64 * 4;
}

// hipErrorNotReady: a launch of two token groups (one workgroup per CU) whose tile groups would
// need a second, nearly empty round of workgroups -- the caller runs four tokens per launch instead.
// M > 4 TG tokens: windows of 4 TG in grid Y, one workgroup per tile group (rounded up to whole XCD
// rounds, so the windows of a tile group share an XCD and its L2).
template <int L, int IT, int C, int TG, int NWV>
static hipError_t qmv_mma_launch(const uint32_t* wq, const uint32_t* sb, int N, int K, int gs, const uint32_t* xp,
                                 int M, bf16* y, float* yf, hipStream_t st) {
  constexpr size_t lds = mma_lds_bytes<L, IT, C, TG, NWV>();
  const int groups = ((N + 15) / 16 + NWV / C - 1) / (NWV / C);
  const int per_cu = lds <= 50 * 1024 ? 3 : lds <= 78 * 1024 ? 2 : 1;  // workgroups resident per CU
  const int slots = per_cu * device_cus();
  const int nwin = (M + MMA_TOK * TG - 1) / (MMA_TOK * TG);
  if (nwin == 1 && TG > 1 && groups > slots && groups < 4 * slots) return hipErrorNotReady;
  const int grid = nwin > 1 ? (groups + 7) / 8 * 8 : groups < slots ? groups : slots;
  if constexpr (TG == 2) {  // two token groups (one workgroup per CU)
    if (nwin == 1 && groups >= 2 * grid) {  // workgroups walk several tile groups: the next one's first body in flight
      static size_t cur = 0;
      hipError_t e = ensure_lds(k_qmv_mma<L, IT, C, TG, true, NWV>, lds, cur);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((k_qmv_mma<L, IT, C, TG, true, NWV>), dim3(grid, nwin), dim3(64 * NWV), lds, st, wq, sb, N,
                         K, gs, xp, M, y, yf);
      return hipGetLastError();
    }
  }
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_qmv_mma<L, IT, C, TG, false, NWV>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_qmv_mma<L, IT, C, TG, false, NWV>), dim3(grid, nwin), dim3(64 * NWV), lds, st, wq, sb, N, K,
                     gs, xp, M, y, yf);
  return hipGetLastError();
}

// One token group: ten-wave workgroups (five tiles of two classes) where they fit a launch that
// eight-wave ones do not in one round -- one workgroup per CU for one window (with eight, the few CUs
// that take a second workgroup finish last: GDN in-projection, 258 groups on 256 CUs), within the
// resident workgroups for several windows (eight: 2 x 264 workgroups of four tokens where 512 fit).
template <int L, int IT, int C, int TG>
static hipError_t qmv_mma_c(const uint32_t* wq, const uint32_t* sb, int N, int K, int gs, const uint32_t* xp, int M,
                            bf16* y, float* yf, hipStream_t st) {
  if constexpr (TG == 1 && C == 2 && mma_lds_bytes<L, IT, C, TG, 10>() <= 78 * 1024 &&
                mma_lds_bytes<L, IT, C, TG, 8>() > 50 * 1024) {  // (two workgroups per CU either way)
    const int tiles = (N + 15) / 16, g8 = (tiles + 3) / 4, g10 = (tiles + 4) / 5, cus = device_cus();
    const int nwin = (M + MMA_TOK - 1) / MMA_TOK;
    const bool ten = nwin == 1 ? g8 > cus && g10 <= cus
                               : (g8 + 7) / 8 * 8 * nwin > 2 * cus && (g10 + 7) / 8 * 8 * nwin <= 2 * cus;
    if (ten) return qmv_mma_launch<L, IT, C, TG, 10>(wq, sb, N, K, gs, xp, M, y, yf, st);
  }
  return qmv_mma_launch<L, IT, C, TG, 8>(wq, sb, N, K, gs, xp, M, y, yf, st);
}

// One token group: two workgroups per CU at least (above that the dot-product path is faster,
// measured).  Two token groups (five to eight tokens): one workgroup per CU, the LDS of a CU.
template <int L, int IT, int C, int TG>
constexpr bool mma_c_ok() {
  constexpr int NB = L * IT, LC = L / C, BC = mma_body_chunks<L, IT, C>();
  return C >= 2 && C <= L && LC <= 16 && NB % (4 * C) == 0 && (NB / C / 4) % BC == 0 &&
         mma_lds_bytes<L, IT, C, TG>() <= (TG == 1 ? 80 : 144) * 1024;
}

// Chain classes per tile: at least two (the per-wave scale/bias region of one class fits beside
// the activations), then the fewest that give about eight waves per CU; with two token groups
// (one workgroup per CU) four classes first, for twice the tile groups to spread over the CUs.
template <int L, int IT, int TG>
static hipError_t qmv_mma_li(const uint32_t* wq, const uint32_t* sb, int N, int K, int gs, const uint32_t* xp, int M,
                             bf16* y, float* yf, hipStream_t st) {
  const int tiles = (N + 15) / 16, want = 8 * device_cus();
  if constexpr (TG == 2 && mma_c_ok<L, IT, 4, TG>()) return qmv_mma_c<L, IT, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
  if constexpr (mma_c_ok<L, IT, 2, TG>()) {
    if (tiles * 2 >= want) return qmv_mma_c<L, IT, 2, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
  }
  if constexpr (mma_c_ok<L, IT, 4, TG>()) {
    if (tiles * 4 >= want) return qmv_mma_c<L, IT, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
  }
  if constexpr (mma_c_ok<L, IT, 8, TG>()) return qmv_mma_c<L, IT, 8, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
  if constexpr (mma_c_ok<L, IT, 4, TG>()) return qmv_mma_c<L, IT, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
  if constexpr (mma_c_ok<L, IT, 2, TG>()) return qmv_mma_c<L, IT, 2, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
  return hipErrorNotSupported;
}

// The matrix-core path takes 2..8 tokens of a matrix with packed scale/bias
// rows whose blocks tile the lanes exactly in four-block chunks.
static bool qmv_mma_ok(const uint32_t* sb, int K, int M) {
  const int nb = K / 32, L = lanes_for_blocks(nb);
  return sb && M >= 2 && nb % L == 0 && nb % 4 == 0;
}

template <int TG>
static hipError_t qmv_mma(const uint32_t* wq, const uint32_t* sb, int N, int K, int gs, const uint32_t* xp, int M,
                          bf16* y, float* yf, hipStream_t st) {
  const int nb = K / 32, L = lanes_for_blocks(nb), IT = nb / L;
  switch (L * 16 + IT) {
    case 16 * 16 + 4: return qmv_mma_li<16, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 16 * 16 + 5: return qmv_mma_li<16, 5, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 32 * 16 + 4: return qmv_mma_li<32, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 32 * 16 + 6: return qmv_mma_li<32, 6, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 64 * 16 + 4: return qmv_mma_li<64, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 64 * 16 + 5: return qmv_mma_li<64, 5, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 8 * 16 + 4: return qmv_mma_li<8, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 8 * 16 + 5: return qmv_mma_li<8, 5, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 4 * 16 + 4: return qmv_mma_li<4, 4, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 4 * 16 + 5: return qmv_mma_li<4, 5, TG>(wq, sb, N, K, gs, xp, M, y, yf, st);
    default: return hipErrorNotSupported;
  }
}

template <int L, int IT, int TG>
constexpr bool mma_any_c() {
  return mma_c_ok<L, IT, 2, TG>() || mma_c_ok<L, IT, 4, TG>() || mma_c_ok<L, IT, 8, TG>();
}

template <int TG>
static bool qmv_mma_shape(int K) {
  const int nb = K / 32, L = lanes_for_blocks(nb), IT = nb / L;
  switch (L * 16 + IT) {
    case 16 * 16 + 4: return mma_any_c<16, 4, TG>();
    case 16 * 16 + 5: return mma_any_c<16, 5, TG>();
    case 32 * 16 + 4: return mma_any_c<32, 4, TG>();
    case 32 * 16 + 6: return mma_any_c<32, 6, TG>();
    case 64 * 16 + 4: return mma_any_c<64, 4, TG>();
    case 64 * 16 + 5: return mma_any_c<64, 5, TG>();
    case 8 * 16 + 4: return mma_any_c<8, 4, TG>();
    case 8 * 16 + 5: return mma_any_c<8, 5, TG>();
    case 4 * 16 + 4: return mma_any_c<4, 4, TG>();
    case 4 * 16 + 5: return mma_any_c<4, 5, TG>();
    default: return false;
  }
}

// Batch GEMM: row tiles of 128 in rounds of eight (one per XCD) times token blocks of 4 QT.
template <int L, int IT, int QT>
static hipError_t qmm_li(const uint32_t* wq, const uint32_t* sb, int N, int K, int gs, const uint32_t* xp, int M,
                         bf16* y, float* yf, hipStream_t st) {
  constexpr size_t lds = (size_t)2 * MMA_TOK * QT * 4 * MB_DW * 4;
  const int tiles = (N + QMM_ROWS - 1) / QMM_ROWS;
  const int tblocks = (M + MMA_TOK * QT - 1) / (MMA_TOK * QT);
  const int grid = (tiles + 7) / 8 * 8 * tblocks;
  hipLaunchKernelGGL((k_qmm<L, IT, QT>), dim3(grid), dim3(QMM_THREADS), lds, st, wq, sb, N, K, gs, xp, M, y, yf,
                     tiles, tblocks);
  return hipGetLastError();
}

template <int L, int IT>
static hipError_t qmm_lq(const uint32_t* wq, const uint32_t* sb, int N, int K, int gs, const uint32_t* xp, int M,
                         bf16* y, float* yf, hipStream_t st) {
  if (M <= 4 * MMA_TOK) return qmm_li<L, IT, 4>(wq, sb, N, K, gs, xp, M, y, yf, st);
  return qmm_li<L, IT, 8>(wq, sb, N, K, gs, xp, M, y, yf, st);
}

// The batch GEMM takes more than MAX_TOKENS tokens of a matrix with packed scale/bias rows whose
// K blocks tile at least four chains exactly.
static bool qmm_ok(const uint32_t* sb, int N, int K, int M) {
  const int nb = K / 32, L = lanes_for_blocks(nb);
  if (!sb || M <= MAX_TOKENS || N < QMM_MIN_ROWS || nb % L != 0) return false;
  switch (L * 16 + nb / L) {
    case 4 * 16 + 4: case 4 * 16 + 5: case 4 * 16 + 6: case 8 * 16 + 4: case 8 * 16 + 5: case 16 * 16 + 4:
    case 16 * 16 + 5: case 32 * 16 + 4: case 32 * 16 + 6: case 64 * 16 + 4: case 64 * 16 + 5: return true;
    default: return false;
  }
}

static hipError_t qmm(const uint32_t* wq, const uint32_t* sb, int N, int K, int gs, const uint32_t* xp, int M,
                      bf16* y, float* yf, hipStream_t st) {
  const int nb = K / 32, L = lanes_for_blocks(nb), IT = nb / L;
  switch (L * 16 + IT) {
    case 4 * 16 + 4: return qmm_lq<4, 4>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 4 * 16 + 5: return qmm_lq<4, 5>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 4 * 16 + 6: return qmm_lq<4, 6>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 8 * 16 + 4: return qmm_lq<8, 4>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 8 * 16 + 5: return qmm_lq<8, 5>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 16 * 16 + 4: return qmm_lq<16, 4>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 16 * 16 + 5: return qmm_lq<16, 5>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 32 * 16 + 4: return qmm_lq<32, 4>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 32 * 16 + 6: return qmm_lq<32, 6>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 64 * 16 + 4: return qmm_lq<64, 4>(wq, sb, N, K, gs, xp, M, y, yf, st);
    case 64 * 16 + 5: return qmm_lq<64, 5>(wq, sb, N, K, gs, xp, M, y, yf, st);
    default: return hipErrorNotSupported;
  }
}

// The MoE down GEMM over the chunk table: grid = max chunks x 128-row tiles of H (chunks past
// *a.chunk_n exit at once), activations = the gate|up output rows prepared into a.xp_act.
template <int L, int IT>
static hipError_t moe_qmm_li(const MoeArgs& a, hipStream_t st) {
  constexpr size_t lds = (size_t)(L > 4 ? 2 : 1) * MQ_CHUNK * 4 * IT * MB_DW * 4;
  static size_t cur = 0;
  const hipError_t le = ensure_lds(k_moe_qmm<L, IT>, lds, cur);
  if (le != hipSuccess) return le;
  const int tiles = (a.H + 127) / 128;
  hipLaunchKernelGGL((k_moe_qmm<L, IT>), dim3(a.max_chunks * tiles), dim3(QMM_THREADS), lds, st, a, tiles);
  return hipGetLastError();
}

static bool moe_qmm_shape(int K) {  // the model's expert width (F = 640: four chains of five blocks)
  const int nb = K / 32, L = lanes_for_blocks(nb);
  return nb % L == 0 && L * 16 + nb / L == 4 * 16 + 5;
}

bool moe_qmm_supported(const MoeArgs& a) { return a.down_sb && a.sh_down_sb && moe_qmm_shape(a.F); }

hipError_t launch_moe_qmm_down(const MoeArgs& a, hipStream_t st) {
  if (!moe_qmm_supported(a) || !a.chunks || !a.chunk_n || !a.xp_act) return hipErrorInvalidValue;
  return moe_qmm_li<4, 5>(a, st);
}

// Two few-row matrices over one batch of prepared activations (the mixer's down and inject
// projections): k_xmb into xmb [M][K/32][MB_DW], then k_qmn.  hipErrorNotSupported: a shape or
// matrix it does not take (the caller runs launch_qmv per matrix).
template <int L, int IT>
static hipError_t qmn_li(const uint32_t* w1, const uint32_t* sb1, int N1, bf16* y1, const uint32_t* w2,
                         const uint32_t* sb2, int N2, bf16* y2, int K, int gs, const uint32_t* xmb, int M,
                         hipStream_t st) {
  constexpr int QT = 4;  // 16 tokens per workgroup (two token groups measured slower at 512-position batches)
  const int tiles1 = (N1 + 15) / 16, tiles = tiles1 + (w2 ? (N2 + 15) / 16 : 0);
  const int tblocks = (M + MMA_TOK * QT - 1) / (MMA_TOK * QT);
  hipLaunchKernelGGL((k_qmn<L, IT, QT>), dim3(tiles * ((tblocks + 7) / 8 * 8)), dim3(QMN_THREADS), 0, st, w1, sb1, N1, y1, w2, sb2, N2,
                     y2, K, gs, xmb, M, tiles1, tiles);
  return hipGetLastError();
}

bool qmv_pair_ok(const uint32_t* sb1, const uint32_t* w2, const uint32_t* sb2, int K, int M) {
  const int nb = K / 32, L = lanes_for_blocks(nb), IT = nb % L == 0 ? nb / L : 0;
  return sb1 && (!w2 || sb2) && M > MAX_TOKENS &&
         (L * 16 + IT == 64 * 16 + 5 || L * 16 + IT == 64 * 16 + 4 || L * 16 + IT == 32 * 16 + 6);
}

hipError_t launch_qmv_pair(const uint32_t* w1, const uint32_t* sb1, int N1, bf16* y1, const uint32_t* w2,
                           const uint32_t* sb2, int N2, bf16* y2, int K, int gs, const uint32_t* xp, uint32_t* xmb,
                           int M, hipStream_t st) {
  if (!qmv_pair_ok(sb1, w2, sb2, K, M)) return hipErrorNotSupported;
  const int nb = K / 32, L = lanes_for_blocks(nb), IT = nb / L;
  const int units = M * nb * 8;
  hipLaunchKernelGGL(k_xmb, dim3((units + 255) / 256), dim3(256), 0, st, xp, units, xmb);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  switch (L * 16 + IT) {
    case 64 * 16 + 5: return qmn_li<64, 5>(w1, sb1, N1, y1, w2, sb2, N2, y2, K, gs, xmb, M, st);
    case 64 * 16 + 4: return qmn_li<64, 4>(w1, sb1, N1, y1, w2, sb2, N2, y2, K, gs, xmb, M, st);
    default: return qmn_li<32, 6>(w1, sb1, N1, y1, w2, sb2, N2, y2, K, gs, xmb, M, st);
  }
}

// Every token's output is the same whatever the launch shape (exact block sums, the lane rule's
// float order), so the token count only picks the path: the batch GEMM above MAX_TOKENS tokens where
// the shape allows, the matrix cores for two or more tokens
// where the shape allows (eight tokens per window when more than four, windows batched in one
// launch), else the dot-product kernel with as many tokens per window as one workgroup's LDS holds.
hipError_t launch_qmv(const uint32_t* wq, const bf16* s, const bf16* b, const uint32_t* sb, int N, int K, int gs,
                      const uint32_t* xp, int M, bf16* y, float* yf, hipStream_t st) {
  if (qmm_ok(sb, N, K, M)) return qmm(wq, sb, N, K, gs, xp, M, y, yf, st);
  // two tokens over many rows: the dot-product path (one window), measured faster than the matrix cores
  // there (GDN in-projection 18.3 -> 15.7 us, lm_head 99.9 -> 87.4 us); from three tokens on, the matrix cores
  const bool two_dot = M == 2 && N >= 8192;
  if (M >= 2 && !two_dot && qmv_mma_ok(sb, K, 2) && qmv_mma_shape<1>(K)) {  // matrix cores
    if (M > MMA_TOK && M <= MAX_TOKENS && qmv_mma_shape<2>(K)) {  // five to eight tokens: one window of eight
      const hipError_t e = qmv_mma<2>(wq, sb, N, K, gs, xp, M, y, yf, st);
      if (e != hipErrorNotReady) return e;
    }
    // else windows of four (a prefill batch too: a quarter of the LDS, three workgroups per CU, measured
    // faster than windows of eight at one per CU); a last window of one token takes the dot-product kernel
    const int full = M % MMA_TOK == 1 ? M - 1 : M;
    if (full > 0) {
      const hipError_t e = qmv_mma<1>(wq, sb, N, K, gs, xp, full, y, yf, st);
      if (e != hipSuccess) return e;
    }
    if (full == M) return hipSuccess;
    return qmv_tokens(wq, s, b, sb, N, K, gs, xp + (size_t)full * (K / 32) * XP_DW, 1, y + (size_t)full * N,
                      yf ? yf + (size_t)full * N : nullptr, 1, st);
  }
  // tokens per window: up to MAX_TOKENS as many prepared activation vectors as fit in one
  // workgroup's LDS; a longer batch: windows sized by the row count (qmv_li)
  const size_t per_token = (size_t)(K / 32) * XP_DW * 4;
  int win = (int)((160 * 1024) / per_token);
  win = win < 1 ? 1 : win;
  // three or more tokens whose rows alone leave CUs idle (fewer row workgroups than CUs): two windows,
  // twice the workgroups with half the tokens each (the K = 6144 output projections at 4 tokens: 13.0 ->
  // 12.6 us)
  const int rows_pass = 8 * (64 / lanes_for_blocks(K / 32));
  if (M >= 3 && M <= MAX_TOKENS && (N + rows_pass - 1) / rows_pass < device_cus()) win = std::min(win, (M + 1) / 2);
  return qmv_tokens(wq, s, b, sb, N, K, gs, xp, M, y, yf, M > MAX_TOKENS ? 0 : win, st);
}

hipError_t launch_quantize(const bf16* w, int64_t rows, int K, int gs, uint32_t* wq, bf16* s, bf16* b,
                           hipStream_t st) {
  const int64_t groups = rows * (K / gs);
  if (groups == 0) return hipSuccess;
  hipLaunchKernelGGL(k_quantize, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, w, groups, gs, wq,
                     s, b);
  return hipGetLastError();
}

hipError_t launch_randn_bf16(bf16* out, int64_t n, uint64_t seed, uint32_t tensor, float sigma,
                             hipStream_t st) {
  const int64_t q = (n + 3) / 4;
  if (q == 0) return hipSuccess;
  hipLaunchKernelGGL(k_randn_bf16, dim3((unsigned)((q + 255) / 256)), dim3(256), 0, st, out, n, seed, tensor,
                     sigma);
  return hipGetLastError();
}

hipError_t launch_fill_bf16(bf16* out, int64_t n, bf16 v, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, v);
  return hipGetLastError();
}

}  // namespace mtpx
