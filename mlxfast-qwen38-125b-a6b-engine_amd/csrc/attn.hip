// Verify attention over a contiguous bf16 KV cache, plus the row norms and
// residual adds around the decoder sublayers.
//   prep    : per (head, token): q/k RMSNorm over D, rotate-half RoPE on the
//             first ROT dims (bf16 arithmetic), k and v written straight into
//             the cache at position pos0 + token (the KV append)
//   partial : per (key chunk, kv head): scores of every query row of the GQA
//             group against the chunk, chunk max, exp, sum and P.V partial
//   combine : per (query row, kv head): fold the chunk partials in chunk order,
//             bf16 output and the sigmoid output gate
// Rollback of rejected draft positions is an offset rewind: positions past the
// offset are overwritten by the next append.
// Reference: FM/TrackFastKernels2.swift:381-510 (prep, gate),
// MLX/backend/metal/kernels/sdpa_vector.h:14-175 (online softmax, causal rule).
#include "mtpx_kernels.h"

namespace mtpx {

constexpr int ATTN_THREADS = 512;    // partial-kernel workgroup
constexpr int COMBINE_BATCH = 48;    // chunk partials per load round in the combine
constexpr int COMBINE_MAXCH = 2048;  // chunks (T <= 2048 * ATTN_CHUNK = 65536)

__global__ void k_attn_prep(const bf16* __restrict__ qkv, int S, int QW, int HQ, int HK, int D, int ROT,
                            const bf16* __restrict__ qnorm, const bf16* __restrict__ knorm, float eps,
                            const bf16* __restrict__ cos_t, const bf16* __restrict__ sin_t, int pos0,
                            bf16* __restrict__ q, bf16* __restrict__ kc, bf16* __restrict__ vc, int64_t tmax) {
  __shared__ float vec[1024];
  const int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
  const int L = D / 4;
  const bf16* row = qkv + (size_t)s * QW;
  const int pos = pos0 + s;
  if (h >= HQ + HK) {  // v: passthrough into the cache
    const int hv = h - HQ - HK;
    const bf16* src = row + 2 * HQ * D + HK * D + hv * D;
    bf16* dst = vc + ((size_t)hv * tmax + pos) * D;
    for (int i = 0; i < 4; ++i) dst[4 * t + i] = src[4 * t + i];
    return;
  }
  const bool isq = h < HQ;
  const int hh = isq ? h : h - HQ;
  const bf16* src = isq ? row + hh * D : row + 2 * HQ * D + hh * D;
  const bf16* wn = isq ? qnorm : knorm;
  // every load first (raw bits; the rotary table at clamped positions, used below ROT only), so
  // nothing waits before the last one is issued
  const bf16* cs = ROT > 0 ? cos_t + (size_t)pos * ROT : src;  // (no rotary: a valid row, unused)
  const bf16* sn = ROT > 0 ? sin_t + (size_t)pos * ROT : src;
  bf16 xr[4], wr[4], cr[4], sr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 4 * t + i, dr = d < ROT ? d : 0;
    xr[i] = src[d];
    wr[i] = wn[d];
    cr[i] = cs[dr];
    sr[i] = sn[dr];
  }
  asm volatile("" ::: "memory");
  float x[4];
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = bf2f(xr[i]);
    acc = __builtin_fmaf(x[i], x[i], acc);
  }
  if (L == 64)  // one wave: the same butterfly by DPP and lane swaps instead of LDS permutes
    acc = wave_fold64(acc);
  else
    for (int off = L / 2; off >= 1; off >>= 1) acc = acc + __shfl_xor(acc, off, 64);
  const float inv = 1.0f / sqrtf(acc / (float)D + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) vec[4 * t + i] = round_bf(bf2f(wr[i]) * round_bf(x[i] * inv));
  __syncthreads();
  bf16* dst = isq ? q + ((size_t)s * HQ + hh) * D : kc + ((size_t)hh * tmax + pos) * D;
  const int half = ROT / 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 4 * t + i;
    float o = vec[d];
    if (d < ROT) {
      const float c = bf2f(cr[i]), sv = bf2f(sr[i]);
      if (d < half) {
        const float t1 = round_bf(vec[d] * c);
        const float t2 = round_bf(-vec[d + half] * sv);
        o = round_bf(t1 + t2);
      } else {
        const float t1 = round_bf(vec[d] * c);
        const float t2 = round_bf(vec[d - half] * sv);
        o = round_bf(t1 + t2);
      }
    }
    dst[d] = f2bf(o);
  }
}

// The chunk's scores, softmax partials and P.V of workgroup (chunk c, kv head hk, query token s) against
// the staged rows (qb: the token's G query rows, bf16 pairs [G][D/2]; kb: the chunk's n visible keys,
// rows of KS dwords; vb: their values [C][D]), written to part.
__device__ __forceinline__ void attn_chunk(int c, int hk, int s, int G, int R, int n, int D, float scale, int nch,
                                           const uint32_t* qb, const uint32_t* kb, const bf16* vb, float* sc,
                                           float* ml, float* __restrict__ part) {
  const int C = ATTN_CHUNK, KS = D / 2 + 4;
  // scores: one (query row g, key j) chain per thread and pass: the sequential
  // d-order fmaf of the canonical order, fed 8 dimensions per 128-bit LDS read
  for (int p = threadIdx.x; p < G * C; p += blockDim.x) {
    const bool on = (p % C) < n;
    const uint32_t* qr = qb + (size_t)(p / C) * (D / 2);
    const uint32_t* kr = kb + (size_t)(on ? p % C : 0) * KS;
    float acc = 0.0f;
#pragma unroll 4
    for (int d0 = 0; d0 < D / 2; d0 += 4) {  // (D / 8 steps, a multiple of 4: the reads of four steps in flight)
      const uint4 q4v = *reinterpret_cast<const uint4*>(qr + d0), k4v = *reinterpret_cast<const uint4*>(kr + d0);
      const uint32_t qa[4] = {q4v.x, q4v.y, q4v.z, q4v.w}, ka[4] = {k4v.x, k4v.y, k4v.z, k4v.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc = __builtin_fmaf(scale * __uint_as_float(qa[t] << 16), __uint_as_float(ka[t] << 16), acc);
        acc = __builtin_fmaf(scale * __uint_as_float(qa[t] & 0xffff0000u), __uint_as_float(ka[t] & 0xffff0000u), acc);
      }
    }
    sc[p] = on ? acc : 0.0f;
  }
  __syncthreads();
  // chunk max per query row (order-free), every exp in parallel, then the row
  // sums in key order
  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    float mx = -__uint_as_float(0x7f800000u);
#pragma unroll 8
    for (int j = 0; j < n; ++j) mx = sc[g * C + j] > mx ? sc[g * C + j] : mx;
    ml[2 * g] = (n > 0) ? mx : -__uint_as_float(0x7f800000u);
  }
  __syncthreads();
  for (int p = threadIdx.x; p < G * C; p += blockDim.x) {
    const int g = p / C, j = p % C;
    if (j < n) sc[p] = expf_det(sc[p] - ml[2 * g]);
  }
  __syncthreads();
  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    float l = 0.0f;
#pragma unroll 8
    for (int j = 0; j < n; ++j) l = l + sc[g * C + j];
    ml[2 * g + 1] = (n > 0) ? l : 0.0f;
  }
  __syncthreads();
  // P.V: a thread owns the adjacent outputs (g, 2e) and (g, 2e+1), one 32-bit V
  // read per key for both; each output is the sequential key-order fmaf
  // (blockDim is a multiple of D / 2, so outputs p, p + blockDim, ... share e: up to PVN of them side by side,
  // one V read per key for all, 2 * PVN independent chains)
  const uint32_t* vb32 = reinterpret_cast<const uint32_t*>(vb);
  constexpr int PVN = 4;
  for (int pb = threadIdx.x; pb < G * (D / 2); pb += PVN * (int)blockDim.x) {
    const int e = pb % (D / 2);
    int gk[PVN];
    float o0[PVN], o1[PVN];
#pragma unroll
    for (int k = 0; k < PVN; ++k) {
      const int p = pb + k * (int)blockDim.x;
      gk[k] = p < G * (D / 2) ? p / (D / 2) : -1;
      o0[k] = 0.0f;
      o1[k] = 0.0f;
    }
    int j = 0;
    for (; j + 8 <= n; j += 8) {
      uint32_t vv[8];
      float pv[PVN][8];
#pragma unroll
      for (int u = 0; u < 8; ++u) vv[u] = vb32[(size_t)(j + u) * (D / 2) + e];
#pragma unroll
      for (int k = 0; k < PVN; ++k)
#pragma unroll
        for (int u = 0; u < 8; ++u) pv[k][u] = sc[(size_t)(gk[k] < 0 ? 0 : gk[k]) * C + j + u];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int k = 0; k < PVN; ++k) {
          o0[k] = __builtin_fmaf(pv[k][u], __uint_as_float(vv[u] << 16), o0[k]);
          o1[k] = __builtin_fmaf(pv[k][u], __uint_as_float(vv[u] & 0xffff0000u), o1[k]);
        }
    }
    for (; j < n; ++j) {
      const uint32_t v = vb32[(size_t)j * (D / 2) + e];
#pragma unroll
      for (int k = 0; k < PVN; ++k) {
        const float w = sc[(size_t)(gk[k] < 0 ? 0 : gk[k]) * C + j];
        o0[k] = __builtin_fmaf(w, __uint_as_float(v << 16), o0[k]);
        o1[k] = __builtin_fmaf(w, __uint_as_float(v & 0xffff0000u), o1[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < PVN; ++k) {
      const int g = gk[k];
      if (g < 0) continue;
      float* dst = part + (((size_t)hk * nch + c) * R + s * G + g) * (D + 2);
      dst[2 + 2 * e] = o0[k];
      dst[3 + 2 * e] = o1[k];
      if (e == 0) {
        dst[0] = ml[2 * g];
        dst[1] = ml[2 * g + 1];
      }
    }
  }
}

// part layout: [(hk * nch + c) * R + ri] * (D + 2): {m, l, o[0..D)}, R = S * G,
// ri = s * G + g.  grid (nch, HK, S): one workgroup per (key chunk, kv head,
// query); its rows are the G query heads of the group.
__global__ __launch_bounds__(ATTN_THREADS) void k_attn_partial(const bf16* __restrict__ q, int S, int HQ, int HK, int D,
                                                      const bf16* __restrict__ kc, const bf16* __restrict__ vc,
                                                      int64_t tmax, int T, float scale, int nch,
                                                      float* __restrict__ part) {
  extern __shared__ float smem[];
  const int c = blockIdx.x, hk = blockIdx.y, s = blockIdx.z;
  const int G = HQ / HK, R = S * G, C = ATTN_CHUNK;
  const int i0 = c * C;
  const int last = T - S + s;                // last key visible to this query
  int n = last + 1 - i0;                     // visible keys of the chunk (a prefix)
  n = n < 0 ? 0 : (n > C ? C : n);
  // K rows padded by 4 dwords: 16-byte aligned rows for 128-bit reads, and 8
  // consecutive keys cover all 32 banks
  const int KS = D / 2 + 4;
  uint32_t* qb = reinterpret_cast<uint32_t*>(smem);         // [G][D/2] bf16 pairs
  uint32_t* kb = qb + (size_t)G * (D / 2);                  // [C][KS]
  bf16* vb = reinterpret_cast<bf16*>(kb + (size_t)C * KS);  // [C][D]
  float* sc = reinterpret_cast<float*>(vb + (size_t)C * D); // [G][C]
  float* ml = sc + (size_t)G * C;                           // [G][2]
  const uint32_t* q32 = reinterpret_cast<const uint32_t*>(q);
  const uint32_t* k32 = reinterpret_cast<const uint32_t*>(kc);
  const uint32_t* v32 = reinterpret_cast<const uint32_t*>(vc);
  // staging: 16-byte loads, up to 8 in flight per thread before the LDS stores
  const uint4* q4 = reinterpret_cast<const uint4*>(q);
  const uint4* k4 = reinterpret_cast<const uint4*>(kc);
  const uint4* v4 = reinterpret_cast<const uint4*>(vc);
  const int RV = D / 8;                   // uint4 per row
  const int nq = G * RV, nkv = n * RV;    // uint4 of q rows, of each of K and V
  for (int base = 0; base < nq + 2 * nkv; base += 8 * (int)blockDim.x) {
    uint4 r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // the source selected by address, one unconditional load (the first q
      const int i = base + u * (int)blockDim.x + (int)threadIdx.x;  // unit past the end): all 8 in flight
      const int ik = i - nq, iv = i - nq - nkv;
      const uint4* src = i < nq ? q4 + ((size_t)s * HQ + hk * G) * RV + i
                         : i < nq + nkv ? k4 + ((size_t)hk * tmax + i0 + ik / RV) * RV + ik % RV
                         : i < nq + 2 * nkv ? v4 + ((size_t)hk * tmax + i0 + iv / RV) * RV + iv % RV
                                            : q4 + ((size_t)s * HQ + hk * G) * RV;
      r[u] = *src;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * (int)blockDim.x + (int)threadIdx.x;
      if (i < nq) {
        reinterpret_cast<uint4*>(qb)[i] = r[u];
      } else if (i < nq + nkv) {
        const int ik = i - nq;
        uint32_t* dst = kb + (size_t)(ik / RV) * KS + (ik % RV) * 4;
        dst[0] = r[u].x;
        dst[1] = r[u].y;
        dst[2] = r[u].z;
        dst[3] = r[u].w;
      } else if (i < nq + 2 * nkv) {
        const int iv = i - nq - nkv;
        reinterpret_cast<uint4*>(vb)[iv] = r[u];
      }
    }
  }
  __syncthreads();
  attn_chunk(c, hk, s, G, R, n, D, scale, nch, qb, kb, vb, sc, ml, part);
}

// The verify window's attention with the prep folded in (S <= MAX_TOKENS, D = 256: a head row per wave,
// four elements a lane, the prep kernel's float steps and butterfly): workgroup (chunk c, kv head hk,
// query token s) normalises and rotates its token's G query rows into LDS itself, stages the chunk's
// visible cached keys and values below the window (positions < T - S), and prepares the window's key
// rows that fall in the chunk (normalised and rotated) and value rows (copied) into LDS; the last
// query's workgroup also appends those rows to the cache.  Every load is issued before the first wait.
constexpr int PP_D = 256;
constexpr int PP_PASSES = 3;  // normed rows per wave: G + (window rows in the chunk) <= 8 waves x 3

// NPS: the norm passes of the launch (G + S <= 8 NPS), so its loads issued up front are all used
template <int NPS>
__global__ __launch_bounds__(ATTN_THREADS) void k_attn_partial_prep(
    const bf16* __restrict__ qkv, int QW, int S, int HQ, int HK, int ROT, const bf16* __restrict__ qnorm,
    const bf16* __restrict__ knorm, float eps, const bf16* __restrict__ cos_t, const bf16* __restrict__ sin_t,
    bf16* __restrict__ kc, bf16* __restrict__ vc, int64_t tmax, int T, float scale, int nch, float* __restrict__ part) {
  constexpr int D = PP_D, RV = D / 8, NW = ATTN_THREADS / 64;
  extern __shared__ float smem[];
  const int c = blockIdx.x, hk = blockIdx.y, s = blockIdx.z;
  const int G = HQ / HK, R = S * G, C = ATTN_CHUNK;
  const int i0 = c * C, pos0 = T - S;
  int n = pos0 + s + 1 - i0;  // visible keys of the chunk (a prefix)
  n = n < 0 ? 0 : (n > C ? C : n);
  const int KS = D / 2 + 4;
  uint32_t* qb = reinterpret_cast<uint32_t*>(smem);          // [G][D/2] bf16 pairs
  uint32_t* kb = qb + (size_t)G * (D / 2);                   // [C][KS]
  bf16* vb = reinterpret_cast<bf16*>(kb + (size_t)C * KS);   // [C][D]
  float* sc = reinterpret_cast<float*>(vb + (size_t)C * D);  // [G][C]
  float* ml = sc + (size_t)G * C;                            // [G][2]
  float* xw = ml + (size_t)2 * G;                            // [NW][D]: a wave's normed row before the rotation
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // the window's rows in this chunk (positions [w0, w1)), and the cached rows staged (below the window)
  const int w0 = i0 > pos0 ? i0 : pos0, w1 = i0 + C < T ? i0 + C : T, nw = w1 > w0 ? w1 - w0 : 0;
  const int lo = pos0 - i0, ncache = lo < 0 ? 0 : (lo > n ? n : lo);
  const bool append = s == S - 1;
  // loads: the normed rows' inputs (item it = wave + NW pass: the G query rows, then the nw key rows;
  // each lane its four elements, the norm weights and the rotary table at a clamped column), the
  // window's value rows, the cached key and value rows
  const int items = G + nw;
  uint2 xin[NPS], win[NPS];
  bf16 cr[NPS][4], sr[NPS][4];
#pragma unroll
  for (int pass = 0; pass < NPS; ++pass) {
    const int it = wave + NW * pass, itc = it < items ? it : 0;
    const bool isq = itc < G;
    const int tok = isq ? s : w0 + (itc - G) - pos0;  // the window token of the row
    const bf16* src = qkv + (size_t)tok * QW + (isq ? (size_t)(hk * G + itc) * D : (size_t)2 * HQ * D + (size_t)hk * D);
    xin[pass] = *reinterpret_cast<const uint2*>(src + 4 * lane);
    win[pass] = *reinterpret_cast<const uint2*>((isq ? qnorm : knorm) + 4 * lane);
    const size_t rp = (size_t)(pos0 + tok) * ROT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 4 * lane + i, dr = d < ROT ? d : 0;
      cr[pass][i] = cos_t[rp + dr];
      sr[pass][i] = sin_t[rp + dr];
    }
  }
  const uint4* k4 = reinterpret_cast<const uint4*>(kc);
  const uint4* v4 = reinterpret_cast<const uint4*>(vc);
  const uint4* qkv4 = reinterpret_cast<const uint4*>(qkv);
  const int nkv = ncache * RV, nwv = nw * RV;  // uint4 of the cached K and V rows each, of the window's V rows
  constexpr int SU = (2 * ATTN_CHUNK * RV + ATTN_THREADS - 1) / ATTN_THREADS;  // staging units per thread
  uint4 r[SU];
#pragma unroll
  for (int u = 0; u < SU; ++u) {  // unit i: cached K (i < nkv), cached V, then window V rows; clamped past the end
    const int i = u * ATTN_THREADS + (int)threadIdx.x;
    const int ik = i, iv = i - nkv, iw = i - 2 * nkv;
    const uint4* src = i < nkv ? k4 + ((size_t)hk * tmax + i0 + ik / RV) * RV + ik % RV
                       : i < 2 * nkv ? v4 + ((size_t)hk * tmax + i0 + iv / RV) * RV + iv % RV
                       : i < 2 * nkv + nwv
                           ? qkv4 + ((size_t)(w0 + iw / RV - pos0) * QW + (size_t)2 * HQ * D + (size_t)HK * D +
                                     (size_t)hk * D) / 8 + iw % RV
                           : qkv4 + ((size_t)s * QW) / 8;
    r[u] = *src;
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int u = 0; u < SU; ++u) {
    const int i = u * ATTN_THREADS + (int)threadIdx.x;
    if (i < nkv) {
      uint32_t* dst = kb + (size_t)(i / RV) * KS + (i % RV) * 4;
      dst[0] = r[u].x;
      dst[1] = r[u].y;
      dst[2] = r[u].z;
      dst[3] = r[u].w;
    } else if (i < 2 * nkv) {
      reinterpret_cast<uint4*>(vb)[i - nkv] = r[u];
    } else if (i < 2 * nkv + nwv) {
      const int iw = i - 2 * nkv, row = w0 - i0 + iw / RV;
      reinterpret_cast<uint4*>(vb)[(size_t)row * RV + iw % RV] = r[u];
      if (append) reinterpret_cast<uint4*>(vc)[((size_t)hk * tmax + w0 + iw / RV) * RV + iw % RV] = r[u];
    }
  }
  // the normed, rotated rows: q into qb, the window's k into kb (and the cache)
  const int half = ROT / 2;
  float* xr = xw + (size_t)wave * D;
#pragma unroll
  for (int pass = 0; pass < NPS; ++pass) {
    const int it = wave + NW * pass;
    if (it >= items) break;  // uniform per wave
    const uint32_t xa[2] = {xin[pass].x, xin[pass].y}, wa[2] = {win[pass].x, win[pass].y};
    float x[4];
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = __uint_as_float((i & 1) ? (xa[i >> 1] & 0xffff0000u) : (xa[i >> 1] << 16));
      acc = __builtin_fmaf(x[i], x[i], acc);
    }
    acc = wave_fold64(acc);
    const float inv = 1.0f / sqrtf(acc / (float)D + eps);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float w = __uint_as_float((i & 1) ? (wa[i >> 1] & 0xffff0000u) : (wa[i >> 1] << 16));
      v[i] = round_bf(w * round_bf(x[i] * inv));
      xr[4 * lane + i] = v[i];
    }
    // this wave reads the row it wrote (LDS operations of one wave complete in order)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool isq = it < G;
    bf16 o16[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 4 * lane + i;
      float o = v[i];
      if (d < ROT) {
        const float cv = bf2f(cr[pass][i]), sv = bf2f(sr[pass][i]);
        if (d < half) {
          const float t1 = round_bf(v[i] * cv);
          const float t2 = round_bf(-xr[d + half] * sv);
          o = round_bf(t1 + t2);
        } else {
          const float t1 = round_bf(v[i] * cv);
          const float t2 = round_bf(xr[d - half] * sv);
          o = round_bf(t1 + t2);
        }
      }
      o16[i] = f2bf(o);
    }
    const uint2 packed = make_uint2((uint32_t)o16[0] | ((uint32_t)o16[1] << 16), (uint32_t)o16[2] | ((uint32_t)o16[3] << 16));
    if (isq) {
      reinterpret_cast<uint2*>(qb + (size_t)it * (D / 2))[lane] = packed;
    } else {
      const int p = w0 + (it - G);
      reinterpret_cast<uint2*>(kb + (size_t)(p - i0) * KS)[lane] = packed;
      if (append) reinterpret_cast<uint2*>(kc + ((size_t)hk * tmax + p) * D)[lane] = packed;
    }
    // the next pass rewrites this wave's row: its reads above complete first (in order)
  }
  __syncthreads();
  attn_chunk(c, hk, s, G, R, n, D, scale, nch, qb, kb, vb, sc, ml, part);
}

// grid (R, HK), max(D, 64) threads (D <= 256).  Fold the chunk partials in chunk order,
// then bf16 output, the sigmoid gate, and (optionally) the prepared activation
// blocks of the gated row for the o_proj GEMV (32 lanes per block).
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ part, int S, int HQ, int HK, int D,
                                                      int nch, const bf16* __restrict__ qkv, int QW, int gate_off,
                                                      bf16* __restrict__ out, bf16* __restrict__ out_gated,
                                                      uint32_t* __restrict__ xp_gated) {
  __shared__ float mc[COMBINE_MAXCH], fc[COMBINE_MAXCH], lc[COMBINE_MAXCH], red[4];
  const int ri = blockIdx.x, hk = blockIdx.y;
  const int G = HQ / HK, R = S * G;
  const int s = ri / G, h = hk * G + ri % G;
  const int t = threadIdx.x, nt = blockDim.x;
  const int d = t;  // blockDim >= D
  auto chunk = [&](int c) { return part + (((size_t)hk * nch + c) * R + ri) * (D + 2); };
  // one round of loads: every chunk's (m, l) into LDS, and this thread's first
  // COMBINE_BATCH output partials into registers
  // unconditional loads (clamped chunk and dimension; the values past the end are not used), so
  // all of them are in flight at once; the gate value too, which is needed only at the end
  const int dc = d < D ? d : D - 1;
  const bf16 gate_raw = out_gated ? qkv[(size_t)s * QW + gate_off + h * D + dc] : (bf16)0;
  float pv[COMBINE_BATCH];
#pragma unroll
  for (int u = 0; u < COMBINE_BATCH; ++u) pv[u] = chunk(u < nch ? u : nch - 1)[2 + dc];
  for (int c = t; c < nch; c += nt) {
    const float* p = chunk(c);
    mc[c] = p[0];
    lc[c] = p[1];
  }
  __syncthreads();
  // M: max of the visible chunks' maxima (order-free)
  float M = -__uint_as_float(0x7f800000u);
  for (int c = t; c < nch; c += nt)
    if (lc[c] > 0.0f && mc[c] > M) M = mc[c];
  {
    float o;
    o = lane_xor_f<32>(M); M = o > M ? o : M;
    o = lane_xor_f<16>(M); M = o > M ? o : M;
    o = lane_xor_f<8>(M); M = o > M ? o : M;
    o = lane_xor_f<4>(M); M = o > M ? o : M;
    o = lane_xor_f<2>(M); M = o > M ? o : M;
    o = lane_xor_f<1>(M); M = o > M ? o : M;
  }
  if ((t & 63) == 0) red[t >> 6] = M;
  __syncthreads();
  for (int wv = 0; wv < nt / 64; ++wv) M = red[wv] > M ? red[wv] : M;
  // the factor of every chunk once, then L and O[d] in chunk order
  for (int c = t; c < nch; c += nt) fc[c] = lc[c] > 0.0f ? expf_det(mc[c] - M) : 0.0f;
  __syncthreads();
  // L and O, each in chunk order, as two chains of one loop; a batch's (l, f) pairs are read from LDS
  // before its folds (clamped indices), so the reads are in flight together
  float L = 0.0f, O = 0.0f;
  for (int cb = 0; cb < nch; cb += COMBINE_BATCH) {
    if (cb > 0) {
#pragma unroll
      for (int u = 0; u < COMBINE_BATCH; ++u) pv[u] = chunk(cb + u < nch ? cb + u : nch - 1)[2 + dc];
    }
    float lb[COMBINE_BATCH], fb[COMBINE_BATCH];
#pragma unroll
    for (int u = 0; u < COMBINE_BATCH; ++u) {
      const int c = cb + u < nch ? cb + u : nch - 1;
      lb[u] = lc[c];
      fb[u] = fc[c];
    }
#pragma unroll
    for (int u = 0; u < COMBINE_BATCH; ++u)
      if (cb + u < nch && lb[u] > 0.0f) {
        L = __builtin_fmaf(lb[u], fb[u], L);
        O = __builtin_fmaf(pv[u], fb[u], O);
      }
  }
  {
    const int d0 = 0;
    bf16 gated = 0;
    if (d < D) {
      const bf16 att = f2bf(O / L);
      if (out) out[((size_t)s * HQ + h) * D + d] = att;
      if (out_gated) {
        const float g = bf2f(gate_raw);
        gated = f2bf(bf2f(att) * sigmoid_bf16(g));
        out_gated[(size_t)s * HQ * D + h * D + d] = gated;
      }
    }
    if (xp_gated && d < D) {
      // block (h*D + d) / 32 of row s; D % 32 == 0 so blocks never straddle heads
      const size_t blk = (size_t)s * (HQ * D / 32) + (h * D + d0) / 32 + (threadIdx.x >> 5);
      xprep_lanes_direct(gated, threadIdx.x & 31, xp_gated + blk * XP_DW);
    }
  }
}

// Row RMSNorm, 256 threads per row: h = x or bf16(x + resid); y = bf16(w * bf16(h * inv)).
// With xp != nullptr also writes the prepared activation blocks of y (32 lanes per block).
// grid (M, ceil(H/256)): every workgroup folds the whole row's sum of squares
// (thread t: elements t, t+256, ... in order; waves summed ((w0+w1)+w2)+w3) and
// writes the 256 outputs of its slice, plus their prepared activation blocks.
constexpr int RMS_IT = 16;  // H <= 16 * 256

__global__ __launch_bounds__(256) void k_rmsnorm(const bf16* __restrict__ x, const bf16* __restrict__ resid,
                                                 int H, const bf16* __restrict__ w, float eps,
                                                 bf16* __restrict__ sum_out, bf16* __restrict__ y,
                                                 uint32_t* __restrict__ xp) {
  __shared__ float wsum[4];
  const int m = blockIdx.x, t = threadIdx.x, sl = blockIdx.y;
  const bf16* xr = x + (size_t)m * H;
  const bf16* rr = resid ? resid + (size_t)m * H : nullptr;
  float v[RMS_IT];
#pragma unroll
  for (int j = 0; j < RMS_IT; ++j) {
    const int i = t + 256 * j;
    v[j] = (i < H) ? bf2f(xr[i]) : 0.0f;
  }
  if (rr) {
#pragma unroll
    for (int j = 0; j < RMS_IT; ++j) {
      const int i = t + 256 * j;
      if (i < H) v[j] = round_bf(v[j] + bf2f(rr[i]));
    }
  }
  float acc = 0.0f, vo = 0.0f;
#pragma unroll
  for (int j = 0; j < RMS_IT; ++j) {
    if (t + 256 * j < H) acc = __builtin_fmaf(v[j], v[j], acc);
    if (j == sl) vo = v[j];
  }
  acc = wave_fold64(acc);
  if ((t & 63) == 0) wsum[t >> 6] = acc;
  __syncthreads();
  const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  const float inv = 1.0f / sqrtf(total / (float)H + eps);
  const int i = sl * 256 + t;
  bf16 out = 0;
  if (i < H) {
    if (rr && sum_out) sum_out[(size_t)m * H + i] = f2bf(vo);
    out = f2bf(bf2f(w[i]) * round_bf(vo * inv));
    y[(size_t)m * H + i] = out;
  }
  if (xp && i < H) xprep_lanes_direct(out, t & 31, xp + ((size_t)m * (H / 32) + i / 32) * XP_DW);
}

__global__ void k_add(const bf16* __restrict__ a, const bf16* __restrict__ b, int64_t n, bf16* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f2bf(bf2f(a[i]) + bf2f(b[i]));
}

// ---------------------------------------------------------------------------
size_t attn_partial_floats(int S, int HQ, int D, int T) {
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;  // chunks of ATTN_CHUNK keys
  return (size_t)nch * S * HQ * (D + 2);
}

hipError_t launch_attn_prep(const bf16* qkv, int S, int QW, int HQ, int HK, int D, int ROT, const bf16* qnorm,
                            const bf16* knorm, float eps, const bf16* cos_t, const bf16* sin_t, int pos0, bf16* q,
                            bf16* kcache, bf16* vcache, int64_t tmax, hipStream_t st) {
  hipLaunchKernelGGL(k_attn_prep, dim3(HQ + 2 * HK, S), dim3(D / 4), 0, st, qkv, S, QW, HQ, HK, D, ROT, qnorm, knorm,
                     eps, cos_t, sin_t, pos0, q, kcache, vcache, tmax);
  return hipGetLastError();
}

hipError_t launch_attn_partial(const bf16* q, int S, int HQ, int HK, int D, const bf16* kc, const bf16* vc,
                               int64_t tmax, int T, float scale, float* part, hipStream_t st) {
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const size_t lds = attn_partial_lds(HQ / HK, D);
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_attn_partial, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_attn_partial, dim3(nch, HK, S), dim3(ATTN_THREADS), lds, st, q, S, HQ, HK, D, kc, vc, tmax, T,
                     scale, nch, part);
  return hipGetLastError();
}

bool attn_prep_fused_ok(int S, int HQ, int HK, int D, int QW) {
  return S >= 1 && S <= MAX_TOKENS && D == PP_D && HQ % HK == 0 && QW % 8 == 0 &&
         attn_partial_lds(HQ / HK, D) + (size_t)(ATTN_THREADS / 64) * D * 4 <= 160 * 1024 &&
         HQ / HK + MAX_TOKENS <= (ATTN_THREADS / 64) * PP_PASSES;
}

hipError_t launch_attn_partial_prep(const bf16* qkv, int QW, int S, int HQ, int HK, int D, int ROT, const bf16* qnorm,
                                    const bf16* knorm, float eps, const bf16* cos_t, const bf16* sin_t, bf16* kcache,
                                    bf16* vcache, int64_t tmax, int T, float scale, float* part, hipStream_t st) {
  if (!attn_prep_fused_ok(S, HQ, HK, D, QW) || T < S) return hipErrorInvalidValue;
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const size_t lds = attn_partial_lds(HQ / HK, D) + (size_t)(ATTN_THREADS / 64) * D * 4;
  // a chunk holds at most S window rows: items <= G + S
  if (HQ / HK + S <= (ATTN_THREADS / 64) * 2) {
    static size_t cur2 = 0;
    hipError_t e = ensure_lds(k_attn_partial_prep<2>, lds, cur2);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_partial_prep<2>, dim3(nch, HK, S), dim3(ATTN_THREADS), lds, st, qkv, QW, S, HQ, HK, ROT,
                       qnorm, knorm, eps, cos_t, sin_t, kcache, vcache, tmax, T, scale, nch, part);
    return hipGetLastError();
  }
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_attn_partial_prep<PP_PASSES>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_attn_partial_prep<PP_PASSES>, dim3(nch, HK, S), dim3(ATTN_THREADS), lds, st, qkv, QW, S, HQ,
                     HK, ROT, qnorm, knorm, eps, cos_t, sin_t, kcache, vcache, tmax, T, scale, nch, part);
  return hipGetLastError();
}

hipError_t launch_attn_combine(int S, int HQ, int HK, int D, int T, const float* part, const bf16* qkv, int QW,
                               int gate_off, bf16* out, bf16* out_gated, uint32_t* xp_gated, hipStream_t st) {
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const int R = S * (HQ / HK);
  hipLaunchKernelGGL(k_attn_combine, dim3(R, HK), dim3(D < 64 ? 64 : D), 0, st, part, S, HQ, HK, D, nch, qkv, QW,
                     gate_off, out, out_gated, xp_gated);
  return hipGetLastError();
}

hipError_t launch_attn_verify(const bf16* q, int S, int HQ, int HK, int D, const bf16* kc, const bf16* vc,
                              int64_t tmax, int T, float scale, float* part, const bf16* qkv, int QW, int gate_off,
                              bf16* out, bf16* out_gated, uint32_t* xp_gated, hipStream_t st) {
  hipError_t e = launch_attn_partial(q, S, HQ, HK, D, kc, vc, tmax, T, scale, part, st);
  if (e != hipSuccess) return e;
  return launch_attn_combine(S, HQ, HK, D, T, part, qkv, QW, gate_off, out, out_gated, xp_gated, st);
}

size_t attn_partial_lds(int G, int D) {
  return (size_t)G * D * 2 + (size_t)ATTN_CHUNK * (D + 8) * 2 + (size_t)ATTN_CHUNK * D * 2 +
         (size_t)G * ATTN_CHUNK * 4 + (size_t)G * 8;
}

hipError_t launch_rmsnorm(const bf16* x, const bf16* resid, int M, int H, const bf16* w, float eps, bf16* sum_out,
                          bf16* y, uint32_t* xp, hipStream_t st) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(M, (H + 255) / 256), dim3(256), 0, st, x, resid, H, w, eps, sum_out, y, xp);
  return hipGetLastError();
}

hipError_t launch_add(const bf16* a, const bf16* b, int64_t n, bf16* out, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, b, n, out);
  return hipGetLastError();
}

}  // namespace mtpx
