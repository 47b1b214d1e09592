// mtpx device numerics for gfx950.
//
// Every routine here fixes an evaluation order; the kernels are compiled with
// -ffp-contract=off so no multiply-add is fused unless written as fmaf.  The
// affine-4-bit dot product is exact integer arithmetic: activations become
// 24-bit fixed point per 32-element block (three byte limbs), nibble x limb
// products are summed with v_dot4 integer instructions (exact and
// order-independent), and only the per-block float combine is ordered.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtpx {

typedef uint16_t bf16;

__device__ __forceinline__ float bf2f(bf16 h) { return __uint_as_float((uint32_t)h << 16); }

// Round to nearest even; NaN -> 0x7fc0.
__device__ __forceinline__ bf16 f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16)(u >> 16);
}

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// The value lane (lane ^ OFF) holds, exactly, from register-file cross-lane
// operations instead of an LDS permute: DPP quad permutes (OFF 1, 2), a row
// shift pair (OFF 4), a row rotate (OFF 8; a 16-lane row rotated by 8 is the
// xor), and the permlane row swaps (OFF 16, 32).  Every lane of the 2*OFF-lane
// group must be active.
__device__ __forceinline__ int lane_id() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

template <int OFF>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "a power of two <= 32");
  const int x = (int)v;
  if constexpr (OFF == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (OFF == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (OFF == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, false);  // row_shl:4 (lane + 4)
    const int dn = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4 (lane - 4)
    return (uint32_t)((lane_id() & 4) ? dn : up);
  } else if constexpr (OFF == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (OFF == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // {r0,r0,r2,r2}, {r1,r1,r3,r3}
    return (lane_id() & 16) ? p[0] : p[1];
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // {lo,lo}, {hi,hi}
    return (lane_id() & 32) ? p[0] : p[1];
  }
}
template <int OFF>
__device__ __forceinline__ float lane_xor_f(float v) { return __uint_as_float(lane_xor<OFF>(__float_as_uint(v))); }
template <int OFF>
__device__ __forceinline__ int lane_xor_i(int v) { return (int)lane_xor<OFF>((uint32_t)v); }

// v + v[lane ^ OFF] for OFF = TOP, TOP/2, ..., 1 (highest level first)
template <int TOP>
__device__ __forceinline__ float fold_sum(float v) {
  if constexpr (TOP >= 1) {
    v = v + lane_xor_f<TOP>(v);
    return fold_sum<TOP / 2>(v);
  } else {
    return v;
  }
}

// exp(x): Cody-Waite split with a two-part ln2, degree-7 Taylor polynomial on
// |r| <= ln2/2, 2^n applied in two exact steps; x < -87.3 -> 0, x > 88.7 -> inf.
__device__ __forceinline__ float expf_det(float x) {
  if (x != x) return x;
  if (x < -87.3f) return 0.0f;
  if (x > 88.7f) return __uint_as_float(0x7f800000u);
  const float n = __builtin_rintf(x * 1.44269504f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.428606765330187e-06f, r);
  float p = 1.98412698e-04f;
  p = __builtin_fmaf(p, r, 1.38888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2, n2 = ni - n1;
  p = p * __uint_as_float((uint32_t)(n1 + 127) << 23);
  p = p * __uint_as_float((uint32_t)(n2 + 127) << 23);
  return p;
}

// MLX Sigmoid functor in bf16 arithmetic (every operation rounds to bf16).
__device__ __forceinline__ float sigmoid_bf16(float x) {
  const float e = round_bf(expf_det(__builtin_fabsf(x)));
  const float d = round_bf(1.0f + e);
  const float y = round_bf(1.0f / d);
  return (x < 0.0f) ? y : round_bf(1.0f - y);
}

__device__ __forceinline__ float silu_bf16(float x) { return round_bf(x * sigmoid_bf16(x)); }

// Lanes sharing one row of the q4 GEMV: largest power of two <= 64 leaving
// every lane at least 4 blocks of 32 elements.
__host__ __device__ constexpr int lanes_for_blocks(int nb) {
  int L = 1;
  while (L < 64 && (L * 2) * 4 <= nb) L *= 2;
  return L;
}

// Packed scale/bias row of a [*, K] q4 matrix (see qrows.h): lane classes Q x
// entries per class, in u32.
__host__ __device__ constexpr int sb_entries_per_class(int K) {
  return (K / 32 + lanes_for_blocks(K / 32) - 1) / lanes_for_blocks(K / 32);
}
__host__ __device__ constexpr int sb_classes(int K, int gs) {
  return lanes_for_blocks(K / 32) / (gs / 32) > 0 ? lanes_for_blocks(K / 32) / (gs / 32) : 1;
}
__host__ __device__ constexpr int sb_row_len(int K, int gs) { return sb_classes(K, gs) * sb_entries_per_class(K); }

// ---------------------------------------------------------------------------
// Prepared activation block: 28 dwords (16-byte aligned for 128-bit LDS reads).
//   [0..7]   limb 0 (bits 0-7 of m):   dwords e0 e1 e2 e3 o0 o1 o2 o3
//   [8..15]  limb 1 (bits 8-15)
//   [16..23] limb 2 (bits 16-23, signed byte)
//   [24] p = 2^(E-149) as float bits, [25] SX = (float)(sum m) * p, [26..27] 0
// e_t holds the limb bytes of elements 8t, 8t+2, 8t+4, 8t+6 and o_t those of
// 8t+1, 8t+3, 8t+5, 8t+7 -- the byte order that (w & 0x0f0f0f0f) and
// ((w >> 4) & 0x0f0f0f0f) give a packed weight word.
constexpr int XP_DW = 28;

__device__ __forceinline__ float block_scale(int E) {
  return (E >= 23) ? __uint_as_float((uint32_t)(E - 22) << 23) : __uint_as_float(1u << E);
}

// Build one prepared block from 32 bf16 values (one thread does a block).
__device__ inline void xprep_block(const bf16* __restrict__ x32, uint32_t* __restrict__ out) {
  uint32_t h[32];
  int E = 1;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    h[i] = x32[i];
    int f = (h[i] >> 7) & 0xff;
    f = f < 1 ? 1 : f;
    E = f > E ? f : E;
  }
  uint32_t limb[3][8];
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) limb[k][j] = 0;
  int32_t sm = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int field = (h[i] >> 7) & 0xff;
    const int f = field < 1 ? 1 : field;
    const int32_t sig = (int32_t)((field ? 0x80u : 0u) | (h[i] & 0x7fu));
    const int sh = f - E + 15;
    int32_t mag = (sh >= 0) ? (sig << sh) : ((sh > -31) ? (sig >> (-sh)) : 0);
    const int32_t m = (h[i] & 0x8000u) ? -mag : mag;
    sm += m;
    const uint32_t u = (uint32_t)m & 0xffffffu;
    const int t = i >> 3, k8 = i & 7;
    const int slot = (k8 & 1) ? 4 + t : t;  // odd elements -> o_t
    const int byte = k8 >> 1;
    limb[0][slot] |= (u & 0xffu) << (8 * byte);
    limb[1][slot] |= ((u >> 8) & 0xffu) << (8 * byte);
    limb[2][slot] |= ((u >> 16) & 0xffu) << (8 * byte);
  }
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) out[k * 8 + j] = limb[k][j];
  const float p = block_scale(E);
  out[24] = __float_as_uint(p);
  out[25] = __float_as_uint((float)sm * p);
  out[26] = 0u;
  out[27] = 0u;
}

// The same prepared block built by 32 consecutive lanes (lane i holding
// element i, bf16 bits h) and written straight to `dst` (28 dwords, LDS or
// global), with no staging and no barrier: limb word (k, slot) holds byte k of
// the elements t*8 + par + 2*b (b = 0..3; slot = t or 4 + t for par 0 or 1),
// so two lane exchanges (xor 2, xor 4) assemble it and lane t*8 + par stores
// it.  Integer sums are exact, so the lane reduction order does not matter.
// All 32 lanes of the group must be active.
__device__ __forceinline__ void xprep_lanes_direct(uint32_t h, int i, uint32_t* __restrict__ dst) {
  const int field = (h >> 7) & 0xff;
  const int f = field < 1 ? 1 : field;
  int E = f;
  E = max(E, lane_xor_i<16>(E));
  E = max(E, lane_xor_i<8>(E));
  E = max(E, lane_xor_i<4>(E));
  E = max(E, lane_xor_i<2>(E));
  E = max(E, lane_xor_i<1>(E));
  const int32_t sig = (int32_t)((field ? 0x80u : 0u) | (h & 0x7fu));
  const int sh = f - E + 15;
  const int32_t mag = (sh >= 0) ? (sig << sh) : ((sh > -31) ? (sig >> (-sh)) : 0);
  const int32_t m = (h & 0x8000u) ? -mag : mag;
  int32_t sm = m;
  sm += lane_xor_i<16>(sm);
  sm += lane_xor_i<8>(sm);
  sm += lane_xor_i<4>(sm);
  sm += lane_xor_i<2>(sm);
  sm += lane_xor_i<1>(sm);
  const uint32_t u = (uint32_t)m & 0xffffffu;
  const int at = 4 * (i & 6);  // bit offset of this element's byte: byte (i & 7) >> 1 of its word
  uint32_t w0 = (u & 0xffu) << at, w1 = ((u >> 8) & 0xffu) << at, w2 = (u >> 16) << at;
  w0 |= lane_xor<2>(w0);
  w1 |= lane_xor<2>(w1);
  w2 |= lane_xor<2>(w2);
  w0 |= lane_xor<4>(w0);
  w1 |= lane_xor<4>(w1);
  w2 |= lane_xor<4>(w2);
  if ((i & 6) == 0) {
    const int slot = (i & 1) ? 4 + (i >> 3) : (i >> 3);
    dst[slot] = w0;
    dst[8 + slot] = w1;
    dst[16 + slot] = w2;
  } else if (i < 8) {  // lanes 2..7: the scale words and the zero pad
    const float p = block_scale(E);
    if (i == 2) dst[24] = __float_as_uint(p);
    if (i == 3) dst[25] = __float_as_uint((float)sm * p);
    if (i == 4) dst[26] = 0u;
    if (i == 5) dst[27] = 0u;
  }
}

// Exact nibble x limb sums of one 32-element block; w = 4 packed words.
// Returns DXraw = fmaf((float)D2, 65536, (float)(D1*256 + D0)).
__device__ __forceinline__ float block_dot(const uint32_t w[4], const uint32_t* __restrict__ xl) {
  const uint4* x4 = reinterpret_cast<const uint4*>(xl);  // 16-byte aligned prepared block
  const uint4 e0 = x4[0], o0 = x4[1], e1 = x4[2], o1 = x4[3], e2 = x4[4], o2 = x4[5];
  const uint32_t l0e[4] = {e0.x, e0.y, e0.z, e0.w}, l0o[4] = {o0.x, o0.y, o0.z, o0.w};
  const uint32_t l1e[4] = {e1.x, e1.y, e1.z, e1.w}, l1o[4] = {o1.x, o1.y, o1.z, o1.w};
  const uint32_t l2e[4] = {e2.x, e2.y, e2.z, e2.w}, l2o[4] = {o2.x, o2.y, o2.z, o2.w};
  uint32_t d0 = 0, d1 = 0;
  int32_t d2 = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = w[t] & 0x0f0f0f0fu;
    const uint32_t hi = (w[t] >> 4) & 0x0f0f0f0fu;
    d0 = __builtin_amdgcn_udot4(lo, l0e[t], d0, false);
    d0 = __builtin_amdgcn_udot4(hi, l0o[t], d0, false);
    d1 = __builtin_amdgcn_udot4(lo, l1e[t], d1, false);
    d1 = __builtin_amdgcn_udot4(hi, l1o[t], d1, false);
    d2 = __builtin_amdgcn_sdot4((int)lo, (int)l2e[t], d2, false);
    d2 = __builtin_amdgcn_sdot4((int)hi, (int)l2o[t], d2, false);
  }
  const int32_t low = (int32_t)(d1 * 256u + d0);
  return __builtin_fmaf((float)d2, 65536.0f, (float)low);
}

// acc <- fmaf(b, SX, fmaf(s, DXraw * p, acc))
__device__ __forceinline__ float block_accum(float acc, float dxraw, float s, float b,
                                             const uint32_t* __restrict__ xl) {
  const uint2 ps = reinterpret_cast<const uint2*>(xl)[12];
  const float p = __uint_as_float(ps.x);
  const float sx = __uint_as_float(ps.y);
  acc = __builtin_fmaf(s, dxraw * p, acc);
  return __builtin_fmaf(b, sx, acc);
}

// xor butterfly over groups of L lanes (every lane of the group ends with the sum)
template <int L>
__device__ __forceinline__ float lane_fold(float v) {
  return fold_sum<L / 2>(v);
}

__device__ __forceinline__ float wave_fold64(float v) { return fold_sum<32>(v); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes global -> LDS with no register round trip (gfx950
// global_load_lds_dwordx4): lane l of the wave writes LDS unit wave_base + l,
// so wave_base must be the same for every lane of the wave; lanes that are
// switched off write nothing.  The data is in LDS once this wave's vector
// memory counter has drained: lds_dma_wait(), then a barrier for the others.
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void lds_dma16(uint4* wave_base, const void* src) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)wave_base, 16, 0, 0);
}
// s_waitcnt vmcnt(0): every vector memory load of this wave has landed (expcnt, lgkmcnt left open)
__device__ __forceinline__ void lds_dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// 16-byte streaming load of packed weights (read once per step: non-temporal)
__device__ __forceinline__ uint4 ldg16(const uint32_t* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace mtpx
