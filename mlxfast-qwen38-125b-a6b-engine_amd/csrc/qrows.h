// Weight-row walker shared by the dense and the expert GEMVs.
//
// A row of an affine-4-bit matrix [*, K] is split over L lanes: lane `sub`
// owns the 32-element blocks sub, sub+L, sub+2L, ... (IT of them when
// K/32 == L*IT exactly; IT == 0 selects a predicated walker for up to QMV_IT
// blocks).  load() issues the 16-byte weight loads and the scale/bias loads;
// dot() consumes them against one prepared activation vector.
//
// Packed scale/bias rows.  Next to the checkpoint's bf16 scales [N, K/gs] and
// biases [N, K/gs], a matrix may carry its (scale, bias) pairs as one u32 each
// (scale in the low half), ordered so that every lane finds the pairs of its
// blocks contiguous: entry [q][it] of a row is the pair of the group of block
// q*r + L*it (r = gs/32, q = sub / r: lanes that share groups share entries).
// A lane then fetches its pairs with one or two vector loads instead of two
// 2-byte loads per block.  Same bytes, same values.
#pragma once
#include "mtpx_kernels.h"

namespace mtpx {

template <int L, int IT>
struct QRow {
  static constexpr int NB = IT ? IT : QMV_IT;
  uint32_t w[NB][4];
  uint32_t sb[NB];  // bf16 scale in the low half, bf16 bias in the high half
  bool ok;          // a real row: dot() of a padding row is 0

  // sbrow: this row's packed pairs (null: the checkpoint's scale and bias rows).
  // A padding row (valid false) must still point at a real row of the matrix:
  // its loads are issued like any other (no branch, so no wait at a join) and
  // its dot is forced to 0.
  // CACHED: plain loads (a prefill batch rereads the rows from L2), else streaming (non-temporal) loads
  template <bool CACHED = false>
  __device__ __forceinline__ void load(const uint32_t* __restrict__ wrow, const bf16* __restrict__ srow,
                                       const bf16* __restrict__ brow, const uint32_t* __restrict__ sbrow, int nb,
                                       int gs, int sub, bool valid) {
    ok = valid;
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int j = sub + it * L;
      if (IT ? true : j < nb) {
        const uint4 v = CACHED ? *reinterpret_cast<const uint4*>(wrow + (size_t)j * 4) : ldg16(wrow + (size_t)j * 4);
        w[it][0] = v.x;
        w[it][1] = v.y;
        w[it][2] = v.z;
        w[it][3] = v.w;
      } else {
        w[it][0] = w[it][1] = w[it][2] = w[it][3] = 0u;
      }
    }
    if (!sbrow) {  // every scale and bias load in flight before the first merge
      uint32_t sv[NB], bv[NB];
#pragma unroll
      for (int it = 0; it < NB; ++it) {
        const int j = sub + it * L;
        const int g = gs == 64 ? (j >> 1) : j;  // group of block j (gs is 32 or 64)
        const bool in = IT ? true : j < nb;
        sv[it] = in ? srow[g] : 0u;
        bv[it] = in ? brow[g] : 0u;
      }
#pragma unroll
      for (int it = 0; it < NB; ++it) sb[it] = sv[it] | (bv[it] << 16);
    } else {
      const int nbv = IT ? IT : (nb + L - 1) / L;  // entries per lane class
      const uint32_t* e = sbrow + (size_t)(gs == 64 ? (sub >> 1) : sub) * nbv;
      if constexpr (IT != 0) {
#pragma unroll
        for (int it = 0; it + 4 <= NB; it += 4) {
          uint4 v;
          __builtin_memcpy(&v, e + it, 16);
          sb[it] = v.x;
          sb[it + 1] = v.y;
          sb[it + 2] = v.z;
          sb[it + 3] = v.w;
        }
#pragma unroll
        for (int it = NB & ~3; it < NB; ++it) sb[it] = e[it];
      } else {
#pragma unroll
        for (int it = 0; it < NB; ++it) sb[it] = (sub + it * L < nb) ? e[it] : 0u;
      }
    }
  }

  // load() with the scale/bias pairs taken from packed rows only (sbrow != null):
  // one code path, so no load of the other layout's path is ever waited for.
  template <bool PK, bool CACHED = false>
  __device__ __forceinline__ void load_as(const uint32_t* __restrict__ wrow, const bf16* __restrict__ srow,
                                          const bf16* __restrict__ brow, const uint32_t* __restrict__ sbrow, int nb,
                                          int gs, int sub, bool valid) {
    if constexpr (PK) {
      load<CACHED>(wrow, nullptr, nullptr, sbrow, nb, gs, sub, valid);
    } else {
      load<CACHED>(wrow, srow, brow, nullptr, nb, gs, sub, valid);
    }
  }

  // Make the held words opaque to the compiler, so the nibble masks of a
  // loop over tokens are recomputed per token instead of hoisted (which would
  // hold two masked copies of every word live and double the registers).
  // It also reads every loaded register, so a loop that may compute zero
  // tokens still retires this row's loads here and not at a later reuse.
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      asm volatile("" : "+v"(w[it][0]), "+v"(w[it][1]), "+v"(w[it][2]), "+v"(w[it][3]), "+v"(sb[it]));
    }
  }

  // lane partial of the row against a prepared activation vector
  __device__ __forceinline__ float dot(const uint32_t* __restrict__ xpv, int nb, int sub) const {
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int j = sub + it * L;
      if (IT ? true : j < nb) {
        const uint32_t* xl = xpv + (size_t)j * XP_DW;
        const float s = __uint_as_float(sb[it] << 16);
        const float b = __uint_as_float(sb[it] & 0xffff0000u);
        acc = block_accum(acc, block_dot(w[it], xl), s, b, xl);
      }
    }
    return ok ? acc : 0.0f;
  }
};

// Lane partials of two rows against one prepared activation vector: each
// activation block is read from LDS once for both rows.  FENCE: keep one
// block's activation words live at a time (fewer registers) instead of
// letting the scheduler overlap blocks (more LDS reads in flight).
template <int L, int IT, bool FENCE = true>
__device__ __forceinline__ void dot2(const QRow<L, IT>& A, const QRow<L, IT>& B, const uint32_t* __restrict__ xpv,
                                     int nb, int sub, float& ra, float& rb) {
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int it = 0; it < QRow<L, IT>::NB; ++it) {
    const int j = sub + it * L;
    if (IT ? true : j < nb) {
      const uint32_t* xl = xpv + (size_t)j * XP_DW;
      a = block_accum(a, block_dot(A.w[it], xl), __uint_as_float(A.sb[it] << 16),
                      __uint_as_float(A.sb[it] & 0xffff0000u), xl);
      b = block_accum(b, block_dot(B.w[it], xl), __uint_as_float(B.sb[it] << 16),
                      __uint_as_float(B.sb[it] & 0xffff0000u), xl);
    }
    if constexpr (FENCE) __builtin_amdgcn_sched_barrier(0);
  }
  ra = A.ok ? a : 0.0f;
  rb = B.ok ? b : 0.0f;
}

// Copy `words` dwords global -> LDS: 16-byte LDS-direct loads when both ends
// allow it (thread t copies units t, t + blockDim, ...; blockDim a multiple of
// 64), else dword copies through registers.  Follow with stage_sync() before
// the LDS is read.
__device__ __forceinline__ void stage16(uint32_t* __restrict__ dst, const uint32_t* __restrict__ src, int words) {
  if ((((uintptr_t)src | (uintptr_t)dst) & 15) == 0 && (words & 3) == 0) {
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    const int n4 = words / 4, lane = threadIdx.x & 63;
    for (int i = threadIdx.x; i < n4; i += blockDim.x) lds_dma16(d4 + (i - lane), s4 + i);
  } else {
    for (int i = threadIdx.x; i < words; i += blockDim.x) dst[i] = src[i];
  }
}

// The staged data of every wave is in LDS (this wave's loads drained, then the barrier).
__device__ __forceinline__ void stage_sync() {
  lds_dma_wait();
  __syncthreads();
}

// Dispatch a launcher templated on <L, IT> for the shapes the model uses, with
// the predicated walker for every other depth.
#define MTPX_QROW_DISPATCH(nb, FN, ...)                                   \
  do {                                                                     \
    const int L_ = lanes_for_blocks(nb);                                   \
    const int IT_ = ((nb) % L_ == 0) ? (nb) / L_ : 0;                      \
    switch (L_ * 16 + (IT_ >= 4 && IT_ <= 7 ? IT_ : 0)) {                  \
      case 2 * 16 + 4: return FN<2, 4>(__VA_ARGS__);                       \
      case 2 * 16 + 5: return FN<2, 5>(__VA_ARGS__);                       \
      case 4 * 16 + 4: return FN<4, 4>(__VA_ARGS__);                       \
      case 4 * 16 + 5: return FN<4, 5>(__VA_ARGS__);                       \
      case 4 * 16 + 6: return FN<4, 6>(__VA_ARGS__);                       \
      case 8 * 16 + 4: return FN<8, 4>(__VA_ARGS__);                       \
      case 8 * 16 + 5: return FN<8, 5>(__VA_ARGS__);                       \
      case 16 * 16 + 4: return FN<16, 4>(__VA_ARGS__);                     \
      case 16 * 16 + 5: return FN<16, 5>(__VA_ARGS__);                     \
      case 32 * 16 + 4: return FN<32, 4>(__VA_ARGS__);                     \
      case 32 * 16 + 6: return FN<32, 6>(__VA_ARGS__);                     \
      case 64 * 16 + 5: return FN<64, 5>(__VA_ARGS__);                     \
      default: break;                                                      \
    }                                                                      \
    switch (L_) {                                                          \
      case 1: return FN<1, 0>(__VA_ARGS__);                                \
      case 2: return FN<2, 0>(__VA_ARGS__);                                \
      case 4: return FN<4, 0>(__VA_ARGS__);                                \
      case 8: return FN<8, 0>(__VA_ARGS__);                                \
      case 16: return FN<16, 0>(__VA_ARGS__);                              \
      case 32: return FN<32, 0>(__VA_ARGS__);                              \
      default: return FN<64, 0>(__VA_ARGS__);                              \
    }                                                                      \
  } while (0)

}  // namespace mtpx
