// Dense affine-4-bit GEMV (y[M,N] = x[M,K] . W[N,K]^T), activation block
// preparation, device-side MLX affine quantisation and seeded weight init.
//
// Weight format (MLX affine 4-bit, unchanged from the reference checkpoint):
// packed uint32 [N, K/8], element k at bits 4*(k%8) of word k/8; bf16 scale
// and bias [N, K/gs].  Arithmetic: see mtpx_device.h.
#include "mtpx_kernels.h"

namespace mtpx {

// One thread per 32-element block of x [M, K] -> xp [M, K/32, XP_DW].
__global__ void k_xprep(const bf16* __restrict__ x, int M, int K, uint32_t* __restrict__ xp) {
  const int nb = K / 32;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * nb) return;
  const int m = i / nb, j = i % nb;
  xprep_block(x + (size_t)m * K + (size_t)j * 32, xp + (size_t)i * XP_DW);
}

// Rows of a 4-bit matrix walked by lanes: `sub` = lane within the row's L
// lanes handles blocks sub, sub+L, ... (at most QMV_IT of them).
template <int L>
struct RowLoad {
  uint32_t w[QMV_IT][4];
  float s[QMV_IT], b[QMV_IT];
  __device__ __forceinline__ void load(const uint32_t* __restrict__ wrow, const bf16* __restrict__ srow,
                                       const bf16* __restrict__ brow, int nb, int gs, int sub,
                                       bool valid) {
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
        s[it] = 0.0f;
        b[it] = 0.0f;
      }
    }
  }
  // lane partial of this row against one prepared activation vector (LDS)
  __device__ __forceinline__ float dot(const uint32_t* __restrict__ xpv, int nb, int sub) const {
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < QMV_IT; ++it) {
      const int j = sub + it * L;
      if (j < nb) {
        const uint32_t* xl = xpv + (size_t)j * XP_DW;
        const float d = block_dot(w[it], xl);
        acc = block_accum(acc, d, s[it], b[it], xl);
      }
    }
    return acc;
  }
};

// Dense GEMV.  256 threads; each lane owns two rows (RPL = 2) so every LDS
// read of a prepared activation block feeds two weight rows.
template <int L>
__global__ __launch_bounds__(256) void k_qmv(const uint32_t* __restrict__ wq, const bf16* __restrict__ sc,
                                             const bf16* __restrict__ bi, int N, int K, int gs,
                                             const uint32_t* __restrict__ xp, int M, bf16* __restrict__ y,
                                             float* __restrict__ yf, int rows_per_wg) {
  extern __shared__ uint32_t lds[];
  const int nb = K / 32, ng = K / gs;
  const int words = M * nb * XP_DW;
  for (int i = threadIdx.x; i < words; i += blockDim.x) lds[i] = xp[i];
  __syncthreads();
  constexpr int RW = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % L, grp = lane / L;
  const int row0 = blockIdx.x * rows_per_wg;
  const int row_end = min(row0 + rows_per_wg, N);
  for (int base = row0 + wave * RW * 2; base < row_end; base += 4 * RW * 2) {
    const int rA = base + grp * 2, rB = rA + 1;
    const bool vA = rA < row_end, vB = rB < row_end;
    RowLoad<L> A, B;
    A.load(wq + (size_t)rA * (K / 8), sc + (size_t)rA * ng, bi + (size_t)rA * ng, nb, gs, sub, vA);
    B.load(wq + (size_t)rB * (K / 8), sc + (size_t)rB * ng, bi + (size_t)rB * ng, nb, gs, sub, vB);
    for (int m = 0; m < M; ++m) {
      const uint32_t* xm = lds + (size_t)m * nb * XP_DW;
      float a = lane_fold<L>(A.dot(xm, nb, sub));
      float b = lane_fold<L>(B.dot(xm, nb, sub));
      if (sub == 0) {
        if (vA) {
          y[(size_t)m * N + rA] = f2bf(a);
          if (yf) yf[(size_t)m * N + rA] = a;
        }
        if (vB) {
          y[(size_t)m * N + rB] = f2bf(b);
          if (yf) yf[(size_t)m * N + rB] = b;
        }
      }
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

// ---------------------------------------------------------------------------
// host launchers

hipError_t launch_xprep(const bf16* x, int M, int K, uint32_t* xp, hipStream_t st) {
  const int n = M * (K / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_xprep, dim3((n + 127) / 128), dim3(128), 0, st, x, M, K, xp);
  return hipGetLastError();
}

template <int L>
static hipError_t qmv_l(const uint32_t* wq, const bf16* s, const bf16* b, int N, int K, int gs,
                        const uint32_t* xp, int M, bf16* y, float* yf, hipStream_t st) {
  constexpr int rows_iter = 4 * (64 / L) * 2;
  // aim for >= 1024 workgroups where the matrix allows, at least one row iteration each
  int iters = (N + rows_iter - 1) / rows_iter;
  int per = (iters + 1023) / 1024;
  if (per < 1) per = 1;
  const int rows_per_wg = per * rows_iter;
  const int grid = (N + rows_per_wg - 1) / rows_per_wg;
  const size_t lds = (size_t)M * (K / 32) * XP_DW * 4;
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_qmv<L>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_qmv<L>, dim3(grid), dim3(256), lds, st, wq, s, b, N, K, gs, xp, M, y, yf,
                     rows_per_wg);
  return hipGetLastError();
}

hipError_t launch_qmv(const uint32_t* wq, const bf16* s, const bf16* b, int N, int K, int gs,
                      const uint32_t* xp, int M, bf16* y, float* yf, hipStream_t st) {
  switch (lanes_for_blocks(K / 32)) {
    case 1: return qmv_l<1>(wq, s, b, N, K, gs, xp, M, y, yf, st);
    case 2: return qmv_l<2>(wq, s, b, N, K, gs, xp, M, y, yf, st);
    case 4: return qmv_l<4>(wq, s, b, N, K, gs, xp, M, y, yf, st);
    case 8: return qmv_l<8>(wq, s, b, N, K, gs, xp, M, y, yf, st);
    case 16: return qmv_l<16>(wq, s, b, N, K, gs, xp, M, y, yf, st);
    case 32: return qmv_l<32>(wq, s, b, N, K, gs, xp, M, y, yf, st);
    default: return qmv_l<64>(wq, s, b, N, K, gs, xp, M, y, yf, st);
  }
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
