// Dense affine-4-bit GEMV (y[M,N] = x[M,K] . W[N,K]^T), activation block
// preparation, device-side MLX affine quantisation and seeded weight init.
//
// Weight format (MLX affine 4-bit, unchanged from the reference checkpoint):
// packed uint32 [N, K/8], element k at bits 4*(k%8) of word k/8; bf16 scale
// and bias [N, K/gs].  Arithmetic: see mtpx_device.h.
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

// Dense GEMV.  256 threads; every lane-group owns two rows (RPL = 2) so each
// LDS read of a prepared activation block feeds two weight rows.  A wave's
// rows are loaded before the activations are staged.
template <int L, int IT>
__global__ __launch_bounds__(256) void k_qmv(const uint32_t* __restrict__ wq, const bf16* __restrict__ sc,
                                             const bf16* __restrict__ bi, const uint32_t* __restrict__ sbp,
                                             int N, int K, int gs,
                                             const uint32_t* __restrict__ xp, int M, bf16* __restrict__ y,
                                             float* __restrict__ yf, int rows_per_wg) {
  extern __shared__ uint32_t lds[];
  constexpr int RW = 64 / L;
  constexpr int RPW = 2 * RW;  // rows per wave pass
  const int nb = K / 32, ng = K / gs, P = sb_row_len(K, gs);
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
    A.load(wq + (size_t)ra * (K / 8), sc + (size_t)ra * ng, bi + (size_t)ra * ng,
           sbp ? sbp + (size_t)ra * P : nullptr, nb, gs, sub, vA);
    B.load(wq + (size_t)rb * (K / 8), sc + (size_t)rb * ng, bi + (size_t)rb * ng,
           sbp ? sbp + (size_t)rb * P : nullptr, nb, gs, sub, vB);
  };
  if (base < row_end) load2(base);  // first rows in flight before the staging
  stage16(lds, xp, M * nb * XP_DW);
  stage_sync();
  for (bool first = true; base < row_end; base += 4 * RPW, first = false) {  // uniform per wave
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

template <int L, int IT>
static hipError_t qmv_li(const uint32_t* wq, const bf16* s, const bf16* b, const uint32_t* sb, int N, int K, int gs,
                         const uint32_t* xp, int M, bf16* y, float* yf, hipStream_t st) {
  constexpr int rows_pass = 4 * (64 / L) * 2;
  // about two workgroups per CU, at least one pass each
  const int passes = (N + rows_pass - 1) / rows_pass;
  const int per = (passes + 511) / 512;
  const int rows_per_wg = per * rows_pass;
  const int grid = (N + rows_per_wg - 1) / rows_per_wg;
  const size_t lds = (size_t)M * (K / 32) * XP_DW * 4;
  static size_t cur = 0;
  hipError_t e = ensure_lds(k_qmv<L, IT>, lds, cur);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_qmv<L, IT>), dim3(grid), dim3(256), lds, st, wq, s, b, sb, N, K, gs, xp, M, y, yf,
                     rows_per_wg);
  return hipGetLastError();
}

static hipError_t qmv_tokens(const uint32_t* wq, const bf16* s, const bf16* b, const uint32_t* sb, int N, int K,
                             int gs, const uint32_t* xp, int M, bf16* y, float* yf, hipStream_t st) {
  MTPX_QROW_DISPATCH(K / 32, qmv_li, wq, s, b, sb, N, K, gs, xp, M, y, yf, st);
}

hipError_t launch_qmv(const uint32_t* wq, const bf16* s, const bf16* b, const uint32_t* sb, int N, int K, int gs,
                      const uint32_t* xp, int M, bf16* y, float* yf, hipStream_t st) {
  // tokens per launch: as many prepared activation vectors as fit in one workgroup's LDS
  const size_t per_token = (size_t)(K / 32) * XP_DW * 4;
  int chunk = (int)((160 * 1024) / per_token);
  chunk = chunk < 1 ? 1 : chunk;
  for (int m0 = 0; m0 < M; m0 += chunk) {
    const int mc = M - m0 < chunk ? M - m0 : chunk;
    const hipError_t e = qmv_tokens(wq, s, b, sb, N, K, gs, xp + (size_t)m0 * (K / 32) * XP_DW, mc, y + (size_t)m0 * N,
                                    yf ? yf + (size_t)m0 * N : nullptr, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
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
