// Pieces of the MTP head's draft step (S <= 8 inputs) that are not GEMVs:
//   embed   : rows of the q4 embedding table, MLX affine_dequantize arithmetic
//             in bf16: w = bf16(bf16(scale * q) + bias)
//   hc_norm : hyper-connection inject + group RMS norm: stream = residual
//             (+ out * inject), normed = scale * bf16(stream * inv_rms) per
//             (row, stream) group, plus the prepared blocks of the normed row
//             for the down GEMV
//   silu    : SiLU (bf16) of the mixer's low-rank rows + their prepared blocks
//   hc_mix  : input = bf16 running sum over streams of
//             bf16(sigmoid(w) * normed); inject = 2 * sigmoid(inj); prepared
//             blocks of the input for the next GEMV
// Every workgroup of hc_norm folds its whole group's sum of squares in the
// order of k_rmsnorm (thread t: elements t, t+256, ...; waves summed
// ((w0+w1)+w2)+w3) and writes a 256-element slice, so the slices of one group
// run in parallel.
// Reference: Runner/Qwen4ExpMTP.swift:101-130 (head wiring),
// Runner/FastModel/TrackFastHead.swift:101-153 (fast head forward),
// Runner/FastModel/TrackFastKernels2.swift:60-280 (injectNorm, hcMix),
// Runner/FastModel/TrackFastMixer.swift:14-224 (downInject, upMix),
// MLX/backend/metal/kernels/quantized.h:3314-3372 (affine_dequantize).
#include "mtpx_kernels.h"

namespace mtpx {

// grid (ceil(H/2048), S), 256 threads; thread = one packed word (8 elements).
// An id outside [0, V) yields a zero row.
__global__ __launch_bounds__(256) void k_embed_rows(const uint32_t* __restrict__ wq, const bf16* __restrict__ sc,
                                                    const bf16* __restrict__ bi, int H, int gs, int64_t V,
                                                    const int32_t* __restrict__ ids, bf16* __restrict__ out) {
  const int s = blockIdx.y;
  const int wd = blockIdx.x * 256 + threadIdx.x;  // word index in the row
  if (wd >= H / 8) return;
  const int64_t id = ids[s];
  bf16* o = out + (size_t)s * H + (size_t)wd * 8;
  if (id < 0 || id >= V) {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0;
    return;
  }
  const uint32_t w = wq[id * (H / 8) + wd];
  const int g = (wd * 8) / gs;  // gs >= 32: the 8 elements share one group
  const float scale = bf2f(sc[id * (H / gs) + g]);
  const float bias = bf2f(bi[id * (H / gs) + g]);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = f2bf(round_bf(scale * (float)((w >> (4 * i)) & 0xfu)) + bias);
}

// grid (hc, S, ceil(H/256)), 256 threads; H <= 256 * IT (EXACT: H == 256 * IT).  MODE 0: stream =
// residual; 1: + out; 2: + bf16(out * inject).  Every load is issued up front and unconditionally
// (clamped indices) and kept as raw bf16 bits until its use, so the residual and sublayer rows, the
// inject value and the norm scale arrive in one round trip.
template <int IT, bool EXACT, int MODE>
__global__ __launch_bounds__(256) void k_hc_norm(const bf16* __restrict__ residual, const bf16* __restrict__ out,
                                                 const bf16* __restrict__ inject, int hc, int H, int tile,
                                                 const bf16* __restrict__ scale, float eps,
                                                 bf16* __restrict__ stream, bf16* __restrict__ normed,
                                                 uint32_t* __restrict__ xp) {
  __shared__ float wsum[4];
  const int c = blockIdx.x, s = blockIdx.y, sl = blockIdx.z, t = threadIdx.x;
  const size_t W = (size_t)hc * H;
  const size_t base = (size_t)s * W + (size_t)c * H;
  const bf16* rr = tile ? residual + (size_t)s * H : residual + base;
  const bf16* orow = MODE > 0 ? out + (size_t)s * H : rr;
  const int d = sl * 256 + t;
  const uint32_t injb = MODE == 2 ? (uint32_t)inject[(size_t)s * hc + c] : 0u;
  const uint32_t scb = scale[(size_t)c * H + (d < H ? d : H - 1)];
  bf16 rv[IT], ov[IT];
#pragma unroll
  for (int j = 0; j < IT; ++j) {
    const int dj = t + 256 * j;
    const int dd = EXACT ? dj : (dj < H ? dj : H - 1);
    rv[j] = rr[dd];
    if (MODE > 0) ov[j] = orow[dd];
  }
  asm volatile("" ::: "memory");
  const float inj = __uint_as_float(injb << 16);
  float v[IT];
  float acc = 0.0f, vo = 0.0f;
#pragma unroll
  for (int j = 0; j < IT; ++j) {
    const bool in = EXACT || t + 256 * j < H;
    float x = bf2f(rv[j]);
    if (MODE > 0) {
      const float o = bf2f(ov[j]);
      x = round_bf(x + (MODE == 2 ? round_bf(o * inj) : o));
    }
    v[j] = in ? x : 0.0f;
    if (in) acc = __builtin_fmaf(v[j], v[j], acc);
    if (j == sl) vo = v[j];
  }
  acc = wave_fold64(acc);
  if ((t & 63) == 0) wsum[t >> 6] = acc;
  __syncthreads();
  const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  const float inv = 1.0f / sqrtf(total / (float)H + eps);
  bf16 n = 0;
  if (d < H) {
    if (stream) stream[base + d] = f2bf(vo);
    n = f2bf(__uint_as_float(scb << 16) * round_bf(vo * inv));
    if (normed) normed[base + d] = n;
  }
  // blocks of the normed row [S, hc*H]: H % 32 == 0, so a block never straddles streams
  if (xp && d < H) xprep_lanes_direct(n, t & 31, xp + (base + d) / 32 * XP_DW);
}

// grid (S, ceil(LW/256)), 256 threads; LW % 32 == 0.
__global__ __launch_bounds__(256) void k_silu_xprep(const bf16* __restrict__ lo, int LW, bf16* __restrict__ act,
                                                    uint32_t* __restrict__ xp) {
  const int s = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
  bf16 a = 0;
  if (j < LW) {
    a = f2bf(silu_bf16(bf2f(lo[(size_t)s * LW + j])));
    act[(size_t)s * LW + j] = a;
  }
  if (j < LW) xprep_lanes_direct(a, threadIdx.x & 31, xp + ((size_t)s * LW + j) / 32 * XP_DW);
}

// grid (S, ceil(H/256)), 256 threads.
__global__ __launch_bounds__(256) void k_hc_mix(const bf16* __restrict__ w, const bf16* __restrict__ normed,
                                                const bf16* __restrict__ inj, int hc, int H,
                                                bf16* __restrict__ input, bf16* __restrict__ inject_out,
                                                uint32_t* __restrict__ xp) {
  const int s = blockIdx.x, d = blockIdx.y * 256 + threadIdx.x;
  const size_t W = (size_t)hc * H;
  bf16 y = 0;
  if (d < H) {
    float acc = 0.0f;
    for (int c = 0; c < hc; ++c) {
      const size_t i = (size_t)s * W + (size_t)c * H + d;
      acc = round_bf(acc + round_bf(sigmoid_bf16(bf2f(w[i])) * bf2f(normed[i])));
    }
    y = f2bf(acc);
    input[(size_t)s * H + d] = y;
  }
  if (inj && inject_out && blockIdx.y == 0 && threadIdx.x < hc)
    inject_out[(size_t)s * hc + threadIdx.x] = f2bf(2.0f * sigmoid_bf16(bf2f(inj[(size_t)s * hc + threadIdx.x])));
  if (xp && d < H) xprep_lanes_direct(y, threadIdx.x & 31, xp + ((size_t)s * H + d) / 32 * XP_DW);
}

// ---------------------------------------------------------------------------
hipError_t launch_embed_rows(const uint32_t* wq, const bf16* s, const bf16* b, int H, int gs, int64_t V,
                             const int32_t* ids, int S, bf16* out, hipStream_t st) {
  hipLaunchKernelGGL(k_embed_rows, dim3((H / 8 + 255) / 256, S), dim3(256), 0, st, wq, s, b, H, gs, V, ids, out);
  return hipGetLastError();
}

template <int IT, bool EXACT>
static void hc_norm_mode(const dim3& grid, const bf16* residual, const bf16* out, const bf16* inject, int hc, int H,
                         int tile, const bf16* scale, float eps, bf16* stream, bf16* normed, uint32_t* xp,
                         hipStream_t st) {
  if (!out)
    hipLaunchKernelGGL((k_hc_norm<IT, EXACT, 0>), grid, dim3(256), 0, st, residual, out, inject, hc, H, tile, scale,
                       eps, stream, normed, xp);
  else if (!inject)
    hipLaunchKernelGGL((k_hc_norm<IT, EXACT, 1>), grid, dim3(256), 0, st, residual, out, inject, hc, H, tile, scale,
                       eps, stream, normed, xp);
  else
    hipLaunchKernelGGL((k_hc_norm<IT, EXACT, 2>), grid, dim3(256), 0, st, residual, out, inject, hc, H, tile, scale,
                       eps, stream, normed, xp);
}

hipError_t launch_hc_norm(const bf16* residual, const bf16* out, const bf16* inject, int S, int hc, int H,
                          int tile, const bf16* scale, float eps, bf16* stream, bf16* normed, uint32_t* xp,
                          hipStream_t st) {
  const dim3 grid(hc, S, (H + 255) / 256);
  if (H == 2560)
    hc_norm_mode<10, true>(grid, residual, out, inject, hc, H, tile, scale, eps, stream, normed, xp, st);
  else if (H <= 256 * 16)
    hc_norm_mode<16, false>(grid, residual, out, inject, hc, H, tile, scale, eps, stream, normed, xp, st);
  else
    hc_norm_mode<48, false>(grid, residual, out, inject, hc, H, tile, scale, eps, stream, normed, xp, st);
  return hipGetLastError();
}

hipError_t launch_silu_xprep(const bf16* lo, int S, int LW, bf16* act, uint32_t* xp, hipStream_t st) {
  hipLaunchKernelGGL(k_silu_xprep, dim3(S, (LW + 255) / 256), dim3(256), 0, st, lo, LW, act, xp);
  return hipGetLastError();
}

hipError_t launch_hc_mix(const bf16* w, const bf16* normed, const bf16* inj, int S, int hc, int H, bf16* input,
                         bf16* inject_out, uint32_t* xp, hipStream_t st) {
  hipLaunchKernelGGL(k_hc_mix, dim3(S, (H + 255) / 256), dim3(256), 0, st, w, normed, inj, hc, H, input,
                     inject_out, xp);
  return hipGetLastError();
}

}  // namespace mtpx
