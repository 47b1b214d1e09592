// The PLE n-gram block of the target's layer index 1
// (Runner/FastModel/TrackFastModel.swift:1011-1144, Runner/FastModel/TrackFastPLE.swift):
//
//   k_ple_rows   token history -> n-gram row ids (the hash of
//                docs/ngram-cache-design.md:47-96) -> the table's rows,
//                dequantized, as the embedding row and its prepared blocks
//   (key_proj and value_proj run on the dense q4 GEMV)
//   k_ple_gate   norm_key(key) * norm_query(stream), the bf16 row sum, the
//                gate scalar chain, the gated value and norm_conv
//   k_ple_conv   the dilated depthwise conv over the carried rows and the
//                window, SiLU, the gated add and the stream add
//
// The table stays resident in HBM (100 bytes a row, 32 GB at the model's
// 320M rows): the reference keeps it on disk behind a host row cache because
// its machine cannot hold it next to the weights; one MI355X can, so the
// gather is a device read and the step has no host round trip.
//
// Window state, as the GDN layers keep it: a forward leaves the committed
// state (carried conv rows and token context) alone and writes this window's
// normed rows, token ids, its base rows and base context to the other slot; a
// commit of n positions is applied by the next window, which reads its base
// through the offset P (rows r + P of the previous base ++ previous window).
#include "mtpx_kernels.h"

namespace mtpx {

// ---------------------------------------------------------------------------
// grid (S, E/256), 256 threads: workgroup (s, y) hashes position s (history
// index u = C + s; hist = the last C tokens before the window, then the
// window) and gathers elements 256y .. 256y+255 of its embedding row.
__global__ __launch_bounds__(256) void k_ple_rows(PleRowArgs a) {
  __shared__ int32_t hist[PLE_MAX_CTX + MAX_TOKENS];
  __shared__ int32_t rid[PLE_MAX_HEADS];
  const int s = blockIdx.x, t = threadIdx.x;
  const int C = a.ctx_len, S = a.S;
  const int nh = (a.ngram - 1) * a.hpn;
  if (t < C + S) {
    int32_t v;
    if (t < C) {
      const int q = t + a.P;  // base context after the P committed positions of the previous window
      v = q < C ? a.ctx_cur[q] : a.ids_prev[q - C];
    } else {
      v = a.ids[t - C];
    }
    hist[t] = v;
  }
  __syncthreads();
  if (s == 0 && blockIdx.y == 0) {
    if (a.ctx_nxt && t < C) a.ctx_nxt[t] = hist[t];
    if (a.ids_nxt && t < S) a.ids_nxt[t] = hist[C + t];
  }
  if (t < nh) {
    const int u = C + s;
    const int n = t / a.hpn + 2;  // n-gram width of head t
    const int64_t* mult = a.hash;
    uint64_t mix = 0;
    bool crossed = false;
    for (int p = 0; p < n; ++p) {
      if (p >= 2 && hist[u - p + 1] == a.eos) crossed = true;  // a shift never crosses an eos
      const int64_t cp = crossed ? (int64_t)a.eos : (int64_t)hist[u - p];
      mix ^= (uint64_t)cp * (uint64_t)mult[p];
    }
    const int64_t vocab = a.hash[a.ngram + t], off = a.hash[a.ngram + nh + t];
    const int64_t id = (int64_t)mix % vocab + off;
    const int32_t r = (id >= 0 && id < a.rows) ? (int32_t)id : -1;
    rid[t] = r;
    if (a.row_ids && blockIdx.y == 0) a.row_ids[(size_t)s * nh + t] = r;
  }
  __syncthreads();
  if (!a.emb) return;
  const int E = nh * a.row_dim, wpr = a.row_dim / 8, gpr = a.row_dim / a.rgs;
  {  // E % 256 == 0: the workgroup's 256 elements are whole 32-lane blocks
    const int d = (int)blockIdx.y * 256 + t;
    const int hh = d / a.row_dim, v = d - hh * a.row_dim;
    const int32_t r = rid[hh];
    bf16 o = 0;
    if (r >= 0) {
      const uint32_t w = a.tw[(size_t)r * wpr + v / 8];
      const float q = (float)((w >> (4 * (v % 8))) & 0xfu);
      const float sc = bf2f(a.ts[(size_t)r * gpr + v / a.rgs]);
      const float bi = bf2f(a.tb[(size_t)r * gpr + v / a.rgs]);
      o = f2bf(round_bf(sc * q) + bi);
    }
    a.emb[(size_t)s * E + d] = o;
    if (a.xp) xprep_lanes_direct(o, t & 31, a.xp + ((size_t)s * E + d) / 32 * XP_DW);
  }
}

hipError_t launch_ple_rows(const PleRowArgs& a, hipStream_t st) {
  if (a.S < 1 || a.S > MAX_TOKENS || a.ctx_len < 1 || a.ctx_len > PLE_MAX_CTX || a.ngram < 2 ||
      a.ngram > PLE_MAX_NGRAM || a.hpn < 1 || (a.ngram - 1) * a.hpn > PLE_MAX_HEADS || a.ctx_len < a.ngram - 1)
    return hipErrorInvalidValue;
  if (a.emb && (((a.ngram - 1) * a.hpn * a.row_dim) % 256 != 0 || a.row_dim % a.rgs != 0 || a.row_dim % 8 != 0))
    return hipErrorInvalidValue;
  const int ny = a.emb ? (a.ngram - 1) * a.hpn * a.row_dim / 256 : 1;
  hipLaunchKernelGGL(k_ple_rows, dim3(a.S, ny), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// grid (hc, S), H/4 threads (H % 256 == 0, H <= 4096): thread l owns elements
// 4l..4l+3 of stream c of position s; 32-lane groups (NG = H/128 of them)
// reduce by an xor butterfly, then the NG group values (zero-padded to 32) by
// another.  The row sum of the products is MLX's bf16 reduction: a bf16 chain
// over each thread's four, a bf16-rounded float sum per group, and again over
// the groups (MLX/backend/metal/kernels/reduction/reduce_row.h, 640 threads of
// four at H = 2560).
__device__ __forceinline__ float group32_total(float* part, float v, int l, int NG) {
  v = fold_sum<16>(v);
  if ((l & 31) == 0) part[l >> 5] = v;
  __syncthreads();
  return fold_sum<16>((l & 31) < NG ? part[l & 31] : 0.0f);
}

__global__ __launch_bounds__(1024) void k_ple_gate(const bf16* __restrict__ key, const bf16* __restrict__ stream,
                                                   const bf16* __restrict__ value, const bf16* __restrict__ kscale,
                                                   const bf16* __restrict__ qscale, const bf16* __restrict__ cscale,
                                                   int H, int hc, float eps, bf16* __restrict__ gated,
                                                   bf16* __restrict__ normed) {
  __shared__ float part[4][32];
  const int c = blockIdx.x, s = blockIdx.y, l = threadIdx.x, NG = H / 128;
  const size_t row = ((size_t)s * hc + c) * H + 4 * l;  // [S, hc*H]
  const size_t sc = (size_t)c * H + 4 * l;
  const uint2 kw = *reinterpret_cast<const uint2*>(key + row);
  const uint2 qw = *reinterpret_cast<const uint2*>(stream + row);
  const uint2 vw = *reinterpret_cast<const uint2*>(value + (size_t)s * H + 4 * l);
  const uint2 ksw = *reinterpret_cast<const uint2*>(kscale + sc);
  const uint2 qsw = *reinterpret_cast<const uint2*>(qscale + sc);
  const uint2 csw = *reinterpret_cast<const uint2*>(cscale + sc);
  auto el = [](uint2 w, int i) -> float {
    const uint32_t u = i < 2 ? w.x : w.y;
    return __uint_as_float((i & 1) ? (u & 0xffff0000u) : (u << 16));
  };
  float kx[4], qx[4];
  float ka = 0.0f, qa = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kx[i] = el(kw, i);
    qx[i] = el(qw, i);
    ka = __builtin_fmaf(kx[i], kx[i], ka);
    qa = __builtin_fmaf(qx[i], qx[i], qa);
  }
  const float kt = group32_total(part[0], ka, l, NG);
  const float qt = group32_total(part[1], qa, l, NG);
  const float kinv = 1.0f / sqrtf(kt / (float)H + eps);
  const float qinv = 1.0f / sqrtf(qt / (float)H + eps);
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float kn = round_bf(round_bf(kx[i] * kinv) * el(ksw, i));
    const float qn = round_bf(round_bf(qx[i] * qinv) * el(qsw, i));
    t = round_bf(round_bf(kn * qn) + t);
  }
  float tg = round_bf(fold_sum<16>(t));
  if ((l & 31) == 0) part[2][l >> 5] = tg;
  __syncthreads();
  const float dot = round_bf(fold_sum<16>((l & 31) < NG ? part[2][l & 31] : 0.0f));
  // the gate scalar, one bf16 rounding per MLX op
  const float divisor = round_bf(sqrtf((float)H));
  const float floor_v = round_bf(1e-6f);
  float g = round_bf(dot / divisor);
  const float ag = fabsf(g);
  const float mx = __builtin_isnan(ag) ? ag : (ag > floor_v ? ag : floor_v);
  const float sg = (float)((g > 0.0f) - (g < 0.0f));
  g = round_bf(round_bf(sqrtf(mx)) * sg);
  const float sgm = sigmoid_bf16(g);
  float v[4], va = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = round_bf(sgm * el(vw, i));
    va = __builtin_fmaf(v[i], v[i], va);
  }
  const float vt = group32_total(part[3], va, l, NG);
  const float vinv = 1.0f / sqrtf(vt / (float)H + eps);
  uint2 go, no;
  go.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
  go.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
  uint16_t nb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) nb[i] = f2bf(round_bf(v[i] * vinv) * el(csw, i));
  no.x = (uint32_t)nb[0] | ((uint32_t)nb[1] << 16);
  no.y = (uint32_t)nb[2] | ((uint32_t)nb[3] << 16);
  *reinterpret_cast<uint2*>(gated + row) = go;
  *reinterpret_cast<uint2*>(normed + row) = no;
}

hipError_t launch_ple_gate(const bf16* key, const bf16* stream, const bf16* value, const bf16* kscale,
                           const bf16* qscale, const bf16* cscale, int S, int hc, int H, float eps, bf16* gated,
                           bf16* normed, hipStream_t st) {
  if (H % 256 != 0 || H > 4096 || S < 1 || hc < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ple_gate, dim3(hc, S), dim3(H / 4), 0, st, key, stream, value, kscale, qscale, cscale, H, hc,
                     eps, gated, normed);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// grid (ceil(W/256), S), 256 threads: channel c of position s.  Row r of the
// conv input: r < nb the base rows (row r + P of the previous base ++ the
// previous window's normed rows), then this window's normed rows.
__global__ __launch_bounds__(256) void k_ple_conv(PleConvArgs a) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int s = blockIdx.y;
  if (c >= a.W) return;
  const int nb = (a.kc - 1) * a.dil;
  auto base = [&](int r) -> bf16 {
    const int q = r + a.P;
    return q < nb ? a.conv_cur[(size_t)q * a.W + c] : a.win_cur[(size_t)(q - nb) * a.W + c];
  };
  float acc = 0.0f;
  for (int j = 0; j < a.kc; ++j) {
    const int r = s + j * a.dil;
    const bf16 x = r < nb ? base(r) : a.win_nxt[(size_t)(r - nb) * a.W + c];
    acc = acc + bf2f(x) * bf2f(a.conv_w[(size_t)c * a.kc + j]);
  }
  const size_t o = (size_t)s * a.W + c;
  const bf16 y = f2bf(bf2f(a.gated[o]) + silu_bf16(round_bf(acc)));
  if (a.out) a.out[o] = y;
  if (a.sum) a.sum[o] = f2bf(bf2f(a.stream[o]) + bf2f(y));
  if (s == 0 && a.conv_nxt)
    for (int r = 0; r < nb; ++r) a.conv_nxt[(size_t)r * a.W + c] = base(r);
}

hipError_t launch_ple_conv(const PleConvArgs& a, hipStream_t st) {
  if (a.S < 1 || a.S > MAX_TOKENS || a.kc < 1 || a.dil < 1 || a.W < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ple_conv, dim3((unsigned)((a.W + 255) / 256), a.S), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace mtpx
