// Speculative acceptance, decided on the device.
//   greedy : argmax of each verify row (lowest id on ties), longest prefix of
//            drafts equal to the row argmaxes, bonus token, KV rollback index
//   sample : temperature rejection sampling (Leviathan et al. 2023) with a
//            Philox4x32-10 stream; probabilities and sums in a fixed order
// Reference: accept/rollback semantics docs/qwen38-125b-a6b-port-notes.md:313-343,
// tie rule Runner/Qwen4ExpMTPDrafter.swift:25-27.  Sampling has no reference
// counterpart (the reference is greedy only).
#include "mtpx_kernels.h"

namespace mtpx {

constexpr int AM_SPAN = 2048;  // elements per argmax partial (8 per thread, loaded together)

struct VI {
  float v;
  int i;
};

// Values enter as no_nan(x): a NaN ranks as -inf, as in MLX's argmax, which only ever takes a
// value strictly greater than its best so far, starting from (index 0, -inf)
// (MLX/backend/metal/kernels/arg_reduce.metal:42-62): a NaN never wins, and a row whose numbers
// are all -inf or NaN gives index 0, the lowest index among equal values.
__device__ __forceinline__ float no_nan(float x) { return x != x ? -__uint_as_float(0x7f800000u) : x; }

__device__ __forceinline__ VI vi_best(VI a, VI b) {
  // larger value; lower index on equal values
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}

template <int OFF>
__device__ __forceinline__ VI vi_xor(VI x) {
  VI o;
  o.v = lane_xor_f<OFF>(x.v);
  o.i = lane_xor_i<OFF>(x.i);
  return vi_best(x, o);
}

__device__ __forceinline__ VI wave_best(VI x) {
  x = vi_xor<32>(x);
  x = vi_xor<16>(x);
  x = vi_xor<8>(x);
  x = vi_xor<4>(x);
  x = vi_xor<2>(x);
  return vi_xor<1>(x);
}

__device__ __forceinline__ float ld_val(const float* p) { return *p; }
__device__ __forceinline__ float ld_val(const bf16* p) { return bf2f(*p); }

// grid (parts, rows): best (value, index) of each AM_SPAN slice of a row.
template <typename T>
__global__ __launch_bounds__(256) void k_argmax_part(const T* __restrict__ x, int64_t V, int parts,
                                                     float* __restrict__ pval, int32_t* __restrict__ pidx) {
  __shared__ VI wb[4];
  const int part = blockIdx.x, row = blockIdx.y;
  const T* xr = x + (size_t)row * V;
  const int64_t b = (int64_t)part * AM_SPAN;
  const int64_t e = b + AM_SPAN < V ? b + AM_SPAN : V;
  constexpr int PER = AM_SPAN / 256;
  float v[PER];  // every load issued before the first comparison (past the end: the slice's first element again)
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int64_t i = b + threadIdx.x + 256 * u;
    v[u] = no_nan(ld_val(xr + (i < e ? i : b)));
  }
  VI best{-__uint_as_float(0x7f800000u), 0x7fffffff};
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int64_t i = b + threadIdx.x + 256 * u;
    if (i < e) best = vi_best(best, VI{v[u], (int)i});
  }
  best = wave_best(best);
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    VI r = wb[0];
    for (int w = 1; w < 4; ++w) r = vi_best(r, wb[w]);
    pval[(size_t)row * parts + part] = r.v;
    pidx[(size_t)row * parts + part] = r.i;
  }
}

__device__ VI reduce_parts(const float* pval, const int32_t* pidx, int parts, int row, int lane) {
  VI best{-__uint_as_float(0x7f800000u), 0x7fffffff};
  for (int p = lane; p < parts; p += 64) best = vi_best(best, VI{pval[(size_t)row * parts + p], pidx[(size_t)row * parts + p]});
  return wave_best(best);
}

// one wave per row; with ids the winning position is mapped through them.  Every row has
// V >= 1 elements, each ranked above the partials' initial index, so b.i < V; the clamp
// only keeps the id lookup in bounds by construction.
__global__ void k_argmax_final(const float* __restrict__ pval, const int32_t* __restrict__ pidx, int rows,
                               int parts, int64_t V, const int32_t* __restrict__ ids, int32_t* __restrict__ out) {
  const int row = blockIdx.x;
  const VI b = reduce_parts(pval, pidx, parts, row, threadIdx.x);
  const int i = b.i >= 0 && b.i < V ? b.i : 0;
  if (threadIdx.x == 0) out[row] = ids ? ids[i] : i;
}

// ---------------------------------------------------------------------------
// top two per row (the argmax order: value desc, lowest index on ties, NaN as -inf)
struct VI2 {
  VI a, b;  // a ranks before b
};

__device__ __forceinline__ VI2 vi2_merge(VI2 x, VI2 y) {
  // the better of the two leaders first; second = the better of the loser and the winner's runner-up
  const VI top = vi_best(x.a, y.a);
  const bool xa = top.i == x.a.i && top.v == x.a.v;
  const VI second = xa ? vi_best(x.b, y.a) : vi_best(x.a, y.b);
  return VI2{top, second};
}

template <int OFF>
__device__ __forceinline__ VI2 vi2_xor(VI2 x) {
  VI2 o;
  o.a.v = lane_xor_f<OFF>(x.a.v);
  o.a.i = lane_xor_i<OFF>(x.a.i);
  o.b.v = lane_xor_f<OFF>(x.b.v);
  o.b.i = lane_xor_i<OFF>(x.b.i);
  return vi2_merge(x, o);
}

__device__ __forceinline__ VI2 wave_best2(VI2 x) {
  x = vi2_xor<32>(x);
  x = vi2_xor<16>(x);
  x = vi2_xor<8>(x);
  x = vi2_xor<4>(x);
  x = vi2_xor<2>(x);
  return vi2_xor<1>(x);
}

// grid (parts, rows): the best two (value, index) pairs of each AM_SPAN slice -> p2 [rows][parts][4]
// as (v1, i1, v2, i2) words
template <typename T>
__global__ __launch_bounds__(256) void k_top2_part(const T* __restrict__ x, int64_t V, int parts,
                                                   float* __restrict__ p2) {
  __shared__ VI2 wb[4];
  const int part = blockIdx.x, row = blockIdx.y;
  const T* xr = x + (size_t)row * V;
  const int64_t b = (int64_t)part * AM_SPAN;
  const int64_t e = b + AM_SPAN < V ? b + AM_SPAN : V;
  constexpr int PER = AM_SPAN / 256;
  float v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int64_t i = b + threadIdx.x + 256 * u;
    v[u] = no_nan(ld_val(xr + (i < e ? i : b)));
  }
  const VI none{-__uint_as_float(0x7f800000u), 0x7fffffff};
  VI2 best{none, none};
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int64_t i = b + threadIdx.x + 256 * u;
    if (i < e) best = vi2_merge(best, VI2{VI{v[u], (int)i}, none});
  }
  best = wave_best2(best);
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    VI2 r = wb[0];
    for (int w = 1; w < 4; ++w) r = vi2_merge(r, wb[w]);
    float* o = p2 + ((size_t)row * parts + part) * 4;
    o[0] = r.a.v;
    o[1] = __int_as_float(r.a.i);
    o[2] = r.b.v;
    o[3] = __int_as_float(r.b.i);
  }
}

// one wave per row: ids [rows, 2], values [rows, 2]
__global__ void k_top2_final(const float* __restrict__ p2, int parts, int32_t* __restrict__ ids,
                             float* __restrict__ vals) {
  const int row = blockIdx.x, lane = threadIdx.x;
  const VI none{-__uint_as_float(0x7f800000u), 0x7fffffff};
  VI2 best{none, none};
  for (int p = lane; p < parts; p += 64) {
    const float* o = p2 + ((size_t)row * parts + p) * 4;
    best = vi2_merge(best, VI2{VI{o[0], __float_as_int(o[1])}, VI{o[2], __float_as_int(o[3])}});
  }
  best = wave_best2(best);
  if (lane == 0) {
    ids[2 * row] = best.a.i;
    ids[2 * row + 1] = best.b.i;
    vals[2 * row] = best.a.v;
    vals[2 * row + 1] = best.b.v;
  }
}

// one workgroup: wave r reduces row r, then thread 0 decides.  Optional outputs: amax [k+1]
// (every row's argmax) and tokens [k+1] (the committed tokens: drafts[0..n-1], then the bonus).
__global__ __launch_bounds__(512) void k_accept_greedy(const float* __restrict__ pval,
                                                       const int32_t* __restrict__ pidx, int k, int parts,
                                                       const int32_t* __restrict__ drafts, int32_t kv_offset,
                                                       int32_t* __restrict__ out3, int32_t* __restrict__ amax,
                                                       int32_t* __restrict__ tokens) {
  __shared__ int am[MAX_TOKENS];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave <= k) {
    const VI b = reduce_parts(pval, pidx, parts, wave, lane);
    if (lane == 0) {
      am[wave] = b.i;
      if (amax) amax[wave] = b.i;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int n = 0;
    while (n < k && drafts[n] == am[n]) ++n;
    out3[0] = n;
    out3[1] = am[n];
    out3[2] = kv_offset + n + 1;
    if (tokens) {
      for (int i = 0; i < n; ++i) tokens[i] = drafts[i];
      tokens[n] = am[n];
    }
  }
}

// ---------------------------------------------------------------------------
// sampling
constexpr int S_CHUNK = 1024;

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
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

__device__ __forceinline__ float uniform24(uint32_t r) { return (float)(r >> 8) * 5.9604644775390625e-08f; }

// The forcing hook of a benchmark drafter (a test hook, not part of the decode rule): with
// probability p, decided by Philox4x32-10 with key = seed and counter = {pos lo, pos hi,
// 0x46524345, 0} (so the decision is a property of the position), *token = teacher[pos].
__global__ void k_force_draft(int32_t* __restrict__ token, const int32_t* __restrict__ teacher, int64_t pos,
                              float p, uint64_t seed) {
  if (threadIdx.x != 0) return;
  const uint4 r = philox4x32_10(make_uint4((uint32_t)pos, (uint32_t)((uint64_t)pos >> 32), 0x46524345u, 0u),
                                make_uint2((uint32_t)seed, (uint32_t)(seed >> 32)));
  if (uniform24(r.x) < p) *token = teacher[pos];
}

// Work layout (floats): rowmax[2k+1], invZ[2k+1], state[8], csum[(2k+1)*nch], vsum[nch]
// rows 0..k: verify rows (tlogits); rows k+1..2k: draft rows (dlogits).  With no draft rows
// (d == null) the draft distribution of row i is one-hot at drafts[i] (a greedy drafter): the
// draft is accepted with probability p_t(d), a rejection samples max(0, p_t - onehot(d)).
struct SampleWork {
  float* rowmax;
  float* invz;
  float* state;  // [0] mode (0 residual, 1 bonus), [1] row, [2] u2, [3] n
  float* csum;
  float* vsum;
};

template <typename T>
__device__ __forceinline__ const T* srow(const T* t, const T* d, int k, int64_t V, int r) {
  return r <= k ? t + (size_t)r * V : d + (size_t)(r - k - 1) * V;
}

// one wave per row: row max from the argmax partials
__global__ void k_sample_rowmax(const float* __restrict__ pval, const int32_t* __restrict__ pidx, int parts,
                                float* __restrict__ rowmax) {
  const VI b = reduce_parts(pval, pidx, parts, blockIdx.x, threadIdx.x);
  if (threadIdx.x == 0) rowmax[blockIdx.x] = b.v;
}

// grid (nch, rows), one wave: chunk sum of exp((l - max) * invT), lane-strided
// (lane l adds base+l, base+l+64, ...) then an xor butterfly.
template <typename T>
__global__ void k_sample_chunks(const T* __restrict__ t, const T* __restrict__ d, int k, int64_t V, float invT,
                                const float* __restrict__ rowmax, int nch, float* __restrict__ csum) {
  const int c = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
  const T* x = srow(t, d, k, V, r);
  const float mx = rowmax[r];
  float acc = 0.0f;
  for (int j = 0; j < S_CHUNK / 64; ++j) {
    const int64_t i = (int64_t)c * S_CHUNK + lane + 64 * j;
    if (i < V) acc = acc + expf_det((ld_val(x + i) - mx) * invT);
  }
  acc = wave_fold64(acc);
  if (lane == 0) csum[(size_t)r * nch + c] = acc;
}

template <typename T>
__device__ __forceinline__ float prob(const T* x, int64_t v, float mx, float invT, float invz) {
  return expf_det((ld_val(x + v) - mx) * invT) * invz;
}

// single thread: Z per row, then the accept/reject walk
template <typename T>
__global__ void k_sample_decide(const T* __restrict__ t, const T* __restrict__ d, int k, int64_t V,
                                const int32_t* __restrict__ drafts, float invT, uint64_t seed, uint64_t offset,
                                int nch, SampleWork w, int32_t* __restrict__ out3, int32_t kv_offset) {
  if (threadIdx.x != 0) return;
  const int rows = d ? 2 * k + 1 : k + 1;
  for (int r = 0; r < rows; ++r) {
    float z = 0.0f;
    for (int c = 0; c < nch; ++c) z = z + w.csum[(size_t)r * nch + c];
    w.invz[r] = 1.0f / z;
  }
  const uint2 key = make_uint2((uint32_t)seed, (uint32_t)(seed >> 32));
  for (int i = 1; i <= k + 1; ++i) {
    const uint4 rnd = philox4x32_10(make_uint4((uint32_t)offset, (uint32_t)(offset >> 32), (uint32_t)i, 0u), key);
    const float u = uniform24(rnd.x), u2 = uniform24(rnd.y);
    if (i == k + 1) {
      w.state[0] = 1.0f;
      w.state[1] = (float)k;
      w.state[2] = u2;
      w.state[3] = (float)k;
      out3[0] = k;
      out3[2] = kv_offset + k + 1;
      return;
    }
    const int dt = drafts[i - 1];
    const T* tr = srow(t, d, k, V, i - 1);
    // a draft id outside the vocabulary is rejected
    const bool ok = dt >= 0 && dt < V;
    const float pt = ok ? prob(tr, dt, w.rowmax[i - 1], invT, w.invz[i - 1]) : 0.0f;
    const float pd = ok && d ? prob(srow(t, d, k, V, k + i), dt, w.rowmax[k + i], invT, w.invz[k + i]) : 1.0f;
    if (u * pd < pt) continue;
    w.state[0] = 0.0f;
    w.state[1] = (float)(i - 1);
    w.state[2] = u2;
    w.state[3] = (float)(i - 1);
    out3[0] = i - 1;
    out3[2] = kv_offset + i;
    return;
  }
}

template <typename T>
__device__ __forceinline__ float sample_val(const T* t, const T* d, const int32_t* drafts, int k, int64_t V,
                                            const SampleWork& w, float invT, int64_t v) {
  const int row = (int)w.state[1];
  const float pt = prob(srow(t, d, k, V, row), v, w.rowmax[row], invT, w.invz[row]);
  if (w.state[0] != 0.0f) return pt;
  const float pd = d ? prob(srow(t, d, k, V, k + 1 + row), v, w.rowmax[k + 1 + row], invT, w.invz[k + 1 + row])
                     : (v == drafts[row] ? 1.0f : 0.0f);
  return fmaxf(pt - pd, 0.0f);
}

// grid (nch), one wave: chunk sums of the residual (or bonus) distribution
template <typename T>
__global__ void k_sample_vchunks(const T* __restrict__ t, const T* __restrict__ d, const int32_t* __restrict__ drafts,
                                 int k, int64_t V, float invT, SampleWork w) {
  const int c = blockIdx.x, lane = threadIdx.x;
  float acc = 0.0f;
  for (int j = 0; j < S_CHUNK / 64; ++j) {
    const int64_t i = (int64_t)c * S_CHUNK + lane + 64 * j;
    if (i < V) acc = acc + sample_val(t, d, drafts, k, V, w, invT, i);
  }
  acc = wave_fold64(acc);
  if (lane == 0) w.vsum[c] = acc;
}

// single thread: inverse CDF over the chunk sums, then inside the chunk.  Optional tokens [k+1]:
// the committed tokens (drafts[0..n-1], then the sampled token).
template <typename T>
__global__ void k_sample_icdf(const T* __restrict__ t, const T* __restrict__ d, const int32_t* __restrict__ drafts,
                              int k, int64_t V, float invT, int nch, SampleWork w, const float* __restrict__ pval,
                              const int32_t* __restrict__ pidx, int parts, int32_t* __restrict__ out3,
                              int32_t* __restrict__ tokens) {
  if (threadIdx.x != 0) return;
  float total = 0.0f;
  for (int c = 0; c < nch; ++c) total = total + w.vsum[c];
  const float tau = w.state[2] * total;
  float cum = 0.0f;
  int64_t res = -1;
  for (int c = 0; c < nch && res < 0; ++c) {
    const float nxt = cum + w.vsum[c];
    if (nxt > tau) {
      const float t2 = tau - cum;
      float run = 0.0f;
      const int64_t b = (int64_t)c * S_CHUNK;
      const int64_t e = b + S_CHUNK < V ? b + S_CHUNK : V;
      for (int64_t i = b; i < e; ++i) {
        run = run + sample_val(t, d, drafts, k, V, w, invT, i);
        if (run > t2) {
          res = i;
          break;
        }
      }
      if (res < 0)
        for (int64_t i = e - 1; i >= b; --i)
          if (sample_val(t, d, drafts, k, V, w, invT, i) > 0.0f) {
            res = i;
            break;
          }
    }
    cum = nxt;
  }
  if (res < 0)
    for (int64_t i = V - 1; i >= 0; --i)
      if (sample_val(t, d, drafts, k, V, w, invT, i) > 0.0f) {
        res = i;
        break;
      }
  if (res < 0) {
    // every entry zero: the target row's argmax (lowest id on ties)
    const int row = (int)w.state[1];
    VI best{-__uint_as_float(0x7f800000u), 0x7fffffff};
    for (int p = 0; p < parts; ++p) best = vi_best(best, VI{pval[(size_t)row * parts + p], pidx[(size_t)row * parts + p]});
    res = best.i;
  }
  out3[1] = (int32_t)res;
  if (tokens) {
    const int n = (int)w.state[3];
    for (int i = 0; i < n; ++i) tokens[i] = drafts[i];
    tokens[n] = (int32_t)res;
  }
}

// ---------------------------------------------------------------------------
size_t argmax_work_items(int rows, int64_t V) { return (size_t)rows * ((V + AM_SPAN - 1) / AM_SPAN); }

hipError_t launch_argmax_rows(const float* x, int rows, int64_t V, float* pval, int32_t* pidx, int32_t* out,
                              hipStream_t st) {
  const int parts = (int)((V + AM_SPAN - 1) / AM_SPAN);
  hipLaunchKernelGGL(k_argmax_part<float>, dim3(parts, rows), dim3(256), 0, st, x, V, parts, pval, pidx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(64), 0, st, pval, pidx, rows, parts, V, nullptr, out);
  return hipGetLastError();
}

hipError_t launch_argmax_rows_bf16(const bf16* x, int rows, int64_t V, float* pval, int32_t* pidx,
                                   const int32_t* ids, int32_t* out, hipStream_t st) {
  const int parts = (int)((V + AM_SPAN - 1) / AM_SPAN);
  hipLaunchKernelGGL(k_argmax_part<bf16>, dim3(parts, rows), dim3(256), 0, st, x, V, parts, pval, pidx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(64), 0, st, pval, pidx, rows, parts, V, ids, out);
  return hipGetLastError();
}

template <typename T>
hipError_t top2_t(const T* x, int rows, int64_t V, float* p2, int32_t* ids, float* vals, hipStream_t st) {
  const int parts = (int)((V + AM_SPAN - 1) / AM_SPAN);
  hipLaunchKernelGGL(k_top2_part<T>, dim3(parts, rows), dim3(256), 0, st, x, V, parts, p2);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_top2_final, dim3(rows), dim3(64), 0, st, p2, parts, ids, vals);
  return hipGetLastError();
}

hipError_t launch_top2(const float* x, const bf16* xb, int rows, int64_t V, float* p2, int32_t* ids, float* vals,
                       hipStream_t st) {
  return x ? top2_t(x, rows, V, p2, ids, vals, st) : top2_t(xb, rows, V, p2, ids, vals, st);
}

template <typename T>
hipError_t accept_greedy_t(const T* logits, int k, int64_t V, const int32_t* drafts, int32_t kv_offset, float* pval,
                           int32_t* pidx, int32_t* out3, int32_t* amax, int32_t* tokens, hipStream_t st) {
  const int parts = (int)((V + AM_SPAN - 1) / AM_SPAN);
  hipLaunchKernelGGL(k_argmax_part<T>, dim3(parts, k + 1), dim3(256), 0, st, logits, V, parts, pval, pidx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_accept_greedy, dim3(1), dim3(64 * (k + 1)), 0, st, pval, pidx, k, parts, drafts, kv_offset,
                     out3, amax, tokens);
  return hipGetLastError();
}

hipError_t launch_accept_greedy(const float* logits, int k, int64_t V, const int32_t* drafts, int32_t kv_offset,
                                float* pval, int32_t* pidx, int32_t* out3, hipStream_t st) {
  return accept_greedy_t(logits, k, V, drafts, kv_offset, pval, pidx, out3, nullptr, nullptr, st);
}

hipError_t launch_accept_greedy_bf16(const bf16* logits, int k, int64_t V, const int32_t* drafts, int32_t kv_offset,
                                     float* pval, int32_t* pidx, int32_t* out3, int32_t* amax, int32_t* tokens,
                                     hipStream_t st) {
  return accept_greedy_t(logits, k, V, drafts, kv_offset, pval, pidx, out3, amax, tokens, st);
}

hipError_t launch_force_draft(int32_t* token, const int32_t* teacher, int64_t pos, float p, uint64_t seed,
                              hipStream_t st) {
  hipLaunchKernelGGL(k_force_draft, dim3(1), dim3(64), 0, st, token, teacher, pos, p, seed);
  return hipGetLastError();
}

size_t accept_sample_work_floats(int k, int64_t V) {
  const int64_t nch = (V + S_CHUNK - 1) / S_CHUNK;
  const int rows = 2 * k + 1;
  const size_t parts = (size_t)((V + AM_SPAN - 1) / AM_SPAN);
  return (size_t)rows * 2 + 8 + (size_t)rows * nch + nch + 2 * rows * parts;
}

template <typename T>
hipError_t accept_sample_t(const T* tlogits, const T* dlogits, int k, int64_t V, const int32_t* drafts,
                           float temperature, uint64_t seed, uint64_t offset, int32_t kv_offset, float* work,
                           int32_t* out3, int32_t* tokens, hipStream_t st) {
  const int rows = dlogits ? 2 * k + 1 : k + 1;
  const int nch = (int)((V + S_CHUNK - 1) / S_CHUNK);
  const int parts = (int)((V + AM_SPAN - 1) / AM_SPAN);
  SampleWork w;
  w.rowmax = work;
  w.invz = work + (2 * k + 1);
  w.state = work + 2 * (2 * k + 1);
  w.csum = w.state + 8;
  w.vsum = w.csum + (size_t)(2 * k + 1) * nch;
  float* pval = w.vsum + nch;
  int32_t* pidx = reinterpret_cast<int32_t*>(pval + (size_t)(2 * k + 1) * parts);
  const float invT = 1.0f / temperature;
  hipError_t e;
  // row maxima: verify rows then draft rows (two launches over the two arrays)
  hipLaunchKernelGGL(k_argmax_part<T>, dim3(parts, k + 1), dim3(256), 0, st, tlogits, V, parts, pval, pidx);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (k > 0 && dlogits) {
    hipLaunchKernelGGL(k_argmax_part<T>, dim3(parts, k), dim3(256), 0, st, dlogits, V, parts,
                       pval + (size_t)(k + 1) * parts, pidx + (size_t)(k + 1) * parts);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_sample_rowmax, dim3(rows), dim3(64), 0, st, pval, pidx, parts, w.rowmax);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(k_sample_chunks<T>, dim3(nch, rows), dim3(64), 0, st, tlogits, dlogits, k, V, invT, w.rowmax,
                     nch, w.csum);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(k_sample_decide<T>, dim3(1), dim3(64), 0, st, tlogits, dlogits, k, V, drafts, invT, seed, offset,
                     nch, w, out3, kv_offset);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(k_sample_vchunks<T>, dim3(nch), dim3(64), 0, st, tlogits, dlogits, drafts, k, V, invT, w);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(k_sample_icdf<T>, dim3(1), dim3(64), 0, st, tlogits, dlogits, drafts, k, V, invT, nch, w, pval,
                     pidx, parts, out3, tokens);
  return hipGetLastError();
}

hipError_t launch_accept_sample(const float* tlogits, const float* dlogits, int k, int64_t V, const int32_t* drafts,
                                float temperature, uint64_t seed, uint64_t offset, int32_t kv_offset, float* work,
                                int32_t* out3, hipStream_t st) {
  return accept_sample_t(tlogits, dlogits, k, V, drafts, temperature, seed, offset, kv_offset, work, out3, nullptr,
                         st);
}

hipError_t launch_accept_sample_bf16(const bf16* tlogits, const bf16* dlogits, int k, int64_t V,
                                     const int32_t* drafts, float temperature, uint64_t seed, uint64_t offset,
                                     int32_t kv_offset, float* work, int32_t* out3, int32_t* tokens, hipStream_t st) {
  return accept_sample_t(tlogits, dlogits, k, V, drafts, temperature, seed, offset, kv_offset, work, out3, tokens, st);
}

}  // namespace mtpx
