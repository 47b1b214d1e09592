// Gated-deltanet (GDN) sublayer core of the target's linear-attention layers
// for a window of S <= 8 positions: causal depthwise conv + SiLU, q/k RMS
// norms and scales, decay/beta gates, the delta-rule recurrence with a
// Kahan-compensated key product, and the gated output RMS norm -- one launch,
// four workgroups per value head (each owns a quarter of the head's state
// rows; the head's last one to finish, by a ticket, runs the gated norm over
// the rows' outputs the others published at device scope).
//
// Window state.  The reference keeps the recurrent state after every window
// position so the engine can roll back to any of them (Runner/FastModel/
// TrackFastModel.swift:726-731, stageCaptured).  Here a window writes a
// journal instead -- its conv input rows, the normalised keys, and per
// (head, value row) the delta and per head the decay of every position, about
// 50 KB per position against 3.1 MB of state -- and leaves the committed state
// alone.  Committing n positions only records n; the next window first replays
// those n steps (the same float operations, so the same bits) onto the
// committed state and stores it, then runs its own positions.  Journal and conv
// base are double-buffered (slot `cur` read, slot `nxt` written) so no
// workgroup overwrites what another still reads; each recurrent state row is
// read and written by the one workgroup that owns it.
//
// Lane structure (fixes the float order): every 128-element reduction is 32
// lanes x 4 consecutive elements, each lane in element order, then an xor
// butterfly over the 32 lanes (half a wave).
// Reference: FM/TrackFastKernels.swift:48-117 (prep), :486-605 (recurrence,
// peeled Kahan form), FM/TrackFastKernels2.swift:325-352 (gated RMS),
// FM/TrackFastGDNDecode.swift:50-274 (the fused decode form this follows),
// FM/TrackFastKernels2.swift:48-58 (logaddexp).
#include "mtpx_kernels.h"

namespace mtpx {

constexpr int GDN_THREADS = 512;  // 16 half-waves
constexpr int GDN_D = 128;
constexpr int GDN_SPLIT = 4;      // workgroups per value head, each owning 128 / GDN_SPLIT state rows
constexpr int GDN_BSPLIT = 8;     // the batch kernel's workgroups per value head (a long recurrence: more, shorter chains)

// log1p(y), y in [0, 1]: 2 atanh(s), s = y / (2 + y), odd series to s^15.
__device__ __forceinline__ float log1p_det(float y) {
  if (y != y) return y;
  const float t = 2.0f + y;
  const float s = y / t;
  const float s2 = s * s;
  float r = 1.0f / 15.0f;
  r = 1.0f / 13.0f + s2 * r;
  r = 1.0f / 11.0f + s2 * r;
  r = 1.0f / 9.0f + s2 * r;
  r = 1.0f / 7.0f + s2 * r;
  r = 1.0f / 5.0f + s2 * r;
  r = 1.0f / 3.0f + s2 * r;
  r = s2 * r;
  const float h = s + s * r;
  return h + h;
}

// MLX logaddexp(x, 0) in bf16 arithmetic.
__device__ __forceinline__ float logaddexp0_bf16(float x) {
  if (x != x) return x;
  const float inf = __uint_as_float(0x7f800000u);
  const float mx = x > 0.0f ? x : 0.0f;
  const float mn = x < 0.0f ? x : 0.0f;
  if (mn == -inf || mx == inf) return mx;
  const float d = round_bf(mn - mx);
  const float e = round_bf(expf_det(d));
  const float l = round_bf(log1p_det(e));
  return round_bf(mx + l);
}

// MLX Sigmoid in f32.
__device__ __forceinline__ float sigmoid_f32(float x) {
  const float e = expf_det(__builtin_fabsf(x));
  const float y = 1.0f / (1.0f + e);
  return (x < 0.0f) ? y : 1.0f - y;
}

__device__ __forceinline__ float half_wave_sum(float v) {
  return fold_sum<16>(v);
}

// Element c of four bf16 packed in two words (little-endian), as a float.
__device__ __forceinline__ float kjournal(uint2 w, int c) {
  const uint32_t v = c < 2 ? w.x : w.y;
  return __uint_as_float((c & 1) ? (v & 0xffff0000u) : (v << 16));
}

// Row r of the virtual input sequence conv_cur (KC-1 rows) ++ the P committed
// journal rows ++ the window's projection rows.
__device__ __forceinline__ float gdn_row(const GdnArgs& a, int r, int ch) {
  const int KM1 = a.kc - 1;
  if (r < KM1) return bf2f(a.conv_cur[(size_t)r * a.cd + ch]);
  r -= KM1;
  if (r < a.P) return bf2f(a.win_cur[(size_t)r * a.cd + ch]);
  r -= a.P;
  return bf2f(a.proj[(size_t)r * a.pw + ch]);
}

// Row r of the same virtual sequence as a pointer to its channel 0 (r is uniform).
__device__ __forceinline__ const bf16* gdn_row_ptr(const GdnArgs& a, int r) {
  const int KM1 = a.kc - 1;
  if (r < KM1) return a.conv_cur + (size_t)r * a.cd;
  r -= KM1;
  if (r < a.P) return a.win_cur + (size_t)r * a.cd;
  return a.proj + (size_t)(r - a.P) * a.pw;
}

// JP: journal steps the launch can replay (P <= JP), so the replay's loads issued up front are its
// own, not clamped duplicates up to MAX_TOKENS ahead of the prep's loads.
template <int KC, int JP>
__global__ __launch_bounds__(GDN_THREADS) void k_gdn_step(GdnArgs a) {
  static_assert(JP >= 1 && JP <= MAX_TOKENS, "journal steps");
  __shared__ float qs[MAX_TOKENS][GDN_D], ks[MAX_TOKENS][GDN_D], vs[MAX_TOKENS][GDN_D], ys[MAX_TOKENS][GDN_D];
  __shared__ float dec[MAX_TOKENS], bet[MAX_TOKENS];
  __shared__ bf16 gated[MAX_TOKENS][GDN_D];
  const int h = blockIdx.x, ratio = a.hv / a.hk, hk = h / ratio;
  const int r0 = blockIdx.y * (GDN_D / GDN_SPLIT);  // this workgroup's state rows r0 .. r0 + 128/GDN_SPLIT - 1
  const bool w0 = blockIdx.y == 0;                  // writes the head's journal rows (conv, keys, decay)
  const bool lead = (h % ratio) == 0 && w0;         // writes the q/k channels' journal and conv rows
  const int hw = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int S = a.S, P = a.P, KM1 = a.kc - 1;
  const float inv_scale = 1.0f / sqrtf((float)GDN_D);
  const float q_mul = round_bf(inv_scale * inv_scale), k_mul = round_bf(inv_scale);

  // The state rows of this half-wave's recurrence (r = r0 + hw + 16 i) and the journal steps it replays,
  // loaded before the prep so their latency hides behind it.
  constexpr int RPH = GDN_D / GDN_SPLIT / (GDN_THREADS / 32);
  float s[RPH][4];
#pragma unroll
  for (int i = 0; i < RPH; ++i) {
    const float4 s4 = *reinterpret_cast<const float4*>(a.ssm + ((size_t)h * GDN_D + r0 + hw + 16 * i) * GDN_D + 4 * l);
    s[i][0] = s4.x;
    s[i][1] = s4.y;
    s[i][2] = s4.z;
    s[i][3] = s4.w;
  }
  float gdp[JP], dlp[JP][RPH];
  uint2 kpw[JP];  // the journal keys' four bf16 (raw until the replay, so no wait for them here)
  if (P > 0) {
#pragma unroll
    for (int p = 0; p < JP; ++p) {
      const int pc = p < P ? p : P - 1;  // clamped: loads beyond P are issued but not used
      gdp[p] = a.decay_cur[(size_t)pc * a.hv + h];
      kpw[p] = *reinterpret_cast<const uint2*>(a.key_cur + ((size_t)pc * a.hk + hk) * GDN_D + 4 * l);
#pragma unroll
      for (int i = 0; i < RPH; ++i) dlp[p][i] = a.delta_cur[((size_t)pc * a.hv + h) * GDN_D + r0 + hw + 16 * i];
    }
  }

  // The inputs of the prep's last steps, loaded now so their latency hides behind the loads above
  // and the conv's: the positions' gate inputs (position t: thread GDN_THREADS - S + t, the last
  // wave, which has no conv task up to five positions) and, in a head's first workgroup, the conv
  // rows R[P .. P+KC-1) that become the next window's base (element i = (j, kind, d)).
  // (every thread loads, position 0 outside the gate threads, no branch; raw bf16 bits until the
  // use, so nothing waits for them here)
  const int gt = (int)threadIdx.x - (GDN_THREADS - S);  // this thread's gate position, or < 0
  const uint16_t* prow = reinterpret_cast<const uint16_t*>(a.proj) + (size_t)(gt >= 0 ? gt : 0) * a.pw;
  const uint32_t g_b = prow[a.b_off + h], g_a = prow[a.a_off + h];
  const uint32_t g_dt = reinterpret_cast<const uint16_t*>(a.dt_bias)[h];
  const float g_al = a.neg_exp_alog[h];
  constexpr int CN = ((KC - 1) * 3 * GDN_D + GDN_THREADS - 1) / GDN_THREADS;
  bf16 cb[CN];
#pragma unroll
  for (int q = 0; q < CN; ++q) {
    const int i = (int)threadIdx.x + q * GDN_THREADS;
    const int j = i / (3 * GDN_D), kind = (i / GDN_D) % 3, d = i % GDN_D;
    const int vec = kind == 0 ? hk : (kind == 1 ? a.hk + hk : 2 * a.hk + h);
    cb[q] = (w0 && i < KM1 * 3 * GDN_D && (kind == 2 || lead)) ? gdn_row_ptr(a, P + j)[vec * GDN_D + d] : (bf16)0;
  }
  asm volatile("" ::: "memory");

  // ---- prep: (q, k, v) vectors x positions, 32 lanes x 4 channels each; a lane's KC input rows
  // (4 channels each) and its 4 x KC conv taps are loaded before the first multiply
  for (int task = hw; task < 3 * S; task += GDN_THREADS / 32) {
    const int t = task / 3, kind = task % 3;
    const int vec = kind == 0 ? hk : (kind == 1 ? a.hk + hk : 2 * a.hk + h);
    const int ch0 = vec * GDN_D + 4 * l;
    uint2 xin[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) xin[j] = *reinterpret_cast<const uint2*>(gdn_row_ptr(a, P + t + j) + ch0);
    uint32_t wt[2 * KC];  // conv_w[ch0 .. ch0+3][0 .. KC-1]: 4*KC bf16, contiguous
#pragma unroll
    for (int q = 0; q < 2 * KC; ++q) wt[q] = reinterpret_cast<const uint32_t*>(a.conv_w + (size_t)ch0 * KC)[q];
    auto hbf = [](uint32_t w, int odd) { return __uint_as_float(odd ? (w & 0xffff0000u) : (w << 16)); };
    float xs[4], acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float c = 0.0f;
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const float xv = hbf(i < 2 ? xin[j].x : xin[j].y, i & 1);
        const int e = i * KC + j;
        c = c + xv * hbf(wt[e >> 1], e & 1);
      }
      const float x = silu_bf16(round_bf(c));
      xs[i] = x;
      acc = __builtin_fmaf(x, x, acc);
    }
    if ((kind == 2 && w0) || lead)  // this position's conv input row (row P + t + KC-1 is projection row t)
      *reinterpret_cast<uint2*>(a.win_nxt + (size_t)t * a.cd + ch0) = xin[KC - 1];
    if (kind < 2) {
      const float inv = 1.0f / sqrtf(half_wave_sum(acc) / 128.0f + 1e-6f);
      const float mul = kind == 0 ? q_mul : k_mul;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float val = round_bf(mul * round_bf(xs[i] * inv));
        if (kind == 0) {
          qs[t][4 * l + i] = val;
        } else {
          ks[t][4 * l + i] = val;
          if (lead) a.key_nxt[((size_t)t * a.hk + hk) * GDN_D + 4 * l + i] = f2bf(val);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) vs[t][4 * l + i] = xs[i];
    }
  }
  if (gt >= 0) {
    const int t = gt;
    const float b = sigmoid_bf16(__uint_as_float(g_b << 16));
    const float ax = round_bf(__uint_as_float(g_a << 16) + __uint_as_float(g_dt << 16));
    const float d = expf_det(g_al * logaddexp0_bf16(ax));
    dec[t] = d;
    bet[t] = b;
    if (w0) a.decay_nxt[(size_t)t * a.hv + h] = d;
  }
  // the committed conv rows R[P .. P+KC-1) become the next window's base
#pragma unroll
  for (int q = 0; q < CN; ++q) {
    const int i = (int)threadIdx.x + q * GDN_THREADS;
    const int j = i / (3 * GDN_D), kind = (i / GDN_D) % 3, d = i % GDN_D;
    const int vec = kind == 0 ? hk : (kind == 1 ? a.hk + hk : 2 * a.hk + h);
    if (w0 && i < KM1 * 3 * GDN_D && (kind == 2 || lead)) a.conv_nxt[(size_t)j * a.cd + vec * GDN_D + d] = cb[q];
  }
  __syncthreads();

  // ---- recurrence: RPH value rows per half-wave (r = r0 + hw + 16 i), lane l owns key elements 4l..4l+3
  if (P > 0) {  // committed steps of the previous window, in order
#pragma unroll
    for (int p = 0; p < JP; ++p) {
      if (p < P) {
#pragma unroll
        for (int i = 0; i < RPH; ++i)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            s[i][c] = s[i][c] * gdp[p];
            s[i][c] = __builtin_fmaf(kjournal(kpw[p], c), dlp[p][i], s[i][c]);
          }
      }
    }
#pragma unroll
    for (int i = 0; i < RPH; ++i)
      *reinterpret_cast<float4*>(a.ssm + ((size_t)h * GDN_D + r0 + hw + 16 * i) * GDN_D + 4 * l) =
          make_float4(s[i][0], s[i][1], s[i][2], s[i][3]);
  }
  // position by position, this thread's RPH state rows side by side (independent chains)
  for (int t = 0; t < S; ++t) {
    const float gd = dec[t], bt = bet[t];
    const float k0 = ks[t][4 * l], k1 = ks[t][4 * l + 1], k2 = ks[t][4 * l + 2], k3 = ks[t][4 * l + 3];
    const float q0 = qs[t][4 * l], q1 = qs[t][4 * l + 1], q2 = qs[t][4 * l + 2], q3 = qs[t][4 * l + 3];
#pragma unroll
    for (int i = 0; i < RPH; ++i) {
      const int r = r0 + hw + 16 * i;
      s[i][0] = s[i][0] * gd;
      float kv = 0.0f + s[i][0] * k0;
      float comp = 0.0f;
      {
        s[i][1] = s[i][1] * gd;
        const float prod = s[i][1] * k1, corr = prod - comp, next = kv + corr;
        comp = (next - kv) - corr;
        kv = next;
      }
      {
        s[i][2] = s[i][2] * gd;
        const float prod = s[i][2] * k2, corr = prod - comp, next = kv + corr;
        comp = (next - kv) - corr;
        kv = next;
      }
      {
        s[i][3] = s[i][3] * gd;
        const float prod = s[i][3] * k3, corr = prod - comp, next = kv + corr;
        kv = next;
      }
      const float kvm = half_wave_sum(kv);
      const float delta = (vs[t][r] - kvm) * bt;
      if (l == 0) a.delta_nxt[((size_t)t * a.hv + h) * GDN_D + r] = delta;
      float o = 0.0f;
      s[i][0] = __builtin_fmaf(k0, delta, s[i][0]);
      o = __builtin_fmaf(s[i][0], q0, o);
      s[i][1] = __builtin_fmaf(k1, delta, s[i][1]);
      o = __builtin_fmaf(s[i][1], q1, o);
      s[i][2] = __builtin_fmaf(k2, delta, s[i][2]);
      o = __builtin_fmaf(s[i][2], q2, o);
      s[i][3] = __builtin_fmaf(k3, delta, s[i][3]);
      o = __builtin_fmaf(s[i][3], q3, o);
      const float y = half_wave_sum(o);
      if (l == 0) st_pub(a.ypub + ((size_t)t * a.hv + h) * GDN_D + r, round_bf(y));
    }
  }
  // the head's last workgroup to finish gathers every row's output and runs the gated norm
  if (!ticket_last(a.tickets + h, GDN_SPLIT - 1)) return;
  for (int i = threadIdx.x; i < S * GDN_D; i += GDN_THREADS)
    ys[i / GDN_D][i % GDN_D] = ld_pub(a.ypub + ((size_t)(i / GDN_D) * a.hv + h) * GDN_D + i % GDN_D);
  __syncthreads();

  // ---- gated RMS norm per position
  for (int t = hw; t < S; t += GDN_THREADS / 32) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(ys[t][4 * l + i], ys[t][4 * l + i], acc);
    const float inv = 1.0f / sqrtf(half_wave_sum(acc) / 128.0f + a.eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 4 * l + i;
      const float n = round_bf(bf2f(a.norm_w[d]) * round_bf(ys[t][d] * inv));
      const float z = bf2f(a.proj[(size_t)t * a.pw + a.z_off + h * GDN_D + d]);
      const bf16 out = f2bf(sigmoid_f32(z) * n);
      gated[t][d] = out;
      if (a.gated) a.gated[(size_t)t * a.hv * GDN_D + h * GDN_D + d] = out;
    }
  }
  __syncthreads();

  // ---- prepared blocks of the gated rows for the output projection (4 per head and position)
  if (a.xp)
    for (int task = hw; task < 4 * S; task += GDN_THREADS / 32) {
      const int t = task >> 2, blk = task & 3;
      xprep_lanes_direct(gated[t][blk * 32 + l], l, a.xp + ((size_t)t * a.hv * 4 + h * 4 + blk) * XP_DW);
    }
}

// A prefill batch through the core (S positions, any count), two launches.
//   k_gdn_prep_batch: one workgroup per position: the conv, SiLU and q/k norms of every key head's
//     q and k and every value head's v (a half-wave per 128-channel vector, as the step kernel
//     does them), and every head's decay and beta gates, into the batch's prep buffers;
//   k_gdn_batch: the step kernel's workgroup layout with eight workgroups per value head (16 state
//     rows each: the batch's long recurrence runs as more, shorter chains), the P committed steps of the
//     previous window replayed onto the state, then the batch's positions in order, the next
//     window's prepped vectors loaded while the current one's recurrence runs; every position
//     committed: the state is stored after the last one, the batch's last kc-1 conv input rows
//     become the conv base (slot nxt), no journal is written; the head's last workgroup runs the
//     gated norm and the prepared output blocks of every position.
// The float operations of every position are a verify window's, so the bits are the same.
template <int KC>
__global__ __launch_bounds__(GDN_THREADS) void k_gdn_prep_batch(GdnArgs a, GdnBatch b) {
  const int t = blockIdx.x, hw = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int P = a.P;
  const float inv_scale = 1.0f / sqrtf((float)GDN_D);
  const float q_mul = round_bf(inv_scale * inv_scale), k_mul = round_bf(inv_scale);
  const int ntask = 2 * a.hk + a.hv;  // q of every key head, k of every key head, v of every value head
  for (int task = hw; task < ntask; task += GDN_THREADS / 32) {
    const int kind = task < a.hk ? 0 : (task < 2 * a.hk ? 1 : 2);
    const int vec = task;  // channel block: q heads, then k heads, then v heads
    const int ch0 = vec * GDN_D + 4 * l;
    uint2 xin[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) xin[j] = *reinterpret_cast<const uint2*>(gdn_row_ptr(a, P + t + j) + ch0);
    uint32_t wt[2 * KC];
#pragma unroll
    for (int q = 0; q < 2 * KC; ++q) wt[q] = reinterpret_cast<const uint32_t*>(a.conv_w + (size_t)ch0 * KC)[q];
    auto hbf = [](uint32_t w, int odd) { return __uint_as_float(odd ? (w & 0xffff0000u) : (w << 16)); };
    float xs[4], acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float c = 0.0f;
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const float xv = hbf(i < 2 ? xin[j].x : xin[j].y, i & 1);
        const int e = i * KC + j;
        c = c + xv * hbf(wt[e >> 1], e & 1);
      }
      const float x = silu_bf16(round_bf(c));
      xs[i] = x;
      acc = __builtin_fmaf(x, x, acc);
    }
    float4 o;
    if (kind < 2) {
      const float inv = 1.0f / sqrtf(half_wave_sum(acc) / 128.0f + 1e-6f);
      const float mul = kind == 0 ? q_mul : k_mul;
      o = make_float4(round_bf(mul * round_bf(xs[0] * inv)), round_bf(mul * round_bf(xs[1] * inv)),
                      round_bf(mul * round_bf(xs[2] * inv)), round_bf(mul * round_bf(xs[3] * inv)));
    } else {
      o = make_float4(xs[0], xs[1], xs[2], xs[3]);
    }
    *reinterpret_cast<float4*>(b.vecs + ((size_t)t * ntask + vec) * GDN_D + 4 * l) = o;
  }
  for (int h = threadIdx.x; h < a.hv; h += GDN_THREADS) {
    const bf16* prow = a.proj + (size_t)t * a.pw;
    const float bt = sigmoid_bf16(bf2f(prow[a.b_off + h]));
    const float ax = round_bf(bf2f(prow[a.a_off + h]) + bf2f(a.dt_bias[h]));
    b.gates[((size_t)t * a.hv + h) * 2] = expf_det(a.neg_exp_alog[h] * logaddexp0_bf16(ax));
    b.gates[((size_t)t * a.hv + h) * 2 + 1] = bt;
  }
}

template <int KC>
__global__ __launch_bounds__(GDN_THREADS) void k_gdn_batch(GdnArgs a, GdnBatch b) {
  __shared__ float qs[2][MAX_TOKENS][GDN_D], ks[2][MAX_TOKENS][GDN_D], vs[2][MAX_TOKENS][GDN_D];
  __shared__ float dec[2][MAX_TOKENS], bet[2][MAX_TOKENS];
  __shared__ float ys[MAX_TOKENS][GDN_D];
  __shared__ bf16 gated[MAX_TOKENS][GDN_D];
  const int h = blockIdx.x, ratio = a.hv / a.hk, hk = h / ratio;
  const int r0 = blockIdx.y * (GDN_D / GDN_BSPLIT);  // this workgroup's state rows
  const bool w0 = blockIdx.y == 0;
  const bool lead = (h % ratio) == 0 && w0;         // writes the q/k channels' conv base rows
  const int hw = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int S = a.S, P = a.P, KM1 = a.kc - 1;
  const int ntask = 2 * a.hk + a.hv;
  constexpr int RPH = GDN_D / GDN_BSPLIT / (GDN_THREADS / 32);
  // a window's prepped vectors: (q, k, v) x MAX_TOKENS x 128 floats as float4 units, and the gates
  constexpr int U4 = 3 * MAX_TOKENS * GDN_D / 4;  // float4 units of a window
  // this thread's units: u0 = threadIdx.x and u1 = threadIdx.x + GDN_THREADS (while < U4) -> (vector which,
  // position tt, float4 e4); the source offsets (relative to the window's first position) and the LDS targets
  // are the same every window
  static_assert(U4 > GDN_THREADS && U4 <= 2 * GDN_THREADS, "two units per thread");
  auto unit = [&](int u, const float*& src, float*& dst, int& tt) {
    const int which = u / (MAX_TOKENS * GDN_D / 4), rem = u % (MAX_TOKENS * GDN_D / 4);
    const int e4 = rem % (GDN_D / 4);
    tt = rem / (GDN_D / 4);
    const int vec = which == 0 ? hk : (which == 1 ? a.hk + hk : 2 * a.hk + h);
    src = b.vecs + (size_t)vec * GDN_D + 4 * e4;
    dst = (which == 0 ? &qs[0][tt][0] : (which == 1 ? &ks[0][tt][0] : &vs[0][tt][0])) + 4 * e4;
  };
  const bool has1 = (int)threadIdx.x + GDN_THREADS < U4;
  const float *src0, *src1;
  float *dst0, *dst1;
  int tt0, tt1;
  unit((int)threadIdx.x, src0, dst0, tt0);
  unit(has1 ? (int)threadIdx.x + GDN_THREADS : (int)threadIdx.x, src1, dst1, tt1);
  const int gt = (int)threadIdx.x / 2, gk = (int)threadIdx.x & 1;  // gate thread: position, decay or beta
  float4 pv0, pv1;
  float pg = 0.0f;
  const size_t pstride = (size_t)ntask * GDN_D;
  // unconditional loads (clamped position: positions past S are loaded again and not used)
#define GDN_FETCH(T0)                                                                                       \
  do {                                                                                                      \
    pv0 = *reinterpret_cast<const float4*>(src0 + (size_t)min((T0) + tt0, S - 1) * pstride);                \
    pv1 = *reinterpret_cast<const float4*>(src1 + (size_t)min((T0) + tt1, S - 1) * pstride);                \
    if ((int)threadIdx.x < 2 * MAX_TOKENS) pg = b.gates[((size_t)min((T0) + gt, S - 1) * a.hv + h) * 2 + gk]; \
  } while (0)
#define GDN_STORE(BUF)                                                                                     \
  do {                                                                                                     \
    *reinterpret_cast<float4*>(dst0 + (BUF) * MAX_TOKENS * GDN_D) = pv0;                                     \
    if (has1) *reinterpret_cast<float4*>(dst1 + (BUF) * MAX_TOKENS * GDN_D) = pv1;                           \
    if ((int)threadIdx.x < 2 * MAX_TOKENS) (gk ? bet : dec)[(BUF)][gt] = pg;                                \
  } while (0)
  GDN_FETCH(0);
  float s[RPH][4];
#pragma unroll
  for (int i = 0; i < RPH; ++i) {
    const float4 s4 = *reinterpret_cast<const float4*>(a.ssm + ((size_t)h * GDN_D + r0 + hw + 16 * i) * GDN_D + 4 * l);
    s[i][0] = s4.x;
    s[i][1] = s4.y;
    s[i][2] = s4.z;
    s[i][3] = s4.w;
  }
  // the previous window's committed steps, in order
  for (int p = 0; p < P; ++p) {
    const float gd = a.decay_cur[(size_t)p * a.hv + h];
    const uint2 kw = *reinterpret_cast<const uint2*>(a.key_cur + ((size_t)p * a.hk + hk) * GDN_D + 4 * l);
    const float kp[4] = {__uint_as_float(kw.x << 16), __uint_as_float(kw.x & 0xffff0000u),
                         __uint_as_float(kw.y << 16), __uint_as_float(kw.y & 0xffff0000u)};
#pragma unroll
    for (int i = 0; i < RPH; ++i) {
      const float dl = a.delta_cur[((size_t)p * a.hv + h) * GDN_D + r0 + hw + 16 * i];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s[i][c] = s[i][c] * gd;
        s[i][c] = __builtin_fmaf(kp[c], dl, s[i][c]);
      }
    }
  }
  GDN_STORE(0);
  __syncthreads();
  for (int t0 = 0, buf = 0; t0 < S; t0 += MAX_TOKENS, buf ^= 1) {
    const int n = S - t0 < MAX_TOKENS ? S - t0 : MAX_TOKENS;
    const bool more = t0 + MAX_TOKENS < S;
    if (more) GDN_FETCH(t0 + MAX_TOKENS);  // in flight during this window's recurrence
    // position by position, this thread's RPH state rows side by side (independent chains, each with the
    // step kernel's operations in its order; the position's k, q and gates read once for all of them)
    for (int t = 0; t < n; ++t) {
      const float gd = dec[buf][t], bt = bet[buf][t];
      const float k0 = ks[buf][t][4 * l], k1 = ks[buf][t][4 * l + 1], k2 = ks[buf][t][4 * l + 2],
                  k3 = ks[buf][t][4 * l + 3];
      const float q0 = qs[buf][t][4 * l], q1 = qs[buf][t][4 * l + 1], q2 = qs[buf][t][4 * l + 2],
                  q3 = qs[buf][t][4 * l + 3];
#pragma unroll
      for (int i = 0; i < RPH; ++i) {
        const int r = r0 + hw + 16 * i;
        s[i][0] = s[i][0] * gd;
        float kv = 0.0f + s[i][0] * k0;
        float comp = 0.0f;
        {
          s[i][1] = s[i][1] * gd;
          const float prod = s[i][1] * k1, corr = prod - comp, next = kv + corr;
          comp = (next - kv) - corr;
          kv = next;
        }
        {
          s[i][2] = s[i][2] * gd;
          const float prod = s[i][2] * k2, corr = prod - comp, next = kv + corr;
          comp = (next - kv) - corr;
          kv = next;
        }
        {
          s[i][3] = s[i][3] * gd;
          const float prod = s[i][3] * k3, corr = prod - comp, next = kv + corr;
          kv = next;
        }
        const float kvm = half_wave_sum(kv);
        const float delta = (vs[buf][t][r] - kvm) * bt;
        float o = 0.0f;
        s[i][0] = __builtin_fmaf(k0, delta, s[i][0]);
        o = __builtin_fmaf(s[i][0], q0, o);
        s[i][1] = __builtin_fmaf(k1, delta, s[i][1]);
        o = __builtin_fmaf(s[i][1], q1, o);
        s[i][2] = __builtin_fmaf(k2, delta, s[i][2]);
        o = __builtin_fmaf(s[i][2], q2, o);
        s[i][3] = __builtin_fmaf(k3, delta, s[i][3]);
        o = __builtin_fmaf(s[i][3], q3, o);
        const float y = half_wave_sum(o);
        if (l == 0) st_pub(a.ypub + ((size_t)(t0 + t) * a.hv + h) * GDN_D + r, round_bf(y));
      }
    }
    if (more) GDN_STORE(buf ^ 1);  // the other buffer: last read in the previous window, before its barrier
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < RPH; ++i)
    *reinterpret_cast<float4*>(a.ssm + ((size_t)h * GDN_D + r0 + hw + 16 * i) * GDN_D + 4 * l) =
        make_float4(s[i][0], s[i][1], s[i][2], s[i][3]);
  // the batch's last kc-1 input rows become the conv base
  for (int i = threadIdx.x; i < (w0 ? KM1 * 3 * GDN_D : 0); i += GDN_THREADS) {
    const int j = i / (3 * GDN_D), kind = (i / GDN_D) % 3, d = i % GDN_D;
    if (kind < 2 && !lead) continue;
    const int vec = kind == 0 ? hk : (kind == 1 ? a.hk + hk : 2 * a.hk + h);
    const int ch = vec * GDN_D + d;
    a.conv_nxt[(size_t)j * a.cd + ch] = f2bf(gdn_row(a, P + S + j, ch));
  }
  if (!ticket_last(a.tickets + h, GDN_BSPLIT - 1)) return;
  for (int t0 = 0; t0 < S; t0 += MAX_TOKENS) {
    const int n = S - t0 < MAX_TOKENS ? S - t0 : MAX_TOKENS;
    for (int i = threadIdx.x; i < n * GDN_D; i += GDN_THREADS)
      ys[i / GDN_D][i % GDN_D] = ld_pub(a.ypub + ((size_t)(t0 + i / GDN_D) * a.hv + h) * GDN_D + i % GDN_D);
    __syncthreads();
    for (int t = hw; t < n; t += GDN_THREADS / 32) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(ys[t][4 * l + i], ys[t][4 * l + i], acc);
      const float inv = 1.0f / sqrtf(half_wave_sum(acc) / 128.0f + a.eps);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 4 * l + i;
        const float nv = round_bf(bf2f(a.norm_w[d]) * round_bf(ys[t][d] * inv));
        const float z = bf2f(a.proj[(size_t)(t0 + t) * a.pw + a.z_off + h * GDN_D + d]);
        const bf16 out = f2bf(sigmoid_f32(z) * nv);
        gated[t][d] = out;
        if (a.gated) a.gated[(size_t)(t0 + t) * a.hv * GDN_D + h * GDN_D + d] = out;
      }
    }
    __syncthreads();
    if (a.xp)
      for (int task = hw; task < 4 * n; task += GDN_THREADS / 32) {
        const int t = task >> 2, blk = task & 3;
        xprep_lanes_direct(gated[t][blk * 32 + l], l, a.xp + ((size_t)(t0 + t) * a.hv * 4 + h * 4 + blk) * XP_DW);
      }
    __syncthreads();  // ys and gated of the next window
  }
}

// Committed state without modifying it: the P journal steps replayed onto the
// state rows into ssm_dst, and the committed conv rows into conv_dst.
__global__ __launch_bounds__(GDN_THREADS) void k_gdn_replay(GdnArgs a, float* ssm_dst, bf16* conv_dst) {
  const int h = blockIdx.x, ratio = a.hv / a.hk, hk = h / ratio;
  const bool lead = (h % ratio) == 0;
  const int hw = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int P = a.P, KM1 = a.kc - 1;
  for (int r = hw; r < GDN_D; r += GDN_THREADS / 32) {
    const float* srow = a.ssm + ((size_t)h * GDN_D + r) * GDN_D + 4 * l;
    const float4 s4 = *reinterpret_cast<const float4*>(srow);
    float s[4] = {s4.x, s4.y, s4.z, s4.w};
    for (int p = 0; p < P; ++p) {
      const float gd = a.decay_cur[(size_t)p * a.hv + h];
      const float dl = a.delta_cur[((size_t)p * a.hv + h) * GDN_D + r];
      const bf16* kp = a.key_cur + ((size_t)p * a.hk + hk) * GDN_D + 4 * l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = s[i] * gd;
        s[i] = __builtin_fmaf(bf2f(kp[i]), dl, s[i]);
      }
    }
    *reinterpret_cast<float4*>(ssm_dst + ((size_t)h * GDN_D + r) * GDN_D + 4 * l) = make_float4(s[0], s[1], s[2], s[3]);
  }
  for (int i = threadIdx.x; i < KM1 * 3 * GDN_D; i += GDN_THREADS) {
    const int j = i / (3 * GDN_D), kind = (i / GDN_D) % 3, d = i % GDN_D;
    if (kind < 2 && !lead) continue;
    const int vec = kind == 0 ? hk : (kind == 1 ? a.hk + hk : 2 * a.hk + h);
    const int ch = vec * GDN_D + d;
    conv_dst[(size_t)j * a.cd + ch] = f2bf(gdn_row(a, P + j, ch));
  }
}

template <int KC>
static hipError_t gdn_step_kc(const GdnArgs& a, hipStream_t st) {
  if (!a.tickets || !a.ypub || a.P < 0 || a.P > MAX_TOKENS) return hipErrorInvalidValue;
  const dim3 grid(a.hv, GDN_SPLIT);
  if constexpr (KC == 4) {  // the model's conv: the replay sized to the journal (1, 2, 4 or 8 steps)
    if (a.P <= 1) {
      hipLaunchKernelGGL((k_gdn_step<KC, 1>), grid, dim3(GDN_THREADS), 0, st, a);
    } else if (a.P <= 2) {
      hipLaunchKernelGGL((k_gdn_step<KC, 2>), grid, dim3(GDN_THREADS), 0, st, a);
    } else if (a.P <= 4) {
      hipLaunchKernelGGL((k_gdn_step<KC, 4>), grid, dim3(GDN_THREADS), 0, st, a);
    } else {
      hipLaunchKernelGGL((k_gdn_step<KC, MAX_TOKENS>), grid, dim3(GDN_THREADS), 0, st, a);
    }
    return hipGetLastError();
  }
  hipLaunchKernelGGL((k_gdn_step<KC, MAX_TOKENS>), grid, dim3(GDN_THREADS), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_gdn_step(const GdnArgs& a, hipStream_t st) {
  switch (a.kc) {
    case 2: return gdn_step_kc<2>(a, st);
    case 3: return gdn_step_kc<3>(a, st);
    case 4: return gdn_step_kc<4>(a, st);
    case 5: return gdn_step_kc<5>(a, st);
    case 6: return gdn_step_kc<6>(a, st);
    case 7: return gdn_step_kc<7>(a, st);
    case 8: return gdn_step_kc<8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

template <int KC>
static hipError_t gdn_batch_kc(const GdnArgs& a, const GdnBatch& b, hipStream_t st) {
  if (!a.tickets || !a.ypub || !b.vecs || !b.gates || a.S < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_prep_batch<KC>, dim3(a.S), dim3(GDN_THREADS), 0, st, a, b);
  hipLaunchKernelGGL(k_gdn_batch<KC>, dim3(a.hv, GDN_BSPLIT), dim3(GDN_THREADS), 0, st, a, b);
  return hipGetLastError();
}

hipError_t launch_gdn_batch(const GdnArgs& a, const GdnBatch& b, hipStream_t st) {
  switch (a.kc) {
    case 2: return gdn_batch_kc<2>(a, b, st);
    case 3: return gdn_batch_kc<3>(a, b, st);
    case 4: return gdn_batch_kc<4>(a, b, st);
    case 5: return gdn_batch_kc<5>(a, b, st);
    case 6: return gdn_batch_kc<6>(a, b, st);
    case 7: return gdn_batch_kc<7>(a, b, st);
    case 8: return gdn_batch_kc<8>(a, b, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gdn_replay(const GdnArgs& a, float* ssm_dst, bf16* conv_dst, hipStream_t st) {
  hipLaunchKernelGGL(k_gdn_replay, dim3(a.hv), dim3(GDN_THREADS), 0, st, a, ssm_dst, conv_dst);
  return hipGetLastError();
}

}  // namespace mtpx
