/*
 * mtpx CPU oracle -- TEST INFRASTRUCTURE ONLY (see mtpx_oracle.h).
 *
 * Reference semantics followed (paths relative to the reference checkout):
 *   MLX = Vendor/mlx-swift/Source/Cmlx/mlx/mlx
 *   FM  = Runner/FastModel
 *
 * Parity status of each function is listed in the header comment of the
 * function and summarised in tests/test_oracle_pin.py.
 */
#include "mtpx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================== */
/* scalar numerics                                                           */
/* ======================================================================== */

float o_bf2f(o_bf16 h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

o_bf16 o_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0; /* NaN */
  u += 0x7fffu + ((u >> 16) & 1u);                      /* round to nearest even */
  return (o_bf16)(u >> 16);
}

float o_round_bf(float f) { return o_bf2f(o_f2bf(f)); }

static float f_from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/*
 * exp(x) in float: Cody-Waite reduction x = n*ln2 + r with a two-part ln2,
 * degree-7 Taylor polynomial on |r| <= ln2/2 (truncation error < 2^-27
 * relative), scale by 2^n in two exact steps.  Inputs below -87.3 return 0
 * (no subnormal results), above 88.7 return +inf.  Pinned against libm expf
 * (<= 2 ulp over a dense sweep) in tests/test_oracle_pin.py.
 */
float o_expf(float x) {
  if (x != x) return x;
  if (x < -87.3f) return 0.0f;
  if (x > 88.7f) return f_from_bits(0x7f800000u);
  const float n = rintf(x * 1.44269504f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187e-06f, r);
  float p = 1.98412698e-04f;
  p = fmaf(p, r, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333333e-03f);
  p = fmaf(p, r, 4.16666667e-02f);
  p = fmaf(p, r, 1.66666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2, n2 = ni - n1;
  p = p * f_from_bits((uint32_t)(n1 + 127) << 23);
  p = p * f_from_bits((uint32_t)(n2 + 127) << 23);
  return p;
}

/*
 * MLX's Sigmoid functor evaluated in bf16 (each operation rounds to bf16):
 * y = 1 / (1 + exp(|x|)); x < 0 ? y : 1 - y.
 * Follows FM/TrackFastKernels2.swift:21-30 (mlx_sigmoid / mlx_silu).
 */
float o_sigmoid_bf16(float x) {
  const float e = o_round_bf(o_expf(fabsf(x)));
  const float d = o_round_bf(1.0f + e);
  const float y = o_round_bf(1.0f / d);
  return (x < 0.0f) ? y : o_round_bf(1.0f - y);
}

float o_silu_bf16(float x) { return o_round_bf(x * o_sigmoid_bf16(x)); }

/* Lanes that share one row of the q4 GEMV: the largest power of two <= 64
 * that still leaves each lane >= 4 blocks of 32 elements. */
int o_lanes_for_blocks(int nb) {
  int L = 1;
  while (L < 64 && (L * 2) * 4 <= nb) L *= 2;
  return L;
}

/* ======================================================================== */
/* a1: MLX affine quantize (MLX/backend/cpu/quantized.cpp:1158-1220,         */
/*     MLX/ops.cpp:5036-5090, pack MLX/ops.cpp:4988-5020)                    */
/* ======================================================================== */

void o_affine_quantize(const o_bf16* w, int64_t rows, int K, int gs, uint32_t* wq,
                       o_bf16* scales, o_bf16* biases) {
  const int ng = K / gs;
  for (int64_t r = 0; r < rows; ++r) {
    for (int g = 0; g < ng; ++g) {
      const o_bf16* wg = w + r * K + (int64_t)g * gs;
      float wmin = INFINITY, wmax = -INFINITY;
      for (int j = 0; j < gs; ++j) {
        const float v = o_bf2f(wg[j]);
        wmax = fmaxf(wmax, v);
        wmin = fminf(wmin, v);
      }
      const int mask = fabsf(wmin) > fabsf(wmax);
      float scale = fmaxf((wmax - wmin) / 15.0f, 1e-7f);
      scale = mask ? scale : -scale;
      const float edge = mask ? wmin : wmax;
      const float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      for (int j = 0; j < gs / 8; ++j) {
        uint32_t word = 0;
        for (int t = 0; t < 8; ++t) {
          float v = rintf((o_bf2f(wg[j * 8 + t]) - bias) / scale);
          v = fminf(fmaxf(v, 0.0f), 15.0f);
          word |= (uint32_t)v << (4 * t);
        }
        wq[r * (K / 8) + (int64_t)g * (gs / 8) + j] = word;
      }
      scales[r * ng + g] = o_f2bf(scale);
      biases[r * ng + g] = o_f2bf(bias);
    }
  }
}

/* ======================================================================== */
/* a2-a4, a12: q4 GEMV                                                       */
/* ======================================================================== */

/*
 * Activation block transform.  A block of 32 bf16 values shares the exponent
 * E = max biased exponent field (a zero field counts as 1).  Each value
 * becomes the integer m = x / 2^(E-149), truncated toward zero, so
 * |m| < 2^23: exact for every element within 2^15 of the block maximum.
 */
void o_xblock(const o_bf16* x32, int32_t* m, int32_t* E_out) {
  int E = 1;
  for (int i = 0; i < 32; ++i) {
    int f = (x32[i] >> 7) & 0xff;
    if (f < 1) f = 1;
    if (f > E) E = f;
  }
  for (int i = 0; i < 32; ++i) {
    const uint32_t h = x32[i];
    const int field = (h >> 7) & 0xff;
    const int f = field < 1 ? 1 : field;
    const int32_t sig = (int32_t)((field ? 0x80u : 0u) | (h & 0x7fu));
    const int sh = f - E + 15;
    int32_t mag;
    if (sh >= 0)
      mag = sig << sh;
    else if (sh > -31)
      mag = sig >> (-sh);
    else
      mag = 0;
    m[i] = (h & 0x8000u) ? -mag : mag;
  }
  *E_out = E;
}

static float block_scale(int E) {
  /* 2^(E - 149) as a float */
  if (E >= 23) return f_from_bits((uint32_t)(E - 22) << 23);
  return f_from_bits(1u << E);
}

/* One row of the GEMV over pre-transformed activation blocks.
 * Per block j: D = sum_i q_i * m_i split over the 24-bit two's-complement
 * limbs of m (l0, l1 unsigned bytes, l2 signed byte); each limb sum is exact.
 *   DXraw = fmaf((float)D2, 65536, (float)(D1*256 + D0))
 *   DX = DXraw * p_j,  SX = (float)(sum_i m_i) * p_j,  p_j = 2^(E_j-149)
 *   acc_lane = fmaf(b_g, SX, fmaf(s_g, DX, acc_lane))
 * Lane l of L accumulates blocks l, l+L, ... in order from 0.0f; the L lane
 * values are then folded by an xor butterfly (offsets L/2 ... 1). */
static float qmv_row(const uint32_t* wrow, const o_bf16* srow, const o_bf16* brow, int K, int gs,
                     const int32_t* m /* [nb*32] */, const float* p /* [nb] */,
                     const float* SX /* [nb] */) {
  const int nb = K / 32;
  const int L = o_lanes_for_blocks(nb);
  float lane[64];
  for (int l = 0; l < L; ++l) {
    float acc = 0.0f;
    for (int j = l; j < nb; j += L) {
      int64_t d0 = 0, d1 = 0, d2 = 0;
      for (int wd = 0; wd < 4; ++wd) {
        const uint32_t word = wrow[j * 4 + wd];
        for (int e = 0; e < 8; ++e) {
          const uint32_t q = (word >> (4 * e)) & 0xfu;
          const uint32_t u = (uint32_t)m[j * 32 + wd * 8 + e] & 0xffffffu;
          const int32_t l0 = (int32_t)(u & 0xffu), l1 = (int32_t)((u >> 8) & 0xffu);
          const int32_t l2 = (int32_t)(int8_t)(uint8_t)(u >> 16);
          d0 += (int64_t)q * l0;
          d1 += (int64_t)q * l1;
          d2 += (int64_t)q * l2;
        }
      }
      const int32_t low = (int32_t)(d1 * 256 + d0);
      const float dxraw = fmaf((float)(int32_t)d2, 65536.0f, (float)low);
      const float dx = dxraw * p[j];
      const int g = (j * 32) / gs;
      acc = fmaf(o_bf2f(srow[g]), dx, acc);
      acc = fmaf(o_bf2f(brow[g]), SX[j], acc);
    }
    lane[l] = acc;
  }
  for (int off = L / 2; off >= 1; off /= 2) {
    float nv[64];
    for (int l = 0; l < L; ++l) nv[l] = lane[l] + lane[l ^ off];
    memcpy(lane, nv, sizeof(float) * L);
  }
  return lane[0];
}

typedef struct {
  int nb;
  int32_t* m;
  float* p;
  float* SX;
} xprep_t;

static void xprep(const o_bf16* x, int K, xprep_t* xp) {
  xp->nb = K / 32;
  xp->m = (int32_t*)malloc(sizeof(int32_t) * K);
  xp->p = (float*)malloc(sizeof(float) * xp->nb);
  xp->SX = (float*)malloc(sizeof(float) * xp->nb);
  for (int j = 0; j < xp->nb; ++j) {
    int32_t E;
    o_xblock(x + j * 32, xp->m + j * 32, &E);
    int32_t sm = 0;
    for (int i = 0; i < 32; ++i) sm += xp->m[j * 32 + i];
    xp->p[j] = block_scale(E);
    xp->SX[j] = (float)sm * xp->p[j];
  }
}

static void xfree(xprep_t* xp) {
  free(xp->m);
  free(xp->p);
  free(xp->SX);
}

void o_qmv(const uint32_t* wq, const o_bf16* scales, const o_bf16* biases, int64_t N, int K,
           int gs, const o_bf16* x, int M, o_bf16* y, float* yf) {
  const int ng = K / gs;
  for (int mm = 0; mm < M; ++mm) {
    xprep_t xp;
    xprep(x + (int64_t)mm * K, K, &xp);
    /* rows are independent: a thread per row block gives the same bits as one thread */
#pragma omp parallel for schedule(static) if (N * (int64_t)K >= ((int64_t)1 << 20))
    for (int64_t r = 0; r < N; ++r) {
      const float v = qmv_row(wq + r * (K / 8), scales + r * ng, biases + r * ng, K, gs, xp.m,
                              xp.p, xp.SX);
      if (y) y[(int64_t)mm * N + r] = o_f2bf(v);
      if (yf) yf[(int64_t)mm * N + r] = v;
    }
    xfree(&xp);
  }
}

/* ======================================================================== */
/* a6 / a9: router GEMV (FM/TrackFastMoE.swift:2246-2310: bf16 weight, f32   */
/* activation, f32 result).  Order: 64 lanes; lane l walks 8-element chunks  */
/* c = l, l+64, ... and accumulates acc = fmaf(w, x, acc) element by element; */
/* then an xor butterfly over the 64 lanes.                                  */
/* ======================================================================== */

static float router_row(const o_bf16* wrow, int H, const float* x) {
  float lane[64];
  const int nc = H / 8;
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int c = l; c < nc; c += 64)
      for (int i = 0; i < 8; ++i) acc = fmaf(o_bf2f(wrow[c * 8 + i]), x[c * 8 + i], acc);
    lane[l] = acc;
  }
  for (int off = 32; off >= 1; off /= 2) {
    float nv[64];
    for (int l = 0; l < 64; ++l) nv[l] = lane[l] + lane[l ^ off];
    memcpy(lane, nv, sizeof(nv));
  }
  return lane[0];
}

void o_router_gemv(const o_bf16* W, int rows, int H, const float* x, int M, float* out) {
  for (int m = 0; m < M; ++m)
#pragma omp parallel for schedule(static) if ((int64_t)rows * H >= ((int64_t)1 << 20))
    for (int r = 0; r < rows; ++r)
      out[(int64_t)m * rows + r] = router_row(W + (int64_t)r * H, H, x + (int64_t)m * H);
}

/* ======================================================================== */
/* a8: top-k + softmax (FM/TrackFastMoE.swift:780-878): the K largest logits, */
/* value descending, ties to the lowest index, a NaN ranked as -inf (so the K */
/* experts are always distinct); softmax over the K selected:                 */
/* max, e_k = exp(v_k - max), sum in rank order, w_k = e_k * (1 / sum).       */
/* ======================================================================== */

void o_topk_softmax(const float* logits, int M, int E, int K, int32_t* idx, float* w) {
  unsigned char* taken = (unsigned char*)malloc((size_t)E);
  for (int m = 0; m < M; ++m) {
    const float* lr = logits + (int64_t)m * E;
    memset(taken, 0, (size_t)E);
    float v[64];
    for (int k = 0; k < K; ++k) {
      int best = -1;
      float bv = -INFINITY;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        const float x = lr[e] == lr[e] ? lr[e] : -INFINITY; /* a NaN logit ranks as -inf */
        if (best < 0 || x > bv) {
          best = e;
          bv = x;
        }
      }
      taken[best] = 1;
      idx[m * K + k] = best;
      v[k] = bv;
    }
    const float mx = v[0];
    float e[64];
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) {
      e[k] = o_expf(v[k] - mx);
      sum = sum + e[k];
    }
    const float inv = 1.0f / sum;
    for (int k = 0; k < K; ++k) w[m * K + k] = e[k] * inv;
  }
  free(taken);
}

/* ======================================================================== */
/* a5, a10, a11: the MoE block (FM/TrackFastModel.swift:867-954,             */
/* FM/TrackFastMoE.swift:1192-1576, FM/TrackFastKernels2.swift:512-567)      */
/* ======================================================================== */

/* MLX col_reduce_small fold over K products (FM/TrackFastKernels2.swift:31-44). */
static float colsum_small(const float* r, int K) {
  const int TY = K < 8 ? K : 8;
  float t[8];
  for (int y = 0; y < TY; ++y) {
    float acc = 0.0f;
    for (int rr = y; rr < K; rr += TY) acc = r[rr] + acc;
    t[y] = acc;
  }
  float total = t[0];
  for (int j = 1; j < TY; ++j) total = t[j] + total;
  return total;
}

/* gate|up GEMV of one expert + SwiGLU: act[f] = bf16(silu_bf16(g) * u). */
static void expert_act(const uint32_t* gw, const o_bf16* gs_, const o_bf16* gb,
                       const uint32_t* uw, const o_bf16* us, const o_bf16* ub, int F, int H,
                       int gsz, const o_bf16* x, o_bf16* act) {
  o_bf16* g = (o_bf16*)malloc(sizeof(o_bf16) * F);
  o_bf16* u = (o_bf16*)malloc(sizeof(o_bf16) * F);
  o_qmv(gw, gs_, gb, F, H, gsz, x, 1, g, NULL);
  o_qmv(uw, us, ub, F, H, gsz, x, 1, u, NULL);
  for (int f = 0; f < F; ++f)
    act[f] = o_f2bf(o_silu_bf16(o_bf2f(g[f])) * o_bf2f(u[f]));
  free(g);
  free(u);
}

void o_moe_block(const o_moe_weights* mw, const o_bf16* x, int M, o_bf16* y, int32_t* idx,
                 float* w, float* logits, o_bf16* gate, o_bf16* act_out) {
  const int H = mw->H, E = mw->E, K = mw->K, F = mw->F, gsz = mw->gs;
  const int64_t ngH = H / gsz, ngF = F / gsz;
  float* xf = (float*)malloc(sizeof(float) * H);
  o_bf16* act = (o_bf16*)malloc(sizeof(o_bf16) * (size_t)(K + 1) * F);
  o_bf16* r = (o_bf16*)malloc(sizeof(o_bf16) * (size_t)(K + 1) * H);
  float* lg = (float*)malloc(sizeof(float) * E);
  for (int m = 0; m < M; ++m) {
    const o_bf16* xm = x + (int64_t)m * H;
    for (int h = 0; h < H; ++h) xf[h] = o_bf2f(xm[h]);
    o_router_gemv(mw->router, E, H, xf, 1, lg);
    float gl;
    if (mw->sg_w) { /* q4 row: the GEMV's value before its bf16 rounding (TrackFastMoE.swift:780-800) */
      o_bf16 gq;
      o_qmv(mw->sg_w, mw->sg_s, mw->sg_b, 1, H, gsz, xm, 1, &gq, &gl);
    } else {
      o_router_gemv(mw->shared_gate, 1, H, xf, 1, &gl);
    }
    const float gbf = o_round_bf(gl);
    if (logits) memcpy(logits + (int64_t)m * E, lg, sizeof(float) * E);
    if (gate) gate[m] = o_f2bf(gl);
    int32_t id[64];
    float wk[64];
    o_topk_softmax(lg, 1, E, K, id, wk);
    if (idx) memcpy(idx + m * K, id, sizeof(int32_t) * K);
    if (w) memcpy(w + m * K, wk, sizeof(float) * K);
    for (int k = 0; k < K; ++k) {
      const int64_t e = id[k];
      expert_act(mw->gate_w + e * F * (H / 8), mw->gate_s + e * F * ngH, mw->gate_b + e * F * ngH,
                 mw->up_w + e * F * (H / 8), mw->up_s + e * F * ngH, mw->up_b + e * F * ngH, F, H,
                 gsz, xm, act + (int64_t)k * F);
      o_qmv(mw->down_w + e * H * (F / 8), mw->down_s + e * H * ngF, mw->down_b + e * H * ngF, H,
            F, gsz, act + (int64_t)k * F, 1, r + (int64_t)k * H, NULL);
    }
    expert_act(mw->sh_gate_w, mw->sh_gate_s, mw->sh_gate_b, mw->sh_up_w, mw->sh_up_s,
               mw->sh_up_b, F, H, gsz, xm, act + (int64_t)K * F);
    o_qmv(mw->sh_down_w, mw->sh_down_s, mw->sh_down_b, H, F, gsz, act + (int64_t)K * F, 1,
          r + (int64_t)K * H, NULL);
    if (act_out) {
      for (int k = 0; k < K; ++k)
        memcpy(act_out + ((int64_t)m * K + k) * F, act + (int64_t)k * F, sizeof(o_bf16) * F);
      memcpy(act_out + ((int64_t)M * K + m) * F, act + (int64_t)K * F, sizeof(o_bf16) * F);
    }
    const float sg = o_sigmoid_bf16(gbf);
    for (int h = 0; h < H; ++h) {
      float prod[64];
      for (int k = 0; k < K; ++k) prod[k] = o_bf2f(r[(int64_t)k * H + h]) * wk[k];
      const float rr = o_round_bf(colsum_small(prod, K));
      const float sh = o_round_bf(sg * o_bf2f(r[(int64_t)K * H + h]));
      y[(int64_t)m * H + h] = o_f2bf(rr + sh);
    }
  }
  free(xf);
  free(act);
  free(r);
  free(lg);
}

/* ======================================================================== */
/* a13: attention prep (FM/TrackFastKernels2.swift:381-476)                  */
/* ======================================================================== */

/* Rotate-half RoPE tables [positions, rot] (bf16): entry d uses frequency
 * theta^(-2*(d mod rot/2)/rot); angles and cos/sin in double, then bf16. */
void o_rope_table(int positions, int rot, double theta, o_bf16* cos_t, o_bf16* sin_t) {
  const int half = rot / 2;
  for (int p = 0; p < positions; ++p)
    for (int d = 0; d < rot; ++d) {
      const int i = d % half;
      const double inv = pow(theta, -2.0 * (double)i / (double)rot);
      const double a = (double)p * inv;
      cos_t[(int64_t)p * rot + d] = o_f2bf((float)cos(a));
      sin_t[(int64_t)p * rot + d] = o_f2bf((float)sin(a));
    }
}

/* RMS statistic of one head of D values: D/4 lanes, lane t squares elements
 * 4t..4t+3 into acc = fmaf(x, x, acc), then an xor butterfly over D/4 lanes;
 * inv = 1 / sqrtf(sum / D + eps). */
static float head_inv_rms(const float* x, int D, float eps) {
  const int L = D / 4;
  float lane[256];
  for (int t = 0; t < L; ++t) {
    float acc = 0.0f;
    for (int i = 0; i < 4; ++i) acc = fmaf(x[4 * t + i], x[4 * t + i], acc);
    lane[t] = acc;
  }
  for (int off = L / 2; off >= 1; off /= 2) {
    float nv[256];
    for (int t = 0; t < L; ++t) nv[t] = lane[t] + lane[t ^ off];
    memcpy(lane, nv, sizeof(float) * L);
  }
  return 1.0f / sqrtf(lane[0] / (float)D + eps);
}

static void norm_rope_head(const o_bf16* src, const o_bf16* wn, int D, int ROT, float eps,
                           const o_bf16* cs, const o_bf16* sn, o_bf16* dst) {
  float x[1024], v[1024];
  for (int d = 0; d < D; ++d) x[d] = o_bf2f(src[d]);
  const float inv = head_inv_rms(x, D, eps);
  for (int d = 0; d < D; ++d) v[d] = o_round_bf(o_bf2f(wn[d]) * o_round_bf(x[d] * inv));
  const int half = ROT / 2;
  for (int d = 0; d < D; ++d) {
    float o = v[d];
    if (d < ROT) {
      const float c = o_bf2f(cs[d]), s = o_bf2f(sn[d]);
      if (d < half) {
        const float t1 = o_round_bf(v[d] * c);
        const float t2 = o_round_bf(-v[d + half] * s);
        o = o_round_bf(t1 + t2);
      } else {
        const float t1 = o_round_bf(v[d] * c);
        const float t2 = o_round_bf(v[d - half] * s);
        o = o_round_bf(t1 + t2);
      }
    }
    dst[d] = o_f2bf(o);
  }
}

/* qkv rows [S, QW] = q(HQ*D) | gate(HQ*D) | k(HK*D) | v(HK*D) | ...
 * -> q [S, HQ, D], k [S, HK, D], v [S, HK, D]; row s uses rope position pos0+s. */
void o_attn_prep(const o_bf16* qkv, int S, int QW, int HQ, int HK, int D, int ROT,
                 const o_bf16* qnorm, const o_bf16* knorm, float eps, const o_bf16* cos_t,
                 const o_bf16* sin_t, int pos0, o_bf16* q, o_bf16* k, o_bf16* v) {
  for (int s = 0; s < S; ++s) {
    const o_bf16* row = qkv + (int64_t)s * QW;
    const o_bf16* cs = cos_t + (int64_t)(pos0 + s) * ROT;
    const o_bf16* sn = sin_t + (int64_t)(pos0 + s) * ROT;
    for (int h = 0; h < HQ; ++h)
      norm_rope_head(row + h * D, qnorm, D, ROT, eps, cs, sn, q + ((int64_t)s * HQ + h) * D);
    for (int h = 0; h < HK; ++h) {
      norm_rope_head(row + 2 * HQ * D + h * D, knorm, D, ROT, eps, cs, sn,
                     k + ((int64_t)s * HK + h) * D);
      memcpy(v + ((int64_t)s * HK + h) * D, row + 2 * HQ * D + HK * D + h * D,
             sizeof(o_bf16) * D);
    }
  }
}

/* ======================================================================== */
/* a14: verify attention over a contiguous KV cache                          */
/* (MLX/backend/metal/kernels/sdpa_vector.h:14-175: f32 online softmax,      */
/* causal rule key i visible to query s iff i <= T - S + s, GQA HQ/HK).      */
/* Order: keys split into chunks of `chunk`; per (head, query, chunk):       */
/*   score_i = sequential fmaf over d of (scale*q_d) * k_d from 0.0f         */
/*   m_c = max score; e_i = exp(score_i - m_c); l_c = sum e_i (key order);   */
/*   o_c[d] = sum_i fmaf(e_i, v_i[d], .) (key order)                         */
/* then over visible chunks in order: M = max m_c; f_c = exp(m_c - M);       */
/*   L = fmaf(l_c, f_c, L); O[d] = fmaf(o_c[d], f_c, O[d]); out = bf16(O/L). */
/* kc/vc layout [HK, tmax, D].                                               */
/* ======================================================================== */

void o_attn_verify(const o_bf16* q, int S, int HQ, int HK, int D, const o_bf16* kc,
                   const o_bf16* vc, int64_t tmax, int T, float scale, int chunk,
                   o_bf16* out) {
  const int G = HQ / HK;
  const int nch = (T + chunk - 1) / chunk;
  float* oc = (float*)malloc(sizeof(float) * (size_t)nch * D);
  float* mc = (float*)malloc(sizeof(float) * (size_t)nch);
  float* lc = (float*)malloc(sizeof(float) * (size_t)nch);
  float qs[1024];
  for (int s = 0; s < S; ++s)
    for (int h = 0; h < HQ; ++h) {
      const int hk = h / G;
      const o_bf16* qh = q + ((int64_t)s * HQ + h) * D;
      for (int d = 0; d < D; ++d) qs[d] = scale * o_bf2f(qh[d]);
      const int last = T - S + s; /* last visible key */
      for (int c = 0; c < nch; ++c) {
        const int i0 = c * chunk;
        int i1 = i0 + chunk;
        if (i1 > last + 1) i1 = last + 1;
        float sc[4096];
        float mx = -INFINITY;
        int n = 0;
        for (int i = i0; i < i1; ++i) {
          const o_bf16* kr = kc + ((int64_t)hk * tmax + i) * D;
          float acc = 0.0f;
          for (int d = 0; d < D; ++d) acc = fmaf(qs[d], o_bf2f(kr[d]), acc);
          sc[i - i0] = acc;
          if (acc > mx) mx = acc;
          ++n;
        }
        mc[c] = mx;
        float l = 0.0f;
        float* o = oc + (int64_t)c * D;
        for (int d = 0; d < D; ++d) o[d] = 0.0f;
        for (int i = i0; i < i0 + n; ++i) {
          const float e = o_expf(sc[i - i0] - mx);
          l = l + e;
          const o_bf16* vr = vc + ((int64_t)hk * tmax + i) * D;
          for (int d = 0; d < D; ++d) o[d] = fmaf(e, o_bf2f(vr[d]), o[d]);
        }
        lc[c] = (n > 0) ? l : 0.0f;
        if (n == 0) mc[c] = -INFINITY;
      }
      float M = -INFINITY;
      for (int c = 0; c < nch; ++c)
        if (lc[c] > 0.0f && mc[c] > M) M = mc[c];
      float L = 0.0f;
      float O[1024];
      for (int d = 0; d < D; ++d) O[d] = 0.0f;
      for (int c = 0; c < nch; ++c) {
        if (!(lc[c] > 0.0f)) continue;
        const float f = o_expf(mc[c] - M);
        L = fmaf(lc[c], f, L);
        for (int d = 0; d < D; ++d) O[d] = fmaf(oc[(int64_t)c * D + d], f, O[d]);
      }
      o_bf16* dst = out + ((int64_t)s * HQ + h) * D;
      for (int d = 0; d < D; ++d) dst[d] = o_f2bf(O[d] / L);
    }
  free(oc);
  free(mc);
  free(lc);
}

/* a15: out[s, j] = bf16(att[s, j] * sigmoid_bf16(gate[s, j]))
 * (FM/TrackFastKernels2.swift:478-510); att [S, width], gate = qkv[s, gate_off + j]. */
void o_attn_gate(const o_bf16* att, const o_bf16* qkv, int S, int QW, int gate_off, int width,
                 o_bf16* out) {
  for (int s = 0; s < S; ++s)
    for (int j = 0; j < width; ++j) {
      const float a = o_bf2f(att[(int64_t)s * width + j]);
      const float g = o_bf2f(qkv[(int64_t)s * QW + gate_off + j]);
      out[(int64_t)s * width + j] = o_f2bf(a * o_sigmoid_bf16(g));
    }
}

/* Row RMSNorm used around the decoder sublayers: 256 lanes, lane t squares
 * elements t, t+256, ... (acc = fmaf(x, x, acc)); the four 64-lane waves fold
 * by xor butterfly; total = ((w0 + w1) + w2) + w3.
 * y = bf16(w * bf16(x * (1 / sqrtf(total / H + eps)))). */
static float block_sum256(const float* lanes256) {
  float w[4];
  for (int wv = 0; wv < 4; ++wv) {
    float lane[64];
    memcpy(lane, lanes256 + wv * 64, sizeof(lane));
    for (int off = 32; off >= 1; off /= 2) {
      float nv[64];
      for (int l = 0; l < 64; ++l) nv[l] = lane[l] + lane[l ^ off];
      memcpy(lane, nv, sizeof(nv));
    }
    w[wv] = lane[0];
  }
  return ((w[0] + w[1]) + w[2]) + w[3];
}

void o_rmsnorm(const o_bf16* x, int M, int H, const o_bf16* w, float eps, o_bf16* y) {
  for (int m = 0; m < M; ++m) {
    const o_bf16* xr = x + (int64_t)m * H;
    float lanes[256];
    for (int t = 0; t < 256; ++t) {
      float acc = 0.0f;
      for (int i = t; i < H; i += 256) acc = fmaf(o_bf2f(xr[i]), o_bf2f(xr[i]), acc);
      lanes[t] = acc;
    }
    const float total = block_sum256(lanes);
    const float inv = 1.0f / sqrtf(total / (float)H + eps);
    for (int i = 0; i < H; ++i)
      y[(int64_t)m * H + i] = o_f2bf(o_bf2f(w[i]) * o_round_bf(o_bf2f(xr[i]) * inv));
  }
}

/* ======================================================================== */
/* a17: MTP head pieces                                                      */
/* ======================================================================== */

/* Rows of a q4 embedding table, dequantized with MLX's affine_dequantize
 * arithmetic in bf16: w = bf16(bf16(scale * q) + bias)
 * (MLX/backend/metal/kernels/quantized.h:3314-3372; the head reads the
 * target's embed_tokens, Runner/Qwen4ExpMTP.swift:111). */
void o_embed_rows(const uint32_t* wq, const o_bf16* scales, const o_bf16* biases, int H, int gs,
                  const int32_t* ids, int S, o_bf16* out) {
  for (int s = 0; s < S; ++s) {
    const int64_t r = ids[s];
    for (int k = 0; k < H; ++k) {
      const uint32_t q = (wq[r * (H / 8) + k / 8] >> (4 * (k % 8))) & 0xfu;
      const float sc = o_bf2f(scales[r * (H / gs) + k / gs]);
      const float bi = o_bf2f(biases[r * (H / gs) + k / gs]);
      out[(int64_t)s * H + k] = o_f2bf(o_round_bf(sc * (float)q) + bi);
    }
  }
}

/* Hyper-connection inject + group RMS norm (TrackFastKernels.injectNorm,
 * Runner/FastModel/TrackFastKernels2.swift:60-113).  Per row s and stream c:
 *   r = residual[s, c*H + d]   (tile: residual[s, d], one row for every stream)
 *   with out and inject: r = bf16(r + bf16(out[s,d] * inject[s,c]))
 *   with out only      : r = bf16(r + out[s,d])   (the head's embedding add,
 *                        Runner/Qwen4ExpMTP.swift:111-115)
 *   stream = r; group sum of squares in the 256-lane order of o_rmsnorm;
 *   normed = bf16(scale[c*H+d] * bf16(r * inv)), inv = 1/sqrt(sum/H + eps). */
void o_hc_norm(const o_bf16* residual, const o_bf16* out, const o_bf16* inject, int S, int hc,
               int H, int tile, const o_bf16* scale, float eps, o_bf16* stream, o_bf16* normed) {
  const int64_t W = (int64_t)hc * H;
  float* r = (float*)malloc(sizeof(float) * (size_t)H);
  for (int s = 0; s < S; ++s)
    for (int c = 0; c < hc; ++c) {
      const int64_t base = s * W + (int64_t)c * H;
      for (int d = 0; d < H; ++d) {
        float v = o_bf2f(residual[tile ? (int64_t)s * H + d : base + d]);
        if (out && inject)
          v = o_round_bf(v + o_round_bf(o_bf2f(out[(int64_t)s * H + d]) * o_bf2f(inject[(int64_t)s * hc + c])));
        else if (out)
          v = o_round_bf(v + o_bf2f(out[(int64_t)s * H + d]));
        r[d] = v;
        stream[base + d] = o_f2bf(v);
      }
      float lanes[256];
      for (int t = 0; t < 256; ++t) {
        float acc = 0.0f;
        for (int d = t; d < H; d += 256) acc = fmaf(r[d], r[d], acc);
        lanes[t] = acc;
      }
      const float inv = 1.0f / sqrtf(block_sum256(lanes) / (float)H + eps);
      for (int d = 0; d < H; ++d)
        normed[base + d] = o_f2bf(o_bf2f(scale[(int64_t)c * H + d]) * o_round_bf(r[d] * inv));
    }
  free(r);
}

void o_silu_rows(const o_bf16* x, int64_t n, o_bf16* y) {
  for (int64_t i = 0; i < n; ++i) y[i] = o_f2bf(o_silu_bf16(o_bf2f(x[i])));
}

/* Mixer combine (TrackFastKernels.hcMix / TrackFastMixerKernels.upMix,
 * Runner/FastModel/TrackFastKernels2.swift:229-280, TrackFastMixer.swift:125-180):
 *   input[s,d] = bf16 running sum over c = 0..hc-1 of
 *                bf16(sigmoid_bf16(w[s, c*H+d]) * normed[s, c*H+d])
 *   inject_out[s,c] = bf16(2 * sigmoid_bf16(inj[s,c]))   (when inj != NULL) */
void o_hc_mix(const o_bf16* w, const o_bf16* normed, const o_bf16* inj, int S, int hc, int H,
              o_bf16* input, o_bf16* inject_out) {
  const int64_t W = (int64_t)hc * H;
  for (int s = 0; s < S; ++s) {
    for (int d = 0; d < H; ++d) {
      float acc = 0.0f;
      for (int c = 0; c < hc; ++c) {
        const int64_t i = s * W + (int64_t)c * H + d;
        const float p = o_round_bf(o_sigmoid_bf16(o_bf2f(w[i])) * o_bf2f(normed[i]));
        acc = o_round_bf(acc + p);
      }
      input[(int64_t)s * H + d] = o_f2bf(acc);
    }
    if (inj && inject_out)
      for (int c = 0; c < hc; ++c)
        inject_out[(int64_t)s * hc + c] = o_f2bf(2.0f * o_sigmoid_bf16(o_bf2f(inj[(int64_t)s * hc + c])));
  }
}

/* ======================================================================== */
/* a18 / a21: argmax and greedy acceptance                                   */
/* Tie rule: the lowest id (Runner/Qwen4ExpMTPDrafter.swift:25-27).          */
/* Accept rule (docs/qwen38-125b-a6b-port-notes.md:313-327): a_i = argmax of  */
/* verify row i; n = longest prefix with drafts[i] == a_i; commit            */
/* d_1..d_n then a_n; KV rollback index = kv_offset + n + 1 (pending + n).    */
/* out3 = {n, bonus token, kv index}.                                        */
/* ======================================================================== */

/* MLX's argmax (MLX/backend/metal/kernels/arg_reduce.metal:42-62): starting from (index 0,
 * -inf), an element replaces the best only when strictly greater, so a NaN never wins (it
 * compares false), equal values keep the lowest index, and a row of only -inf / NaN gives 0. */
void o_argmax_rows(const float* x, int rows, int64_t V, int32_t* out) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (int64_t)r * V;
    int64_t b = 0;
    float bv = -INFINITY;
    for (int64_t v = 0; v < V; ++v)
      if (xr[v] > bv) {
        bv = xr[v];
        b = v;
      }
    out[r] = (int32_t)b;
  }
}

/* Top two of each row in the argmax order (value descending, lowest index among equal values,
 * NaN as -inf): ids[2r] = the argmax, ids[2r+1] = the argmax of the row without it; values are
 * the entries (NaN reported as -inf).  V >= 2. */
void o_top2_rows(const float* x, int rows, int64_t V, int32_t* ids, float* vals) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (int64_t)r * V;
    int64_t b[2] = {-1, -1};
    for (int j = 0; j < 2; ++j) {
      float bv = 0.0f;
      for (int64_t v = 0; v < V; ++v) {
        if (v == b[0]) continue;
        const float xv = isnan(xr[v]) ? -INFINITY : xr[v];
        if (b[j] < 0 || xv > bv) {
          bv = xv;
          b[j] = v;
        }
      }
      ids[2 * r + j] = (int32_t)b[j];
      vals[2 * r + j] = bv;
    }
  }
}

void o_accept_greedy(const float* logits, int k, int64_t V, const int32_t* drafts,
                     int32_t kv_offset, int32_t* out3) {
  int32_t a[64];
  o_argmax_rows(logits, k + 1, V, a);
  int n = 0;
  while (n < k && drafts[n] == a[n]) ++n;
  out3[0] = n;
  out3[1] = a[n];
  out3[2] = kv_offset + n + 1;
}

/* ======================================================================== */
/* a22: temperature rejection sampling (Leviathan et al. 2023, Chen et al.   */
/* 2023) with Philox4x32-10 (Salmon et al., SC'11).  No counterpart in the   */
/* reference (it is greedy only).                                            */
/* ======================================================================== */

void o_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

/* top 24 bits -> [0, 1) exactly */
float o_uniform(uint32_t r) { return (float)(r >> 8) * 5.9604644775390625e-08f; }

#define O_CHUNK 1024
/* Chunk sum: 64 lanes, lane l adds elements base+l, base+l+64, ... (16 per
 * lane) in order from 0.0f; then an xor butterfly over 64 lanes. */
static float chunk_sum(const float* v, int64_t base, int64_t V) {
  float lane[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int j = 0; j < O_CHUNK / 64; ++j) {
      const int64_t i = base + l + 64 * j;
      if (i < V) acc = acc + v[i];
    }
    lane[l] = acc;
  }
  for (int off = 32; off >= 1; off /= 2) {
    float nv[64];
    for (int l = 0; l < 64; ++l) nv[l] = lane[l] + lane[l ^ off];
    memcpy(lane, nv, sizeof(nv));
  }
  return lane[0];
}

/* Row total: chunk sums added in chunk order from 0.0f. */
float o_softmax_row_sum(const float* e, int64_t V) {
  float t = 0.0f;
  for (int64_t b = 0; b < V; b += O_CHUNK) t = t + chunk_sum(e, b, V);
  return t;
}

/* Inverse CDF over non-negative vals: tau = u * total; pick the first chunk
 * whose running sum passes tau, then scan that chunk in index order against
 * tau - (sum before the chunk).  If rounding lets the scan run off the chunk,
 * return the chunk's last positive entry; if no chunk passes, the last
 * positive entry overall; if every entry is 0, -1. */
static int64_t icdf(const float* vals, int64_t V, float u) {
  const int64_t nc = (V + O_CHUNK - 1) / O_CHUNK;
  float* S = (float*)malloc(sizeof(float) * (size_t)nc);
  float total = 0.0f;
  for (int64_t c = 0; c < nc; ++c) {
    S[c] = chunk_sum(vals, c * O_CHUNK, V);
    total = total + S[c];
  }
  const float tau = u * total;
  float cum = 0.0f;
  int64_t res = -1;
  for (int64_t c = 0; c < nc && res < 0; ++c) {
    const float nxt = cum + S[c];
    if (nxt > tau) {
      const float t2 = tau - cum;
      float run = 0.0f;
      const int64_t b = c * O_CHUNK;
      const int64_t e = (b + O_CHUNK < V) ? b + O_CHUNK : V;
      for (int64_t i = b; i < e; ++i) {
        run = run + vals[i];
        if (run > t2) {
          res = i;
          break;
        }
      }
      if (res < 0)
        for (int64_t i = e - 1; i >= b; --i)
          if (vals[i] > 0.0f) {
            res = i;
            break;
          }
    }
    cum = nxt;
  }
  if (res < 0)
    for (int64_t i = V - 1; i >= 0; --i)
      if (vals[i] > 0.0f) {
        res = i;
        break;
      }
  free(S);
  return res;
}

/* Softmax at temperature: e_v = exp((l_v - max) * (1/T)); p_v = e_v * (1/Z). */
static void row_probs(const float* l, int64_t V, float invT, float* p) {
  float mx = -INFINITY; /* the row's argmax value: NaN never taken */
  for (int64_t v = 0; v < V; ++v)
    if (l[v] > mx) mx = l[v];
  for (int64_t v = 0; v < V; ++v) p[v] = o_expf((l[v] - mx) * invT);
  const float invZ = 1.0f / o_softmax_row_sum(p, V);
  for (int64_t v = 0; v < V; ++v) p[v] = p[v] * invZ;
}

/* tlogits [k+1, V]: verify rows; dlogits [k, V]: the draft distribution that
 * proposed drafts[i] is row i, or NULL: one-hot draft distributions at the
 * drafts (a greedy drafter: p_d(v) = [v == d_i]).  For i = 1..k (counter {offset lo, offset hi,
 * i, 0}, key {seed lo, seed hi}): u = U(word0), u2 = U(word1); accept draft i
 * iff u * p_d(d_i) < p_t(d_i) (p_t from verify row i-1).  First rejection at
 * i: token = icdf(max(0, p_t - p_d), u2) over row i-1, n = i-1.  All
 * accepted: n = k, token = icdf(p_t row k, u2 of counter i = k+1).
 * out3 = {n, token, kv_offset + n + 1}. */
void o_accept_sample(const float* tlogits, const float* dlogits, int k, int64_t V,
                     const int32_t* drafts, float temperature, uint64_t seed, uint64_t offset,
                     int32_t kv_offset, int32_t* out3) {
  const float invT = 1.0f / temperature;
  float* pt = (float*)malloc(sizeof(float) * (size_t)V);
  float* pd = (float*)malloc(sizeof(float) * (size_t)V);
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  int n = 0;
  int64_t tok = -1;
  for (int i = 1; i <= k + 1; ++i) {
    uint32_t ctr[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), (uint32_t)i, 0u};
    uint32_t rnd[4];
    o_philox4x32_10(ctr, key, rnd);
    const float u = o_uniform(rnd[0]), u2 = o_uniform(rnd[1]);
    row_probs(tlogits + (int64_t)(i - 1) * V, V, invT, pt);
    if (i == k + 1) {
      n = k;
      tok = icdf(pt, V, u2);
      if (tok < 0) {
        int32_t a;
        o_argmax_rows(tlogits + (int64_t)k * V, 1, V, &a);
        tok = a;
      }
      break;
    }
    const int32_t d = drafts[i - 1];
    /* a draft id outside the vocabulary is rejected */
    const int ok = d >= 0 && d < V;
    if (dlogits) {
      row_probs(dlogits + (int64_t)(i - 1) * V, V, invT, pd);
    } else {
      for (int64_t v = 0; v < V; ++v) pd[v] = 0.0f;
      if (ok) pd[d] = 1.0f;
    }
    if (ok && u * pd[d] < pt[d]) continue;
    n = i - 1;
    for (int64_t v = 0; v < V; ++v) pd[v] = fmaxf(pt[v] - pd[v], 0.0f);
    tok = icdf(pd, V, u2);
    if (tok < 0) {
      int32_t a;
      o_argmax_rows(tlogits + (int64_t)(i - 1) * V, 1, V, &a);
      tok = a;
    }
    break;
  }
  out3[0] = n;
  out3[1] = (int32_t)tok;
  out3[2] = kv_offset + n + 1;
  free(pt);
  free(pd);
}

/* ======================================================================== */
/* a20: the gated-deltanet (GDN) sublayer of the target                     */
/* Runner/FastModel/TrackFastKernels.swift:48-117 (prep), :148-208 and      */
/* :486-605 (recurrence, peeled Kahan form), TrackFastKernels2.swift:325-352 */
/* (gated RMS), TrackFastModel.swift:404-432,655-737 (binding, forward).     */
/* Every 128-channel reduction is 32 lanes x 4 consecutive elements, each    */
/* lane in element order, then an xor butterfly over the 32 lanes.           */
/* ======================================================================== */

/* log1p(y) for y in [0, 1]: 2 atanh(s), s = y / (2 + y) <= 1/3, odd series to
 * s^15 in Horner form (truncation < 4e-9 relative).  The build's own, so host
 * and device agree bit for bit. */
float o_log1p_det(float y) {
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

/* MLX logaddexp(x, 0) in bf16 arithmetic (TrackFastKernels2.swift:48-58):
 * max + log1p(exp(min - max)), each op rounded to bf16. */
float o_logaddexp0_bf16(float x) {
  if (x != x) return x;
  const float inf = f_from_bits(0x7f800000u);
  const float mx = x > 0.0f ? x : 0.0f;
  const float mn = x < 0.0f ? x : 0.0f;
  if (mn == -inf || mx == inf) return mx;
  const float d = o_round_bf(mn - mx);
  const float e = o_round_bf(o_expf(d));
  const float l = o_round_bf(o_log1p_det(e));
  return o_round_bf(mx + l);
}

/* MLX Sigmoid functor in f32: y = 1/(1+exp(|x|)); x < 0 ? y : 1 - y. */
float o_sigmoid_f32(float x) {
  const float e = o_expf(fabsf(x));
  const float y = 1.0f / (1.0f + e);
  return (x < 0.0f) ? y : 1.0f - y;
}

static float bfly32(const float* lanes) {
  float v[32];
  memcpy(v, lanes, sizeof(v));
  for (int off = 16; off >= 1; off /= 2) {
    float n[32];
    for (int l = 0; l < 32; ++l) n[l] = v[l] + v[l ^ off];
    memcpy(v, n, sizeof(v));
  }
  return v[0];
}

/* One position of the prep.  conv_state: the KC-1 previous conv input rows
 * [KC-1][conv_dim]; prow: this position's projection row [proj_w].
 *   conv  = sum_j win_j * w[ch][j] (f32, j = 0..KC-1, mul then add)
 *   x     = silu_bf16(bf16(conv))
 *   q/k heads: inv = 1/sqrt(sum x^2 / 128 + 1e-6); n = bf16(x * inv);
 *              q = bf16(bf16(1/Dk) * n), k = bf16(bf16(1/sqrt(Dk)) * n)
 *   v heads:   v = x
 *   beta  = sigmoid_bf16(b);  decay = exp(-exp(A_log) * softplus_bf16(bf16(a + dt_bias))) */
void o_gdn_prep(const o_gdn_geom* g, const o_bf16* conv_state, const o_bf16* prow, const o_bf16* conv_w,
                const float* neg_exp_alog, const o_bf16* dt_bias, o_bf16* q, o_bf16* k, o_bf16* v,
                float* decay, float* beta) {
  const int KM1 = g->kc - 1, CD = g->conv_dim, D = 128;
  const int nvec = 2 * g->hk + g->hv;
  const float inv_scale = 1.0f / sqrtf((float)g->dk);
  const float q_mul = o_round_bf(inv_scale * inv_scale);
  const float k_mul = o_round_bf(inv_scale);
  for (int vec = 0; vec < nvec; ++vec) {
    float xs[128], lanes[32];
    for (int l = 0; l < 32; ++l) {
      float acc = 0.0f;
      for (int i = 0; i < 4; ++i) {
        const int ch = vec * D + l * 4 + i;
        float c = 0.0f;
        for (int j = 0; j < g->kc; ++j) {
          const float win = j < KM1 ? o_bf2f(conv_state[(int64_t)j * CD + ch]) : o_bf2f(prow[ch]);
          c = c + win * o_bf2f(conv_w[(int64_t)ch * g->kc + j]);
        }
        const float x = o_silu_bf16(o_round_bf(c));
        xs[l * 4 + i] = x;
        acc = fmaf(x, x, acc);
      }
      lanes[l] = acc;
    }
    if (vec < 2 * g->hk) {
      const float inv = 1.0f / sqrtf(bfly32(lanes) / 128.0f + 1e-6f);
      const float mul = vec < g->hk ? q_mul : k_mul;
      o_bf16* dst = vec < g->hk ? q + (int64_t)vec * D : k + (int64_t)(vec - g->hk) * D;
      for (int d = 0; d < D; ++d) dst[d] = o_f2bf(mul * o_round_bf(xs[d] * inv));
    } else {
      o_bf16* dst = v + (int64_t)(vec - 2 * g->hk) * D;
      for (int d = 0; d < D; ++d) dst[d] = o_f2bf(xs[d]);
    }
  }
  for (int h = 0; h < g->hv; ++h) {
    beta[h] = o_sigmoid_bf16(o_bf2f(prow[g->b_off + h]));
    const float ax = o_round_bf(o_bf2f(prow[g->a_off + h]) + o_bf2f(dt_bias[h]));
    decay[h] = o_expf(neg_exp_alog[h] * o_logaddexp0_bf16(ax));
  }
}

/* One position of the delta rule for every (value head, value row), in place
 * on ssm [hv][dv][dk] (f32); y [hv][dv] bf16; delta_out [hv][dv] (may be NULL):
 *   s *= decay; kv = Kahan sum of s*k (lane-peeled: i = 0 plain, i = 1..3
 *   compensated, last compensation dropped), butterfly;
 *   delta = (v - kv) * beta; s = fmaf(k, delta, s); out = sum fmaf(s, q, out). */
void o_gdn_step(const o_gdn_geom* g, float* ssm, const o_bf16* q, const o_bf16* k, const o_bf16* v,
                const float* decay, const float* beta, o_bf16* y, float* delta_out) {
  const int ratio = g->hv / g->hk, D = 128;
  for (int h = 0; h < g->hv; ++h) {
    const o_bf16* qh = q + (int64_t)(h / ratio) * D;
    const o_bf16* kh = k + (int64_t)(h / ratio) * D;
    const float gd = decay[h], bt = beta[h];
    for (int r = 0; r < D; ++r) {
      float* s = ssm + ((int64_t)h * D + r) * D;
      float kvl[32], ol[32];
      for (int l = 0; l < 32; ++l) {
        float* sl = s + 4 * l;
        const o_bf16* kl = kh + 4 * l;
        sl[0] = sl[0] * gd;
        float kv = 0.0f + sl[0] * o_bf2f(kl[0]);
        float comp = 0.0f;
        for (int i = 1; i < 4; ++i) {
          sl[i] = sl[i] * gd;
          const float prod = sl[i] * o_bf2f(kl[i]);
          const float corr = prod - comp;
          const float next = kv + corr;
          if (i + 1 < 4) comp = (next - kv) - corr;
          kv = next;
        }
        kvl[l] = kv;
      }
      const float kvm = bfly32(kvl);
      const float delta = (o_bf2f(v[(int64_t)h * D + r]) - kvm) * bt;
      if (delta_out) delta_out[(int64_t)h * D + r] = delta;
      for (int l = 0; l < 32; ++l) {
        float o = 0.0f;
        for (int i = 0; i < 4; ++i) {
          const int d = 4 * l + i;
          s[d] = fmaf(o_bf2f(kh[d]), delta, s[d]);
          o = fmaf(s[d], o_bf2f(qh[d]), o);
        }
        ol[l] = o;
      }
      y[(int64_t)h * D + r] = o_f2bf(bfly32(ol));
    }
  }
}

/* Gated RMS of one position (TrackFastKernels2.swift:325-352):
 *   inv = 1/sqrt(sum y^2 / 128 + eps); n = bf16(w * bf16(y * inv));
 *   out = bf16(sigmoid_f32(z) * n). */
void o_gdn_gated_rms(const o_gdn_geom* g, const o_bf16* y, const o_bf16* z, const o_bf16* w, float eps,
                     o_bf16* out) {
  const int D = 128;
  for (int h = 0; h < g->hv; ++h) {
    const o_bf16* yh = y + (int64_t)h * D;
    float lanes[32];
    for (int l = 0; l < 32; ++l) {
      float acc = 0.0f;
      for (int i = 0; i < 4; ++i) {
        const float x = o_bf2f(yh[4 * l + i]);
        acc = fmaf(x, x, acc);
      }
      lanes[l] = acc;
    }
    const float inv = 1.0f / sqrtf(bfly32(lanes) / 128.0f + eps);
    for (int d = 0; d < D; ++d) {
      const float n = o_round_bf(o_bf2f(w[d]) * o_round_bf(o_bf2f(yh[d]) * inv));
      out[(int64_t)h * D + d] = o_f2bf(o_sigmoid_f32(o_bf2f(z[(int64_t)h * D + d])) * n);
    }
  }
}

/* S positions of the GDN core in order: prep, step, gated RMS; conv_state
 * [KC-1][conv_dim] and ssm advance by S.  proj [S][proj_w] -> gated [S][hv*128];
 * optional per-position outputs (NULL to skip): q,k [S][hk*128], v,y [S][hv*128],
 * decay, beta [S][hv], delta [S][hv*128]. */
void o_gdn_core(const o_gdn_geom* g, const o_bf16* proj, int S, o_bf16* conv_state, float* ssm,
                const o_bf16* conv_w, const float* neg_exp_alog, const o_bf16* dt_bias, const o_bf16* norm_w,
                float eps, o_bf16* gated, o_bf16* q_out, o_bf16* k_out, o_bf16* v_out, o_bf16* y_out,
                float* decay_out, float* beta_out, float* delta_out) {
  const int KM1 = g->kc - 1, CD = g->conv_dim, D = 128;
  o_bf16* q = (o_bf16*)malloc(sizeof(o_bf16) * (size_t)g->hk * D);
  o_bf16* k = (o_bf16*)malloc(sizeof(o_bf16) * (size_t)g->hk * D);
  o_bf16* v = (o_bf16*)malloc(sizeof(o_bf16) * (size_t)g->hv * D);
  o_bf16* y = (o_bf16*)malloc(sizeof(o_bf16) * (size_t)g->hv * D);
  float* dec = (float*)malloc(sizeof(float) * (size_t)g->hv);
  float* bet = (float*)malloc(sizeof(float) * (size_t)g->hv);
  for (int t = 0; t < S; ++t) {
    const o_bf16* prow = proj + (int64_t)t * g->proj_w;
    o_gdn_prep(g, conv_state, prow, conv_w, neg_exp_alog, dt_bias, q, k, v, dec, bet);
    o_gdn_step(g, ssm, q, k, v, dec, bet, y, delta_out ? delta_out + (int64_t)t * g->hv * D : NULL);
    o_gdn_gated_rms(g, y, prow + g->z_off, norm_w, eps, gated + (int64_t)t * g->hv * D);
    /* conv tail: drop the oldest row, append this position's conv input */
    for (int j = 0; j + 1 < KM1; ++j) memcpy(conv_state + (int64_t)j * CD, conv_state + (int64_t)(j + 1) * CD, 2 * (size_t)CD);
    if (KM1 > 0) memcpy(conv_state + (int64_t)(KM1 - 1) * CD, prow, 2 * (size_t)CD);
    if (q_out) memcpy(q_out + (int64_t)t * g->hk * D, q, 2 * (size_t)g->hk * D);
    if (k_out) memcpy(k_out + (int64_t)t * g->hk * D, k, 2 * (size_t)g->hk * D);
    if (v_out) memcpy(v_out + (int64_t)t * g->hv * D, v, 2 * (size_t)g->hv * D);
    if (y_out) memcpy(y_out + (int64_t)t * g->hv * D, y, 2 * (size_t)g->hv * D);
    if (decay_out) memcpy(decay_out + (int64_t)t * g->hv, dec, 4 * (size_t)g->hv);
    if (beta_out) memcpy(beta_out + (int64_t)t * g->hv, bet, 4 * (size_t)g->hv);
  }
  free(q);
  free(k);
  free(v);
  free(y);
  free(dec);
  free(bet);
}

/* ======================================================================== */
/* PLE n-gram block (layer index 1 of the target)                            */
/* ======================================================================== */

/* Row ids of the n-gram table for the last S positions of a token history
 * (docs/ngram-cache-design.md:47-96, the hash the reference's host row source
 * computes at FM/TrackFastModel.swift:1036-1060):
 *   history [ctx_len + S]: the carried context, then the window's tokens;
 *   copy p (p = 0..ngram_size-1) of position u is history[u-p], or eos when an
 *   eos token lies strictly between u-p and u (a shift never crosses an eos);
 *   width n = 2..ngram_size: mix = XOR_{p<n} copy_p * mult[p] (64-bit);
 *   head h of width n (global head (n-2)*heads_per_ngram + h):
 *   id = mix % vocab[head] + offset[head].
 * out [S][(ngram_size-1)*heads_per_ngram]; an id outside [0, rows) -> -1.
 * Parity: the prime rule for vocab[] is pinned by the design note's row total;
 * the eos-barrier extent and the head order are restated from the note's
 * prose (the fork's hash and its tests are absent): parity unpinned. */
void o_ngram_row_ids(const int32_t* history, int ctx_len, int S, int ngram_size, int heads_per_ngram,
                     const int64_t* mult, const int64_t* vocab, const int64_t* offs, int64_t rows, int32_t eos,
                     int32_t* out) {
  const int nh = (ngram_size - 1) * heads_per_ngram;
  for (int i = 0; i < S; ++i) {
    const int u = ctx_len + i;
    int64_t copy[16];
    int crossed = 0;
    for (int p = 0; p < ngram_size; ++p) {
      if (p >= 2 && history[u - p + 1] == eos) crossed = 1; /* eos at u-1 .. u-p+1 */
      copy[p] = crossed ? (int64_t)eos : (int64_t)history[u - p];
    }
    for (int n = 2; n <= ngram_size; ++n) {
      uint64_t mix = 0;
      for (int p = 0; p < n; ++p) mix ^= (uint64_t)copy[p] * (uint64_t)mult[p];
      for (int h = 0; h < heads_per_ngram; ++h) {
        const int hd = (n - 2) * heads_per_ngram + h;
        const int64_t m = (int64_t)mix;
        const int64_t id = m % vocab[hd] + offs[hd];
        out[(int64_t)i * nh + hd] = (id >= 0 && id < rows) ? (int32_t)id : -1;
      }
    }
  }
}

/* The gate of one (position, stream) pair of the PLE block
 * (FM/TrackFastPLE.swift:60-220: track_ple_prod, MLX's sum, track_ple_gated),
 * in this build's evaluation order.  H % 128 == 0, H <= 4096; lane l of H/4
 * owns elements 4l..4l+3, lanes form groups of 32 (NG = H/128):
 *   kacc = fmaf chain of k^2 over the lane's 4, bfly32 per group, bfly32 over
 *   the NG group sums (zero-padded to 32); kinv = 1/sqrt(kacc/H + eps); same q;
 *   kn = bf16(bf16(k*kinv) * kscale); qn = bf16(bf16(q*qinv) * qscale);
 *   p = bf16(kn*qn);
 *   dot: MLX's bf16 row sum -- per lane t = bf16(p_i + t) over its 4, then
 *   bf16(bfly32) per group, then bf16(bfly32) over the groups;
 *   g = bf16(dot / bf16(sqrt(H))); g = bf16(sqrt(max(|g|, bf16(1e-6)))) * sign(g);
 *   sgm = sigmoid_bf16(g); v = bf16(sgm * value);
 *   vacc as kacc over v; normed = bf16(bf16(v * vinv) * cscale).
 * key, stream, kscale, qscale, cscale, gated, normed: this pair's H elements;
 * value [H].  Returns the bf16 dot (as float). */
float o_ple_gate(const o_bf16* key, const o_bf16* stream, const o_bf16* value, const o_bf16* kscale,
                 const o_bf16* qscale, const o_bf16* cscale, int H, float eps, o_bf16* gated, o_bf16* normed) {
  const int NL = H / 4, NG = H / 128;
  float kl[1024], ql[1024], tl[1024], grp[32], gk[32], gq[32];
  for (int l = 0; l < NL; ++l) {
    float ka = 0.0f, qa = 0.0f;
    for (int i = 0; i < 4; ++i) {
      const float k = o_bf2f(key[4 * l + i]), q = o_bf2f(stream[4 * l + i]);
      ka = fmaf(k, k, ka);
      qa = fmaf(q, q, qa);
    }
    kl[l] = ka;
    ql[l] = qa;
  }
  for (int g = 0; g < 32; ++g) {
    gk[g] = g < NG ? bfly32(kl + 32 * g) : 0.0f;
    gq[g] = g < NG ? bfly32(ql + 32 * g) : 0.0f;
  }
  const float kinv = 1.0f / sqrtf(bfly32(gk) / (float)H + eps);
  const float qinv = 1.0f / sqrtf(bfly32(gq) / (float)H + eps);
  for (int l = 0; l < NL; ++l) {
    float t = 0.0f;
    for (int i = 0; i < 4; ++i) {
      const int d = 4 * l + i;
      const float kn = o_round_bf(o_round_bf(o_bf2f(key[d]) * kinv) * o_bf2f(kscale[d]));
      const float qn = o_round_bf(o_round_bf(o_bf2f(stream[d]) * qinv) * o_bf2f(qscale[d]));
      t = o_round_bf(o_round_bf(kn * qn) + t);
    }
    tl[l] = t;
  }
  for (int g = 0; g < 32; ++g) grp[g] = g < NG ? o_round_bf(bfly32(tl + 32 * g)) : 0.0f;
  const float dot = o_round_bf(bfly32(grp));
  const float divisor = o_round_bf(sqrtf((float)H));
  const float floor_v = o_round_bf(1e-6f);
  float g = o_round_bf(dot / divisor);
  const float a = fabsf(g);
  const float mx = isnan(a) ? a : (a > floor_v ? a : floor_v);
  const float sg = (float)((g > 0.0f) - (g < 0.0f));
  g = o_round_bf(o_round_bf(sqrtf(mx)) * sg);
  const float sgm = o_sigmoid_bf16(g);
  float vl[1024], gv[32];
  for (int l = 0; l < NL; ++l) {
    float va = 0.0f;
    for (int i = 0; i < 4; ++i) {
      const int d = 4 * l + i;
      const float v = o_round_bf(sgm * o_bf2f(value[d]));
      gated[d] = o_f2bf(v);
      va = fmaf(v, v, va);
    }
    vl[l] = va;
  }
  for (int q = 0; q < 32; ++q) gv[q] = q < NG ? bfly32(vl + 32 * q) : 0.0f;
  const float vinv = 1.0f / sqrtf(bfly32(gv) / (float)H + eps);
  for (int d = 0; d < H; ++d)
    normed[d] = o_f2bf(o_round_bf(o_bf2f(gated[d]) * vinv) * o_bf2f(cscale[d]));
  return dot;
}

/* The dilated depthwise conv, SiLU and gated add of the PLE block
 * (FM/TrackFastPLE.swift:222-262, track_ple_conv):
 *   full [nb + S][W] (carried rows, then the window's normed rows),
 *   nb = (kc-1)*dil; conv_w [W][kc]:
 *   acc = sum_j full[t + j*dil][c] * conv_w[c][j] (f32, j ascending, mul then add);
 *   out[t][c] = bf16(gated[t][c] + silu_bf16(bf16(acc))). */
void o_ple_conv(const o_bf16* full, const o_bf16* conv_w, const o_bf16* gated, int S, int64_t W, int kc, int dil,
                o_bf16* out) {
  for (int t = 0; t < S; ++t)
    for (int64_t c = 0; c < W; ++c) {
      float acc = 0.0f;
      for (int j = 0; j < kc; ++j) acc = acc + o_bf2f(full[(int64_t)(t + j * dil) * W + c]) * o_bf2f(conv_w[c * kc + j]);
      out[(int64_t)t * W + c] = o_f2bf(o_bf2f(gated[(int64_t)t * W + c]) + o_silu_bf16(o_round_bf(acc)));
    }
}

/* ======================================================================== */
/* Thread count of the oracle's row-parallel loops (o_qmv, o_router_gemv,   */
/* o_qmm_t_bf16).  The results do not depend on it.                          */
/* ======================================================================== */
#include <omp.h>

void o_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int o_get_threads(void) { return omp_get_max_threads(); }

/* ======================================================================== */
/* mlx_cpu mode: MLX's CPU quantized matmul with T = bfloat16               */
/* (MLX/backend/cpu/quantized.cpp:153-212, _qmm_t, 4 bits): per output a    */
/* bf16 running sum over K in element order, every operation rounded to     */
/* bf16 as MLX's _MLX_BFloat16 operators do (MLX/types/bf16.h:72-143):      */
/*   sum = bf16(sum + bf16(x * bf16(bf16(scale * q) + bias))).              */
/* Used only as the CPU timing baseline (its bits are not the GPU path's).  */
/* OpenMP over output rows when threads > 1 (MLX runs one thread per op).   */
/* ======================================================================== */
void o_qmm_t_bf16(const o_bf16* x, const uint32_t* wq, const o_bf16* scales, const o_bf16* biases,
                  int M, int64_t N, int K, int gs, o_bf16* y) {
  const int ng = K / gs;
  for (int m = 0; m < M; ++m) {
    const o_bf16* xm = x + (int64_t)m * K;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      const uint32_t* wr = wq + n * (K / 8);
      float sum = 0.0f;
      for (int g = 0; g < ng; ++g) {
        const float sc = o_bf2f(scales[n * ng + g]), bi = o_bf2f(biases[n * ng + g]);
        for (int k = g * gs; k < (g + 1) * gs; ++k) {
          const float q = (float)((wr[k / 8] >> (4 * (k % 8))) & 0xfu);
          const float wv = o_round_bf(o_round_bf(sc * q) + bi);
          sum = o_round_bf(sum + o_round_bf(o_bf2f(xm[k]) * wv));
        }
      }
      y[(int64_t)m * N + n] = o_f2bf(sum);
    }
  }
}
