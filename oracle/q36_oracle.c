/* CPU oracle for the qwen36 decode/verify kernel nodes -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's arithmetic, used as the checker for the HIP
 * kernels and timed as the CPU baseline.  Never linked into the product library.
 * Build: oracle/Makefile (gcc -O3 -march=native -fopenmp -ffp-contract=off).  Contraction
 * is off so that every fused multiply-add below is an explicit fmaf() and every other
 * product and sum is rounded on its own, exactly as the kernels spell them.
 *
 * Citations: R = /root/reference/qwen36_nodes_kb34, L = R/qwen36_layer, H = R/qwen36_lmhead8.
 */
#include "q36_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------ */
/* codecs                                                                               */
/* ------------------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t q36o_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float q36o_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }
static inline float bf(float f) { return q36o_bf16_to_f32(q36o_f32_to_bf16(f)); }

/* OCP e4m3fn: bias 7, 3 mantissa bits, max 448 (0x7e), NaN 0x7f/0xff, no inf.  Round to
 * nearest even, saturating like cvt.rn.satfinite.e4m3x2.f32 (L/qk_attn_verify.cu:142-145). */
uint8_t q36o_f32_to_e4m3(float f) {
  uint32_t u = f2u(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f);
  float af = u2f(a);
  if (af >= 448.f) return (uint8_t)(sign | 0x7e);
  if (af < 0.015625f) {               /* below 2^-6: subnormal grid m * 2^-9 */
    float m = rintf(af * 512.f);       /* exact scaling, RNE; m == 8 is 2^-6 = code 0x08 */
    return (uint8_t)(sign | (uint8_t)m);
  }
  int e = (int)((a >> 23) & 0xffu) - 127;
  uint32_t keep = (a & 0x7fffffu) >> 20, rest = a & 0xfffffu;
  if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) keep++;
  if (keep == 8u) { keep = 0; e++; }
  if (e > 8 || (e == 8 && keep > 6u)) return (uint8_t)(sign | 0x7e);
  return (uint8_t)(sign | (uint8_t)(((e + 7) << 3) | (int)keep));
}

float q36o_e4m3_to_f32(uint8_t b) {
  int e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7) v = NAN;
  else if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.f + (float)m * 0.125f, e - 7);
  return (b & 0x80) ? -v : v;
}

/* exp(x): Cody-Waite reduction x = n ln2 + r with ln2 split hi/lo, then the degree-7 Taylor
 * polynomial of e^r by Horner in fmaf, then ldexp.  Every step is a correctly rounded IEEE op,
 * so the HIP kernels' copy gives the same bits.  |error| < 2 ulp against libm (tested). */
float q36o_expf(float x) {
  if (x != x) return x;
  if (x > 88.7228394f) return INFINITY;
  if (x < -103.972084f) return 0.f;
  float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187e-06f, r);
  float p = 1.f / 5040.f;
  p = fmaf(p, r, 1.f / 720.f);
  p = fmaf(p, r, 1.f / 120.f);
  p = fmaf(p, r, 1.f / 24.f);
  p = fmaf(p, r, 1.f / 6.f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.f);
  p = fmaf(p, r, 1.f);
  return ldexpf(p, (int)n);
}
static inline float sigmoidf_q(float z) { return 1.f / (1.f + q36o_expf(-z)); }

/* 64 lane partials combined by an xor butterfly (offsets 32..1): the reduction tree a 64-wide
 * wavefront computes with v + shfl_xor(v, o).  Commutative adds make every lane's total equal. */
static float bfly64(float* p) {
  float q[64];
  for (int o = 32; o > 0; o >>= 1) {
    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ o];
    memcpy(p, q, sizeof(q));
  }
  return p[0];
}

/* Dot product in the fixed order the routing kernels use: lane l owns the 8-element chunks
 * c = l + 64 j (j = 0 .. n/512-1), accumulates them with fmaf from zero in (j, i) order, then
 * the 64 partials meet in bfly64.  n must be a multiple of 512.  (The reference fixes its own
 * order the same way: 4 K-quarters, ((p0+p1)+p2)+p3, L/qk_route.cu:3-4; an order-free spec
 * cannot be bit-exact in the bf16-rounded logits that decide the expert ids.) */
float q36o_dot_canon(const float* a, const float* b, int n) {
  float p[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.f;
    for (int j = 0; j < n / 512; ++j) {
      int c = l + 64 * j;
      for (int i = 0; i < 8; ++i) acc = fmaf(a[8 * c + i], b[8 * c + i], acc);
    }
    p[l] = acc;
  }
  return bfly64(p);
}

/* ------------------------------------------------------------------------------------ */
/* quantizers                                                                           */
/* ------------------------------------------------------------------------------------ */

/* Per-row symmetric int8 (H/w8a8.py:16-23 _round_int8; the weight twin H/lmhead8.py:95-108):
 * s = amax/127 (correctly rounded), q = clamp(round_half_away(x / (amax > 0 ? s : 1)), +-127). */
static void quant_row_i8(const float* x, int K, int8_t* q, float* s) {
  float amax = 0.f;
  for (int i = 0; i < K; ++i) amax = fmaxf(amax, fabsf(x[i]));
  float sc = amax / 127.f, safe = amax > 0.f ? sc : 1.f;
  for (int i = 0; i < K; ++i) {
    float v = x[i] / safe;
    float r = v >= 0.f ? floorf(v + 0.5f) : -floorf(0.5f - v);
    r = fminf(fmaxf(r, -127.f), 127.f);
    q[i] = (int8_t)r;
  }
  *s = sc;
}
void q36o_quant_rows_i8(const float* x, int rows, int K, int8_t* q, float* s) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) quant_row_i8(x + (size_t)r * K, K, q + (size_t)r * K, s + r);
}

/* Per-group e4m3 (the per-token x 128-channel rule of L/qk_moe_prefill_i8.cu:3671-3705 with 448
 * in place of 127): s = amax/448, inv = amax > 0 ? 448/amax : 0, q = e4m3_rn_sat(x * inv). */
static void quant_group_e4m3(const float* x, int n, int stride, int rows, uint8_t* q, int qstride,
                             float* s) {
  float amax = 0.f;
  for (int r = 0; r < rows; ++r)
    for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(x[(size_t)r * stride + i]));
  float sc = amax / 448.f, inv = amax > 0.f ? 448.f / amax : 0.f;
  for (int r = 0; r < rows; ++r)
    for (int i = 0; i < n; ++i) q[(size_t)r * qstride + i] = q36o_f32_to_e4m3(x[(size_t)r * stride + i] * inv);
  *s = sc;
}
void q36o_quant_groups_e4m3(const float* x, int rows, int K, int group, uint8_t* q, float* s) {
  int ng = K / group;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r)
    for (int g = 0; g < ng; ++g)
      quant_group_e4m3(x + (size_t)r * K + g * group, group, K, 1, q + (size_t)r * K + g * group, K,
                       s + (size_t)r * ng + g);
}
/* 128x128 block weights: the same rule over each block; s [N/128, K/128]. */
void q36o_quant_blocks_e4m3(const float* w, int N, int K, uint8_t* q, float* s) {
  int nb = N / 128, kb = K / 128;
#pragma omp parallel for collapse(2) schedule(static)
  for (int i = 0; i < nb; ++i)
    for (int j = 0; j < kb; ++j)
      quant_group_e4m3(w + (size_t)i * 128 * K + j * 128, 128, K, 128, q + (size_t)i * 128 * K + j * 128, K,
                       s + (size_t)i * kb + j);
}

/* ------------------------------------------------------------------------------------ */
/* prepare-time weight formats of the reference                                         */
/* ------------------------------------------------------------------------------------ */

uint16_t q36o_f32_to_f16(float f) {
  uint32_t u = f2u(f), sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);            /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);           /* >= 65520: rounds to inf */
  if (a < 0x38800000u) {                                             /* below 2^-14: subnormal grid 2^-24 */
    double q = (double)u2f(a) * 16777216.0, fl = floor(q), r = q - fl;
    if (r > 0.5 || (r == 0.5 && fmod(fl, 2.0) != 0.0)) fl += 1.0;
    return (uint16_t)(sign | (uint32_t)fl);                          /* 1024 is the smallest normal */
  }
  uint32_t keep = a >> 13, rest = a & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) keep++;
  return (uint16_t)(sign | (keep - ((127u - 15u) << 10)));
}
float q36o_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 0) return u2f(sign) + (sign ? -1.f : 1.f) * ldexpf((float)m, -24);
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* One row (or one 128-group) of n weights: the scale rule of L/i8x_kernels.py:119-131 and
 * L/dense8.py:153-166 (one fp16 ulp of headroom above amax / 127), codes rounded half away. */
static uint16_t quant_f16_scaled(const float* w, int n, int8_t* q) {
  float amax = 0.f;
  for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(w[i]));
  const uint16_t s16 = q36o_f32_to_f16((amax / 127.f) * 1.0009765625f);
  const float sc = q36o_f16_to_f32(s16), safe = sc > 0.f ? sc : 1.f;
  for (int i = 0; i < n; ++i) {
    float v = w[i] / safe;
    float r = v >= 0.f ? floorf(v + 0.5f) : -floorf(0.5f - v);
    q[i] = (int8_t)fminf(fmaxf(r, -127.f), 127.f);
  }
  return s16;
}

size_t q36o_q8_block_bytes(int H, int I) {
  return (size_t)2 * I * H + (size_t)H * I + (size_t)2 * I * (H / 128) * 2 + (size_t)H * (I / 128) * 2;
}

void q36o_quant_q8_block_v1(const float* w13, const float* w2, int E, int H, int I, int channel, uint8_t* blocks) {
  const size_t eb = q36o_q8_block_bytes(H, I), o2 = (size_t)2 * I * H, oc13 = o2 + (size_t)H * I,
               oc2 = oc13 + (size_t)2 * I * (H / 128) * 2;
#pragma omp parallel for schedule(static)
  for (int e = 0; e < E; ++e) {
    uint8_t* b = blocks + (size_t)e * eb;
    for (int part = 0; part < 2; ++part) {
      const int rows = part ? H : 2 * I, K = part ? I : H;
      const float* w = part ? w2 + (size_t)e * H * I : w13 + (size_t)e * 2 * I * H;
      int8_t* q = (int8_t*)(b + (part ? o2 : 0));
      uint16_t* c = (uint16_t*)(b + (part ? oc2 : oc13));
      for (int r = 0; r < rows; ++r) {
        if (channel) {
          const uint16_t s16 = quant_f16_scaled(w + (size_t)r * K, K, q + (size_t)r * K);
          for (int g = 0; g < K / 128; ++g) c[(size_t)r * (K / 128) + g] = s16;
        } else {
          for (int g = 0; g < K / 128; ++g)
            c[(size_t)r * (K / 128) + g] = quant_f16_scaled(w + (size_t)r * K + g * 128, 128, q + (size_t)r * K + g * 128);
        }
      }
    }
  }
}

void q36o_quant_dense8(const float* w, int N, int K, int8_t* q, uint16_t* s, int s_stride) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < K / 128; ++g)
      s[(size_t)g * s_stride + n] = quant_f16_scaled(w + (size_t)n * K + g * 128, 128, q + (size_t)n * K + g * 128);
}

/* ------------------------------------------------------------------------------------ */
/* routing                                                                              */
/* ------------------------------------------------------------------------------------ */

/* logits = bf16(dot_canon(x_t, Wr_e) [+ bias_e]); softmax over E in fp32; top-k by (bf16 logit
 * desc, expert id asc); w_j = p_j / sum_j p_j  (L/i8x_decode.py:98-117 _top8; L/qk_route.cu:117-192).
 * The softmax sum uses lane partials over experts l + 64 m, then bfly64.  Padded rows (pos==0)
 * get ids -1, weight 0 and stay out of the lists (L/qk_route.cu:225-229,307).
 * Lists (canonical order; the reference leaves it to atomics, L/qk_route.cu:9-10):
 *   counts[e], offsets[e] = exclusive scan, sorted position p of slot s = t*k + j is
 *   offsets[e] + #{t' < t : e in ids[t']};  perm[p] = s, inv_perm[s] = p (-1 for padding);
 *   active[u] = the u-th expert with counts > 0, ascending; n_active = their number. */
int q36o_route(const uint16_t* x, const uint16_t* wr, const float* bias, const int32_t* pos, int M, int E,
               int H, int k, float* logits, int32_t* ids, float* wts, int32_t* counts, int32_t* offsets,
               int32_t* perm, int32_t* inv_perm, int32_t* active, int32_t* n_active) {
  if (H % 512 || E % 64 || k > E || k > 64) return -1;
  float* xf = (float*)malloc(sizeof(float) * (size_t)M * H);
  float* wf = (float*)malloc(sizeof(float) * (size_t)E * H);
  for (size_t i = 0; i < (size_t)M * H; ++i) xf[i] = q36o_bf16_to_f32(x[i]);
  for (size_t i = 0; i < (size_t)E * H; ++i) wf[i] = q36o_bf16_to_f32(wr[i]);
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < M; ++t)
    for (int e = 0; e < E; ++e) {
      float d = q36o_dot_canon(xf + (size_t)t * H, wf + (size_t)e * H, H);
      if (bias) d = d + bias[e];
      logits[(size_t)t * E + e] = bf(d);
    }
  free(xf);
  free(wf);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < M; ++t) {
    const float* lg = logits + (size_t)t * E;
    if (pos && pos[t] == 0) {
      for (int j = 0; j < k; ++j) { ids[t * k + j] = -1; wts[t * k + j] = 0.f; }
      continue;
    }
    float mx = -INFINITY;
    for (int e = 0; e < E; ++e) mx = fmaxf(mx, lg[e]);
    float part[64];
    for (int l = 0; l < 64; ++l) {
      float acc = 0.f;
      for (int m = 0; m < E / 64; ++m) acc = acc + q36o_expf(lg[l + 64 * m] - mx);
      part[l] = acc;
    }
    float sum = bfly64(part);
    unsigned char taken[4096] = {0};
    float wsum = 0.f, pj[64];
    for (int j = 0; j < k; ++j) {
      int best = -1;
      for (int e = 0; e < E; ++e)
        if (!taken[e] && (best < 0 || lg[e] > lg[best])) best = e;
      taken[best] = 1;
      ids[t * k + j] = best;
      pj[j] = q36o_expf(lg[best] - mx) / sum;
      wsum = wsum + pj[j];
    }
    float div = wsum > 0.f ? wsum : 1.f;
    for (int j = 0; j < k; ++j) wts[t * k + j] = pj[j] / div;
  }
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int t = 0; t < M; ++t)
    for (int j = 0; j < k; ++j)
      if (ids[t * k + j] >= 0) counts[ids[t * k + j]]++;
  offsets[0] = 0;
  int nu = 0;
  for (int e = 0; e < E; ++e) {
    offsets[e + 1] = offsets[e] + counts[e];
    if (counts[e]) active[nu++] = e;
  }
  *n_active = nu;
  int* fill = (int*)calloc((size_t)E, sizeof(int));
  for (int s = 0; s < M * k; ++s) inv_perm[s] = -1;
  for (int t = 0; t < M; ++t)      /* token-major walk = (expert, token, j) order inside each expert */
    for (int j = 0; j < k; ++j) {
      int e = ids[t * k + j];
      if (e < 0) continue;
      int p = offsets[e] + fill[e]++;
      perm[p] = t * k + j;
      inv_perm[t * k + j] = p;
    }
  for (int p = offsets[E]; p < M * k; ++p) perm[p] = -1;
  free(fill);
  return 0;
}

/* ------------------------------------------------------------------------------------ */
/* MoE block                                                                            */
/* ------------------------------------------------------------------------------------ */

/* Dot of one quantized activation row with one quantized weight row.
 * mode 0: exact int32 sum (L/qk_moe_prefill_i8.cu:3646-3654 up_w8a8; H/w8a8.py:39-75).
 * mode 1: e4m3 128-blocks; each block sum of e4m3 x e4m3 products is formed exactly (double
 * holds it: products span 2^-18 .. 2^17.6, a 128-term sum needs < 44 bits), rounded once to
 * fp32, then acc = fma(bsum, xs[kb] * ws[kb], acc) in increasing kb from zero (the block dequant
 * of DeepSeek-style fp8 GEMMs, accumulator += partial * (scale_a * scale_b); the configuration asks
 * for it and the reference has no counterpart). */
static const float* g_e4m3_lut(void) {
  static float lut[256];
  static int init = 0;
  if (!init) {
#pragma omp critical(q36o_lut)
    {
      if (!init) {
        for (int i = 0; i < 256; ++i) lut[i] = q36o_e4m3_to_f32((uint8_t)i);
        init = 1;
      }
    }
  }
  return lut;
}

static float fp8_row_dot(const uint8_t* xq, const float* xs, const uint8_t* wq, const float* ws, int K) {
  const float* lut = g_e4m3_lut();
  float acc = 0.f;
  for (int kb = 0; kb < K / 128; ++kb) {
    double bs = 0.0;
    for (int i = 0; i < 128; ++i) bs += (double)lut[xq[kb * 128 + i]] * (double)lut[wq[kb * 128 + i]];
    acc = fmaf((float)bs, xs[kb] * ws[kb], acc);
  }
  return acc;
}
static int32_t i8_row_dot(const int8_t* a, const int8_t* b, int K) {
  int32_t acc = 0;
  for (int i = 0; i < K; ++i) acc += (int32_t)a[i] * (int32_t)b[i];
  return acc;
}

/* One expert applied to one activation row (x already quantized).
 * Up (L/i8x_decode.py:305-341, :151-156; L/qk_moe_up16.cu:110-124): g, u dequantized in fp32,
 * rounded to bf16, h = bf16(silu(g) * u) with silu(g) = g / (1 + exp(-g)); gate rows 0..I-1,
 * up rows I..2I-1 (L/i8x_decode.py:335-340).
 * Down (L/i8x_decode.py:343-422; L/qk_moe_dn16.cu:1-14): h re-quantized per row (int8) or per
 * 128-group (e4m3); y = bf16(acc * hs * ws * wt), the routing weight applied before the store. */
typedef struct {
  int mode, H, I;
  const void* w13; const float* s13; const void* w2; const float* s2;
} expert_t;

static void expert_rows(const expert_t* ex, const void* xq, const float* xs, float wt, uint16_t* y_out,
                        int32_t* acc13, int32_t* acc2, uint16_t* h_out, const uint16_t* h_in) {
  int H = ex->H, I = ex->I;
  float* hf = (float*)malloc(sizeof(float) * I);
  if (h_in) {
    for (int n = 0; n < I; ++n) hf[n] = q36o_bf16_to_f32(h_in[n]);
  } else if (ex->mode == 0) {
    const int8_t* w = (const int8_t*)ex->w13;
    for (int n = 0; n < I; ++n) {
      int32_t ag = i8_row_dot((const int8_t*)xq, w + (size_t)n * H, H);
      int32_t au = i8_row_dot((const int8_t*)xq, w + (size_t)(I + n) * H, H);
      if (acc13) { acc13[n] = ag; acc13[I + n] = au; }
      float g = bf(((float)ag * xs[0]) * ex->s13[n]);
      float u = bf(((float)au * xs[0]) * ex->s13[I + n]);
      hf[n] = bf((g / (1.f + q36o_expf(-g))) * u);
    }
  } else {
    const uint8_t* w = (const uint8_t*)ex->w13;
    int kb = H / 128;
    for (int n = 0; n < I; ++n) {
      float g = fp8_row_dot((const uint8_t*)xq, xs, w + (size_t)n * H, ex->s13 + (size_t)(n / 128) * kb, H);
      float u = fp8_row_dot((const uint8_t*)xq, xs, w + (size_t)(I + n) * H,
                            ex->s13 + (size_t)((I + n) / 128) * kb, H);
      g = bf(g);
      u = bf(u);
      hf[n] = bf((g / (1.f + q36o_expf(-g))) * u);
    }
  }
  if (h_out)
    for (int n = 0; n < I; ++n) h_out[n] = q36o_f32_to_bf16(hf[n]);
  if (ex->mode == 0) {
    int8_t* hq = (int8_t*)malloc(I);
    float hs;
    quant_row_i8(hf, I, hq, &hs);
    const int8_t* w = (const int8_t*)ex->w2;
    for (int n = 0; n < H; ++n) {
      int32_t a2 = i8_row_dot(hq, w + (size_t)n * I, I);
      if (acc2) acc2[n] = a2;
      y_out[n] = q36o_f32_to_bf16((((float)a2 * hs) * ex->s2[n]) * wt);
    }
    free(hq);
  } else {
    int kb = I / 128;
    uint8_t* hq = (uint8_t*)malloc(I);
    float hs[64];
    for (int g = 0; g < kb; ++g) quant_group_e4m3(hf + g * 128, 128, I, 1, hq + g * 128, I, &hs[g]);
    const uint8_t* w = (const uint8_t*)ex->w2;
    for (int n = 0; n < H; ++n) {
      float a2 = fp8_row_dot(hq, hs, w + (size_t)n * I, ex->s2 + (size_t)(n / 128) * kb, I);
      y_out[n] = q36o_f32_to_bf16(a2 * wt);
    }
    free(hq);
  }
  free(hf);
}

/* The whole MoE block of one row batch (L/i8x_decode.py:528-605 moe_row_batch):
 * route -> quantize x -> routed experts (y per slot, weighted) + shared expert ->
 * out[t] = bf16(fma(gate_t, y_shared, ((0 + y_0) + y_1) ... + y_{k-1})), gate_t =
 * sigmoid(dot_canon(x_t, gate_w)) (L/i8x_decode.py:424-443; L/qk_route.cu:630-722).
 * Padded rows produce zeros. */
int q36o_moe(const q36o_moe_args* a) {
  int M = a->M, E = a->E, H = a->H, I = a->I, k = a->k;
  if (H % 512 || I % 128 || E % 64) return -1;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
  int S = M * k;
  float* logits = (float*)malloc(sizeof(float) * (size_t)M * E);
  int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * E);
  int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (E + 1));
  int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * S);
  int32_t* inv = (int32_t*)malloc(sizeof(int32_t) * S);
  int32_t* active = (int32_t*)malloc(sizeof(int32_t) * E);
  int32_t nact = 0;
  int rc = q36o_route(a->x, a->wr, a->bias, a->pos, M, E, H, k, logits, a->ids, a->wts, counts, offsets, perm,
                      inv, active, &nact);
  if (rc) return rc;

  float* xf = (float*)malloc(sizeof(float) * (size_t)M * H);
  for (size_t i = 0; i < (size_t)M * H; ++i) xf[i] = q36o_bf16_to_f32(a->x[i]);
  int ng = a->mode == 0 ? 1 : H / 128;
  void* xq = malloc((size_t)M * H);
  float* xs = (float*)malloc(sizeof(float) * (size_t)M * ng);
  if (a->mode == 0) q36o_quant_rows_i8(xf, M, H, (int8_t*)xq, xs);
  else q36o_quant_groups_e4m3(xf, M, H, 128, (uint8_t*)xq, xs);

  uint16_t* y = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(S + M) * H);
  size_t eb13 = (size_t)2 * I * H, eb2 = (size_t)H * I;
  size_t es13 = a->mode == 0 ? (size_t)2 * I : (size_t)(2 * I / 128) * (H / 128);
  size_t es2 = a->mode == 0 ? (size_t)H : (size_t)(H / 128) * (I / 128);
#pragma omp parallel for schedule(dynamic, 1)
  for (int p = 0; p < S + M; ++p) {  /* p = slot: t*k + j routed, S + t shared */
    int t, e;
    float wt;
    expert_t ex = {a->mode, H, I, 0, 0, 0, 0};
    if (p < S) {
      if (a->ids[p] < 0) continue;
      t = p / k;
      e = a->ids[p];
      wt = a->wts[p];
      ex.w13 = (const char*)a->w13 + (size_t)e * eb13;
      ex.s13 = a->s13 + (size_t)e * es13;
      ex.w2 = (const char*)a->w2 + (size_t)e * eb2;
      ex.s2 = a->s2 + (size_t)e * es2;
    } else {
      t = p - S;
      if (a->pos && a->pos[t] == 0) continue;
      wt = 1.f;
      ex.w13 = a->sw13; ex.s13 = a->ss13; ex.w2 = a->sw2; ex.s2 = a->ss2;
    }
    expert_rows(&ex, (const char*)xq + (size_t)t * H, xs + (size_t)t * ng, wt, y + (size_t)p * H,
                a->acc13 ? a->acc13 + (size_t)p * 2 * I : NULL, a->acc2 ? a->acc2 + (size_t)p * H : NULL,
                a->h ? a->h + (size_t)p * I : NULL, a->h_in ? a->h_in + (size_t)p * I : NULL);
  }
  if (a->y) memcpy(a->y, y, sizeof(uint16_t) * (size_t)(S + M) * H);
  if (a->y_in) memcpy(y, a->y_in, sizeof(uint16_t) * (size_t)(S + M) * H);
  float* gw = (float*)malloc(sizeof(float) * H);
  for (int i = 0; i < H; ++i) gw[i] = q36o_bf16_to_f32(a->gate_w[i]);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < M; ++t) {
    uint16_t* o = a->out + (size_t)t * H;
    if (a->pos && a->pos[t] == 0) {
      memset(o, 0, sizeof(uint16_t) * H);
      continue;
    }
    float gate = sigmoidf_q(q36o_dot_canon(xf + (size_t)t * H, gw, H));
    const uint16_t* ysh = y + (size_t)(S + t) * H;
    for (int n = 0; n < H; ++n) {
      float acc = 0.f;
      for (int j = 0; j < k; ++j) acc = acc + q36o_bf16_to_f32(y[(size_t)(t * k + j) * H + n]);
      o[n] = q36o_f32_to_bf16(fmaf(gate, q36o_bf16_to_f32(ysh[n]), acc));
    }
  }
  free(gw); free(y); free(xs); free(xq); free(xf);
  free(logits); free(counts); free(offsets); free(perm); free(inv); free(active);
  return 0;
}

/* ------------------------------------------------------------------------------------ */
/* GDN verify                                                                           */
/* ------------------------------------------------------------------------------------ */

enum { GK = 128, GV = 128, GHK = 16, GHV = 32, GQKV = 8192, GZ = GHV * GV };

/* One (sequence, value head) unit over T positions (L/qk_gdn_verify.cu:293-794 restated in
 * its sequential form; L/gdn.py:43-141 and L/qk_conv_gate.cu:1-17 document the shared front).
 *  conv  (:238-247): window [s0 s1 s2 x_0 .. x_{T-1}], out_t = silu(sum_i bf16(w_{t+i} * cw_i))
 *        summed oldest first in fp32, silu(a) = a / (1 + exp(-a)), rounded to bf16.
 *  norm  (:575-581): q, k scaled by 1/sqrt(sum^2 + 1e-6); q also by 128^-1/2.
 *  gates (:616-622): g = -exp(A_log) * softplus(a + dt_bias) (softplus = x above 20),
 *        beta = sigmoid(b).
 *  recurrence: S_t = e^{g_t} S_{t-1} + beta_t (v_t - e^{g_t} S_{t-1} k_t) k_t^T, o_t = S_t q_t
 *        (the WY form of :684-762 is the same algebra); value head hv reads key head hv/2.
 *  output (:786-791): y = bf16(((o * rstd) * w) * (z * sigmoid(z))), o rounded to bf16 first,
 *        rstd = 1/sqrt(mean(o^2) + eps).
 * The snapshot S_t of every position is written (configuration's rollback form). */
static void gdn_unit(const q36o_gdn_args* a, int bq, int hv, const float* convd /* [T][8192] */) {
  int T = a->T, hk = hv / 2;
  float q[64][GK], kk[64][GK], vv[64][GV], g[64], beta[64];
  const float scale = 1.f / sqrtf((float)GK);
  for (int t = 0; t < T; ++t) {
    const float* row = convd + (size_t)t * GQKV;
    float nq = 0.f, nk = 0.f;
    for (int i = 0; i < GK; ++i) {
      float xq = row[hk * GK + i], xk = row[GHK * GK + hk * GK + i];
      nq = nq + xq * xq;
      nk = nk + xk * xk;
    }
    float rq = (1.f / sqrtf(nq + 1e-6f)) * scale, rk = 1.f / sqrtf(nk + 1e-6f);
    for (int i = 0; i < GK; ++i) {
      q[t][i] = row[hk * GK + i] * rq;
      kk[t][i] = row[GHK * GK + hk * GK + i] * rk;
    }
    for (int i = 0; i < GV; ++i) vv[t][i] = row[2 * GHK * GK + hv * GV + i];
    size_t r = (size_t)bq * T + t;
    float av = q36o_bf16_to_f32(a->a[r * GHV + hv]), bv = q36o_bf16_to_f32(a->b[r * GHV + hv]);
    float xg = av + a->dt_bias[hv];
    float sp = xg <= 20.f ? logf(1.f + q36o_expf(xg)) : xg;
    g[t] = -q36o_expf(a->A_log[hv]) * sp;
    beta[t] = sigmoidf_q(bv);
  }
  const float* S0 = a->S0 + ((size_t)bq * GHV + hv) * GV * GK;
  float nw[GV];
  for (int i = 0; i < GV; ++i) nw[i] = q36o_bf16_to_f32(a->norm_w[i]);
  if (a->use_f64) {
    double* S = (double*)malloc(sizeof(double) * GV * GK);
    for (int i = 0; i < GV * GK; ++i) S[i] = S0[i];
    for (int t = 0; t < T; ++t) {
      double eg = exp((double)g[t]);
      float o[GV];
      for (int v = 0; v < GV; ++v) {
        double* Sr = S + (size_t)v * GK;
        double kv = 0.0;
        for (int c = 0; c < GK; ++c) kv += Sr[c] * kk[t][c];
        double u = beta[t] * (vv[t][v] - eg * kv);
        double ov = 0.0;
        for (int c = 0; c < GK; ++c) {
          Sr[c] = eg * Sr[c] + u * kk[t][c];
          ov += Sr[c] * q[t][c];
        }
        o[v] = bf((float)ov);
      }
      float* snap = a->snaps + ((((size_t)bq * T + t) * GHV + hv) * GV) * GK;
      for (int i = 0; i < GV * GK; ++i) snap[i] = (float)S[i];
      double ss = 0.0;
      for (int v = 0; v < GV; ++v) ss += (double)o[v] * o[v];
      float rstd = 1.f / sqrtf((float)(ss / GV) + a->eps);
      size_t r = (size_t)bq * T + t;
      for (int v = 0; v < GV; ++v) {
        float zz = q36o_bf16_to_f32(a->z[r * GZ + hv * GV + v]);
        a->out[r * GZ + hv * GV + v] = q36o_f32_to_bf16(((o[v] * rstd) * nw[v]) * (zz * sigmoidf_q(zz)));
      }
    }
    free(S);
    return;
  }
  float* S = (float*)malloc(sizeof(float) * GV * GK);
  memcpy(S, S0, sizeof(float) * GV * GK);
  for (int t = 0; t < T; ++t) {
    float eg = q36o_expf(g[t]);
    float o[GV];
    for (int v = 0; v < GV; ++v) {
      float* Sr = S + (size_t)v * GK;
      float kv = 0.f;
      for (int c = 0; c < GK; ++c) kv = fmaf(Sr[c], kk[t][c], kv);
      float u = beta[t] * (vv[t][v] - eg * kv);
      float ov = 0.f;
      for (int c = 0; c < GK; ++c) {
        Sr[c] = fmaf(eg, Sr[c], u * kk[t][c]);
        ov = fmaf(Sr[c], q[t][c], ov);
      }
      o[v] = bf(ov);
    }
    float* snap = a->snaps + ((((size_t)bq * T + t) * GHV + hv) * GV) * GK;
    memcpy(snap, S, sizeof(float) * GV * GK);
    float ss = 0.f;
    for (int v = 0; v < GV; ++v) ss = ss + o[v] * o[v];
    float rstd = 1.f / sqrtf(ss / (float)GV + a->eps);
    size_t r = (size_t)bq * T + t;
    for (int v = 0; v < GV; ++v) {
      float zz = q36o_bf16_to_f32(a->z[r * GZ + hv * GV + v]);
      a->out[r * GZ + hv * GV + v] = q36o_f32_to_bf16(((o[v] * rstd) * nw[v]) * (zz * sigmoidf_q(zz)));
    }
  }
  free(S);
}

int q36o_gdn_verify(const q36o_gdn_args* a) {
  int B = a->B, T = a->T;
  if (T < 1 || T > 64) return -1;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
  float* convd = (float*)malloc(sizeof(float) * (size_t)B * T * GQKV);
  /* conv for every channel of every sequence, then the state roll */
#pragma omp parallel for schedule(static)
  for (int bq = 0; bq < B; ++bq) {
    for (int c = 0; c < GQKV; ++c) {
      float w[64 + 3];
      uint16_t* st = a->conv_state + ((size_t)bq * GQKV + c) * 3;
      for (int i = 0; i < 3; ++i) w[i] = q36o_bf16_to_f32(st[i]);
      for (int t = 0; t < T; ++t) w[3 + t] = q36o_bf16_to_f32(a->mixed[((size_t)bq * T + t) * GQKV + c]);
      float cw[4];
      for (int i = 0; i < 4; ++i) cw[i] = q36o_bf16_to_f32(a->conv_w[(size_t)c * 4 + i]);
      for (int t = 0; t < T; ++t) {
        float acc = bf(w[t] * cw[0]);
        acc = acc + bf(w[t + 1] * cw[1]);
        acc = acc + bf(w[t + 2] * cw[2]);
        acc = acc + bf(w[t + 3] * cw[3]);
        convd[((size_t)bq * T + t) * GQKV + c] = bf(acc / (1.f + q36o_expf(-acc)));
      }
      for (int i = 0; i < 3; ++i) st[i] = q36o_f32_to_bf16(w[T + i]);
    }
  }
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int bq = 0; bq < B; ++bq)
    for (int hv = 0; hv < GHV; ++hv) gdn_unit(a, bq, hv, convd + (size_t)bq * T * GQKV);
  free(convd);
  return 0;
}

/* ---- GDN verify over the ReplaySSM ring ---- */
enum { GRING = 16 };

/* One (request, value head) unit of the ring verify (L/qk_gdn_verify.cu:575-791 restated
 * sequentially).  The history state is materialised first:
 *   pre_c = g_0 + .. + g_c (logical order, sequential), total = pre_{n-1},
 *   decay_c = exp(total - pre_c), td = exp(total)                        (:634-648)
 *   S = td * h0, then S += (decay_c * dhat_c) khat_c^T for c = 0 .. n-1   (:709-721, :745-751)
 * with the ring's bf16 high parts (the verify never reads the low parts, :598-605, :711).  The
 * window then runs the sequential delta rule of gdn_unit; d_t = beta_t (v_t - e^{g_t} S_{t-1} k_t)
 * is the ring's d entry (the WY form's D of :752-755). */
static void gdn_ring_unit(const q36o_gdn_ring_args* a, int r, int hv, const float* convd /* [T][8192] */) {
  const int T = a->T, hk = hv / 2;
  const int64_t slot = a->state_idx[r], rp = a->replay_idx[r];
  const size_t bos = (size_t)a->qsl[r];
  int wp = a->write_pos[rp], cb = a->cache_base[rp];
  const int nv = wp < 0 ? 0 : wp > GRING ? GRING : wp;
  float q[8][GK], kk[8][GK], vv[8][GV], g[8], beta[8];
  for (int t = 0; t < T; ++t) {
    const float* row = convd + (size_t)t * GQKV;
    float nq = 0.f, nk = 0.f;
    for (int i = 0; i < GK; ++i) {
      float xq = row[hk * GK + i], xk = row[GHK * GK + hk * GK + i];
      nq = nq + xq * xq;
      nk = nk + xk * xk;
    }
    float rq = (1.f / sqrtf(nq + 1e-6f)) * a->scale, rk = 1.f / sqrtf(nk + 1e-6f);
    for (int i = 0; i < GK; ++i) {
      q[t][i] = row[hk * GK + i] * rq;
      kk[t][i] = row[GHK * GK + hk * GK + i] * rk;
    }
    for (int i = 0; i < GV; ++i) vv[t][i] = row[2 * GHK * GK + hv * GV + i];
    const size_t rr = bos + t;
    float av = q36o_bf16_to_f32(a->a[rr * GHV + hv]), bv = q36o_bf16_to_f32(a->b[rr * GHV + hv]);
    float xg = av + a->dt_bias[hv];
    float sp = xg <= 20.f ? logf(1.f + q36o_expf(xg)) : xg;
    g[t] = -q36o_expf(a->A_log[hv]) * sp;
    beta[t] = sigmoidf_q(bv);
  }
  /* committed history, logical order */
  const uint16_t* kr = a->k_ring + ((size_t)rp * GHK + hk) * GRING * GK;
  const uint16_t* dr = a->d_ring + ((size_t)rp * GHV + hv) * GRING * GV;
  const float* gr = a->g_ring + ((size_t)rp * GHV + hv) * GRING;
  float pre[GRING], decay[GRING], total = 0.f;
  for (int c = 0; c < nv; ++c) {
    total = total + gr[(cb + c) & (GRING - 1)];
    pre[c] = total;
  }
  for (int c = 0; c < nv; ++c) decay[c] = q36o_expf(total - pre[c]);
  const float td = q36o_expf(total);
  const float* H = a->h0 + ((size_t)slot * GHV + hv) * GV * GK;
  float nw[GV];
  for (int i = 0; i < GV; ++i) nw[i] = q36o_bf16_to_f32(a->norm_w[i]);
  float o[8][GV], d[8][GV];
  if (a->use_f64) {
    double* S = (double*)malloc(sizeof(double) * GV * GK);
    for (int i = 0; i < GV * GK; ++i) S[i] = (double)td * H[i];
    for (int c = 0; c < nv; ++c) {
      const int p = (cb + c) & (GRING - 1);
      for (int v = 0; v < GV; ++v) {
        double dc = (double)decay[c] * q36o_bf16_to_f32(dr[p * GV + v]);
        for (int j = 0; j < GK; ++j) S[v * GK + j] += dc * q36o_bf16_to_f32(kr[p * GK + j]);
      }
    }
    for (int t = 0; t < T; ++t) {
      double eg = exp((double)g[t]);
      for (int v = 0; v < GV; ++v) {
        double* Sr = S + (size_t)v * GK;
        double kv = 0.0;
        for (int c = 0; c < GK; ++c) kv += Sr[c] * kk[t][c];
        double u = beta[t] * (vv[t][v] - eg * kv), ov = 0.0;
        for (int c = 0; c < GK; ++c) {
          Sr[c] = eg * Sr[c] + u * kk[t][c];
          ov += Sr[c] * q[t][c];
        }
        d[t][v] = (float)u;
        o[t][v] = bf((float)ov);
      }
    }
    free(S);
  } else {
    float* S = (float*)malloc(sizeof(float) * GV * GK);
    for (int i = 0; i < GV * GK; ++i) S[i] = td * H[i];
    for (int c = 0; c < nv; ++c) {
      const int p = (cb + c) & (GRING - 1);
      for (int v = 0; v < GV; ++v) {
        float dc = decay[c] * q36o_bf16_to_f32(dr[p * GV + v]);
        for (int j = 0; j < GK; ++j) S[v * GK + j] = fmaf(dc, q36o_bf16_to_f32(kr[p * GK + j]), S[v * GK + j]);
      }
    }
    for (int t = 0; t < T; ++t) {
      float eg = q36o_expf(g[t]);
      for (int v = 0; v < GV; ++v) {
        float* Sr = S + (size_t)v * GK;
        float kv = 0.f;
        for (int c = 0; c < GK; ++c) kv = fmaf(Sr[c], kk[t][c], kv);
        float u = beta[t] * (vv[t][v] - eg * kv), ov = 0.f;
        for (int c = 0; c < GK; ++c) {
          Sr[c] = fmaf(eg, Sr[c], u * kk[t][c]);
          ov = fmaf(Sr[c], q[t][c], ov);
        }
        d[t][v] = u;
        o[t][v] = bf(ov);
      }
    }
    free(S);
  }
  /* ring appends at logical nv + t while they fit (k :583-596, g :631, d :770-781) */
  for (int t = 0; t < T && nv + t < GRING; ++t) {
    const int p = (cb + nv + t) & (GRING - 1);
    uint16_t* dh = a->d_ring + (((size_t)rp * GHV + hv) * GRING + p) * GV;
    uint16_t* dl = a->dlo_ring + (((size_t)rp * GHV + hv) * GRING + p) * GV;
    for (int v = 0; v < GV; ++v) {
      dh[v] = q36o_f32_to_bf16(d[t][v]);
      dl[v] = q36o_f32_to_bf16(d[t][v] - q36o_bf16_to_f32(dh[v]));
    }
    a->g_ring[((size_t)rp * GHV + hv) * GRING + p] = g[t];
    if ((hv & 1) == 0) {
      uint16_t* kh = a->k_ring + (((size_t)rp * GHK + hk) * GRING + p) * GK;
      uint16_t* kl = a->klo_ring + (((size_t)rp * GHK + hk) * GRING + p) * GK;
      for (int j = 0; j < GK; ++j) {
        kh[j] = q36o_f32_to_bf16(kk[t][j]);
        kl[j] = q36o_f32_to_bf16(kk[t][j] - q36o_bf16_to_f32(kh[j]));
      }
    }
  }
  for (int t = 0; t < T; ++t) {
    float ss = 0.f;
    for (int v = 0; v < GV; ++v) ss = ss + o[t][v] * o[t][v];
    float rstd = 1.f / sqrtf(ss / (float)GV + a->eps);
    const size_t rr = bos + t;
    for (int v = 0; v < GV; ++v) {
      float zz = q36o_bf16_to_f32(a->z[rr * GZ + hv * GV + v]);
      a->out[rr * GZ + hv * GV + v] = q36o_f32_to_bf16(((o[t][v] * rstd) * nw[v]) * (zz * sigmoidf_q(zz)));
    }
  }
}

int q36o_gdn_verify_ring(const q36o_gdn_ring_args* a) {
  const int B = a->B, T = a->T;
  if (B < 0 || T < 1 || T > 8) return -1;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
  float* convd = (float*)malloc(sizeof(float) * ((size_t)B * T * GQKV + 1));
  /* conv per request: window record [s1 s2 x0 .. x_{T-1}], state rolled to the last three inputs
   * (L/qk_gdn_verify.cu:277-291 record layout, :607-613 the roll after every read) */
#pragma omp parallel for schedule(static)
  for (int r = 0; r < B; ++r) {
    const int64_t slot = a->state_idx[r];
    const size_t bos = (size_t)a->qsl[r];
    if (slot < 0) {
      for (int t = 0; t < T; ++t)
        for (int c = 0; c < GZ; ++c) a->out[(bos + t) * GZ + c] = 0;
      continue;
    }
    const int64_t ws = a->win_idx[r];
    for (int c = 0; c < GQKV; ++c) {
      float w[8 + 3];
      uint16_t* st = a->conv_state + ((size_t)slot * GQKV + c) * 3;
      for (int i = 0; i < 3; ++i) w[i] = q36o_bf16_to_f32(st[i]);
      for (int t = 0; t < T; ++t) w[3 + t] = q36o_bf16_to_f32(a->mixed[(bos + t) * GQKV + c]);
      float cw[4];
      for (int i = 0; i < 4; ++i) cw[i] = q36o_bf16_to_f32(a->conv_w[(size_t)c * 4 + i]);
      for (int t = 0; t < T; ++t) {
        float acc = bf(w[t] * cw[0]);
        acc = acc + bf(w[t + 1] * cw[1]);
        acc = acc + bf(w[t + 2] * cw[2]);
        acc = acc + bf(w[t + 3] * cw[3]);
        convd[((size_t)r * T + t) * GQKV + c] = bf(acc / (1.f + q36o_expf(-acc)));
      }
      uint16_t* rec = a->window + ((size_t)ws * GQKV + c) * (T + 2);
      for (int i = 0; i < T + 2; ++i) rec[i] = q36o_f32_to_bf16(w[1 + i]);
      for (int i = 0; i < 3; ++i) st[i] = q36o_f32_to_bf16(w[T + i]);
    }
  }
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int r = 0; r < B; ++r)
    for (int hv = 0; hv < GHV; ++hv)
      if (a->state_idx[r] >= 0) gdn_ring_unit(a, r, hv, convd + (size_t)r * T * GQKV);
  free(convd);
  return 0;
}

/* ------------------------------------------------------------------------------------ */
/* attention projections                                                                */
/* ------------------------------------------------------------------------------------ */

/* y[t, n] = the e4m3 block dots (exact, rounded once) accumulated as fma(dot, xs * ws, acc) over
 * the 128-blocks in order, the same block rule as the fp8 experts; the result is rounded to bf16
 * (the projection's output dtype). */
static void fp8_linear(const uint8_t* xq, const float* xs, int T, const uint8_t* w, const float* s, int N,
                       int K, float* y) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < T; ++t)
    for (int n = 0; n < N; ++n)
      y[(size_t)t * N + n] = bf(fp8_row_dot(xq + (size_t)t * K, xs + (size_t)t * (K / 128), w + (size_t)n * K,
                                           s + (size_t)(n / 128) * (K / 128), K));
}

/* Gemma RMSNorm of one 256-wide head then neox RoPE on dims 0..63, pairs (i, i + 32)
 * (L/qk_attn_verify.cu:180-208 norm_rope_e4m3, :156-177 load_rope):
 *   x = bf16(x * inv * (w + 1)), inv = 1/sqrt(sum x^2 / 256 + eps);
 *   x_i' = bf16(x_i c - x_{i+32} s), x_{i+32}' = bf16(x_{i+32} c + x_i s), i < 32. */
static void norm_rope(float* x, const uint16_t* w, float eps, const float* cs) {
  float ss = 0.f;
  for (int i = 0; i < 256; ++i) ss = ss + x[i] * x[i];
  float inv = 1.f / sqrtf(ss / 256.f + eps);
  for (int i = 0; i < 256; ++i) x[i] = bf((x[i] * inv) * (q36o_bf16_to_f32(w[i]) + 1.f));
  float r[64];
  for (int i = 0; i < 32; ++i) {
    r[i] = bf(x[i] * cs[i] - x[i + 32] * cs[32 + i]);
    r[i + 32] = bf(x[i + 32] * cs[i] + x[i] * cs[32 + i]);
  }
  memcpy(x, r, sizeof(r));
}

int q36o_attn_proj(const q36o_attn_args* a) {
  int T = a->T;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
  float* xf = (float*)malloc(sizeof(float) * (size_t)T * 2048);
  for (size_t i = 0; i < (size_t)T * 2048; ++i) xf[i] = q36o_bf16_to_f32(a->x[i]);
  uint8_t* xq = (uint8_t*)malloc((size_t)T * 2048);
  float* xs = (float*)malloc(sizeof(float) * T * 16);
  q36o_quant_groups_e4m3(xf, T, 2048, 128, xq, xs);
  float* qg = (float*)malloc(sizeof(float) * (size_t)T * 8192);
  float* kf = (float*)malloc(sizeof(float) * (size_t)T * 512);
  float* vf = (float*)malloc(sizeof(float) * (size_t)T * 512);
  fp8_linear(xq, xs, T, a->wqg, a->sqg, 8192, 2048, qg);
  fp8_linear(xq, xs, T, a->wk, a->sk, 512, 2048, kf);
  fp8_linear(xq, xs, T, a->wv, a->sv, 512, 2048, vf);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    const float* cs = a->cos_sin + (size_t)a->positions[t] * 64;
    for (int hd = 0; hd < 16; ++hd) {
      float* qh = qg + (size_t)t * 8192 + hd * 512;     /* [q(256) gate(256)] per head */
      norm_rope(qh, a->q_norm_w, a->eps, cs);
      for (int i = 0; i < 256; ++i) {
        a->q[((size_t)t * 16 + hd) * 256 + i] = q36o_f32_to_bf16(qh[i]);
        a->gate[((size_t)t * 16 + hd) * 256 + i] = q36o_f32_to_bf16(qh[256 + i]);
      }
    }
    for (int hd = 0; hd < 2; ++hd) {
      float* kh = kf + (size_t)t * 512 + hd * 256;
      norm_rope(kh, a->k_norm_w, a->eps, cs);
      for (int i = 0; i < 256; ++i) {
        size_t o = ((size_t)t * 2 + hd) * 256 + i;
        a->k[o] = q36o_f32_to_bf16(kh[i]);
        a->k8[o] = q36o_f32_to_e4m3(kh[i]);
        float vv = vf[(size_t)t * 512 + hd * 256 + i];
        a->v[o] = q36o_f32_to_bf16(vv);
        a->v8[o] = q36o_f32_to_e4m3(vv);
      }
    }
  }
  free(xf); free(xq); free(xs); free(qg); free(kf); free(vf);
  return 0;
}

/* o_proj input = bf16(attn * sigmoid(gate)) (L/qk_attn_verify.cu:730-737), quantized per token x
 * 128-group to e4m3, then the block-scaled GEMM against Wo [2048, 4096]. */
int q36o_attn_oproj(const q36o_oproj_args* a) {
  int T = a->T;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
  float* g = (float*)malloc(sizeof(float) * (size_t)T * 4096);
  for (size_t i = 0; i < (size_t)T * 4096; ++i) {
    float gv = q36o_bf16_to_f32(a->gate[i]);
    g[i] = bf(q36o_bf16_to_f32(a->attn[i]) * sigmoidf_q(gv));
  }
  uint8_t* xq = (uint8_t*)malloc((size_t)T * 4096);
  float* xs = (float*)malloc(sizeof(float) * T * 32);
  q36o_quant_groups_e4m3(g, T, 4096, 128, xq, xs);
  float* y = (float*)malloc(sizeof(float) * (size_t)T * 2048);
  fp8_linear(xq, xs, T, a->wo, a->so, 2048, 4096, y);
  for (size_t i = 0; i < (size_t)T * 2048; ++i) a->out[i] = q36o_f32_to_bf16(y[i]);
  free(g); free(xq); free(xs); free(y);
  return 0;
}

/* ------------------------------------------------------------------------------------ */
/* hybrid-layer glue: block-scaled linear, add + Gemma RMSNorm                           */
/* ------------------------------------------------------------------------------------ */

/* The decode projections around the hybrid layer's mixers (gdn_in_proj, out_proj, o_proj before the
 * add-norm; L/qk_proj_decode.cu:409,434, L/proj.py:84-112) in the configuration's e4m3 format: x
 * quantized per token x 128 channels, then the block rule of fp8_linear, all N columns. */
int q36o_fp8_linear(int T, int N, int K, const uint16_t* x, const uint8_t* wq, const float* ws, uint16_t* out,
                    int n_threads) {
  if (K % 128 || N % 128 || T < 1) return -1;
  if (n_threads > 0) omp_set_num_threads(n_threads);
  float* xf = (float*)malloc(sizeof(float) * (size_t)T * K);
  for (size_t i = 0; i < (size_t)T * K; ++i) xf[i] = q36o_bf16_to_f32(x[i]);
  uint8_t* xq = (uint8_t*)malloc((size_t)T * K);
  float* xs = (float*)malloc(sizeof(float) * (size_t)T * (K / 128));
  q36o_quant_groups_e4m3(xf, T, K, 128, xq, xs);
  float* y = (float*)malloc(sizeof(float) * (size_t)T * N);
  fp8_linear(xq, xs, T, wq, ws, N, K, y);
  for (size_t i = 0; i < (size_t)T * N; ++i) out[i] = q36o_f32_to_bf16(y[i]);
  free(xf); free(xq); free(xs); free(y);
  return 0;
}

int q36o_dense8_linear(int T, int N, int K, const uint16_t* x, const int8_t* q, const uint16_t* s, int64_t s_ld,
                       uint16_t* out, int n_threads) {
  if (K % 128 || T < 1 || N < 1 || s_ld < N) return -1;
  if (n_threads > 0) omp_set_num_threads(n_threads);
  float* xf = (float*)malloc(sizeof(float) * (size_t)T * K);
  for (size_t i = 0; i < (size_t)T * K; ++i) xf[i] = q36o_bf16_to_f32(x[i]);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const int8_t* w = q + (size_t)n * K;
    for (int t = 0; t < T; ++t) {
      const float* xr = xf + (size_t)t * K;
      float acc = 0.f;
      for (int g = 0; g < K / 128; ++g) {
        double dot = 0.0;
        for (int i = 128 * g; i < 128 * g + 128; ++i) dot += (double)xr[i] * (double)w[i];
        acc = fmaf((float)dot, q36o_f16_to_f32(s[(size_t)g * s_ld + n]), acc);
      }
      out[(size_t)t * N + n] = q36o_f32_to_bf16(acc);
    }
  }
  free(xf);
  return 0;
}

/* The add-norm between blocks (L/proj.py:60-81): z = bf16 delta + residual in fp32 (no delta:
 * z = residual); residual <- bf16(z) when delta is given; out = bf16((z * rstd) * (1 + w)),
 * rstd = 1 / sqrt(ss / H + eps), ss = q36o_dot_canon(z, z) (the kernel's fixed order). */
int q36o_add_rmsnorm(int T, int H, const uint16_t* delta, uint16_t* residual, const uint16_t* w, float eps,
                     uint16_t* out) {
  if (H % 512 || T < 1) return -1;
  float* z = (float*)malloc(sizeof(float) * H);
  for (int t = 0; t < T; ++t) {
    for (int i = 0; i < H; ++i) {
      float r = q36o_bf16_to_f32(residual[(size_t)t * H + i]);
      z[i] = delta ? q36o_bf16_to_f32(delta[(size_t)t * H + i]) + r : r;
      if (delta) residual[(size_t)t * H + i] = q36o_f32_to_bf16(z[i]);
    }
    float ss = q36o_dot_canon(z, z, H);
    float rstd = 1.f / sqrtf(ss / (float)H + eps);
    for (int i = 0; i < H; ++i)
      out[(size_t)t * H + i] = q36o_f32_to_bf16((z[i] * rstd) * (1.f + q36o_bf16_to_f32(w[i])));
  }
  free(z);
  return 0;
}

/* ------------------------------------------------------------------------------------ */
/* decode / verify attention                                                            */
/* ------------------------------------------------------------------------------------ */

/* IEEE binary16 round-to-nearest-even of a float, returned as the float it represents (normal
 * and subnormal range; |x| above the f16 maximum saturates, which softmax weights in [0, 1] never
 * reach). */
float q36o_f16_round(float x) {
  uint32_t u = f2u(x), sign = u & 0x80000000u;
  float ax = fabsf(x);
  if (!(ax == ax)) return x;
  if (ax >= 65504.f) return u2f(sign | f2u(65504.f));
  if (ax < 6.103515625e-05f) {  /* below 2^-14: a multiple of the subnormal step 2^-24 */
    double q = (double)ax * 16777216.0, f = floor(q), r = q - f;
    if (r > 0.5 || (r == 0.5 && fmod(f, 2.0) != 0.0)) f += 1.0;
    return u2f(sign | f2u((float)(f / 16777216.0)));
  }
  uint32_t a = f2u(ax), lsb = (a >> 13) & 1u, rest = a & 0x1fffu;
  a &= ~0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && lsb)) a += 0x2000u;
  return u2f(sign | a);
}

/* Attention of each query token over its request's keys, the restatement of the verify kernel's
 * arithmetic (L/qk_attn_verify.cu:156-208 q -> e4m3, :233-337 scores and softmax, :480-560 P V with
 * f16 weights, :560-600 the normalised output): query token t of request r sees key positions
 * 0 .. seqlens[r] - NT + t (the causal rule among the NT new tokens); q head i reads kv head
 * i / (HQ / HKV).  s_k = (sum_d e4m3(q)_d k_d) * scale exactly, p_k = exp(s_k - max s), the P V
 * product uses p_k rounded to f16 and the normaliser the unrounded p_k: out = bf16(sum p16 v / sum p).
 * The sums are exact (double); the kernel's split / online order is a rounding difference. */
int q36o_attn_decode(const q36o_decode_args* a) {
  const int B = a->B, NT = a->NT, HQ = a->HQ, HKV = a->HKV, D = a->D, G = HQ / HKV;
  if (HQ % HKV || NT < 1) return -1;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int r = 0; r < B; ++r)
    for (int t = 0; t < NT; ++t)
      for (int i = 0; i < HQ; ++i) {
        const int h = i / G, nk = a->seqlens[r] - NT + t + 1;
        const uint16_t* qr = a->q + (((size_t)r * NT + t) * HQ + i) * D;
        uint16_t* o = a->out + (((size_t)r * NT + t) * HQ + i) * D;
        if (nk <= 0) {
          for (int d = 0; d < D; ++d) o[d] = 0;
          continue;
        }
        float* q8 = (float*)malloc(sizeof(float) * D);
        double* sc = (double*)malloc(sizeof(double) * nk);
        double* acc = (double*)calloc(D, sizeof(double));
        for (int d = 0; d < D; ++d) q8[d] = q36o_e4m3_to_f32(q36o_f32_to_e4m3(q36o_bf16_to_f32(qr[d])));
        double mx = -INFINITY;
        for (int k = 0; k < nk; ++k) {
          const uint8_t* kr = a->kcache + ((size_t)a->page_table[(size_t)r * a->pt_stride + k] * HKV + h) * D;
          double dot = 0.0;
          for (int d = 0; d < D; ++d) dot += (double)q8[d] * (double)q36o_e4m3_to_f32(kr[d]);
          sc[k] = (double)(float)dot * (double)a->scale;
          if (sc[k] > mx) mx = sc[k];
        }
        double l = 0.0;
        for (int k = 0; k < nk; ++k) {
          const double p = exp(sc[k] - mx);
          const double p16 = (double)q36o_f16_round((float)p);
          l += p;
          const uint8_t* vr = a->vcache + ((size_t)a->page_table[(size_t)r * a->pt_stride + k] * HKV + h) * D;
          for (int d = 0; d < D; ++d) acc[d] += p16 * (double)q36o_e4m3_to_f32(vr[d]);
        }
        for (int d = 0; d < D; ++d) o[d] = q36o_f32_to_bf16((float)(acc[d] / l));
        free(q8); free(sc); free(acc);
      }
  return 0;
}

/* ------------------------------------------------------------------------------------ */
/* int8 lm_head + argmax                                                                */
/* ------------------------------------------------------------------------------------ */

/* Final Gemma RMSNorm y = bf16((h * rstd) * (1 + w)), rstd = 1/sqrt(ss/H + eps) with ss in the
 * canonical order (L/proj.py:60-81 restates the same norm), then per-row int8 quantization
 * (H/w8a8.py:16-23), acc = sum xq * wq (int32), logit = (acc * xs) * ws (H/w8a8.py:66-71), rounded
 * to bf16 (the node's output dtype), and the greedy id = the first index of the largest bf16
 * logit (torch.argmax order; the reference leaves argmax to the stock sampler, H/node.py:136-151). */
/* W8A16 lm_head (H/lmhead8.py:57-91 _w8a16_kernel): logit = bf16(acc * ws[n]) with acc the sum of the
 * bf16 row times the int8 weights (every product exact in fp32), taken exactly (double) and rounded
 * once to fp32: the kernel sums in fp32 in its own order, so this form is the tolerance reference. */
static int lmhead_w8a16(const q36o_lmhead_args* a) {
  int R = a->R, H = a->H, V = a->V;
  float* y = (float*)malloc(sizeof(float) * (size_t)R * H);
  for (int r = 0; r < R; ++r) {
    float* yr = y + (size_t)r * H;
    for (int i = 0; i < H; ++i) yr[i] = q36o_bf16_to_f32(a->h[(size_t)r * H + i]);
    if (a->norm_w) {
      float ss = q36o_dot_canon(yr, yr, H);
      float rstd = 1.f / sqrtf(ss / (float)H + a->eps);
      for (int i = 0; i < H; ++i) yr[i] = bf((yr[i] * rstd) * (1.f + q36o_bf16_to_f32(a->norm_w[i])));
    }
  }
#pragma omp parallel for schedule(dynamic, 1)
  for (int r = 0; r < R; ++r) {
    const float* yr = y + (size_t)r * H;
    float best = -INFINITY;
    int bi = 0;
    for (int n = 0; n < V; ++n) {
      const int8_t* w = a->wq + (size_t)n * H;
      double acc = 0.0;
      for (int i = 0; i < H; ++i) acc += (double)yr[i] * (double)w[i];
      float lg = bf((float)acc * a->ws[n]);
      if (a->logits) a->logits[(size_t)r * V + n] = q36o_f32_to_bf16(lg);
      if (lg > best) { best = lg; bi = n; }
    }
    a->ids[r] = bi;
  }
  free(y);
  return 0;
}

int q36o_lmhead(const q36o_lmhead_args* a) {
  int R = a->R, H = a->H, V = a->V;
  if (H % 512 || a->mode < 0 || a->mode > 2) return -1;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
  if (a->mode == 2) return lmhead_w8a16(a);
  const int two = a->mode == 1;
  if (a->n_threads > 0) omp_set_num_threads(a->n_threads);
  /* term u of row r at xq + (2 r + u) H (two terms) or r H (one term) */
  int8_t* xq = (int8_t*)malloc((size_t)R * H * (two ? 2 : 1));
  float* xs = (float*)malloc(sizeof(float) * R * (two ? 2 : 1));
#pragma omp parallel for schedule(static)
  for (int r = 0; r < R; ++r) {
    float* y = (float*)malloc(sizeof(float) * H);
    for (int i = 0; i < H; ++i) y[i] = q36o_bf16_to_f32(a->h[(size_t)r * H + i]);
    if (a->norm_w) {
      float ss = q36o_dot_canon(y, y, H);
      float rstd = 1.f / sqrtf(ss / (float)H + a->eps);
      for (int i = 0; i < H; ++i) y[i] = bf((y[i] * rstd) * (1.f + q36o_bf16_to_f32(a->norm_w[i])));
    }
    int8_t* q1 = xq + (size_t)r * H * (two ? 2 : 1);
    float* s1 = xs + (size_t)r * (two ? 2 : 1);
    quant_row_i8(y, H, q1, s1);
    if (two) {
      /* H/w8a8.py:33-36: the second term quantizes x - q1 * s1 (one fused multiply-add) by the
       * same rule */
      for (int i = 0; i < H; ++i) y[i] = fmaf(-(float)q1[i], s1[0], y[i]);
      quant_row_i8(y, H, q1 + H, s1 + 1);
    }
    free(y);
  }
#pragma omp parallel for schedule(dynamic, 1)
  for (int r = 0; r < R; ++r) {
    float best = -INFINITY;
    int bi = 0;
    const int8_t* q1 = xq + (size_t)r * H * (two ? 2 : 1);
    const float* s1 = xs + (size_t)r * (two ? 2 : 1);
    for (int n = 0; n < V; ++n) {
      int32_t acc = i8_row_dot(q1, a->wq + (size_t)n * H, H);
      float lg;
      if (two) {
        /* H/w8a8.py:66-70 (the contraction L/qk_proj_decode.cu:1103-1107 states):
         * fma(acc1, s1, acc2 * s2) * ws, rounded to bf16 */
        int32_t acc2 = i8_row_dot(q1 + H, a->wq + (size_t)n * H, H);
        lg = bf(fmaf((float)acc, s1[0], (float)acc2 * s1[1]) * a->ws[n]);
      } else {
        lg = bf(((float)acc * s1[0]) * a->ws[n]);
      }
      if (a->logits) a->logits[(size_t)r * V + n] = q36o_f32_to_bf16(lg);
      if (lg > best) { best = lg; bi = n; }
    }
    a->ids[r] = bi;
  }
  free(xq); free(xs);
  return 0;
}
