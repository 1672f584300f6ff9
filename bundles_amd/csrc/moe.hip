// Decode MoE block for gfx950: routing, expert lists, grouped W8A8 / e4m3 expert GEMMs on MFMA,
// SwiGLU, shared expert with sigmoid gate, and the weighted combine.
//
// Reference behaviour (R = qwen36_nodes_kb34, L = R/qwen36_layer):
//   routing + lists  L/qk_route.cu:213-358, top-k rule L/i8x_decode.py:98-117
//   up + SwiGLU      L/i8x_decode.py:305-341,151-156; L/qk_moe_up16.cu:110-124
//   down x weight    L/i8x_decode.py:343-422; L/qk_moe_dn16.cu:1-14
//   combine          L/i8x_decode.py:424-443; L/qk_route.cu:630-722
//
// Launch sequence on the caller's stream (no host synchronisation, graph-capturable):
//   1. route_logits  router GEMV (bf16 logits) + per-token activation quantization
//   2. route_topk    softmax / top-k / renormalise per token; the last workgroup (ticket) builds
//                    the expert lists (counts, offsets, perm, inv_perm, active) in canonical order
//   3. moe_up        one workgroup per (active expert, 16 gate + 16 up rows): weights streamed once
//                    into registers, MFMA over every 16-token tile of the expert, SwiGLU -> h
//   4. moe_down      one workgroup per (active expert, 64 output rows): h re-quantized in LDS,
//                    MFMA, x routing weight -> y per sorted position
//   5. moe_combine   out = bf16(fma(sigmoid(x . gate_w), y_shared, sum_j y_j))
// The shared expert is unit 0 of the up/down grids and covers every token.
#include <string.h>

#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int kMaxM = 256;
constexpr int kMaxE = 1024;

struct MoeDev {
  int M, E, H, I, k;
  const uint16_t* x;
  const uint16_t* wr;
  const float* bias;
  const int32_t* pos;
  const uint8_t* w13;
  const float* s13;
  const uint8_t* w2;
  const float* s2;
  const uint8_t* sw13;
  const float* ss13;
  const uint8_t* sw2;
  const float* ss2;
  const uint16_t* gate_w;
  uint16_t* out;
  float* logits;
  int32_t* ids;
  float* wts;
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm;
  int32_t* inv_perm;
  int32_t* active;
  int32_t* ctl;
  uint8_t* xq;
  float* xs;
  uint16_t* h;
  uint16_t* y;
  int32_t* dbg_acc13;
  int32_t* dbg_acc2;
  uint16_t* dbg_h;
};

__device__ __forceinline__ v4i ldg16(const uint8_t* p) { return *reinterpret_cast<const v4i*>(p); }
__device__ __forceinline__ v4i ldg16_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}
__device__ __forceinline__ v8i cat8(v4i a, v4i b) {
  v8i r = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return r;
}

__device__ __forceinline__ v4f mfma_fp8(v8i a, v8i b) {
  v4f z = {0.f, 0.f, 0.f, 0.f};
  // e4m3 x e4m3, unit (2^0) block scales: a plain 16x16x128 product.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}
__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------
// 1. router logits + activation quantization
// ------------------------------------------------------------------------------------------
// Router workgroup (expert group of 16, token tile of 16): wave w owns experts e0 .. e0+3; lane l
// accumulates the 8-element chunks c = l + 64 j with fma in (j, i) order, the 64 partials meet in
// an xor butterfly: the fixed reduction order the oracle restates (q36o_dot_canon).
template <int DT>
__global__ __launch_bounds__(256) void route_logits_kernel(MoeDev d, int n_router_wg) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int bid = blockIdx.x;
  if (bid < n_router_wg) {
    const int neg = d.E / 16;
    const int eg = bid % neg, tg = bid / neg;
    const int e0 = eg * 16 + wave * 4;
    const int t0 = tg * 16;
    const int nt = min(16, d.M - t0);
    float acc[16][4];
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[t][e] = 0.f;
    const int nj = d.H / 512;
    for (int j = 0; j < nj; ++j) {
      const int c = lane + 64 * j;
      v4i w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = ldg16(reinterpret_cast<const uint8_t*>(d.wr + (size_t)(e0 + e) * d.H + 8 * c));
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        if (t < nt) {
          v4i xv = ldg16(reinterpret_cast<const uint8_t*>(d.x + (size_t)(t0 + t) * d.H + 8 * c));
          float xf[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            xf[2 * q] = bf_lo((uint32_t)xv[q]);
            xf[2 * q + 1] = bf_hi((uint32_t)xv[q]);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float a = acc[t][e];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              a = __builtin_fmaf(xf[2 * q], bf_lo((uint32_t)w[e][q]), a);
              a = __builtin_fmaf(xf[2 * q + 1], bf_hi((uint32_t)w[e][q]), a);
            }
            acc[t][e] = a;
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      if (t < nt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = wave_sum_bfly(acc[t][e]);
          if (d.bias) v = v + d.bias[e0 + e];
          if (lane == e) d.logits[(size_t)(t0 + t) * d.E + e0 + e] = rbf(v);
        }
      }
    }
    return;
  }
  // Quantization workgroup: one token.  Thread tid owns the 8-element chunks tid + 256 r.
  const int t = bid - n_router_wg;
  const int tid = threadIdx.x;
  const int nr = d.H / 2048 > 0 ? d.H / 2048 : 1;
  __shared__ float red[4];
  float xf[4][8];
  float amax_t = 0.f;
  for (int r = 0; r < nr; ++r) {
    const int c = tid + 256 * r;
    if (8 * c < d.H) {
      v4i xv = ldg16(reinterpret_cast<const uint8_t*>(d.x + (size_t)t * d.H + 8 * c));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xf[r][2 * q] = bf_lo((uint32_t)xv[q]);
        xf[r][2 * q + 1] = bf_hi((uint32_t)xv[q]);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) xf[r][q] = 0.f;
    }
  }
  if constexpr (DT == Q36_MOE_INT8) {
    for (int r = 0; r < nr; ++r)
#pragma unroll
      for (int q = 0; q < 8; ++q) amax_t = fmaxf(amax_t, fabsf(xf[r][q]));
    amax_t = wave_max(amax_t);
    if (lane == 0) red[wave] = amax_t;
    __syncthreads();
    const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = amax / 127.f, safe = amax > 0.f ? s : 1.f;
    for (int r = 0; r < nr; ++r) {
      const int c = tid + 256 * r;
      if (8 * c < d.H) {
        uint32_t wd[2] = {0u, 0u};
#pragma unroll
        for (int q = 0; q < 8; ++q) wd[q >> 2] |= ((uint32_t)round_i8(xf[r][q] / safe) & 0xffu) << (8 * (q & 3));
        *reinterpret_cast<uint2*>(d.xq + (size_t)t * d.H + 8 * c) = make_uint2(wd[0], wd[1]);
      }
    }
    if (tid == 0) d.xs[t] = s;
  } else {
    // 128-channel groups: the 16 consecutive threads of a chunk run.
    const int ng = d.H / 128;
    for (int r = 0; r < nr; ++r) {
      const int c = tid + 256 * r;
      float m = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(xf[r][q]));
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
      if (8 * c < d.H) {
        const float s = m / 448.f, inv = m > 0.f ? 448.f / m : 0.f;
        uint32_t wd[2] = {0u, 0u};
#pragma unroll
        for (int q = 0; q < 8; ++q) wd[q >> 2] |= f2e4m3(xf[r][q] * inv) << (8 * (q & 3));
        *reinterpret_cast<uint2*>(d.xq + (size_t)t * d.H + 8 * c) = make_uint2(wd[0], wd[1]);
        if ((c & 15) == 0) d.xs[(size_t)t * ng + c / 16] = s;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// 2. top-k per token, then the expert lists (last workgroup)
// ------------------------------------------------------------------------------------------
__device__ void build_lists(const MoeDev& d) {
  __shared__ int cnt[kMaxE];
  __shared__ int off[kMaxE + 1];
  __shared__ uint32_t mask[kMaxE][kMaxM / 32];
  __shared__ int wsum[4], wact[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = d.E, S = d.M * d.k, mw = (d.M + 31) / 32;
  for (int e = tid; e < E; e += 256) {
    cnt[e] = 0;
    for (int w = 0; w < mw; ++w) mask[e][w] = 0u;
  }
  __syncthreads();
  for (int s = tid; s < S; s += 256) {
    const int e = __hip_atomic_load(d.ids + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (e >= 0) {
      const int t = s / d.k;
      atomicAdd(&cnt[e], 1);
      atomicOr(&mask[e][t >> 5], 1u << (t & 31));
    }
  }
  __syncthreads();
  // Exclusive scan of counts and of the active flags: thread tid owns experts 4 tid .. 4 tid + 3.
  int c4[4], csum = 0, asum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * tid + i;
    c4[i] = e < E ? cnt[e] : 0;
    csum += c4[i];
    asum += c4[i] > 0;
  }
  int ci = csum, ai = asum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int cn = __shfl_up(ci, o), an = __shfl_up(ai, o);
    if (lane >= o) { ci += cn; ai += an; }
  }
  if (lane == 63) { wsum[wave] = ci; wact[wave] = ai; }
  __syncthreads();
  int cbase = 0, abase = 0;
  for (int w = 0; w < wave; ++w) { cbase += wsum[w]; abase += wact[w]; }
  int ce = cbase + ci - csum, ae = abase + ai - asum;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * tid + i;
    if (e < E) {
      off[e] = ce;
      d.offsets[e] = ce;
      d.counts[e] = c4[i];
      if (c4[i] > 0) d.active[ae++] = e;
      ce += c4[i];
    }
  }
  if (tid == 255) {
    off[E] = ce;
    d.offsets[E] = ce;
    d.ctl[1] = ae;
  }
  __syncthreads();
  for (int s = tid; s < S; s += 256) {
    const int e = __hip_atomic_load(d.ids + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (e < 0) {
      d.inv_perm[s] = -1;
      continue;
    }
    const int t = s / d.k, tw = t >> 5;
    int rank = __popc(mask[e][tw] & ((1u << (t & 31)) - 1u));
    for (int w = 0; w < tw; ++w) rank += __popc(mask[e][w]);
    const int p = off[e] + rank;
    d.perm[p] = s;
    d.inv_perm[s] = p;
  }
  for (int p = off[E] + tid; p < S; p += 256) d.perm[p] = -1;
  if (tid == 0) d.ctl[0] = 0;  // reset the ticket for the next call
}

__global__ __launch_bounds__(256) void route_topk_kernel(MoeDev d) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t < d.M) {
    const bool valid = d.pos == nullptr || d.pos[t] != 0;
    if (!valid) {
      if (lane < d.k) {
        d.ids[t * d.k + lane] = -1;
        d.wts[t * d.k + lane] = 0.f;
      }
    } else {
      const int nm = d.E / 64;
      float lg[16];
      float mx = -__builtin_inff();
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        lg[m] = m < nm ? d.logits[(size_t)t * d.E + lane + 64 * m] : -__builtin_inff();
        mx = fmaxf(mx, lg[m]);
      }
      mx = wave_max(mx);
      float part = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m)
        if (m < nm) part = part + expf_q(lg[m] - mx);
      const float sum = wave_sum_bfly(part);
      uint32_t taken = 0u;
      float wsum = 0.f, my_p = 0.f;
      int my_id = -1;
      for (int j = 0; j < d.k; ++j) {
        float bv = -__builtin_inff();
        int bi = 0x7fffffff;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          const int id = lane + 64 * m;
          if (m < nm && !((taken >> m) & 1u) && (lg[m] > bv || (lg[m] == bv && id < bi))) {
            bv = lg[m];
            bi = id;
          }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float ov = __shfl_xor(bv, o);
          const int oi = __shfl_xor(bi, o);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        const float p = expf_q(bv - mx) / sum;
        wsum = wsum + p;
        if (lane == j) {
          my_p = p;
          my_id = bi;
        }
      }
      const float div = wsum > 0.f ? wsum : 1.f;
      if (lane < d.k) {
        d.ids[t * d.k + lane] = my_id;
        d.wts[t * d.k + lane] = my_p / div;
      }
    }
  }
  __shared__ int last;
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    const int old = atomicAdd(d.ctl, 1);
    last = old == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  build_lists(d);
}

// ------------------------------------------------------------------------------------------
// 3. up GEMM + SwiGLU
// ------------------------------------------------------------------------------------------
// Workgroup = (unit, chunk of 16 gate rows + the matching 16 up rows); unit 0 is the shared
// expert over all M tokens, unit u >= 1 the (u-1)-th active expert.  Wave w owns K range
// [w H/4, (w+1) H/4); its weight fragments are loaded once and reused for every 16-token tile.
// MFMA operands: src0 = activation tile (lane -> token row l%16), src1 = weight rows (lane ->
// row l%16); lane group l/16 carries the same K bytes of both, so the products pair up; the
// 16x16 result gives lane l column l%16 (weight row) and rows 4(l/16)+r (tokens).
template <int DT>
__global__ __launch_bounds__(256) void moe_up_kernel(MoeDev d) {
  constexpr int H = 2048;
  constexpr int KW = H / 4;                        // K per wave
  constexpr int NS = DT == Q36_MOE_FP8 ? KW / 128 : KW / 64;  // MFMA K steps per wave
  const int I = d.I;
  const int nch = I / 16;
  const int ug = blockIdx.x / nch, ch = blockIdx.x % nch;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lr = lane & 15, lgp = lane >> 4;
  const bool shared = ug == 0;
  const uint8_t* W;
  const float* S;
  int p0, cnt;
  if (shared) {
    W = d.sw13;
    S = d.ss13;
    p0 = d.M * d.k;
    cnt = d.M;
  } else {
    const int u = ug - 1;
    if (u >= d.ctl[1]) return;
    const int e = d.active[u];
    W = d.w13 + (size_t)e * 2 * I * H;
    S = d.s13 + (DT == Q36_MOE_FP8 ? (size_t)e * (2 * I / 128) * (H / 128) : (size_t)e * 2 * I);
    p0 = d.offsets[e];
    cnt = d.counts[e];
  }
  const int ng = ch * 16 + lr;  // this lane's gate row (its up row is I + ng)
  const int kw0 = wave * KW;
  constexpr int FB = DT == Q36_MOE_FP8 ? 32 : 16;  // fragment bytes per lane per step
  constexpr int KS = DT == Q36_MOE_FP8 ? 128 : 64;
  const uint8_t* bg = W + (size_t)ng * H + kw0 + lgp * FB;
  const uint8_t* bu = W + (size_t)(I + ng) * H + kw0 + lgp * FB;
  v4i Bg[NS][FB / 16], Bu[NS][FB / 16];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int h2 = 0; h2 < FB / 16; ++h2) {
      Bg[s][h2] = ldg16_nt(bg + s * KS + 16 * h2);
      Bu[s][h2] = ldg16_nt(bu + s * KS + 16 * h2);
    }
  // Per-lane weight scales.
  float wsg[NS], wsu[NS];
  if constexpr (DT == Q36_MOE_FP8) {
    const int nkb = H / 128;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      wsg[s] = S[(size_t)(ng / 128) * nkb + kw0 / 128 + s];
      wsu[s] = S[(size_t)((I + ng) / 128) * nkb + kw0 / 128 + s];
    }
  }
  __shared__ int red[4][2][64][4];                          // INT8: per-wave int32 partials
  __shared__ float redf[4][DT == Q36_MOE_FP8 ? NS : 1][2][64][4];  // FP8: one term per 128-block
  for (int t0 = 0; t0 < cnt; t0 += 16) {
    // activation rows of this tile
    const int ti = t0 + lr;
    int tok = -1;
    if (ti < cnt) tok = shared ? ti : d.perm[p0 + ti] / d.k;
    v4i A[NS][FB / 16];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int h2 = 0; h2 < FB / 16; ++h2) {
        if (tok >= 0) A[s][h2] = ldg16(d.xq + (size_t)tok * H + kw0 + s * KS + lgp * FB + 16 * h2);
        else A[s][h2] = v4i{0, 0, 0, 0};
      }
    if constexpr (DT == Q36_MOE_FP8) {
      // tokens of this lane's 4 output rows
      float xsv[4][NS];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tr = t0 + 4 * lgp + r;
        int tk = -1;
        if (tr < cnt) tk = shared ? tr : d.perm[p0 + tr] / d.k;
#pragma unroll
        for (int s = 0; s < NS; ++s) xsv[r][s] = tk >= 0 ? d.xs[(size_t)tk * (H / 128) + kw0 / 128 + s] : 0.f;
      }
      // Each 128-block term (block sum * xs * ws) goes to LDS; the epilogue adds the H/128 terms
      // in increasing block order from zero, the order of the block dequant sum.
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const v8i a8 = cat8(A[s][0], A[s][1]);
        const v4f rg = mfma_fp8(a8, cat8(Bg[s][0], Bg[s][1]));
        const v4f ru = mfma_fp8(a8, cat8(Bu[s][0], Bu[s][1]));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          redf[wave][s][0][lane][r] = (rg[r] * xsv[r][s]) * wsg[s];
          redf[wave][s][1][lane][r] = (ru[r] * xsv[r][s]) * wsu[s];
        }
      }
    } else {
      v4i ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        ag = mfma_i8(A[s][0], Bg[s][0], ag);
        au = mfma_i8(A[s][0], Bu[s][0], au);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red[wave][0][lane][r] = ag[r];
        red[wave][1][lane][r] = au[r];
      }
    }
    __syncthreads();
    {
      // epilogue: thread -> (lane' = tid % 64, r = tid / 64): token row 4 (lane'/16) + r, column lane' % 16
      const int l2 = threadIdx.x & 63, r = threadIdx.x >> 6;
      const int row = 4 * (l2 >> 4) + r, col = l2 & 15;
      const int ti2 = t0 + row;
      if (ti2 < cnt) {
        const int p = p0 + ti2;
        const int n = ch * 16 + col;
        float g, u;
        if constexpr (DT == Q36_MOE_FP8) {
          g = 0.f;
          u = 0.f;
#pragma unroll
          for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int s = 0; s < NS; ++s) {
              g = g + redf[w][s][0][l2][r];
              u = u + redf[w][s][1][l2][r];
            }
        } else {
          const int ai = red[0][0][l2][r] + red[1][0][l2][r] + red[2][0][l2][r] + red[3][0][l2][r];
          const int au = red[0][1][l2][r] + red[1][1][l2][r] + red[2][1][l2][r] + red[3][1][l2][r];
          if (d.dbg_acc13) {
            d.dbg_acc13[(size_t)p * 2 * I + n] = ai;
            d.dbg_acc13[(size_t)p * 2 * I + I + n] = au;
          }
          const int tk = shared ? ti2 : d.perm[p] / d.k;
          const float xsc = d.xs[tk];
          g = ((float)ai * xsc) * S[n];
          u = ((float)au * xsc) * S[I + n];
        }
        g = rbf(g);
        u = rbf(u);
        const uint32_t hb = f2bf((g / (1.f + expf_q(-g))) * u);
        d.h[(size_t)p * I + n] = (uint16_t)hb;
        if (d.dbg_h) d.dbg_h[(size_t)p * I + n] = (uint16_t)hb;
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------
// 4. down GEMM x routing weight
// ------------------------------------------------------------------------------------------
// Workgroup = (unit, chunk of 64 output rows).  Per 16-token tile the tile's h rows are loaded
// and quantized into LDS (int8 per row over I, e4m3 per 128-group); wave w owns K block
// [w I/4, (w+1) I/4) = one 128-group, four 16-row MFMA column tiles.
template <int DT>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeDev d) {
  constexpr int H = 2048, I = 512;
  constexpr int KW = I / 4;                                   // 128
  constexpr int NS = DT == Q36_MOE_FP8 ? KW / 128 : KW / 64;  // 1 or 2
  constexpr int FB = DT == Q36_MOE_FP8 ? 32 : 16;
  constexpr int KS = DT == Q36_MOE_FP8 ? 128 : 64;
  constexpr int nch = H / 64;
  const int ug = blockIdx.x / nch, ch = blockIdx.x % nch;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lgp = lane >> 4;
  const bool shared = ug == 0;
  const uint8_t* W;
  const float* S;
  int p0, cnt;
  if (shared) {
    W = d.sw2;
    S = d.ss2;
    p0 = d.M * d.k;
    cnt = d.M;
  } else {
    const int u = ug - 1;
    if (u >= d.ctl[1]) return;
    const int e = d.active[u];
    W = d.w2 + (size_t)e * H * I;
    S = d.s2 + (DT == Q36_MOE_FP8 ? (size_t)e * (H / 128) * (I / 128) : (size_t)e * H);
    p0 = d.offsets[e];
    cnt = d.counts[e];
  }
  const int kw0 = wave * KW;
  v4i B[4][NS][FB / 16];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const uint8_t* b = W + (size_t)(ch * 64 + nt * 16 + lr) * I + kw0 + lgp * FB;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int h2 = 0; h2 < FB / 16; ++h2) B[nt][s][h2] = ldg16_nt(b + s * KS + 16 * h2);
  }
  float wsc[4];
  if constexpr (DT == Q36_MOE_FP8) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) wsc[nt] = S[(size_t)((ch * 64 + nt * 16) / 128) * (I / 128) + wave];
  }
  __shared__ __align__(16) uint8_t hq[16][I];
  __shared__ float hs[16][4];
  __shared__ float red[4][4][64][4];
  for (int t0 = 0; t0 < cnt; t0 += 16) {
    {
      // quantize the tile's h rows: thread -> (row tid/16, 32 elements at 32 (tid%16))
      const int tr = tid >> 4, q16 = tid & 15;
      float hv[32];
      if (t0 + tr < cnt) {
        const uint8_t* src = reinterpret_cast<const uint8_t*>(d.h + (size_t)(p0 + t0 + tr) * I + q16 * 32);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const v4i raw = ldg16(src + 16 * v);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            hv[8 * v + 2 * q] = bf_lo((uint32_t)raw[q]);
            hv[8 * v + 2 * q + 1] = bf_hi((uint32_t)raw[q]);
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < 32; ++v) hv[v] = 0.f;
      }
      float m = 0.f;
#pragma unroll
      for (int v = 0; v < 32; ++v) m = fmaxf(m, fabsf(hv[v]));
      uint32_t wd[8];
      if constexpr (DT == Q36_MOE_FP8) {
        m = fmaxf(m, __shfl_xor(m, 1));
        m = fmaxf(m, __shfl_xor(m, 2));
        const float s = m / 448.f, inv = m > 0.f ? 448.f / m : 0.f;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          wd[v] = 0u;
#pragma unroll
          for (int q = 0; q < 4; ++q) wd[v] |= f2e4m3(hv[4 * v + q] * inv) << (8 * q);
        }
        if ((q16 & 3) == 0) hs[tr][q16 >> 2] = s;
      } else {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float s = m / 127.f, safe = m > 0.f ? s : 1.f;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          wd[v] = 0u;
#pragma unroll
          for (int q = 0; q < 4; ++q) wd[v] |= ((uint32_t)round_i8(hv[4 * v + q] / safe) & 0xffu) << (8 * q);
        }
        if (q16 == 0) hs[tr][0] = s;
      }
      uint4* dst = reinterpret_cast<uint4*>(&hq[tr][q16 * 32]);
      dst[0] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      dst[1] = make_uint4(wd[4], wd[5], wd[6], wd[7]);
    }
    __syncthreads();
    v4i A[NS][FB / 16];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int h2 = 0; h2 < FB / 16; ++h2)
        A[s][h2] = *reinterpret_cast<const v4i*>(&hq[lr][kw0 + s * KS + lgp * FB + 16 * h2]);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      if constexpr (DT == Q36_MOE_FP8) {
        const v4f rr = mfma_fp8(cat8(A[0][0], A[0][1]), cat8(B[nt][0][0], B[nt][0][1]));
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][nt][lane][r] = (rr[r] * hs[4 * lgp + r][wave]) * wsc[nt];
      } else {
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = mfma_i8(A[s][0], B[nt][s][0], acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][nt][lane][r] = __int_as_float(acc[r]);
      }
    }
    __syncthreads();
    {
      const int nt = tid >> 6, l2 = tid & 63;
      const int n = ch * 64 + nt * 16 + (l2 & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * (l2 >> 4) + r;
        const int ti2 = t0 + row;
        if (ti2 < cnt) {
          const int p = p0 + ti2;
          const float wt = shared ? 1.f : d.wts[d.perm[p]];
          float yv;
          if constexpr (DT == Q36_MOE_FP8) {
            const float acc = (((0.f + red[0][nt][l2][r]) + red[1][nt][l2][r]) + red[2][nt][l2][r]) + red[3][nt][l2][r];
            yv = acc * wt;
          } else {
            const int ai = __float_as_int(red[0][nt][l2][r]) + __float_as_int(red[1][nt][l2][r]) +
                           __float_as_int(red[2][nt][l2][r]) + __float_as_int(red[3][nt][l2][r]);
            if (d.dbg_acc2) d.dbg_acc2[(size_t)p * H + n] = ai;
            yv = (((float)ai * hs[row][0]) * S[n]) * wt;
          }
          d.y[(size_t)p * H + n] = (uint16_t)f2bf(yv);
        }
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------
// 5. combine
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeDev d) {
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool valid = d.pos == nullptr || d.pos[t] != 0;
  __shared__ float gate_s;
  if (valid && wave == 0) {
    float acc = 0.f;
    for (int j = 0; j < d.H / 512; ++j) {
      const int c = lane + 64 * j;
      const v4i xv = ldg16(reinterpret_cast<const uint8_t*>(d.x + (size_t)t * d.H + 8 * c));
      const v4i gv = ldg16(reinterpret_cast<const uint8_t*>(d.gate_w + 8 * c));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc = __builtin_fmaf(bf_lo((uint32_t)xv[q]), bf_lo((uint32_t)gv[q]), acc);
        acc = __builtin_fmaf(bf_hi((uint32_t)xv[q]), bf_hi((uint32_t)gv[q]), acc);
      }
    }
    acc = wave_sum_bfly(acc);
    if (lane == 0) gate_s = sigmoid_q(acc);
  }
  __syncthreads();
  const int S = d.M * d.k;
  for (int c = tid; 8 * c < d.H; c += 256) {
    uint4 o = make_uint4(0u, 0u, 0u, 0u);
    if (valid) {
      float acc[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = 0.f;
      for (int j = 0; j < d.k; ++j) {
        const int p = d.inv_perm[t * d.k + j];
        const v4i yv = ldg16(reinterpret_cast<const uint8_t*>(d.y + (size_t)p * d.H + 8 * c));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = acc[2 * q] + bf_lo((uint32_t)yv[q]);
          acc[2 * q + 1] = acc[2 * q + 1] + bf_hi((uint32_t)yv[q]);
        }
      }
      const v4i sv = ldg16(reinterpret_cast<const uint8_t*>(d.y + (size_t)(S + t) * d.H + 8 * c));
      const float g = gate_s;
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[q] = pack_bf2(__builtin_fmaf(g, bf_lo((uint32_t)sv[q]), acc[2 * q]),
                        __builtin_fmaf(g, bf_hi((uint32_t)sv[q]), acc[2 * q + 1]));
      o = make_uint4(w[0], w[1], w[2], w[3]);
    }
    *reinterpret_cast<uint4*>(d.out + (size_t)t * d.H + 8 * c) = o;
  }
}

// ------------------------------------------------------------------------------------------
// prepare-time quantizers
// ------------------------------------------------------------------------------------------
// One workgroup per row; K % 8 == 0.
__global__ __launch_bounds__(256) void quant_rows_i8_kernel(const uint16_t* w, int K, int8_t* q, float* s) {
  const size_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* src = w + row * K;
  float m = 0.f;
  for (int c = tid; 8 * c < K; c += 256) {
    const v4i v = ldg16(reinterpret_cast<const uint8_t*>(src + 8 * c));
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf_lo((uint32_t)v[i])), fabsf(bf_hi((uint32_t)v[i]))));
  }
  __shared__ float red[4];
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = amax / 127.f, safe = amax > 0.f ? sc : 1.f;
  for (int c = tid; 8 * c < K; c += 256) {
    const v4i v = ldg16(reinterpret_cast<const uint8_t*>(src + 8 * c));
    uint32_t wd[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wd[i >> 1] |= ((uint32_t)round_i8(bf_lo((uint32_t)v[i]) / safe) & 0xffu) << (16 * (i & 1));
      wd[i >> 1] |= ((uint32_t)round_i8(bf_hi((uint32_t)v[i]) / safe) & 0xffu) << (16 * (i & 1) + 8);
    }
    *reinterpret_cast<uint2*>(q + row * K + 8 * c) = make_uint2(wd[0], wd[1]);
  }
  if (tid == 0) s[row] = sc;
}

// One workgroup per 128x128 block: thread -> (row tid/2, 64 columns at 64 (tid%2)).
__global__ __launch_bounds__(256) void quant_blocks_e4m3_kernel(const uint16_t* w, int K, uint8_t* q, float* s) {
  const int kb = blockIdx.x, nb = blockIdx.y, nkb = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t row = (size_t)nb * 128 + (tid >> 1);
  const int col = kb * 128 + (tid & 1) * 64;
  const uint16_t* src = w + row * K + col;
  float v[64];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const v4i r = ldg16(reinterpret_cast<const uint8_t*>(src + 8 * c));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[8 * c + 2 * i] = bf_lo((uint32_t)r[i]);
      v[8 * c + 2 * i + 1] = bf_hi((uint32_t)r[i]);
    }
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) m = fmaxf(m, fabsf(v[i]));
  __shared__ float red[4];
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = amax / 448.f, inv = amax > 0.f ? 448.f / amax : 0.f;
  uint8_t* dst = q + row * K + col;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wd[i] = 0u;
#pragma unroll
      for (int b = 0; b < 4; ++b) wd[i] |= f2e4m3(v[16 * c + 4 * i + b] * inv) << (8 * b);
    }
    *reinterpret_cast<uint4*>(dst + 16 * c) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }
  if (tid == 0) s[(size_t)nb * nkb + kb] = sc;
}

// ------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------
int layout(int M, int E, int H, int I, int k, int dtype, q36_moe_ws_layout* L) {
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t r = o;
    o = align_up(o + bytes, 256);
    return r;
  };
  const size_t S = (size_t)M * k;
  // ctl first: its offset must not depend on M, so the ticket stays zero across calls of any size
  L->ctl = take(sizeof(int32_t) * 64);
  L->logits = take(sizeof(float) * (size_t)M * E);
  L->ids = take(sizeof(int32_t) * S);
  L->wts = take(sizeof(float) * S);
  L->counts = take(sizeof(int32_t) * E);
  L->offsets = take(sizeof(int32_t) * (E + 1));
  L->perm = take(sizeof(int32_t) * S);
  L->inv_perm = take(sizeof(int32_t) * S);
  L->active = take(sizeof(int32_t) * E);
  L->xq = take((size_t)M * H);
  L->xs = take(sizeof(float) * (size_t)M * (dtype == Q36_MOE_FP8 ? H / 128 : 1));
  L->h = take(sizeof(uint16_t) * (S + M) * I);
  L->y = take(sizeof(uint16_t) * (S + M) * H);
  L->total = o;
  return 0;
}

int validate(const q36_moe_args* a, MoeDev* d, bool need_experts) {
  Q36_REQUIRE(a != nullptr, "q36_moe: null args");
  Q36_REQUIRE(a->dtype == Q36_MOE_INT8 || a->dtype == Q36_MOE_FP8, "q36_moe: dtype %d unknown", a->dtype);
  Q36_REQUIRE(a->H == 2048, "q36_moe: H=%d unsupported (this build is specialised to H=2048)", a->H);
  Q36_REQUIRE(a->I == 512, "q36_moe: I=%d unsupported (this build is specialised to I=512)", a->I);
  Q36_REQUIRE(a->E >= 64 && a->E % 64 == 0 && a->E <= kMaxE, "q36_moe: E=%d must be a multiple of 64 in [64,%d]",
              a->E, kMaxE);
  Q36_REQUIRE(a->topk >= 1 && a->topk <= 16 && a->topk <= a->E, "q36_moe: topk=%d must be in [1, min(16, E)]",
              a->topk);
  Q36_REQUIRE(a->M >= 1 && a->M <= kMaxM, "q36_moe: M=%d must be in [1,%d]", a->M, kMaxM);
  Q36_REQUIRE(a->x && a->router_w && a->workspace, "q36_moe: x, router_w and workspace are required");
  Q36_REQUIRE(!need_experts || (a->w13 && a->s13 && a->w2 && a->s2 && a->sw13 && a->ss13 && a->sw2 && a->ss2 &&
                                a->gate_w && a->out),
              "q36_moe_forward: an expert weight, scale, gate_w or out pointer is null");
  const void* ptrs[] = {a->x, a->router_w, a->w13, a->w2, a->sw13, a->sw2, a->gate_w, a->out, a->workspace,
                        a->dbg_acc13, a->dbg_acc2, a->dbg_h};
  for (const void* p : ptrs) Q36_REQUIRE(aligned16(p), "q36_moe: pointer %p is not 16-byte aligned", p);
  Q36_REQUIRE((reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0, "q36_moe: workspace must be 256-byte aligned");
  q36_moe_ws_layout L;
  layout(a->M, a->E, a->H, a->I, a->topk, a->dtype, &L);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_moe: workspace of %zu bytes is smaller than the %zu required",
              a->workspace_bytes, L.total);
  char* ws = static_cast<char*>(a->workspace);
  *d = MoeDev{a->M, a->E, a->H, a->I, a->topk,
              static_cast<const uint16_t*>(a->x), static_cast<const uint16_t*>(a->router_w), a->router_bias,
              a->positions, static_cast<const uint8_t*>(a->w13), a->s13, static_cast<const uint8_t*>(a->w2), a->s2,
              static_cast<const uint8_t*>(a->sw13), a->ss13, static_cast<const uint8_t*>(a->sw2), a->ss2,
              static_cast<const uint16_t*>(a->gate_w), static_cast<uint16_t*>(a->out),
              reinterpret_cast<float*>(ws + L.logits), reinterpret_cast<int32_t*>(ws + L.ids),
              reinterpret_cast<float*>(ws + L.wts), reinterpret_cast<int32_t*>(ws + L.counts),
              reinterpret_cast<int32_t*>(ws + L.offsets), reinterpret_cast<int32_t*>(ws + L.perm),
              reinterpret_cast<int32_t*>(ws + L.inv_perm), reinterpret_cast<int32_t*>(ws + L.active),
              reinterpret_cast<int32_t*>(ws + L.ctl), reinterpret_cast<uint8_t*>(ws + L.xq),
              reinterpret_cast<float*>(ws + L.xs), reinterpret_cast<uint16_t*>(ws + L.h),
              reinterpret_cast<uint16_t*>(ws + L.y), a->dbg_acc13, a->dbg_acc2,
              static_cast<uint16_t*>(a->dbg_h)};
  return Q36_OK;
}

int launch_route(const MoeDev& d, int dtype, hipStream_t st) {
  const int n_router = (d.E / 16) * ((d.M + 15) / 16);
  if (dtype == Q36_MOE_FP8)
    route_logits_kernel<Q36_MOE_FP8><<<n_router + d.M, 256, 0, st>>>(d, n_router);
  else
    route_logits_kernel<Q36_MOE_INT8><<<n_router + d.M, 256, 0, st>>>(d, n_router);
  route_topk_kernel<<<(d.M + 3) / 4, 256, 0, st>>>(d);
  return check_launch("q36_moe_route");
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" size_t q36_moe_workspace_bytes(int32_t M, int32_t E, int32_t H, int32_t I, int32_t topk, int32_t dtype) {
  q36_moe_ws_layout L;
  layout(M, E, H, I, topk, dtype, &L);
  return L.total;
}

extern "C" int q36_moe_workspace_layout(int32_t M, int32_t E, int32_t H, int32_t I, int32_t topk, int32_t dtype,
                                        q36_moe_ws_layout* out) {
  Q36_REQUIRE(out != nullptr, "q36_moe_workspace_layout: null out");
  return layout(M, E, H, I, topk, dtype, out);
}

extern "C" int q36_moe_route(const q36_moe_args* a, q36_stream_t stream) {
  MoeDev d;
  int rc = validate(a, &d, false);
  if (rc) return rc;
  return launch_route(d, a->dtype, static_cast<hipStream_t>(stream));
}

namespace q36 {
namespace {
int launch_up(const MoeDev& d, int dtype, hipStream_t st) {
  const int units = 1 + (d.E < d.M * d.k ? d.E : d.M * d.k);
  if (dtype == Q36_MOE_FP8)
    moe_up_kernel<Q36_MOE_FP8><<<units * (d.I / 16), 256, 0, st>>>(d);
  else
    moe_up_kernel<Q36_MOE_INT8><<<units * (d.I / 16), 256, 0, st>>>(d);
  return check_launch("q36_moe_up");
}
int launch_down(const MoeDev& d, int dtype, hipStream_t st) {
  const int units = 1 + (d.E < d.M * d.k ? d.E : d.M * d.k);
  if (dtype == Q36_MOE_FP8)
    moe_down_kernel<Q36_MOE_FP8><<<units * (d.H / 64), 256, 0, st>>>(d);
  else
    moe_down_kernel<Q36_MOE_INT8><<<units * (d.H / 64), 256, 0, st>>>(d);
  return check_launch("q36_moe_down");
}
int launch_combine(const MoeDev& d, hipStream_t st) {
  moe_combine_kernel<<<d.M, 256, 0, st>>>(d);
  return check_launch("q36_moe_combine");
}
}  // namespace
}  // namespace q36

extern "C" int q36_moe_up(const q36_moe_args* a, q36_stream_t stream) {
  MoeDev d;
  int rc = validate(a, &d, true);
  return rc ? rc : launch_up(d, a->dtype, static_cast<hipStream_t>(stream));
}

extern "C" int q36_moe_down(const q36_moe_args* a, q36_stream_t stream) {
  MoeDev d;
  int rc = validate(a, &d, true);
  return rc ? rc : launch_down(d, a->dtype, static_cast<hipStream_t>(stream));
}

extern "C" int q36_moe_combine(const q36_moe_args* a, q36_stream_t stream) {
  MoeDev d;
  int rc = validate(a, &d, true);
  return rc ? rc : launch_combine(d, static_cast<hipStream_t>(stream));
}

extern "C" int q36_moe_forward(const q36_moe_args* a, q36_stream_t stream) {
  MoeDev d;
  int rc = validate(a, &d, true);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((rc = launch_route(d, a->dtype, st))) return rc;
  if ((rc = launch_up(d, a->dtype, st))) return rc;
  if ((rc = launch_down(d, a->dtype, st))) return rc;
  return launch_combine(d, st);
}

extern "C" int q36_quant_rows_i8(const void* w, int64_t N, int32_t K, int8_t* q, float* s, q36_stream_t stream) {
  Q36_REQUIRE(w && q && s, "q36_quant_rows_i8: null pointer");
  Q36_REQUIRE(N >= 1 && N <= 0x7fffffff && K >= 8 && K % 8 == 0, "q36_quant_rows_i8: bad shape N=%lld K=%d",
              (long long)N, K);
  Q36_REQUIRE(aligned16(w) && aligned16(q), "q36_quant_rows_i8: w and q must be 16-byte aligned");
  quant_rows_i8_kernel<<<(unsigned)N, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const uint16_t*>(w), K,
                                                                                  q, s);
  return check_launch("q36_quant_rows_i8");
}

extern "C" int q36_quant_blocks_e4m3(const void* w, int64_t N, int32_t K, uint8_t* q, float* s, q36_stream_t stream) {
  Q36_REQUIRE(w && q && s, "q36_quant_blocks_e4m3: null pointer");
  Q36_REQUIRE(N >= 128 && N % 128 == 0 && N / 128 <= 65535 && K >= 128 && K % 128 == 0,
              "q36_quant_blocks_e4m3: N=%lld and K=%d must be positive multiples of 128", (long long)N, K);
  Q36_REQUIRE(aligned16(w) && aligned16(q), "q36_quant_blocks_e4m3: w and q must be 16-byte aligned");
  dim3 grid(K / 128, (unsigned)(N / 128));
  quant_blocks_e4m3_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const uint16_t*>(w), K, q,
                                                                               s);
  return check_launch("q36_quant_blocks_e4m3");
}
