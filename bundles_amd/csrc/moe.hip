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
//   1. route_logits  router GEMV (bf16 logits, canonical reduction order) + per-token activation
//                    quantization and shared-expert gate sigmoid(x . gate_w); also clears the
//                    per-expert counters for step 2
//   2. route_topk    softmax / top-k / renormalise, one wave per token; each pick appends its slot
//                    (t * k + j) to its expert's slot list through an atomic counter (the order
//                    inside a list changes no output: every result is stored by slot)
//      route_lists   (q36_moe_route only) the canonical maps: counts, offsets, perm, inv_perm and
//                    active, expert ascending, then token, then pick
//   3. moe_up        one workgroup per (unit, 64 gate + 64 up rows): each wave streams its 16 + 16
//                    weight rows over the whole K once, MFMA against every 16-token tile of the
//                    unit's tokens (staged in LDS), SwiGLU -> h per slot
//   4. moe_down      one workgroup per (unit, 128 output rows): the unit's h rows re-quantized
//                    once in LDS, MFMA, x routing weight -> y per slot
//   5. moe_combine   out = bf16(fma(gate, y_shared, sum_j y_j)), j in pick order, gate from step 1
// The shared expert is unit 0 of the up/down grids and covers every token.
#include <string.h>

#include <mutex>

#include <type_traits>

#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int kMaxM = 256;
constexpr int kMaxE = 1024;
// Token block of an expert work item: a workgroup takes at most 64 of a unit's tokens (one, two or
// four 16-token tiles); an expert past 64 tokens gets one more work item per further 64.  (Blocks of
// 32 were measured at decode batch 64: the hot experts' extra workgroups push the grid past one
// round of two workgroups a CU, and the layer got slower, 60.1 against 59.2 us.)
constexpr int kTokBlock = 64, kTokBlockShift = 6;

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
  float* gate;      // [M] sigmoid(x . gate_w) of each token (route_logits, when gate_w is given)
  int32_t* ids;
  float* wts;
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm;
  int32_t* inv_perm;
  int32_t* active;
  int32_t* ctl;
  int32_t* ecount;  // tokens per expert, counted by route_topk (zeroed by route_logits)
  int32_t* eact;    // routed work items e | j << 16 (token block j of expert e), in the order
                    // route_topk opened them: [0, E) experts' first blocks (ctl[2] counts them),
                    // [E, 2E) their further blocks, past 64 tokens (ctl[3])
  int32_t* elist;   // [E][M] slots of each expert, in the order route_topk met them
  int nsh;          // the shared expert's token blocks past its first: ceil(M / kTokBlock) - 1
  uint8_t* xq;
  float* xs;
  uint16_t* h;
  uint16_t* y;
  int32_t* dbg_acc13;
  int32_t* dbg_acc2;
  uint16_t* dbg_h;
  uint16_t* resid;        // the fused add-norm (norm_out != nullptr)
  const uint16_t* norm_w;
  float norm_eps;
  uint16_t* norm_out;
  uint8_t* norm_q8;       // norm_out's e4m3 codes (fragment order when norm_q8_frag), or null
  float* norm_q8s;
  int norm_q8_frag;
  // this block's own input add-norm, run by the route kernel (in_norm_w != nullptr): x is formed
  // there from in_delta + in_resid, in_resid_out receives the bf16 sum, xn (optional) the normed rows
  const uint16_t* in_delta;
  const uint16_t* in_resid;
  uint16_t* in_resid_out;
  const uint16_t* in_norm_w;
  float in_eps;
  uint16_t* xn;
};

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
// Router workgroup = TT tokens x 4 EPW experts; wave w owns experts e0 .. e0 + EPW - 1.  The x tile
// is staged in LDS as fp32 (each bf16 unpacked once, when the tile is filled, instead of once per
// wave and expert group); lane l keeps the 8-element chunks c = l + 64 j (j < H/512) of its EPW expert
// rows in registers and accumulates every (token, expert) dot with fma in (j, i) order.  The 64 lane
// partials of each output then meet in a recursive-halving reduce-scatter (xor 32, 16, ... over the
// NO = TT EPW outputs), then the xor butterfly's remaining stages: every sum pairs the same two
// operands as the xor butterfly (offsets 32 .. 1) of q36o_dot_canon, so the logits are
// bit-identical to the oracle's.
// One reduce-scatter stage over N values: lanes whose bit O is set keep the upper half, and add the
// partner's (lane l ^ O) copy of it.  O = 32 / 16: v_permlane32_swap / v_permlane16_swap of the
// halves (v[i], v[i + N / 2]) leaves, in every lane, the kept value and the partner's in its two
// results (no select); below 16 a select per half and a DPP / swizzle move.  Every sum pairs the same
// two operands as a __shfl_xor stage.
template <int N, int O>
__device__ __forceinline__ void rs_stage(float* v, int lane) {
  if constexpr (O == 32 || O == 16) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const uint32_t a = __float_as_uint(v[i]), b = __float_as_uint(v[i + N / 2]);
      uint32_t r0, r1;
      if constexpr (O == 32) {
        const auto p = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        r0 = p[0], r1 = p[1];
      } else {
        const auto p = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        r0 = p[0], r1 = p[1];
      }
      v[i] = __uint_as_float(r0) + __uint_as_float(r1);
    }
  } else {
    const bool hi = (lane & O) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float send = hi ? v[i] : v[i + N / 2];
      const float keep = hi ? v[i + N / 2] : v[i];
      v[i] = keep + lane_xor<O>(send);
    }
  }
}
// The xor butterfly's stages O, O / 2, .. 1 on one value (O <= 16; O = 0: none)
template <int O>
__device__ __forceinline__ float bfly_from(float v) {
  if constexpr (O == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return bfly_from<8>(__uint_as_float(p[0]) + __uint_as_float(p[1]));
  } else if constexpr (O >= 1) {
    return bfly_from<O / 2>(v + lane_xor<O>(v));
  } else {
    return v;
  }
}
// Stages xor O, O / 2, ... until one value is left: lane l then holds output (l / (64 / N)) % N
// (its bits above log2(64 / N)), summed over the lanes that share those bits.
template <int N, int O>
__device__ __forceinline__ void rs_all(float* v, int lane) {
  if constexpr (N > 1) {
    rs_stage<N, O>(v, lane);
    rs_all<N / 2, O / 2>(v, lane);
  }
}
constexpr int kRouteH = 2048;
// Router shapes, TT tokens x EPW experts a wave, by batch: one token group per 1 or 2 tokens, groups
// of 4 up to 16 tokens and of 8 up to 32 with EPW = 2 (64 workgroups a token group: the GEMV spread
// over many CUs, no wave computing a padding token's copy of another token), from 33 tokens on
// TT = 8, EPW = 4 (each unpacked activation feeds 4 experts; one workgroup a CU at batch 64), and past
// 128 tokens EPW = 8 (32 experts a workgroup: half the workgroups, so half the re-reads of each
// token group's rows and, with the input add-norm, half the redundant norms; measured at 256 rows:
// the layer 92.0 -> 90.9 us, the hybrid step with the add-norm in the route 938-946 -> 924-927 us).
constexpr int kRouteT4Max = 16, kRouteE2Max = 32, kRouteE4Max = 128;
// The block's input add-norm into a route workgroup's fp32 tile (256 threads, H = 2048: thread c owns
// the 8-element chunk c of each of the TT rows): z = delta + resid, then the sum of squares of each
// row in q36_add_rmsnorm's order (lane l of one wave takes chunks l + 64 j, fma from zero in (j,
// element) order, then the xor butterfly) and the normed row, bf16-rounded, in place of z.  Ends with
// the tile holding the rows x of the block; the caller's barrier publishes it.  ROW_OUT (one row, the
// row's quantization workgroup): also in_resid_out <- bf16(z) and, when xn is set, xn <- x.
template <int TT, bool ROW_OUT = false>
__device__ __forceinline__ void in_norm_tile(const MoeDev& d, int t0, float4 (*xlo)[kRouteH / 8],
                                             float4 (*xhi)[kRouteH / 8]) {
  static_assert(!ROW_OUT || TT == 1, "one row per quantization workgroup");
  const int c = threadIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ float rstd_s[TT];
  float z[TT][8];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const size_t at = (size_t)min(t0 + t, d.M - 1) * kRouteH + 8 * c;
    const v4i dv = ldg16(reinterpret_cast<const uint8_t*>(d.in_delta + at));
    const v4i rv = ldg16(reinterpret_cast<const uint8_t*>(d.in_resid + at));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      z[t][2 * q] = bf_lo((uint32_t)dv[q]) + bf_lo((uint32_t)rv[q]);
      z[t][2 * q + 1] = bf_hi((uint32_t)dv[q]) + bf_hi((uint32_t)rv[q]);
    }
    xlo[t][c] = make_float4(z[t][0], z[t][1], z[t][2], z[t][3]);
    xhi[t][c] = make_float4(z[t][4], z[t][5], z[t][6], z[t][7]);
    if constexpr (ROW_OUT) {
      v4i nv;
#pragma unroll
      for (int q = 0; q < 4; ++q) nv[q] = (int)pack_bf2(z[t][2 * q], z[t][2 * q + 1]);
      *reinterpret_cast<v4i*>(d.in_resid_out + at) = nv;
    }
  }
  const v4i wv = ldg16(reinterpret_cast<const uint8_t*>(d.in_norm_w + 8 * c));
  __syncthreads();
  for (int t = wave; t < TT; t += 4) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kRouteH / 512; ++j) {
      const float4 lo = xlo[t][lane + 64 * j], hi = xhi[t][lane + 64 * j];
      const float e[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(e[i], e[i], acc);
    }
    const float ss = wave_sum_bfly(acc);
    if (lane == 0) rstd_s[t] = 1.f / sqrtf(ss / (float)kRouteH + d.in_eps);
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const float rstd = rstd_s[t];
    float y[8];
    v4i yv;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t p = pack_bf2((z[t][2 * q] * rstd) * (1.f + bf_lo((uint32_t)wv[q])),
                                  (z[t][2 * q + 1] * rstd) * (1.f + bf_hi((uint32_t)wv[q])));
      yv[q] = (int)p;
      y[2 * q] = bf_lo(p);
      y[2 * q + 1] = bf_hi(p);
    }
    xlo[t][c] = make_float4(y[0], y[1], y[2], y[3]);
    xhi[t][c] = make_float4(y[4], y[5], y[6], y[7]);
    if constexpr (ROW_OUT)
      if (d.xn) *reinterpret_cast<v4i*>(d.xn + (size_t)t0 * kRouteH + 8 * c) = yv;
  }
}
__host__ __device__ constexpr int route_tt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= kRouteT4Max ? 4 : 8; }
__host__ __device__ constexpr int route_epw(int M) { return M <= kRouteE2Max ? 2 : M <= kRouteE4Max ? 4 : 8; }
template <int DT, int TT, int EPW>
__global__ __launch_bounds__(256) void route_logits_kernel(MoeDev d, int n_router_wg) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int bid = blockIdx.x;
  constexpr int EW = 4 * EPW;  // experts a workgroup
  __shared__ float4 xlo[TT][kRouteH / 8], xhi[TT][kRouteH / 8];  // elements 0-3 / 4-7 of each chunk
  if (bid < n_router_wg) {
    constexpr int NJ = kRouteH / 512;
    constexpr int NO = TT * EPW;  // outputs per wave: (expert, token) pairs
    static_assert(NO >= 2 && NO <= 64 && (NO & (NO - 1)) == 0, "outputs per wave: a power of two, 2 .. 64");
    constexpr int S = __builtin_ctz(NO);  // reduce-scatter stages
    const int neg = d.E / EW;
    const int eg = bid % neg, tg = bid / neg;
    const int e0 = eg * EW + wave * EPW;
    const int t0 = tg * TT;
    v4i w[EPW][NJ];
#pragma unroll
    for (int x = 0; x < EPW; ++x)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        w[x][j] = ldg16(reinterpret_cast<const uint8_t*>(d.wr + (size_t)(e0 + x) * kRouteH + 8 * (lane + 64 * j)));
    if (d.in_norm_w) {
      in_norm_tile<TT>(d, t0, xlo, xhi);
    } else {
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int tok = min(t0 + t, d.M - 1);
        const v4i xv = ldg16(reinterpret_cast<const uint8_t*>(d.x + (size_t)tok * kRouteH + 8 * threadIdx.x));
        xlo[t][threadIdx.x] = make_float4(bf_lo((uint32_t)xv[0]), bf_hi((uint32_t)xv[0]), bf_lo((uint32_t)xv[1]),
                                          bf_hi((uint32_t)xv[1]));
        xhi[t][threadIdx.x] = make_float4(bf_lo((uint32_t)xv[2]), bf_hi((uint32_t)xv[2]), bf_lo((uint32_t)xv[3]),
                                          bf_hi((uint32_t)xv[3]));
      }
    }
    __syncthreads();
    float v[NO];  // output o = x * TT + t
#pragma unroll
    for (int i = 0; i < NO; ++i) v[i] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float wf[EPW][8];
#pragma unroll
      for (int x = 0; x < EPW; ++x)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          wf[x][2 * q] = bf_lo((uint32_t)w[x][j][q]);
          wf[x][2 * q + 1] = bf_hi((uint32_t)w[x][j][q]);
        }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const float4 lo = xlo[t][lane + 64 * j], hi = xhi[t][lane + 64 * j];
        const float xf[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int x = 0; x < EPW; ++x) {
          float a = v[x * TT + t];
#pragma unroll
          for (int i = 0; i < 8; ++i) a = __builtin_fmaf(xf[i], wf[x][i], a);
          v[x * TT + t] = a;
        }
      }
    }
    rs_all<NO, 32>(v, lane);
    const float tot0 = bfly_from<(32 >> S)>(v[0]);
    float tot = tot0;
    const int o = (lane >> (6 - S)) & (NO - 1), t = o % TT, e = e0 + o / TT;
    if ((lane & ((64 >> S) - 1)) == 0 && t0 + t < d.M) {
      if (d.bias) tot = tot + d.bias[e];
      d.logits[(size_t)(t0 + t) * d.E + e] = rbf(tot);
    }
    return;
  }
  // Quantization workgroup: one token.  Thread tid owns the 8-element chunks tid + 256 r.  Wave 0
  // also forms the shared expert's gate sigmoid(x . gate_w) in the canonical order (lane l owns the
  // 8-element chunks l + 64 j, fma in (j, element) order from zero, then an xor butterfly), so the
  // combine reads one value instead of a dot product.
  const int t = bid - n_router_wg;
  const int tid = threadIdx.x;
  // with the input add-norm, the row x is formed here (H = 2048: thread tid owns chunk tid) and
  // stays in the LDS tile for the gate's canonical order
  if (d.in_norm_w) {
    in_norm_tile<1, true>(d, t, xlo, xhi);
    __syncthreads();
  }
  if (wave == 0 && d.gate_w != nullptr) {
    float xe[kRouteH / 512][8];
    v4i gg[kRouteH / 512], xg[kRouteH / 512];
    // every load first, none under a branch (the compiler waits for a load at the join of the branch
    // it sits in: four round trips one after another).  The x chunks go through a buffer resource
    // that is empty when the row comes from the LDS tile (reads of it return zeros, touch nothing).
    const bool tile = d.in_norm_w != nullptr;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(tile ? reinterpret_cast<const void*>(d.gate_w) : reinterpret_cast<const void*>(d.x)), (short)0,
        tile ? 0 : d.M * kRouteH * 2, 0x00020000);
#pragma unroll
    for (int j = 0; j < kRouteH / 512; ++j) {
      const int c = lane + 64 * j;
      gg[j] = ldg16(reinterpret_cast<const uint8_t*>(d.gate_w + 8 * c));
      xg[j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (t * kRouteH + 8 * c) * 2, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kRouteH / 512; ++j) {
      const int c = lane + 64 * j;
      const float4 lo = xlo[0][c], hi = xhi[0][c];  // the tile row (read either way, used with it)
      const float tv[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xe[j][2 * q] = tile ? tv[2 * q] : bf_lo((uint32_t)xg[j][q]);
        xe[j][2 * q + 1] = tile ? tv[2 * q + 1] : bf_hi((uint32_t)xg[j][q]);
      }
    }
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kRouteH / 512; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc = __builtin_fmaf(xe[j][2 * q], bf_lo((uint32_t)gg[j][q]), acc);
        acc = __builtin_fmaf(xe[j][2 * q + 1], bf_hi((uint32_t)gg[j][q]), acc);
      }
    acc = wave_sum_bfly(acc);
    if (lane == 0) d.gate[t] = sigmoid_q(acc);
  }
  if (t == 0) {
    for (int e = tid; e < d.E; e += 256) d.ecount[e] = 0;  // route_topk counts into them next
    if (tid == 0) {
      d.ctl[2] = 0;
      d.ctl[3] = 0;
    }
  }
  const int nr = d.H / 2048 > 0 ? d.H / 2048 : 1;
  __shared__ float red[4];
  float xf[4][8];
  float amax_t = 0.f;
  for (int r = 0; r < nr; ++r) {
    const int c = tid + 256 * r;
    if (d.in_norm_w) {  // this thread's own chunk of the tile
      const float4 lo = xlo[0][c], hi = xhi[0][c];
      xf[r][0] = lo.x, xf[r][1] = lo.y, xf[r][2] = lo.z, xf[r][3] = lo.w;
      xf[r][4] = hi.x, xf[r][5] = hi.y, xf[r][6] = hi.z, xf[r][7] = hi.w;
    } else if (8 * c < d.H) {
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
      m = __uint_as_float(row16_max_u32(__float_as_uint(m)));  // m >= 0: the bits order as the values
      if (8 * c < d.H) {
        const float s = m / 448.f, inv = m > 0.f ? 448.f / m : 0.f;
        uint32_t wd[2] = {0u, 0u};
#pragma unroll
        for (int q = 0; q < 8; q += 2) wd[q >> 2] |= f2e4m3x2_hw(xf[r][q] * inv, xf[r][q + 1] * inv) << (8 * (q & 3));
        *reinterpret_cast<uint2*>(d.xq + (size_t)t * d.H + 8 * c) = make_uint2(wd[0], wd[1]);
        if ((c & 15) == 0) d.xs[(size_t)t * ng + c / 16] = s;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// 2. top-k per token (one wave per token), and the expert lists
// ------------------------------------------------------------------------------------------
// Order-preserving 32-bit key of a bf16-valued logit and its expert id: (value desc, id asc) is
// the unsigned order of the key, so one wave max picks the next expert of the top-k.
__device__ __forceinline__ uint32_t logit_key(float lg, int id) {
  uint32_t b = __float_as_uint(lg) >> 16;  // the logits hold bf16 values exactly
  if (b == 0x8000u) b = 0u;                // -0 ties with +0
  b = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return (b << 16) | (0xffffu - (uint32_t)id);
}
__device__ __forceinline__ float key_logit(uint32_t key) {
  uint32_t b = key >> 16;
  b = (b & 0x8000u) ? (b & 0x7fffu) : (~b & 0xffffu);
  return __uint_as_float(b << 16);
}

// Sorts the NM keys of a lane into descending order (bitonic network, NM a power of two).
template <int NM>
__device__ __forceinline__ void sort_desc(uint32_t* key) {
#pragma unroll
  for (int k2 = 2; k2 <= NM; k2 <<= 1)
#pragma unroll
    for (int j = k2 >> 1; j > 0; j >>= 1)
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        const int l = i ^ j;
        if (l > i) {
          const uint32_t hi = max(key[i], key[l]), lo = min(key[i], key[l]);
          const bool desc = (i & k2) == 0;
          key[i] = desc ? hi : lo;
          key[l] = desc ? lo : hi;
        }
      }
}

// softmax / top-k / renormalise (L/i8x_decode.py:98-117).  One wave per token; lane l holds the
// experts l + 64 m (NM = E / 64 keys, padded with zero keys to a power of two), sorted descending
// in the lane, so each of the k picks is one wave max over the lanes' heads and a shift in the
// winning lane.  The weights keep the oracle's arithmetic: p_j = exp(v_j - v_0) / sum in lane j,
// their total added in pick order.
// EXACT: E == 64 NM (every key of a lane is an expert; no per-key bounds test).  KF: k fixed at
// compile time (0: d.k), so the picks unroll and the softmax's exponentials, which need only the
// first pick (the maximum), interleave with the later picks' cross-lane maxima.
template <int NM, bool EXACT, int KF>
__global__ __launch_bounds__(64) void route_topk_kernel(MoeDev d) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x;  // one wave (and workgroup) per token: a batch's tokens on as many CUs
  if (t >= d.M) return;
  const int E = d.E, k = KF ? KF : d.k, nm = EXACT ? NM : E / 64;
  const bool valid = d.pos == nullptr || d.pos[t] != 0;
  if (!valid) {
    if (lane < k) {
      d.ids[t * k + lane] = -1;
      d.wts[t * k + lane] = 0.f;
    }
    return;
  }
  float lg[NM];
  uint32_t key[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) lg[m] = d.logits[(size_t)t * E + lane + 64 * (m < nm ? m : nm - 1)];
#pragma unroll
  for (int m = 0; m < NM; ++m) key[m] = m < nm ? logit_key(lg[m], lane + 64 * m) : 0u;
  sort_desc<NM>(key);
  float my_v = 0.f;
  int my_id = -1;
  // pick j: one wave max over the lanes' heads; keys are distinct, so one lane pops its head (a bit
  // select per key, no index arithmetic)
  auto pick = [&](int j) {
    const uint32_t win = wave_max_u32(key[0]);
    const float v = key_logit(win);
    my_v = lane == j ? v : my_v;
    my_id = lane == j ? (int)(0xffffu - (win & 0xffffu)) : my_id;
    const uint32_t pop = key[0] == win ? 0xffffffffu : 0u;
#pragma unroll
    for (int i = 0; i + 1 < NM; ++i) key[i] = (key[i + 1] & pop) | (key[i] & ~pop);
    key[NM - 1] &= ~pop;
    return v;
  };
  const float mx = pick(0);
  float part = 0.f;
  if constexpr (KF > 0) {
    // exponential m goes between picks m + 1 and m + 2 (the sum keeps its order m = 0, 1, ...)
#pragma unroll
    for (int j = 1; j < KF; ++j) {
      pick(j);
      if (j - 1 < NM && j - 1 < nm) part = part + expf_q(lg[j - 1] - mx);
    }
#pragma unroll
    for (int m = KF - 1; m < NM; ++m)
      if (m < nm) part = part + expf_q(lg[m] - mx);
  } else {
#pragma unroll
    for (int m = 0; m < NM; ++m)
      if (m < nm) part = part + expf_q(lg[m] - mx);
    for (int j = 1; j < k; ++j) pick(j);  // k is uniform
  }
  const float sum = wave_sum_bfly(part);
  const float my_p = lane < k ? expf_q(my_v - mx) / sum : 0.f;
  float wsum = 0.f;
  for (int j = 0; j < k; ++j) wsum = wsum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_p), j));
  const float div = wsum > 0.f ? wsum : 1.f;
  if (lane < k) {
    d.ids[t * k + lane] = my_id;
    d.wts[t * k + lane] = my_p / div;
    // the expert's slot list and the active-expert list, for the expert kernels (their order
    // follows the atomics; every output element is computed from its own row, so the results do
    // not depend on it)
    const int pos = atomicAdd(&d.ecount[my_id], 1);
    d.elist[(size_t)my_id * d.M + pos] = t * k + lane;
    // an expert's first token, and every 64th after it, opens a token block: one work item of the
    // expert kernels.  First blocks go to one compact list, further blocks (a hot expert's, past 64
    // tokens, four-tile work) to another that the expert kernels' grid takes first, so that with
    // more items than a round of workgroups the heavy ones are not left for the second round.
    if (pos == 0)
      d.eact[atomicAdd(&d.ctl[2], 1)] = my_id;
    else if ((pos & (kTokBlock - 1)) == 0)
      d.eact[d.E + atomicAdd(&d.ctl[3], 1)] = my_id | ((pos >> kTokBlockShift) << 16);
  }
}

// Expert lists in LDS, in canonical order (expert asc, token asc, j asc): counts, exclusive
// offsets, the active experts, and perm (sorted position -> slot t*k + j).  Every workgroup of
// the expert kernels builds them from ids in its prologue (a 256-thread pass over M*k ids), so
// no workgroup waits on another; with `publish` the workgroup also writes them to the workspace.
struct Lists {
  int* cnt;      // [E]
  int* off;      // [E+1]
  int* active;   // [E]
  uint32_t* mask;  // [E][mw]
  int* perm;     // [M*k]
  int* misc;     // [0] n_active, [1..4] wave count totals, [5..8] wave active totals
};
__host__ __device__ inline size_t lists_lds_bytes(int E, int M, int k) {
  const int mw = (M + 31) / 32;
  return sizeof(int) * ((size_t)E + (E + 1) + E + (size_t)E * mw + (size_t)M * k + 16);
}
__device__ __forceinline__ Lists lists_carve(char* base, int E, int M, int k) {
  Lists L;
  const int mw = (M + 31) / 32;
  int* p = reinterpret_cast<int*>(base);
  L.cnt = p;
  p += E;
  L.off = p;
  p += E + 1;
  L.active = p;
  p += E;
  L.mask = reinterpret_cast<uint32_t*>(p);
  p += E * mw;
  L.perm = p;
  p += M * k;
  L.misc = p;
  return L;
}
__device__ void lists_build(const MoeDev& d, const Lists& L, bool publish) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = d.E, M = d.M, k = d.k, S = M * k, mw = (M + 31) / 32;
  for (int e = tid; e < E; e += 256) {
    L.cnt[e] = 0;
    for (int w = 0; w < mw; ++w) L.mask[e * mw + w] = 0u;
  }
  __syncthreads();
  for (int s = tid; s < S; s += 256) {
    const int e = d.ids[s];
    if (e >= 0) {
      const int t = s / k;
      atomicAdd(&L.cnt[e], 1);
      atomicOr(&L.mask[e * mw + (t >> 5)], 1u << (t & 31));
    }
  }
  __syncthreads();
  // exclusive scans of counts and active flags: thread tid owns experts 4 tid .. 4 tid + 3
  int c4[4], csum = 0, asum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * tid + i;
    c4[i] = e < E ? L.cnt[e] : 0;
    csum += c4[i];
    asum += c4[i] > 0;
  }
  int ci = csum, ai = asum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int cn = __shfl_up(ci, o), an = __shfl_up(ai, o);
    if (lane >= o) {
      ci += cn;
      ai += an;
    }
  }
  if (lane == 63) {
    L.misc[1 + wave] = ci;
    L.misc[5 + wave] = ai;
  }
  __syncthreads();
  int ce = ci - csum, ae = ai - asum;
  for (int w = 0; w < wave; ++w) {
    ce += L.misc[1 + w];
    ae += L.misc[5 + w];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * tid + i;
    if (e < E) {
      L.off[e] = ce;
      if (c4[i] > 0) L.active[ae++] = e;
      ce += c4[i];
    }
  }
  if (tid == 255) {
    L.off[E] = ce;
    L.misc[0] = ae;
  }
  __syncthreads();
  for (int s = tid; s < S; s += 256) {
    const int e = d.ids[s];
    int p = -1;
    if (e >= 0) {
      const int t = s / k, tw = t >> 5;
      int rank = __popc(L.mask[e * mw + tw] & ((1u << (t & 31)) - 1u));
      for (int w = 0; w < tw; ++w) rank += __popc(L.mask[e * mw + w]);
      p = L.off[e] + rank;
      L.perm[p] = s;
    }
    if (publish) {
      d.inv_perm[s] = p;
      if (p >= 0) d.perm[p] = s;
    }
  }
  if (publish) {
    for (int p = L.off[E] + tid; p < S; p += 256) d.perm[p] = -1;
    for (int e = tid; e < E; e += 256) {
      d.counts[e] = L.cnt[e];
      d.offsets[e] = L.off[e];
    }
    const int na = L.misc[0];
    for (int u = tid; u < na; u += 256) d.active[u] = L.active[u];
    if (tid == 0) {
      d.offsets[E] = L.off[E];
      d.ctl[1] = na;
    }
  }
  __syncthreads();
}

// Lists alone (q36_moe_route): one workgroup builds and publishes them.
__global__ __launch_bounds__(256) void route_lists_kernel(MoeDev d) {
  extern __shared__ __align__(16) char dyn_lds[];
  const Lists L = lists_carve(dyn_lds, d.E, d.M, d.k);
  lists_build(d, L, true);
}

// ------------------------------------------------------------------------------------------
// Expert work: token lists, MFMA fragments
// ------------------------------------------------------------------------------------------
// The expert kernels take an expert's tokens from the per-expert slot lists route_topk builds
// (elist, ecount; the order inside a list changes no output, every result is stored by slot); the
// shared expert lists slot M*k + t of every non-padding token.  h and y are indexed by slot, so no
// sorted-position lists sit on the forward path (q36_moe_route still publishes them).
// Unit u of an expert kernel: 0 is the shared expert (slots M*k + t of the non-padding tokens),
// u >= 1 the (u-1)-th entry of the active list, whose expert e the caller has read already (with
// the active count, in one round trip).  The list is fetched in two steps, so the caller can put its
// first weight loads between them: slots_request issues the loads (the expert's count and its whole
// list row, one entry a thread; for the shared expert the positions), slots_finish fills slots[] in
// LDS and returns the count.  Vector loads complete in issue order, so loads issued after the request
// do not delay it.
struct SlotReq {
  int v;  // routed unit: list entry tid; shared unit: position of token tid (0 marks padding)
};
__device__ __forceinline__ SlotReq slots_request(const MoeDev& d, int unit, int e) {
  const int tid = threadIdx.x;
  if (unit == 0) {
    const int pbytes = d.pos ? d.M * 4 : 0;
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc((void*)d.pos, (short)0, pbytes, 0x00020000);
    return SlotReq{(int)__builtin_amdgcn_raw_buffer_load_b32(prs, tid < d.M ? tid * 4 : pbytes, 0, 0)};
  }
  const int lbytes = d.M * 4;
  const __amdgpu_buffer_rsrc_t lrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(d.elist + (size_t)e * d.M), (short)0, lbytes, 0x00020000);
  return SlotReq{(int)__builtin_amdgcn_raw_buffer_load_b32(lrs, tid < d.M ? tid * 4 : lbytes, 0, 0)};
}
// toks (when given) receives each slot's token row, one division per thread here instead of one per
// row copy later
__device__ __forceinline__ int slots_finish(const MoeDev& d, int unit, int e, const SlotReq& r, int* slots,
                                            int* wtot, int* toks) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (unit != 0) {
    // the expert's count by a scalar load through the constant address space (the expert kernels
    // never write ecount; a plain load here is compiled as a vector load, which would complete
    // behind the weights); issued here, after the caller's weight loads, it does not hold them up
    const int cnt = ((const __attribute__((address_space(4))) int*)(d.ecount))[e];
    if (tid < cnt) {
      slots[tid] = r.v;
      if (toks) toks[tid] = r.v / d.k;  // a routed slot is token * k + pick
    }
    __syncthreads();
    return cnt;
  }
  // the shared expert: slot M*k + t of every non-padding token, in token order (ballot compaction)
  const int my = tid < d.M && (d.pos == nullptr || r.v != 0) ? d.M * d.k + tid : -1;
  const unsigned long long b = __ballot(my >= 0);
  const int below = __popcll(b & ((1ull << lane) - 1ull));
  if (lane == 0) wtot[wave] = __popcll(b);
  __syncthreads();
  int base = 0, tot = 0;
  for (int w = 0; w < 4; ++w) {
    base += w < wave ? wtot[w] : 0;
    tot += wtot[w];
  }
  if (my >= 0) {
    slots[base + below] = my;
    if (toks) toks[base + below] = tid;
  }
  __syncthreads();
  return tot;
}
// The work item of expert-kernel workgroup b (8 consecutive workgroups per item, one per slice, on
// the 8 XCDs).  Items 0 .. nsh are the shared expert's token blocks; the items after them are the
// routed blocks route_topk listed, compact at the front of the grid (idle past its count), so the
// workgroups with work are dispatched first and a hot expert's later blocks start with the rest.
// The list entry and its count come in one round trip (the entry's index does not depend on the
// count).  e: -2 idle, -1 the shared expert, else the expert; unit 0 is the shared expert, 1 routed.
struct WorkItem {
  int unit, e, tb, grp;
};
__device__ __forceinline__ WorkItem work_item(const MoeDev& d) {
  const int b = blockIdx.x, x = b >> 3, r = x - 1 - d.nsh;
  WorkItem it;
  it.grp = b & 7;
  if (r < 0) {
    it.unit = 0;
    it.e = -1;
    it.tb = x;
    return it;
  }
  it.unit = 1;
  if (d.M <= kTokBlock) {
    // no further blocks: the first-block list alone, its count and entry in one round trip
    const int n = d.ctl[2];
    const int ent = d.eact[min(r, d.E - 1)];
    asm volatile("" ::"s"(n), "s"(ent));  // both loads issued before either is tested
    it.e = r < n ? ent : -2;
    it.tb = 0;
    return it;
  }
  // further blocks first, then the first blocks (the entry's index depends on the further count: a
  // second round trip, past 64 tokens only)
  const int nx = d.ctl[3], n = d.ctl[2];
  const int i = r < nx ? d.E + r : r - nx;
  const int ent = d.eact[min(i, 2 * d.E - 1)];
  it.e = r < nx + n ? (ent & 0xffff) : -2;
  it.tb = ent >> 16;
  return it;
}

constexpr int kMoeH = 2048, kMoeI = 512;

// ------------------------------------------------------------------------------------------
// 3. up GEMM + SwiGLU
// ------------------------------------------------------------------------------------------
// Workgroup = (unit, group of 4 chunks); unit 0 is the shared expert, unit 1 + e expert e (the
// workgroup returns at once when e has no tokens).  Each wave owns one chunk: 16 gate rows and
// the matching 16 up rows over the whole K = H, streamed from HBM in 16 stages of 128 bytes per
// row with kUpD stages in flight; no reduction across waves.  The activation rows of up to 64
// tokens (4 tiles of 16) are shared by the four waves through LDS (one tile: the whole K; four
// tiles: 512-byte K chunks through two buffers); the token list, rows and scales are requested
// before the weights.
// Weights are stored in MFMA fragment order (q36_pack_frag8).  Per stage a lane holds 32 bytes of
// its row (row = lane % 16, bytes 32 (lane / 16) of the 128-byte stage) of both operands -- one e4m3 16x16x128 MFMA, or two int8 16x16x64 MFMAs on the two 16-byte
// halves (their K pairing is the same for src0 and src1, so the int32 sums are exact).  The
// 16x16 result gives lane l weight row l%16 and token rows 4(l/16)+r; SwiGLU happens in the
// lane.  For e4m3 the block sums are accumulated as acc = fma(block sum, xs * ws, acc) in
// increasing block order from zero.
constexpr int kUpD = 2;                    // weight stages in flight per wave
constexpr int kUpBuf0 = 16 * (kMoeH + 16);  // 16 padded whole-K rows, or one 64 x 512-byte chunk
constexpr int kUpBuf1 = 16 * (kMoeH + 16);  // the second tile's 16 rows, or the other chunk
constexpr int kUpGroups = kMoeI / 16 / 4;  // workgroups per unit (4 chunks each)
// Buffer load of 16 bytes per lane straight into LDS (lane l writes lds + 16 l); offsets past the
// buffer's size read as zero.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds, 16, voff, 0, 0, 0);
}

template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void moe_up_kernel(MoeDev d) {
  constexpr int H = kMoeH, I = kMoeI, NSTG = H / 128, TG = 64;
  // activation rows: buffer 0 holds tile 0's 16 padded whole-K rows (one- and two-tile groups) or
  // the even K chunks of a four-tile group, buffer 1 tile 1's rows or the odd chunks.  Separate
  // objects, so the compiler sees that a copy into one buffer does not touch reads of the other.
  __shared__ __align__(16) uint8_t a_b0[kUpBuf0];
  __shared__ __align__(16) uint8_t a_b1[kUpBuf1];
  __shared__ __align__(16) float xs_t[TG * NSTG];            // [NSTG][TG] (token fastest)
  __shared__ float ws_l[(2 * I / 128) * NSTG];               // [2I/128][NSTG]
  __shared__ int slots[kMaxM];
  __shared__ int toks[kMaxM];  // token row of each slot
  __shared__ int wtot[4];
  static_assert(kUpGroups == 8, "8 workgroups per work item");
  const WorkItem it = work_item(d);
  if (it.e == -2) return;
  const int unit = it.unit, grp = it.grp, e = it.e, g0 = it.tb << kTokBlockShift;
  const bool shared = unit == 0;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lgp = lane >> 4;
  const uint8_t* W = shared ? d.sw13 : d.w13 + (size_t)e * 2 * I * H;
  const float* S = shared ? d.ss13
                          : d.s13 + (DT == Q36_MOE_FP8 ? (size_t)e * (2 * I / 128) * NSTG : (size_t)e * 2 * I);
  const int ch = grp * 4 + wave;
  const int ng = ch * 16 + lr;
  // weights in fragment order: 16-row tile t, stage s at (t * NSTG + s) * 2048, the lane's two
  // 16-byte halves at 16 lane and 1024 + 16 lane (one 1 KB contiguous load per half per wave)
  // Buffer loads: the stage offset goes in the scalar offset, so the unrolled stages share one
  // address register (global loads would need a 64-bit address per stage: the 2 KB steps
  // overflow their immediate offset).
  const int chu = __builtin_amdgcn_readfirstlane(ch);
  const __amdgpu_buffer_rsrc_t grs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(W + ((size_t)chu * NSTG << 11)), (short)0, NSTG << 11, 0x00020000);
  const __amdgpu_buffer_rsrc_t urs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + ((size_t)(I / 16 + chu) * NSTG << 11)), (short)0, NSTG << 11, 0x00020000);
  const int lo = lane * 16;
  v4i Bq[kUpD][4];
  auto issue = [&](int s, int q) {
    Bq[q][0] = __builtin_amdgcn_raw_buffer_load_b128(grs, lo, s * 2048, 2);
    Bq[q][1] = __builtin_amdgcn_raw_buffer_load_b128(grs, lo, s * 2048 + 1024, 2);
    Bq[q][2] = __builtin_amdgcn_raw_buffer_load_b128(urs, lo, s * 2048, 2);
    Bq[q][3] = __builtin_amdgcn_raw_buffer_load_b128(urs, lo, s * 2048 + 1024, 2);
  };
  // the token list is requested, then the first group's first weight stages, as soon as the expert
  // is known; the activation rows and their scales (which depend on the list) follow
  const SlotReq req = slots_request(d, unit, e);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < kUpD; ++s) issue(s, s);
  __builtin_amdgcn_sched_barrier(0);
  const int cnt = slots_finish(d, unit, e, req, slots, wtot, toks);
  if (cnt <= g0) return;
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)d.xq, (short)0, d.M * H, 0x00020000);
  constexpr int NXS = DT == Q36_MOE_FP8 ? NSTG : 1;  // activation scales per token
  const int xsbytes = d.M * NXS * 4;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc((void*)d.xs, (short)0, xsbytes, 0x00020000);
  const int n = ch * 16 + lr;
  // One group of up to TG tokens with NTT 16-token tiles (rows past the group's tokens are zero):
  // per 128-byte stage every fragment and scale read first, then the independent MFMAs, then the
  // scaled accumulates (e4m3: in block order from zero), then SwiGLU -> h per slot.  One- and
  // two-tile groups hold their rows' whole K in LDS (a tile a buffer); a four-tile group streams K.
  auto group = [&](int g0, auto nttc, auto firstc) {
    constexpr int NTT = decltype(nttc)::value;
    constexpr bool FIRST = decltype(firstc)::value;  // the weight stages 0 .. kUpD-1 are in flight
    // activation rows in LDS: one- and two-tile groups hold their rows' whole K (padded rows, tile t
    // in buffer t); a four-tile group streams K in 4 chunks of 512 bytes through two buffers, so the
    // next chunk's copy overlaps the current chunk's stages and the weight stream never drains.
    // Ring rows are unpadded: 16-byte piece p of row r sits at position p ^ (r % 16), which puts
    // the 16 rows of one MFMA read on distinct banks.
    static_assert(NTT == 1 || NTT == 2 || NTT == 4, "one, two or four token tiles");
    constexpr int NC = NTT == 4 ? 4 : 1, KC = H / NC, SPC = NSTG / NC;
    constexpr int ROWB = NC == 1 ? KC + 16 : KC, BUFB = 16 * (NC == 1 ? 1 : NTT) * ROWB;
    static_assert(BUFB <= kUpBuf0 && BUFB <= kUpBuf1, "activation rows exceed their buffers");
    static_assert(NC == 1 || kUpD <= SPC, "a chunk must issue a full window of weight stages");
    using Acc = typename std::conditional<DT == Q36_MOE_FP8, v4f, v4i>::type;
    // The byte offset of each row this lane copies (its token row, or past the activations for rows
    // past the group, which read as zero), formed once for all chunks.  The token reads are made
    // unconditional: left to the compiler they sat in branches, one LDS round trip per copy.
    // One or two tiles: wave w copies rows w, w + 4, ..., 1 KB per call (lane l: bytes 16 l ..).
    // Four tiles: one call fills two rows (lanes 0-31 row 2m, lanes 32-63 row 2m + 1), wave w takes
    // the row pairs w, w + 4, ..., and a lane fetches the piece that belongs at its position.
    constexpr int NRC = NC == 1 ? 4 * NTT : 8 * NTT / 4;
    int rowoff[NRC];
#pragma unroll
    for (int k = 0; k < NRC; ++k) {
      const int rr = NC == 1 ? wave + 4 * k : 2 * (wave + 4 * k) + (lane >> 5), ti = g0 + rr;
      int tk = toks[ti & (kMaxM - 1)];
      asm volatile("" : "+v"(tk));
      rowoff[k] = ti < cnt ? tk * H : d.M * H;
    }
    // chunk c of the group's rows into its buffer by buffer DMA
    auto rows_dma = [&](int c) {
      if constexpr (NC == 1) {
#pragma unroll
        for (int k = 0; k < NRC; ++k) {
          const int rr = wave + 4 * k;  // rows 0-15 tile 0 (buffer 0), 16-31 tile 1 (buffer 1)
          uint8_t* dst = (rr < 16 ? a_b0 : a_b1) + (rr & 15) * ROWB;
          const int voff = rowoff[k] < d.M * H ? rowoff[k] + lane * 16 : d.M * H;
#pragma unroll
          for (int h = 0; h < KC / 1024; ++h) dma16(xrs, dst + h * 1024, voff + h * 1024);
        }
      } else {
        uint8_t* buf = (c & 1) ? a_b1 : a_b0;
#pragma unroll
        for (int k = 0; k < NRC; ++k) {
          const int m = wave + 4 * k, rr = 2 * m + (lane >> 5), p = lane & 31;
          const int voff = rowoff[k] < d.M * H ? rowoff[k] + c * KC + 16 * (p ^ (rr & 15)) : d.M * H;
          dma16(xrs, buf + 2 * m * KC, voff);
        }
      }
    };
    // scales of the group (x: [NXS][TG], token fastest; e4m3 weights: [2I/128][NSTG]) into
    // registers now, into LDS after the weight stages are requested
    float xsr[TG * NSTG / 256], wsr = 0.f;
#pragma unroll
    for (int q = 0; q < TG * NSTG / 256; ++q) {
      const int i = tid + 256 * q, ti = g0 + i % TG, sx = i / TG;
      int tk = toks[ti & (kMaxM - 1)];
      asm volatile("" : "+v"(tk));
      const int off = ti < cnt && sx < NXS ? (tk * NXS + sx) * 4 : xsbytes;
      xsr[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, off, 0, 0));
    }
    if constexpr (DT == Q36_MOE_FP8) {
      constexpr int NW = (2 * I / 128) * NSTG;
      static_assert(NW <= 256, "one weight scale per thread");
      const __amdgpu_buffer_rsrc_t wss = __builtin_amdgcn_make_buffer_rsrc((void*)S, (short)0, NW * 4, 0x00020000);
      wsr = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wss, tid < NW ? tid * 4 : NW * 4, 0, 0));
    }
    rows_dma(0);
    if constexpr (!FIRST) {
#pragma unroll
      for (int s = 0; s < kUpD; ++s) issue(s, s);
    }
#pragma unroll
    for (int q = 0; q < TG * NSTG / 256; ++q) xs_t[tid + 256 * q] = xsr[q];
    if constexpr (DT == Q36_MOE_FP8)
      if (tid < (2 * I / 128) * NSTG) ws_l[tid] = wsr;
    // the rows (and for later groups not the weights, requested after them; the first group's
    // weights are older than the rows)
    if constexpr (FIRST)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * kUpD) : "memory");
    __syncthreads();
    asm volatile("" ::: "memory");
    Acc ag[NTT], au[NTT];
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      ag[tt] = Acc{0, 0, 0, 0};
      au[tt] = Acc{0, 0, 0, 0};
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c > 0) {
        // chunk c landed (its copy is older than the chunk's 4 * SPC weight loads) and every wave
        // is done with chunk c - 1, whose buffer the next copy reuses
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * SPC) : "memory");
        __syncthreads();
        asm volatile("" ::: "memory");
      }
      if (c + 1 < NC) rows_dma(c + 1);
#pragma unroll
      for (int sl = 0; sl < SPC; ++sl) {
        const int s = c * SPC + sl;
        const int q = s % kUpD;
        v4i a[NTT][2];
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
          // whole K: tile tt's rows in buffer tt; chunks: chunk c in buffer c % 2, rows of every tile
          const uint8_t* buf = NC == 1 ? (tt == 0 ? a_b0 : a_b1) : ((c & 1) ? a_b1 : a_b0);
          const int row = NC == 1 ? lr : tt * 16 + lr;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int piece = sl * 8 + lgp * 2 + h;  // 16-byte piece within the row's chunk
            a[tt][h] = *reinterpret_cast<const v4i*>(buf + row * ROWB + 16 * (NC == 1 ? piece : piece ^ lr));
          }
        }
        if constexpr (DT == Q36_MOE_FP8) {
          const float wg = ws_l[(ng / 128) * NSTG + s], wu = ws_l[((I + ng) / 128) * NSTG + s];
          const v8i bgq = cat8(Bq[q][0], Bq[q][1]), buq = cat8(Bq[q][2], Bq[q][3]);
#pragma unroll
          for (int tt = 0; tt < NTT; ++tt) {
            const v8i a8 = cat8(a[tt][0], a[tt][1]);
            const v4f rg = mfma_fp8(a8, bgq);
            const v4f ru = mfma_fp8(a8, buq);
            const float4 xsv = *reinterpret_cast<const float4*>(xs_t + s * TG + tt * 16 + 4 * lgp);
            const float xr[4] = {xsv.x, xsv.y, xsv.z, xsv.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              ag[tt][r] = __builtin_fmaf(rg[r], xr[r] * wg, ag[tt][r]);
              au[tt][r] = __builtin_fmaf(ru[r], xr[r] * wu, au[tt][r]);
            }
          }
          // the running sums are formed here (left alone, the compiler sinks the chain below the
          // stage loop and keeps every stage's MFMA results live)
#pragma unroll
          for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(ag[tt][r]), "+v"(au[tt][r]));
        } else {
#pragma unroll
          for (int tt = 0; tt < NTT; ++tt) {
            ag[tt] = mfma_i8(a[tt][0], Bq[q][0], ag[tt]);
            ag[tt] = mfma_i8(a[tt][1], Bq[q][1], ag[tt]);
            au[tt] = mfma_i8(a[tt][0], Bq[q][2], au[tt]);
            au[tt] = mfma_i8(a[tt][1], Bq[q][3], au[tt]);
          }
        }
        if (s + kUpD < NSTG) issue(s + kUpD, q);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ti = g0 + tt * 16 + 4 * lgp + r;
        if (ti < cnt) {
          const int s = slots[ti];
          float g, u;
          if constexpr (DT == Q36_MOE_FP8) {
            g = ag[tt][r];
            u = au[tt][r];
          } else {
            if (d.dbg_acc13) {
              d.dbg_acc13[(size_t)s * 2 * I + n] = ag[tt][r];
              d.dbg_acc13[(size_t)s * 2 * I + I + n] = au[tt][r];
            }
            const float xsc = xs_t[tt * 16 + 4 * lgp + r];
            g = ((float)ag[tt][r] * xsc) * S[n];
            u = ((float)au[tt][r] * xsc) * S[I + n];
          }
          g = rbf(g);
          u = rbf(u);
          const uint32_t hb = f2bf((g / (1.f + expf_q(-g))) * u);
          d.h[(size_t)s * I + n] = (uint16_t)hb;
          if (d.dbg_h) d.dbg_h[(size_t)s * I + n] = (uint16_t)hb;
        }
      }
  };
  // the work item's token block (at most 64 tokens) as one, two or four 16-token tiles (rows past
  // the tokens are zero)
  const int nb = min(cnt - g0, kTokBlock);
  if (nb <= 16)
    group(g0, std::integral_constant<int, 1>{}, std::true_type{});
  else if (nb <= 32)
    group(g0, std::integral_constant<int, 2>{}, std::true_type{});
  else
    group(g0, std::integral_constant<int, 4>{}, std::true_type{});
}

// ------------------------------------------------------------------------------------------
// 4. down GEMM x routing weight
// ------------------------------------------------------------------------------------------
// Workgroup = (unit, group of 4 x 64 output rows); each wave owns 64 rows (four 16-row MFMA
// tiles) over the whole K = I (4 stages of 128 bytes): 32 KB of weights per wave, loaded into
// registers right after the first group's h rows, so the grid (8 workgroups per active unit, two per CU) streams
// the down weights in a single round.  Tokens go in groups of up to 64 (one or four 16-token
// tiles): the workgroup loads every h row of the group, and the routing weight of every slot, in
// one go, quantizes the rows into LDS (e4m3 per 128-group, int8 per row), and every wave reads its
// MFMA operands from there.  The weights are the MFMA's first operand, so lane l ends with token
// l%16 and four consecutive output columns 4(l/16) .. +3: one 8-byte store per tile.  The weight
// tiles go in pairs, so one pair's accumulators and one stage's operands stay in registers.
constexpr int kDnRows = 64;
constexpr int kDnCT = kDnRows / 16;
static_assert(kDnCT == 4, "the down weights are issued as two tile pairs");
constexpr int kDnGroups = kMoeH / (4 * kDnRows);
constexpr int kDnTG = 64;
constexpr int kDnRow = kMoeI + 16;  // padded LDS row: 16 rows' 16-byte reads hit distinct banks
template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void moe_down_kernel(MoeDev d) {
  constexpr int H = kMoeH, I = kMoeI, NSTG = I / 128;
  __shared__ int slots[kMaxM];
  __shared__ int wtot[4];
  __shared__ __align__(16) uint8_t hq[kDnTG * kDnRow];
  __shared__ float hs[kDnTG][NSTG];      // activation scales per row (e4m3: per 128-group)
  __shared__ float wl[kDnTG];            // routing weight per row of the group
  __shared__ __align__(16) float sn[4 * kDnRows];  // int8 weight scale per output row of the workgroup
  static_assert(kDnGroups == 8, "8 workgroups per work item");
  const WorkItem it = work_item(d);
  if (it.e == -2) return;
  const int unit = it.unit, grp = it.grp, e = it.e, g0 = it.tb << kTokBlockShift;
  const bool shared = unit == 0;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lgp = lane >> 4;
  const uint8_t* W = shared ? d.sw2 : d.w2 + (size_t)e * H * I;
  const float* S =
      shared ? d.ss2 : d.s2 + (DT == Q36_MOE_FP8 ? (size_t)e * (H / 128) * NSTG : (size_t)e * H);
  const int n0 = __builtin_amdgcn_readfirstlane((grp * 4 + wave) * kDnRows);  // wave-uniform
  // weights in fragment order, loaded through one buffer resource per wave with the tile and
  // stage offsets in the scalar offset (one address register for all 32 loads)
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + ((size_t)(n0 >> 4) * NSTG << 11)), (short)0, kDnCT * NSTG << 11, 0x00020000);
  v4i B[kDnCT][NSTG][2];
  // K stages [S0, S1) of the tile pair c0, c0 + 1
  auto issue_weights = [&](auto c0c, auto s0c, auto s1c) {
    constexpr int C0 = decltype(c0c)::value, S0 = decltype(s0c)::value, S1 = decltype(s1c)::value;
#pragma unroll
    for (int ct = C0; ct < C0 + 2; ++ct)
#pragma unroll
      for (int s = S0; s < S1; ++s) {
        B[ct][s][0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, lane * 16, (ct * NSTG + s) << 11, 2);
        B[ct][s][1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, lane * 16, ((ct * NSTG + s) << 11) + 1024, 2);
      }
  };
  // the token list is requested and the first tile pair's first two K stages go out as soon as the
  // expert is known, then the first group's h rows, then the rest of the weights: the rows'
  // quantization waits for those 8 KB a wave only (vector loads complete in issue order) and overlaps
  // the remaining 24 KB (with the whole first pair, 16 KB, ahead of the rows the batch-64 layer was
  // 0.5 us slower)
  constexpr int kDnEarly = 2;
  static_assert(kDnEarly < NSTG, "the rest of the first pair goes out after the rows");
  const SlotReq req = slots_request(d, unit, e);
  __builtin_amdgcn_sched_barrier(0);
  issue_weights(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, kDnEarly>{});
  __builtin_amdgcn_sched_barrier(0);
  const int cnt = slots_finish(d, unit, e, req, slots, wtot, nullptr);
  if (cnt <= g0) return;
  // weight scales: e4m3 per 128x128 block (the wave's 64 rows sit in one block row), int8 per row
  float wsc[NSTG], snv = 0.f;
  if constexpr (DT == Q36_MOE_FP8) {
#pragma unroll
    for (int s = 0; s < NSTG; ++s) wsc[s] = S[(size_t)(n0 / 128) * NSTG + s];
  } else {
    snv = S[grp * 4 * kDnRows + tid];
  }
  const int hbytes = (d.M * d.k + d.M) * I * 2, tbytes = d.M * d.k * 4;
  const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc((void*)d.h, (short)0, hbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc((void*)d.wts, (short)0, tbytes, 0x00020000);
  auto group = [&](int g0, auto nttc, auto firstc) {
    constexpr int NTT = decltype(nttc)::value;
    constexpr bool FIRST = decltype(firstc)::value;
    {
      // load: thread -> rows tid/16 + 16 j (j < NTT), values 32 (tid%16) .. +31 of each; a
      // 128-group is four neighbouring threads, a row sixteen
      // (buffer loads: rows past the tokens read as zero without a branch, which would make the
      // compiler wait for each load at the join)
      const int tr = tid >> 4, q16 = tid & 15;
      v4i raw[NTT][4];
#pragma unroll
      for (int j = 0; j < NTT; ++j) {
        const int ti = g0 + tr + 16 * j;
        const int voff = ti < cnt ? slots[ti] * (I * 2) + q16 * 64 : hbytes;
#pragma unroll
        for (int v = 0; v < 4; ++v) raw[j][v] = __builtin_amdgcn_raw_buffer_load_b128(hrs, voff + 16 * v, 0, 0);
      }
      const bool wok = tid < 16 * NTT && g0 + tid < cnt;
      float wv = wok ? 1.f : 0.f;
      if (!shared)
        wv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(trs, wok ? slots[g0 + tid] * 4 : tbytes, 0, 0));
      if constexpr (FIRST) {
        issue_weights(std::integral_constant<int, 0>{}, std::integral_constant<int, kDnEarly>{}, std::integral_constant<int, NSTG>{});
        issue_weights(std::integral_constant<int, 2>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, NSTG>{});
        if constexpr (DT != Q36_MOE_FP8) sn[tid] = snv;
      }
#pragma unroll
      for (int j = 0; j < NTT; ++j) {
        const int row = tr + 16 * j;
        auto hval = [&](int i) {  // value i (0..31) of the thread's 32 in row j
          const uint32_t w = (uint32_t)raw[j][i >> 3][(i >> 1) & 3];
          return (i & 1) ? bf_hi(w) : bf_lo(w);
        };
        float m = 0.f;
#pragma unroll
        for (int v = 0; v < 32; ++v) m = fmaxf(m, fabsf(hval(v)));
        uint32_t wd[8];
        if constexpr (DT == Q36_MOE_FP8) {
          m = fmaxf(m, lane_xor<1>(m));
          m = fmaxf(m, lane_xor<2>(m));
          const float inv = m > 0.f ? 448.f / m : 0.f;
#pragma unroll
          for (int v = 0; v < 8; ++v)
            wd[v] = f2e4m3x2_hw(hval(4 * v) * inv, hval(4 * v + 1) * inv) |
                    (f2e4m3x2_hw(hval(4 * v + 2) * inv, hval(4 * v + 3) * inv) << 16);
          if ((q16 & 3) == 0) hs[row][q16 >> 2] = m / 448.f;
        } else {
          m = fmaxf(m, lane_xor<1>(m));
          m = fmaxf(m, lane_xor<2>(m));
          m = fmaxf(m, lane_xor<4>(m));
          m = fmaxf(m, lane_xor<8>(m));
          const float sc = m / 127.f, safe = m > 0.f ? sc : 1.f;
#pragma unroll
          for (int v = 0; v < 8; ++v) {
            wd[v] = 0u;
#pragma unroll
            for (int q = 0; q < 4; ++q) wd[v] |= ((uint32_t)round_i8(hval(4 * v + q) / safe) & 0xffu) << (8 * q);
          }
          if (q16 == 0) hs[row][0] = sc;
        }
        uint4* dst = reinterpret_cast<uint4*>(&hq[row * kDnRow + q16 * 32]);
        dst[0] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        dst[1] = make_uint4(wd[4], wd[5], wd[6], wd[7]);
      }
      if (tid < 16 * NTT) wl[tid] = wv;
    }
    __syncthreads();
#pragma unroll
    for (int cp = 0; cp < kDnCT; cp += 2) {
      using Acc = typename std::conditional<DT == Q36_MOE_FP8, v4f, v4i>::type;
      Acc acc[2][NTT];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) acc[c][tt] = Acc{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < NSTG; ++s) {
        v4i a[NTT][2];
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
          const uint8_t* ap = &hq[(tt * 16 + lr) * kDnRow + s * 128 + lgp * 32];
          a[tt][0] = *reinterpret_cast<const v4i*>(ap);
          a[tt][1] = *reinterpret_cast<const v4i*>(ap + 16);
        }
        if constexpr (DT == Q36_MOE_FP8) {
#pragma unroll
          for (int tt = 0; tt < NTT; ++tt) {
            const float xw = hs[tt * 16 + lr][s] * wsc[s];  // this lane's token
            const v8i a8 = cat8(a[tt][0], a[tt][1]);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              const v4f rr = mfma_fp8(cat8(B[cp + c][s][0], B[cp + c][s][1]), a8);
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[c][tt][r] = __builtin_fmaf(rr[r], xw, acc[c][tt][r]);
            }
          }
          // the running sums are formed per stage (left alone, the compiler sinks the chain and
          // keeps every stage's MFMA results live)
#pragma unroll
          for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
              for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(acc[c][tt][r]));
        } else {
#pragma unroll
          for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              acc[c][tt] = mfma_i8(B[cp + c][s][0], a[tt][0], acc[c][tt]);
              acc[c][tt] = mfma_i8(B[cp + c][s][1], a[tt][1], acc[c][tt]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // lane: token tt*16 + l%16, output columns n .. n+3
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) {
        const int row = tt * 16 + lr, ti = g0 + row;
        if (ti < cnt) {
          const int sl = slots[ti];
          const float wt = wl[row];
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int nl = wave * kDnRows + (cp + c) * 16 + 4 * lgp;  // column within the workgroup
            const int n = grp * 4 * kDnRows + nl;
            float yv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if constexpr (DT == Q36_MOE_FP8) {
                yv[r] = acc[c][tt][r];
              } else {
                if (d.dbg_acc2) d.dbg_acc2[(size_t)sl * H + n + r] = acc[c][tt][r];
                yv[r] = ((float)acc[c][tt][r] * hs[row][0]) * sn[nl + r];
              }
            }
            *reinterpret_cast<uint2*>(&d.y[(size_t)sl * H + n]) =
                make_uint2(pack_bf2(yv[0] * wt, yv[1] * wt), pack_bf2(yv[2] * wt, yv[3] * wt));
          }
        }
      }
    }
  };
  static_assert(kDnTG == 64, "a work item is one token block of at most 64 tokens");
  const int nb = min(cnt - g0, kTokBlock);
  if (nb <= 16)
    group(g0, std::integral_constant<int, 1>{}, std::true_type{});
  else if (nb <= 32)
    group(g0, std::integral_constant<int, 2>{}, std::true_type{});
  else
    group(g0, std::integral_constant<int, 4>{}, std::true_type{});
}

// ------------------------------------------------------------------------------------------
// 5. combine
// ------------------------------------------------------------------------------------------
// One workgroup per token; every y row of the token (its k routed slots t*k + j and the shared
// slot M*k + t) is loaded before any is added, then
// out = bf16(fma(gate, y_shared, ((0 + y_0) + y_1) ... + y_{k-1})).
// With the fused add-norm (L/qk_route.cu:630-820 combine_norm): z = out + resid in fp32,
// resid <- bf16(z), and the Gemma RMSNorm of z; the sum of squares runs in q36_add_rmsnorm's order
// (lane l owns the 8-element chunks l + 64 j, fma from zero in j order, then an xor butterfly): the
// workgroup's chunk c sits with thread c, so the z values meet in LDS and wave 0 adds them up.
constexpr int kCombH = 2048;
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeDev d) {
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (t >= d.M) {
    // the fused add-norm's e4m3 rows in fragment order: the padding tokens up to a multiple of 16
    *reinterpret_cast<uint2*>(d.norm_q8 + frag_offset(t, 8 * tid, kCombH)) = make_uint2(0u, 0u);
    if ((tid & 15) == 0) d.norm_q8s[(size_t)t * (kCombH / 128) + tid / 16] = 0.f;
    return;
  }
  const bool valid = d.pos == nullptr || d.pos[t] != 0;
  const int S = d.M * d.k;
  __shared__ float rstd_s;
  __shared__ float zs[kCombH / 8][8];
  const int c = tid;  // the thread's 8-element chunk (H = 2048: one per thread)
  const size_t at = (size_t)t * kCombH + 8 * c;
  // the fused add-norm's residual chunk and norm weights are requested with the y rows (one round
  // trip for every operand; out and resid do not overlap, checked on the host)
  v4i rv = {0, 0, 0, 0}, wv = {0, 0, 0, 0};
  if (d.norm_out != nullptr) {
    rv = *reinterpret_cast<const v4i*>(d.resid + at);
    wv = *reinterpret_cast<const v4i*>(d.norm_w + 8 * c);
  }
  uint4 o = make_uint4(0u, 0u, 0u, 0u);
  if (valid) {
    // every y row of the token and its gate in one round trip (rows past k repeat the shared row)
    const float gate = d.gate[t];
    v4i yv[17];
#pragma unroll
    for (int j = 0; j < 17; ++j) {
      const int row = j < d.k ? t * d.k + j : S + t;
      yv[j] = ldg16(reinterpret_cast<const uint8_t*>(d.y + (size_t)row * kCombH + 8 * c));
    }
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (j < d.k) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = acc[2 * q] + bf_lo((uint32_t)yv[j][q]);
          acc[2 * q + 1] = acc[2 * q + 1] + bf_hi((uint32_t)yv[j][q]);
        }
      }
    }
    v4i sv = yv[0];
#pragma unroll
    for (int j = 1; j < 17; ++j)
      if (j == d.k) sv = yv[j];
    const float g = gate;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[q] = pack_bf2(__builtin_fmaf(g, bf_lo((uint32_t)sv[q]), acc[2 * q]),
                      __builtin_fmaf(g, bf_hi((uint32_t)sv[q]), acc[2 * q + 1]));
    o = make_uint4(w[0], w[1], w[2], w[3]);
  }
  *reinterpret_cast<uint4*>(d.out + at) = o;
  if (d.norm_out == nullptr) return;
  // the fused add-norm
  const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
  float z[8];
  v4i nv;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    z[2 * q] = bf_lo(ow[q]) + bf_lo((uint32_t)rv[q]);
    z[2 * q + 1] = bf_hi(ow[q]) + bf_hi((uint32_t)rv[q]);
    nv[q] = (int)pack_bf2(z[2 * q], z[2 * q + 1]);
  }
  *reinterpret_cast<v4i*>(d.resid + at) = nv;
#pragma unroll
  for (int i = 0; i < 8; ++i) zs[c][i] = z[i];
  __syncthreads();
  if (wave == 0) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kCombH / 512; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float zv = zs[lane + 64 * j][i];
        ss = __builtin_fmaf(zv, zv, ss);
      }
    ss = wave_sum_bfly(ss);
    if (lane == 0) rstd_s = 1.f / sqrtf(ss / (float)kCombH + d.norm_eps);
  }
  __syncthreads();
  const float rstd = rstd_s;
  v4i ov;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    ov[q] = (int)pack_bf2((z[2 * q] * rstd) * (1.f + bf_lo((uint32_t)wv[q])),
                          (z[2 * q + 1] * rstd) * (1.f + bf_hi((uint32_t)wv[q])));
  *reinterpret_cast<v4i*>(d.norm_out + at) = ov;
  if (d.norm_q8 == nullptr) return;
  // the normed row's e4m3 codes for the next projection (a 128-group is 16 neighbouring threads)
  float f[8];
  float m = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = bf_lo((uint32_t)ov[q]);
    f[2 * q + 1] = bf_hi((uint32_t)ov[q]);
    m = fmaxf(m, fmaxf(fabsf(f[2 * q]), fabsf(f[2 * q + 1])));
  }
  m = __uint_as_float(row16_max_u32(__float_as_uint(m)));  // non-negative: integer order; the 16 lanes of a group
  const float inv = m > 0.f ? 448.f / m : 0.f;
  *reinterpret_cast<uint2*>(d.norm_q8 + (d.norm_q8_frag ? frag_offset(t, 8 * c, kCombH) : at)) = e4m3_run8(f, inv);
  if ((c & 15) == 0) d.norm_q8s[(size_t)t * (kCombH / 128) + c / 16] = m / 448.f;
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
  L->ctl = take(sizeof(int32_t) * 64);
  L->logits = take(sizeof(float) * (size_t)M * E);
  L->gate = take(sizeof(float) * (size_t)M);
  L->ids = take(sizeof(int32_t) * S);
  L->wts = take(sizeof(float) * S);
  L->counts = take(sizeof(int32_t) * E);
  L->offsets = take(sizeof(int32_t) * (E + 1));
  L->perm = take(sizeof(int32_t) * S);
  L->inv_perm = take(sizeof(int32_t) * S);
  L->active = take(sizeof(int32_t) * E);
  L->ecount = take(sizeof(int32_t) * E);
  L->eact = take(sizeof(int32_t) * 2 * (size_t)E);
  L->elist = take(sizeof(int32_t) * (size_t)E * M);
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
  Q36_REQUIRE((a->x || a->in_norm_w) && a->router_w && a->workspace,
              "q36_moe: x (or the input add-norm), router_w and workspace are required");
  Q36_REQUIRE(!a->in_norm_w || (a->in_delta && a->in_resid && a->in_resid_out),
              "q36_moe: the input add-norm (in_norm_w) needs in_delta, in_resid and in_resid_out");
  Q36_REQUIRE(!need_experts || (a->w13 && a->s13 && a->w2 && a->s2 && a->sw13 && a->ss13 && a->sw2 && a->ss2 &&
                                a->gate_w && a->out),
              "q36_moe_forward: an expert weight, scale, gate_w or out pointer is null");
  const void* ptrs[] = {a->x, a->router_w, a->w13, a->w2, a->sw13, a->sw2, a->gate_w, a->out, a->workspace,
                        a->dbg_acc13, a->dbg_acc2, a->dbg_h, a->resid, a->norm_w, a->norm_out,
                        a->in_delta, a->in_resid, a->in_resid_out, a->in_norm_w};
  for (const void* p : ptrs) Q36_REQUIRE(aligned16(p), "q36_moe: pointer %p is not 16-byte aligned", p);
  if (a->in_norm_w) {
    // the route reads in_delta and in_resid while its row workgroups write in_resid_out and x
    const uintptr_t nb = (uintptr_t)a->M * (uintptr_t)a->H * 2u;
    auto apart = [&](const void* p, const void* q) {
      const uintptr_t u = reinterpret_cast<uintptr_t>(p), v = reinterpret_cast<uintptr_t>(q);
      return p == nullptr || q == nullptr || u + nb <= v || v + nb <= u;
    };
    Q36_REQUIRE(apart(a->in_resid_out, a->in_delta) && apart(a->in_resid_out, a->in_resid) &&
                    apart(a->x, a->in_delta) && apart(a->x, a->in_resid) && apart(a->x, a->in_resid_out),
                "q36_moe: in_resid_out and x must overlap neither in_delta, in_resid nor each other");
  }
  Q36_REQUIRE((reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0, "q36_moe: workspace must be 256-byte aligned");
  Q36_REQUIRE(a->norm_out == nullptr || (a->resid && a->norm_w),
              "q36_moe: the fused add-norm (norm_out) needs resid and norm_w");
  {
    const uintptr_t o0 = reinterpret_cast<uintptr_t>(a->out), r0 = reinterpret_cast<uintptr_t>(a->resid);
    const uintptr_t nb = (uintptr_t)a->M * (uintptr_t)a->H * 2u;
    Q36_REQUIRE(a->norm_out == nullptr || a->out == nullptr || o0 + nb <= r0 || r0 + nb <= o0,
                "q36_moe: out and resid must not overlap");
  }
  Q36_REQUIRE((a->norm_q8 == nullptr) == (a->norm_q8s == nullptr) && (a->norm_q8 == nullptr || a->norm_out),
              "q36_moe: norm_q8 and norm_q8s go together, with norm_out");
  Q36_REQUIRE(!a->norm_q8 || ((reinterpret_cast<uintptr_t>(a->norm_q8) & 7u) == 0 &&
                              (reinterpret_cast<uintptr_t>(a->norm_q8s) & 3u) == 0),
              "q36_moe: norm_q8 must be 8-byte and norm_q8s 4-byte aligned");
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
              reinterpret_cast<float*>(ws + L.logits), reinterpret_cast<float*>(ws + L.gate),
              reinterpret_cast<int32_t*>(ws + L.ids),
              reinterpret_cast<float*>(ws + L.wts), reinterpret_cast<int32_t*>(ws + L.counts),
              reinterpret_cast<int32_t*>(ws + L.offsets), reinterpret_cast<int32_t*>(ws + L.perm),
              reinterpret_cast<int32_t*>(ws + L.inv_perm), reinterpret_cast<int32_t*>(ws + L.active),
              reinterpret_cast<int32_t*>(ws + L.ctl), reinterpret_cast<int32_t*>(ws + L.ecount),
              reinterpret_cast<int32_t*>(ws + L.eact), reinterpret_cast<int32_t*>(ws + L.elist),
              (a->M + kTokBlock - 1) / kTokBlock - 1,
              reinterpret_cast<uint8_t*>(ws + L.xq),
              reinterpret_cast<float*>(ws + L.xs), reinterpret_cast<uint16_t*>(ws + L.h),
              reinterpret_cast<uint16_t*>(ws + L.y), a->dbg_acc13, a->dbg_acc2,
              static_cast<uint16_t*>(a->dbg_h), static_cast<uint16_t*>(a->resid),
              static_cast<const uint16_t*>(a->norm_w), a->norm_eps, static_cast<uint16_t*>(a->norm_out),
              static_cast<uint8_t*>(a->norm_q8), a->norm_q8s, a->norm_q8_frag != 0};
  if (a->in_norm_w) {
    d->x = nullptr;  // formed by the route kernel
    d->in_delta = static_cast<const uint16_t*>(a->in_delta);
    d->in_resid = static_cast<const uint16_t*>(a->in_resid);
    d->in_resid_out = static_cast<uint16_t*>(a->in_resid_out);
    d->in_norm_w = static_cast<const uint16_t*>(a->in_norm_w);
    d->in_eps = a->in_norm_eps;
    d->xn = static_cast<uint16_t*>(const_cast<void*>(a->x));
  }
  return Q36_OK;
}

// Raise a kernel's dynamic-LDS limit (once per device and kernel) when a launch needs more than
// the 64 KiB default; gfx950 has 160 KiB per CU.
int launch_route(const MoeDev& d, int dtype, hipStream_t st) {
  const int tt = route_tt(d.M), epw = route_epw(d.M), n_router = (d.E / (4 * epw)) * ((d.M + tt - 1) / tt);
  auto go = [&](auto dt, auto tt_c, auto epw_c) {
    constexpr int DT = decltype(dt)::value, TT = decltype(tt_c)::value, EPW = decltype(epw_c)::value;
    route_logits_kernel<DT, TT, EPW><<<n_router + d.M, 256, 0, st>>>(d, n_router);
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  auto go_tt = [&](auto dt) {
    if (tt == 1) go(dt, I1{}, I2{});
    else if (tt == 2) go(dt, I2{}, I2{});
    else if (tt == 4) go(dt, I4{}, I2{});
    else if (epw == 2) go(dt, I8{}, I2{});
    else if (epw == 4) go(dt, I8{}, I4{});
    else go(dt, I8{}, std::integral_constant<int, 8>{});
  };
  if (dtype == Q36_MOE_FP8) go_tt(std::integral_constant<int, Q36_MOE_FP8>{});
  else go_tt(std::integral_constant<int, Q36_MOE_INT8>{});
  if (d.E == 512 && d.k == 10)
    route_topk_kernel<8, true, 10><<<d.M, 64, 0, st>>>(d);
  else if (d.E == 512)
    route_topk_kernel<8, true, 0><<<d.M, 64, 0, st>>>(d);
  else if (d.E < 512)
    route_topk_kernel<8, false, 0><<<d.M, 64, 0, st>>>(d);
  else if (d.E == 1024)
    route_topk_kernel<16, true, 0><<<d.M, 64, 0, st>>>(d);
  else
    route_topk_kernel<16, false, 0><<<d.M, 64, 0, st>>>(d);
  return check_launch("q36_moe_route");
}
int launch_lists(const MoeDev& d, hipStream_t st) {
  const size_t lds = lists_lds_bytes(d.E, d.M, d.k);
  int rc = ensure_lds(reinterpret_cast<const void*>(&route_lists_kernel), lds, "q36_moe_route");
  if (rc) return rc;
  route_lists_kernel<<<1, 256, lds, st>>>(d);
  return check_launch("q36_moe_route");
}

// Expert-kernel grid: 8 workgroups per work item: the shared expert's 1 + nsh blocks, and room for
// every routed block (one per active expert, at most min(E, M k) of them, and the further ones: an
// expert past 64 tokens only when M > 64, at most M k / 64 of them, fewer than E, so the list holds
// 2E).  A decode batch of a few rows launches only as many workgroups as its picks can keep busy.
int expert_grid(const MoeDev& d) {
  const int nrb = d.M > kTokBlock ? d.M * d.k / kTokBlock : 0;
  const int picks = d.M * d.k < d.E ? d.M * d.k : d.E;
  return 8 * (picks + 1 + d.nsh + nrb);
}
template <int DT>
int launch_up_t(const MoeDev& d, hipStream_t st) {
  moe_up_kernel<DT><<<expert_grid(d), 256, 0, st>>>(d);
  return check_launch("q36_moe_up");
}
template <int DT>
int launch_down_t(const MoeDev& d, hipStream_t st) {
  moe_down_kernel<DT><<<expert_grid(d), 256, 0, st>>>(d);
  return check_launch("q36_moe_down");
}
int launch_up(const MoeDev& d, int dtype, hipStream_t st) {
  return dtype == Q36_MOE_FP8 ? launch_up_t<Q36_MOE_FP8>(d, st) : launch_up_t<Q36_MOE_INT8>(d, st);
}
int launch_down(const MoeDev& d, int dtype, hipStream_t st) {
  return dtype == Q36_MOE_FP8 ? launch_down_t<Q36_MOE_FP8>(d, st) : launch_down_t<Q36_MOE_INT8>(d, st);
}
int launch_combine(const MoeDev& d, hipStream_t st) {
  // fragment-order e4m3 rows pad the tokens to a multiple of 16 (zero rows)
  const int grid = d.norm_q8 && d.norm_q8_frag ? (d.M + 15) / 16 * 16 : d.M;
  moe_combine_kernel<<<grid, 256, 0, st>>>(d);
  return check_launch("q36_moe_combine");
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
  rc = launch_route(d, a->dtype, static_cast<hipStream_t>(stream));
  return rc ? rc : launch_lists(d, static_cast<hipStream_t>(stream));
}


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

// ------------------------------------------------------------------------------------------
// The no-allocation MoE entry: the workspace is a file-scope device array of fixed size instead of
// a caller buffer.  Its host-side name is not a device address: the address is looked up once per
// device (hipGetSymbolAddress, with that device current) and only that address is used.
// ------------------------------------------------------------------------------------------
namespace q36 {
namespace {
constexpr size_t kMoeStaticBytes = (size_t)Q36_MOE_STATIC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kMoeStaticBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The calling thread's current device's copy of `scratch` (looked up on the first call per device).
int static_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("q36_moe_forward_static: no current HIP device (or device id %d >= %d)", dev, kMaxDevices);
    return Q36_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("q36_moe_forward_static: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return Q36_ELAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return Q36_OK;
}
}  // namespace
}  // namespace q36

extern "C" int q36_moe_forward_static(const q36_moe_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_moe_forward_static: null args");
  Q36_REQUIRE(a->workspace == nullptr && a->workspace_bytes == 0,
              "q36_moe_forward_static: the workspace is the library's own; pass workspace = NULL, workspace_bytes = 0");
  q36_moe_ws_layout L;
  const bool shape_ok = a->M >= 1 && a->M <= kMaxM && a->E >= 1 && a->E <= kMaxE && a->topk >= 1 && a->topk <= 16;
  if (shape_ok) layout(a->M, a->E, a->H, a->I, a->topk, a->dtype, &L);
  Q36_REQUIRE(!shape_ok || L.total <= kMoeStaticBytes,
              "q36_moe_forward_static: M=%d E=%d topk=%d needs %zu bytes of scratch, more than the library's %zu "
              "(M <= 256 with E <= 512 and topk <= 10 fit)", a->M, a->E, a->topk, L.total, kMoeStaticBytes);
  void* ws = nullptr;
  int rc = static_scratch(&ws);
  if (rc) return rc;
  q36_moe_args b = *a;
  b.workspace = ws;
  b.workspace_bytes = kMoeStaticBytes;
  return q36_moe_forward(&b, stream);
}
