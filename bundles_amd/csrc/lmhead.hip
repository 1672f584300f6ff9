// Int8 lm_head fused with greedy argmax for gfx950.
//
// Reference behaviour (R = qwen36_nodes_kb34, H = R/qwen36_lmhead8): per-row int8 activations
// (H/w8a8.py:16-23), per-channel int8 weights with fp32 scales (H/lmhead8.py:95-143), int32
// accumulation, logit = (acc * xs) * ws (H/w8a8.py:66-71) rounded to bf16 (the node's output
// dtype); the greedy token is the first index of the largest bf16 logit (torch.argmax order; the
// reference leaves the argmax to the stock sampler, H/node.py:136-151).  A final Gemma RMSNorm
// y = bf16((x * rstd) * (1 + w)) precedes the quantization (L/proj.py:60-81 restates the form).
//
// Kernels:
//   lmh_prep   one wave per row: norm (sum of squares in the fixed 64-lane order), int8 quant,
//              and the row's argmax key reset to 0.
//   lmh_gemm   256 x 256 output tile per workgroup (4 waves, 128 x 128 each, 32x32x32 int8 MFMAs
//              with the weights as operand A, int32 accumulators in AGPRs), K in 64-byte steps
//              through a 4-stage LDS ring filled by buffer loads straight into LDS, three steps
//              ahead (no register staging).  Epilogue: bf16 logits, per-row max of the 64-bit key
//              (order-preserving bf16 bits << 32 | ~index) over the tile, one 64-bit atomic max per
//              row and tile: the result does not depend on the order the workgroups finish in.
//   lmh_ids    key -> token id.
// Block -> tile mapping: block b runs on XCD b % 8; the eight row tiles of one vocab tile are
// consecutive blocks of the same XCD, so the weight tile is fetched from HBM once and served to
// the eight from that XCD's L2.
#include <type_traits>

#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int kLH = 2048;       // hidden (K)
constexpr int kBM = 256, kBN = 256, kBK = 64;

struct LmhDev {
  int R, V;
  const uint16_t* h;
  const uint16_t* norm_w;
  float eps;
  const int8_t* wq;
  const float* ws;
  int32_t* ids;
  uint16_t* logits;
  int8_t* xq;
  float* xs;
  unsigned long long* keys;
};

__global__ __launch_bounds__(256) void lmh_prep_kernel(LmhDev d) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + wave;
  if (r >= d.R) return;
  constexpr int NJ = kLH / 512;
  float y[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const v4i v = *reinterpret_cast<const v4i*>(d.h + (size_t)r * kLH + 8 * (lane + 64 * j));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      y[j][2 * q] = bf_lo((uint32_t)v[q]);
      y[j][2 * q + 1] = bf_hi((uint32_t)v[q]);
    }
  }
  if (d.norm_w) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(y[j][i], y[j][i], acc);
    const float ss = wave_sum_bfly(acc);
    const float rstd = 1.f / sqrtf(ss / (float)kLH + d.eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const v4i wv = *reinterpret_cast<const v4i*>(d.norm_w + 8 * (lane + 64 * j));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        y[j][2 * q] = rbf((y[j][2 * q] * rstd) * (1.f + bf_lo((uint32_t)wv[q])));
        y[j][2 * q + 1] = rbf((y[j][2 * q + 1] * rstd) * (1.f + bf_hi((uint32_t)wv[q])));
      }
    }
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(y[j][i]));
  m = wave_max(m);
  const float sc = m / 127.f, safe = m > 0.f ? sc : 1.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    uint32_t wd[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) wd[i >> 2] |= ((uint32_t)round_i8(y[j][i] / safe) & 0xffu) << (8 * (i & 3));
    *reinterpret_cast<uint2*>(d.xq + (size_t)r * kLH + 8 * (lane + 64 * j)) = make_uint2(wd[0], wd[1]);
  }
  if (lane == 0) {
    d.xs[r] = sc;
    d.keys[r] = 0ull;
  }
}

// LDS position of 16-byte chunk kc (0..3) of tile row c in one K step: rows are 64 bytes, unpadded,
// with the chunk order xor-swizzled by (c >> 1) & 3, so that the eight lanes of a fragment read
// (chunk kc of eight consecutive rows) touch eight distinct 16-byte bank windows.
__device__ __forceinline__ int bswz(int c, int kc) { return c * kBK + ((kc ^ ((c >> 1) & 3)) << 4); }

template <int N>
using ic = std::integral_constant<int, N>;

// x rounded to bf16 (round to nearest even), returned as the float it represents: one
// v_cvt_pk_bf16_f32 with a zero low half.
__device__ __forceinline__ float round_bf16(float x) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(float, __builtin_convertvector((v2f){0.f, x}, v2bf));
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void lmh_gemm_kernel(LmhDev d) {
  // Four LDS stages per operand, one object each: the compiler tracks the buffer-to-LDS loads of
  // each object separately and waits only for those of the stage being read.
  __shared__ __align__(1024) int8_t a_s0[kBM * kBK], a_s1[kBM * kBK], a_s2[kBM * kBK], a_s3[kBM * kBK];
  __shared__ __align__(1024) int8_t b_s0[kBN * kBK], b_s1[kBN * kBK], b_s2[kBN * kBK], b_s3[kBN * kBK];
  __shared__ uint32_t rkey[2][kBM];
  __shared__ __align__(16) float ws_l[kBN];  // the tile's weight scales
  auto a_st = [&](auto st) -> int8_t* {
    if constexpr (decltype(st)::value == 0) return a_s0;
    else if constexpr (decltype(st)::value == 1) return a_s1;
    else if constexpr (decltype(st)::value == 2) return a_s2;
    else return a_s3;
  };
  auto b_st = [&](auto st) -> int8_t* {
    if constexpr (decltype(st)::value == 0) return b_s0;
    else if constexpr (decltype(st)::value == 1) return b_s1;
    else if constexpr (decltype(st)::value == 2) return b_s2;
    else return b_s3;
  };
  const int nvt = (d.V + kBN - 1) / kBN, nrt = (d.R + kBM - 1) / kBM;
  // XCD-aware mapping (block b -> XCD b % 8): consecutive blocks of an XCD sweep the row tiles of
  // one vocab tile, which is then fetched from HBM once per XCD and served from its L2
  const int b = blockIdx.x, xcd = b & 7, j = b >> 3;
  const int rt = j % nrt, vt = (j / nrt) * 8 + xcd;
  if (vt >= nvt) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;  // 2 x 2 waves of 128 x 128
  const int r0 = rt * kBM, v0 = vt * kBN;
  // global -> LDS by buffer loads with the LDS bit (no registers; rows past R or V read as zero).
  // Load i of wave w fills 1 KB chunk q = 4 w + i of a stage (tile rows 16 q .. 16 q + 15); lane l
  // writes bytes 16 l .. 16 l + 15 of the chunk, which bswz assigns to row 16 q + l / 4, logical
  // 16-byte chunk (l % 4) ^ ((l / 8) % 4).
  const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(d.xq + (size_t)r0 * kLH), (short)0, min(d.R - r0, kBM) * kLH, 0x00020000);
  const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(d.wq + (size_t)v0 * kLH), (short)0, min(d.V - v0, kBN) * kLH, 0x00020000);
  if (tid < kBN / 4)
    *reinterpret_cast<float4*>(&ws_l[4 * tid]) =
        v0 + 4 * tid < d.V ? *reinterpret_cast<const float4*>(d.ws + v0 + 4 * tid) : make_float4(0.f, 0.f, 0.f, 0.f);
  const int voff = (lane >> 2) * kLH + (((lane & 3) ^ ((lane >> 3) & 3)) << 4);
  const int wq4 = __builtin_amdgcn_readfirstlane(wave) * 4;
  auto issue_to = [&](int ks, int8_t* as, int8_t* bs) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = wq4 + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, as + q * 1024, 16, voff, q * 16 * kLH + ks * kBK, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(brsrc, bs + q * 1024, 16, voff, q * 16 * kLH + ks * kBK, 0, 2);
    }
  };
  auto issue = [&](int ks, auto st) { issue_to(ks, a_st(st), b_st(st)); };
  constexpr int NK = kLH / kBK;
  static_assert(NK % 4 == 0 && NK >= 8, "K steps");
  // 32x32x32 int8 MFMA (twice the rate of 16x16x64 on gfx950): the weight rows are operand A, the
  // token rows operand B.  Lane l reads tile row 32 t + l % 32, K bytes 16 (l / 32) of each 32-byte
  // half step (LDS chunk 2 h + l / 32); the result gives lane l token l % 32 and vocab rows
  // 8 (j / 4) + 4 (l / 32) + j % 4 of register j.
  const int l32 = lane & 31, lh = lane >> 5;
  const int fx0 = bswz(wm * 128 + l32, lh), fx1 = bswz(wm * 128 + l32, 2 + lh);  // + 32 kBK per tile
  const int fw0 = bswz(wn * 128 + l32, lh), fw1 = bswz(wn * 128 + l32, 2 + lh);
  v16i acc[4][4];  // [vocab tile][token tile]
  // One K step.  The wait leaves the 16 loads of steps ks + 1 and ks + 2 in flight, so this wave's
  // loads of step ks are in LDS and its LDS reads of step ks - 1 are done; after the barrier both
  // hold for all four waves.  Step ks + 3 then refills the stage step ks - 1 used (past the end the
  // loads repeat step NK - 1 into stages nobody reads again, keeping the count in flight uniform).
  // The first step starts the accumulators from zero inside the MFMA (a zero-initialised
  // accumulator array carried into the loop makes the register allocator shuffle it every step).
  auto body = [&](int ks, auto cur, auto nxt, auto first) {
    asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(min(ks + 3, NK - 1), nxt);
    const int8_t* as = a_st(cur);
    const int8_t* bs = b_st(cur);
    v4i xf[2][4], wf[2][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      xf[0][t] = *reinterpret_cast<const v4i*>(as + fx0 + t * 32 * kBK);
      xf[1][t] = *reinterpret_cast<const v4i*>(as + fx1 + t * 32 * kBK);
      wf[0][t] = *reinterpret_cast<const v4i*>(bs + fw0 + t * 32 * kBK);
      wf[1][t] = *reinterpret_cast<const v4i*>(bs + fw1 + t * 32 * kBK);
    }
    // all 16 fragment reads go out before the first MFMA (left alone, the scheduler reuses one
    // fragment register and waits out a full LDS latency per row of MFMAs)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int vi = 0; vi < 4; ++vi)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
          acc[vi][ti] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
              wf[h][vi], xf[h][ti], (decltype(first)::value && h == 0) ? v16i{} : acc[vi][ti], 0, 0, 0);
  };
  issue(0, ic<0>{});
  issue(1, ic<1>{});
  issue(2, ic<2>{});
  body(0, ic<0>{}, ic<3>{}, std::true_type{});
  body(1, ic<1>{}, ic<0>{}, std::false_type{});
  body(2, ic<2>{}, ic<1>{}, std::false_type{});
  body(3, ic<3>{}, ic<2>{}, std::false_type{});
  for (int ks = 4; ks < NK; ks += 4) {
    body(ks, ic<0>{}, ic<3>{}, std::false_type{});
    body(ks + 1, ic<1>{}, ic<0>{}, std::false_type{});
    body(ks + 2, ic<2>{}, ic<1>{}, std::false_type{});
    body(ks + 3, ic<3>{}, ic<2>{}, std::false_type{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // Epilogue: lane l holds tokens r0 + wm*128 + 32 ti + l % 32 and, per token, vocab columns
  // cb + 32 vi + 8 (j / 4) + 4 (l / 32) + j % 4.  Each logit is rounded to bf16 once (hardware
  // round-to-nearest-even) and folded into a 32-bit key (order-preserving bf16 bits << 16 |
  // 0xffff - column in the tile; -0 and +0 share a key, as in the bf16 argmax): the lane's max key
  // over its 64 columns, one exchange with lane l ^ 32, the two column waves through LDS, and the
  // tile through one 64-bit atomic max per row.  Columns past V are skipped.
  auto epilogue = [&](auto store, auto partial) {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int rl = wm * 128 + ti * 32 + l32;
      const int row = r0 + rl;
      const float xsr = row < d.R ? d.xs[row] : 0.f;
      uint32_t best = 0u;
#pragma unroll
      for (int vi = 0; vi < 4; ++vi)
#pragma unroll
        for (int jg = 0; jg < 4; ++jg) {
          const int cl = wn * 128 + vi * 32 + 8 * jg + 4 * lh;  // first of the 4 columns, in the tile
          const float4 w4 = *reinterpret_cast<const float4*>(&ws_l[cl]);
          const float wq[4] = {w4.x, w4.y, w4.z, w4.w};
          float lg[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            lg[q] = round_bf16(((float)acc[vi][ti][4 * jg + q] * xsr) * wq[q]);
            uint32_t b16 = __float_as_uint(lg[q] + 0.f) >> 16;
            b16 = (b16 & 0x8000u) ? (~b16 & 0xffffu) : (b16 | 0x8000u);
            const uint32_t key = (b16 << 16) | (0xffffu - (uint32_t)(cl + q));
            if (!decltype(partial)::value || v0 + cl + q < d.V) best = max(best, key);
          }
          if constexpr (decltype(store)::value)
            if (row < d.R && v0 + cl < d.V)  // V % 16 == 0: the 4 columns are all in or all out
              *reinterpret_cast<uint2*>(d.logits + (size_t)row * d.V + v0 + cl) =
                  make_uint2((__float_as_uint(lg[0]) >> 16) | (__float_as_uint(lg[1]) & 0xffff0000u),
                             (__float_as_uint(lg[2]) >> 16) | (__float_as_uint(lg[3]) & 0xffff0000u));
        }
      best = max(best, (uint32_t)__shfl_xor((int)best, 32));
      if (lh == 0) rkey[wn][rl] = best;
    }
  };
  // the column checks only in the last vocab tile
  if (v0 + kBN <= d.V) {
    if (d.logits)
      epilogue(std::true_type{}, std::false_type{});
    else
      epilogue(std::false_type{}, std::false_type{});
  } else {
    if (d.logits)
      epilogue(std::true_type{}, std::true_type{});
    else
      epilogue(std::false_type{}, std::true_type{});
  }
  __syncthreads();
  if (r0 + tid < d.R) {
    const uint32_t k = max(rkey[0][tid], rkey[1][tid]);
    const uint32_t col = (uint32_t)v0 + (0xffffu - (k & 0xffffu));
    atomicMax(&d.keys[r0 + tid], ((unsigned long long)(k >> 16) << 32) | (unsigned long long)(0xffffffffu - col));
  }
}

__global__ __launch_bounds__(256) void lmh_ids_kernel(LmhDev d) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r < d.R) d.ids[r] = (int32_t)(0xffffffffu - (uint32_t)(d.keys[r] & 0xffffffffull));
}

struct LmhWs {
  size_t xq, xs, keys, total;
};
LmhWs lmh_ws(int R) {
  LmhWs w;
  size_t o = 0;
  auto take = [&](size_t b) {
    size_t r = o;
    o = align_up(o + b, 256);
    return r;
  };
  w.xq = take((size_t)R * kLH);
  w.xs = take(sizeof(float) * (size_t)R);
  w.keys = take(sizeof(unsigned long long) * (size_t)R);
  w.total = o;
  return w;
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" size_t q36_lmhead_workspace_bytes(int32_t R) { return lmh_ws(R).total; }

extern "C" int q36_lmhead_argmax(const q36_lmhead_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_lmhead_argmax: null args");
  Q36_REQUIRE(a->H == kLH, "q36_lmhead_argmax: H=%d unsupported (this build is specialised to 2048)", a->H);
  Q36_REQUIRE(a->R >= 1 && a->R <= (1 << 20), "q36_lmhead_argmax: R=%d out of range", a->R);
  Q36_REQUIRE(a->V >= 16 && a->V % 16 == 0, "q36_lmhead_argmax: V=%d must be a positive multiple of 16", a->V);
  Q36_REQUIRE(a->h && a->wq && a->ws && a->ids && a->workspace, "q36_lmhead_argmax: a required pointer is null");
  Q36_REQUIRE(aligned16(a->h) && aligned16(a->wq) && aligned16(a->ws) && aligned16(a->norm_w) &&
                  (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_lmhead_argmax: h, wq, ws, norm_w must be 16-byte and workspace 256-byte aligned");
  const LmhWs L = lmh_ws(a->R);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_lmhead_argmax: workspace of %zu bytes < %zu required",
              a->workspace_bytes, L.total);
  char* ws = static_cast<char*>(a->workspace);
  LmhDev d{a->R, a->V, static_cast<const uint16_t*>(a->h), static_cast<const uint16_t*>(a->norm_w), a->eps,
           static_cast<const int8_t*>(a->wq), a->ws, a->ids, static_cast<uint16_t*>(a->logits),
           reinterpret_cast<int8_t*>(ws + L.xq), reinterpret_cast<float*>(ws + L.xs),
           reinterpret_cast<unsigned long long*>(ws + L.keys)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  lmh_prep_kernel<<<(a->R + 3) / 4, 256, 0, st>>>(d);
  const int nvt = (a->V + kBN - 1) / kBN, nrt = (a->R + kBM - 1) / kBM;
  const int blocks = ((nvt + 7) / 8) * 8 * nrt;
  lmh_gemm_kernel<<<blocks, 256, 0, st>>>(d);
  lmh_ids_kernel<<<(a->R + 255) / 256, 256, 0, st>>>(d);
  return check_launch("q36_lmhead_argmax");
}
