// Fused gated full-attention projections for gfx950: e4m3 128x128 block-scaled QKV + output-gate
// projection, per-head Gemma RMSNorm on q and k, neox RoPE on the first 64 of 256 dims, the e4m3
// K/V cache write, and the o_proj of the sigmoid-gated attention output.
//
// Reference behaviour (R = qwen36_nodes_kb34, L = R/qwen36_layer):
//   qkv layout [T, 8192 q/gate | 512 k | 512 v], q/gate interleaved per head (L/attn_fused.py:209)
//   norm + RoPE + e4m3 (L/qk_attn_verify.cu:156-208 norm_rope_e4m3, :765-797 prefill front)
//   gate: o_proj input = bf16(attn * sigmoid(gate)) (L/qk_attn_verify.cu:730-737)
// The block-scaled e4m3 weights are the configuration's format (the reference projects in bf16
// or W8A16); their numerics follow the MoE experts: per-token x 128-channel activation scales,
// one e4m3 block sum per 128-channel block, terms added in block order.
//
// Kernels: act_quant (bf16 -> e4m3 + scales, optionally gated), fp8_gemm (skinny GEMM: each wave
// streams 16 weight rows over the whole K; the workgroup shares the activation tile in LDS, one
// 512-byte K chunk at a time), norm_rope (one workgroup per token).
#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

__device__ __forceinline__ v4i ldg16a(const uint8_t* p) { return *reinterpret_cast<const v4i*>(p); }
__device__ __forceinline__ v4i ldg16a_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}
__device__ __forceinline__ v8i cat8a(v4i a, v4i b) {
  v8i r = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return r;
}
__device__ __forceinline__ v4f mfma_e4m3(v8i a, v8i b) {
  v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}

// ------------------------------------------------------------------------------------------
// activation quantization: one workgroup per token; thread tid owns 8-element chunks tid + 256 r.
// gate != nullptr: the value quantized is bf16(x * sigmoid(gate)) (the o_proj input).
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* x, const uint16_t* gate, int K, uint8_t* q,
                                                        float* s) {
  const int t = blockIdx.x, tid = threadIdx.x;
  const int ng = K / 128;
  for (int c = tid; 8 * c < K; c += 256) {
    const v4i xv = ldg16a(reinterpret_cast<const uint8_t*>(x + (size_t)t * K + 8 * c));
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf_lo((uint32_t)xv[i]);
      f[2 * i + 1] = bf_hi((uint32_t)xv[i]);
    }
    if (gate) {
      const v4i gv = ldg16a(reinterpret_cast<const uint8_t*>(gate + (size_t)t * K + 8 * c));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = rbf(f[2 * i] * sigmoid_q(bf_lo((uint32_t)gv[i])));
        f[2 * i + 1] = rbf(f[2 * i + 1] * sigmoid_q(bf_hi((uint32_t)gv[i])));
      }
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(f[i]));
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));  // 16 threads = one 128-group
    const float inv = m > 0.f ? 448.f / m : 0.f;
    uint32_t wd[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; i += 2) wd[i >> 2] |= f2e4m3x2_hw(f[i] * inv, f[i + 1] * inv) << (8 * (i & 3));
    *reinterpret_cast<uint2*>(q + (size_t)t * K + 8 * c) = make_uint2(wd[0], wd[1]);
    if ((c & 15) == 0) s[(size_t)t * ng + c / 16] = m / 448.f;
  }
}

// ------------------------------------------------------------------------------------------
// skinny e4m3 GEMM: Y[t, n] = bf16(sum_kb (blocksum_kb(t, n) * xs[t, kb]) * ws[n/128, kb])
// Workgroup = (64 weight rows, 64 tokens); wave w owns rows n0 + 16 w .. + 15 over the whole K
// (stages of 128 bytes, kD in flight); the token tile (4 x 16 rows) lives in LDS one 512-byte K
// chunk at a time.  MFMA src0 = tokens (lane row l%16), src1 = weight rows; lane l of the 16x16
// result holds weight row l%16 and token rows 4 (l/16) + r.
// ------------------------------------------------------------------------------------------
constexpr int kGD = 4, kGKC = 512, kGRow = kGKC + 16, kGTB = 64;
struct GemmDev {
  const uint8_t* A;
  const float* As;
  int T, K;
  const uint8_t* W;
  const float* Ws;
  int N;
  uint16_t* Y;
};
__global__ __launch_bounds__(256) void fp8_gemm_kernel(GemmDev g) {
  __shared__ __align__(16) uint8_t a_l[kGTB][kGRow];
  __shared__ float as_l[kGTB][kGKC / 128];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lgp = lane >> 4;
  const int n0 = blockIdx.x * 64 + wave * 16;
  const int t0 = blockIdx.y * kGTB;
  const int nst = g.K / 128, nkb = g.K / 128;
  const uint8_t* wrow = g.W + (size_t)(n0 + lr) * g.K + lgp * 32;
  const float* wsr = g.Ws + (size_t)(n0 / 128) * nkb;
  v4i Bq[kGD][2];
#pragma unroll
  for (int s = 0; s < kGD; ++s) {
    Bq[s][0] = ldg16a_nt(wrow + s * 128);
    Bq[s][1] = ldg16a_nt(wrow + s * 128 + 16);
  }
  const int nt = min(4, (g.T - t0 + 15) / 16);
  float acc[4][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[tt][r] = 0.f;
  for (int kc = 0; kc < g.K; kc += kGKC) {
    __syncthreads();
    {
      // activation chunk: thread -> (row tid/4, 128 bytes at 128 (tid%4))
      const int rr = tid >> 2, seg = tid & 3;
      const bool ok = t0 + rr < g.T;
      const uint8_t* src = g.A + (size_t)(ok ? t0 + rr : 0) * g.K + kc + seg * 128;
      v4i v[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) v[c] = ok ? ldg16a(src + 16 * c) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 8; ++c) *reinterpret_cast<v4i*>(&a_l[rr][seg * 128 + 16 * c]) = v[c];
      as_l[rr][seg] = ok ? g.As[(size_t)(t0 + rr) * nkb + kc / 128 + seg] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int sc = 0; sc < kGKC / 128; ++sc) {
      const int s = kc / 128 + sc;
      const int q = s % kGD;
      const float ws = wsr[s];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        if (tt < nt) {
          const uint8_t* ap = &a_l[tt * 16 + lr][sc * 128 + lgp * 32];
          const v4f rr = mfma_e4m3(cat8a(*reinterpret_cast<const v4i*>(ap), *reinterpret_cast<const v4i*>(ap + 16)),
                                   cat8a(Bq[q][0], Bq[q][1]));
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float a = acc[tt][r] + (rr[r] * as_l[tt * 16 + 4 * lgp + r][sc]) * ws;
            asm volatile("" : "+v"(a));  // keep the block-order sum inside its stage
            acc[tt][r] = a;
          }
        }
      }
      if (s + kGD < nst) {
        Bq[q][0] = ldg16a_nt(wrow + (s + kGD) * 128);
        Bq[q][1] = ldg16a_nt(wrow + (s + kGD) * 128 + 16);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const int n = n0 + lr;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + tt * 16 + 4 * lgp + r;
      if (tt < nt && t < g.T) g.Y[(size_t)t * g.N + n] = (uint16_t)f2bf(acc[tt][r]);
    }
}

// ------------------------------------------------------------------------------------------
// per-token epilogue of the QKV projection: one workgroup per token, wave w handles heads
// w, w + 8 of the 20 (16 q/gate, 2 k, 2 v).  q and k: Gemma RMSNorm over 256 dims (sum of squares
// by an xor butterfly over the wave, rstd = 1/sqrt(ss/256 + eps)), x = bf16((x * rstd) * (1 + w)),
// then neox RoPE on dims 0..63 (pairs i, i + 32) with the fp32 cos|sin row of the position;
// k and v also go to the e4m3 cache (satfinite, no scale).
// ------------------------------------------------------------------------------------------
struct RopeDev {
  int T, max_pos;
  const uint16_t* qkv;  // bf16 [T, 9216]
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  float eps;
  const float* cos_sin;  // [max_pos, 64]
  const int32_t* positions;
  uint16_t* q;
  uint16_t* gate;
  uint16_t* k;
  uint16_t* v;
  uint8_t* k8;
  uint8_t* v8;
};
__global__ __launch_bounds__(512) void norm_rope_kernel(RopeDev d) {
  const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint16_t* row = d.qkv + (size_t)t * 9216;
  int pos = d.positions[t];
  pos = pos < 0 ? 0 : (pos >= d.max_pos ? d.max_pos - 1 : pos);
  const float* cs = d.cos_sin + (size_t)pos * 64;
  for (int h = wave; h < 20; h += 8) {
    // lane holds dims lane, lane + 64, lane + 128, lane + 192 of the head
    const uint16_t* src;
    const uint16_t* nw = nullptr;
    if (h < 16) {
      src = row + h * 512;  // q half of the head's [q(256) gate(256)]
      nw = d.q_norm_w;
      const uint16_t* gsrc = row + h * 512 + 256;
#pragma unroll
      for (int i = 0; i < 4; ++i) d.gate[((size_t)t * 16 + h) * 256 + lane + 64 * i] = gsrc[lane + 64 * i];
    } else if (h < 18) {
      src = row + 8192 + (h - 16) * 256;
      nw = d.k_norm_w;
    } else {
      src = row + 8704 + (h - 18) * 256;
    }
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = bf2f(src[lane + 64 * i]);
    if (nw) {
      const float ss = wave_sum_bfly((x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]));
      const float inv = 1.f / sqrtf(ss / 256.f + d.eps);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = rbf((x[i] * inv) * (bf2f(nw[lane + 64 * i]) + 1.f));
      // RoPE on dims 0..63 = x[0] of every lane: pair (i, i + 32) = lanes (l, l ^ 32)
      const float other = __shfl_xor(x[0], 32);
      const int i = lane & 31;
      const float c = cs[i], s = cs[32 + i];
      x[0] = lane < 32 ? rbf(x[0] * c - other * s) : rbf(x[0] * c + other * s);
    }
    if (h < 16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) d.q[((size_t)t * 16 + h) * 256 + lane + 64 * i] = (uint16_t)f2bf(x[i]);
    } else {
      const int hh = h < 18 ? h - 16 : h - 18;
      uint16_t* dst = h < 18 ? d.k : d.v;
      uint8_t* dst8 = h < 18 ? d.k8 : d.v8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const size_t o = ((size_t)t * 2 + hh) * 256 + lane + 64 * i;
        dst[o] = (uint16_t)f2bf(x[i]);
        dst8[o] = (uint8_t)(f2e4m3x2_hw(x[i], 0.f) & 0xffu);
      }
    }
  }
}

struct AttnWs {
  size_t xq, xs, qkv, total;
};
AttnWs attn_ws(int T) {
  AttnWs w;
  size_t o = 0;
  auto take = [&](size_t b) {
    size_t r = o;
    o = align_up(o + b, 256);
    return r;
  };
  w.xq = take((size_t)T * 2048);
  w.xs = take(sizeof(float) * (size_t)T * 16);
  w.qkv = take(sizeof(uint16_t) * (size_t)T * 9216);
  w.total = o;
  return w;
}
struct OprojWs {
  size_t aq, as, total;
};
OprojWs oproj_ws(int T) {
  OprojWs w;
  size_t o = 0;
  auto take = [&](size_t b) {
    size_t r = o;
    o = align_up(o + b, 256);
    return r;
  };
  w.aq = take((size_t)T * 4096);
  w.as = take(sizeof(float) * (size_t)T * 32);
  w.total = o;
  return w;
}

int launch_gemm(const uint8_t* A, const float* As, int T, int K, const uint8_t* W, const float* Ws, int N,
                uint16_t* Y, hipStream_t st) {
  GemmDev g{A, As, T, K, W, Ws, N, Y};
  dim3 grid(N / 64, (T + kGTB - 1) / kGTB);
  fp8_gemm_kernel<<<grid, 256, 0, st>>>(g);
  return Q36_OK;
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" size_t q36_attn_workspace_bytes(int32_t T) { return attn_ws(T).total; }
extern "C" size_t q36_oproj_workspace_bytes(int32_t T) { return oproj_ws(T).total; }

extern "C" int q36_attn_proj(const q36_attn_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_attn_proj: null args");
  Q36_REQUIRE(a->T >= 1 && a->T <= 65535, "q36_attn_proj: T=%d out of range", a->T);
  Q36_REQUIRE(a->max_pos >= 1, "q36_attn_proj: max_pos=%d", a->max_pos);
  Q36_REQUIRE(a->x && a->wqkv && a->sqkv && a->q_norm_w && a->k_norm_w && a->cos_sin && a->positions && a->q &&
                  a->gate && a->k && a->v && a->k8 && a->v8 && a->workspace,
              "q36_attn_proj: a required pointer is null");
  Q36_REQUIRE(aligned16(a->x) && aligned16(a->wqkv) && (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_attn_proj: x, wqkv must be 16-byte and workspace 256-byte aligned");
  const AttnWs L = attn_ws(a->T);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_attn_proj: workspace of %zu bytes < %zu required",
              a->workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(a->workspace);
  uint8_t* xq = reinterpret_cast<uint8_t*>(ws + L.xq);
  float* xs = reinterpret_cast<float*>(ws + L.xs);
  uint16_t* qkv = reinterpret_cast<uint16_t*>(ws + L.qkv);
  act_quant_kernel<<<a->T, 256, 0, st>>>(static_cast<const uint16_t*>(a->x), nullptr, 2048, xq, xs);
  launch_gemm(xq, xs, a->T, 2048, static_cast<const uint8_t*>(a->wqkv), a->sqkv, 9216, qkv, st);
  RopeDev r{a->T, a->max_pos, qkv, static_cast<const uint16_t*>(a->q_norm_w),
            static_cast<const uint16_t*>(a->k_norm_w), a->eps, a->cos_sin, a->positions,
            static_cast<uint16_t*>(a->q), static_cast<uint16_t*>(a->gate), static_cast<uint16_t*>(a->k),
            static_cast<uint16_t*>(a->v), static_cast<uint8_t*>(a->k8), static_cast<uint8_t*>(a->v8)};
  norm_rope_kernel<<<a->T, 512, 0, st>>>(r);
  return check_launch("q36_attn_proj");
}

extern "C" int q36_attn_oproj(const q36_oproj_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_attn_oproj: null args");
  Q36_REQUIRE(a->T >= 1 && a->T <= 65535, "q36_attn_oproj: T=%d out of range", a->T);
  Q36_REQUIRE(a->attn && a->gate && a->wo && a->so && a->out && a->workspace,
              "q36_attn_oproj: a required pointer is null");
  Q36_REQUIRE(aligned16(a->attn) && aligned16(a->gate) && aligned16(a->wo) &&
                  (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_attn_oproj: attn, gate, wo must be 16-byte and workspace 256-byte aligned");
  const OprojWs L = oproj_ws(a->T);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_attn_oproj: workspace of %zu bytes < %zu required",
              a->workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(a->workspace);
  uint8_t* aq = reinterpret_cast<uint8_t*>(ws + L.aq);
  float* as = reinterpret_cast<float*>(ws + L.as);
  act_quant_kernel<<<a->T, 256, 0, st>>>(static_cast<const uint16_t*>(a->attn), static_cast<const uint16_t*>(a->gate),
                                         4096, aq, as);
  launch_gemm(aq, as, a->T, 4096, static_cast<const uint8_t*>(a->wo), a->so, 2048, static_cast<uint16_t*>(a->out), st);
  return check_launch("q36_attn_oproj");
}
