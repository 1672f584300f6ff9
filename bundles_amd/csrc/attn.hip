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
// streams the whole K for its own tokens with both operands straight from global memory), norm_rope
// (one wave per token and head).
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
// The e4m3 values are written in MFMA fragment order (below), the GEMM's activation loads then
// being 1 KB contiguous per wave instruction.
// gate != nullptr: the value quantized is bf16(x * sigmoid(gate)) (the o_proj input).  Scales are
// stored transposed with the token count rounded up to 4, s[group][Tp], so that a GEMM lane reads
// its four tokens' scales with one 16-byte load.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* x, const uint16_t* gate, int K, uint8_t* q,
                                                        float* s) {
  const int t = blockIdx.x, tid = threadIdx.x, Tp = (gridDim.x + 3) & ~3;
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
    // fragment layout: 16-token tile, 128-block kb, half h, lane l = 16 g + t % 16, byte j holds
    // element k = 128 kb + 32 g + 16 h + j of token t (the lane's MFMA operand is its two 16-byte
    // halves, 1 KB apart)
    const int k = 8 * c, kb = k >> 7, g = (k >> 5) & 3, h = (k >> 4) & 1, j = k & 15;
    const size_t off = (((size_t)(t >> 4) * (K >> 7) + kb) << 11) + (h << 10) + ((g * 16 + (t & 15)) << 4) + j;
    *reinterpret_cast<uint2*>(q + off) = make_uint2(wd[0], wd[1]);
    if ((c & 15) == 0) s[(size_t)(c / 16) * Tp + t] = m / 448.f;
  }
}

// ------------------------------------------------------------------------------------------
// skinny e4m3 GEMM:  Y[t, n] = bf16(acc), acc = fma(blocksum_kb(t, n), xs[t, kb] * ws[n / 128, kb], acc)
// over the 128-blocks kb in increasing order from zero.
// Both operands are stored in MFMA fragment order: for a 16-row tile and a 128-block, 2 KB holding
// half h (16 bytes) of lane l's operand at h * 1024 + 16 l, so that a wave reads a fragment with two
// 1 KB contiguous loads (row-major rows are K bytes apart: a lane-per-row load is 64 separate
// requests).
// Workgroup = RT 16-row weight tiles x 4 waves of TPW 16-token tiles each.  Every wave streams the
// whole K for its own tokens, loading both MFMA operands straight from global memory four blocks
// ahead (the K loop is fully unrolled, so the register stages rotate by name); the weight
// fragments the four waves share come from L1 after the first.  No LDS.  MFMA src0 = tokens
// (lane row l%16), src1 = weight rows; lane l of the 16x16 result holds weight row l%16 and token
// rows 4 (l/16) + r.
// ------------------------------------------------------------------------------------------
struct GemmDev {
  const uint8_t* A;   // e4m3 [T16 / 16 tiles][K / 128 blocks][2 halves][64 lanes][16 B]
  const float* AsT;   // [K/128, Tp], Tp = T rounded up to 4
  int T, K;
  const uint8_t* W;   // e4m3 in fragment order [N / 16][K / 128][2][64][16 B]
  const float* Ws;    // [N/128, K/128]
  int N;
  uint16_t* Y;        // bf16 [T, N]
};

template <int RT, int TPW, int NKB>
__global__ __launch_bounds__(256) void fp8_gemm_kernel(GemmDev g) {
  constexpr int D = 4;  // blocks in flight
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lgp = lane >> 4;
  const int n0 = blockIdx.x * 16 * RT;
  const int tw = (blockIdx.y * 4 + wave) * TPW * 16;  // first token of this wave
  if (tw >= g.T) return;                                // no tokens: nothing to do (no barriers)
  const int Tp = (g.T + 3) & ~3;
  const uint8_t* wp[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) wp[r] = g.W + ((size_t)((n0 >> 4) + r) * NKB << 11) + lane * 16;
  const uint8_t* ap[TPW];
  int sct[TPW];  // first of the lane's four output tokens per tile, clamped into the scale row
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int tile = min((tw >> 4) + tt, (g.T - 1) >> 4);  // tiles past T: the last one (discarded)
    ap[tt] = g.A + ((size_t)tile * NKB << 11) + lane * 16;
    sct[tt] = min(tw + tt * 16 + 4 * lgp, (g.T - 1) & ~3);
  }
  const float* wsr = g.Ws + (size_t)(n0 / 128) * NKB;
  struct Stage {
    v4i w[RT][2];
    v4i a[TPW][2];
    float4 sc[TPW];
    float ws;
  };
  auto load = [&](Stage& st, int kb) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      st.w[r][0] = ldg16a(wp[r] + kb * 2048);
      st.w[r][1] = ldg16a(wp[r] + kb * 2048 + 1024);
    }
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      st.a[tt][0] = ldg16a(ap[tt] + kb * 2048);
      st.a[tt][1] = ldg16a(ap[tt] + kb * 2048 + 1024);
      // tokens past T read padding or the next row: their results are never stored
      st.sc[tt] = *reinterpret_cast<const float4*>(g.AsT + (size_t)kb * Tp + sct[tt]);
    }
    st.ws = wsr[kb];
  };
  float acc[RT][TPW][4];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[r][tt][q] = 0.f;
  auto compute = [&](const Stage& st) {
    v4f rr[RT][TPW];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt)
        rr[r][tt] = mfma_e4m3(cat8a(st.a[tt][0], st.a[tt][1]), cat8a(st.w[r][0], st.w[r][1]));
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) {
        acc[r][tt][0] = __builtin_fmaf(rr[r][tt][0], st.sc[tt].x * st.ws, acc[r][tt][0]);
        acc[r][tt][1] = __builtin_fmaf(rr[r][tt][1], st.sc[tt].y * st.ws, acc[r][tt][1]);
        acc[r][tt][2] = __builtin_fmaf(rr[r][tt][2], st.sc[tt].z * st.ws, acc[r][tt][2]);
        acc[r][tt][3] = __builtin_fmaf(rr[r][tt][3], st.sc[tt].w * st.ws, acc[r][tt][3]);
      }
    // the sums are formed here (left alone, the compiler sinks them below the K loop and keeps
    // every MFMA result live)
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
        for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(acc[r][tt][q]));
  };
  Stage st[D];
#pragma unroll
  for (int i = 0; i < D; ++i) load(st[i], i);
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    compute(st[kb % D]);
    if (kb + D < NKB) load(st[kb % D], kb + D);
  }
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      const int n = n0 + r * 16 + lr;
      const int t = tw + tt * 16 + 4 * lgp;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (t + q < g.T) g.Y[(size_t)(t + q) * g.N + n] = (uint16_t)f2bf(acc[r][tt][q]);
    }
}

// ------------------------------------------------------------------------------------------
// per-(token, head) epilogue of the QKV projection: one wave per item, 20 items per token (16 q
// heads with their gates, 2 k, 2 v); lane holds dims lane + 64 i.  q and k: Gemma RMSNorm over 256
// dims (sum
// of squares by an xor butterfly over the wave, rstd = 1/sqrt(ss/256 + eps)), x = bf16((x * rstd) *
// (1 + w)), then neox RoPE on dims 0..63 (pairs i, i + 32) with the fp32 cos|sin row of the
// position; k and v also go to the e4m3 cache (satfinite, no scale).
// ------------------------------------------------------------------------------------------
struct RopeDev {
  int T, max_pos;
  const uint16_t* qkv;  // bf16 [T, 8192 q/gate | 512 k | 512 v]
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
__global__ __launch_bounds__(256) void norm_rope_kernel(RopeDev d) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (item >= d.T * 20) return;
  const int t = item / 20, h = item % 20;
  // the head's values (and, for q heads, its gate) are loaded before the position's cos|sin row,
  // whose address depends on another load
  const uint16_t* row = d.qkv + (size_t)t * 9216;
  int col;
  const uint16_t* nw = nullptr;
  if (h < 16) {
    col = h * 512;  // q half of the head's [q(256) gate(256)]
    nw = d.q_norm_w;
  } else if (h < 18) {
    col = 8192 + (h - 16) * 256;
    nw = d.k_norm_w;
  } else {
    col = 8704 + (h - 18) * 256;
  }
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = bf2f(row[col + lane + 64 * i]);
  if (h < 16) {
    uint16_t gv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) gv[i] = row[col + 256 + lane + 64 * i];
#pragma unroll
    for (int i = 0; i < 4; ++i) d.gate[((size_t)t * 16 + h) * 256 + lane + 64 * i] = gv[i];
  }
  int pos = d.positions[t];
  pos = pos < 0 ? 0 : (pos >= d.max_pos ? d.max_pos - 1 : pos);
  const float* cs = d.cos_sin + (size_t)pos * 64;
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
  w.xq = take((size_t)((T + 15) & ~15) * 2048);
  w.xs = take(sizeof(float) * (size_t)16 * ((T + 3) & ~3));
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
  w.aq = take((size_t)((T + 15) & ~15) * 4096);
  w.as = take(sizeof(float) * (size_t)32 * ((T + 3) & ~3));
  w.total = o;
  return w;
}

// RT 16-row tiles per workgroup; TPW token tiles per wave (a workgroup covers 64 TPW tokens)
template <int RT, int TPW, int NKB>
void launch_gemm(const GemmDev& g, hipStream_t st) {
  const dim3 grid(g.N / (16 * RT), (g.T + 64 * TPW - 1) / (64 * TPW));
  fp8_gemm_kernel<RT, TPW, NKB><<<grid, 256, 0, st>>>(g);
}

// 8-bit codes (e4m3 or int8) [N, K] row-major -> fragment order; thread = one 16-byte chunk of the output
__global__ __launch_bounds__(256) void pack_frag_kernel(const uint8_t* q, int64_t N, int K, uint8_t* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // output chunk
  const int64_t total = N * K / 16;
  if (i >= total) return;
  const int l = (int)(i & 63), h = (int)((i >> 6) & 1);
  const int64_t frag = i >> 7;  // (tile, block)
  const int nkb = K >> 7;
  const int64_t tile = frag / nkb;
  const int kb = (int)(frag % nkb);
  const uint8_t* src = q + (tile * 16 + (l & 15)) * (int64_t)K + kb * 128 + (l >> 4) * 32 + h * 16;
  *reinterpret_cast<v4i*>(out + i * 16) = *reinterpret_cast<const v4i*>(src);
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
  const GemmDev g{xq, xs, a->T, 2048, static_cast<const uint8_t*>(a->wqkv), a->sqkv, 9216, qkv};
  if (a->T > 64)
    launch_gemm<2, 2, 16>(g, st);
  else
    launch_gemm<1, 1, 16>(g, st);
  RopeDev r{a->T, a->max_pos, qkv, static_cast<const uint16_t*>(a->q_norm_w),
            static_cast<const uint16_t*>(a->k_norm_w), a->eps, a->cos_sin, a->positions,
            static_cast<uint16_t*>(a->q), static_cast<uint16_t*>(a->gate), static_cast<uint16_t*>(a->k),
            static_cast<uint16_t*>(a->v), static_cast<uint8_t*>(a->k8), static_cast<uint8_t*>(a->v8)};
  norm_rope_kernel<<<(a->T * 20 + 3) / 4, 256, 0, st>>>(r);
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
  const GemmDev g{aq, as, a->T, 4096, static_cast<const uint8_t*>(a->wo), a->so, 2048, static_cast<uint16_t*>(a->out)};
  launch_gemm<1, 1, 32>(g, st);
  return check_launch("q36_attn_oproj");
}

extern "C" int q36_pack_frag8(const void* q, int64_t N, int32_t K, void* packed, q36_stream_t stream) {
  Q36_REQUIRE(q && packed, "q36_pack_frag8: null pointer");
  Q36_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 128 == 0, "q36_pack_frag8: N=%lld K=%d must be multiples of 16 and 128",
              (long long)N, K);
  Q36_REQUIRE(aligned16(q) && aligned16(packed), "q36_pack_frag8: pointers must be 16-byte aligned");
  const int64_t chunks = N * K / 16;
  pack_frag_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t*>(q), N, K, static_cast<uint8_t*>(packed));
  return check_launch("q36_pack_frag8");
}
