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
// Kernels: act_quant (bf16 -> e4m3 + scales, optionally gated), proj_gemm (each wave streams two
// 16-row weight tiles over K from HBM; the token group's activations come through an LDS chunk
// ring shared by the workgroup), norm_rope (one wave per token and head).
#include <type_traits>
#include <utility>

#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

__device__ __forceinline__ v4i ldg16a(const uint8_t* p) { return *reinterpret_cast<const v4i*>(p); }
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
// e4m3 codes q and per 128-group scales s[T][K/128]; the codes row-major [T][K], or (frag) in MFMA
// fragment order: token tile t / 16 and 128-block kb at ((t / 16) * K / 128 + kb) * 2048, byte j of
// the block at (j % 32) / 16 * 1024 + 16 * (t % 16 + 16 * (j / 32)) + j % 16 -- the 32 bytes lane
// t % 16 + 16 (j / 32) feeds the MFMA, as two 16-byte halves 1 KB apart.  In fragment order the grid
// also covers the tokens up to the next multiple of 16, whose codes and scales are zero.
// gate != nullptr: the value quantized is bf16(x * sigmoid(gate)) (the o_proj input).
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* x, const uint16_t* gate, int T, int K, bool frag,
                                                        uint8_t* q, float* s) {
  const int t = blockIdx.x, tid = threadIdx.x;
  if (t >= T) {  // fragment-order padding token
    for (int c = tid; 8 * c < K; c += 256) {
      *reinterpret_cast<uint2*>(q + frag_offset(t, 8 * c, K)) = make_uint2(0u, 0u);
      if ((c & 15) == 0) s[(size_t)t * (K >> 7) + c / 16] = 0.f;
    }
    return;
  }
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
    *reinterpret_cast<uint2*>(q + (frag ? frag_offset(t, 8 * c, K) : (size_t)t * K + 8 * c)) = e4m3_run8(f, inv);
    if ((c & 15) == 0) s[(size_t)t * (K >> 7) + c / 16] = m / 448.f;
  }
}

// ------------------------------------------------------------------------------------------
// e4m3 projection GEMM:  Y[t, n] = bf16(acc), acc = fma(blocksum_kb(t, n), xs[t, kb] * ws[n / 128, kb],
// acc) over the 128-blocks kb in increasing order from zero.
// Weights in MFMA fragment order (q36_pack_frag8): for a 16-row tile and a 128-block, 2 KB holding
// half h (16 bytes) of lane l's operand at h * 1024 + 16 l; a wave reads a fragment with two 1 KB
// contiguous loads.
// Workgroup = 64 TPW weight rows (4 waves x TPW 16-row tiles) x one group of 16 NTT tokens.  Each
// wave streams its tiles over K from HBM in 128-byte stages, kPD stages in flight, through buffer
// loads with the stage offset in the scalar offset.  The group's activation rows go through LDS
// in 512-byte K chunks, double-buffered (a chunk's copy overlaps the previous chunk's stages, so the
// weight stream never drains), shared by the four waves; a chunk row's 16-byte piece p sits at
// position p ^ (row % 16), which puts the 16 rows of one MFMA read on distinct banks.  The weights
// are the MFMA's first operand: lane l ends with token l % 16 of the tile and rows 4 (l / 16) .. +3,
// one 8-byte store.  The token groups of a row block are 72 or 32 workgroups apart in the grid, so
// they run on one XCD and share its L2 for the weights.
// ------------------------------------------------------------------------------------------
struct GemmDev {
  const uint8_t* A;   // e4m3 [T, K] row-major
  const float* As;    // [T, K/128]
  int T, K;
  const uint8_t* W;   // e4m3 in fragment order [N / 16][K / 128][2][64][16 B]
  const float* Ws;    // [N/128, K/128]
  int N;
  // bf16 outputs: columns [c0[i], c0[i + 1]) of the first nout go to ys[i] with row stride ld[i]
  // (column c0[i] at ys[i][t * ld[i]]); the rest are padding rows of W and are not written
  int nseg, nout;
  int c0[4], ld[4];
  uint16_t* ys[4];
};
GemmDev gemm_dev(const uint8_t* A, const float* As, int T, int K, const uint8_t* W, const float* Ws, int N,
                 uint16_t* Y) {
  return GemmDev{A, As, T, K, W, Ws, N, 1, N, {0, 0, 0, 0}, {N, 0, 0, 0}, {Y, nullptr, nullptr, nullptr}};
}
constexpr int kPKC = 512;  // K bytes per LDS chunk
__device__ __forceinline__ void pdma16(__amdgpu_buffer_rsrc_t rs, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds, 16, voff, 0, 0, 0);
}

// token tiles, K blocks, weight stages in flight per wave, 16-row weight tiles per wave (the
// workgroup covers 64 TPW rows)
template <int NTT, int NKB, int kPD, int TPW>
__global__ __launch_bounds__(256) void proj_gemm_kernel(GemmDev g) {
  constexpr int TG = 16 * NTT, SPC = kPKC / 128, NC = NKB / SPC;
  static_assert(NKB % SPC == 0 && kPD <= SPC, "K must be whole chunks, a chunk a full window of stages");
  // separate objects, so the compiler sees that a copy into one buffer does not touch reads of the other
  __shared__ __align__(16) uint8_t a_b0[TG * kPKC];
  __shared__ __align__(16) uint8_t a_b1[TG * kPKC];
  __shared__ __align__(16) float xs_l[NKB * TG];  // [NKB][TG], token fastest
  __shared__ float ws_l[4][NKB];                  // each wave's weight block scales
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lgp = lane >> 4;
  // XCD-aware order: workgroup b runs on XCD b % 8, which owns the row blocks rb = xcd (mod 8) with
  // every token group of each, so a weight tile is fetched into one L2 and its re-reads by the other
  // token groups hit there
  const int nrb = g.N / (64 * TPW), ntg = (g.T + TG - 1) / TG;
  const int xcd = blockIdx.x & 7, jj = blockIdx.x >> 3;
  const int rb = xcd + 8 * (jj / ntg);
  if (rb >= nrb) return;
  const int t0 = (jj % ntg) * TG;
  const int n0 = __builtin_amdgcn_readfirstlane(rb * 64 * TPW + wave * 16 * TPW);  // the wave's tiles
  const int K = NKB * 128;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.W + ((size_t)(n0 >> 4) * NKB << 11)), (short)0, TPW * NKB << 11, 0x00020000);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)g.A, (short)0, g.T * K, 0x00020000);
  const int xsbytes = g.T * NKB * 4;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc((void*)g.As, (short)0, xsbytes, 0x00020000);
  // the wave's weight scales (one 128-row block) go to LDS with the activation scales: a vector load
  // per stage would be the newest load at its wait and drain the weight stream
  const float wsv = lane < NKB ? g.Ws[(size_t)(n0 / 128) * NKB + lane] : 0.f;
  v4i Bq[kPD][2 * TPW];
  auto issue = [&](int s, int q) {
#pragma unroll
    for (int c = 0; c < TPW; ++c) {
      Bq[q][2 * c] = __builtin_amdgcn_raw_buffer_load_b128(wrs, lane * 16, (c * NKB + s) * 2048, 2);
      Bq[q][2 * c + 1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, lane * 16, (c * NKB + s) * 2048 + 1024, 2);
    }
  };
  // chunk c of the group's rows: one call fills two rows (lanes 0-31 row 2m, 32-63 row 2m + 1); a
  // lane fetches the piece that belongs at its position; rows past T read as zero
  auto rows_dma = [&](int c) {
    uint8_t* buf = (c & 1) ? a_b1 : a_b0;
#pragma unroll
    for (int k = 0; k < TG / 8; ++k) {
      const int m = wave + 4 * k, rr = 2 * m + (lane >> 5), p = lane & 31;
      const int voff = t0 + rr < g.T ? (t0 + rr) * K + c * kPKC + 16 * (p ^ (rr & 15)) : g.T * K;
      pdma16(xrs, buf + 2 * m * kPKC, voff);
    }
  };
  // the group's activation scales into registers, then LDS once the first weights are requested
  float xsr[NKB * TG / 256];
#pragma unroll
  for (int q = 0; q < NKB * TG / 256; ++q) {
    const int i = tid + 256 * q, tt = i % TG, kb = i / TG;
    const int off = t0 + tt < g.T ? ((t0 + tt) * NKB + kb) * 4 : xsbytes;
    xsr[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, off, 0, 0));
  }
  rows_dma(0);
#pragma unroll
  for (int s = 0; s < kPD; ++s) issue(s, s);
#pragma unroll
  for (int q = 0; q < NKB * TG / 256; ++q) xs_l[tid + 256 * q] = xsr[q];
  if (lane < NKB) ws_l[wave][lane] = wsv;
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * TPW * kPD) : "memory");  // the rows, not the weights
  __syncthreads();
  asm volatile("" ::: "memory");
  v4f acc[TPW][NTT];
#pragma unroll
  for (int c = 0; c < TPW; ++c)
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) acc[c][tt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c > 0) {
      // chunk c landed (its copy is older than the chunk's 2 TPW SPC weight loads) and every wave
      // is done with chunk c - 1, whose buffer the next copy reuses
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * TPW * SPC) : "memory");
      __syncthreads();
      asm volatile("" ::: "memory");
    }
    if (c + 1 < NC) rows_dma(c + 1);
    const uint8_t* buf = (c & 1) ? a_b1 : a_b0;
#pragma unroll
    for (int sl = 0; sl < SPC; ++sl) {
      const int s = c * SPC + sl, q = s % kPD;
      const float ws = ws_l[wave][s];
      v8i a[NTT];
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) {
        const int row = tt * 16 + lr;
        const v4i a0 = *reinterpret_cast<const v4i*>(buf + row * kPKC + 16 * ((sl * 8 + lgp * 2) ^ lr));
        const v4i a1 = *reinterpret_cast<const v4i*>(buf + row * kPKC + 16 * ((sl * 8 + lgp * 2 + 1) ^ lr));
        a[tt] = cat8a(a0, a1);
      }
      v8i wt[TPW];
#pragma unroll
      for (int c = 0; c < TPW; ++c) wt[c] = cat8a(Bq[q][2 * c], Bq[q][2 * c + 1]);
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) {
        const float xw = xs_l[s * TG + tt * 16 + lr] * ws;  // this lane's token
#pragma unroll
        for (int c = 0; c < TPW; ++c) {
          const v4f r = mfma_e4m3(wt[c], a[tt]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[c][tt][i] = __builtin_fmaf(r[i], xw, acc[c][tt][i]);
        }
      }
      // the running sums are formed here (left alone, the compiler sinks the chain below the
      // stage loop and keeps every stage's MFMA results live)
#pragma unroll
      for (int c2 = 0; c2 < TPW; ++c2)
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
          for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(acc[c2][tt][r]));
      if (s + kPD < NKB) issue(s + kPD, q);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // lane: token t0 + 16 tt + l % 16, rows n0 + 16 c + 4 (l / 16) .. +3 (four columns never straddle
  // a segment: the boundaries are multiples of 4)
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) {
    const int t = t0 + tt * 16 + lr;
    if (t < g.T) {
#pragma unroll
      for (int c = 0; c < TPW; ++c) {
        const int col = n0 + c * 16 + 4 * lgp;
        if (col < g.nout) {
          const int sg = (g.nseg > 1 && col >= g.c0[1]) + (g.nseg > 2 && col >= g.c0[2]) + (g.nseg > 3 && col >= g.c0[3]);
          *reinterpret_cast<uint2*>(g.ys[sg] + (size_t)t * g.ld[sg] + (col - g.c0[sg])) =
              make_uint2(pack_bf2(acc[c][tt][0], acc[c][tt][1]), pack_bf2(acc[c][tt][2], acc[c][tt][3]));
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// K-sliced e4m3 projection GEMM: the same Y = bf16(sum_kb blocksum_kb(t, n) * xs[t, kb] * ws[n / 128, kb])
// with the activations in fragment order (act_quant frag).  Workgroup = RG x KS waves over a tile of
// 16 RT RG weight rows x 16 TT tokens; wave (rg, ks) owns RT 16-row tiles and the KB 128-blocks
// ks KB .. +KB-1 of K, and keeps DEPTH blocks of its weight fragments in flight from the start, so
// no wave waits on more than KB / DEPTH round trips.  Its running sums acc = fma(blocksum, xs * ws,
// acc) go over its own blocks in increasing order from zero; the KS slices then meet in LDS and are
// added in slice order (the K order of the slices).  The token group's activation fragments
// (TT x K/128 x 2 KB) are copied into LDS once by buffer DMA and read by the RG row groups there.
// The token groups of a row block are 8 workgroups apart in the grid, so they run on one XCD and
// share its L2 for the weights.
// ------------------------------------------------------------------------------------------
template <int RT, int TT, int KB, int RG, int KS, int DEPTH>
__global__ __launch_bounds__(64 * RG * KS) __attribute__((amdgpu_waves_per_eu(RG * KS / 4, RG * KS / 4))) void
ks_gemm_kernel(GemmDev g) {
  constexpr int NW = RG * KS, NKB = KB * KS, TG = 16 * TT, RB = 16 * RT * RG;
  constexpr int QW = RT * TT;                   // output fragments (16 x 16) per wave
  constexpr int PART = KS * RG * QW * 64 * 16;  // partial sums, bytes
  constexpr int ABYTES = TT * NKB * 2048;
  static_assert(KB % DEPTH == 0 && DEPTH <= KB, "whole rounds of blocks in flight");
  __shared__ __align__(16) uint8_t lds[PART > ABYTES ? PART : ABYTES];
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave / KS, ks = wave % KS;
  const int nrb = g.N / RB, ntg = (g.T + TG - 1) / TG;
  const int xcd = blockIdx.x & 7, jj = blockIdx.x >> 3;
  const int rb = xcd + 8 * (jj / ntg);
  if (rb >= nrb) return;
  const int t0 = (jj % ntg) * TG;
  const int tile0 = __builtin_amdgcn_readfirstlane((rb * RB) / 16 + rg * RT);  // the wave's first row tile
  const int kb0 = ks * KB;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.W + ((size_t)tile0 * NKB << 11)), (short)0, RT * NKB << 11, 0x00020000);
  // activation fragments of the token group: tiles t0 / 16 .. (tiles past the padded T read zero)
  const int ntile_a = (g.T + 15) / 16 - t0 / 16;
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.A + ((size_t)(t0 / 16) * NKB << 11)), (short)0, (ntile_a < TT ? ntile_a : TT) * NKB << 11, 0x00020000);
  const int xsbytes = g.T * NKB * 4;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc((void*)g.As, (short)0, xsbytes, 0x00020000);
  // scales: the lane's token for every (token tile, block), the wave's weight block of every (tile, block)
  float xs[TT][KB], wsc[RT][KB];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int t = t0 + 16 * tt + lr;
      xs[tt][kb] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(srs, t < g.T ? (t * NKB + kb0 + kb) * 4 : xsbytes, 0, 0));
    }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) wsc[rt][kb] = g.Ws[(size_t)((tile0 + rt) >> 3) * NKB + kb0 + kb];
  // 1 KB per DMA instruction, the group's fragments copied in global order
  for (int i = wave; i < TT * NKB * 2; i += NW) pdma16(ars, lds + i * 1024, lane * 16 + i * 1024);
  asm volatile("" ::: "memory");  // the copies stay ahead of the weight loads (the wait below counts on it)
  v4i Wf[DEPTH][RT][2];
  auto issue = [&](int kb, int sl) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        Wf[sl][rt][h] = __builtin_amdgcn_raw_buffer_load_b128(wrs, lane * 16, ((rt * NKB + kb0 + kb) << 11) + h * 1024, 2);
  };
  __builtin_amdgcn_sched_barrier(0);  // the scales first: they are needed by the first accumulate
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) issue(d, d);
  __builtin_amdgcn_sched_barrier(0);  // every round in flight before the first MFMA
  // the copies are older than the DEPTH rounds of weight loads just issued
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DEPTH * RT * 2) : "memory");
  __syncthreads();
  asm volatile("" ::: "memory");
  v4f acc[RT][TT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[rt][tt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int sl = kb % DEPTH;
    v8i a[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const uint8_t* ap = lds + ((tt * NKB + kb0 + kb) << 11) + lane * 16;
      a[tt] = cat8a(*reinterpret_cast<const v4i*>(ap), *reinterpret_cast<const v4i*>(ap + 1024));
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const v8i w = cat8a(Wf[sl][rt][0], Wf[sl][rt][1]);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const v4f r = mfma_e4m3(w, a[tt]);
        const float xw = xs[tt][kb] * wsc[rt][kb];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rt][tt][i] = __builtin_fmaf(r[i], xw, acc[rt][tt][i]);
      }
    }
    if (kb + DEPTH < KB) issue(kb + DEPTH, sl);
  }
  // the slices meet in LDS: [ks][rg][rt][tt][lane] float4
  __syncthreads();  // every wave is done reading the activation fragments
  float4* part = reinterpret_cast<float4*>(lds);
  constexpr int Q = RG * QW * 64;  // output quads of the workgroup
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
      part[(size_t)ks * Q + ((rg * RT + rt) * TT + tt) * 64 + lane] =
          make_float4(acc[rt][tt][0], acc[rt][tt][1], acc[rt][tt][2], acc[rt][tt][3]);
  __syncthreads();
  for (int qd = tid; qd < Q; qd += 64 * NW) {
    float4 v = part[qd];
#pragma unroll
    for (int k = 1; k < KS; ++k) {
      const float4 u = part[(size_t)k * Q + qd];
      v.x += u.x;
      v.y += u.y;
      v.z += u.z;
      v.w += u.w;
    }
    // quad qd = ((rg' RT + rt) TT + tt) 64 + l: token t0 + 16 tt + l % 16, rows 4 (l / 16) .. +3 of tile rg' RT + rt
    const int l = qd & 63, f = qd >> 6, tt = f % TT, tr = f / TT;
    const int t = t0 + 16 * tt + (l & 15);
    const int col = rb * RB + tr * 16 + 4 * (l >> 4);
    if (t < g.T && col < g.nout) {
      const int sg = (g.nseg > 1 && col >= g.c0[1]) + (g.nseg > 2 && col >= g.c0[2]) + (g.nseg > 3 && col >= g.c0[3]);
      *reinterpret_cast<uint2*>(g.ys[sg] + (size_t)t * g.ld[sg] + (col - g.c0[sg])) =
          make_uint2(pack_bf2(v.x, v.y), pack_bf2(v.z, v.w));
    }
  }
}

// ------------------------------------------------------------------------------------------
// Tiled e4m3 projection GEMM for 64 tokens and more: the same Y = bf16(sum_kb blocksum_kb(t, n) *
// xs[t, kb] * ws[n / 128, kb]) (running sums fma(blocksum, xs * ws, acc) in increasing kb order from
// zero, so the bits equal the streaming and K-sliced GEMMs'), with both operands in MFMA fragment
// order (the weights as packed, the activations from act_quant's fragment mode).
// Workgroup = one 128-row block (one weight scale per K block) x BT tokens, 8 waves, two a SIMD:
// wave w owns row tiles 4 (w & 1) .. +3 and token tiles TTW (w >> 1) .. +TTW-1 (TTW = BT / 64).  K
// goes in 128-byte steps (one K block, one MFMA deep) through two LDS rings that buffer loads fill
// straight from global memory: the block's 8 weight tiles (6 stages, copied by waves 0-3 six steps
// ahead) and the BT / 16 token tiles (3 stages, L2-resident, copied by waves 4-7), 2 KB a tile,
// exactly as they lie in memory.  Vector-memory loads complete in order per wave, so one operand a
// wave lets each ring have its own depth.  The fragments (and scales) of step
// s + 1 are read while the MFMAs of step s run.  Per call every weight byte passes through L2
// ceil(T / BT) times and every activation byte N / 128 times (the streaming GEMM's 16- or 32-token
// groups re-read the weights T / 16 or T / 32 times).
// ------------------------------------------------------------------------------------------
template <int N>
using ic = std::integral_constant<int, N>;
// s_waitcnt with only the vector-memory count constrained (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int N>
__device__ __forceinline__ void tg_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// f(ic<0>{}), f(ic<1>{}), ... in order, each step's index a compile-time constant
template <typename F, int... KS>
__device__ __forceinline__ void for_steps(F& f, std::integer_sequence<int, KS...>) {
  (f(ic<KS>{}), ...);
}
constexpr int kTileNSW = 6, kTileNSA = 3;  // LDS ring stages of the weight tiles and of the token tiles
template <int BT, int NKB>
struct TileLds {
  static constexpr int WB = 8 * 2048, AB = (BT / 16) * 2048;  // stage bytes: weight tiles, token tiles
  uint8_t* w[kTileNSW];
  uint8_t* a[kTileNSA];
  float* xs;  // [NKB][BT]
  float* ws;  // [NKB]
};
// ROLE: the copies this wave issues (0: the weight tiles, waves 0-3; 1: the token tiles, waves 4-7);
// everything else is the same in both.  Each role is its own instantiation, so the compiler's wait
// counting sees only the wave's own operand in flight.
template <int BT, int NKB, int ROLE>
__device__ __forceinline__ void tile_gemm_body(const GemmDev& g, const TileLds<BT, NKB>& L) {
  constexpr int WB = TileLds<BT, NKB>::WB, AB = TileLds<BT, NKB>::AB;
  constexpr int CP = (ROLE == 0 ? WB : AB) / 1024 / 4;  // 1 KB copies a wave issues per step
  constexpr int NS = ROLE == 0 ? kTileNSW : kTileNSA;  // stages of its operand's ring
  constexpr int TTW = BT / 64;
  static_assert(CP >= 1 && NKB >= kTileNSW && TTW >= 1, "tile shape");
  auto w_st = [&](auto st) -> uint8_t* { return L.w[decltype(st)::value]; };
  auto a_st = [&](auto st) -> uint8_t* { return L.a[decltype(st)::value]; };
  float* const xs_l = L.xs;
  float* const ws_l = L.ws;
  // XCD-aware order: workgroup b runs on XCD b % 8, which owns the row blocks rb = xcd (mod 8) with
  // every token group of each, so a weight block is fetched into one L2 for all its token groups
  const int nrb = g.N / 128, ntg = (g.T + BT - 1) / BT;
  const int xcd = blockIdx.x & 7, jj = blockIdx.x >> 3;
  const int rb = xcd + 8 * (jj / ntg);
  if (rb >= nrb) return;
  const int t0 = (jj % ntg) * BT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), wr = wv & 1, wt = wv >> 1;
  // token tiles of this group that exist (act_quant pads T to whole tiles); the rest read as zero:
  // the tile offset rides in the VGPR offset, which the buffer range check covers
  const int Tq = (g.T + 15) & ~15, ntile = min(BT, Tq - t0) >> 4;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.W + (size_t)rb * 8 * NKB * 2048), (short)0, 8 * NKB * 2048, 0x00020000);
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.A + (size_t)(t0 >> 4) * NKB * 2048), (short)0, ntile * NKB * 2048, 0x00020000);
  // copy i of step ks: 1 KB chunk q = CP (w % 4) + i of the wave's operand's stage (tile q / 2,
  // half q % 2)
  auto issue = [&](auto ksc) {
    constexpr int ks = decltype(ksc)::value;
#pragma unroll
    for (int i = 0; i < CP; ++i) {
      const int q = (wv & 3) * CP + i;
      const int voff = lane * 16 + (q >> 1) * NKB * 2048 + (q & 1) * 1024;
      if constexpr (ROLE == 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, w_st(ic<ks % kTileNSW>{}) + q * 1024, 16, voff, ks * 2048, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, a_st(ic<ks % kTileNSA>{}) + q * 1024, 16, voff, ks * 2048, 0, 0);
    }
  };
  // the group's scales: activations [NKB][BT] and the block's weight scales, through registers
  constexpr int NXS = NKB * BT / 512;
  const int xsbytes = g.T * NKB * 4;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc((void*)g.As, (short)0, xsbytes, 0x00020000);
  float xsr[NXS];
#pragma unroll
  for (int q = 0; q < NXS; ++q) {
    const int i = tid + 512 * q, tt = i % BT, kb = i / BT;
    const int off = t0 + tt < g.T ? ((t0 + tt) * NKB + kb) * 4 : xsbytes;
    xsr[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, off, 0, 0));
  }
  const float wsv = tid < NKB ? g.Ws[(size_t)rb * NKB + tid] : 0.f;
  auto issue_one = [&](auto sc) { issue(sc); };
  for_steps(issue_one, std::make_integer_sequence<int, NS>{});
  tg_wait_vm<(NS - 1) * CP>();  // the scales and step 0 (the wave's loads complete in order)
#pragma unroll
  for (int q = 0; q < NXS; ++q) xs_l[tid + 512 * q] = xsr[q];
  if (tid < NKB) ws_l[tid] = wsv;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  v4f acc[4][TTW];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int tt = 0; tt < TTW; ++tt) acc[rt][tt] = v4f{0.f, 0.f, 0.f, 0.f};
  v8i wf[2][4], af[2][TTW];
  float xw[2][TTW];
  const int lo = lane * 16;
  auto read_frags = [&](auto ksc, auto fb) {
    constexpr int ks = decltype(ksc)::value, f = decltype(fb)::value;
    const uint8_t* wsp = w_st(ic<ks % kTileNSW>{});
    const uint8_t* asp = a_st(ic<ks % kTileNSA>{});
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const uint8_t* p = wsp + (4 * wr + rt) * 2048 + lo;
      wf[f][rt] = cat8a(*reinterpret_cast<const v4i*>(p), *reinterpret_cast<const v4i*>(p + 1024));
    }
#pragma unroll
    for (int tt = 0; tt < TTW; ++tt) {
      const uint8_t* p = asp + (TTW * wt + tt) * 2048 + lo;
      af[f][tt] = cat8a(*reinterpret_cast<const v4i*>(p), *reinterpret_cast<const v4i*>(p + 1024));
    }
    const float wsk = ws_l[ks];
#pragma unroll
    for (int tt = 0; tt < TTW; ++tt) xw[f][tt] = xs_l[ks * BT + (TTW * wt + tt) * 16 + (lane & 15)] * wsk;
  };
  read_frags(ic<0>{}, ic<0>{});
  auto step = [&](auto ksc) {
    constexpr int ks = decltype(ksc)::value, f = ks & 1;
    // this wave's copies of step ks + 1 have landed (only those of steps ks + 2 .. ks + NS - 1 went
    // out after them), its reads of step ks are done, and after the barrier every wave's are: the
    // stage step ks used is free
    constexpr int later = (ks + NS - 1 < NKB - 1 ? ks + NS - 1 : NKB - 1) - (ks + 1);
    tg_wait_vm<CP * (later > 0 ? later : 0)>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    using nfb = ic<1 - f>;
    if constexpr (ks + NS < NKB) issue(ic<ks + NS>{});
    if constexpr (ks + 1 < NKB) read_frags(ic<ks + 1>{}, nfb{});
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int tt = 0; tt < TTW; ++tt) {
        const v4f r = mfma_e4m3(wf[f][rt], af[f][tt]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rt][tt][i] = __builtin_fmaf(r[i], xw[f][tt], acc[rt][tt][i]);
      }
    // the running sums are formed here (left alone, the compiler may keep every step's MFMA
    // results live and sink the chain)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int tt = 0; tt < TTW; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[rt][tt][i]));
  };
  for_steps(step, std::make_integer_sequence<int, NKB>{});
  // lane: token t0 + BT / 4 wt + 16 tt + l % 16, rows 128 rb + 64 wr + 16 rt + 4 (l / 16) .. +3 (four
  // columns never straddle a segment: the boundaries are multiples of 4)
#pragma unroll
  for (int tt = 0; tt < TTW; ++tt) {
    const int t = t0 + (TTW * wt + tt) * 16 + (lane & 15);
    if (t < g.T) {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int col = rb * 128 + (4 * wr + rt) * 16 + 4 * (lane >> 4);
        if (col < g.nout) {
          const int sg = (g.nseg > 1 && col >= g.c0[1]) + (g.nseg > 2 && col >= g.c0[2]) + (g.nseg > 3 && col >= g.c0[3]);
          *reinterpret_cast<uint2*>(g.ys[sg] + (size_t)t * g.ld[sg] + (col - g.c0[sg])) =
              make_uint2(pack_bf2(acc[rt][tt][0], acc[rt][tt][1]), pack_bf2(acc[rt][tt][2], acc[rt][tt][3]));
        }
      }
    }
  }
}

template <int BT, int NKB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void tile_gemm_kernel(GemmDev g) {
  // one object per stage and operand: the compiler tracks the buffer-to-LDS loads of each apart
  constexpr int WB = TileLds<BT, NKB>::WB, AB = TileLds<BT, NKB>::AB;
  static_assert(kTileNSW == 6 && kTileNSA == 3, "the stage arrays below");
  __shared__ __align__(1024) uint8_t w_s0[WB], w_s1[WB], w_s2[WB], w_s3[WB], w_s4[WB], w_s5[WB];
  __shared__ __align__(1024) uint8_t a_s0[AB], a_s1[AB], a_s2[AB];
  __shared__ __align__(16) float xs_l[NKB * BT];  // [kb][token of the tile]
  __shared__ float ws_l[NKB];
  const TileLds<BT, NKB> L{{w_s0, w_s1, w_s2, w_s3, w_s4, w_s5}, {a_s0, a_s1, a_s2}, xs_l, ws_l};
  if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) < 4)
    tile_gemm_body<BT, NKB, 0>(g, L);
  else
    tile_gemm_body<BT, NKB, 1>(g, L);
}

// ------------------------------------------------------------------------------------------
// per-(token, head) epilogue of the QKV projection: one wave per item, 18 items per token (16 q heads
// with their gates, 2 kv heads).  Lanes 0-31 hold the normed head (q, or k), 8 consecutive dims a
// lane, lanes 32-63 its companion (the gate, or v); every access is 16 bytes a lane.  q and k: Gemma
// RMSNorm over 256 dims (sum of squares by an xor butterfly over the 32 lanes (ds_swizzle), rstd =
// 1/sqrt(ss/256 + eps)), x = bf16((x * rstd) * (1 + w)), then neox RoPE on dims 0..63 (pairs i,
// i + 32: lanes j and j ^ 4 of the first 8) with the fp32 cos|sin row of the position; k and v also
// go to the e4m3 cache (satfinite, no scale).
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
  const int64_t* out_loc;  // the cache append (optional): row out_loc[t] of kc / vc
  uint8_t* kc;
  uint8_t* vc;
  int64_t num_slots;
};
constexpr int kRopeItems = 18;  // waves per token
__global__ __launch_bounds__(256) void norm_rope_kernel(RopeDev d) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (item >= d.T * kRopeItems) return;
  const int t = item / kRopeItems, h = item % kRopeItems;
  const int half = lane >> 5, j = lane & 31;
  const bool qhead = h < 16;
  const int hh = h - 16;
  const int col = qhead ? h * 512 + half * 256 + 8 * j : (half ? 8704 : 8192) + hh * 256 + 8 * j;
  // the head's values and norm weights are requested before the position's cos|sin row, whose
  // address depends on another load
  const v4i raw = ldg16a(reinterpret_cast<const uint8_t*>(d.qkv + (size_t)t * 9216 + col));
  const v4i wraw = ldg16a(reinterpret_cast<const uint8_t*>((qhead ? d.q_norm_w : d.k_norm_w) + 8 * j));
  int pos = d.positions[t];
  pos = pos < 0 ? 0 : (pos >= d.max_pos ? d.max_pos - 1 : pos);
  // lanes j < 8 rotate dims 8 j .. 8 j + 7 with cos|sin entries i = 8 (j & 3) + e
  const float* cs = d.cos_sin + (size_t)pos * 64 + 8 * (j & 3);
  const float4 c0 = *reinterpret_cast<const float4*>(cs), c1 = *reinterpret_cast<const float4*>(cs + 4);
  const float4 s0 = *reinterpret_cast<const float4*>(cs + 32), s1 = *reinterpret_cast<const float4*>(cs + 36);
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = bf_lo((uint32_t)raw[i]);
    x[2 * i + 1] = bf_hi((uint32_t)raw[i]);
  }
  // the sum of squares: every lane takes part (the companion half's sums are not used)
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
  ss += xor_swz<16>(ss);
  ss += xor_swz<8>(ss);
  ss += xor_swz<4>(ss);
  ss += xor_swz<2>(ss);
  ss += xor_swz<1>(ss);
  const bool normed = half == 0;
  // branch-free: every lane computes the normed and rotated values, the selects keep what applies
  const float inv = 1.f / sqrtf(ss / 256.f + d.eps);
  float y[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[2 * i] = rbf_hw((x[2 * i] * inv) * (bf_lo((uint32_t)wraw[i]) + 1.f));
    y[2 * i + 1] = rbf_hw((x[2 * i + 1] * inv) * (bf_hi((uint32_t)wraw[i]) + 1.f));
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = normed ? y[e] : x[e];
  // RoPE: lanes j < 4 take x c - x' s, lanes 4 <= j < 8 take x c + x' s (a sign flip is exact)
  const float sg = j < 4 ? -1.f : 1.f;
  const bool rot = normed && j < 8;
  const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float other = xor_swz<4>(y[e]);
    const float r = rbf_hw(y[e] * c[e] + (sg * other) * sn[e]);
    x[e] = rot ? r : y[e];
  }
  const uint4 packed =
      make_uint4(pack_bf2_hw(x[0], x[1]), pack_bf2_hw(x[2], x[3]), pack_bf2_hw(x[4], x[5]), pack_bf2_hw(x[6], x[7]));
  if (qhead) {
    uint16_t* dst = normed ? d.q : d.gate;  // the gate half stores its own values (x = y = the loaded row)
    *reinterpret_cast<uint4*>(dst + ((size_t)t * 16 + h) * 256 + 8 * j) = packed;
  } else {
    const size_t o = ((size_t)t * 2 + hh) * 256 + 8 * j;
    *reinterpret_cast<uint4*>((normed ? d.k : d.v) + o) = packed;
    uint2 e8;
    e8.x = f2e4m3x2_hw(x[0], x[1]) | (f2e4m3x2_hw(x[2], x[3]) << 16);
    e8.y = f2e4m3x2_hw(x[4], x[5]) | (f2e4m3x2_hw(x[6], x[7]) << 16);
    *reinterpret_cast<uint2*>((normed ? d.k8 : d.v8) + o) = e8;
    if (d.out_loc) {
      const int64_t slot = d.out_loc[t];
      if (slot >= 0 && slot < d.num_slots)
        *reinterpret_cast<uint2*>((normed ? d.kc : d.vc) + ((size_t)slot * 2 + hh) * 256 + 8 * j) = e8;
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
  const size_t T16 = (size_t)(T + 15) / 16 * 16;  // fragment order pads the tokens to whole tiles
  w.xq = take(T16 * 2048);
  w.xs = take(sizeof(float) * 16 * T16);
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
  w.as = take(sizeof(float) * (size_t)32 * T);
  w.total = o;
  return w;
}

struct LinWs {
  size_t xq, xs, total;
};
LinWs lin_ws(int T, int K) {
  LinWs w;
  size_t o = 0;
  auto take = [&](size_t b) {
    size_t r = o;
    o = align_up(o + b, 256);
    return r;
  };
  const size_t T16 = (size_t)(T + 15) / 16 * 16;  // fragment order (the tiled GEMM) pads to whole tiles
  w.xq = take(T16 * K);
  w.xs = take(sizeof(float) * (size_t)(K / 128) * T16);
  w.total = o;
  return w;
}

// grid: the row blocks (N / (64 TPW), rounded up to a multiple of the 8 XCDs) x token groups of 16 NTT
template <int NTT, int NKB, int PD, int TPW = 2>
void launch_gemm(const GemmDev& g, hipStream_t st) {
  const int nrb = g.N / (64 * TPW), ntg = (g.T + 16 * NTT - 1) / (16 * NTT);
  proj_gemm_kernel<NTT, NKB, PD, TPW><<<8 * ((nrb + 7) / 8) * ntg, 256, 0, st>>>(g);
}

// grid: the row blocks (N / (16 RT RG), rounded up to a multiple of the 8 XCDs) x token groups of 16 TT
template <int RT, int TT, int KB, int RG, int KS, int DEPTH>
void launch_ks(const GemmDev& g, hipStream_t st) {
  const int nrb = g.N / (16 * RT * RG), ntg = (g.T + 16 * TT - 1) / (16 * TT);
  ks_gemm_kernel<RT, TT, KB, RG, KS, DEPTH><<<8 * ((nrb + 7) / 8) * ntg, 64 * RG * KS, 0, st>>>(g);
}
// token counts from which the projections take the K-sliced GEMM (fragment-order activations)
constexpr int kKsMinT = 32;

// The tiled GEMM past this many tokens, for K = 2048 (its activations in fragment order).  Token
// groups of 64 while the grid stays within one workgroup per CU, else of 128.  Measured (graph-timed
// bench legs and kernel traces): at 256 tokens it takes 18.7 us for the GDN in_proj and the attention
// QKV against 24.1 and 23.2 us for the streaming and K-sliced GEMMs; at 128 tokens 12.4 against
// 11.7 us, and for K = 4096 (2048 rows: 32-64 workgroups) 18.7 against 11.7 us.  Its copies into
// LDS are latency-bound: at most three 24-32 KB steps in flight a CU (the LDS holds four), about 30-45
// GB/s a CU, where the streaming GEMM spreads the same bytes over every CU's waves.
constexpr int kTileMinT = 129;
template <int NKB>
void launch_tile(const GemmDev& g, hipStream_t st) {
  const int nrb = g.N / 128, g64 = (g.T + 63) / 64;
  const int grid64 = 8 * ((nrb + 7) / 8) * g64;
  if (grid64 <= 256 || g.T <= 64)
    tile_gemm_kernel<64, NKB><<<grid64, 512, 0, st>>>(g);
  else
    tile_gemm_kernel<128, NKB><<<8 * ((nrb + 7) / 8) * ((g.T + 127) / 128), 512, 0, st>>>(g);
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
extern "C" int q36_attn_act_frag(int32_t T) { return T >= kKsMinT ? 1 : 0; }
extern "C" size_t q36_oproj_workspace_bytes(int32_t T) { return oproj_ws(T).total; }

extern "C" int q36_attn_proj(const q36_attn_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_attn_proj: null args");
  Q36_REQUIRE(a->T >= 1 && a->T <= 65535, "q36_attn_proj: T=%d out of range", a->T);
  Q36_REQUIRE(a->max_pos >= 1, "q36_attn_proj: max_pos=%d", a->max_pos);
  Q36_REQUIRE((a->x || a->xq) && a->wqkv && a->sqkv && a->q_norm_w && a->k_norm_w && a->cos_sin && a->positions &&
                  a->q && a->gate && a->k && a->v && a->k8 && a->v8 && a->workspace,
              "q36_attn_proj: a required pointer is null");
  Q36_REQUIRE((a->xq == nullptr) == (a->xqs == nullptr), "q36_attn_proj: xq and xqs go together");
  Q36_REQUIRE(aligned16(a->xq) && (reinterpret_cast<uintptr_t>(a->xqs) & 3u) == 0,
              "q36_attn_proj: xq must be 16-byte and xqs 4-byte aligned");
  Q36_REQUIRE(aligned16(a->x) && aligned16(a->wqkv) && aligned16(a->q_norm_w) && aligned16(a->k_norm_w) &&
                  aligned16(a->cos_sin) && aligned16(a->q) && aligned16(a->gate) && aligned16(a->k) &&
                  aligned16(a->v) && (reinterpret_cast<uintptr_t>(a->k8) & 7u) == 0 &&
                  (reinterpret_cast<uintptr_t>(a->v8) & 7u) == 0 &&
                  (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_attn_proj: x, wqkv, the norm weights, cos_sin, q, gate, k, v must be 16-byte, k8 and v8 8-byte "
              "and workspace 256-byte aligned");
  Q36_REQUIRE(!a->out_loc || (a->k_cache && a->v_cache && a->num_slots >= 1 &&
                               a->num_slots * 2 * 256 < ((int64_t)1 << 40) &&
                               (reinterpret_cast<uintptr_t>(a->k_cache) & 7u) == 0 &&
                               (reinterpret_cast<uintptr_t>(a->v_cache) & 7u) == 0),
              "q36_attn_proj: out_loc needs k_cache and v_cache (8-byte aligned) and num_slots >= 1 (got %lld)",
              (long long)a->num_slots);
  const AttnWs L = attn_ws(a->T);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_attn_proj: workspace of %zu bytes < %zu required",
              a->workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(a->workspace);
  const uint8_t* xq = reinterpret_cast<uint8_t*>(ws + L.xq);
  const float* xs = reinterpret_cast<float*>(ws + L.xs);
  uint16_t* qkv = reinterpret_cast<uint16_t*>(ws + L.qkv);
  const bool ks = a->T >= kKsMinT;
  const int Tq = ks ? (a->T + 15) / 16 * 16 : a->T;
  if (a->xq) {  // quantized by the rows' producer, in this entry's layout (q36_attn_act_frag)
    xq = static_cast<const uint8_t*>(a->xq);
    xs = a->xqs;
  } else {
    act_quant_kernel<<<Tq, 256, 0, st>>>(static_cast<const uint16_t*>(a->x), nullptr, a->T, 2048, ks,
                                         reinterpret_cast<uint8_t*>(ws + L.xq), reinterpret_cast<float*>(ws + L.xs));
  }
  const GemmDev g = gemm_dev(xq, xs, a->T, 2048, static_cast<const uint8_t*>(a->wqkv), a->sqkv, 9216, qkv);
  // 144-row x 32-token workgroups, 3 row groups x 4 K quarters (12 waves): 256 workgroups at 128
  // tokens, 17.9 us per graph-timed call against 19.2 us for the streaming GEMM (128 x 32 tiles, 288
  // workgroups).  Both move about 90 MB through L2 per call (the token groups re-read the weights, the
  // row blocks the activations), which at ~18 TB/s across the chip is what bounds them.  (norm_rope
  // fused into the K-sliced GEMM's epilogue, which needs one 256-row head per workgroup: 144
  // workgroups of 256 rows x 32 tokens, or 288 of 16 tokens, measured 14.1-22.1 us for the fused call
  // against 13.4 us for the GEMM and norm_rope at 128 tokens with prequantized rows.)
  if (a->T >= kTileMinT)
    launch_tile<16>(g, st);
  else if (ks)
    launch_ks<3, 2, 4, 3, 4, 2>(g, st);
  else
    launch_gemm<1, 16, 4>(g, st);
  RopeDev r{a->T, a->max_pos, qkv, static_cast<const uint16_t*>(a->q_norm_w),
            static_cast<const uint16_t*>(a->k_norm_w), a->eps, a->cos_sin, a->positions,
            static_cast<uint16_t*>(a->q), static_cast<uint16_t*>(a->gate), static_cast<uint16_t*>(a->k),
            static_cast<uint16_t*>(a->v), static_cast<uint8_t*>(a->k8), static_cast<uint8_t*>(a->v8),
            a->out_loc, static_cast<uint8_t*>(a->k_cache), static_cast<uint8_t*>(a->v_cache), a->num_slots};
  norm_rope_kernel<<<(a->T * kRopeItems + 3) / 4, 256, 0, st>>>(r);
  return check_launch("q36_attn_proj");
}

extern "C" int q36_attn_oproj(const q36_oproj_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_attn_oproj: null args");
  Q36_REQUIRE(a->T >= 1 && a->T <= 65535, "q36_attn_oproj: T=%d out of range", a->T);
  Q36_REQUIRE(((a->attn && a->gate) || a->aq) && a->wo && a->so && a->out && a->workspace,
              "q36_attn_oproj: a required pointer is null");
  Q36_REQUIRE((a->aq == nullptr) == (a->aqs == nullptr), "q36_attn_oproj: aq and aqs go together");
  Q36_REQUIRE(aligned16(a->aq) && (reinterpret_cast<uintptr_t>(a->aqs) & 3u) == 0,
              "q36_attn_oproj: aq must be 16-byte and aqs 4-byte aligned");
  Q36_REQUIRE(aligned16(a->attn) && aligned16(a->gate) && aligned16(a->wo) &&
                  (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_attn_oproj: attn, gate, wo must be 16-byte and workspace 256-byte aligned");
  const OprojWs L = oproj_ws(a->T);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_attn_oproj: workspace of %zu bytes < %zu required",
              a->workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(a->workspace);
  const uint8_t* aq = reinterpret_cast<uint8_t*>(ws + L.aq);
  const float* as = reinterpret_cast<float*>(ws + L.as);
  if (a->aq) {  // quantized by the attention's epilogue (q36_attn_decode's oq / oqs)
    aq = static_cast<const uint8_t*>(a->aq);
    as = a->aqs;
  } else {
    act_quant_kernel<<<a->T, 256, 0, st>>>(static_cast<const uint16_t*>(a->attn),
                                           static_cast<const uint16_t*>(a->gate), a->T, 4096, false,
                                           reinterpret_cast<uint8_t*>(ws + L.aq), reinterpret_cast<float*>(ws + L.as));
  }
  const GemmDev g =
      gemm_dev(aq, as, a->T, 4096, static_cast<const uint8_t*>(a->wo), a->so, 2048, static_cast<uint16_t*>(a->out));
  // 64-row blocks (one 16-row tile per wave), one-tile token groups, 4 stages in flight: 256
  // workgroups at 128 tokens.  Measured at 128 tokens: 6.8 us against 8.1 us for 128-row blocks; the
  // K-sliced GEMM (8 slices of 512, 32 x 32 tiles) 1 us slower per call: with every load of a wave in
  // flight at once the token groups' shared weight lines leave L2 before the last group reads them.
  // Past 128 tokens two-tile token groups keep the grid at one round.
  if (a->T > 128)
    launch_gemm<2, 32, 4, 1>(g, st);
  else
    launch_gemm<1, 32, 4, 1>(g, st);
  return check_launch("q36_attn_oproj");
}

extern "C" size_t q36_fp8_linear_workspace_bytes(int32_t T, int32_t K) { return lin_ws(T, K).total; }
extern "C" int q36_fp8_linear_act_frag(int32_t T, int32_t K) { return T >= kTileMinT && K == 2048 ? 1 : 0; }

extern "C" int q36_fp8_linear(const q36_fp8_linear_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_fp8_linear: null args");
  Q36_REQUIRE(a->T >= 1 && a->T <= 65535, "q36_fp8_linear: T=%d out of range", a->T);
  Q36_REQUIRE(a->K == 2048 || a->K == 4096, "q36_fp8_linear: K=%d unsupported (2048 or 4096)", a->K);
  Q36_REQUIRE(a->N >= 128 && a->N % 128 == 0 && a->N <= (1 << 20), "q36_fp8_linear: N=%d must be a multiple of 128",
              a->N);
  Q36_REQUIRE(a->n_out >= 4 && a->n_out <= a->N && a->n_out % 4 == 0, "q36_fp8_linear: n_out=%d (N=%d)", a->n_out,
              a->N);
  Q36_REQUIRE((a->x || a->xq) && a->w && a->ws && a->workspace, "q36_fp8_linear: a required pointer is null");
  Q36_REQUIRE((a->xq == nullptr) == (a->xqs == nullptr), "q36_fp8_linear: xq and xqs go together");
  Q36_REQUIRE(aligned16(a->xq) && (reinterpret_cast<uintptr_t>(a->xqs) & 3u) == 0,
              "q36_fp8_linear: xq must be 16-byte and xqs 4-byte aligned");
  Q36_REQUIRE(aligned16(a->x) && aligned16(a->w) && (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_fp8_linear: x, w must be 16-byte and workspace 256-byte aligned");
  Q36_REQUIRE(a->nseg >= 1 && a->nseg <= 4 && a->seg[0].col0 == 0, "q36_fp8_linear: nseg=%d, first segment at %d",
              a->nseg, a->seg[0].col0);
  for (int i = 0; i < a->nseg; ++i) {
    const int end = i + 1 < a->nseg ? a->seg[i + 1].col0 : a->n_out;
    Q36_REQUIRE(a->seg[i].out && (reinterpret_cast<uintptr_t>(a->seg[i].out) & 7u) == 0,
                "q36_fp8_linear: segment %d output null or not 8-byte aligned", i);
    Q36_REQUIRE(a->seg[i].col0 % 4 == 0 && end > a->seg[i].col0 && a->seg[i].ld >= end - a->seg[i].col0 &&
                    a->seg[i].ld % 4 == 0,
                "q36_fp8_linear: segment %d columns [%d, %d) with row stride %d", i, a->seg[i].col0, end,
                a->seg[i].ld);
  }
  const LinWs L = lin_ws(a->T, a->K);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_fp8_linear: workspace of %zu bytes < %zu required",
              a->workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(a->workspace);
  const uint8_t* xq = reinterpret_cast<uint8_t*>(ws + L.xq);
  const float* xs = reinterpret_cast<float*>(ws + L.xs);
  const bool tiled = a->T >= kTileMinT && a->K == 2048;
  if (a->xq) {  // quantized by the rows' producer, in this entry's layout (q36_fp8_linear_act_frag)
    xq = static_cast<const uint8_t*>(a->xq);
    xs = a->xqs;
  } else {
    act_quant_kernel<<<tiled ? (a->T + 15) / 16 * 16 : a->T, 256, 0, st>>>(
        static_cast<const uint16_t*>(a->x), nullptr, a->T, a->K, tiled, reinterpret_cast<uint8_t*>(ws + L.xq),
        reinterpret_cast<float*>(ws + L.xs));
  }
  GemmDev g = gemm_dev(xq, xs, a->T, a->K, static_cast<const uint8_t*>(a->w), a->ws, a->N, nullptr);
  g.nseg = a->nseg;
  g.nout = a->n_out;
  for (int i = 0; i < 4; ++i) {
    g.c0[i] = i < a->nseg ? a->seg[i].col0 : a->n_out;
    g.ld[i] = i < a->nseg ? a->seg[i].ld : 0;
    g.ys[i] = i < a->nseg ? static_cast<uint16_t*>(a->seg[i].out) : nullptr;
  }
  if (tiled)
    launch_tile<16>(g, st);
  else if (a->K == 4096 && a->T > 128)
    launch_gemm<2, 32, 4, 1>(g, st);
  else if (a->K == 4096)
    launch_gemm<1, 32, 4, 1>(g, st);
  else if (a->T > 16)
    launch_gemm<2, 16, 2>(g, st);
  else
    launch_gemm<1, 16, 4>(g, st);
  return check_launch("q36_fp8_linear");
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
