// W8A16 GEMMs for gfx950: int8 weights widened exactly to bf16, bf16 activations, bf16 MFMA with fp32
// accumulation.  Two consumers:
//   - the lm_head at small row counts (the reference's rule below 64 rows: H/lmhead8.py:57-91,
//     171-197; H/node.py:144-151): logit = bf16(acc * ws[row]) with one fp32 scale per vocab row, fused
//     with the greedy argmax (q36_lmhead_argmax, mode Q36_LMH_W8A16);
//   - the DENSE8 decode projections (L/dense8.py:1-28,229-401; the copy q36_quant_dense8 writes):
//     one fp16 scale per (row, 128-column group), acc = fma(group dot, scale, acc) in group order,
//     outputs bf16 split into column segments (q36_dense8_linear).
//
// Layout of the work: a workgroup owns 128 weight rows, each of its four waves 32 (two 16-row MFMA
// tiles), against every token (up to 64: NTT tiles of 16).  K advances 64 columns a step: lane l loads
// 16 int8 of row l % 16 at column 64 s + 16 (l / 16) (four lanes cover 64 contiguous bytes of a row),
// and the 16 bf16 of its token at the same columns; the low and high 8 of each feed two
// v_mfma_f32_16x16x32_bf16 (the same column split on both operands, so every product is formed once).
// int8 -> bf16 is exact: v_cvt_f32_i32 with a sign-extended byte select, then the high half of the f32.
// The weights stream from HBM kDepth steps ahead in registers; the activations (a few hundred KB at
// most) come from L2.  With the weights as the first operand a lane ends with token l % 16 and four
// consecutive rows 4 (l / 16) .. + 3 of each tile.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "q36_device.h"
#include "q36_host.h"
#include "q36_w8a16.h"

namespace q36 {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kRowsWG = 128;   // weight rows per workgroup
constexpr int kDepth = 4;      // weight steps in flight per wave

// 16 int8 (one v4i) -> two fragments of 8 bf16 (low 8 bytes, high 8 bytes)
__device__ __forceinline__ void widen16(v4i w, v8bf& lo, v8bf& hi) {
  uint32_t o[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int x = w[k];
    const float f0 = (float)(signed char)(x), f1 = (float)(signed char)(x >> 8);
    const float f2 = (float)(signed char)(x >> 16), f3 = (float)(x >> 24);
    o[2 * k] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    o[2 * k + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  }
  const v4i l4 = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]}, h4 = {(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
  lo = __builtin_bit_cast(v8bf, l4);
  hi = __builtin_bit_cast(v8bf, h4);
}

__device__ __forceinline__ v4f mfma_bf16(v8bf a, v8bf b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// x rounded to bf16, as the float it represents (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ float round_bf16_w(float x) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(float, __builtin_convertvector((v2f){0.f, x}, v2bf));
}

template <int NTT, int MODE>
__global__ __launch_bounds__(256) void w8a16_kernel(W16Dev d) {
  __shared__ uint32_t rkey[4][64];  // MODE 0: each wave's best key per token
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int r0 = blockIdx.x * kRowsWG + wave * 32;  // the wave's rows (N % 32 == 0: all in or all out)
  const bool active = r0 < d.N;
  const int K = d.K, nsteps = K / 64;
  // weights: row r0 + 16 rt + lr, bytes 64 s + 16 lg of it
  const int8_t* wrow = d.q + (size_t)(active ? r0 : 0) * K;
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)wrow, (short)0, active ? 32 * K : 0, 0x00020000);
  const int wv0 = lr * K + 16 * lg, wv1 = (16 + lr) * K + 16 * lg;
  // activations: token 16 tt + lr (rows past T read as zero), elements 64 s + 16 lg .. + 15
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)d.x, (short)0, d.T * K * 2, 0x00020000);
  int xv[NTT];
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) {
    const int t = 16 * tt + lr;
    xv[tt] = t < d.T ? (t * K + 16 * lg) * 2 : d.T * K * 2;
  }
  v4f acc[2][NTT], part[2][NTT];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) acc[rt][tt] = part[rt][tt] = v4f{0.f, 0.f, 0.f, 0.f};
  v4i wq[kDepth][2];
  if (active) {
#pragma unroll
    for (int s = 0; s < kDepth; ++s) {
      wq[s][0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wv0, 64 * s, 2);
      wq[s][1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wv1, 64 * s, 2);
    }
    for (int s0 = 0; s0 < nsteps; s0 += kDepth) {
#pragma unroll
      for (int u = 0; u < kDepth; ++u) {
        const int s = s0 + u;
        v4i xa[NTT], xb[NTT];
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
          xa[tt] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xv[tt], 128 * s, 0);
          xb[tt] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xv[tt], 128 * s + 16, 0);
        }
        v8bf alo[2], ahi[2];
        widen16(wq[u][0], alo[0], ahi[0]);
        widen16(wq[u][1], alo[1], ahi[1]);
        if (s + kDepth < nsteps) {
          wq[u][0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wv0, 64 * (s + kDepth), 2);
          wq[u][1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wv1, 64 * (s + kDepth), 2);
        }
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
          const v8bf blo = __builtin_bit_cast(v8bf, xa[tt]), bhi = __builtin_bit_cast(v8bf, xb[tt]);
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            v4f& p = MODE == 0 ? acc[rt][tt] : part[rt][tt];
            p = mfma_bf16(alo[rt], blo, p);
            p = mfma_bf16(ahi[rt], bhi, p);
          }
        }
        if constexpr (MODE == 1) {
          // the end of a 128-column group: acc = fma(group dot, s16[group][row], acc), group dot reset
          if (s & 1) {
            const int g = s >> 1;
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              const uint2 sv = *reinterpret_cast<const uint2*>(d.s16 + (size_t)g * d.s_ld + r0 + 16 * rt + 4 * lg);
              const float sc[4] = {__half2float(__ushort_as_half((unsigned short)(sv.x & 0xffffu))),
                                   __half2float(__ushort_as_half((unsigned short)(sv.x >> 16))),
                                   __half2float(__ushort_as_half((unsigned short)(sv.y & 0xffffu))),
                                   __half2float(__ushort_as_half((unsigned short)(sv.y >> 16)))};
#pragma unroll
              for (int tt = 0; tt < NTT; ++tt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[rt][tt][i] = __builtin_fmaf(part[rt][tt][i], sc[i], acc[rt][tt][i]);
                part[rt][tt] = v4f{0.f, 0.f, 0.f, 0.f};
              }
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  if constexpr (MODE == 0) {
    // logit = bf16(acc * ws[row]); the first row of each token's largest logit in this workgroup
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      const int t = 16 * tt + lr;
      float bv = -__builtin_inff();
      int bi = 0;
      if (active) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int rb = r0 + 16 * rt + 4 * lg;
          const float4 w4 = *reinterpret_cast<const float4*>(d.ws + rb);
          const float wsv[4] = {w4.x, w4.y, w4.z, w4.w};
          float lg4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            lg4[i] = round_bf16_w(acc[rt][tt][i] * wsv[i]);
            if (lg4[i] > bv) bv = lg4[i], bi = rb + i - blockIdx.x * kRowsWG;
          }
          if (d.logits && t < d.T)
            *reinterpret_cast<uint2*>(d.logits + (size_t)t * d.N + rb) =
                make_uint2((__float_as_uint(lg4[0]) >> 16) | (__float_as_uint(lg4[1]) & 0xffff0000u),
                           (__float_as_uint(lg4[2]) >> 16) | (__float_as_uint(lg4[3]) & 0xffff0000u));
        }
      }
      // order-preserving bf16 key, first row on ties (the larger 0xffff - row)
      uint32_t b16 = __float_as_uint(bv + 0.f) >> 16;
      b16 = (b16 & 0x8000u) ? (~b16 & 0xffffu) : (b16 | 0x8000u);
      uint32_t key = active ? ((b16 << 16) | (0xffffu - (uint32_t)bi)) : 0u;
      key = max(key, (uint32_t)__shfl_xor((int)key, 16));
      key = max(key, (uint32_t)__shfl_xor((int)key, 32));
      if (lg == 0) rkey[wave][16 * tt + lr] = key;
    }
    __syncthreads();
    if (tid < 16 * NTT && tid < d.T) {
      const uint32_t k = max(max(rkey[0][tid], rkey[1][tid]), max(rkey[2][tid], rkey[3][tid]));
      if (k != 0u) {
        const uint32_t row = (uint32_t)(blockIdx.x * kRowsWG) + (0xffffu - (k & 0xffffu));
        atomicMax(&d.keys[tid], ((unsigned long long)(k >> 16) << 32) | (unsigned long long)(0xffffffffu - row));
      }
    }
  } else {
    if (!active) return;
    // column segments (four columns never straddle a boundary: the boundaries are multiples of 4)
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      const int t = 16 * tt + lr;
      if (t >= d.T) continue;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int col = r0 + 16 * rt + 4 * lg;
        if (col >= d.nout) continue;
        const int sg = (d.nseg > 1 && col >= d.c0[1]) + (d.nseg > 2 && col >= d.c0[2]) + (d.nseg > 3 && col >= d.c0[3]);
        *reinterpret_cast<uint2*>(d.ys[sg] + (size_t)t * d.ld[sg] + (col - d.c0[sg])) =
            make_uint2(pack_bf2(acc[rt][tt][0], acc[rt][tt][1]), pack_bf2(acc[rt][tt][2], acc[rt][tt][3]));
      }
    }
  }
}

template <int MODE>
int launch_ntt(const W16Dev& d, hipStream_t st) {
  const int grid = (d.N + kRowsWG - 1) / kRowsWG;
  if (d.T <= 16)
    w8a16_kernel<1, MODE><<<grid, 256, 0, st>>>(d);
  else if (d.T <= 32)
    w8a16_kernel<2, MODE><<<grid, 256, 0, st>>>(d);
  else
    w8a16_kernel<4, MODE><<<grid, 256, 0, st>>>(d);
  return Q36_OK;
}

}  // namespace

int launch_w8a16(const W16Dev& d, int mode, hipStream_t st) {
  return mode == 0 ? launch_ntt<0>(d, st) : launch_ntt<1>(d, st);
}

}  // namespace q36

using namespace q36;

extern "C" int q36_dense8_linear(const q36_dense8_linear_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_dense8_linear: null args");
  Q36_REQUIRE(a->T >= 1 && a->T <= 64, "q36_dense8_linear: T=%d must be in [1, 64]", a->T);
  Q36_REQUIRE(a->K >= 256 && a->K % 256 == 0 && a->K <= 8192, "q36_dense8_linear: K=%d must be a multiple of 256",
              a->K);
  Q36_REQUIRE(a->N >= 32 && a->N % 32 == 0 && a->N <= (1 << 20), "q36_dense8_linear: N=%d must be a multiple of 32",
              a->N);
  Q36_REQUIRE(a->n_out >= 4 && a->n_out <= a->N && a->n_out % 4 == 0, "q36_dense8_linear: n_out=%d (N=%d)",
              a->n_out, a->N);
  Q36_REQUIRE(a->x && a->q && a->s, "q36_dense8_linear: a required pointer is null");
  Q36_REQUIRE(a->s_ld >= a->N && a->s_ld % 4 == 0, "q36_dense8_linear: s_ld=%lld must be >= N and a multiple of 4",
              (long long)a->s_ld);
  Q36_REQUIRE(aligned16(a->x) && aligned16(a->q) && (reinterpret_cast<uintptr_t>(a->s) & 7u) == 0,
              "q36_dense8_linear: x, q must be 16-byte and s 8-byte aligned");
  Q36_REQUIRE(a->nseg >= 1 && a->nseg <= 4 && a->seg[0].col0 == 0, "q36_dense8_linear: nseg=%d, first segment at %d",
              a->nseg, a->seg[0].col0);
  for (int i = 0; i < a->nseg; ++i) {
    const int end = i + 1 < a->nseg ? a->seg[i + 1].col0 : a->n_out;
    Q36_REQUIRE(a->seg[i].out && (reinterpret_cast<uintptr_t>(a->seg[i].out) & 7u) == 0,
                "q36_dense8_linear: segment %d output null or not 8-byte aligned", i);
    Q36_REQUIRE(a->seg[i].col0 % 4 == 0 && end > a->seg[i].col0 && a->seg[i].ld >= end - a->seg[i].col0 &&
                    a->seg[i].ld % 4 == 0,
                "q36_dense8_linear: segment %d columns [%d, %d) with row stride %d", i, a->seg[i].col0, end,
                a->seg[i].ld);
  }
  W16Dev d{};
  d.T = a->T;
  d.N = a->N;
  d.K = a->K;
  d.x = static_cast<const uint16_t*>(a->x);
  d.q = static_cast<const int8_t*>(a->q);
  d.s16 = static_cast<const uint16_t*>(a->s);
  d.s_ld = a->s_ld;
  d.nseg = a->nseg;
  d.nout = a->n_out;
  for (int i = 0; i < 4; ++i) {
    d.c0[i] = i < a->nseg ? a->seg[i].col0 : a->n_out;
    d.ld[i] = i < a->nseg ? a->seg[i].ld : 0;
    d.ys[i] = i < a->nseg ? static_cast<uint16_t*>(a->seg[i].out) : nullptr;
  }
  launch_w8a16(d, 1, static_cast<hipStream_t>(stream));
  return check_launch("q36_dense8_linear");
}
