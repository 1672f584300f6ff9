// Device-side primitives shared by the q36 kernels (gfx950, wave64).
//
// Every floating-point step that decides a bit of an integer output (expert ids, quantized
// activations, argmax ids) is spelled as an explicit IEEE operation: the library is compiled with
// -ffp-contract=off, fused multiply-adds are written as __builtin_fmaf, and divisions are the
// correctly rounded '/' (hipcc's default).  The same steps on the host give the same bits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q36 {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// One 16-byte global load.
__device__ __forceinline__ v4i ldg16(const uint8_t* p) { return *reinterpret_cast<const v4i*>(p); }
__device__ __forceinline__ float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// float -> bf16 bits, round to nearest even (NaN kept quiet, sign and high payload kept).  Both
// results are computed and one selected: written as an early return for NaN, the compiler emitted a
// divergent branch (exec-mask save and restore) around every rounding.
__device__ __forceinline__ uint32_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t q = (u >> 16) | 0x40u;
  return (u & 0x7fffffffu) > 0x7f800000u ? q : r;
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
// The same rounding for finite values by one v_cvt_pk_bf16_f32 (round to nearest even); NaN becomes
// the canonical quiet NaN.  rbf_hw: the rounded value as the float it represents; pack_bf2_hw: two
// values packed, lo in bits 0..15.
typedef float q36_v2f __attribute__((ext_vector_type(2)));
typedef __bf16 q36_v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float rbf_hw(float x) {
  return __builtin_bit_cast(float, __builtin_convertvector((q36_v2f){0.f, x}, q36_v2bf));
}
__device__ __forceinline__ uint32_t pack_bf2_hw(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((q36_v2f){lo, hi}, q36_v2bf));
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }

// float -> OCP e4m3fn code: round to nearest even, saturate to +-448, NaN -> 0x7f.
__device__ __forceinline__ uint32_t f2e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  float af = __uint_as_float(a);
  if (af >= 448.f) return sign | 0x7eu;
  if (af < 0.015625f) return sign | (uint32_t)__builtin_rintf(af * 512.f);
  int e = (int)((a >> 23) & 0xffu) - 127;
  uint32_t keep = (a & 0x7fffffu) >> 20, rest = a & 0xfffffu;
  if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) keep++;
  if (keep == 8u) { keep = 0; e++; }
  if (e > 8 || (e == 8 && keep > 6u)) return sign | 0x7eu;
  return sign | ((uint32_t)(e + 7) << 3) | keep;
}
// Two floats -> two e4m3fn codes (low 16 bits of the result) with the gfx950 conversion
// instruction on inputs clamped to +-448.  For finite inputs this equals f2e4m3 bit for bit
// (checked on the GPU over 1e7 inputs including every tie and saturation edge).
__device__ __forceinline__ uint32_t f2e4m3x2_hw(float a, float b) {
  a = fminf(fmaxf(a, -448.f), 448.f);
  b = fminf(fmaxf(b, -448.f), 448.f);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}
__device__ __forceinline__ float e4m3_to_f(uint32_t b) {
  uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float v;
  if (e == 15u && m == 7u) v = __builtin_nanf("");
  else if (e == 0u) v = __builtin_ldexpf((float)m, -9);
  else v = __builtin_ldexpf(1.f + (float)m * 0.125f, (int)e - 7);
  return (b & 0x80u) ? -v : v;
}

// exp(x): Cody-Waite reduction with ln2 split hi/lo, degree-7 Taylor polynomial by Horner fma,
// ldexp.  All steps correctly rounded, so host and device agree bit for bit.  Branch-free: the
// overflow / underflow / NaN cases are selected at the end (the main path stays finite for them).
__device__ __forceinline__ float expf_q(float x) {
  const float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.428606765330187e-06f, r);
  float p = 1.f / 5040.f;
  p = __builtin_fmaf(p, r, 1.f / 720.f);
  p = __builtin_fmaf(p, r, 1.f / 120.f);
  p = __builtin_fmaf(p, r, 1.f / 24.f);
  p = __builtin_fmaf(p, r, 1.f / 6.f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.f);
  p = __builtin_fmaf(p, r, 1.f);
  const int ni = (int)fminf(fmaxf(n, -200.f), 200.f);
  float res = __builtin_ldexpf(p, ni);
  res = x > 88.7228394f ? __builtin_inff() : res;
  res = x < -103.972084f ? 0.f : res;
  return x != x ? x : res;
}
__device__ __forceinline__ float sigmoid_q(float z) { return 1.f / (1.f + expf_q(-z)); }

// xor-butterfly over the 64 lanes (offsets 32 .. 1): every lane ends with the same total.
// v of lane l ^ M within each 32-lane half (ds_swizzle bit mode: and 0x1f, xor M), M < 32
template <int M>
__device__ __forceinline__ float xor_swz(float v) {
  static_assert(M > 0 && M < 32, "xor mask within 32 lanes");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (M << 10)));
}
// v of lane l ^ O, O < 16, without LDS: DPP row_ror:8 (within a 16-lane row lane i + 8 mod 16 is
// lane i ^ 8), ds_swizzle xor 4, DPP quad_perm xor 2 / xor 1
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(O == 8 || O == 4 || O == 2 || O == 1, "xor offset below 16");
  if constexpr (O == 8) return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
  else if constexpr (O == 4) return xor_swz<4>(v);
  else if constexpr (O == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
  else return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
}
// The xor butterfly over the 64 lanes without LDS round trips: stage o combines v(l) with v(l ^ o),
// o = 32, 16, 8, 4, 2, 1, exactly as a __shfl_xor butterfly does (the same pairs in the same stage
// order, so the same bits for a commutative op), through v_permlane32_swap / v_permlane16_swap (the
// swapped pair's two halves are v(l) and v(l ^ o) in some order), DPP row_ror:8 (within a 16-lane
// row, lane i + 8 mod 16 is lane i ^ 8), ds_swizzle xor 4 and DPP quad_perm xor 2 / xor 1.
template <typename Op>
__device__ __forceinline__ float wave_bfly(float v, Op op) {
  const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
  const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false)));  // xor 8
  v = op(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (4 << 10))));         // xor 4
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false)));   // xor 2
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false)));   // xor 1
  return v;
}
__device__ __forceinline__ float wave_sum_bfly(float v) {
  return wave_bfly(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_bfly(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

// Row-local DPP move (no LDS): quad_perm / row_mirror patterns.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
// Unsigned max over the wave: xor 1, xor 2 (quad_perm), half-row and row mirrors (the mirrors pair
// lanes holding already-reduced quads / half-rows), then the rows through v_permlane16_swap and
// v_permlane32_swap (VALU only: no readlane, whose SGPR results the next VALU use waits for).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  const auto p16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((uint32_t)p16[0], (uint32_t)p16[1]);
  const auto p32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((uint32_t)p32[0], (uint32_t)p32[1]);
}

// Unsigned max over each row of 16 lanes (every lane of the row gets the row's maximum).
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  return v;
}

// Byte offset of element (token t, channel k) of e4m3 activations [T, K] in MFMA fragment order
// (the operand layout the projection GEMMs read): token tile t / 16 and 128-block kb at
// ((t / 16) * K / 128 + kb) * 2048, byte j of the block at (j % 32) / 16 * 1024 +
// 16 * (t % 16 + 16 * (j / 32)) + j % 16 -- the 32 bytes lane t % 16 + 16 (j / 32) feeds the MFMA,
// as two 16-byte halves 1 KB apart.  8-byte runs k .. k + 7 (k % 8 == 0) stay contiguous.
__host__ __device__ __forceinline__ size_t frag_offset(int t, int k, int K) {
  const int kb = k >> 7, j = k & 127;
  return ((size_t)(t >> 4) * (K >> 7) + kb) * 2048 + ((j & 31) >> 4) * 1024 + 16 * ((t & 15) + 16 * (j >> 5)) + (j & 15);
}

// e4m3 codes of 8 values (one 8-byte run) of a 128-channel group quantized with inverse scale inv
// (448 / group amax, 0 for an all-zero group), round to nearest even with saturation.
__device__ __forceinline__ uint2 e4m3_run8(const float* f, float inv) {
  uint32_t wd[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; i += 2) wd[i >> 2] |= f2e4m3x2_hw(f[i] * inv, f[i + 1] * inv) << (8 * (i & 3));
  return make_uint2(wd[0], wd[1]);
}

// Round half away from zero and clamp to +-127 (the int8 activation / weight rule).
__device__ __forceinline__ int round_i8(float v) {
  float r = v >= 0.f ? __builtin_floorf(v + 0.5f) : -__builtin_floorf(0.5f - v);
  r = fminf(fmaxf(r, -127.f), 127.f);
  return (int)r;
}

}  // namespace q36
