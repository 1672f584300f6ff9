// Prepare-time weight quantizers for gfx950: per-row int8 (the reference's quantize_rows rule) and
// e4m3 with one fp32 scale per 128x128 block.  Both logits-processor and decoder-layer nodes use them
// to build their weight copies once, outside the decode step.
//
// Reference behaviour (R = qwen36_nodes_kb34, H = R/qwen36_lmhead8):
//   per-row int8   H/lmhead8.py:95-108 (_quant_rows_kernel), torch form :129-143: scale = amax / 127,
//                  codes = round-half-away(w / scale) clamped to +-127, scale 0 (codes 0) for a zero row
//   e4m3 blocks    no reference counterpart (the configuration's fp8 format): scale = amax / 448 per
//                  128x128 block, codes = e4m3 RNE satfinite of w * (448 / amax)
#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {
// ------------------------------------------------------------------------------------------
// prepare-time quantizers
// ------------------------------------------------------------------------------------------
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
      for (int b = 0; b < 4; b += 2) wd[i] |= f2e4m3x2_hw(v[16 * c + 4 * i + b] * inv, v[16 * c + 4 * i + b + 1] * inv) << (8 * b);
    }
    *reinterpret_cast<uint4*>(dst + 16 * c) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }
  if (tid == 0) s[(size_t)nb * nkb + kb] = sc;
}
}  // namespace
}  // namespace q36

using namespace q36;

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
