// Fused residual add + Gemma RMSNorm for gfx950 (the add-norm between the hybrid layer's blocks).
//
// Reference behaviour (L = qwen36_nodes_kb34/qwen36_layer): L/proj.py:60-81 (_add_norm_kernel):
// z = bf16(projection) + residual in fp32, residual <- bf16(z), y = bf16(z * rsqrt(mean z^2 + eps)
// * (1 + w)).  Here the sum of squares runs in one fixed order (lane l of a wave owns the 8-element
// chunks l + 64 j, fma from zero, then an xor butterfly 32..1) so that the CPU oracle gives the
// same bits, and rsqrt is the correctly rounded 1 / sqrt.
//
// Kernel: one wave per row, one row per workgroup (a workgroup per row spreads a decode batch's
// few hundred rows over as many CUs); a row is 2048 bf16 = 4 chunks of 8 per lane.
// Optionally the normed row also leaves as e4m3 codes per 128-channel group (the next projection's
// input, so that projection skips its own quantization launch): a group is 16 neighbouring lanes.
#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int kNH = 2048, kNJ = kNH / 512;

struct NormDev {
  int T;
  const uint16_t* delta;
  uint16_t* residual;
  const uint16_t* w;
  float eps;
  uint16_t* out;
  uint8_t* q8;   // e4m3 codes of out (fragment order when frag), or null
  float* q8s;    // [tokens, 16] group scales
  int frag;
};

__global__ __launch_bounds__(64) void add_rmsnorm_kernel(NormDev d) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = blockIdx.x * (blockDim.x >> 6) + wave;
  if (r >= d.T) {
    // fragment order pads the tokens to a multiple of 16: zero codes and scales
    if (d.q8 && d.frag && r < (d.T + 15) / 16 * 16) {
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        const int c = lane + 64 * j;
        *reinterpret_cast<uint2*>(d.q8 + frag_offset(r, 8 * c, kNH)) = make_uint2(0u, 0u);
        if ((c & 15) == 0) d.q8s[(size_t)r * (kNH / 128) + c / 16] = 0.f;
      }
    }
    return;
  }
  float z[kNJ][8];
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const size_t at = (size_t)r * kNH + 8 * (lane + 64 * j);
    const v4i rv = *reinterpret_cast<const v4i*>(d.residual + at);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      z[j][2 * q] = bf_lo((uint32_t)rv[q]);
      z[j][2 * q + 1] = bf_hi((uint32_t)rv[q]);
    }
    if (d.delta) {
      const v4i dv = *reinterpret_cast<const v4i*>(d.delta + at);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        z[j][2 * q] = bf_lo((uint32_t)dv[q]) + z[j][2 * q];
        z[j][2 * q + 1] = bf_hi((uint32_t)dv[q]) + z[j][2 * q + 1];
      }
      v4i nv;
#pragma unroll
      for (int q = 0; q < 4; ++q) nv[q] = (int)pack_bf2(z[j][2 * q], z[j][2 * q + 1]);
      *reinterpret_cast<v4i*>(d.residual + at) = nv;
    }
  }
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < kNJ; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(z[j][i], z[j][i], acc);
  const float ss = wave_sum_bfly(acc);
  const float rstd = 1.f / sqrtf(ss / (float)kNH + d.eps);
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const v4i wv = *reinterpret_cast<const v4i*>(d.w + 8 * (lane + 64 * j));
    v4i ov;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      ov[q] = (int)pack_bf2((z[j][2 * q] * rstd) * (1.f + bf_lo((uint32_t)wv[q])),
                            (z[j][2 * q + 1] * rstd) * (1.f + bf_hi((uint32_t)wv[q])));
    *reinterpret_cast<v4i*>(d.out + (size_t)r * kNH + 8 * (lane + 64 * j)) = ov;
    if (d.q8) {
      // the bf16 outputs' e4m3 codes: the same arithmetic as the projections' own quantization
      const int c = lane + 64 * j;
      float f[8];
      float m = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f[2 * q] = bf_lo((uint32_t)ov[q]);
        f[2 * q + 1] = bf_hi((uint32_t)ov[q]);
        m = fmaxf(m, fmaxf(fabsf(f[2 * q]), fabsf(f[2 * q + 1])));
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
      const float inv = m > 0.f ? 448.f / m : 0.f;
      *reinterpret_cast<uint2*>(d.q8 + (d.frag ? frag_offset(r, 8 * c, kNH) : (size_t)r * kNH + 8 * c)) =
          e4m3_run8(f, inv);
      if ((c & 15) == 0) d.q8s[(size_t)r * (kNH / 128) + c / 16] = m / 448.f;
    }
  }
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" int q36_add_rmsnorm(const q36_add_norm_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_add_rmsnorm: null args");
  Q36_REQUIRE(a->H == kNH, "q36_add_rmsnorm: H=%d unsupported (this build: 2048)", a->H);
  Q36_REQUIRE(a->T >= 1 && a->T <= (1 << 24), "q36_add_rmsnorm: T=%d out of range", a->T);
  Q36_REQUIRE(a->residual && a->norm_w && a->out, "q36_add_rmsnorm: a required pointer is null");
  Q36_REQUIRE(aligned16(a->residual) && aligned16(a->norm_w) && aligned16(a->out) && (!a->delta || aligned16(a->delta)),
              "q36_add_rmsnorm: pointers must be 16-byte aligned");
  Q36_REQUIRE((a->q8 == nullptr) == (a->q8s == nullptr), "q36_add_rmsnorm: q8 and q8s go together");
  Q36_REQUIRE(!a->q8 || ((reinterpret_cast<uintptr_t>(a->q8) & 7u) == 0 && (reinterpret_cast<uintptr_t>(a->q8s) & 3u) == 0),
              "q36_add_rmsnorm: q8 must be 8-byte and q8s 4-byte aligned");
  NormDev d{a->T, static_cast<const uint16_t*>(a->delta), static_cast<uint16_t*>(a->residual),
            static_cast<const uint16_t*>(a->norm_w), a->eps, static_cast<uint16_t*>(a->out),
            static_cast<uint8_t*>(a->q8), a->q8s, a->q8_frag != 0};
  const int rows = a->q8 && a->q8_frag ? (a->T + 15) / 16 * 16 : a->T;
  add_rmsnorm_kernel<<<rows, 64, 0, static_cast<hipStream_t>(stream)>>>(d);
  return check_launch("q36_add_rmsnorm");
}
