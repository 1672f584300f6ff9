// The reference's prepare-time int8 weight formats, written and read on gfx950.
//
//   q8-block-v1 (R = qwen36_nodes_kb34, L = R/qwen36_layer; L/i8x_kernels.py:12,69-141): per routed
//     expert one block [q13 int8 (2I x H) | q2 int8 (H x I) | c13 fp16 (2I x H/128) | c2 fp16 (H x I/128)]
//   DENSE8 (L/dense8.py:1-9,140-188): q int8 [N, K] and fp16 scales stored group-major [K/128][ld]
//
// Both quantize a row (or a 128-group) with s16 = fp16(fp32(amax / 127) * (1 + 2^-10)) -- one fp16
// ulp of headroom so the largest element never clamps -- and q = clamp(round_half_away(w / s16), +-127).
// A channel-mode q8-block-v1 copy writes each row's one scale into all of its group slots.
//
// quant_f16rows_kernel: one wave per row, a lane holds 8 consecutive elements of each 512-column chunk,
// so a 128-group is the 16 lanes of one DPP row: the group max is four row-local DPP steps, the row max
// two more readlane steps.  import_q8v1_kernel repacks a channel-mode copy into the decode MoE's int8
// experts: codes in MFMA fragment order (q36_pack_frag8's order), scales widened to fp32.
#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

// One segment of rows to quantize: row r of expert e = r / rows_pe reads src + r * K and writes its codes
// at q + e * q_es + (r % rows_pe) * K and its scale for group g at s + e * s_es + (r % rows_pe) * s_rs + g * s_gs
// (bytes for q / s offsets).
struct RowSeg {
  const uint16_t* src;
  uint8_t* q;
  uint8_t* s;
  int64_t rows, rows_pe, q_es, s_es, s_rs, s_gs;
  int K;
};
struct QuantDev {
  RowSeg seg[2];
  int nseg, channel;
};

__device__ __forceinline__ uint32_t f2h_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);  // IEEE round to nearest even
}
__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// fp16 scale of a row / group with maximum magnitude amax, and the divisor for its codes
__device__ __forceinline__ uint32_t scale16(float amax) { return f2h_bits((amax / 127.f) * 1.0009765625f); }

__global__ __launch_bounds__(256) void quant_f16rows_kernel(QuantDev d) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int sg = (d.nseg > 1 && row >= d.seg[0].rows) ? 1 : 0;
  const RowSeg& S = d.seg[sg];
  const int64_t r = sg ? row - d.seg[0].rows : row;
  if (r >= S.rows) return;  // the last workgroup's spare waves
  const int64_t e = r / S.rows_pe, rr = r % S.rows_pe;
  const int K = S.K, nch = K >> 9;  // 512-column chunks (K <= 4096)
  const uint16_t* src = S.src + r * K;
  v4i raw[8];
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if (c < nch) {
      raw[c] = *reinterpret_cast<const v4i*>(src + c * 512 + lane * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        amax = fmaxf(amax, fmaxf(fabsf(bf_lo((uint32_t)raw[c][j])), fabsf(bf_hi((uint32_t)raw[c][j]))));
    }
  }
  uint8_t* q = S.q + e * S.q_es + rr * K;
  uint8_t* s = S.s + e * S.s_es + rr * S.s_rs;
  if (d.channel) {
    const float m = __uint_as_float(wave_max_u32(__float_as_uint(amax)));  // non-negative: integer order
    const uint32_t s16 = scale16(m);
    const float sc = h2f(s16), safe = sc > 0.f ? sc : 1.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (c < nch) {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t a = (uint32_t)round_i8(bf_lo((uint32_t)raw[c][j]) / safe) & 0xffu;
          const uint32_t b = (uint32_t)round_i8(bf_hi((uint32_t)raw[c][j]) / safe) & 0xffu;
          const uint32_t pair = a | (b << 8);
          if (j < 2) w0 |= pair << (16 * j);
          else w1 |= pair << (16 * (j - 2));
        }
        *reinterpret_cast<v2i*>(q + c * 512 + lane * 8) = v2i{(int)w0, (int)w1};
      }
    }
    if (lane < (K >> 7)) *reinterpret_cast<uint16_t*>(s + lane * S.s_gs) = (uint16_t)s16;
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (c < nch) {
        float ga = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          ga = fmaxf(ga, fmaxf(fabsf(bf_lo((uint32_t)raw[c][j])), fabsf(bf_hi((uint32_t)raw[c][j]))));
        const float m = __uint_as_float(row16_max_u32(__float_as_uint(ga)));  // the 16 lanes of a 128-group
        const uint32_t s16 = scale16(m);
        const float sc = h2f(s16), safe = sc > 0.f ? sc : 1.f;
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t a = (uint32_t)round_i8(bf_lo((uint32_t)raw[c][j]) / safe) & 0xffu;
          const uint32_t b = (uint32_t)round_i8(bf_hi((uint32_t)raw[c][j]) / safe) & 0xffu;
          const uint32_t pair = a | (b << 8);
          if (j < 2) w0 |= pair << (16 * j);
          else w1 |= pair << (16 * (j - 2));
        }
        *reinterpret_cast<v2i*>(q + c * 512 + lane * 8) = v2i{(int)w0, (int)w1};
        if ((lane & 15) == 0) *reinterpret_cast<uint16_t*>(s + (c * 4 + (lane >> 4)) * S.s_gs) = (uint16_t)s16;
      }
    }
  }
}

// q8-block-v1 copy -> the decode MoE's int8 experts.  Output chunk i (16 bytes) of a fragment-ordered
// array of N = E * rows_pe rows and K columns: lane l = i % 64, half h = (i / 64) % 2, 16-row tile and
// 128-column block from i / 128 (the order of q36_pack_frag8); its source is the block's row-major codes.
struct ImportDev {
  const uint8_t* blocks;
  int64_t eb;              // block bytes
  int E, H, I;
  uint8_t* w13;            // [E * 2I, H] fragment order
  uint8_t* w2;             // [E * H, I] fragment order
  float* s13;              // [E, 2I]
  float* s2;               // [E, H]
};

__global__ __launch_bounds__(256) void import_q8v1_kernel(ImportDev d) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n13 = (int64_t)d.E * 2 * d.I * d.H / 16, n2 = (int64_t)d.E * d.H * d.I / 16;
  const int64_t ns13 = (int64_t)d.E * 2 * d.I, ns2 = (int64_t)d.E * d.H;
  const int64_t o2 = (int64_t)2 * d.I * d.H, oc13 = o2 + (int64_t)d.H * d.I, oc2 = oc13 + (int64_t)2 * d.I * (d.H / 128) * 2;
  if (i < n13 + n2) {
    const bool second = i >= n13;
    const int64_t j = second ? i - n13 : i;
    const int K = second ? d.I : d.H, rows_pe = second ? d.H : 2 * d.I;
    const int l = (int)(j & 63), h = (int)((j >> 6) & 1);
    const int64_t frag = j >> 7;
    const int nkb = K >> 7;
    const int64_t tile = frag / nkb;
    const int kb = (int)(frag % nkb);
    const int64_t row = tile * 16 + (l & 15), e = row / rows_pe, rr = row % rows_pe;
    const uint8_t* src = d.blocks + e * d.eb + (second ? o2 : 0) + rr * K + kb * 128 + (l >> 4) * 32 + h * 16;
    *reinterpret_cast<v4i*>((second ? d.w2 : d.w13) + j * 16) = *reinterpret_cast<const v4i*>(src);
    return;
  }
  const int64_t k = i - n13 - n2;  // a scale: the row's first group slot (a channel copy holds one per row)
  if (k < ns13) {
    const int64_t e = k / (2 * d.I), rr = k % (2 * d.I);
    d.s13[k] = h2f(*reinterpret_cast<const uint16_t*>(d.blocks + e * d.eb + oc13 + rr * (d.H / 128) * 2));
  } else if (k < ns13 + ns2) {
    const int64_t m = k - ns13, e = m / d.H, rr = m % d.H;
    d.s2[m] = h2f(*reinterpret_cast<const uint16_t*>(d.blocks + e * d.eb + oc2 + rr * (d.I / 128) * 2));
  }
}

int64_t q8v1_block_bytes(int H, int I) {
  return (int64_t)2 * I * H + (int64_t)H * I + (int64_t)2 * I * (H / 128) * 2 + (int64_t)H * (I / 128) * 2;
}

int launch_quant(const QuantDev& d, int64_t rows, hipStream_t st, const char* what) {
  const int64_t wgs = (rows + 3) / 4;
  Q36_REQUIRE(wgs <= 0x7fffffff, "%s: %lld rows exceed one launch", what, (long long)rows);
  quant_f16rows_kernel<<<(unsigned)wgs, 256, 0, st>>>(d);
  return check_launch(what);
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" size_t q36_q8_block_v1_bytes(int32_t H, int32_t I) {
  return (H > 0 && I > 0) ? (size_t)q8v1_block_bytes(H, I) : 0;
}

extern "C" int q36_quant_q8_block_v1(const void* w13, const void* w2, int32_t E, int32_t H, int32_t I, int32_t channel,
                                     void* blocks, q36_stream_t stream) {
  Q36_REQUIRE(w13 && w2 && blocks, "q36_quant_q8_block_v1: null pointer");
  Q36_REQUIRE(E >= 1 && H >= 512 && I >= 512 && H <= 4096 && I <= 4096 && H % 512 == 0 && I % 512 == 0,
              "q36_quant_q8_block_v1: E=%d H=%d I=%d (H, I multiples of 512 up to 4096)", E, H, I);
  Q36_REQUIRE(aligned16(w13) && aligned16(w2) && aligned16(blocks), "q36_quant_q8_block_v1: pointers must be 16-byte aligned");
  const int64_t eb = q8v1_block_bytes(H, I), o2 = (int64_t)2 * I * H, oc13 = o2 + (int64_t)H * I,
                oc2 = oc13 + (int64_t)2 * I * (H / 128) * 2;
  uint8_t* b = static_cast<uint8_t*>(blocks);
  QuantDev d{};
  d.nseg = 2;
  d.channel = channel ? 1 : 0;
  d.seg[0] = RowSeg{static_cast<const uint16_t*>(w13), b, b + oc13, (int64_t)E * 2 * I, 2 * I, eb, eb, (H / 128) * 2, 2, H};
  d.seg[1] = RowSeg{static_cast<const uint16_t*>(w2), b + o2, b + oc2, (int64_t)E * H, H, eb, eb, (I / 128) * 2, 2, I};
  return launch_quant(d, (int64_t)E * (2 * I + H), static_cast<hipStream_t>(stream), "q36_quant_q8_block_v1");
}

extern "C" int q36_quant_dense8(const void* w, int64_t N, int32_t K, void* q, void* s, int64_t s_ld,
                                q36_stream_t stream) {
  Q36_REQUIRE(w && q && s, "q36_quant_dense8: null pointer");
  Q36_REQUIRE(N >= 1 && K >= 512 && K <= 4096 && K % 512 == 0, "q36_quant_dense8: N=%lld K=%d (K a multiple of 512 up to 4096)",
              (long long)N, K);
  Q36_REQUIRE(s_ld >= N, "q36_quant_dense8: scale row stride %lld < N=%lld", (long long)s_ld, (long long)N);
  Q36_REQUIRE(aligned16(w) && aligned16(q) && (reinterpret_cast<uintptr_t>(s) & 1) == 0,
              "q36_quant_dense8: w, q 16-byte and s 2-byte aligned");
  QuantDev d{};
  d.nseg = 1;
  d.channel = 0;
  // group g of row n at s[g * s_ld + n]: row step 2 bytes, group step 2 * s_ld bytes
  d.seg[0] = RowSeg{static_cast<const uint16_t*>(w), static_cast<uint8_t*>(q), static_cast<uint8_t*>(s), N, N, 0, 0, 2,
                    2 * s_ld, K};
  return launch_quant(d, N, static_cast<hipStream_t>(stream), "q36_quant_dense8");
}

extern "C" int q36_import_q8_block_v1(const void* blocks, int32_t E, int32_t H, int32_t I, void* w13, float* s13, void* w2,
                                      float* s2, q36_stream_t stream) {
  Q36_REQUIRE(blocks && w13 && s13 && w2 && s2, "q36_import_q8_block_v1: null pointer");
  Q36_REQUIRE(E >= 1 && H >= 512 && I >= 512 && H <= 4096 && I <= 4096 && H % 512 == 0 && I % 512 == 0,
              "q36_import_q8_block_v1: E=%d H=%d I=%d (H, I multiples of 512 up to 4096)", E, H, I);
  Q36_REQUIRE(aligned16(blocks) && aligned16(w13) && aligned16(w2), "q36_import_q8_block_v1: blocks, w13, w2 16-byte aligned");
  ImportDev d{static_cast<const uint8_t*>(blocks), q8v1_block_bytes(H, I), E, H, I, static_cast<uint8_t*>(w13),
              static_cast<uint8_t*>(w2), s13, s2};
  const int64_t total = (int64_t)E * 3 * I * H / 16 + (int64_t)E * (2 * I + H);
  const int64_t wgs = (total + 255) / 256;
  Q36_REQUIRE(wgs <= 0x7fffffff, "q36_import_q8_block_v1: too large for one launch");
  import_q8v1_kernel<<<(unsigned)wgs, 256, 0, static_cast<hipStream_t>(stream)>>>(d);
  return check_launch("q36_import_q8_block_v1");
}
