// W8A16 GEMMs for gfx950: int8 weights widened exactly to bf16, bf16 activations, bf16 MFMA with fp32
// accumulation.  Two consumers:
//   - the lm_head at small row counts (the reference's rule below 64 rows: H/lmhead8.py:57-91,
//     171-197; H/node.py:144-151): logit = bf16(acc * ws[row]) with one fp32 scale per vocab row, fused
//     with the greedy argmax (q36_lmhead_argmax, mode Q36_LMH_W8A16);
//   - the DENSE8 decode projections (L/dense8.py:1-28,229-401; the copy q36_quant_dense8 writes):
//     one fp16 scale per (row, 128-column group), acc = fma(group dot, scale, acc) in group order
//     within a K chunk, the chunks' sums added in order, outputs bf16 split into column segments
//     (q36_dense8_linear).
//
// Layout of the work: a wave owns 16 RT weight rows (RT 16-row MFMA tiles) over a chunk of K, against
// every token (up to 64: NTT tiles of 16).  K advances 64 columns a step: lane l loads
// 16 int8 of row l % 16 at column 64 s + 16 (l / 16) (four lanes cover 64 contiguous bytes of a row),
// and the 16 bf16 of its token at the same columns; the low and high 8 of each feed two
// v_mfma_f32_16x16x32_bf16 (the same column split on both operands, so every product is formed once).
// int8 -> bf16 is exact: v_cvt_f32_i32 with a sign-extended byte select, then the high half of the f32.
// The weights stream from HBM kDepth steps ahead in registers, the activations (a few hundred KB at
// most, read from L2) with them.  With the weights as the first operand a lane ends with token l % 16 and four
// consecutive rows 4 (l / 16) .. + 3 of each tile.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "q36_device.h"
#include "q36_host.h"
#include "q36_w8a16.h"

namespace q36 {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

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


// One workgroup: WAVES waves in RG = WAVES / KS row groups of 16 RT rows; the KS waves of a row group
// split K into KS contiguous chunks (a multiple of 128 columns each) and their fp32 partial sums meet in
// LDS, added in chunk order by the first wave of the group, which runs the epilogue.
template <int NTT, int RT, int KS, int WAVES, int MODE, int K>
__global__ __launch_bounds__(64 * WAVES) void w8a16_kernel(W16Dev d) {
  constexpr int RG = WAVES / KS;
  constexpr int RW = 16 * RT;      // rows per wave
  // steps in flight: weights, activations (and mode 1's group scales); four token tiles hold half as many
  constexpr int D = NTT >= 4 || RT >= 8 ? kDepth / 2 : kDepth;
  constexpr int NACC = RT * NTT * 4;
  __shared__ float red[KS > 1 ? WAVES - RG : 1][KS > 1 ? NACC : 1][KS > 1 ? 64 : 1];
  __shared__ uint32_t rkey[MODE == 0 ? RG : 1][64];
  // the wave index through readfirstlane: uniform to the compiler, so the buffer descriptors built from
  // it live in SGPRs (a descriptor in VGPRs turns every buffer load into a readfirstlane loop)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lr = lane & 15,
            lg = lane >> 4;
  const int ks = wave % KS, rg = wave / KS;
  const int r0 = blockIdx.x * (RG * RW) + rg * RW;  // N % RW == 0: a wave's rows are all in or all out
  const bool active = r0 < d.N;
  // K is a template argument so the step loop unrolls completely: with a loop edge the compiler waits for
  // every outstanding load at the top of each pass, which caps the loads in flight at one pass
  constexpr int kc = K / KS, nsteps = kc / 64;
  const int k0 = ks * kc;
  // weights: row r0 + 16 rt + lr, bytes k0 + 64 s + 16 lg .. + 15 of it
  const int8_t* wrow = d.q + (size_t)(active ? r0 : 0) * K;
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)wrow, (short)0, active ? RW * K : 0, 0x00020000);
  // row-major: lane (lr, lg) reads row lr at columns 64 s + 16 lg (an instruction spans 16 rows); tiled:
  // the same 16 bytes at 16 lane of the step's 1 KB piece (an instruction reads 1 KB contiguous)
  const int tiled = d.tiled, sstep = tiled ? 1024 : 64;
  int wv[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    wv[rt] = tiled ? 16 * rt * K + (k0 >> 6) * 1024 + 16 * lane : (16 * rt + lr) * K + k0 + 16 * lg;
  // activations: token 16 tt + lr (tokens past T read as zero), elements k0 + 64 s + 16 lg .. + 15
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)d.x, (short)0, d.T * K * 2, 0x00020000);
  int xv[NTT];
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) {
    const int t = 16 * tt + lr;
    xv[tt] = t < d.T ? (t * K + k0 + 16 * lg) * 2 : d.T * K * 2;
  }
  v4f acc[RT][NTT], part[RT][NTT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) acc[rt][tt] = part[rt][tt] = v4f{0.f, 0.f, 0.f, 0.f};
  if (active) {
    v4i wq[D][RT], xa[D][NTT], xb[D][NTT];
    uint2 scl[D / 2][RT];  // mode 1: the fp16 scales of the group starting at an even step
    // Loads are issued without a branch (a conditional load makes the compiler wait for every
    // outstanding load at the join): a step past the chunk gets a VGPR offset past both descriptors'
    // ranges, which returns zeros and moves no data.  The out-of-range amount rides in the VGPR offset
    // because only that one is range-checked; the SGPR offset carries in-range step offsets only.
    // (nsteps is a compile-time constant and the step loop unrolls, so `in` folds away per step.)
    auto issue = [&](int u, int s) {
      const bool in = s < nsteps;
      const int wo = in ? sstep * s : 0, xo = in ? 128 * s : 0, oob = in ? 0 : (1 << 30);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) wq[u][rt] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wv[rt] + oob, wo, 2);
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) {
        xa[u][tt] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xv[tt] + oob, xo, 0);
        xb[u][tt] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xv[tt] + oob, xo + 16, 0);
      }
      if constexpr (MODE == 1) {
        if (!(u & 1)) {
          const int g = (k0 >> 7) + (min(s, nsteps - 2) >> 1);  // past the chunk: its last group again
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            scl[u >> 1][rt] = *reinterpret_cast<const uint2*>(d.s16 + (size_t)g * d.s_ld + r0 + 16 * rt + 4 * lg);
        }
      }
    };
#pragma unroll
    for (int u = 0; u < D; ++u) issue(u, u);
    uint2 sc_cur[RT];  // mode 1: the current group's scales, taken at its first step before the refill
#pragma unroll
    for (int s0 = 0; s0 < nsteps; s0 += D) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const int s = s0 + u;
        v8bf alo[RT], ahi[RT], blo[NTT], bhi[NTT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) widen16(wq[u][rt], alo[rt], ahi[rt]);
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
          blo[tt] = __builtin_bit_cast(v8bf, xa[u][tt]);
          bhi[tt] = __builtin_bit_cast(v8bf, xb[u][tt]);
        }
        if constexpr (MODE == 1) {
          if (!(u & 1)) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) sc_cur[rt] = scl[u >> 1][rt];
          }
        }
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            v4f& p = MODE == 0 ? acc[rt][tt] : part[rt][tt];
            p = mfma_bf16(alo[rt], blo[tt], p);
            p = mfma_bf16(ahi[rt], bhi[tt], p);
          }
        // the refill after the last read of the slot's registers, so the loads land in the same
        // registers every iteration (no copies at the loop edge, which would wait for them)
        issue(u, s + D);
        if constexpr (MODE == 1) {
          // the end of a 128-column group: acc = fma(group dot, s16[group][row], acc), group dot reset
          if (u & 1) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
              const float sc[4] = {__half2float(__ushort_as_half((unsigned short)(sc_cur[rt].x & 0xffffu))),
                                   __half2float(__ushort_as_half((unsigned short)(sc_cur[rt].x >> 16))),
                                   __half2float(__ushort_as_half((unsigned short)(sc_cur[rt].y & 0xffffu))),
                                   __half2float(__ushort_as_half((unsigned short)(sc_cur[rt].y >> 16)))};
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
  if constexpr (KS > 1) {
    // partial sums of the later K chunks through LDS, added in chunk order
    if (ks > 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) red[rg * (KS - 1) + ks - 1][(rt * NTT + tt) * 4 + i][lane] = acc[rt][tt][i];
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int j = 0; j < KS - 1; ++j)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[rt][tt][i] += red[rg * (KS - 1) + j][(rt * NTT + tt) * 4 + i][lane];
    }
  }
  const bool owner = active && ks == 0;  // the wave that finishes its row group
  if constexpr (MODE == 0) {
    // logit = bf16(acc * ws[row]); the first row of each token's largest logit in this workgroup
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      const int t = 16 * tt + lr;
      float bv = -__builtin_inff();
      int bi = 0;
      if (owner) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const int rb = r0 + 16 * rt + 4 * lg;
          const float4 w4 = *reinterpret_cast<const float4*>(d.ws + rb);
          const float wsv[4] = {w4.x, w4.y, w4.z, w4.w};
          float lg4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            lg4[i] = rbf_hw(acc[rt][tt][i] * wsv[i]);
            if (lg4[i] > bv) bv = lg4[i], bi = rb + i - blockIdx.x * (RG * RW);
          }
          if (d.logits && t < d.T)
            *reinterpret_cast<uint2*>(d.logits + (size_t)t * d.N + rb) =
                make_uint2((__float_as_uint(lg4[0]) >> 16) | (__float_as_uint(lg4[1]) & 0xffff0000u),
                           (__float_as_uint(lg4[2]) >> 16) | (__float_as_uint(lg4[3]) & 0xffff0000u));
          if (d.logits32 && t < d.T)
            *reinterpret_cast<float4*>(d.logits32 + (size_t)t * d.N + rb) = make_float4(lg4[0], lg4[1], lg4[2], lg4[3]);
        }
      }
      // order-preserving bf16 key, first row on ties (the larger 0xffff - row)
      uint32_t b16 = __float_as_uint(bv + 0.f) >> 16;
      b16 = (b16 & 0x8000u) ? (~b16 & 0xffffu) : (b16 | 0x8000u);
      uint32_t key = owner ? ((b16 << 16) | (0xffffu - (uint32_t)bi)) : 0u;
      key = max(key, (uint32_t)__shfl_xor((int)key, 16));
      key = max(key, (uint32_t)__shfl_xor((int)key, 32));
      if (ks == 0 && lg == 0) rkey[rg][16 * tt + lr] = key;
    }
    __syncthreads();
    if (tid < 16 * NTT && tid < d.T) {
      uint32_t k = rkey[0][tid];
#pragma unroll
      for (int j = 1; j < RG; ++j) k = max(k, rkey[j][tid]);
      if (k != 0u) {
        const uint32_t row = (uint32_t)(blockIdx.x * (RG * RW)) + (0xffffu - (k & 0xffffu));
        atomicMax(&d.keys[tid], ((unsigned long long)(k >> 16) << 32) | (unsigned long long)(0xffffffffu - row));
      }
    }
  } else {
    if (!owner) return;
    // column segments (four columns never straddle a boundary: the boundaries are multiples of 4)
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      const int t = 16 * tt + lr;
      if (t >= d.T) continue;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int col = r0 + 16 * rt + 4 * lg;
        if (col >= d.nout) continue;
        const int sg = (d.nseg > 1 && col >= d.c0[1]) + (d.nseg > 2 && col >= d.c0[2]) + (d.nseg > 3 && col >= d.c0[3]);
        *reinterpret_cast<uint2*>(d.ys[sg] + (size_t)t * d.ld[sg] + (col - d.c0[sg])) =
            make_uint2(pack_bf2(acc[rt][tt][0], acc[rt][tt][1]), pack_bf2(acc[rt][tt][2], acc[rt][tt][3]));
      }
    }
  }
}

// The launch shape: token tiles NTT (T <= 16 NTT), row tiles per wave RT, K split KS, waves per
// workgroup WAVES.  Every shape the policy can pick is instantiated here.
#define Q36_W16_SHAPES_0(X) X(1, 2, 1, 4) X(1, 4, 1, 2) X(2, 2, 1, 4) X(2, 4, 1, 2) X(2, 8, 1, 2) X(4, 2, 1, 4) X(4, 4, 1, 2)
#define Q36_W16_SHAPES_1(X) \
  X(1, 2, 4, 8) X(2, 2, 4, 8) X(4, 2, 4, 8) \
  X(1, 1, 8, 8) X(2, 1, 8, 8) X(4, 1, 8, 8)

struct W16Shape {
  int ntt, rt, ks, waves;
};

// Measured on MI355X (the lm_head, N = 151936, codes in the tile order, graph-timed): the lm_head
// streams whole rows, 32 a wave in four-wave workgroups up to 8 tokens (61 us; 64-row waves 63 us,
// too few loads in flight); from 9 tokens on the activation fragments each wave reads from L2 weigh
// more, so wider waves serve more weight rows with each: 64 rows a wave in two-wave workgroups up to
// 24 tokens (16: 62.7 against 66.1 us), 128 rows from 25 to 32 tokens (32: 73.6 against 78.0 us), and
// 64 rows with four token tiles (48: 99 against 138 us for 32-row waves, 63: 112 against 160 us).
// The projections split K so that every CU has waves: in quarters for the 9216- and 12352-row
// in_proj / qkv, in eighths for the 2048-row o_proj / out_proj.
W16Shape w16_shape(const W16Dev& d, int mode) {
  const int ntt = d.T <= 16 ? 1 : d.T <= 32 ? 2 : 4;
  // (a wave's rows are all in or all out: 64-row waves need N % 64 == 0, 128-row waves N % 128 == 0)
  if (mode == 0) {
    if (d.T <= 8 || d.N % 64 != 0) return W16Shape{ntt, 2, 1, 4};
    if (ntt == 2 && d.T > 24 && d.N % 128 == 0) return W16Shape{ntt, 8, 1, 2};
    return W16Shape{ntt, 4, 1, 2};
  }
  return d.N >= 8192 ? W16Shape{ntt, 2, 4, 8} : W16Shape{ntt, 1, 8, 8};
}

template <int NTT, int RT, int KS, int WAVES, int MODE>
void launch_shape(const W16Dev& d, hipStream_t st) {
  constexpr int rows_wg = (WAVES / KS) * 16 * RT;
  const int grid = (d.N + rows_wg - 1) / rows_wg;
  if constexpr (MODE == 1) {
    if (d.K == 4096) {
      w8a16_kernel<NTT, RT, KS, WAVES, MODE, 4096><<<grid, 64 * WAVES, 0, st>>>(d);
      return;
    }
  }
  w8a16_kernel<NTT, RT, KS, WAVES, MODE, 2048><<<grid, 64 * WAVES, 0, st>>>(d);
}

template <int MODE>
int launch_mode(const W16Dev& d, hipStream_t st) {
  const W16Shape s = w16_shape(d, MODE);
#define Q36_W16_CASE(NTT, RT, KS, W)                                              \
  if (s.ntt == NTT && s.rt == RT && s.ks == KS && s.waves == W) {                 \
    launch_shape<NTT, RT, KS, W, MODE>(d, st);                                    \
    return Q36_OK;                                                                \
  }
  if constexpr (MODE == 0) {
    Q36_W16_SHAPES_0(Q36_W16_CASE)
  } else {
    Q36_W16_SHAPES_1(Q36_W16_CASE)
  }
#undef Q36_W16_CASE
  return Q36_EINVAL;
}

}  // namespace

int launch_w8a16(const W16Dev& d, int mode, hipStream_t st) {
  return mode == 0 ? launch_mode<0>(d, st) : launch_mode<1>(d, st);
}

}  // namespace q36

using namespace q36;

namespace q36 {
namespace {
// Row-major int8 [N, K] -> the tile order: one thread per 16-byte piece of the output.
__global__ __launch_bounds__(256) void tile_w16_kernel(const int8_t* q, int64_t N, int K, int8_t* out) {
  const int64_t o = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
  if (o >= N * K) return;
  const int64_t piece = o >> 10;            // (row tile, column step)
  const int l = (int)((o & 1023) >> 4);     // 16-byte lane of the piece
  const int64_t tile = piece / (K >> 6);
  const int step = (int)(piece % (K >> 6));
  const int64_t row = tile * 16 + (l & 15);
  const int col = step * 64 + 16 * (l >> 4);
  *reinterpret_cast<v4i*>(out + o) = *reinterpret_cast<const v4i*>(q + row * K + col);
}
}  // namespace
}  // namespace q36

extern "C" int q36_tile_w16(const void* q, int64_t N, int32_t K, void* tiled, q36_stream_t stream) {
  Q36_REQUIRE(q && tiled, "q36_tile_w16: null pointer");
  Q36_REQUIRE(N >= 16 && N % 16 == 0 && K >= 64 && K % 64 == 0 && N * (int64_t)K < ((int64_t)1 << 40),
              "q36_tile_w16: N=%lld K=%d must be multiples of 16 and 64", (long long)N, K);
  Q36_REQUIRE(aligned16(q) && aligned16(tiled) && q != tiled, "q36_tile_w16: 16-byte aligned, distinct buffers");
  const int64_t pieces = N * K / 16;
  tile_w16_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const int8_t*>(q), N, K, static_cast<int8_t*>(tiled));
  return check_launch("q36_tile_w16");
}

extern "C" int q36_dense8_linear(const q36_dense8_linear_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_dense8_linear: null args");
  Q36_REQUIRE(a->T >= 1 && a->T <= 64, "q36_dense8_linear: T=%d must be in [1, 64]", a->T);
  Q36_REQUIRE(a->K == 2048 || a->K == 4096, "q36_dense8_linear: K=%d must be 2048 or 4096 (the model's widths)",
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
  d.tiled = a->tiled != 0;
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
