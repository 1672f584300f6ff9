// GDN (gated delta net) speculative-verify step for gfx950: causal conv1d + SiLU, q/k L2 norm,
// gates, the gated delta-rule recurrence over the T draft positions with the per-position fp32
// state snapshots, and the gated RMSNorm of the output.
//
// Reference behaviour (R = qwen36_nodes_kb34, L = R/qwen36_layer): L/qk_gdn_verify.cu:293-794
//   conv (:238-247), q/k norm (:575-581), gates (:616-622), recurrence (:684-762, the WY form of
//   S_t = e^{g_t} S_{t-1} + beta_t (v_t - e^{g_t} S_{t-1} k_t) k_t^T, o_t = S_t q_t), output norm
//   (:786-791); value head hv reads key head hv / 2 (:9-11,520).  The reference keeps a replay
//   ring for rollback; this node writes every position's state instead.
//
// One workgroup of 512 threads per (sequence, value head).  Thread (r = tid / 8, c8 = tid % 8)
// holds rows r and r + 64 of the 128x128 fp32 state in registers, columns
// {32 jj + 4 c8 + i : jj < 4, i < 4} of each: a row dot is 16 local fma plus a three-step
// reduction over the row's 8 threads, and a snapshot store writes whole 128-byte lines (8 rows x
// 128 contiguous bytes per instruction).  The prologue requests the conv inputs, the output
// gate z and the gate inputs, then the state rows (half before the conv, half after); it computes
// the unit's conv outputs (q and k of key head hv/2, v of head hv), the norms and the gates into
// LDS while the state arrives.
#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int GK = 128, GV = 128, GHK = 16, GHV = 32, GQKV = 8192, GZ = GHV * GV;
constexpr int kTMax = 8;

struct GdnDev {
  int B, T;
  const uint16_t* mixed;
  const uint16_t* z;
  const uint16_t* a;
  const uint16_t* b;
  const uint16_t* conv_state;
  uint16_t* conv_state_out;
  const uint16_t* conv_w;
  const float* A_log;
  const float* dt_bias;
  const float* S0;
  const uint16_t* norm_w;
  float eps;
  uint16_t* out;
  float* snaps;
};

__device__ __forceinline__ float bfs(const uint16_t* p) { return bf2f(*p); }

// 8 waves per SIMD: the 1024 workgroups of a 32-sequence step are resident in one round.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(8, 8))) void gdn_verify_kernel(GdnDev d) {
  __shared__ float qs[kTMax][GK], ks[kTMax][GK], vs[kTMax][GV];
  __shared__ float os[kTMax][GV];
  __shared__ float zs[kTMax][GV], nws[GV];  // the output gate's z and the norm weight, prefetched
  __shared__ float gate_g[kTMax], gate_b[kTMax];
  const int unit = blockIdx.x;
  const int bq = unit / GHV, hv = unit % GHV, hk = hv / 2;
  const int T = d.T;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r0 = tid >> 3, c8 = tid & 7;
  // state register j (< 8): row r0 + 64 (j / 4), columns 32 (j % 4) + 4 c8 .. +3
  auto soff = [&](int j) { return (r0 + 64 * (j >> 2)) * GK + 32 * (j & 3) + 4 * c8; };

  // Requests first, in this order: the conv inputs (threads < 384), the output gate z and the norm
  // weight (threads >= 384), the gate inputs, then the 64 KB of state rows.  Loads complete in
  // issue order, so the conv and the prefetch wait only for their own data while the state is in
  // flight.
  const int part = tid >> 7, i = tid & 127;  // conv channel (part < 3) or value channel (part 3)
  const int ch = part == 0 ? hk * GK + i : part == 1 ? GHK * GK + hk * GK + i : 2 * GHK * GK + hv * GV + i;
  float w[kTMax + 3], cw[4];
  v4i zr = {0, 0, 0, 0};
  float nwv = 0.f;
  if (part < 3) {
    const uint16_t* cs = d.conv_state + ((size_t)bq * GQKV + ch) * 3;
    w[0] = bfs(cs);
    w[1] = bfs(cs + 1);
    w[2] = bfs(cs + 2);
#pragma unroll
    for (int t = 0; t < kTMax; ++t)
      w[3 + t] = t < T ? bfs(d.mixed + ((size_t)bq * T + t) * GQKV + ch) : 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) cw[q] = bfs(d.conv_w + (size_t)ch * 4 + q);
  } else {
    // z of the unit's positions: thread i < 16 T loads 8 values of position i / 16
    if (i < 16 * T)
      zr = *reinterpret_cast<const v4i*>(d.z + ((size_t)bq * T + (i >> 4)) * GZ + hv * GV + (i & 15) * 8);
    nwv = bfs(d.norm_w + i);
  }
  float av = 0.f, bv = 0.f;
  if (tid < T) {
    const size_t r = (size_t)bq * T + tid;
    av = bfs(d.a + r * GHV + hv);
    bv = bfs(d.b + r * GHV + hv);
  }
  const float* s0 = d.S0 + ((size_t)bq * GHV + hv) * GV * GK;
  v4f st[8];
  // half of the state before the conv and half after it (all of it at once would not fit the
  // 64 registers of eight waves per SIMD beside the conv's inputs)
#pragma unroll
  for (int j = 0; j < 4; ++j) st[j] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(s0 + soff(j)));

  if (part < 3) {
    // conv + SiLU for the unit's 384 channels: q (hk), k (hk), v (hv)
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
      if (t < T) {
        float acc = rbf(w[t] * cw[0]);
        acc = acc + rbf(w[t + 1] * cw[1]);
        acc = acc + rbf(w[t + 2] * cw[2]);
        acc = acc + rbf(w[t + 3] * cw[3]);
        const float o = rbf(acc / (1.f + expf_q(-acc)));
        if (part == 0) qs[t][i] = o;
        else if (part == 1) ks[t][i] = o;
        else vs[t][i] = o;
      }
    }
    // the rolled state: the last three inputs (q/k channels written by the even value head only)
    if (part == 2 || (hv & 1) == 0) {
      uint16_t* co = d.conv_state_out + ((size_t)bq * GQKV + ch) * 3;
#pragma unroll
      for (int q = 0; q < 3; ++q) co[q] = (uint16_t)f2bf(w[T + q]);
    }
  } else {
    if (i < 16 * T) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        zs[i >> 4][(i & 15) * 8 + 2 * q] = bf_lo((uint32_t)zr[q]);
        zs[i >> 4][(i & 15) * 8 + 2 * q + 1] = bf_hi((uint32_t)zr[q]);
      }
    }
    nws[i] = nwv;
  }
#pragma unroll
  for (int j = 4; j < 8; ++j) st[j] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(s0 + soff(j)));
  if (tid < T) {
    const float xg = av + d.dt_bias[hv];
    const float sp = xg <= 20.f ? logf(1.f + expf_q(xg)) : xg;
    gate_g[tid] = expf_q(-expf_q(d.A_log[hv]) * sp);  // e^{g}
    gate_b[tid] = sigmoid_q(bv);
  }
  __syncthreads();
  // q, k L2 norms: wave w handles (t, q|k) pairs w, w + 8
  for (int p = wave; p < 2 * T; p += 8) {
    const int t = p >> 1;
    float* x = (p & 1) ? ks[t] : qs[t];
    const float a0 = x[lane], a1 = x[lane + 64];
    const float ss = wave_sum_bfly(a0 * a0 + a1 * a1);
    float r = 1.f / sqrtf(ss + 1e-6f);
    if (!(p & 1)) r = r * (1.f / sqrtf((float)GK));
    x[lane] = a0 * r;
    x[lane + 64] = a1 * r;
  }
  __syncthreads();

  // snapshot stores through a buffer resource: the lane's offset in one register, the position's
  // block and the register's row/column step (the same for every lane) in the scalar offset, so no
  // store needs an address register of its own: the recurrence fits the 64 registers of eight
  // waves per SIMD
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(  // the sequence's T x 2 MB
      d.snaps + (size_t)__builtin_amdgcn_readfirstlane(bq * T) * GHV * GV * GK, (short)0,
      __builtin_amdgcn_readfirstlane(T * GHV * GV * GK * 4), 0x00020000);
  const int slane = soff(0) * 4;
  for (int t = 0; t < T; ++t) {
    const float eg = gate_g[t], beta = gate_b[t];
    float kv[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const v4f kk = *reinterpret_cast<const v4f*>(&ks[t][32 * (j & 3) + 4 * c8]);
#pragma unroll
      for (int i = 0; i < 4; ++i) kv[j >> 2] = __builtin_fmaf(st[j][i], kk[i], kv[j >> 2]);
    }
    float u[2], ov[2] = {0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      kv[h] = kv[h] + lane_xor<1>(kv[h]);  // DPP / swizzle moves: the __shfl_xor pairs without LDS
      kv[h] = kv[h] + lane_xor<2>(kv[h]);
      kv[h] = kv[h] + lane_xor<4>(kv[h]);
      u[h] = beta * (vs[t][r0 + 64 * h] - eg * kv[h]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const v4f kk = *reinterpret_cast<const v4f*>(&ks[t][32 * (j & 3) + 4 * c8]);
      const v4f qq = *reinterpret_cast<const v4f*>(&qs[t][32 * (j & 3) + 4 * c8]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st[j][i] = __builtin_fmaf(eg, st[j][i], u[j >> 2] * kk[i]);
        ov[j >> 2] = __builtin_fmaf(st[j][i], qq[i], ov[j >> 2]);
      }
      // plain stores: measured 89 us per 32 x 5 step against 128 us with non-temporal ones
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, st[j]), srs, slane,
                                             (t * GHV + hv) * (GV * GK * 4) + ((j >> 2) * 64 * GK + (j & 3) * 32) * 4, 0);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      ov[h] = ov[h] + lane_xor<1>(ov[h]);
      ov[h] = ov[h] + lane_xor<2>(ov[h]);
      ov[h] = ov[h] + lane_xor<4>(ov[h]);
      if (c8 == 0) os[t][r0 + 64 * h] = rbf(ov[h]);  // the core output is bf16
    }
  }
  __syncthreads();
  // gated RMSNorm per position: y = bf16(((o * rstd) * w) * (z * sigmoid(z)))
  for (int t = wave; t < T; t += 8) {
    const float o0 = os[t][lane], o1 = os[t][lane + 64];
    const float ss = wave_sum_bfly(o0 * o0 + o1 * o1);
    const float rstd = 1.f / sqrtf(ss / (float)GV + d.eps);
    const size_t r = (size_t)bq * T + t;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int v = lane + 64 * h;
      const float o = h ? o1 : o0;
      const float zz = zs[t][v];
      const float y = ((o * rstd) * nws[v]) * (zz * sigmoid_q(zz));
      d.out[r * GZ + hv * GV + v] = (uint16_t)f2bf(y);
    }
  }
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" int q36_gdn_verify(const q36_gdn_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_gdn_verify: null args");
  Q36_REQUIRE(a->B >= 1 && a->B <= 65535, "q36_gdn_verify: B=%d out of range", a->B);
  Q36_REQUIRE(a->T >= 1 && a->T <= kTMax, "q36_gdn_verify: T=%d must be in [1,%d]", a->T, kTMax);
  Q36_REQUIRE(a->mixed && a->z && a->a && a->b && a->conv_state && a->conv_state_out && a->conv_w && a->A_log &&
                  a->dt_bias && a->S0 && a->norm_w && a->out && a->snaps,
              "q36_gdn_verify: a required pointer is null");
  Q36_REQUIRE(a->conv_state_out != a->conv_state, "q36_gdn_verify: conv_state_out must not alias conv_state");
  Q36_REQUIRE(aligned16(a->S0) && aligned16(a->snaps), "q36_gdn_verify: S0 and snaps must be 16-byte aligned");
  GdnDev d{a->B, a->T,
           static_cast<const uint16_t*>(a->mixed), static_cast<const uint16_t*>(a->z),
           static_cast<const uint16_t*>(a->a), static_cast<const uint16_t*>(a->b),
           static_cast<const uint16_t*>(a->conv_state), static_cast<uint16_t*>(a->conv_state_out),
           static_cast<const uint16_t*>(a->conv_w), a->A_log, a->dt_bias, a->S0,
           static_cast<const uint16_t*>(a->norm_w), a->eps, static_cast<uint16_t*>(a->out), a->snaps};
  gdn_verify_kernel<<<a->B * GHV, 512, 0, static_cast<hipStream_t>(stream)>>>(d);
  return check_launch("q36_gdn_verify");
}
