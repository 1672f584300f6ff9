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
// One workgroup of 512 threads per (sequence, value head).  Thread (v = tid / 4, c4 = tid % 4)
// holds row v of the 128x128 fp32 state in registers, columns {16 j + 4 c4 + i : j < 8, i < 4}:
// a row dot is 32 local fma plus a two-step quad reduction, a snapshot store writes 64
// contiguous bytes per row per instruction.  The prologue computes the unit's conv outputs
// (q and k of key head hv/2, v of head hv), the norms and the gates into LDS.
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
  __shared__ float gate_g[kTMax], gate_b[kTMax];
  const int unit = blockIdx.x;
  const int bq = unit / GHV, hv = unit % GHV, hk = hv / 2;
  const int T = d.T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = tid >> 2, c4 = tid & 3;

  // conv + SiLU for the unit's 384 channels: q (hk), k (hk), v (hv)
  if (tid < 3 * 128) {
    const int part = tid >> 7, i = tid & 127;
    const int ch = part == 0 ? hk * GK + i : part == 1 ? GHK * GK + hk * GK + i : 2 * GHK * GK + hv * GV + i;
    float w[kTMax + 3];
    const uint16_t* cs = d.conv_state + ((size_t)bq * GQKV + ch) * 3;
    w[0] = bfs(cs);
    w[1] = bfs(cs + 1);
    w[2] = bfs(cs + 2);
#pragma unroll
    for (int t = 0; t < kTMax; ++t)
      w[3 + t] = t < T ? bfs(d.mixed + ((size_t)bq * T + t) * GQKV + ch) : 0.f;
    float cw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) cw[q] = bfs(d.conv_w + (size_t)ch * 4 + q);
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
  }
  // the state row into registers; it lands while the gates and the norms are computed
  const float* s0 = d.S0 + (((size_t)bq * GHV + hv) * GV + row) * GK + 4 * c4;
  v4f st[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) st[j] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(s0 + 16 * j));
  if (tid < T) {
    const size_t r = (size_t)bq * T + tid;
    const float av = bfs(d.a + r * GHV + hv), bv = bfs(d.b + r * GHV + hv);
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

  const size_t snap_stride = (size_t)GHV * GV * GK;  // one position of one sequence
  float* snap = d.snaps + ((((size_t)bq * T) * GHV + hv) * GV + row) * GK + 4 * c4;
  for (int t = 0; t < T; ++t) {
    const float eg = gate_g[t], beta = gate_b[t];
    float kv = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const v4f kk = *reinterpret_cast<const v4f*>(&ks[t][16 * j + 4 * c4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) kv = __builtin_fmaf(st[j][i], kk[i], kv);
    }
    kv = kv + __shfl_xor(kv, 1);
    kv = kv + __shfl_xor(kv, 2);
    const float u = beta * (vs[t][row] - eg * kv);
    float ov = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const v4f kk = *reinterpret_cast<const v4f*>(&ks[t][16 * j + 4 * c4]);
      const v4f qq = *reinterpret_cast<const v4f*>(&qs[t][16 * j + 4 * c4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st[j][i] = __builtin_fmaf(eg, st[j][i], u * kk[i]);
        ov = __builtin_fmaf(st[j][i], qq[i], ov);
      }
      // plain stores: measured 89 us per 32 x 5 step against 128 us with non-temporal ones
      *reinterpret_cast<v4f*>(snap + (size_t)t * snap_stride + 16 * j) = st[j];
    }
    ov = ov + __shfl_xor(ov, 1);
    ov = ov + __shfl_xor(ov, 2);
    if (c4 == 0) os[t][row] = rbf(ov);  // the core output is bf16
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
      const float zz = bfs(d.z + r * GZ + hv * GV + v);
      const float y = ((o * rstd) * bfs(d.norm_w + v)) * (zz * sigmoid_q(zz));
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
