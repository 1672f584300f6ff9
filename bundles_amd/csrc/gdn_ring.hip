// GDN speculative verify over the ReplaySSM ring for gfx950: the served form of the recurrent
// block's verify step, where the rollback state is a read-only fp32 checkpoint h0 plus a 16-entry
// circular ring of (d, k, g) entries instead of per-position state snapshots.
//
// Reference behaviour (R = qwen36_nodes_kb34, L = R/qwen36_layer): L/qk_gdn_verify.cu:1-20 (design),
//   conv window record and roll (:277-291, :607-613), q/k L2 norm (:575-581), gates and the g ring
//   (:616-632), history decay (:634-648), ring keys (:583-605), the window recurrence (:684-762) and
//   the d ring appends (:770-781), output norm (:786-791); host checks :850-919.  The state the
//   window starts from is S = td h0 + sum_c decay_c dhat_c khat_c^T over the n committed entries
//   (bf16 high parts), decay_c = exp(g_{c+1} + .. + g_{n-1}), td = exp(g_0 + .. + g_{n-1}).
//
// One 512-thread workgroup per (request, key head): it owns both value heads of the key head, so
// the q/k conv runs once and the conv state rolls in place with no other workgroup reading it.
// Everything is a dot product against X = [q_0 .. q_7 | k_0 .. k_7] (the window's unit vectors):
//   * h0 rows (2 heads x 128 rows x 128 fp32 = 128 KB, the only large read): each wave streams 32
//     rows into registers and multiplies them by X with the fp32 MFMA v_mfma_f32_16x16x4f32 (rows as
//     operand A, 16 B per lane per step, the k order permuted so a lane's four consecutive columns
//     feed four MFMAs), requested after every small operand so nothing waits behind them;
//   * the ring keys and the window keys (rows of LDS) the same way, by two waves;
//   * per value row, P_x = S x for the 16 vectors starts as td (h0 . x) + sum_c decay_c dhat_c
//     (khat_c . x) and the delta rule runs in that basis: u_t = beta_t (v_t - e^{g_t} P_{k_t}),
//     P_x <- e^{g_t} P_x + u_t (k_t . x), o_t = P_{q_t}; u_t is the ring's d entry.
#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int RK = 128, RV = 128, RHK = 16, RHV = 32, RQKV = 8192, RZ = RHV * RV, RL = 16, RTMAX = 8;
constexpr int KW_STRIDE = 132;  // padded fp32 key rows: the 16 rows a tile step reads hit distinct banks
constexpr int HX_STRIDE = 20;  // 16 dots + pad: 16-byte aligned rows, read as four v4f

struct GdnRingDev {
  int B, T, rows, slots, rslots, wslots;
  const uint16_t* mixed;
  const uint16_t* z;
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* conv_state;
  int64_t cs_slot;
  const uint16_t* conv_w;
  uint16_t* window;
  int64_t win_slot;
  const float* A_log;
  const void* dt_bias;
  int dt_f32;
  const float* h0;
  uint16_t* d_ring;
  uint16_t* dlo_ring;
  int64_t d_slot, dlo_slot;
  uint16_t* k_ring;
  uint16_t* klo_ring;
  int64_t k_slot, klo_slot;
  float* g_ring;
  int64_t g_slot;
  const int32_t* qsl;
  const void* state_idx;
  const void* replay_idx;
  const void* win_idx;
  int idx_i64;
  const int32_t* write_pos;
  const int32_t* cache_base;
  const uint16_t* norm_w;
  float eps, scale;
  uint16_t* out;
  uint8_t* oq;   // out's e4m3 codes per value head (the out_proj's input), or null
  float* oqs;    // [rows, 32] their scales
};

// Four waves per SIMD (two workgroups per CU): at most 128 VGPRs, of which the 16 x 4 h0 values are 64.
// TM bounds T (4, 5 or 8): the conv's input registers are sized by it.
template <int TM>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void gdn_ring_kernel(GdnRingDev d) {
  __shared__ __attribute__((aligned(16))) float xf[8][64][4];      // MFMA B fragments of X (step, lane)
  __shared__ __attribute__((aligned(16))) float kw[32][KW_STRIDE];  // rows 0-15 ring keys, 16-23 window keys
  __shared__ float qko[2][RTMAX][RK];     // raw conv q (0) / k (1); later the bf16-rounded o of head 0 / 1
  __shared__ float vs[2][RTMAX][RV];
  __shared__ __attribute__((aligned(16))) float hx[2][RV][HX_STRIDE];  // h0 row . X, per value head
  __shared__ __attribute__((aligned(16))) float xr[32][HX_STRIDE];     // kw row . X
  __shared__ __attribute__((aligned(16))) uint16_t dh[2][RL][RV];     // committed d entries, logical order
  __shared__ __attribute__((aligned(16))) uint16_t zs[RTMAX][2 * RV];  // the output gate's z
  __shared__ float nws[RV], rg[2][RL];
  __shared__ float gg[2][RTMAX], gbeta[2][RTMAX], geg[2][RTMAX];
  __shared__ float dec[2][RL], tdec[2];

  const int r = blockIdx.x >> 4, hk = blockIdx.x & 15;
  const int T = d.T, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The request's row offset and its three indices (int32, or int64 as two 32-bit words), all
  // requested before any is used: one scalar round trip.
  const int f = d.idx_i64;
  const int32_t* si = reinterpret_cast<const int32_t*>(d.state_idx);
  const int32_t* ri = reinterpret_cast<const int32_t*>(d.replay_idx);
  const int32_t* wi = reinterpret_cast<const int32_t*>(d.win_idx);
  int32_t s0 = si[(f & 1) ? 2 * r : r], s1 = si[(f & 1) ? 2 * r + 1 : r];
  int32_t r0 = ri[(f & 2) ? 2 * r : r], r1 = ri[(f & 2) ? 2 * r + 1 : r];
  int32_t w0 = wi[(f & 4) ? 2 * r : r], w1 = wi[(f & 4) ? 2 * r + 1 : r];
  int32_t q0 = d.qsl[r];
  // keeps every load above unconditional (the high words would otherwise sink into the int64 branch)
  asm volatile("" : "+s"(s0), "+s"(s1), "+s"(r0), "+s"(r1), "+s"(w0), "+s"(w1), "+s"(q0));
  auto join = [](int i64, int32_t lo, int32_t hi) {
    return i64 ? (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo) : (int64_t)lo;
  };
  const int64_t slot = join(f & 1, s0, s1), rp = join(f & 2, r0, r1), ws = join(f & 4, w0, w1);
  const int64_t bos = q0;
  if (bos < 0 || bos + T > d.rows) return;  // rows outside the batch: nothing of this request is written
  if (slot < 0 || slot >= d.slots || rp < 0 || rp >= d.rslots || ws < 0 || ws >= d.wslots) {
    // a padded request: zero output (both value heads' 256 columns), nothing else
    if (tid < 64 * T) {
      const int t = tid >> 6, c = (tid & 63) * 4;
      *reinterpret_cast<v2i*>(d.out + (bos + t) * RZ + hk * 2 * RV + c) = v2i{0, 0};
      if (d.oq) {
        *reinterpret_cast<uint32_t*>(d.oq + (bos + t) * RZ + hk * 2 * RV + c) = 0u;
        if (c == 0) {  // the key head's two value heads
          d.oqs[(bos + t) * RHV + 2 * hk] = 0.f;
          d.oqs[(bos + t) * RHV + 2 * hk + 1] = 0.f;
        }
      }
    }
    return;
  }

  // unused parts of the MFMA operands are zero
  reinterpret_cast<v4f*>(&xf[0][0][0])[tid] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int i = tid; i < 16 * KW_STRIDE; i += 512) (&kw[16][0])[i] = 0.f;

  // ---- requests.  First every small operand (conv inputs, gate inputs, ring cursors, z, the norm
  // weight, the committed ring entries by physical slot, so no address waits on the cursors), then
  // the first checkpoint rows, then a wait for the small operands only.  Vector loads complete in
  // issue order, so nothing the phases below need may be requested after a checkpoint row: a wait
  // for it would wait for the rows too.  Every load is unconditional (indices clamped into range,
  // unused values selected away): a load under a branch makes the compiler wait for it at the join.
  const int cur_wp = d.write_pos[rp], cur_cb = d.cache_base[rp];
  // conv inputs, one channel per thread: q, k of key head hk, v of both value heads.  The unit's
  // channels are three runs of the channel axis (q: 128, k: 128, v: 256); its conv state (3 bf16 a
  // channel) is read as 192 16-byte pieces of those runs and handed out through LDS, and its window
  // record and rolled state are written back the same way: a 2-byte access per lane and channel
  // costs the CU's address unit a cycle per lane.
  const int ch = tid < 256 ? (tid >> 7) * (RHK * RK) + hk * RK + (tid & 127) : 2 * RHK * RK + hk * 2 * RV + (tid - 256);
  // the 16-byte piece j of a per-channel array of `per` bf16: the run it falls in and its element offset
  auto run_piece = [&](int j, int per, int64_t& elem) {
    const int q8 = 128 * per / 8;  // pieces in the q run (and the k run); the v run has twice as many
    const int run = j < q8 ? 0 : j < 2 * q8 ? 1 : 2;
    const int base = run == 0 ? hk * RK : run == 1 ? RHK * RK + hk * RK : 2 * RHK * RK + hk * 2 * RV;
    elem = (int64_t)base * per + 8 * (j - run * q8);
  };
  uint16_t* const cs_base = d.conv_state + slot * d.cs_slot;
  int64_t cs_elem;
  run_piece(min(tid, 191), 3, cs_elem);
  const v4i csv = *reinterpret_cast<const v4i*>(cs_base + cs_elem);
  float w[TM + 3];
#pragma unroll
  for (int t = 0; t < TM; ++t) w[3 + t] = bf2f(d.mixed[(bos + min(t, T - 1)) * RQKV + ch]);
  const v2i cwr = *reinterpret_cast<const v2i*>(d.conv_w + (int64_t)ch * 4);
  // gate inputs: thread tid < 2 T serves head tid & 1, position tid >> 1
  const int gt = min(tid, 2 * T - 1), ghv = 2 * hk + (gt & 1);
  const int64_t grow = bos + (gt >> 1);
  const float av = bf2f(d.a[grow * RHV + ghv]), bv = bf2f(d.b[grow * RHV + ghv]);
  const uint32_t dtw = reinterpret_cast<const uint32_t*>(d.dt_bias)[d.dt_f32 ? ghv : ghv >> 1];
  const float alog = d.A_log[ghv];
  // z: position tid >> 6 (rows past T read row T - 1), columns 4 (tid & 63) .. + 3 of the unit's 256
  const v2i zraw = *reinterpret_cast<const v2i*>(d.z + (bos + min(tid >> 6, T - 1)) * RZ + hk * 2 * RV + (tid & 63) * 4);
  const uint32_t nwraw = d.norm_w[tid & (RV - 1)];
  // the committed ring entries by physical slot (placed in logical order, zero past the history, when
  // they go to LDS) and gates
  const int kc = tid >> 5, kcol = (tid & 31) * 4;  // keys: 16 slots x 32 x 4 columns
  const v2i kraw = *reinterpret_cast<const v2i*>(d.k_ring + rp * d.k_slot + ((int64_t)hk * RL + kc) * RK + kcol);
  const int dhd = tid >> 8, dc = (tid >> 4) & 15, dv = (tid & 15) * 8;  // d: 2 heads x 16 x 16 x 8
  const v4i draw = *reinterpret_cast<const v4i*>(d.d_ring + rp * d.d_slot + ((int64_t)(2 * hk + dhd) * RL + dc) * RV + dv);
  const float graw = d.g_ring[rp * d.g_slot + (2 * hk + ((tid >> 4) & 1)) * RL + (tid & 15)];
  // the checkpoint: wave w holds head w >> 2, rows 32 (w & 3) .. + 31 as two 16-row tiles; lane l
  // reads row l & 15 of a tile, columns 16 s + 4 (l >> 4) .. + 3 at step s.  Its 8 steps are
  // requested two at a time through the phases below (about 64 KB in flight a CU: enough to keep
  // HBM busy, little enough that a phase's own stores, issued before its next request, do not queue
  // behind a deep stream in the CU's in-order memory pipe)
  const int hh = wave >> 2, rb = (wave & 3) * 32;
  const float* hp = d.h0 + ((slot * RHV + 2 * hk + hh) * RV + rb + (lane & 15)) * RK + 4 * (lane >> 4);
  v4f hr[2][8];
  auto request = [&](int s0) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int s = s0; s < s0 + 2; ++s)
        hr[i][s] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(hp + i * 16 * RK + 16 * s));
    asm volatile("" ::: "memory");
  };
  request(0);
  // The small operands have arrived (the 4 row requests may fly).  The wait comes from the compiler,
  // through a use of each value: a hand-written wait is invisible to its accounting, which would then
  // place its own wait for these values later, counted past the rows, and so wait for the rows.
#pragma unroll
  for (int i = 3; i < TM + 3; ++i) asm volatile("" ::"v"(w[i]));
  asm volatile("" ::"v"(cwr), "v"(av), "v"(bv), "v"(dtw), "v"(alog), "v"(zraw), "v"(nwraw));
  asm volatile("" ::"v"(kraw), "v"(draw), "v"(graw), "v"(csv));
  // the unit's conv state through LDS (hx is free until the checkpoint dots): channel L = tid at
  // elements 3 L .. 3 L + 2 of the staging run, in the order of the three runs
  uint16_t* const stage = reinterpret_cast<uint16_t*>(&hx[0][0][0]);
  if (tid < 192) *reinterpret_cast<v4i*>(stage + 8 * tid) = csv;
  __syncthreads();
  w[0] = bf2f(stage[3 * tid]);
  w[1] = bf2f(stage[3 * tid + 1]);
  w[2] = bf2f(stage[3 * tid + 2]);
  if ((tid >> 6) < T) *reinterpret_cast<v2i*>(&zs[tid >> 6][(tid & 63) * 4]) = zraw;
  if (tid < RV) nws[tid] = bf2f(nwraw);
  const int nv = min(max(__builtin_amdgcn_readfirstlane(cur_wp), 0), RL);
  const int cb = __builtin_amdgcn_readfirstlane(cur_cb);

  // ---- conv + SiLU (bf16 tap products, oldest first), the rolled state and the window record
  {
    const float cw0 = bf_lo((uint32_t)cwr[0]), cw1 = bf_hi((uint32_t)cwr[0]);
    const float cw2 = bf_lo((uint32_t)cwr[1]), cw3 = bf_hi((uint32_t)cwr[1]);
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      if (t < T) {
        float acc = rbf(w[t] * cw0);
        acc = acc + rbf(w[t + 1] * cw1);
        acc = acc + rbf(w[t + 2] * cw2);
        acc = acc + rbf(w[t + 3] * cw3);
        const float o = rbf(acc / (1.f + expf_q(-acc)));
        if (wave < 4) qko[tid >> 7][t][tid & 127] = o;  // wave-uniform: one object per store
        else vs[(tid - 256) >> 7][t][(tid - 256) & 127] = o;
      }
    }
    // the window record (T + 2 values a channel) into LDS after the conv state's 1536 elements;
    // the rolled state over this channel's own three staged values (read above, by this thread only)
    uint16_t* const rec = stage + 1536 + tid * (T + 2);
#pragma unroll
    for (int i = 0; i < TM + 2; ++i)
      if (i < T + 2) rec[i] = (uint16_t)f2bf(w[1 + i]);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      float v = 0.f;
#pragma unroll
      for (int t = 0; t < TM + 3; ++t) v = t == T + i ? w[t] : v;
      stage[3 * tid + i] = (uint16_t)f2bf(v);
    }
  }
  if (tid < 2 * T) {
    const int h = tid & 1, t = tid >> 1;
    // dt_bias: the fp32 word, or the bf16 half of the word that holds element ghv (shift and mask, no
    // branch on the loaded value)
    const uint32_t dsh = d.dt_f32 ? 0u : ((ghv & 1) ? 0u : 16u);
    const uint32_t dmask = d.dt_f32 ? 0xffffffffu : 0xffff0000u;
    const float dtb = __uint_as_float((dtw << dsh) & dmask);
    const float xg = av + dtb;
    const float sp = xg <= 20.f ? logf(1.f + expf_q(xg)) : xg;
    const float g = -expf_q(alog) * sp;
    gg[h][t] = g;
    gbeta[h][t] = sigmoid_q(bv);
    geg[h][t] = expf_q(g);
  }
  request(2);
  __syncthreads();
  // the rolled conv state and the window record, 16 bytes a lane, from the staging runs
  if (tid < 192) *reinterpret_cast<v4i*>(cs_base + cs_elem) = *reinterpret_cast<const v4i*>(stage + 8 * tid);
  for (int j = tid; j < 64 * (T + 2); j += 512) {
    int64_t we;
    run_piece(j, T + 2, we);
    *reinterpret_cast<v4i*>(d.window + ws * d.win_slot + we) = *reinterpret_cast<const v4i*>(stage + 1536 + 8 * j);
  }

  // ---- the committed entries into LDS: physical slot p holds logical entry (p - cb) mod 16; keys
  // into key rows 0-15 (logical order, zero past the history), d entries (zero past the history), gates
  {
    const int lk = (kc - cb) & 15, ldc = (dc - cb) & 15;
    const bool kon = lk < nv;
    kw[lk][kcol] = kon ? bf_lo((uint32_t)kraw[0]) : 0.f;
    kw[lk][kcol + 1] = kon ? bf_hi((uint32_t)kraw[0]) : 0.f;
    kw[lk][kcol + 2] = kon ? bf_lo((uint32_t)kraw[1]) : 0.f;
    kw[lk][kcol + 3] = kon ? bf_hi((uint32_t)kraw[1]) : 0.f;
    const v4i dz = {0, 0, 0, 0};
    *reinterpret_cast<v4i*>(&dh[dhd][ldc][dv]) = ldc < nv ? draw : dz;
    if (tid < 32) rg[tid >> 4][((tid & 15) - cb) & 15] = graw;
  }
  // ---- q/k unit vectors into the X fragments (q_t = vector t, k_t = vector 8 + t), the window keys
  // into key rows 16 + t; the window's key and gate appends (logical entries nv + t that fit)
  for (int p = wave; p < 2 * T; p += 8) {
    const int part = p & 1, t = p >> 1, vec = part * 8 + t;
    const float x0 = qko[part][t][lane], x1 = qko[part][t][lane + 64];
    const float ss = wave_sum_bfly(x0 * x0 + x1 * x1);
    float rr = 1.f / sqrtf(ss + 1e-6f);
    if (part == 0) rr = rr * d.scale;
    const float y0 = x0 * rr, y1 = x1 * rr;
    // column c sits at xf[c >> 4][((c >> 2) & 3) * 16 + vec][c & 3]
    xf[lane >> 4][((lane >> 2) & 3) * 16 + vec][lane & 3] = y0;
    xf[(lane + 64) >> 4][((lane >> 2) & 3) * 16 + vec][lane & 3] = y1;
    if (part == 1) {
      kw[16 + t][lane] = y0;
      kw[16 + t][lane + 64] = y1;
      if (nv + t < RL) {
        const int ph = (cb + nv + t) & 15;
        const int64_t off = ((int64_t)hk * RL + ph) * RK + lane;
        const uint32_t h0b = f2bf(y0), h1b = f2bf(y1);
        d.k_ring[rp * d.k_slot + off] = (uint16_t)h0b;
        d.k_ring[rp * d.k_slot + off + 64] = (uint16_t)h1b;
        d.klo_ring[rp * d.klo_slot + off] = (uint16_t)f2bf(y0 - bf2f(h0b));
        d.klo_ring[rp * d.klo_slot + off + 64] = (uint16_t)f2bf(y1 - bf2f(h1b));
        if (lane < 2) d.g_ring[rp * d.g_slot + (2 * hk + lane) * RL + ph] = gg[lane][t];
      }
    }
  }
  request(4);
  __syncthreads();

  // ---- dots that need no checkpoint row, while the early rows stream: ring keys (wave 0) and window
  // keys (wave 1) against X, and the history's decays (32 lanes of wave 7).
  // key rows r0 .. r0 + 15 of kw against X -> xr rows r0 .. r0 + 15 (two accumulation chains)
  auto xr_tile = [&](int r0) {
    v4f a2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const v4f ka = *reinterpret_cast<const v4f*>(&kw[r0 + (lane & 15)][16 * s + 4 * (lane >> 4)]);
      const v4f xb = *reinterpret_cast<const v4f*>(&xf[s][lane][0]);
#pragma unroll
      for (int j = 0; j < 4; ++j) a2[s & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[j], xb[j], a2[s & 1], 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) xr[r0 + 4 * (lane >> 4) + q][lane & 15] = a2[0][q] + a2[1][q];
  };
  if (wave == 0) xr_tile(0);
  else if (wave == 1) xr_tile(16);
  else if (tid >= 448 && tid < 480) {  // decay of entry c: exp(total - prefix_c), sums in logical order
    const int h = (tid - 448) >> 4, c = tid & 15;
    float tot = 0.f, pre = 0.f;
#pragma unroll
    for (int e = 0; e < RL; ++e) {
      if (e < nv) tot = tot + rg[h][e];
      if (e == c) pre = tot;
    }
    dec[h][c] = c < nv ? expf_q(tot - pre) : 0.f;
    if (c == 0) tdec[h] = expf_q(tot);
  }
  request(6);
  __syncthreads();
  // The history's part of each row's dots: R_x = sum_c decay_c dhat_c (khat_c . x).  Lanes 2j and
  // 2j + 1 share row tid >> 1: the even lane keeps the q-vectors (x < 8), the odd lane the k-vectors
  // (x >= 8).  Past the history the entries and decays are zero, so the loop has no branch.
  const int row = tid >> 1, part = tid & 1, rh = row >> 7, rv = row & 127;
  float P[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < RL; ++c) {
    const float dsc = bf2f(dh[rh][c][rv]) * dec[rh][c];
#pragma unroll
    for (int x4 = 0; x4 < 2; ++x4) {
      const v4f xv = *reinterpret_cast<const v4f*>(&xr[c][8 * part + 4 * x4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) P[4 * x4 + i] = __builtin_fmaf(dsc, xv[i], P[4 * x4 + i]);
    }
  }

  // ---- the checkpoint rows' dots, step by step as they arrive
  {
    v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const v4f xb = *reinterpret_cast<const v4f*>(&xf[s][lane][0]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(hr[0][s][j], xb[j], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(hr[1][s][j], xb[j], acc[1], 0, 0, 0);
      }
    }
    // D: lane l, register q = row 4 (l >> 4) + q of the tile, vector l & 15
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) hx[hh][rb + 16 * i + 4 * (lane >> 4) + q][lane & 15] = acc[i][q];
  }
  __syncthreads();

  // ---- per value row: P_x = td (h0 . x) + R_x = S x for the window's vectors, then the delta rule
  // in that basis; u_t comes from the odd lane's P_{k_t} through a DPP swap
  {
    const float td = tdec[rh];
#pragma unroll
    for (int x4 = 0; x4 < 2; ++x4) {
      const v4f hv4 = *reinterpret_cast<const v4f*>(&hx[rh][rv][8 * part + 4 * x4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) P[4 * x4 + i] = __builtin_fmaf(td, hv4[i], P[4 * x4 + i]);
    }
    const int64_t dro = rp * d.d_slot + (int64_t)(2 * hk + rh) * RL * RV + rv;
    const int64_t dlo = rp * d.dlo_slot + (int64_t)(2 * hk + rh) * RL * RV + rv;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      if (t < T) {
        const float eg = geg[rh][t];
        // P_{k_t}: the odd lane's own P[t], the even lane's partner's
        const float other = __uint_as_float(dpp_u32<0xB1>(__float_as_uint(P[t])));
        const float kt = part ? P[t] : other;
        const float u = gbeta[rh][t] * (vs[rh][t][rv] - eg * kt);
#pragma unroll
        for (int x4 = 0; x4 < 2; ++x4) {
          const v4f xv = *reinterpret_cast<const v4f*>(&xr[16 + t][8 * part + 4 * x4]);
#pragma unroll
          for (int i = 0; i < 4; ++i) P[4 * x4 + i] = __builtin_fmaf(eg, P[4 * x4 + i], u * xv[i]);
        }
        if (part == 0) {
          qko[rh][t][rv] = rbf(P[t]);  // the core output is bf16
        } else if (nv + t < RL) {
          const int ph = (cb + nv + t) & 15;
          const uint32_t hi = f2bf(u);
          d.d_ring[dro + ph * RV] = (uint16_t)hi;
          d.dlo_ring[dlo + ph * RV] = (uint16_t)f2bf(u - bf2f(hi));
        }
      }
    }
  }
  __syncthreads();

  // ---- gated RMSNorm per (head, position): y = bf16(((o * rstd) * w) * (z * sigmoid(z)))
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int p = wave + 8 * jj;
    if (p < 2 * T) {
      const int h = p & 1, t = p >> 1;
      const float o0 = qko[h][t][lane], o1 = qko[h][t][lane + 64];
      const float ss = wave_sum_bfly(o0 * o0 + o1 * o1);
      const float rstd = 1.f / sqrtf(ss / (float)RV + d.eps);
      const float z0 = bf2f(zs[t][h * RV + lane]), z1 = bf2f(zs[t][h * RV + lane + 64]);
      uint16_t* op = d.out + (bos + t) * RZ + (2 * hk + h) * RV + lane;
      const uint32_t y0 = f2bf(((o0 * rstd) * nws[lane]) * (z0 * sigmoid_q(z0)));
      const uint32_t y1 = f2bf(((o1 * rstd) * nws[lane + 64]) * (z1 * sigmoid_q(z1)));
      op[0] = (uint16_t)y0;
      op[64] = (uint16_t)y1;
      if (d.oq) {
        // the value head's 128 outputs are one e4m3 group of the out_proj's input (the wave's lanes)
        const float f0 = bf2f(y0), f1 = bf2f(y1);
        const float m = wave_max(fmaxf(fabsf(f0), fabsf(f1)));
        const float inv = m > 0.f ? 448.f / m : 0.f;
        const uint32_t cd = f2e4m3x2_hw(f0 * inv, f1 * inv);
        uint8_t* qp = d.oq + (bos + t) * RZ + (2 * hk + h) * RV + lane;
        qp[0] = (uint8_t)(cd & 0xffu);
        qp[64] = (uint8_t)((cd >> 8) & 0xffu);
        if (lane == 0) d.oqs[(bos + t) * RHV + 2 * hk + h] = m / 448.f;
      }
    }
  }
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" int q36_gdn_verify_ring(const q36_gdn_ring_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_gdn_verify_ring: null args");
  Q36_REQUIRE(a->B >= 0 && a->B <= (1 << 20), "q36_gdn_verify_ring: B=%d out of range", a->B);
  Q36_REQUIRE(a->T >= 1 && a->T <= RTMAX, "q36_gdn_verify_ring: T=%d must be in [1,%d]", a->T, RTMAX);
  if (a->B == 0) return Q36_OK;
  Q36_REQUIRE(a->mixed && a->z && a->a && a->b && a->conv_state && a->conv_w && a->window && a->A_log &&
                  a->dt_bias && a->h0 && a->d_ring && a->dlo_ring && a->k_ring && a->klo_ring && a->g_ring &&
                  a->qsl && a->state_idx && a->replay_idx && a->win_idx && a->write_pos && a->cache_base &&
                  a->norm_w && a->out,
              "q36_gdn_verify_ring: a required pointer is null");
  Q36_REQUIRE(a->rows >= a->T && a->slots >= 1 && a->rslots >= 1 && a->wslots >= 1,
              "q36_gdn_verify_ring: rows=%d slots=%d rslots=%d wslots=%d", a->rows, a->slots, a->rslots, a->wslots);
  Q36_REQUIRE(a->cs_slot >= RQKV * 3 && a->cs_slot % 8 == 0, "q36_gdn_verify_ring: conv_state slot stride %lld",
              (long long)a->cs_slot);
  Q36_REQUIRE(a->win_slot >= (int64_t)RQKV * (a->T + 2) && a->win_slot % 8 == 0,
              "q36_gdn_verify_ring: window slot stride %lld must be >= 8192 x %d and a multiple of 8",
              (long long)a->win_slot, a->T + 2);
  Q36_REQUIRE(a->d_slot >= RHV * RL * RV && a->dlo_slot >= RHV * RL * RV && a->d_slot % 8 == 0 && a->dlo_slot % 8 == 0,
              "q36_gdn_verify_ring: d ring slot strides must be >= 32 x 16 x 128 and multiples of 8");
  Q36_REQUIRE(a->k_slot >= RHK * RL * RK && a->klo_slot >= RHK * RL * RK && a->k_slot % 8 == 0 && a->klo_slot % 8 == 0,
              "q36_gdn_verify_ring: k ring slot strides must be >= 16 x 16 x 128 and multiples of 8");
  Q36_REQUIRE(a->g_slot >= RHV * RL && a->g_slot % 4 == 0, "q36_gdn_verify_ring: g ring slot stride %lld",
              (long long)a->g_slot);
  Q36_REQUIRE(aligned16(a->h0) && aligned16(a->z) && aligned16(a->conv_state) && aligned16(a->window) &&
                  aligned16(a->conv_w) && aligned16(a->d_ring) &&
                  aligned16(a->dlo_ring) && aligned16(a->k_ring) && aligned16(a->klo_ring) && aligned16(a->g_ring) &&
                  aligned16(a->out),
              "q36_gdn_verify_ring: h0, z, conv_state, window, conv_w, the rings and out must be 16-byte aligned");
  Q36_REQUIRE((reinterpret_cast<uintptr_t>(a->dt_bias) & 3) == 0, "q36_gdn_verify_ring: dt_bias must be 4-byte aligned");
  Q36_REQUIRE((a->oq == nullptr) == (a->oqs == nullptr), "q36_gdn_verify_ring: oq and oqs go together");
  Q36_REQUIRE(!a->oq || ((reinterpret_cast<uintptr_t>(a->oq) & 3u) == 0 && (reinterpret_cast<uintptr_t>(a->oqs) & 3u) == 0),
              "q36_gdn_verify_ring: oq and oqs must be 4-byte aligned");
  GdnRingDev d{a->B, a->T, a->rows, a->slots, a->rslots, a->wslots,
               static_cast<const uint16_t*>(a->mixed), static_cast<const uint16_t*>(a->z),
               static_cast<const uint16_t*>(a->a), static_cast<const uint16_t*>(a->b),
               static_cast<uint16_t*>(a->conv_state), a->cs_slot, static_cast<const uint16_t*>(a->conv_w),
               static_cast<uint16_t*>(a->window), a->win_slot, a->A_log, a->dt_bias, a->dt_f32 ? 1 : 0, a->h0,
               static_cast<uint16_t*>(a->d_ring), static_cast<uint16_t*>(a->dlo_ring), a->d_slot, a->dlo_slot,
               static_cast<uint16_t*>(a->k_ring), static_cast<uint16_t*>(a->klo_ring), a->k_slot, a->klo_slot,
               a->g_ring, a->g_slot, a->qsl, a->state_idx, a->replay_idx, a->win_idx, a->idx_i64 & 7,
               a->write_pos, a->cache_base, static_cast<const uint16_t*>(a->norm_w), a->eps, a->scale,
               static_cast<uint16_t*>(a->out), static_cast<uint8_t*>(a->oq), a->oqs};
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->T <= 4) gdn_ring_kernel<4><<<a->B * RHK, 512, 0, st>>>(d);
  else if (a->T == 5) gdn_ring_kernel<5><<<a->B * RHK, 512, 0, st>>>(d);
  else gdn_ring_kernel<8><<<a->B * RHK, 512, 0, st>>>(d);
  return check_launch("q36_gdn_verify_ring");
}
