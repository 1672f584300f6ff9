// Int8 lm_head fused with greedy argmax for gfx950.
//
// Reference behaviour (R = qwen36_nodes_kb34, H = R/qwen36_lmhead8): per-row int8 activations
// (H/w8a8.py:16-23), per-channel int8 weights with fp32 scales (H/lmhead8.py:95-143), int32
// accumulation, logit = (acc * xs) * ws (H/w8a8.py:66-71) rounded to bf16 (the node's output
// dtype); in the two-term form (H/w8a8.py:25-37, the reference's rule from 64 rows on) a second
// int8 term quantizes the residual x - q1 s1 and logit = bf16(fma(acc1, s1, acc2 * s2) * ws)
// (H/w8a8.py:66-70; L/qk_proj_decode.cu:1103-1107); the greedy token is the first index of the largest bf16 logit (torch.argmax order; the
// reference leaves the argmax to the stock sampler, H/node.py:136-151).  A final Gemma RMSNorm
// y = bf16((x * rstd) * (1 + w)) precedes the quantization (L/proj.py:60-81 restates the form).
//
// Kernels:
//   lmh_prep   one wave per row: norm (sum of squares in the fixed 64-lane order), int8 quant,
//              and the row's argmax key reset to 0.
//   lmh_gemm   persistent, one 512-thread workgroup per CU walking 256 x 256 output tiles (8 waves,
//              two a SIMD, each 128 vocab rows x 64 tokens, 32x32x32 int8 MFMAs with the weights as
//              operand A, int32 accumulators); K in 64-byte steps through LDS rings filled by
//              buffer loads straight into LDS (weights 6 stages, loaded by four waves six steps
//              ahead; activations 3 stages, loaded by the other four), fragments double-buffered
//              in registers, and the next tile's first steps requested before the epilogue.
//              Epilogue: bf16 logits, the
//              first column of each row's largest value folded into an order-preserving key, and one
//              64-bit atomic max per row and tile: the result does not depend on the order the
//              workgroups finish in.  lmh_gemm_logits: the same, writing the bf16 logits too.
//   lmh_ids    key -> token id.
// Tile order: two row groups of XCDs (see lmh_gemm_body); the row tiles of one vocab tile run side
// by side on one XCD, whose L2 serves them the weight tile and keeps their activations resident.
#include <type_traits>

#include "q36_device.h"
#include "q36_host.h"
#include "q36_w8a16.h"

namespace q36 {
namespace {

constexpr int kLH = 2048;       // hidden (K)
constexpr int kBM = 256, kBN = 256, kBK = 64, kNK = kLH / kBK;  // 32 K steps
constexpr int kLmhWaves = 8;  // waves of the GEMM workgroup: two a SIMD
constexpr int kNSA = 3, kNSB = 6;  // LDS ring stages of the activations and of the weights

struct LmhDev {
  int R, V;
  int Rs;   // activation rows in xq: R (one term) or 64 * ceil(R / 32) (two terms, see act_row)
  int x2;   // two activation terms (Q36_LMH_W8A8X2)
  int w16;  // W8A16: the prep writes the (normed) bf16 rows to xq instead of quantizing them
  const uint16_t* h;
  const uint16_t* norm_w;
  float eps;
  const int8_t* wq;
  const float* ws;
  int32_t* ids;
  uint16_t* logits;   // bf16 [R, V] or null
  float* logits32;    // fp32 [R, V] (bf16-rounded values) or null; at most one of the two is set
  int8_t* xq;
  float* xs;
  unsigned long long* keys;
};

// Row of the activation codes holding term `term` of token r.  One term: row r.  Two terms: the
// tokens go in groups of 32, each group's term-1 rows followed by its term-2 rows (row 64 (r / 32) +
// 32 term + r % 32), so one lane of the GEMM holds both terms of the same token in its accumulators.
__host__ __device__ __forceinline__ int act_row(int r, int term, int x2) {
  return x2 ? 64 * (r >> 5) + 32 * term + (r & 31) : r;
}
__host__ __device__ __forceinline__ int act_rows(int R, int x2) { return x2 ? 64 * ((R + 31) >> 5) : R; }

// one wave (and workgroup) per row: a batch's rows spread over as many CUs
__global__ __launch_bounds__(64) void lmh_prep_kernel(LmhDev d) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x;
  if (r >= d.R) return;
  constexpr int NJ = kLH / 512;
  float y[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const v4i v = *reinterpret_cast<const v4i*>(d.h + (size_t)r * kLH + 8 * (lane + 64 * j));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      y[j][2 * q] = bf_lo((uint32_t)v[q]);
      y[j][2 * q + 1] = bf_hi((uint32_t)v[q]);
    }
  }
  if (d.norm_w) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(y[j][i], y[j][i], acc);
    const float ss = wave_sum_bfly(acc);
    const float rstd = 1.f / sqrtf(ss / (float)kLH + d.eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const v4i wv = *reinterpret_cast<const v4i*>(d.norm_w + 8 * (lane + 64 * j));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        y[j][2 * q] = rbf((y[j][2 * q] * rstd) * (1.f + bf_lo((uint32_t)wv[q])));
        y[j][2 * q + 1] = rbf((y[j][2 * q + 1] * rstd) * (1.f + bf_hi((uint32_t)wv[q])));
      }
    }
  }
  if (d.w16) {  // W8A16: the bf16 rows themselves
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      v4i ov;
#pragma unroll
      for (int q = 0; q < 4; ++q) ov[q] = (int)pack_bf2(y[j][2 * q], y[j][2 * q + 1]);
      *reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(d.xq) + (size_t)r * kLH + 8 * (lane + 64 * j)) = ov;
    }
    if (lane == 0) d.keys[r] = 0ull;
    return;
  }
  // one int8 term per row; with two terms the second quantizes the residual y - q1 s1 (formed as
  // one fma) by the same rule, so y = q1 s1 + q2 s2 to within s2 / 2
  for (int term = 0; term < (d.x2 ? 2 : 1); ++term) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(y[j][i]));
    m = wave_max(m);
    const float sc = m / 127.f, safe = m > 0.f ? sc : 1.f;
    const int row = act_row(r, term, d.x2);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      uint32_t wd[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int qv = round_i8(y[j][i] / safe);
        wd[i >> 2] |= ((uint32_t)qv & 0xffu) << (8 * (i & 3));
        y[j][i] = __builtin_fmaf(-(float)qv, sc, y[j][i]);
      }
      *reinterpret_cast<uint2*>(d.xq + (size_t)row * kLH + 8 * (lane + 64 * j)) = make_uint2(wd[0], wd[1]);
    }
    if (lane == 0) d.xs[row] = sc;
  }
  if (lane == 0) d.keys[r] = 0ull;
}

// LDS position of 16-byte chunk kc (0..3) of tile row c in one K step: rows are 64 bytes, unpadded,
// with the chunk order xor-swizzled by ((c >> 1) & 3) ^ ((c >> 3) & 1).  A fragment read takes chunk
// kc of consecutive rows; LDS serves a 16-byte read 16 lanes at a time over 64 banks, and with this
// swizzle any 16 consecutive rows (and any 8) land in distinct 16-byte bank windows.
__device__ __forceinline__ int bswz(int c, int kc) { return c * kBK + ((kc ^ ((c >> 1) & 3) ^ ((c >> 3) & 1)) << 4); }

template <int N>
using ic = std::integral_constant<int, N>;
// f(ic<0>{}), f(ic<1>{}), ... in order, each index a compile-time constant
template <typename F, int... KS>
__device__ __forceinline__ void for_steps(F&& f, std::integer_sequence<int, KS...>) {
  (f(ic<KS>{}), ...);
}

// threadIdx.x through an empty asm: values derived from it are recomputed where they are used
// instead of being kept (or spilled) across the K loop
__device__ __forceinline__ int opaque_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}


// s_waitcnt with only the vector-memory count constrained (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Persistent GEMM + argmax: one 512-thread workgroup per CU walks its XCD's tiles.  The XCDs form
// ngrp row groups (2 when the row tiles split evenly, else 1): XCD x serves the rpg = nrt / ngrp
// row tiles of group x % ngrp and the vocab tiles v = x / ngrp (mod 8 / ngrp).  Its workgroups take
// tiles j = loc, loc + nloc, ... (loc = blockIdx / 8, nloc = gridDim / 8), tile j being row tile
// (x % ngrp) * rpg + j % rpg of vocab tile (j / rpg) * (8 / ngrp) + x / ngrp: the row tiles of one
// vocab tile run side by side on one XCD (its weight tile comes from HBM once per XCD), and an
// XCD's activations (rpg row tiles, 2 MB at 2048 rows) stay resident in its L2 while the weights
// stream through.
//
// Per tile, 32 K steps of 64 bytes through two LDS rings filled by buffer loads straight into LDS
// (no register staging): the weights' 6 stages, loaded by waves 0-3 six steps ahead, and the
// activations' 3 stages (L2-resident), loaded by waves 4-7 three steps ahead.  Vector-memory loads
// complete in order per wave, so a wave that loaded both operands could give neither a deeper
// lookahead than the other; with one operand a wave, each ring has its own depth.  Each wave owns a
// 128 x 64 block (32x32x32 int8 MFMAs, weights as operand A, int32 accumulators) and keeps two
// register sets of fragments: while the 16 MFMAs of step ks run on one set, the 12 LDS reads of step
// ks + 1 fill the other and the wave's loads of step ks + (6 or 3) go out.  One barrier per step:
// before it, each wave waits for its own loads of step ks + 1 and its LDS reads of step ks (the
// stages the loads issued after the barrier overwrite).  The next tile's scales and first steps go
// out before the epilogue, so it runs while they land.  The LDS reads, 96 KB a step besides the
// 32 KB the loads write, keep the matrix cores below full rate: the ring depth changes little.
// row groups of XCDs (see lmh_gemm_body): two when there are at least 4 row tiles, evenly split
__host__ __device__ __forceinline__ int lmh_groups(int nrt) { return nrt >= 4 && nrt % 2 == 0 ? 2 : 1; }

// LDS of the GEMM workgroup, declared once in the kernel and shared by both load roles
struct LmhLds {
  int8_t* a[kNSA];  // activation stages
  int8_t* b[kNSB];  // weight stages
  float (*sc)[2][kBN];
  uint32_t (*rkey)[kBM];
};

// STORE: 0 no logits, 1 bf16 logits, 2 fp32 logits (the bf16-rounded values widened).  ROLE: the
// loads this wave issues (0: weights, waves 0-3; 1: activations, waves 4-7); everything else is the
// same in both.  Each role is its own instantiation, so the compiler's wait counting sees only the
// wave's own operand in flight.
template <int STORE, bool X2, int NW, int ROLE, bool WT>
__device__ __forceinline__ void lmh_gemm_body(const LmhDev& d, const LmhLds& L) {
  // NW waves: two vocab halves (wn) x NW / 2 token groups (wm); a wave owns 128 vocab columns (VB = 4
  // blocks of 32) x TW tokens (TB blocks of 32)
  constexpr int WM = NW / 2, TW = kBM / WM, TB = TW / 32, VB = 4;
  static_assert(NW == 8, "eight waves: four load each operand");
  constexpr int CPL = 16 / (NW / 2);      // 1 KB chunks a wave loads per step (its operand only)
  constexpr int NS = ROLE == 0 ? kNSB : kNSA;  // stages of its operand's ring: loads go NS steps ahead
  constexpr int NRD = 2 * TB + 2 * VB;    // its fragment reads per step
  constexpr int NMF = 2 * TB * VB;        // its MFMAs per step
  auto a_st = [&](auto st) -> int8_t* { return L.a[decltype(st)::value]; };
  auto b_st = [&](auto st) -> int8_t* { return L.b[decltype(st)::value]; };
  float (*sc_l)[2][kBN] = L.sc;
  uint32_t (*rkey)[kBM] = L.rkey;
  const int nvt = (d.V + kBN - 1) / kBN, nrt = (d.Rs + kBM - 1) / kBM;
  const int xcd = blockIdx.x & 7, loc = blockIdx.x >> 3, nloc = gridDim.x >> 3;
  const int ngrp = lmh_groups(nrt), rpg = nrt / ngrp, vstep = 8 / ngrp;
  const int rbase = (xcd % ngrp) * rpg, vres = xcd / ngrp;
  auto vt_of = [&](int jj) { return (jj / rpg) * vstep + vres; };
  int j = loc;
  if (vt_of(j) >= nvt) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;  // token group, vocab half
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  // Load i of a loading wave fills 1 KB chunk q = CPL (w % 4) + i of its operand's stage (tile rows
  // 16 q .. 16 q + 15); lane l writes bytes 16 l .. 16 l + 15 of the chunk, which bswz assigns to row
  // 16 q + l / 4, logical 16-byte chunk (l % 4) ^ ((l / 8) % 4) ^ (l / 32).  Rows past R or V read as
  // zero (buffer bounds).
  const int voff = (lane >> 2) * kLH + (((lane & 3) ^ ((lane >> 3) & 3) ^ (lane >> 5)) << 4);
  struct Tile {
    int r0, v0;
    __amdgpu_buffer_rsrc_t a, b;
  };
  auto tile = [&](int jj) {
    Tile t;
    t.r0 = (rbase + jj % rpg) * kBM;
    t.v0 = vt_of(jj) * kBN;
    t.a = __builtin_amdgcn_make_buffer_rsrc((void*)(d.xq + (size_t)t.r0 * kLH), (short)0,
                                            min(d.Rs - t.r0, kBM) * kLH, 0x00020000);
    t.b = __builtin_amdgcn_make_buffer_rsrc((void*)(d.wq + (size_t)t.v0 * kLH), (short)0,
                                            min(d.V - t.v0, kBN) * kLH, 0x00020000);
    return t;
  };
  // The row offset rides in the VGPR offset, the K offset in the SGPR offset: the buffer range
  // check covers only the former, so rows past the tile's last valid row read zero.
  int vrow[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i)
    vrow[i] = ROLE == 0 && WT ? 16 * lane + (CPL * (wv & 3) + i) * 16 * kLH : voff + (CPL * (wv & 3) + i) * 16 * kLH;
  auto issue_to = [&](const Tile& t, int ks, int8_t* s, int i) {
    const int q = (wv & 3) * CPL + i;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ROLE == 0 ? t.b : t.a, s + q * 1024, 16, vrow[i],
                                             ROLE == 0 && WT ? ks * 1024 : ks * kBK, 0, 0);
  };
  // load i of step KS (its stage KS % NS of the wave's operand)
  auto issue_one = [&](const Tile& t, auto ksc, int i) {
    constexpr int KS = decltype(ksc)::value;
    if constexpr (ROLE == 0) issue_to(t, KS, b_st(ic<KS % kNSB>{}), i);
    else issue_to(t, KS, a_st(ic<KS % kNSA>{}), i);
  };
  // the tile's weight and row scales (wave w < 4: entries 64 w .. 64 w + 63 of each; past V or R: zero)
  auto issue_scales = [&](const Tile& t, int par) {
    if (wv >= 4) return;
    const __amdgpu_buffer_rsrc_t ws = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(d.ws + t.v0), (short)0, min(d.V - t.v0, kBN) * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(d.xs + t.r0), (short)0, min(d.Rs - t.r0, kBM) * 4, 0x00020000);
    const int so = 4 * (opaque_tid() & 63) + 256 * wv;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ws, &sc_l[par][0][64 * wv], 4, so, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xs, &sc_l[par][1][64 * wv], 4, so, 0, 0, 0);
  };
  // Fragments: lane l reads tile row 32 t + l % 32, K bytes 16 (l / 32) of each 32-byte half step
  // (LDS chunk 2 h + l / 32); the MFMA gives lane l token l % 32 and vocab rows
  // 8 (j / 4) + 4 (l / 32) + j % 4 of register j.
  const int l32 = lane & 31, lh = lane >> 5;
  const int fx0 = bswz(wm * TW + l32, lh), fx1 = bswz(wm * TW + l32, 2 + lh);  // + 32 kBK per t
  // WT (weights in the tile order, each 16-row x 64-byte piece 1 KB contiguous): the DMA puts lane l's
  // 16 bytes (row 16 q + l % 16, K chunk l / 16 of the step) at 16 l of chunk q, and a fragment read's
  // 16 lanes take 256 contiguous bytes
  const int fw0 = WT ? ((wn * 128 + l32) >> 4) * 1024 + ((l32 & 15) + 16 * lh) * 16 : bswz(wn * 128 + l32, lh);
  const int fw1 = WT ? fw0 + 512 : bswz(wn * 128 + l32, 2 + lh);
  v16i acc[VB][TB];     // [vocab block][token block]
  v4i fx[2][2][TB], fw[2][2][VB];  // [register set][half step][block]
  auto read_one = [&](auto ksc, auto fb, int k) {  // fragment k (0..NRD-1) of step KS
    constexpr int KS = decltype(ksc)::value;
    const int8_t* as = a_st(ic<KS % kNSA>{});
    const int8_t* bs = b_st(ic<KS % kNSB>{});
    constexpr int f = decltype(fb)::value;
    if (k < 2 * TB) {
      const int h = k / TB, t = k % TB;
      fx[f][h][t] = *reinterpret_cast<const v4i*>(as + (h ? fx1 : fx0) + t * 32 * kBK);
    } else {
      const int h = (k - 2 * TB) / VB, t = (k - 2 * TB) % VB;
      fw[f][h][t] = *reinterpret_cast<const v4i*>(bs + (h ? fw1 : fw0) + t * 32 * kBK);
    }
  };
  auto mfma_one = [&](auto fb, auto first, int k) {  // MFMA k (0..NMF-1) of a step
    constexpr int f = decltype(fb)::value;
    const int h = k / (VB * TB), vi = (k / TB) % VB, ti = k % TB;
    acc[vi][ti] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
        fw[f][h][vi], fx[f][h][ti], (decltype(first)::value && h == 0) ? v16i{} : acc[vi][ti], 0, 0, 0);
  };
  // Step KS on register set KS % 2 (read during step KS - 1).  At its top the wave waits for its own
  // loads of step KS + 1: only those of steps KS + 2 .. KS + NS - 1 were issued after them (loads
  // complete in order; the previous tile's epilogue stores and atomics still in flight only lengthen
  // the wait), then one barrier makes every wave's loads of step KS + 1 visible and every wave's reads
  // of step KS complete, so the loads of step KS + NS may overwrite the stage step KS used.
  auto step = [&](const Tile& t, auto ksc) {
    constexpr int KS = decltype(ksc)::value;
    if constexpr (KS + 1 < kNK) {
      constexpr int later = (KS + NS - 1 < kNK - 1 ? KS + NS - 1 : kNK - 1) - (KS + 1);
      wait_vm<(later > 0 ? later : 0) * CPL>();
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    using fb = ic<KS & 1>;
    using nb = ic<(KS + 1) & 1>;
    using first = std::integral_constant<bool, KS == 0>;
#pragma unroll
    for (int k = 0; k < NMF; ++k) {
      mfma_one(fb{}, first{}, k);
      if constexpr (KS + 1 < kNK)
        if (k < NRD) read_one(ic<KS + 1>{}, nb{}, k);
      if constexpr (KS + NS < kNK)
        if (k >= NMF / 2 && k < NMF / 2 + CPL) issue_one(t, ic<KS + NS>{}, k - NMF / 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto prologue = [&](const Tile& t) {
    for_steps([&](auto sc) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) issue_one(t, sc, i);
    }, std::make_integer_sequence<int, NS>{});
  };
  int par = 0;
  Tile t = tile(j);
  issue_scales(t, 0);
  prologue(t);
  for (;;) {
    // step 0 of this tile has landed: only steps 1 .. NS - 1 of the wave's operand went out after it
    wait_vm<(NS - 1) * CPL>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < NRD; ++k) read_one(ic<0>{}, ic<0>{}, k);
    for_steps([&](auto sc) { step(t, sc); }, std::make_integer_sequence<int, kNK>{});
    // every wave is past the last step's barrier: no wave reads the ring any more
    j += nloc;
    const bool more = vt_of(j) < nvt;
    const Tile tn = more ? tile(j) : t;
    // The lane's indices are derived afresh from the thread id here: values computed before the K
    // loop and kept across it were spilled (the loop holds 224 of the 256 registers), and their
    // reloads, queued behind the next tile's loads, held the epilogue until those loads landed.
    // A read of the scale buffer issued after the next tile's scale loads waits for them (the
    // compiler cannot tell the parities apart).  One term: this tile's scales go into registers
    // first, then the next tile's scales and steps are requested (measured 1 % faster than
    // requesting the scales after the epilogue).  Two terms: the 64 registers this takes made the K
    // loop spill, so the epilogue reads the buffer and the next tile's scales are requested after it
    // (they are needed a whole tile later).
    const int et = opaque_tid(), ewm = (et >> 6) >> 1, ewn = (et >> 6) & 1, el32 = et & 31, elh = (et >> 5) & 1;
    constexpr int NTB = X2 ? TB / 2 : TB;
    constexpr bool kRegScales = !X2;
    auto wscale = [&](int vi, int jg) {
      return *reinterpret_cast<const float4*>(&sc_l[par][0][ewn * 128 + vi * 32 + 8 * jg + 4 * elh]);
    };
    float4 wsr[kRegScales ? VB : 1][4];
    float xsr[NTB], xs2[NTB];
#pragma unroll
    for (int tb = 0; tb < NTB; ++tb) {
      const int ti = X2 ? 2 * tb : tb;
      xsr[tb] = sc_l[par][1][ewm * TW + ti * 32 + el32];
      xs2[tb] = X2 ? sc_l[par][1][ewm * TW + (ti + 1) * 32 + el32] : 0.f;
    }
    if constexpr (kRegScales) {
#pragma unroll
      for (int vi = 0; vi < VB; ++vi)
#pragma unroll
        for (int jg = 0; jg < 4; ++jg) wsr[vi][jg] = wscale(vi, jg);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    if (more) {
      if constexpr (kRegScales) issue_scales(tn, par ^ 1);
      prologue(tn);
    }
    asm volatile("" ::: "memory");
    // Epilogue: lane l holds tokens r0 + wm*TW + 32 ti + l % 32 and, per token, vocab columns
    // cb + 32 vi + 8 (j / 4) + 4 (l / 32) + j % 4, visited in increasing order.  Each logit
    // (acc * xs) * ws is rounded to bf16 once (hardware round-to-nearest-even); the lane keeps the
    // first column of its largest value (-0 and +0 compare equal, as in the bf16 argmax), folds it
    // into a 32-bit key (order-preserving bf16 bits << 16 | 0xffff - column in the tile), exchanges
    // it with lane l ^ 32 and the other column wave through LDS, and the tile's best per row goes
    // out as one 64-bit atomic max.  Columns past V are skipped (nin: the lane's columns in range,
    // counted from its first; V % 16 == 0 keeps each group of 4 all in or all out).
    const int nin = d.V - t.v0 - (ewn * 128 + 4 * elh);
    // One term: token block ti is rows wm*TW + 32 ti of the tile.  Two terms: blocks 2b and 2b + 1
    // hold the two terms of the same 32 tokens (act_row), token wm*TW/2 + 32 b + l32 of the tile.
    const int tok0 = X2 ? t.r0 / 2 : t.r0;
    {
#pragma unroll
      for (int tb = 0; tb < NTB; ++tb) {
        const int ti = X2 ? 2 * tb : tb;
        const int rl = X2 ? ewm * (TW / 2) + tb * 32 + el32 : ewm * TW + ti * 32 + el32;  // token of the tile
        const int row = tok0 + rl;
        float bv = -__builtin_inff();
        int bi = 0;  // column offset from cbase
#pragma unroll
        for (int vi = 0; vi < VB; ++vi)
#pragma unroll
          for (int jg = 0; jg < 4; ++jg) {
            const int co = vi * 32 + 8 * jg;
            const int cl = ewn * 128 + co + 4 * elh;  // first of the lane's 4 columns, in the tile
            float4 w4;
            if constexpr (kRegScales) w4 = wsr[vi][jg];
            else w4 = wscale(vi, jg);
            const float wq[4] = {w4.x, w4.y, w4.z, w4.w};
            float lg[4];
            const bool in = co < nin;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if constexpr (X2)
                lg[q] = rbf_hw(__builtin_fmaf((float)acc[vi][ti][4 * jg + q], xsr[tb],
                                                  (float)acc[vi][ti + 1][4 * jg + q] * xs2[tb]) * wq[q]);
              else
                lg[q] = rbf_hw(((float)acc[vi][ti][4 * jg + q] * xsr[tb]) * wq[q]);
              if (in && lg[q] > bv) bv = lg[q], bi = co + q;
            }
            if constexpr (STORE == 1)
              if (row < d.R && in)
                *reinterpret_cast<uint2*>(d.logits + (size_t)row * d.V + t.v0 + cl) =
                    make_uint2((__float_as_uint(lg[0]) >> 16) | (__float_as_uint(lg[1]) & 0xffff0000u),
                               (__float_as_uint(lg[2]) >> 16) | (__float_as_uint(lg[3]) & 0xffff0000u));
            if constexpr (STORE == 2)
              if (row < d.R && in)
                *reinterpret_cast<float4*>(d.logits32 + (size_t)row * d.V + t.v0 + cl) =
                    make_float4(lg[0], lg[1], lg[2], lg[3]);
          }
        uint32_t b16 = __float_as_uint(bv + 0.f) >> 16;
        b16 = (b16 & 0x8000u) ? (~b16 & 0xffffu) : (b16 | 0x8000u);
        uint32_t best = (b16 << 16) | (0xffffu - (uint32_t)(ewn * 128 + 4 * elh + bi));
        // lane l and l ^ 32 exchange by v_permlane32_swap (a shuffle would keep the lane id live,
        // or spilled, across the K loop)
        const auto bsw = __builtin_amdgcn_permlane32_swap(best, best, false, false);
        best = max(bsw[0], bsw[1]);
        if (elh == 0) rkey[ewn][rl] = best;
      }
    }
    // LDS-only barrier for the key exchange: a full __syncthreads also waits for the next tile's
    // loads in flight
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // two terms: every wave has read this tile's scales, the next tile's may now be requested
    if constexpr (!kRegScales)
      if (more) issue_scales(tn, par ^ 1);
    if (et < (X2 ? kBM / 2 : kBM) && tok0 + et < d.R) {
      const uint32_t k = max(rkey[0][et], rkey[1][et]);
      const uint32_t col = (uint32_t)t.v0 + (0xffffu - (k & 0xffffu));
      atomicMax(&d.keys[tok0 + et], ((unsigned long long)(k >> 16) << 32) | (unsigned long long)(0xffffffffu - col));
    }
    if (!more) break;
    t = tn;
    par ^= 1;
  }
}

// The GEMM's LDS: kNSA activation and kNSB weight stages, the scales and the row keys
#define LMH_GEMM_LDS                                                                                  \
  __shared__ __align__(1024) int8_t a_s0[kBM * kBK], a_s1[kBM * kBK], a_s2[kBM * kBK];               \
  __shared__ __align__(1024) int8_t b_s0[kBN * kBK], b_s1[kBN * kBK], b_s2[kBN * kBK], b_s3[kBN * kBK], \
      b_s4[kBN * kBK], b_s5[kBN * kBK];                                                               \
  __shared__ __align__(16) float sc_l[2][2][kBN];                                                     \
  __shared__ uint32_t rkey[2][kBM];                                                                   \
  static_assert(kNSA == 3 && kNSB == 6, "the stage arrays above");                                   \
  const LmhLds L{{a_s0, a_s1, a_s2}, {b_s0, b_s1, b_s2, b_s3, b_s4, b_s5}, sc_l, rkey};

// WT: the weights in the tile order (q36_lmhead_args.wq_t) instead of row-major
template <bool X2, bool WT>
__global__ __launch_bounds__(64 * kLmhWaves) __attribute__((amdgpu_waves_per_eu(kLmhWaves / 4, kLmhWaves / 4))) void
lmh_gemm_kernel(LmhDev d) {
  LMH_GEMM_LDS
  if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) < kLmhWaves / 2)
    lmh_gemm_body<0, X2, kLmhWaves, 0, WT>(d, L);
  else
    lmh_gemm_body<0, X2, kLmhWaves, 1, WT>(d, L);
}
// the same with the logits written out (F32: as fp32)
template <bool X2, bool F32, bool WT>
__global__ __launch_bounds__(64 * kLmhWaves) __attribute__((amdgpu_waves_per_eu(kLmhWaves / 4, kLmhWaves / 4))) void
lmh_gemm_logits_kernel(LmhDev d) {
  LMH_GEMM_LDS
  if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) < kLmhWaves / 2)
    lmh_gemm_body<F32 ? 2 : 1, X2, kLmhWaves, 0, WT>(d, L);
  else
    lmh_gemm_body<F32 ? 2 : 1, X2, kLmhWaves, 1, WT>(d, L);
}

__global__ __launch_bounds__(256) void lmh_ids_kernel(LmhDev d) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r < d.R) d.ids[r] = (int32_t)(0xffffffffu - (uint32_t)(d.keys[r] & 0xffffffffull));
}

int lmh_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    cached[dev] = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus >= 8
                      ? cus : 256;
  }
  return cached[dev];
}

struct LmhWs {
  size_t xq, xs, keys, total;
};
LmhWs lmh_ws(int R) {
  LmhWs w;
  size_t o = 0;
  auto take = [&](size_t b) {
    size_t r = o;
    o = align_up(o + b, 256);
    return r;
  };
  const size_t rows = (size_t)act_rows(R, 1);  // room for two activation terms, whatever the mode
  w.xq = take(rows * kLH);
  w.xs = take(sizeof(float) * rows);
  w.keys = take(sizeof(unsigned long long) * (size_t)R);
  w.total = o;
  return w;
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" size_t q36_lmhead_workspace_bytes(int32_t R) { return lmh_ws(R).total; }

extern "C" int q36_lmhead_argmax(const q36_lmhead_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_lmhead_argmax: null args");
  Q36_REQUIRE(a->H == kLH, "q36_lmhead_argmax: H=%d unsupported (this build is specialised to 2048)", a->H);
  Q36_REQUIRE(a->R >= 1 && a->R <= (1 << 20), "q36_lmhead_argmax: R=%d out of range", a->R);
  Q36_REQUIRE(a->V >= 16 && a->V % 16 == 0, "q36_lmhead_argmax: V=%d must be a positive multiple of 16", a->V);
  Q36_REQUIRE(a->mode == Q36_LMH_W8A8 || a->mode == Q36_LMH_W8A8X2 || a->mode == Q36_LMH_W8A16,
              "q36_lmhead_argmax: mode %d unknown", a->mode);
  Q36_REQUIRE(a->mode != Q36_LMH_W8A16 || (a->R <= 64 && a->V % 32 == 0),
              "q36_lmhead_argmax: the W8A16 form serves R <= 64 rows and V a multiple of 32 (R=%d V=%d)", a->R, a->V);
  Q36_REQUIRE(a->h && (a->wq || a->wq_t) && a->ws && a->ids && a->workspace,
              "q36_lmhead_argmax: a required pointer is null");
  Q36_REQUIRE(aligned16(a->h) && aligned16(a->wq) && aligned16(a->ws) && aligned16(a->norm_w) && aligned16(a->wq_t) &&
                  (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_lmhead_argmax: h, wq, ws, norm_w must be 16-byte and workspace 256-byte aligned");
  const LmhWs L = lmh_ws(a->R);
  Q36_REQUIRE(a->workspace_bytes >= L.total, "q36_lmhead_argmax: workspace of %zu bytes < %zu required",
              a->workspace_bytes, L.total);
  char* ws = static_cast<char*>(a->workspace);
  const int x2 = a->mode == Q36_LMH_W8A8X2, w16 = a->mode == Q36_LMH_W8A16;
  Q36_REQUIRE(!a->logits_f32 || a->logits, "q36_lmhead_argmax: logits_f32 set without a logits buffer");
  Q36_REQUIRE(aligned16(a->logits), "q36_lmhead_argmax: logits must be 16-byte aligned");
  const bool f32 = a->logits && a->logits_f32;
  LmhDev d{a->R, a->V, act_rows(a->R, x2), x2, w16, static_cast<const uint16_t*>(a->h), static_cast<const uint16_t*>(a->norm_w), a->eps,
           a->wq_t ? a->wq_t : static_cast<const int8_t*>(a->wq), a->ws, a->ids, f32 ? nullptr : static_cast<uint16_t*>(a->logits),
           f32 ? static_cast<float*>(a->logits) : nullptr, reinterpret_cast<int8_t*>(ws + L.xq), reinterpret_cast<float*>(ws + L.xs),
           reinterpret_cast<unsigned long long*>(ws + L.keys)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  lmh_prep_kernel<<<a->R, 64, 0, st>>>(d);
  if (w16) {
    W16Dev g{};
    g.T = a->R;
    g.N = a->V;
    g.K = kLH;
    g.x = reinterpret_cast<const uint16_t*>(d.xq);  // the prep's bf16 rows (2 R * H bytes fit in xq)
    // the codes in the tile order when the caller keeps that copy: each piece the kernel loads at once
    // is then 1 KB contiguous (1 row 77 -> 61 us, 32 rows 115 -> 79 us at V = 151936)
    g.q = d.wq;
    g.tiled = a->wq_t != nullptr;
    g.ws = d.ws;
    g.logits = d.logits;
    g.logits32 = d.logits32;
    g.keys = d.keys;
    launch_w8a16(g, 0, st);
    lmh_ids_kernel<<<(a->R + 255) / 256, 256, 0, st>>>(d);
    return check_launch("q36_lmhead_argmax");
  }
  const int nvt = (a->V + kBN - 1) / kBN, nrt = (d.Rs + kBM - 1) / kBM;
  // persistent: one workgroup per CU (a multiple of 8, one XCD in eight), never more than the
  // busiest XCD's tiles
  const int ngrp = lmh_groups(nrt), vstep = 8 / ngrp;
  const int blocks = 8 * std::max(1, std::min(lmh_cus() / 8, ((nvt + vstep - 1) / vstep) * (nrt / ngrp)));
  // the weights' tile order: their DMA reads 1 KB contiguous pieces (2048 rows 697-702 -> 674-683 us,
  // 256 rows two terms 171-178 -> 164-166 us against the row-major codes)
  auto go = [&](auto wt) {
    constexpr bool WT = decltype(wt)::value;
    if (d.logits32 && x2)
      lmh_gemm_logits_kernel<true, true, WT><<<blocks, 64 * kLmhWaves, 0, st>>>(d);
    else if (d.logits32)
      lmh_gemm_logits_kernel<false, true, WT><<<blocks, 64 * kLmhWaves, 0, st>>>(d);
    else if (d.logits && x2)
      lmh_gemm_logits_kernel<true, false, WT><<<blocks, 64 * kLmhWaves, 0, st>>>(d);
    else if (d.logits)
      lmh_gemm_logits_kernel<false, false, WT><<<blocks, 64 * kLmhWaves, 0, st>>>(d);
    else if (x2)
      lmh_gemm_kernel<true, WT><<<blocks, 64 * kLmhWaves, 0, st>>>(d);
    else
      lmh_gemm_kernel<false, WT><<<blocks, 64 * kLmhWaves, 0, st>>>(d);
  };
  if (a->wq_t)
    go(std::true_type{});
  else
    go(std::false_type{});
  lmh_ids_kernel<<<(a->R + 255) / 256, 256, 0, st>>>(d);
  return check_launch("q36_lmhead_argmax");
}
