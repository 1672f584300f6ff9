// Decode / verify attention for gfx950 over an e4m3 KV cache: 16 query heads grouped onto 2 KV
// heads of 256 dims, up to 4 query tokens per request (the verify draft; 1 for plain decode) with
// the causal rule among them, one-token pages through a page table, split over the keys.
//
// Reference behaviour (R = qwen36_nodes_kb34, L = R/qwen36_layer): L/qk_attn_verify.cu:354-760
// (attn_verify_kernel: q -> e4m3, scores of e4m3 q and k, base-2 online softmax, P rounded to
// f16 for P V with V widened to f16, the split partials and their combine), L/attn_fused.py:110-124
// (split count min(64, CUs / (requests * KV heads))).  The new tokens' K/V go into the cache at
// their slots first (the reference writes them there as well).  The output is the normalised
// attention bf16(o / l); the o_proj applies the sigmoid gate.
//
// Kernels:
//   kv_scatter      the new tokens' e4m3 K and V rows into the cache slots out_loc[t].
//   decode_split    workgroup = (split, KV head, request), 4 independent waves; each wave streams
//                   its own contiguous run of 32-key steps for the group's 8 query heads x NT tokens
//                   (16 or 32 query rows) with its own running max / weight sum / output, and the
//                   four are merged once at the end.  Scores S^T = K Q^T: e4m3 16x16x128 MFMA with
//                   the keys as operand A straight from the cache (registers) and the e4m3 query
//                   fragments as operand B, so a lane holds one query row: the row max needs two
//                   cross-lane steps and the output rescale is one factor per lane.  O^T += V^T P^T:
//                   f16 16x16x32 MFMA, V^T read from LDS with the transpose read (V rows staged by
//                   buffer DMA in the key order the lane's weights are in), P^T the lane's own
//                   weights rounded to f16.  Keys, values and page-table entries stream through a
//                   per-wave pipeline (2 stages at two waves a SIMD for one row tile, 4 at one wave
//                   a SIMD for two) with no workgroup barrier; the output is rescaled only
//                   when a row max grows by more than 2^8 (weights up to 2^8 are exact in f16).
//   decode_combine  the splits' partials weighted by exp2(m_s - M) / L (with one split the split
//                   kernel writes the output itself).
#include <math.h>

#include <type_traits>

#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int kQH = 16, kKVH = 2, kDD = 256, kGQ = kQH / kKVH, kDNT = 4, kDRows = kGQ * kDNT;
constexpr int kST = 32;              // keys per wave step
// NS (kernel template): key / value stages per wave (steps in flight + 1); the page-table entries run
// 2 NS steps ahead, so an entry's DMA is older than every key and value load a wait leaves in flight
constexpr int kPTR = 8;              // page-table ring entries per wave (one step each)
// The two forms' shapes (alternating builds on one box, three rounds): the one-row-tile form (decode,
// NT <= 2) with 2 stages fits 224 registers and 77 KB of LDS, so two workgroups share a CU (two waves
// a SIMD): decode 189.9 -> 182.7 us against 3 stages at one wave a SIMD; the two-row-tile form
// (verify) keeps one wave a SIMD and runs 4 stages (456 registers, 145 KB): 62.0 -> 60.6 us.
constexpr int kDecNS1 = 2, kDecWPE1 = 2, kDecNS2 = 4;
constexpr int kVG = 4 * kDD + 64;    // a group of 4 value rows in LDS (64 bytes of padding)
constexpr int kVW = 8 * kVG;         // one wave's 32 value rows
constexpr int kVS = 4 * kVW;         // one stage of the four waves' value rows
constexpr float kLazy = 8.f;
// Key and value reads carry the non-temporal cache policy (nt): each row is read once per call, and
// inside the hybrid node (after a GDN verify has left ~0.5 GB of snapshot writes dirty in the
// caches) the plain reads ran at half speed, evicting that data; measured 111 -> 63 us per call.
constexpr int kKVAux = 2;         // rescale when a row max grows past the reference by 2^8
static_assert((kPTR & (kPTR - 1)) == 0, "page-table ring");
static_assert(kVS >= 2 * 16 * kDD * 4, "a stage holds two waves' fp32 output of one row tile at the merge");

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

struct DecodeDev {
  int B, NT, splits, pt_stride;
  const uint16_t* q;        // bf16 [B*NT, 16, 256]
  const uint8_t* kc;        // e4m3 [slots, 2, 256]
  const uint8_t* vc;
  int64_t kv_bytes;         // bytes of each cache
  const int32_t* pt;        // [B, pt_stride]
  const int32_t* seqlens;   // [B], new tokens included
  float scale_log2;
  float* ws_o;              // [B*2*splits][32][256] unnormalised partial outputs
  float* ws_ml;             // [B*2*splits][2][32]: running max (base 2) and weight sum per row
  uint16_t* out;            // bf16 [B*NT, 16, 256]
  const uint16_t* gate;     // bf16 [B*NT, 16 * 256] or null: with oq, the o_proj's quantized input
  uint8_t* oq;              // e4m3 [B*NT, 16 * 256] of bf16(out * sigmoid(gate)) per 128-group
  float* oqs;               // [B*NT, 32] group scales
};

// The output's 4 values at dims 4c .. 4c + 3 of row (token tok, head) after the bf16 store: the o_proj
// input bf16(o * sigmoid(gate)) in e4m3 per 128-channel group (32 neighbouring lanes of one wave hold
// a group), the same arithmetic as the o_proj's own quantization of the bf16 output.
__device__ __forceinline__ void gated_e4m3(const DecodeDev& d, int tok, int head, int c, uint32_t o01, uint32_t o23) {
  const size_t at = (size_t)tok * (kQH * kDD) + head * kDD + 4 * c;
  const uint2 gv = *reinterpret_cast<const uint2*>(d.gate + at);
  float f[4] = {rbf(bf_lo(o01) * sigmoid_q(bf_lo(gv.x))), rbf(bf_hi(o01) * sigmoid_q(bf_hi(gv.x))),
                rbf(bf_lo(o23) * sigmoid_q(bf_lo(gv.y))), rbf(bf_hi(o23) * sigmoid_q(bf_hi(gv.y)))};
  float m = fmaxf(fmaxf(fabsf(f[0]), fabsf(f[1])), fmaxf(fabsf(f[2]), fabsf(f[3])));
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  const float inv = m > 0.f ? 448.f / m : 0.f;
  *reinterpret_cast<uint32_t*>(d.oq + at) = f2e4m3x2_hw(f[0] * inv, f[1] * inv) | (f2e4m3x2_hw(f[2] * inv, f[3] * inv) << 16);
  if ((c & 31) == 0) d.oqs[(size_t)tok * (kQH * kDD / 128) + head * 2 + c / 32] = m / 448.f;
}

__device__ __forceinline__ v4f mfma_e4m3(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
__device__ __forceinline__ v8i cat8d(v4i a, v4i b) {
  v8i r = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return r;
}
// 8 e4m3 codes (two words) -> 8 f16 (every e4m3 value is an f16 value: exact at scale 1)
__device__ __forceinline__ v8h widen8(int w0, int w1) {
  const v2h a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.f, false);
  const v2h b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.f, true);
  const v2h c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.f, false);
  const v2h e = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.f, true);
  return v8h{a.x, a.y, b.x, b.y, c.x, c.y, e.x, e.y};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) uint8_t*)p);
}
// LDS read by asm: the compiler counts the buffer DMA into the same array as a pending write and
// would wait for every load in flight; the caller waits (lgkmcnt) before using the value.
__device__ __forceinline__ int lds_ld32_asm(const void* p) {
  int v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(lds_addr(p)) : "memory");
  return v;
}

__global__ __launch_bounds__(256) void kv_scatter_kernel(const uint8_t* k8, const uint8_t* v8, const int64_t* loc, int T,
                                                        int64_t num_slots, uint8_t* kc, uint8_t* vc) {
  // thread: 16 bytes of one token's K or V row pair (2 heads x 256 bytes = 32 pieces per row);
  // a slot outside the cache is skipped
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= T * 64) return;
  const int t = i / 64, piece = i % 64, isv = piece >= 32, p = piece & 31;
  if (loc[t] < 0 || loc[t] >= num_slots) return;
  const size_t src = (size_t)t * (kKVH * kDD) + 16 * p, dst = (size_t)loc[t] * (kKVH * kDD) + 16 * p;
  *reinterpret_cast<v4i*>((isv ? vc : kc) + dst) = *reinterpret_cast<const v4i*>((isv ? v8 : k8) + src);
}

template <int RT, int NS, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void decode_split_kernel(DecodeDev d) {
  constexpr int PTD = 2 * NS;
  static_assert(NS >= 2 && NS <= 4, "the prologue and the step loop are written out for 2 to 4 stages");
  static_assert(kPTR >= PTD, "the ring holds the entries of every step in flight");
  // one object per stage: the compiler then sees that a stage's DMA does not write what another
  // stage's reads read (in one array it waits for every DMA in flight before each read)
  __shared__ __align__(16) uint8_t vs0[kVS];
  __shared__ __align__(16) uint8_t vs1[kVS];
  __shared__ __align__(16) uint8_t vs2[NS >= 3 ? kVS : 16];
  __shared__ __align__(16) uint8_t vs3[NS >= 4 ? kVS : 16];
  __shared__ __align__(16) int32_t ptl[4][kPTR][64];
  __shared__ float mw[4][kDRows], lwv[4][kDRows], rowM[kDRows], rowL[kDRows];
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z, S = d.splits;
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
  const int NT = d.NT, nk = d.seqlens[b], npre = nk - NT;
  // steps of the request, the split's share (contiguous), the wave's share of that
  const int steps = nk > 0 ? (nk + kST - 1) / kST : 0, per = steps / S, rem = steps % S;
  const int st0 = s * per + min(s, rem), nst = per + (s < rem ? 1 : 0);
  const int ws0 = st0 + (wave * nst) / 4, ws1 = st0 + ((wave + 1) * nst) / 4;
  const int kbeg = ws0 * kST, kend = min(ws1 * kST, nk);  // the wave's keys [kbeg, kend)
  const int npad = (ws1 - ws0 + NS - 1) / NS * NS;        // steps run (a multiple of the stages)
  const int kfull = min(kend - 1, npre);  // keys up to here are visible to every query row
  const int grp = (b * kKVH + h) * S + s;
  // query fragments (score operand B): column 16 rt + l16 = query row (token row / 8, head
  // h * 8 + row % 8), dims 128 kb + 32 lg .. +31 rounded to e4m3; rows of tokens past NT are zero
  v8i qb[RT][2];
  int lim[RT];  // the row's last visible key (-1: none): causal among the new tokens, wave range
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = 16 * rt + l16, t = row >> 3;
    lim[rt] = t < NT ? min(kend - 1, npre + t) : -1;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      int w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (t < NT) {
        const uint16_t* src = d.q + (((size_t)b * NT + t) * kQH + h * kGQ + (row & 7)) * kDD + 128 * kb + 32 * lg;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const v4i raw = *reinterpret_cast<const v4i*>(src + 8 * c);
#pragma unroll
          for (int j = 0; j < 2; ++j)
            w[2 * c + j] = (int)(f2e4m3x2_hw(bf_lo((uint32_t)raw[2 * j]), bf_hi((uint32_t)raw[2 * j])) |
                                 (f2e4m3x2_hw(bf_lo((uint32_t)raw[2 * j + 1]), bf_hi((uint32_t)raw[2 * j + 1])) << 16));
        }
      }
      qb[rt][kb] = v8i{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]};
    }
  }
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)d.kc, (short)0, (int)d.kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)d.vc, (short)0, (int)d.kv_bytes, 0x00020000);
  // the request's page-table row through a bounded buffer (an entry past the row reads as slot 0)
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(d.pt + (size_t)b * d.pt_stride), (short)0, 4 * d.pt_stride, 0x00020000);
  int32_t* ring = &ptl[wave][0][0];
  // Page-table entries of step j into ring entry j % 8 (lanes 32..63 repeat lanes 0..31).  Keys past
  // the wave's range take the slot of its last key: their loads are repeats that stay in L2, their
  // scores are masked and their values are real cache rows (finite), so 0 * V stays 0.
  auto pt_dma = [&](int j) {
    const int key = max(min(kbeg + kST * j + (lane & 31), kend - 1), 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(prs, ring + (j & (kPTR - 1)) * 64, 4, 4 * key, 0, 0, 0);
  };
  // Step j into stage Q: the 32 keys' rows as score operand A (kf[Q][kt]: key 16 kt + l16, dims
  // 128 half + 32 lg ..), and the 32 value rows into the wave's LDS rows: DMA call m writes rows
  // 4 m .. 4 m + 3 with key 16 (m & 1) + 4 (m >> 1) + (row % 4), so rows 8 g .. 8 g + 7 hold keys
  // 4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3 (the order of lane group g's weights).  Row group m
  // (one DMA call, 1 KB) starts at m * (1 KB + 64 B) and 16-byte piece p of its row i sits at position
  // p ^ i: the eight rows a lane group reads for one dim tile fall on eight distinct 16-byte bank
  // slots, and only the low two bits of a piece's position depend on the lane.
  v4i kf[NS][2][4];
  auto stage = [&](auto qc) -> uint8_t* {
    constexpr int Q = decltype(qc)::value;
    return (Q == 0 ? vs0 : Q == 1 ? vs1 : Q == 2 ? vs2 : vs3) + wave * kVW;
  };
  auto fetch = [&](int j, auto qc) {
    constexpr int Q = decltype(qc)::value;
    const int32_t* e = ring + (j & (kPTR - 1)) * 64;
    int ks0 = lds_ld32_asm(e + l16), ks1 = lds_ld32_asm(e + 16 + l16);
    int vsl0 = lds_ld32_asm(e + lg), vsl1 = lds_ld32_asm(e + 16 + lg), vsl2 = lds_ld32_asm(e + 4 + lg),
        vsl3 = lds_ld32_asm(e + 20 + lg), vsl4 = lds_ld32_asm(e + 8 + lg), vsl5 = lds_ld32_asm(e + 24 + lg),
        vsl6 = lds_ld32_asm(e + 12 + lg), vsl7 = lds_ld32_asm(e + 28 + lg);
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(ks0), "+v"(ks1), "+v"(vsl0), "+v"(vsl1), "+v"(vsl2), "+v"(vsl3), "+v"(vsl4), "+v"(vsl5),
                   "+v"(vsl6), "+v"(vsl7)::"memory");
    const int kb0 = (ks0 * kKVH + h) * kDD + 32 * lg, kb1 = (ks1 * kKVH + h) * kDD + 32 * lg;
    kf[Q][0][0] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb0, 0, kKVAux);
    kf[Q][0][1] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb0 + 16, 0, kKVAux);
    kf[Q][0][2] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb0 + 128, 0, kKVAux);
    kf[Q][0][3] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb0 + 144, 0, kKVAux);
    kf[Q][1][0] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb1, 0, kKVAux);
    kf[Q][1][1] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb1 + 16, 0, kKVAux);
    kf[Q][1][2] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb1 + 128, 0, kKVAux);
    kf[Q][1][3] = __builtin_amdgcn_raw_buffer_load_b128(krs, kb1 + 144, 0, kKVAux);
    uint8_t* vb = stage(qc);
    const int vsl[8] = {vsl0, vsl1, vsl2, vsl3, vsl4, vsl5, vsl6, vsl7};
#pragma unroll
    for (int m = 0; m < 8; ++m)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, vb + m * kVG, 16, (vsl[m] * kKVH + h) * kDD + 16 * (l16 ^ lg), 0, 0,
                                               kKVAux);
  };
  // per-lane state: running max (base 2) of query row 16 rt + l16, the lane's share of its weight
  // sum, and O^T (lane: row 16 rt + l16, dims 16 dt + 4 lg + r)
  float m[RT], l[RT];
  v4f o[RT][16];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m[rt] = -1e30f;
    l[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) o[rt][dt] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  // lane's value-read address: row 8 lg + l16 / 2 = group 2 lg + l16 / 8, row (l16 / 2) % 4 in it,
  // half l16 % 2; dim tile dt adds 64 (dt / 4) + 16 ((dt % 4) ^ row)
  const int vri = (l16 >> 1) & 3, vbase = (2 * lg + (l16 >> 3)) * kVG + vri * kDD + 8 * (l16 & 1);
  auto compute = [&](int j, auto qc) {
    constexpr int Q = decltype(qc)::value;
    // this stage's values have landed (newer: NS page-table DMAs and NS - 1 steps' requests); all
    // sixteen transposed reads are issued now and complete under the scores and the softmax
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NS + (NS - 1) * 16) : "memory");
    const uint8_t* vb = stage(qc) + vbase;
    v2i vraw[16];
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
      vraw[dt] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (__attribute__((address_space(3))) v2i*)(vb + 64 * (dt >> 2) + 16 * ((dt & 3) ^ vri)));
    v4f sc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        sc[rt][kt] = mfma_e4m3(cat8d(kf[Q][kt][0], kf[Q][kt][1]), qb[rt][0], v4f{0.f, 0.f, 0.f, 0.f});
        sc[rt][kt] = mfma_e4m3(cat8d(kf[Q][kt][2], kf[Q][kt][3]), qb[rt][1], sc[rt][kt]);
      }
    // Softmax weights.  Only a step with keys some query row must not see (the causal edge, the end
    // of the wave's range) masks them to -inf; rows of tokens past NT have zero queries, stay finite
    // and are never written.  The running max starts at a finite -1e30, so exp2 of a masked score
    // is 0 with no special case.  Scores are raw MFMA sums, scaled inside the exponent's fma.
    const float sl2 = d.scale_log2;
    float sv[RT][8];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[rt][i] = sc[rt][i >> 2][i & 3];
    if (kbeg + kST * j + kST - 1 > kfull) {  // uniform over the wave
      const int key0 = kbeg + kST * j + 4 * lg;  // lane's keys: key0 + 16 kt + r
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (key0 + 16 * (i >> 2) + (i & 3) > lim[rt]) sv[rt][i] = -INFINITY;
    }
    float tmax[RT];
    bool need = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float mx = fmaxf(fmaxf(fmaxf(sv[rt][0], sv[rt][1]), fmaxf(sv[rt][2], sv[rt][3])),
                       fmaxf(fmaxf(sv[rt][4], sv[rt][5]), fmaxf(sv[rt][6], sv[rt][7])));
      // across the four lane groups (rows of 16 lanes) that hold the same query row
      const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
      const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      tmax[rt] = fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1])) * sl2;
      need |= tmax[rt] > m[rt] + kLazy;
    }
    // Rare (a row max grew past its reference by 2^8), and marked so: with the branch at its default
    // weight the compiler placed the output accumulators' AGPR -> VGPR copies for it above the branch,
    // some 120 copies every step.
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(need) != 0, 0)) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float mn = fmaxf(m[rt], tmax[rt]);
        const float al = __builtin_amdgcn_exp2f(m[rt] - mn);
        m[rt] = mn;
        l[rt] *= al;
        // four dim tiles at a time: the accumulators live in AGPRs and go through VGPRs to scale
#pragma unroll
        for (int dg = 0; dg < 16; dg += 4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // taken from the AGPRs here (an opaque redefinition: a VGPR copy made before the branch
            // would be stale), scaled, and put back (no VGPR copy across the join)
            asm volatile("" : "+a"(o[rt][dg + i]));
            o[rt][dg + i] *= al;
            asm volatile("" : "+a"(o[rt][dg + i]));
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    v8h pb[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[rt][i], sl2, -m[rt]));
        ps += p;
        pb[rt][i] = (_Float16)p;
      }
      l[rt] += ps;
    }
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const v8h vv = widen8(vraw[dt].x, vraw[dt].y);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, pb[rt], o[rt][dt], 0, 0, 0);
    }
  };
  // prologue: entries of steps 0 .. PTD - NS, then the first NS - 1 steps' requests, each
  // followed by the page-table DMA PTD steps ahead (the order every step keeps)
  for (int j = 0; j <= PTD - NS; ++j) pt_dma(j);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  fetch(0, std::integral_constant<int, 0>{});
  pt_dma(PTD - NS + 1);
  if constexpr (NS >= 3) {
    fetch(1, std::integral_constant<int, 1>{});
    pt_dma(PTD - NS + 2);
  }
  if constexpr (NS == 4) {
    fetch(2, std::integral_constant<int, 2>{});
    pt_dma(PTD - NS + 3);
  }
  auto step = [&](int j, auto qc) {
    constexpr int Q = decltype(qc)::value;
    fetch(j + NS - 1, std::integral_constant<int, (Q + NS - 1) % NS>{});
    pt_dma(j + PTD);
    __builtin_amdgcn_sched_barrier(0);  // requests first: the compute below waits for step j's data
    compute(j, qc);
    __builtin_amdgcn_sched_barrier(0);  // and the next step's requests stay after it
  };
  for (int j = 0; j < npad; j += NS) {
    step(j, std::integral_constant<int, 0>{});
    step(j + 1, std::integral_constant<int, 1>{});
    if constexpr (NS >= 3) step(j + 2, std::integral_constant<int, 2>{});
    if constexpr (NS == 4) step(j + 3, std::integral_constant<int, 3>{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // merge the four waves: M = max of the waves' maxima, L = sum of exp2(m_w - M) l_w; per row
  // tile, each wave's output scaled by exp2(m - M) into its own 16 KB (fp32 [16 rows][256], 16-byte
  // piece c of row r at c ^ r), then summed in wave order into this split's partial (or, with one
  // split, normalised by L into the bf16 output)
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float lt = l[rt] + __shfl_xor(l[rt], 16);
    lt = lt + __shfl_xor(lt, 32);
    if (lg == 0) {
      mw[wave][16 * rt + l16] = m[rt];
      lwv[wave][16 * rt + l16] = lt;
    }
  }
  __syncthreads();
  if (tid < kDRows) {
    const int row = tid;
    float M = -1e30f, L = 0.f;
    if (row < 16 * RT) {
      M = fmaxf(fmaxf(mw[0][row], mw[1][row]), fmaxf(mw[2][row], mw[3][row]));
#pragma unroll
      for (int w = 0; w < 4; ++w) L += __builtin_amdgcn_exp2f(mw[w][row] - M) * lwv[w][row];
    }
    rowM[row] = M;
    rowL[row] = L;
    if (S > 1) {
      d.ws_ml[(size_t)grp * 2 * kDRows + row] = M;
      d.ws_ml[(size_t)grp * 2 * kDRows + kDRows + row] = L;
    }
  }
  __syncthreads();
  float* ob = reinterpret_cast<float*>((wave < 2 ? vs0 : vs1) + (wave & 1) * (kVS / 2));
  const float* o0 = reinterpret_cast<const float*>(vs0);
  const float* o1 = reinterpret_cast<const float*>(vs0 + kVS / 2);
  const float* o2 = reinterpret_cast<const float*>(vs1);
  const float* o3 = reinterpret_cast<const float*>(vs1 + kVS / 2);
  float* wo = d.ws_o + (size_t)grp * kDRows * kDD;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (rt > 0) __syncthreads();  // the previous tile's sums have read the buffers
    const float M = rowM[16 * rt + l16];
    const float f = __builtin_amdgcn_exp2f(m[rt] - M);
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
      *reinterpret_cast<v4f*>(ob + l16 * kDD + 4 * ((4 * dt + lg) ^ l16)) = o[rt][dt] * f;
    __syncthreads();
    const int rows = min(16, NT * kGQ - 16 * rt);
    for (int e = tid; e < rows * (kDD / 4); e += 256) {
      const int r = e / (kDD / 4), c = e % (kDD / 4), at = r * kDD + 4 * (c ^ r), row = 16 * rt + r;
      const v4f a = (*reinterpret_cast<const v4f*>(o0 + at) + *reinterpret_cast<const v4f*>(o1 + at)) +
                    (*reinterpret_cast<const v4f*>(o2 + at) + *reinterpret_cast<const v4f*>(o3 + at));
      if (S > 1) {
        *reinterpret_cast<v4f*>(wo + row * kDD + 4 * c) = a;
      } else {
        const float L = rowL[row], il = L > 0.f ? 1.f / L : 0.f;
        uint16_t* dst = d.out + (((size_t)b * NT + (row >> 3)) * kQH + h * kGQ + (row & 7)) * kDD + 4 * c;
        const uint32_t o01 = pack_bf2(a[0] * il, a[1] * il), o23 = pack_bf2(a[2] * il, a[3] * il);
        *reinterpret_cast<uint2*>(dst) = make_uint2(o01, o23);
        // a wave holds one row (rows * 64 threads, whole waves): its two 128-groups are its lane halves
        if (d.oq) gated_e4m3(d, b * NT + (row >> 3), h * kGQ + (row & 7), c, o01, o23);
      }
    }
  }
}

// out = bf16(sum_s exp2(m_s - M) o_s / L), L = sum_s exp2(m_s - M) l_s, splits in order; one
// thread per 4 dims of one query row (rows b, t, head over the batch)
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeDev d) {
  const int e = blockIdx.x * 256 + threadIdx.x, NT = d.NT, S = d.splits;
  if (e >= d.B * NT * kQH * (kDD / 4)) return;
  const int c = e % (kDD / 4), qr = e / (kDD / 4);  // qr = (b * NT + t) * 16 + head
  const int head = qr % kQH, bt = qr / kQH, t = bt % NT, b = bt / NT;
  const int h = head / kGQ, gr = t * kGQ + head % kGQ, g0 = (b * kKVH + h) * S;
  float M = -1e30f;  // the split kernel's maxima are finite (-1e30 for a split with no visible key)
  for (int s = 0; s < S; ++s) M = fmaxf(M, d.ws_ml[(size_t)(g0 + s) * 2 * kDRows + gr]);
  float L = 0.f;
  v4f a = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; ++s) {
    const float ms = d.ws_ml[(size_t)(g0 + s) * 2 * kDRows + gr];
    const float w = exp2f(ms - M);
    L += w * d.ws_ml[(size_t)(g0 + s) * 2 * kDRows + kDRows + gr];
    a += w * *reinterpret_cast<const v4f*>(d.ws_o + ((size_t)(g0 + s) * kDRows + gr) * kDD + 4 * c);
  }
  const float il = L > 0.f ? 1.f / L : 0.f;
  const uint32_t o01 = pack_bf2(a[0] * il, a[1] * il), o23 = pack_bf2(a[2] * il, a[3] * il);
  *reinterpret_cast<uint2*>(d.out + (size_t)qr * kDD + 4 * c) = make_uint2(o01, o23);
  // 64 consecutive threads are one row (the row count is whole waves): lanes 0-31 / 32-63 its groups
  if (d.oq) gated_e4m3(d, qr / kQH, head, c, o01, o23);
}

int decode_splits(int B, int splits) {
  if (splits > 0) return min(splits, 64);
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  return max(1, min(64, cus / (B * kKVH)));
}
size_t decode_ws_bytes(int B, int S) {
  return align_up(sizeof(float) * (size_t)B * kKVH * S * kDRows * kDD, 256) +
         align_up(sizeof(float) * (size_t)B * kKVH * S * 2 * kDRows, 256);
}

}  // namespace
}  // namespace q36

using namespace q36;

extern "C" size_t q36_attn_decode_workspace_bytes(int32_t B, int32_t splits) {
  return decode_ws_bytes(B, decode_splits(B, splits));
}

extern "C" int q36_attn_decode(const q36_decode_args* a, q36_stream_t stream) {
  Q36_REQUIRE(a != nullptr, "q36_attn_decode: null args");
  Q36_REQUIRE(a->HQ == kQH && a->HKV == kKVH && a->D == kDD,
              "q36_attn_decode: HQ=%d HKV=%d D=%d unsupported (this build: 16 / 2 / 256)", a->HQ, a->HKV, a->D);
  Q36_REQUIRE(a->B >= 1 && a->B <= 65535 && a->NT >= 1 && a->NT <= kDNT, "q36_attn_decode: B=%d NT=%d out of range",
              a->B, a->NT);
  Q36_REQUIRE(a->q && a->k_cache && a->v_cache && a->page_table && a->seqlens && a->out && a->workspace,
              "q36_attn_decode: a required pointer is null");
  Q36_REQUIRE(aligned16(a->q) && aligned16(a->k_cache) && aligned16(a->v_cache) &&
                  (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0,
              "q36_attn_decode: q, k_cache, v_cache must be 16-byte and workspace 256-byte aligned");
  Q36_REQUIRE(a->num_slots >= 1 && (int64_t)a->num_slots * kKVH * kDD < ((int64_t)1 << 31),
              "q36_attn_decode: num_slots=%lld out of range", (long long)a->num_slots);
  Q36_REQUIRE(a->pt_stride >= 1, "q36_attn_decode: pt_stride=%d", a->pt_stride);
  Q36_REQUIRE(!a->out_loc || (a->k_new && a->v_new), "q36_attn_decode: out_loc needs k_new and v_new");
  Q36_REQUIRE((a->gate == nullptr) == (a->oq == nullptr) && (a->oq == nullptr) == (a->oqs == nullptr),
              "q36_attn_decode: gate, oq and oqs go together");
  Q36_REQUIRE(!a->oq || ((reinterpret_cast<uintptr_t>(a->gate) & 7u) == 0 &&
                         (reinterpret_cast<uintptr_t>(a->oq) & 3u) == 0 && (reinterpret_cast<uintptr_t>(a->oqs) & 3u) == 0),
              "q36_attn_decode: gate must be 8-byte, oq and oqs 4-byte aligned");
  const int S = decode_splits(a->B, a->splits);
  const size_t need = decode_ws_bytes(a->B, S);
  Q36_REQUIRE(a->workspace_bytes >= need, "q36_attn_decode: workspace of %zu bytes < %zu required", a->workspace_bytes,
              need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(a->workspace);
  const int T = a->B * a->NT;
  if (a->out_loc)
    kv_scatter_kernel<<<(T * 64 + 255) / 256, 256, 0, st>>>(static_cast<const uint8_t*>(a->k_new),
                                                            static_cast<const uint8_t*>(a->v_new), a->out_loc, T, a->num_slots,
                                                            static_cast<uint8_t*>(a->k_cache),
                                                            static_cast<uint8_t*>(a->v_cache));
  DecodeDev d{a->B, a->NT, S, a->pt_stride,
              static_cast<const uint16_t*>(a->q), static_cast<const uint8_t*>(a->k_cache),
              static_cast<const uint8_t*>(a->v_cache), (int64_t)a->num_slots * kKVH * kDD, a->page_table, a->seqlens,
              a->scale * 1.44269504088896340736f, reinterpret_cast<float*>(ws),
              reinterpret_cast<float*>(ws + align_up(sizeof(float) * (size_t)a->B * kKVH * S * kDRows * kDD, 256)),
              static_cast<uint16_t*>(a->out), static_cast<const uint16_t*>(a->gate), static_cast<uint8_t*>(a->oq),
              a->oqs};
  if (a->NT <= 2)
    decode_split_kernel<1, kDecNS1, kDecWPE1><<<dim3(S, kKVH, a->B), 256, 0, st>>>(d);
  else
    decode_split_kernel<2, kDecNS2, 1><<<dim3(S, kKVH, a->B), 256, 0, st>>>(d);
  if (S > 1) decode_combine_kernel<<<(a->B * a->NT * kQH * (kDD / 4) + 255) / 256, 256, 0, st>>>(d);
  return check_launch("q36_attn_decode");
}
