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
//   decode_split    workgroup = (split, KV head, request), 4 waves; the 32 query rows (4 tokens x 8
//                   heads) of the group against 64-key tiles of the split's key range.  Scores:
//                   wave w takes keys 16 w .. of the tile, e4m3 16x16x128 MFMA of the query
//                   fragments (registers, whole kernel) and the keys (straight from the cache by
//                   page table).  Softmax: tile row max through LDS, online rescale, weights
//                   rounded to f16 into LDS.  P V: wave w owns dims 64 w ..; f16 16x16x32 MFMA, V
//                   staged in LDS by buffer DMA (16-byte pieces XOR-swizzled by key) and read
//                   key-major with the LDS transpose read, widened e4m3 -> f16 (exact).  The next
//                   tile's keys and values are requested while this one computes.
//   decode_combine  per (request, KV head): the splits' partials weighted by exp2(m_s - M) / L.
#include <math.h>

#include <type_traits>

#include "q36_device.h"
#include "q36_host.h"

namespace q36 {
namespace {

constexpr int kQH = 16, kKVH = 2, kDD = 256, kGQ = kQH / kKVH, kDNT = 4, kDRows = kGQ * kDNT, kKT = 64;
constexpr int kPRow = kKT * 2 + 16;  // P row in LDS: 64 f16 weights + 16 bytes (16 rows on distinct banks)

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v2f __attribute__((ext_vector_type(2)));

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
};

__device__ __forceinline__ v4f mfma_e4m3(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
__device__ __forceinline__ v8i cat8d(v4i a, v4i b) {
  v8i r = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return r;
}
// 8 e4m3 codes (two words) -> 8 f16 (every e4m3 value is an f16 value: exact)
__device__ __forceinline__ v8h widen8(int w0, int w1) {
  const v2f a = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false), b = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
  const v2f c = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false), d = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
  v8h r = {(_Float16)a.x, (_Float16)a.y, (_Float16)b.x, (_Float16)b.y,
           (_Float16)c.x, (_Float16)c.y, (_Float16)d.x, (_Float16)d.y};
  return r;
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

__global__ __launch_bounds__(256) void decode_split_kernel(DecodeDev d) {
  __shared__ __align__(16) uint8_t vbuf0[kKT * kDD];
  __shared__ __align__(16) uint8_t vbuf1[kKT * kDD];
  __shared__ __align__(16) uint8_t ps[kDRows * kPRow];
  __shared__ float red_m[4][kDRows], red_l[4][kDRows];
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z, S = d.splits;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
  const int NT = d.NT, nk = d.seqlens[b], npre = nk - NT;
  const int tiles = (nk + kKT - 1) / kKT, per = tiles / S, rem = tiles % S;
  const int t0 = s * per + min(s, rem), t1 = t0 + per + (s < rem ? 1 : 0);
  const int grp = (b * kKVH + h) * S + s;
  // query fragments (score MFMA operand A): row 16 rt + l16 = token (row / 8), head h*8 + row % 8;
  // dims 128 kb + 32 lg .. +31 rounded to e4m3 (rows of tokens past NT are zero)
  v8i qa[2][2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int row = 16 * rt + l16, t = row >> 3;
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
      qa[rt][kb] = v8i{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]};
    }
  }
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)d.kc, (short)0, (int)d.kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)d.vc, (short)0, (int)d.kv_bytes, 0x00020000);
  // the request's page-table row through a bounded buffer (an entry past the row reads as slot 0)
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(d.pt + (size_t)b * d.pt_stride), (short)0, 4 * d.pt_stride, 0x00020000);
  auto ptr_at = [&](int key) { return __builtin_amdgcn_raw_buffer_load_b32(prs, 4 * key, 0, 0); };
  // per-lane state for rows 16 rt + 4 lg + r (index 4 rt + r): running max, this wave's weight sum
  float m[8], lw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m[i] = -INFINITY;
    lw[i] = 0.f;
  }
  v4f o[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[rt][dt] = v4f{0.f, 0.f, 0.f, 0.f};
  // Requests of tile it into buffer set Q (registers kf[Q], LDS vbuf_Q): the wave's 16 keys (score
  // operand B: key 16 w + l16, dims 128 kb + 32 lg ..) and its 16 value rows (4 calls of 4 keys;
  // lane l: key 4 c + l / 16, position l16 holds piece l16 ^ key % 16).  The page-table entry of a
  // tile is loaded one tile earlier, so a fetch never waits on it.
  v4i kf[2][4];
  auto key_of = [&](int it) { return min(it * kKT + 16 * wave + l16, nk - 1); };
  auto fetch = [&](int it, int slot, auto qc) {
    constexpr int Q = decltype(qc)::value;
    (void)it;
    const int kbase = (slot * kKVH + h) * kDD + 32 * lg;
    kf[Q][0] = __builtin_amdgcn_raw_buffer_load_b128(krs, kbase, 0, 0);
    kf[Q][1] = __builtin_amdgcn_raw_buffer_load_b128(krs, kbase + 16, 0, 0);
    kf[Q][2] = __builtin_amdgcn_raw_buffer_load_b128(krs, kbase + 128, 0, 0);
    kf[Q][3] = __builtin_amdgcn_raw_buffer_load_b128(krs, kbase + 144, 0, 0);
    uint8_t* vb = Q ? vbuf1 : vbuf0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kl = 16 * wave + 4 * c + lg;       // key within the tile
      const int vslot = __shfl(slot, 4 * c + lg);  // lane 4 c + lg holds that key's slot
      const int voff = (vslot * kKVH + h) * kDD + 16 * (l16 ^ (kl & 15));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, vb + (16 * wave + 4 * c) * kDD, 16, voff, 0, 0, 0);
    }
  };
  int slot_next = ptr_at(key_of(min(t0 + 1, max(t1 - 1, t0))));
  if (t0 < t1) fetch(t0, ptr_at(key_of(t0)), std::integral_constant<int, 0>{});
  auto step = [&](int it, auto qc) {
    constexpr int Q = decltype(qc)::value;
    const bool more = it + 1 < t1;
    // scores of the wave's 16 keys for the 32 rows
    v4f sr[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      sr[rt] = mfma_e4m3(qa[rt][0], cat8d(kf[Q][0], kf[Q][1]), v4f{0.f, 0.f, 0.f, 0.f});
      sr[rt] = mfma_e4m3(qa[rt][1], cat8d(kf[Q][2], kf[Q][3]), sr[rt]);
    }
    const int key = it * kKT + 16 * wave + l16;
    float sv[8];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * rt + 4 * lg + r, t = row >> 3;
        const bool ok = t < NT && key <= npre + t;  // key < nk follows
        sv[4 * rt + r] = ok ? sr[rt][r] * d.scale_log2 : -INFINITY;
      }
    // tile row max: the wave's 16 keys (lanes l16), then the four waves through LDS
    float mx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = sv[i];
#pragma unroll
      for (int o2 = 1; o2 < 16; o2 <<= 1) v = fmaxf(v, __shfl_xor(v, o2));
      mx[i] = v;
    }
    __syncthreads();  // the previous tile's reads of red_m, ps and the other value buffer are done
    if (more) fetch(it + 1, slot_next, std::integral_constant<int, Q ^ 1>{});
    // always one page-table load (clamped), so the count of loads after this tile's values is fixed
    slot_next = ptr_at(key_of(min(it + 2, t1 - 1)));
    if (l16 == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) red_m[wave][16 * (i >> 2) + 4 * lg + (i & 3)] = mx[i];
    }
    __syncthreads();
    float alpha[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 16 * (i >> 2) + 4 * lg + (i & 3);
      const float tm = fmaxf(fmaxf(red_m[0][row], red_m[1][row]), fmaxf(red_m[2][row], red_m[3][row]));
      const float mn = fmaxf(m[i], tm);
      alpha[i] = mn == -INFINITY ? 1.f : exp2f(m[i] - mn);
      m[i] = mn;
      const float p = sv[i] == -INFINITY ? 0.f : exp2f(sv[i] - mn);
      *reinterpret_cast<_Float16*>(ps + row * kPRow + 2 * (16 * wave + l16)) = (_Float16)p;
      float ssum = p;
#pragma unroll
      for (int o2 = 1; o2 < 16; o2 <<= 1) ssum += __shfl_xor(ssum, o2);
      lw[i] = lw[i] * alpha[i] + ssum;
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[rt][dt][r] *= alpha[4 * rt + r];
    // this tile's values have landed: newer are the next tile's 4 key and 4 value loads (if any)
    // and one page-table load
    if (more)
      asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
    __syncthreads();
    asm volatile("" ::: "memory");
    const uint8_t* vb = Q ? vbuf1 : vbuf0;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      v8h pa[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        pa[rt] = *reinterpret_cast<const v8h*>(ps + (16 * rt + l16) * kPRow + 64 * kk + 16 * lg);
      const int kr = 32 * kk + 8 * lg + (l16 >> 1);  // the value row (key) this lane addresses
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int pos = (4 * wave + dt) ^ (kr & 15);
        const v2i raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) v2i*)(vb + kr * kDD + 16 * pos + 8 * (l16 & 1)));
        const v8h vv = widen8(raw.x, raw.y);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rt], vv, o[rt][dt], 0, 0, 0);
      }
    }
  };
  for (int it = t0; it < t1; it += 2) {
    step(it, std::integral_constant<int, 0>{});
    if (it + 1 < t1) step(it + 1, std::integral_constant<int, 1>{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // partials: unnormalised o, the running max and the weight sum (summed over the four waves)
  float* wo = d.ws_o + (size_t)grp * kDRows * kDD;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) wo[(16 * rt + 4 * lg + r) * kDD + 64 * wave + 16 * dt + l16] = o[rt][dt][r];
  __syncthreads();
  if (l16 == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) red_l[wave][16 * (i >> 2) + 4 * lg + (i & 3)] = lw[i];
  }
  if (wave == 0 && l16 == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) red_m[0][16 * (i >> 2) + 4 * lg + (i & 3)] = m[i];
  }
  __syncthreads();
  if (tid < kDRows) {
    d.ws_ml[(size_t)grp * 2 * kDRows + tid] = red_m[0][tid];
    d.ws_ml[(size_t)grp * 2 * kDRows + kDRows + tid] = (red_l[0][tid] + red_l[1][tid]) + (red_l[2][tid] + red_l[3][tid]);
  }
}

// per (request, KV head): out = bf16(sum_s exp2(m_s - M) o_s / sum_s exp2(m_s - M) l_s), splits in order
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeDev d) {
  __shared__ float wgt[64][kDRows];
  __shared__ float inv_l[kDRows];
  const int h = blockIdx.x, b = blockIdx.y, S = d.splits, tid = threadIdx.x;
  const int g0 = (b * kKVH + h) * S;
  if (tid < kDRows) {
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = fmaxf(M, d.ws_ml[(size_t)(g0 + s) * 2 * kDRows + tid]);
    float L = 0.f;
    for (int s = 0; s < S; ++s) {
      const float ms = d.ws_ml[(size_t)(g0 + s) * 2 * kDRows + tid];
      const float w = ms == -INFINITY ? 0.f : exp2f(ms - M);
      wgt[s][tid] = w;
      L += w * d.ws_ml[(size_t)(g0 + s) * 2 * kDRows + kDRows + tid];
    }
    inv_l[tid] = L > 0.f ? 1.f / L : 0.f;
  }
  __syncthreads();
  for (int e = tid; e < d.NT * kGQ * kDD / 4; e += 256) {
    const int row = e / (kDD / 4), dim = 4 * (e % (kDD / 4));
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < S; ++s) {
      const float w = wgt[s][row];
      const float4 v = *reinterpret_cast<const float4*>(d.ws_o + ((size_t)(g0 + s) * kDRows + row) * kDD + dim);
      a.x += w * v.x;
      a.y += w * v.y;
      a.z += w * v.z;
      a.w += w * v.w;
    }
    const float il = inv_l[row];
    const int t = row >> 3;
    uint16_t* dst = d.out + (((size_t)b * d.NT + t) * kQH + h * kGQ + (row & 7)) * kDD + dim;
    *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf2(a.x * il, a.y * il), pack_bf2(a.z * il, a.w * il));
  }
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
              static_cast<uint16_t*>(a->out)};
  decode_split_kernel<<<dim3(S, kKVH, a->B), 256, 0, st>>>(d);
  decode_combine_kernel<<<dim3(kKVH, a->B), 256, 0, st>>>(d);
  return check_launch("q36_attn_decode");
}
