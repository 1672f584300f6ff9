/* CPU oracle for the qwen36 decode/verify kernel nodes.
 *
 * TEST INFRASTRUCTURE ONLY.  This C restatement of the reference's arithmetic is the
 * checker that the HIP kernels are compared against (and the CPU baseline that bench.py
 * times beside them).  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library (bundles_amd/libq36.so) never links or calls it.
 *
 * All arrays are host memory, row-major, contiguous.  bf16 values travel as uint16_t
 * bit patterns, OCP e4m3fn values as uint8_t.  Every function cites the reference
 * file:line it restates (R = /root/reference/qwen36_nodes_kb34, L = R/qwen36_layer,
 * H = R/qwen36_lmhead8).
 *
 * Parity status of each function (how it is pinned) is listed in oracle/README.md.
 */
#ifndef Q36_ORACLE_H
#define Q36_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs and math ---- */
uint16_t q36o_f32_to_bf16(float f);          /* IEEE round-to-nearest-even, NaN kept quiet */
float q36o_bf16_to_f32(uint16_t h);
uint8_t q36o_f32_to_e4m3(float f);           /* OCP e4m3fn, RNE, saturate to +-448 (satfinite) */
float q36o_e4m3_to_f32(uint8_t b);
float q36o_expf(float x);                    /* Cody-Waite + degree-7 Taylor, all IEEE ops */
float q36o_dot_canon(const float* a, const float* b, int n); /* fixed 64-lane reduction order */

/* ---- quantizers ---- */
void q36o_quant_rows_i8(const float* x, int rows, int K, int8_t* q, float* s);
void q36o_quant_groups_e4m3(const float* x, int rows, int K, int group, uint8_t* q, float* s);
void q36o_quant_blocks_e4m3(const float* w, int N, int K, uint8_t* q, float* s);

/* ---- prepare-time weight formats of the reference ----
 * q8-block-v1 (L/i8x_kernels.py:12,69-110,119-141): per expert one block of
 *   [q13 int8 (2I x H) | q2 int8 (H x I) | c13 fp16 (2I x H/128) | c2 fp16 (H x I/128)]
 * q36o_q8_block_bytes(H, I) bytes apart.  A row's scale s16 = fp16(fp32(amax / 127) * (1 + 2^-10)),
 * q = clamp(round_half_away(w / (s16 > 0 ? s16 : 1)), +-127); channel = 1: one scale per row written
 * into every 128-group slot of the row; channel = 0: one scale per 128-group (the DENSE8 rule).
 * DENSE8 (L/dense8.py:140-188): q int8 [N, K] and fp16 scales group-major s [K/128][s_stride]
 * (element (g, n) at s[g * s_stride + n]), one per row and 128-group. */
uint16_t q36o_f32_to_f16(float f);           /* IEEE round-to-nearest-even, overflow to inf, NaN kept */
float q36o_f16_to_f32(uint16_t h);
size_t q36o_q8_block_bytes(int H, int I);
void q36o_quant_q8_block_v1(const float* w13, const float* w2, int E, int H, int I, int channel, uint8_t* blocks);
void q36o_quant_dense8(const float* w, int N, int K, int8_t* q, uint16_t* s, int s_stride);

/* ---- routing: router GEMV + softmax + top-k + renorm + expert lists ---- */
int q36o_route(const uint16_t* x, const uint16_t* wr, const float* bias, const int32_t* pos, int M, int E,
               int H, int k, float* logits, int32_t* ids, float* wts, int32_t* counts, int32_t* offsets,
               int32_t* perm, int32_t* inv_perm, int32_t* active, int32_t* n_active);

/* ---- MoE block (routed experts + shared expert + sigmoid gate + combine) ----
 * mode 0: int8 W8A8 (per-token / per-slot int8 activations, per-channel fp32 weight scales)
 * mode 1: fp8 e4m3 (per-token x 128-group activations, 128x128 block weight scales)
 * Optional debug outputs, indexed by slot (routed t*k + j, shared M*k + t):
 *   acc13 int32 [M*k+M, 2I] and acc2 int32 [M*k+M, H] (mode 0 only), h bf16 [M*k+M, I]. */
typedef struct {
  int mode, M, E, H, I, k;
  const uint16_t* x;       /* bf16 [M,H] */
  const uint16_t* wr;      /* bf16 [E,H] */
  const float* bias;       /* fp32 [E] or NULL */
  const int32_t* pos;      /* int32 [M] or NULL (rows with pos==0 are padding) */
  const void* w13;         /* int8 / e4m3 [E,2I,H] */
  const float* s13;        /* mode0 [E,2I]; mode1 [E,2I/128,H/128] */
  const void* w2;          /* [E,H,I] */
  const float* s2;         /* mode0 [E,H]; mode1 [E,H/128,I/128] */
  const void* sw13;        /* shared expert [2I,H] */
  const float* ss13;
  const void* sw2;         /* [H,I] */
  const float* ss2;
  const uint16_t* gate_w;  /* bf16 [H] */
  uint16_t* out;           /* bf16 [M,H] */
  int32_t* ids;            /* [M,k] */
  float* wts;              /* [M,k] */
  int32_t* acc13;          /* optional */
  int32_t* acc2;           /* optional */
  uint16_t* h;             /* optional */
  int n_threads;           /* 0 = OpenMP default */
  /* Teacher forcing (NULL: off).  h_in bf16 [M*k+M, I]: the down stage reads these SwiGLU rows
   * instead of its own; y_in bf16 [M*k+M, H]: the combine reads these weighted expert rows instead
   * of its own.  Each stage can then be judged on the other implementation's inputs. */
  const uint16_t* h_in;
  const uint16_t* y_in;
  uint16_t* y;             /* optional: the weighted expert rows by slot [M*k+M, H] */
} q36o_moe_args;
int q36o_moe(const q36o_moe_args* a);

/* ---- GDN speculative verify ---- */
typedef struct {
  int B, T;                 /* sequences, positions per sequence */
  const uint16_t* mixed;    /* bf16 [B*T, 8192] = q 16x128 | k 16x128 | v 32x128 */
  const uint16_t* z;        /* bf16 [B*T, 4096] */
  const uint16_t* a;        /* bf16 [B*T, 32] */
  const uint16_t* b;        /* bf16 [B*T, 32] */
  uint16_t* conv_state;     /* bf16 [B, 8192, 3], rolled in place */
  const uint16_t* conv_w;   /* bf16 [8192, 4] */
  const float* A_log;       /* [32] */
  const float* dt_bias;     /* [32] */
  const float* S0;          /* fp32 [B, 32, 128(V), 128(K)] */
  const uint16_t* norm_w;   /* bf16 [128] */
  float eps;
  uint16_t* out;            /* bf16 [B*T, 4096] */
  float* snaps;             /* fp32 [B, T, 32, 128, 128] */
  int use_f64;              /* 1: recurrence in double (check variant) */
  int n_threads;
} q36o_gdn_args;
int q36o_gdn_verify(const q36o_gdn_args* a);

/* ---- GDN speculative verify over the ReplaySSM ring (read-only checkpoint + 16-entry ring) ----
 * L/qk_gdn_verify.cu:1-20 (design), :583-605 (ring keys), :616-632 (gates, g ring), :634-648
 * (history decay), :684-762 (window recurrence), :770-781 (d ring); host checks :850-919.
 * Request r owns rows qsl[r] .. qsl[r] + T - 1; state_idx < 0 marks a padded request (zero output,
 * nothing else written).  The history state is td * h0 + sum_c decay_c dhat_c khat_c^T over the
 * committed entries c < write_pos (logical order, physical slot (cache_base + c) & 15), with the
 * bf16 high parts only; the window's d, k (high and low bf16 parts) and g are appended at logical
 * positions write_pos + t while they fit the ring.  conv_state is rolled in place and the draft
 * windows [s1 s2 x0 .. x_{T-1}] are written per channel. */
typedef struct {
  int B, T;                 /* requests, tokens per request (1..8) */
  const uint16_t* mixed;    /* bf16 [rows, 8192] */
  const uint16_t* z;        /* bf16 [rows, 4096] */
  const uint16_t* a;        /* bf16 [rows, 32] */
  const uint16_t* b;        /* bf16 [rows, 32] */
  uint16_t* conv_state;     /* bf16 [slots, 8192, 3], rolled in place */
  const uint16_t* conv_w;   /* bf16 [8192, 4] */
  uint16_t* window;         /* bf16 [wslots, 8192, T + 2] */
  const float* A_log;       /* [32] */
  const float* dt_bias;     /* [32] */
  const float* h0;          /* fp32 [slots, 32, 128 (V), 128 (K)] checkpoint, read only */
  uint16_t* d_ring;         /* bf16 [rslots, 32, 16, 128] */
  uint16_t* dlo_ring;
  uint16_t* k_ring;         /* bf16 [rslots, 16, 16, 128] */
  uint16_t* klo_ring;
  float* g_ring;            /* fp32 [rslots, 32, 16] */
  const int32_t* qsl;       /* [B + 1] */
  const int64_t* state_idx; /* [B] checkpoint / conv-state slot, < 0: padded */
  const int64_t* replay_idx;/* [B] ring slot */
  const int64_t* win_idx;   /* [B] window slot */
  const int32_t* write_pos; /* [rslots] committed entries */
  const int32_t* cache_base;/* [rslots] physical slot of logical entry 0 */
  const uint16_t* norm_w;   /* bf16 [128] */
  float eps, scale;
  uint16_t* out;            /* bf16 [rows, 4096] */
  int use_f64;              /* 1: history state and recurrence in double (check variant) */
  int n_threads;
} q36o_gdn_ring_args;
int q36o_gdn_verify_ring(const q36o_gdn_ring_args* a);

/* ---- fused gated full-attention projections (fp8 128x128 block weights) ---- */
typedef struct {
  int T;                    /* tokens */
  const uint16_t* x;        /* bf16 [T, 2048] */
  const uint8_t* wqg;       /* e4m3 [8192, 2048], rows [q(256) gate(256)] x 16 heads */
  const float* sqg;         /* [64, 16] */
  const uint8_t* wk;        /* e4m3 [512, 2048] */
  const float* sk;          /* [4, 16] */
  const uint8_t* wv;
  const float* sv;
  const uint16_t* q_norm_w; /* bf16 [256] */
  const uint16_t* k_norm_w; /* bf16 [256] */
  float eps;
  const float* cos_sin;     /* fp32 [max_pos, 64]: cos[0..31] | sin[0..31] */
  const int32_t* positions; /* [T] */
  uint16_t* q;              /* bf16 [T, 16, 256] normed + roped */
  uint16_t* gate;           /* bf16 [T, 16, 256] */
  uint16_t* k;              /* bf16 [T, 2, 256] normed + roped */
  uint16_t* v;              /* bf16 [T, 2, 256] */
  uint8_t* k8;              /* e4m3 [T, 2, 256] (cache write, satfinite) */
  uint8_t* v8;
  int n_threads;
} q36o_attn_args;
int q36o_attn_proj(const q36o_attn_args* a);

typedef struct {
  int T;
  const uint16_t* attn;     /* bf16 [T, 4096] attention output */
  const uint16_t* gate;     /* bf16 [T, 4096] */
  const uint8_t* wo;        /* e4m3 [2048, 4096] */
  const float* so;          /* [16, 32] */
  uint16_t* out;            /* bf16 [T, 2048] */
  int n_threads;
} q36o_oproj_args;
int q36o_attn_oproj(const q36o_oproj_args* a);

/* ---- int8 lm_head + greedy argmax ---- */
typedef struct {
  int R, H, V;
  const uint16_t* h;        /* bf16 [R, H] final hidden */
  const uint16_t* norm_w;   /* bf16 [H] Gemma RMSNorm weight (y = x*rstd*(1+w)); NULL = no norm */
  float eps;
  const int8_t* wq;         /* int8 [V, H] */
  const float* ws;          /* fp32 [V] */
  int32_t* ids;             /* [R] */
  uint16_t* logits;         /* optional bf16 [R, V] */
  int n_threads;
  int mode;                 /* 0: one int8 activation term; 1: two terms (H/w8a8.py:25-37);
                               2: W8A16, bf16 rows x int8 weights (H/lmhead8.py:57-91) */
} q36o_lmhead_args;
int q36o_lmhead(const q36o_lmhead_args* a);

/* ---- DENSE8 W8A16 linear (L/dense8.py:1-28,229-401) ----
 * x bf16 [T, K], q int8 [N, K], s fp16 bits [K/128][s_ld]: y[t, n] = bf16(acc), acc = fmaf(dot_g, s[g][n], acc)
 * over the 128-column groups in order from zero, dot_g the exact sum of the group's products rounded once
 * to fp32. */
int q36o_dense8_linear(int T, int N, int K, const uint16_t* x, const int8_t* q, const uint16_t* s, int64_t s_ld,
                       uint16_t* out, int n_threads);

/* ---- decode / verify attention over an e4m3 KV cache ---- */
typedef struct {
  int B, NT, HQ, HKV, D;            /* requests, query tokens per request, q heads, kv heads, head dim */
  const uint16_t* q;                /* bf16 [B*NT, HQ, D]: normed and roped queries */
  const uint8_t* kcache;            /* e4m3 [slots, HKV, D] */
  const uint8_t* vcache;            /* e4m3 [slots, HKV, D] */
  const int32_t* page_table;        /* [B, pt_stride]: the cache slot of key position i */
  int pt_stride;
  const int32_t* seqlens;           /* [B]: key positions per request, the NT new ones included */
  float scale;                      /* softmax scale */
  uint16_t* out;                    /* bf16 [B*NT, HQ, D] */
  int n_threads;
} q36o_decode_args;
int q36o_attn_decode(const q36o_decode_args* a);
float q36o_f16_round(float x);

/* hybrid-layer glue: e4m3 block-scaled linear (x bf16 [T, K], wq row-major e4m3 [N, K], ws
 * [N/128, K/128], out bf16 [T, N]) and the add + Gemma RMSNorm (delta may be NULL) */
int q36o_fp8_linear(int T, int N, int K, const uint16_t* x, const uint8_t* wq, const float* ws, uint16_t* out,
                    int n_threads);
int q36o_add_rmsnorm(int T, int H, const uint16_t* delta, uint16_t* residual, const uint16_t* w, float eps,
                     uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif
