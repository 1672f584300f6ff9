/* q36 -- MI355X (gfx950) kernel nodes for the qwen36_layer / qwen36_lmhead8 bundle slots.
 *
 * The drop-in boundary: a flat extern "C" API over raw device pointers.  Every entry point
 * validates its arguments, launches on the caller's stream, never allocates, never frees and
 * never synchronises, so a caller may capture it into a hipGraph.  Return codes: Q36_OK, or
 * Q36_EINVAL (a shape / alignment / size violation; nothing was launched) or Q36_ELAUNCH (a HIP
 * error); q36_last_error() gives the thread's last message.  No exception crosses this boundary.
 *
 * Reference interfaces replaced (R = qwen36_nodes_kb34, L = R/qwen36_layer, H = R/qwen36_lmhead8):
 *   q36_moe_route      <- qk_route.route / route48 / route16w     (L/qk_route.cu:1124,1162,1219)
 *   q36_moe_forward    <- i8x_decode.moe_row_batch: route + fused/up + down + combine
 *                         (L/i8x_decode.py:528-605; L/qk_moe_up16.cu:915; L/qk_moe_dn16.cu:301;
 *                          L/qk_route.cu:1270)
 *   q36_gdn_verify     <- qk_gdn_verify.gdn_verify_fused           (L/qk_gdn_verify.cu:841-849)
 *                         with per-position state snapshots in place of the replay ring
 *   q36_gdn_verify_ring <- qk_gdn_verify.gdn_verify_fused over the ReplaySSM ring
 *                         (L/qk_gdn_verify.cu:841-990; L/gdn_fused.py:37-57)
 *   q36_attn_proj      <- qkv_proj + attn_prefill_front            (L/qk_proj_decode.cu:434;
 *                         L/qk_attn_verify.cu:981)
 *   q36_attn_oproj     <- o_proj of the gated attention output    (L/attn_fused.py:232-273;
 *                         gate L/qk_attn_verify.cu:730-737)
 *   q36_lmhead_argmax  <- lmh8_w8a8x2 / w8a8_linear + the stock greedy sampler
 *                         (L/qk_proj_decode.cu:1354; H/w8a8.py:116-120; H/node.py:136-151)
 *   q36_quant_rows_i8  <- lmhead8.quantize_rows / w8a8.quantize_act (H/lmhead8.py:111; H/w8a8.py:77)
 *   q36_quant_q8_block_v1 <- i8x_kernels.fill_expert / quantize_channel (L/i8x_kernels.py:119-141):
 *                         the q8-block-v1 expert copy
 *   q36_import_q8_block_v1 <- i8x_kernels.block_parts (L/i8x_kernels.py:99-103): a channel-mode copy
 *                         read back as the decode MoE's int8 experts
 *   q36_quant_dense8   <- dense8.quantize (L/dense8.py:168-188): the DENSE8 copy
 *   q36_quant_blocks_e4m3 <- (no reference counterpart: the 128x128 block-scaled e4m3 weight
 *                         format the configuration asks for)
 *   q36_pack_frag8     <- (no reference counterpart: a prepare-time reordering of the 8-bit
 *                         weights into the operand order of the gfx950 MFMA)
 */
#ifndef Q36_ABI_H
#define Q36_ABI_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q36_ABI_VERSION 7
#define Q36_OK 0
#define Q36_EINVAL 1
#define Q36_ELAUNCH 2

#define Q36_MOE_INT8 0 /* W8A8: per-token int8 x, per-channel int8 weights, fp32 scales */
#define Q36_MOE_FP8 1  /* OCP e4m3fn: per-token x 128-group x, 128x128 block weight scales */

typedef void* q36_stream_t; /* a hipStream_t (0 = the null stream) */

int q36_abi_version(void);
const char* q36_last_error(void);

/* ---------------------------------------------------------------------------------------
 * Decode MoE block (one row batch of M <= 256 tokens).
 * Layouts (row-major, K innermost):
 *   x bf16 [M,H]; router_w bf16 [E,H]; router_bias fp32 [E] or NULL (added before the bf16
 *   rounding of the logits); positions int32 [M] or NULL (rows whose position is 0 are padding:
 *   no experts, zero output);
 *   w13 [E,2I,H] (gate rows 0..I-1, up rows I..2I-1), w2 [E,H,I], int8 or e4m3 bytes, each
 *   (and the shared expert's) in MFMA fragment order (q36_pack_frag8 of the row-major codes);
 *   INT8 scales: s13 fp32 [E,2I], s2 fp32 [E,H]; FP8 scales: s13 [E,2I/128,H/128], s2 [E,H/128,I/128];
 *   shared expert sw13 [2I,H], sw2 [H,I] with scales of the same form (no E);
 *   gate_w bf16 [H]; out bf16 [M,H].
 * Constraints: H == 2048 and I == 512 (this build), E % 64 == 0, 64 <= E <= 1024,
 *   1 <= topk <= min(16, E), 1 <= M <= 256; every pointer 16-byte aligned.
 * Workspace: q36_moe_workspace_bytes() bytes, 256-byte aligned, no initial contents required
 *   (every call writes what it reads).  q36_moe_workspace_layout() gives the byte offset of each
 *   list inside it.
 * Debug outputs (NULL to skip), indexed by slot (routed t*topk + j, shared M*topk + t):
 *   dbg_acc13 int32 [M*topk+M, 2I], dbg_acc2 int32 [M*topk+M, H] (INT8 only: the GEMM
 *   accumulators before scaling), dbg_h bf16 [M*topk+M, I] (SwiGLU output).
 * Calls that overlap on one workspace race; distinct workspaces are independent. */
typedef struct q36_moe_args {
  int32_t M, E, H, I, topk, dtype;
  const void* x;
  const void* router_w;
  const float* router_bias;
  const int32_t* positions;
  const void* w13;
  const float* s13;
  const void* w2;
  const float* s2;
  const void* sw13;
  const float* ss13;
  const void* sw2;
  const float* ss2;
  const void* gate_w;
  void* out;
  void* workspace;
  size_t workspace_bytes;
  int32_t* dbg_acc13;
  int32_t* dbg_acc2;
  void* dbg_h;
  /* Optional: the next block's input add-norm fused into the combine (the reference's combine_norm,
   * L/qk_route.cu:630-820), when norm_out is not NULL: z = out + resid (fp32, out the bf16 combine
   * result), resid <- bf16(z) in place, norm_out = bf16((z * rstd) * (1 + norm_w)) with rstd over z
   * in q36_add_rmsnorm's order: the same bits as q36_add_rmsnorm(out, resid, norm_w) after the block.
   * resid, norm_out bf16 [M, H]; norm_w bf16 [H].  norm_q8 / norm_q8s / norm_q8_frag (optional, with
   * norm_out): also norm_out's e4m3 codes as q36_add_rmsnorm's q8 / q8s / q8_frag. */
  void* resid;
  const void* norm_w;
  float norm_eps;
  void* norm_out;
  void* norm_q8;
  float* norm_q8s;
  int32_t norm_q8_frag;
  /* Optional (no reference counterpart as one launch; the arithmetic is q36_add_rmsnorm's): this
   * block's own input add-norm run by the route kernel, when in_norm_w is not NULL.  z = in_delta +
   * in_resid (fp32), in_resid_out <- bf16(z), and the block runs on x = bf16((z * rstd) *
   * (1 + in_norm_w)) with rstd over z in q36_add_rmsnorm's order: the same bits as q36_add_rmsnorm
   * (in_delta, residual, in_norm_w, out = x) followed by the block.  x is then an optional output
   * (those rows, or NULL).  in_delta, in_resid, in_resid_out bf16 [M, H], in_norm_w bf16 [H];
   * in_resid_out and x overlap neither in_delta nor in_resid (the route reads those while it writes). */
  const void* in_delta;
  const void* in_resid;
  void* in_resid_out;
  const void* in_norm_w;
  float in_norm_eps;
} q36_moe_args;

typedef struct q36_moe_ws_layout {
  size_t logits;   /* fp32 [M,E] bf16-rounded router logits (+bias) */
  size_t gate;     /* fp32 [M] shared-expert gate sigmoid(x . gate_w) (route-internal) */
  size_t ids;      /* int32 [M,topk], -1 for padding rows */
  size_t wts;      /* fp32 [M,topk] renormalised routing weights */
  size_t counts;   /* int32 [E] */
  size_t offsets;  /* int32 [E+1] exclusive scan of counts */
  size_t perm;     /* int32 [M*topk] sorted position -> slot t*topk+j (-1 past offsets[E]) */
  size_t inv_perm; /* int32 [M*topk] slot -> sorted position (-1 for padding) */
  size_t active;   /* int32 [E] experts with counts > 0, ascending */
  size_t ctl;      /* int32 [64]: [1] n_active (published by q36_moe_route) */
  size_t xq;       /* quantized x [M,H] */
  size_t xs;       /* fp32 [M, H/128] (INT8: [M]) */
  size_t h;        /* bf16 [M*topk+M, I] by slot (t*topk + j; shared M*topk + t) */
  size_t y;        /* bf16 [M*topk+M, H] by slot, routing weight applied */
  size_t ecount;   /* int32 [E] tokens per expert (route-internal) */
  size_t eact;     /* int32 [2E] work items of the expert kernels, e | j << 16 (token block j of expert e):
                    * [0, E) first blocks (ctl[2] counts them), [E, 2E) further blocks (ctl[3]); unordered
                    * (route-internal) */
  size_t elist;    /* int32 [E, M] slots of each expert, unordered (route-internal) */
  size_t total;
} q36_moe_ws_layout;

size_t q36_moe_workspace_bytes(int32_t M, int32_t E, int32_t H, int32_t I, int32_t topk, int32_t dtype);
int q36_moe_workspace_layout(int32_t M, int32_t E, int32_t H, int32_t I, int32_t topk, int32_t dtype,
                             q36_moe_ws_layout* out);
/* Routing only: logits, ids, wts and the expert lists, plus the quantized x and, when gate_w is
 * given, the shared expert's gate sigmoid(x . gate_w) per token (the combine reads it). */
int q36_moe_route(const q36_moe_args* a, q36_stream_t stream);
/* The phases of the block, each one stream-ordered launch set over the same workspace, for
 * callers that schedule them apart (the reference exposes the same split: up
 * L/qk_moe_up16.cu:329, down L/qk_moe_dn16.cu:301, combine_norm L/qk_route.cu:1270).
 *   q36_moe_up:      routed + shared gate/up GEMM and SwiGLU -> h   (needs q36_moe_route first)
 *   q36_moe_down:    down GEMM x routing weight -> y               (needs q36_moe_up first)
 *   q36_moe_combine: out = bf16(fma(sigmoid(x . gate_w), y_shared, sum_j y_j))
 *                    (the gate as the preceding q36_moe_route with gate_w formed it) */
int q36_moe_up(const q36_moe_args* a, q36_stream_t stream);
int q36_moe_down(const q36_moe_args* a, q36_stream_t stream);
int q36_moe_combine(const q36_moe_args* a, q36_stream_t stream);
/* The whole MoE block: route, up, down, combine. */
int q36_moe_forward(const q36_moe_args* a, q36_stream_t stream);

/* q36_moe_forward without a caller workspace (no reference counterpart: for callers that cannot
 * allocate, e.g. code under graph capture or a serving loop that forbids hipMalloc).  The workspace
 * is a device array inside the library of Q36_MOE_STATIC_SCRATCH_BYTES bytes, one per GPU, held until
 * the process ends; pass workspace = NULL and workspace_bytes = 0.  A call whose
 * q36_moe_workspace_bytes(M, E, H, I, topk, dtype) exceeds it returns Q36_EINVAL (M <= 256 with
 * E <= 512 and topk <= 10 fit).  Nothing is allocated or freed.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (two streams, two threads) race.  The array keeps the
 * last call's contents; no call needs initial contents. */
#define Q36_MOE_STATIC_SCRATCH_BYTES (16u << 20)
int q36_moe_forward_static(const q36_moe_args* a, q36_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * GDN speculative-verify step (L/qk_gdn_verify.cu:841-849 gdn_verify_fused), fixed head
 * geometry: 16 key heads x 128, 32 value heads x 128 (value head h reads key head h/2).
 *   mixed bf16 [B*T, 8192] = q (16x128) | k (16x128) | v (32x128), row b*T + t
 *   z bf16 [B*T, 4096]; a, b bf16 [B*T, 32]
 *   conv_state bf16 [B, 8192, 3] (taps oldest first, read only); conv_state_out bf16 [B, 8192, 3]
 *     receives the state after the T positions (the last three inputs); must not alias conv_state
 *   conv_w bf16 [8192, 4]; A_log, dt_bias fp32 [32]; norm_w bf16 [128]
 *   S0 fp32 [B, 32, 128 (v), 128 (k)] (read only)
 *   out bf16 [B*T, 4096] = gated RMSNorm of o_t = S_t q_t
 *   snaps fp32 [B, T, 32, 128, 128]: S_t after position t (the rollback states)
 * 1 <= T <= 8; S0 and snaps 16-byte aligned. */
typedef struct q36_gdn_args {
  int32_t B, T;
  const void* mixed;
  const void* z;
  const void* a;
  const void* b;
  const void* conv_state;
  void* conv_state_out;
  const void* conv_w;
  const float* A_log;
  const float* dt_bias;
  const float* S0;
  const void* norm_w;
  float eps;
  void* out;
  float* snaps;
} q36_gdn_args;
int q36_gdn_verify(const q36_gdn_args* a, q36_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * GDN speculative verify over the ReplaySSM ring: the served form of gdn_verify_fused
 * (L/qk_gdn_verify.cu:841-849, argument checks :850-919; glue L/gdn_fused.py:37-57).  The
 * rollback state is not materialised: the fp32 checkpoint h0 is read only, the committed history
 * is a 16-entry circular ring of (d, k, g) entries, and the window's entries are appended to it.
 *   Request r (< B) owns rows qsl[r] .. qsl[r] + T - 1 of mixed / z / a / b / out.
 *   state_idx[r]  checkpoint and conv-state slot; replay_idx[r] ring slot; win_idx[r] draft-window
 *                 slot.  state_idx < 0 marks a padded request (the reference's rule); so does any
 *                 index outside [0, slots) / [0, rslots) / [0, wslots): its rows of out are zeroed
 *                 and nothing else is written.  A request whose rows fall outside [0, rows) is
 *                 skipped entirely.
 *   idx_i64 bit 0 / 1 / 2: state_idx / replay_idx / win_idx hold int64 (else int32)
 *   write_pos[rs] committed entries n (clamped to [0, 16]); cache_base[rs] physical slot of
 *                 logical entry 0 (entry c lives at (cache_base + c) & 15)
 *   conv_state bf16 [slots, 8192, 3] (slot stride cs_slot elements), rolled in place to the last
 *                 three inputs; window bf16 [wslots, 8192, T + 2] (slot stride win_slot): per
 *                 channel [s1 s2 x0 .. x_{T-1}], whose rows [t, t + 3) are the conv state after
 *                 draft t
 *   h0 fp32 [slots, 32, 128 (v), 128 (k)], read only
 *   d_ring, dlo_ring bf16 [rslots, 32, 16, 128]; k_ring, klo_ring bf16 [rslots, 16, 16, 128];
 *   g_ring fp32 [rslots, 32, 16] (slot strides *_slot elements).  The verify reads the high
 *                 parts of the n committed entries and appends the window's d (the delta-rule
 *                 update beta (v - e^g S k)), unit key k and gate g at logical n + t while
 *                 n + t < 16, each bf16 value split into high and low parts.
 *   dt_bias fp32 (dt_f32 = 1) or bf16 [32]; A_log fp32 [32]; norm_w bf16 [128]; scale: the q
 *                 scale (128^-1/2 for this model)
 * 1 <= T <= 8; h0, z, conv_state, window, conv_w, the rings and out 16-byte aligned, the slot
 * strides multiples of 16 bytes.  Requests must name distinct slots (they write them).  B = 0 launches
 * nothing. */
typedef struct q36_gdn_ring_args {
  int32_t B, T, rows;
  int32_t slots, rslots, wslots;
  const void* mixed;
  const void* z;
  const void* a;
  const void* b;
  void* conv_state;
  int64_t cs_slot;
  const void* conv_w;
  void* window;
  int64_t win_slot;
  const float* A_log;
  const void* dt_bias;
  int32_t dt_f32;
  const float* h0;
  void* d_ring;
  void* dlo_ring;
  int64_t d_slot, dlo_slot;
  void* k_ring;
  void* klo_ring;
  int64_t k_slot, klo_slot;
  float* g_ring;
  int64_t g_slot;
  const int32_t* qsl;
  const void* state_idx;
  const void* replay_idx;
  const void* win_idx;
  int32_t idx_i64;
  const int32_t* write_pos;
  const int32_t* cache_base;
  const void* norm_w;
  float eps, scale;
  void* out;
  /* optional (no reference counterpart): out's e4m3 codes row-major [rows, 4096] per 128 channels (one
   * value head) and fp32 scales [rows, 32], the input q36_fp8_linear takes as xq / xqs for the
   * out_proj (K = 4096 reads row-major); a padded request's rows get zero codes and scales */
  void* oq;
  float* oqs;
} q36_gdn_ring_args;
int q36_gdn_verify_ring(const q36_gdn_ring_args* a, q36_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Fused gated full-attention projections (16 q heads x 256 with an output gate per head,
 * 2 KV heads x 256, hidden 2048), e4m3 weights with fp32 128x128 block scales.
 *   q36_attn_proj:  x bf16 [T, 2048] -> e4m3 activations (per token x 128 channels) ->
 *     qkv = x . wqkv^T with wqkv e4m3 [9216, 2048] = rows [q(256) gate(256)] x 16 | k 2x256 | v 2x256
 *     (the reference's fused qkv layout, L/attn_fused.py:209) passed in fragment order
 *     (q36_pack_frag8), sqkv fp32 [72, 16], rounded to bf16;
 *     then per head: Gemma RMSNorm on q and k (q_norm_w, k_norm_w bf16 [256], eps), neox RoPE on
 *     dims 0..63 with cos_sin fp32 [max_pos, 64] (cos 0..31 | sin 0..31) at positions int32 [T]
 *     (L/qk_attn_verify.cu:156-208).  Outputs: q bf16 [T,16,256], gate bf16 [T,16,256],
 *     k, v bf16 [T,2,256], k8, v8 e4m3 [T,2,256] (the cache write, satfinite, no scale).
 *   q36_attn_oproj: out bf16 [T, 2048] = (bf16(attn * sigmoid(gate)) in e4m3) . wo^T with
 *     attn, gate bf16 [T, 4096], wo e4m3 [2048, 4096] in fragment order, so fp32 [16, 32]
 *     (L/qk_attn_verify.cu:730-737).
 * Alignment: x, wqkv, attn, gate, wo, the norm weights, cos_sin and q, gate, k, v 16 bytes; k8, v8,
 * k_cache, v_cache 8 bytes.
 * Workspaces: q36_attn_workspace_bytes(T), q36_oproj_workspace_bytes(T), 256-byte aligned.
 * Activations quantized by their producer (no reference counterpart: the quantization folded into the
 * kernel that writes the rows, so these entries skip their own act_quant launch):
 *   q36_attn_proj with xq / xqs set (x then unused, may be NULL): the e4m3 codes of x's rows per token
 *     x 128 channels, in fragment order when q36_attn_act_frag(T) (codes [ceil(T/16)*16, 2048] by
 *     q36_pack_frag8's order of tokens x channels, the padding tokens' codes and scales zero), else
 *     row-major [T, 2048]; xqs fp32 [that many tokens, 16] = group amax / 448.  q36_add_rmsnorm
 *     (q8 / q8s / q8_frag) and q36_moe_forward's fused add-norm (norm_q8 ...) write exactly these.
 *   q36_attn_oproj with aq / aqs set (attn, gate unused, may be NULL): e4m3 codes row-major [T, 4096]
 *     of bf16(attn * sigmoid(gate)) and fp32 [T, 32] scales, as q36_attn_decode writes them
 *     (its gate / oq / oqs).
 * Either way the projection's outputs are the same bits as from the bf16 inputs. */
typedef struct q36_attn_args {
  int32_t T, max_pos;
  const void* x;
  const void* wqkv;
  const float* sqkv;
  const void* q_norm_w;
  const void* k_norm_w;
  float eps;
  const float* cos_sin;
  const int32_t* positions;
  void* q;
  void* gate;
  void* k;
  void* v;
  void* k8;
  void* v8;
  void* workspace;
  size_t workspace_bytes;
  const void* xq;  /* optional producer-quantized x (see above) */
  const float* xqs;
  /* optional cache append: with out_loc set, the new tokens' e4m3 K and V rows (k8 / v8's bytes) are
   * also written to row out_loc[t] (int64 [T]) of k_cache / v_cache e4m3 [num_slots, 2, 256]; a slot
   * outside [0, num_slots) is skipped.  The reference writes the cache in the same step
   * (L/qk_attn_verify.cu:431-465, :774-797); q36_attn_decode's out_loc then is not needed. */
  const int64_t* out_loc;
  void* k_cache;
  void* v_cache;
  int64_t num_slots;
} q36_attn_args;
typedef struct q36_oproj_args {
  int32_t T;
  const void* attn;
  const void* gate;
  const void* wo;
  const float* so;
  void* out;
  void* workspace;
  size_t workspace_bytes;
  const void* aq;  /* optional producer-quantized o_proj input (see above) */
  const float* aqs;
} q36_oproj_args;
/* 1 when q36_attn_proj reads T tokens' activations in fragment order (its K-sliced and tiled GEMMs,
 * T >= 32), 0 when row-major (the streaming GEMM below 32 tokens). */
int q36_attn_act_frag(int32_t T);
size_t q36_attn_workspace_bytes(int32_t T);
size_t q36_oproj_workspace_bytes(int32_t T);
int q36_attn_proj(const q36_attn_args* a, q36_stream_t stream);
int q36_attn_oproj(const q36_oproj_args* a, q36_stream_t stream);

/* ---- e4m3 block-scaled linear with column-segmented bf16 outputs: replaces the decode
 * projections the hybrid layer makes around its mixers, gdn_in_proj / qkv_proj
 * (L/qk_proj_decode.cu:409,434) with the column split of their outputs (the DENSE8 seg kernel,
 * L/qk_proj_decode.cu:483-1102; L/dense8.py:317-353) and the out_proj / o_proj GEMM before the
 * add-norm (L/proj.py:84-112) ----
 * x bf16 [T, K] (K = 2048 or 4096) is quantized per token x 128 channels to e4m3; w e4m3 [N, K]
 * in fragment order (q36_pack_frag8), N a multiple of 128 (rows past n_out are padding), ws fp32
 * [N/128, K/128].  y[t, n] = bf16(sum over 128-blocks kb in order of fma(blocksum, xs * ws, acc)).
 * Column n < n_out goes to the segment i with seg[i].col0 <= n < seg[i+1].col0 (or n_out), at
 * seg[i].out[t * seg[i].ld + n - seg[i].col0]; col0 and ld multiples of 4, outputs 8-byte aligned.
 * xq / xqs (optional, no reference counterpart): x already quantized by its producer (x then unused),
 * as q36_attn_proj's xq / xqs but in the layout q36_fp8_linear_act_frag(T, K) names. */
typedef struct q36_linear_seg {
  int32_t col0;
  int32_t ld;
  void* out;
} q36_linear_seg;
typedef struct q36_fp8_linear_args {
  int32_t T, N, K, n_out;
  const void* x;
  const void* w;
  const float* ws;
  int32_t nseg;
  q36_linear_seg seg[4];
  void* workspace;
  size_t workspace_bytes;
  const void* xq;
  const float* xqs;
} q36_fp8_linear_args;
/* 1 when q36_fp8_linear reads T tokens' activations of width K in fragment order (its tiled GEMM,
 * T >= 129 and K = 2048), 0 when row-major. */
int q36_fp8_linear_act_frag(int32_t T, int32_t K);
size_t q36_fp8_linear_workspace_bytes(int32_t T, int32_t K);
int q36_fp8_linear(const q36_fp8_linear_args* a, q36_stream_t stream);

/* ---- DENSE8 W8A16 linear: the reference's decode projections on its int8 copies (dense8 seg / part,
 * L/qk_proj_decode.cu:483-1102; L/dense8.py:229-401), for the verify row batches ----
 * x bf16 [T, K] (1 <= T <= 64), q int8 [N, K] row-major, s fp16 [K/128][s_ld] group-major (the layout
 * q36_quant_dense8 writes; s_ld >= N).  y[t, n] = bf16(acc): within each of up to 8 K chunks,
 * acc_c = fma(sum over the group's 128 columns of x * q (exact products, fp32 accumulation), s[g][n], acc_c)
 * over the chunk's groups in order; acc = the chunk sums added in chunk order.  Column
 * segments as q36_fp8_linear's (col0, ld multiples of 4, outputs 8-byte aligned).  N % 32 == 0,
 * K is 2048 or 4096 (the model's projection widths).  No workspace.
 * tiled (no reference counterpart): q is in the tile order q36_tile_w16 writes instead of row-major
 * (the same bytes reordered so that each 16-row x 64-column piece the kernel loads is 1 KB
 * contiguous); the results are the same bits. */
typedef struct q36_dense8_linear_args {
  int32_t T, N, K, n_out;
  const void* x;
  const void* q;
  const void* s;
  int64_t s_ld;
  int32_t nseg;
  q36_linear_seg seg[4];
  int32_t tiled;
} q36_dense8_linear_args;
int q36_dense8_linear(const q36_dense8_linear_args* a, q36_stream_t stream);
/* Row-major int8 q [N, K] -> the W8A16 tile order (prepare time; N % 16 == 0, K % 64 == 0): the 16-row x
 * 64-column piece (row tile i, column step j) at byte (i * K / 64 + j) * 1024, row r and columns
 * 16 g .. 16 g + 15 of it at byte 16 (r + 16 g) of the piece. */
int q36_tile_w16(const void* q, int64_t N, int32_t K, void* tiled, q36_stream_t stream);

/* ---- Fused residual add + Gemma RMSNorm between the hybrid layer's blocks: replaces the add-norm
 * of L/proj.py:60-81 (_add_norm_kernel) and the stock fused add-RMSNorm it reproduces ----
 * z = bf16 delta + residual in fp32 (delta NULL: z = residual); residual <- bf16(z) when delta is
 * given; out = bf16((z * rstd) * (1 + w)), rstd = 1 / sqrt(sum z^2 / H + eps) with the sum in the
 * fixed order lane l of 64 owns the 8-element chunks l + 64 j (fma from zero), then an xor
 * butterfly 32..1.  H = 2048; delta, residual, out and w 16-byte aligned.
 * q8 (optional, no reference counterpart): also the e4m3 codes of out per token x 128 channels, the
 * input q36_attn_proj takes as xq / xqs for the next layer's projection: q8 in fragment order when
 * q8_frag (then ceil(T/16)*16 tokens, padding zero), else row-major [T, 2048]; q8s fp32 [tokens, 16]. */
typedef struct q36_add_norm_args {
  int32_t T, H;
  const void* delta;
  void* residual;
  const void* norm_w;
  float eps;
  void* out;
  void* q8;
  float* q8s;
  int32_t q8_frag;
} q36_add_norm_args;
int q36_add_rmsnorm(const q36_add_norm_args* a, q36_stream_t stream);

/* ---- Decode / verify attention over the e4m3 KV cache: replaces attn_verify_kernel
 * (L/qk_attn_verify.cu:354-760) with its split count (L/attn_fused.py:110-124) ----
 * q bf16 [B*NT, HQ, D] (normed, roped, as q36_attn_proj writes it); k_cache, v_cache e4m3
 * [num_slots, HKV, D]; page_table int32 [B, pt_stride]: the cache slot of key position i (one-token
 * pages); seqlens int32 [B]: key positions of each request, its NT new tokens included (query token t
 * sees positions 0 .. seqlens - NT + t).  out_loc (optional) int64 [B*NT]: the slots the new tokens'
 * K/V rows (k_new, v_new e4m3 [B*NT, HKV, D], q36_attn_proj's k8 / v8) are written to first.
 * Scores s = (e4m3(q) . k) * scale, softmax weights rounded to f16 for P V, V widened to f16.
 * out bf16 [B*NT, HQ, D] = bf16(o / l), not gated (the o_proj applies the sigmoid gate).
 * gate / oq / oqs (optional, no reference counterpart: the o_proj's input quantization folded in):
 * with gate bf16 [B*NT, HQ*D] (q36_attn_proj's gate output), oq receives the e4m3 codes row-major
 * [B*NT, HQ*D] of bf16(out * sigmoid(gate)) per 128-channel group and oqs fp32 [B*NT, HQ*D/128] the
 * group scales (amax / 448): q36_attn_oproj's aq / aqs.
 * splits: 0 = min(64, CUs / (B * HKV)).  Constraints: HQ = 16, HKV = 2, D = 256, 1 <= NT <= 4,
 * num_slots * HKV * D < 2^31; q, caches 16-byte aligned. */
typedef struct q36_decode_args {
  int32_t B, NT, HQ, HKV, D, splits;
  const void* q;
  void* k_cache;
  void* v_cache;
  int64_t num_slots;
  const int32_t* page_table;
  int32_t pt_stride;
  const int32_t* seqlens;
  const int64_t* out_loc;
  const void* k_new;
  const void* v_new;
  float scale;
  void* out;
  void* workspace;
  size_t workspace_bytes;
  const void* gate;
  void* oq;
  float* oqs;
} q36_decode_args;
size_t q36_attn_decode_workspace_bytes(int32_t B, int32_t splits);
int q36_attn_decode(const q36_decode_args* a, q36_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Int8 lm_head fused with greedy argmax (H/w8a8.py:116-120 w8a8_linear + the stock argmax,
 * H/node.py:136-151).  h bf16 [R, H] (H = 2048) -> optional final Gemma RMSNorm (norm_w bf16 [H],
 * NULL to skip; y = bf16((h * rstd) * (1 + w))) -> per-row int8 (s = amax/127, half away) ->
 * acc = xq . wq^T (int32, wq int8 [V, H], ws fp32 [V]) -> logit = bf16((acc * xs) * ws) ->
 * ids int32 [R] = first index of the row's largest logit.  logits bf16 [R, V] is optional (NULL
 * skips the store); with logits_f32 nonzero it is fp32 [R, V] instead and receives the same
 * bf16-rounded values widened (stock's fp32 next_token_logits_buffer, H/node.py:68-88,136-149).  V % 16 == 0.  Workspace: q36_lmhead_workspace_bytes(R), 256-byte aligned
 * (enough for every mode).
 * mode Q36_LMH_W8A8X2: two activation terms (H/w8a8.py:25-37 quantize_act two_term, the reference's
 * arithmetic from 64 rows): q1, s1 as above, then q2, s2 the same rule on the residual
 * fma(-q1, s1, y); logit = bf16(fma(acc1, s1, acc2 * s2) * ws) (H/w8a8.py:66-70).
 * mode Q36_LMH_W8A16 (R <= 64, V % 32 == 0): the reference's arithmetic below 64 rows (H/lmhead8.py:57-91):
 * the bf16 rows (normed when norm_w is given) times the int8 weights widened exactly to bf16, fp32
 * accumulation, logit = bf16(acc * ws). */
#define Q36_LMH_W8A8 0
#define Q36_LMH_W8A8X2 1
#define Q36_LMH_W8A16 2
typedef struct q36_lmhead_args {
  int32_t R, H, V;
  const void* h;
  const void* norm_w;
  float eps;
  const int8_t* wq; /* row-major, or NULL with wq_t */
  const float* ws;
  int32_t* ids;
  void* logits;
  void* workspace;
  size_t workspace_bytes;
  int32_t mode; /* Q36_LMH_W8A8, Q36_LMH_W8A8X2 or Q36_LMH_W8A16 */
  int32_t logits_f32; /* 0: logits is bf16 [R, V]; nonzero: fp32 [R, V] (bf16-rounded values) */
  /* Optional (no reference counterpart): wq's codes in q36_tile_w16's order (each 16-row x 64-column
   * piece 1 KB contiguous, V % 16 == 0), read instead of wq by every mode, which may then be NULL; the
   * same bits out, faster (the weight loads read contiguous 1 KB pieces).  NULL: wq row-major. */
  const int8_t* wq_t;
} q36_lmhead_args;
size_t q36_lmhead_workspace_bytes(int32_t R);
int q36_lmhead_argmax(const q36_lmhead_args* a, q36_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Prepare-time weight quantizers (device to device).
 *   q36_quant_rows_i8:     w bf16 [N,K] -> q int8 [N,K], s fp32 [N]   (s = amax/127, half-away)
 *   q36_quant_blocks_e4m3: w bf16 [N,K] -> q e4m3 [N,K], s fp32 [N/128, K/128]
 *                          (s = amax/448, q = e4m3_rn_sat(w * (448/amax)))
 *   q36_pack_frag8:        8-bit codes (e4m3 or int8) [N,K] row-major -> packed, the MFMA
 *                          fragment order the MoE and attention kernels read: for row tile
 *                          r = n / 16 and block b = k / 128,
 *                          2048 bytes at (r * K/128 + b) * 2048; inside, byte h*1024 + 16*l + j
 *                          holds q[16 r + l % 16][128 b + 32 (l / 16) + 16 h + j] (h < 2, l < 64).
 * K % 128 == 0 (and N % 128 == 0 for blocks, N % 16 == 0 for the packing). */
int q36_quant_rows_i8(const void* w, int64_t N, int32_t K, int8_t* q, float* s, q36_stream_t stream);
int q36_quant_blocks_e4m3(const void* w, int64_t N, int32_t K, uint8_t* q, float* s, q36_stream_t stream);
int q36_pack_frag8(const void* q, int64_t N, int32_t K, void* packed, q36_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * The reference's prepare-time int8 weight formats (read only weights in, copies out).
 * Scale rule (both formats): s16 = fp16(fp32(amax / 127) * (1 + 2^-10)) per row or 128-group,
 * q = clamp(round_half_away(w / (s16 > 0 ? s16 : 1)), +-127).
 *
 * q8-block-v1 (L/i8x_kernels.py:12,69-110): per routed expert e one block of
 * q36_q8_block_v1_bytes(H, I) bytes at blocks + e * bytes:
 *   [q13 int8 [2I, H] | q2 int8 [H, I] | c13 fp16 [2I, H/128] | c2 fp16 [H, I/128]]
 * from bf16 w13 [E, 2I, H] (gate rows 0..I-1, up rows I..2I-1) and w2 [E, H, I].
 * channel = 1: one scale per row, written into all of the row's group slots (the reference's
 * SCALES = 'channel'); channel = 0: one scale per 128-group.  H, I multiples of 512 up to 4096.
 *
 * q36_import_q8_block_v1 reads a channel-mode copy back as the decode MoE's int8 experts
 * (q36_moe_args with dtype Q36_MOE_INT8): w13 [E, 2I, H] and w2 [E, H, I] codes in MFMA fragment
 * order (as q36_pack_frag8 writes them), s13 [E, 2I] and s2 [E, H] fp32 (each row's first group
 * slot widened exactly).  The shared expert is not part of the copy.
 *
 * DENSE8 (L/dense8.py:1-9,140-188): q int8 [N, K] row-major and fp16 scales group-major, scale of
 * row n and group g at s[g * s_ld + n] (s_ld >= N: s may be a column block of a wider buffer).
 * K a multiple of 512 up to 4096. */
size_t q36_q8_block_v1_bytes(int32_t H, int32_t I);
int q36_quant_q8_block_v1(const void* w13, const void* w2, int32_t E, int32_t H, int32_t I, int32_t channel,
                          void* blocks, q36_stream_t stream);
int q36_import_q8_block_v1(const void* blocks, int32_t E, int32_t H, int32_t I, void* w13, float* s13, void* w2,
                           float* s2, q36_stream_t stream);
int q36_quant_dense8(const void* w, int64_t N, int32_t K, void* q, void* s, int64_t s_ld, q36_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
