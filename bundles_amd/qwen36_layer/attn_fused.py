"""Fused gated full attention on libq36 (q36_attn_proj, q36_attn_decode, q36_attn_oproj).

Mirrors the reference's attention glue (R = qwen36_nodes_kb34, L = R/qwen36_layer): the fused
qkv projection + q/k norm + partial RoPE + e4m3 KV write (L/attn_fused.py:232-273,
L/qk_attn_verify.cu:765-797 attn_prefill_front), the decode / verify attention over the e4m3
KV cache with its split count (L/attn_fused.py:110-124 attn_verify_fused, L/qk_attn_verify.cu:354-760)
and the gated o_proj input (L/qk_attn_verify.cu:730-737).  Weights are e4m3 with 128x128 block
scales (prepare_weights).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from .. import _lib
from .._lib import AttnArgs, DecodeArgs, OprojArgs, check, ptr
from .moe import quantize_blocks_e4m3

N_Q_HEADS, N_KV_HEADS, HEAD_DIM, HIDDEN = 16, 2, 256, 2048
QKV_ROWS = 2 * N_Q_HEADS * HEAD_DIM + 2 * N_KV_HEADS * HEAD_DIM  # 9216


@dataclass
class AttnWeights:
    wqkv: torch.Tensor   # e4m3 codes [9216, 2048] (row-major)
    sqkv: torch.Tensor   # fp32 [72, 16]
    wo: torch.Tensor     # e4m3 codes [2048, 4096] (row-major)
    so: torch.Tensor     # fp32 [16, 32]
    wqkv_p: torch.Tensor = None  # the same codes in MFMA fragment order (what the kernels read)
    wo_p: torch.Tensor = None


def pack_frag(q: torch.Tensor, stream=None) -> torch.Tensor:
    """e4m3 codes [N, K] row-major -> the MFMA fragment order of q36_pack_frag8 (same bytes)."""
    N, K = q.shape
    out = torch.empty_like(q)
    check(_lib.lib().q36_pack_frag8(ptr(q), N, K, ptr(out), _lib.stream_handle(stream)), "q36_pack_frag8")
    return out


def prepare_weights(wqg: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor, wo: torch.Tensor) -> AttnWeights:
    """bf16 Wqg [8192,2048] (q/gate interleaved per head), Wk/Wv [512,2048], Wo [2048,4096] -> e4m3 blocks."""
    qkv = torch.cat([wqg, wk, wv], dim=0).contiguous()
    q, s = quantize_blocks_e4m3(qkv)
    qo, so = quantize_blocks_e4m3(wo.contiguous())
    return AttnWeights(q, s, qo, so, pack_frag(q), pack_frag(qo))


def rope_cos_sin(max_pos: int, theta: float = 1e7, rot_dim: int = 64, device="cpu") -> torch.Tensor:
    inv = theta ** (-torch.arange(0, rot_dim, 2, dtype=torch.float64) / rot_dim)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cat([ang.cos(), ang.sin()], dim=1).to(torch.float32).to(device)


@dataclass
class QuantRows:
    """e4m3 rows a producer kernel quantized for the next projection: codes per token x 128 channels
    (fragment order when frag, tokens padded to a multiple of 16) and fp32 scales [tokens, K/128]."""
    codes: torch.Tensor   # uint8 [tokens, K]
    scales: torch.Tensor  # fp32 [tokens, K / 128]
    T: int
    frag: bool

    @staticmethod
    def alloc(T: int, K: int, frag: bool, device) -> "QuantRows":
        n = (T + 15) // 16 * 16 if frag else T
        return QuantRows(torch.empty((n, K), dtype=torch.uint8, device=device),
                         torch.empty((n, K // 128), dtype=torch.float32, device=device), T, frag)


def proj_rows(T: int, device) -> QuantRows:
    """Buffers for q36_attn_proj's pre-quantized input of T tokens, in the layout it reads
    (q36_attn_act_frag); a producer (glue.add_rmsnorm, moe_row_batch's fused add-norm) fills them."""
    return QuantRows.alloc(T, HIDDEN, bool(_lib.lib().q36_attn_act_frag(T)), device)


def oproj_rows(T: int, device) -> QuantRows:
    """Buffers for q36_attn_oproj's pre-quantized input (row-major), filled by attn_decode(gate=...)."""
    return QuantRows.alloc(T, N_Q_HEADS * HEAD_DIM, False, device)


class Workspace:
    def __init__(self, T_max: int, device):
        L = _lib.lib()
        self.T_max = T_max
        self.proj = torch.empty(L.q36_attn_workspace_bytes(T_max), dtype=torch.uint8, device=device)
        self.oproj = torch.empty(L.q36_oproj_workspace_bytes(T_max), dtype=torch.uint8, device=device)


def attn_proj(x, w: AttnWeights, q_norm_w, k_norm_w, eps, cos_sin, positions, ws: Workspace, out=None, stream=None,
              xq: QuantRows | None = None, cache=None):
    """Returns dict(q, gate, k, v, k8, v8) for tokens x bf16 [T, 2048].  xq: the rows already quantized
    by their producer (proj_rows); x is then not read (may be None) and the projection skips its own
    quantization launch, with the same output bits.  cache = (k_cache, v_cache, out_loc): the new
    tokens' e4m3 K / V rows also go into the cache (e4m3 codes, uint8 [slots, 2, 256]) at slots out_loc
    (int64 [T]; slots outside the cache are skipped), as the reference's verify step writes them
    (L/qk_attn_verify.cu:431-465); attn_decode then needs no out_loc."""
    T = x.shape[0] if x is not None else xq.T
    if xq is not None and (xq.T != T or xq.frag != bool(_lib.lib().q36_attn_act_frag(T))):
        raise ValueError("attn_proj: xq was not made for this token count (proj_rows)")
    if T > ws.T_max:
        raise ValueError(f"attn_proj: {T} tokens exceed the workspace's {ws.T_max}")
    dev = x.device if x is not None else xq.codes.device
    o = out or dict(q=torch.empty((T, N_Q_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev),
                    gate=torch.empty((T, N_Q_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev),
                    k=torch.empty((T, N_KV_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev),
                    v=torch.empty((T, N_KV_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=dev),
                    k8=torch.empty((T, N_KV_HEADS, HEAD_DIM), dtype=torch.uint8, device=dev),
                    v8=torch.empty((T, N_KV_HEADS, HEAD_DIM), dtype=torch.uint8, device=dev))
    kc = vc = loc = None
    slots = 0
    if cache is not None:
        kc, vc, loc = cache
        for name, t in (("k_cache", kc), ("v_cache", vc)):
            if t.dtype != torch.uint8 or not t.is_contiguous() or t.dim() != 3 or tuple(t.shape[1:]) != (N_KV_HEADS,
                                                                                                      HEAD_DIM):
                raise ValueError(f"attn_proj: {name} must be contiguous uint8 [slots, {N_KV_HEADS}, {HEAD_DIM}]")
        if kc.shape != vc.shape:
            raise ValueError("attn_proj: k_cache and v_cache differ in shape")
        if loc.dtype != torch.int64 or not loc.is_contiguous() or loc.numel() < T:
            raise ValueError(f"attn_proj: out_loc must be contiguous int64 with at least {T} entries")
        slots = kc.shape[0]
    a = AttnArgs(T, cos_sin.shape[0], ptr(x), ptr(w.wqkv_p), ptr(w.sqkv), ptr(q_norm_w), ptr(k_norm_w), eps,
                 ptr(cos_sin), ptr(positions), ptr(o["q"]), ptr(o["gate"]), ptr(o["k"]), ptr(o["v"]), ptr(o["k8"]),
                 ptr(o["v8"]), ptr(ws.proj), ws.proj.numel(), ptr(None if xq is None else xq.codes),
                 ptr(None if xq is None else xq.scales), ptr(loc), ptr(kc), ptr(vc), slots)
    check(_lib.lib().q36_attn_proj(C.byref(a), _lib.stream_handle(stream)), "q36_attn_proj")
    return o


def attn_oproj(attn, gate, w: AttnWeights, ws: Workspace, out=None, stream=None, aq: QuantRows | None = None):
    """out bf16 [T, 2048] = o_proj(bf16(attn * sigmoid(gate))), attn / gate bf16 [T, 4096].  aq: that
    input already quantized by the attention (attn_decode(gate=..., oq=...)); attn, gate are then
    not read (may be None)."""
    T = attn.shape[0] if attn is not None else aq.T
    if aq is not None and (aq.T != T or aq.frag):
        raise ValueError("attn_oproj: aq must be row-major rows of this token count (oproj_rows)")
    dev = attn.device if attn is not None else aq.codes.device
    out = torch.empty((T, HIDDEN), dtype=torch.bfloat16, device=dev) if out is None else out
    a = OprojArgs(T, ptr(attn), ptr(gate), ptr(w.wo_p), ptr(w.so), ptr(out), ptr(ws.oproj), ws.oproj.numel(),
                  ptr(None if aq is None else aq.codes), ptr(None if aq is None else aq.scales))
    check(_lib.lib().q36_attn_oproj(C.byref(a), _lib.stream_handle(stream)), "q36_attn_oproj")
    return out


class DecodeWorkspace:
    """Split partials of q36_attn_decode for up to B_max requests at a fixed split count
    (0 = the library's default min(64, CUs / (B * 2)), resolved per call: the buffer is sized for
    the largest count any B <= B_max can take)."""

    def __init__(self, B_max: int, device, splits: int = 0):
        L = _lib.lib()
        self.B_max, self.splits = B_max, splits
        need = max(L.q36_attn_decode_workspace_bytes(b, splits) for b in range(1, B_max + 1))
        self.buf = torch.empty(need, dtype=torch.uint8, device=device)


def attn_decode(q, k_cache, v_cache, page_table, seqlens, NT: int, scale: float, ws: DecodeWorkspace,
                out_loc=None, k_new=None, v_new=None, out=None, stream=None, gate=None, oq: QuantRows | None = None):
    """Attention of B requests' NT new tokens over the e4m3 KV cache (one-token pages).

    q bf16 [B*NT, 16, 256]; k_cache / v_cache e4m3 codes (uint8) [slots, 2, 256]; page_table int32
    [B, >= max seqlens]; seqlens int32 [B] (new tokens included).  With out_loc (int64 [B*NT]) the
    new tokens' k_new / v_new rows are written into the cache first.  Returns bf16 [B*NT, 16, 256]
    = softmax(scale * e4m3(q) k^T) V per query head, causal among the new tokens, not gated.
    gate (bf16 [B*NT, 4096], attn_proj's gate) with oq (oproj_rows): the o_proj's input
    bf16(out * sigmoid(gate)) is also written there, quantized as attn_oproj would.
    """
    T = q.shape[0]
    if T % NT:
        raise ValueError(f"attn_decode: {T} query rows are not a multiple of NT={NT}")
    B = T // NT
    if B > ws.B_max:
        raise ValueError(f"attn_decode: {B} requests exceed the workspace's {ws.B_max}")
    for name, t, dt in (("q", q, torch.bfloat16), ("k_cache", k_cache, torch.uint8), ("v_cache", v_cache, torch.uint8),
                        ("page_table", page_table, torch.int32), ("seqlens", seqlens, torch.int32)):
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"attn_decode: {name} must be a contiguous {dt} tensor")
    if out_loc is not None and (out_loc.dtype != torch.int64 or k_new is None or v_new is None):
        raise ValueError("attn_decode: out_loc must be int64 and comes with k_new and v_new")
    if (gate is None) != (oq is None):
        raise ValueError("attn_decode: gate and oq go together")
    if oq is not None and (oq.T != T or oq.frag or gate.dtype != torch.bfloat16 or not gate.is_contiguous()
                           or gate.numel() != T * N_Q_HEADS * HEAD_DIM):
        raise ValueError("attn_decode: gate must be contiguous bf16 [T, 4096] and oq row-major rows (oproj_rows)")
    out = torch.empty_like(q) if out is None else out
    a = DecodeArgs(B, NT, q.shape[1], k_cache.shape[1], q.shape[2], ws.splits, ptr(q), ptr(k_cache), ptr(v_cache),
                   k_cache.shape[0], ptr(page_table), page_table.shape[1], ptr(seqlens), ptr(out_loc), ptr(k_new),
                   ptr(v_new), scale, ptr(out), ptr(ws.buf), ws.buf.numel(), ptr(gate),
                   ptr(None if oq is None else oq.codes), ptr(None if oq is None else oq.scales))
    check(_lib.lib().q36_attn_decode(C.byref(a), _lib.stream_handle(stream)), "q36_attn_decode")
    return out
