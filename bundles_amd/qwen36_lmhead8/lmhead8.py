"""Int8 lm_head with fused greedy argmax on libq36 (q36_lmhead_argmax, q36_quant_rows_i8).

Mirrors the reference's lm_head glue (R = qwen36_nodes_kb34, H = R/qwen36_lmhead8):
  quantize_rows       <- H/lmhead8.py:111 (per-row int8, fp32 scale amax/127, round half away)
  w8a8_lmhead_argmax  <- H/w8a8.py:116-120 w8a8_linear (one or two activation terms) and
                         H/lmhead8.py:57-91 (W8A16), with the greedy argmax of the stock sampler
                         (H/node.py:136-151) fused in; logits are returned only when asked for.
"""
from __future__ import annotations

import ctypes as C

import torch

from .. import _lib
from .._lib import LmheadArgs, check, ptr


def quantize_rows(w: torch.Tensor, stream=None):
    """bf16 [N, K] -> (int8 [N, K], fp32 scale [N]): s = amax / 127, codes rounded half away from
    zero (H/lmhead8.py:95-108,129-143), by q36_quant_rows_i8."""
    if w.dtype != torch.bfloat16 or w.dim() != 2 or not w.is_cuda:
        raise ValueError(f"quantize_rows: expects a 2-D bf16 CUDA tensor, got {w.dtype} {tuple(w.shape)}")
    w = w.contiguous()
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    s = torch.empty(N, dtype=torch.float32, device=w.device)
    check(_lib.lib().q36_quant_rows_i8(ptr(w), N, K, ptr(q), ptr(s), _lib.stream_handle(stream)), "q36_quant_rows_i8")
    return q, s


class Workspace:
    def __init__(self, R_max: int, device):
        self.R_max = R_max
        self.buf = torch.empty(_lib.lib().q36_lmhead_workspace_bytes(R_max), dtype=torch.uint8, device=device)


def tile_rows_w16(q: torch.Tensor, stream=None) -> torch.Tensor:
    """The int8 head [V, 2048] reordered into the tile order (q36_tile_w16): each 16-row x 64-column
    piece becomes 1 KB contiguous.  w8a8_lmhead_argmax(..., q_t=...) reads it in every mode, with the
    same bits out."""
    V, H = q.shape
    if q.dtype != torch.int8 or not q.is_contiguous() or V % 16 or H % 64:
        raise ValueError("tile_rows_w16: q must be contiguous int8 [V, H], V % 16 == 0, H % 64 == 0")
    out = torch.empty_like(q)
    check(_lib.lib().q36_tile_w16(ptr(q), V, H, ptr(out), _lib.stream_handle(stream)), "q36_tile_w16")
    return out


def w8a8_lmhead_argmax(h, q, scale, ws: Workspace, norm_w=None, eps: float = 1e-6, want_logits: bool = False,
                       ids=None, stream=None, two_term: bool = False, logits=None, w8a16: bool = False, q_t=None):
    """h bf16 [R, 2048] -> ids int32 [R] (and bf16 logits [R, V] when want_logits, into `logits` when
    given: bf16, or fp32 receiving the same bf16-rounded values, as the reference writes stock's fp32
    next_token_logits_buffer, H/node.py:68-88,136-149).  two_term: the reference's two-term activation
    form (H/w8a8.py:25-37); w8a16: the bf16 rows times the int8 weights unquantized (H/lmhead8.py:57-91;
    R <= 64, V a multiple of 32); q_t (optional): tile_rows_w16(q), read instead of q by every form, q
    may then be None (the same bits; 3-5 % faster for W8A8, 20-30 % for W8A16)."""
    R, H = h.shape
    if q is None and q_t is None:
        raise ValueError("w8a8_lmhead_argmax: q or q_t is required")
    V = (q if q is not None else q_t).shape[0]
    if R > ws.R_max:
        raise ValueError(f"w8a8_lmhead_argmax: {R} rows exceed the workspace's {ws.R_max}")
    for name, t, dt in (("h", h, torch.bfloat16), ("q", q, torch.int8), ("scale", scale, torch.float32),
                        ("q_t", q_t, torch.int8)):
        if t is not None and (t.dtype != dt or not t.is_contiguous()):
            raise ValueError(f"w8a8_lmhead_argmax: {name} must be contiguous {dt}")
    ids = torch.empty(R, dtype=torch.int32, device=h.device) if ids is None else ids
    if want_logits and logits is None:
        logits = torch.empty((R, V), dtype=torch.bfloat16, device=h.device)
    if logits is not None and (logits.dtype not in (torch.bfloat16, torch.float32) or tuple(logits.shape) != (R, V)
                               or not logits.is_contiguous()):
        raise ValueError(f"w8a8_lmhead_argmax: logits must be contiguous bf16 or fp32 [{R}, {V}]")
    if q_t is not None and (tuple(q_t.shape) != (V, H) or (q is not None and tuple(q.shape) != (V, H))):
        raise ValueError(f"w8a8_lmhead_argmax: q_t is tile_rows_w16(q), int8 [{V}, {H}]")
    a = LmheadArgs(R, H, V, ptr(h), ptr(norm_w), eps, ptr(q), ptr(scale), ptr(ids), ptr(logits), ptr(ws.buf),
                   ws.buf.numel(),
                   _lib.Q36_LMH_W8A16 if w8a16 else _lib.Q36_LMH_W8A8X2 if two_term else _lib.Q36_LMH_W8A8,
                   int(logits is not None and logits.dtype == torch.float32), ptr(q_t))
    check(_lib.lib().q36_lmhead_argmax(C.byref(a), _lib.stream_handle(stream)), "q36_lmhead_argmax")
    return (ids, logits) if (want_logits or logits is not None) else ids
