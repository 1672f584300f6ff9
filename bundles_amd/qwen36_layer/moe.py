"""Decode MoE row batch on libq36 (q36_moe_route / q36_moe_forward).

Mirrors the reference's decode MoE glue (R = qwen36_nodes_kb34, L = R/qwen36_layer):
  Workspace        <- L/i8x_decode.py:495-526 (persistent per-device scratch, zero on entry)
  ExpertWeights    <- the i8x expert copy (L/i8x_kernels.py:69-110, L/i8x_reloc.py:193-241):
                      here either int8 per-channel (W8A8) or e4m3 128x128 block-scaled weights
  prepare_experts  <- i8x_kernels.make_copy / fill_layer (quantize once at prepare time)
  route            <- qk_route.route (L/qk_route.cu:1124)
  moe_row_batch    <- i8x_decode.moe_row_batch (L/i8x_decode.py:528-605)
All launches go on the current torch stream; nothing allocates inside moe_row_batch except the
output tensor when the caller passes none (the reference does the same, L/i8x_decode.py:575).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from .. import _lib
from .._lib import MoeArgs, MoeWsLayout, Q36_MOE_FP8, Q36_MOE_INT8, check, ptr

MAX_TOKENS = 256  # the reference's row-batch limit (L/layer.py:50)


@dataclass
class ExpertWeights:
    """Quantized routed experts + shared expert of one MoE layer (device tensors)."""
    dtype: int                  # Q36_MOE_INT8 or Q36_MOE_FP8
    # the code tensors (w13, w2, sw13, sw2) hold their bytes in MFMA fragment order (pack_frag8);
    # unpack_frag8_np gives the row-major view
    w13: torch.Tensor           # [E, 2I, H] int8 / uint8 (e4m3 codes)
    s13: torch.Tensor           # INT8 [E, 2I]; FP8 [E, 2I/128, H/128]
    w2: torch.Tensor            # [E, H, I]
    s2: torch.Tensor            # INT8 [E, H]; FP8 [E, H/128, I/128]
    sw13: torch.Tensor          # [2I, H]
    ss13: torch.Tensor
    sw2: torch.Tensor           # [H, I]
    ss2: torch.Tensor

    @property
    def E(self) -> int:
        return self.w13.shape[0]

    @property
    def H(self) -> int:
        return self.w13.shape[2]

    @property
    def I(self) -> int:  # noqa: E743
        return self.w13.shape[1] // 2


def _bf16_weight(w: torch.Tensor, what: str) -> None:
    """The quantizers read 2-byte bf16 elements: any other dtype would be misread (an fp8 tensor
    would also be read past its end)."""
    if w.dtype != torch.bfloat16 or not w.is_cuda:
        raise ValueError(f"{what}: w must be a bf16 device tensor, got {w.dtype} on {w.device}")


def quantize_rows_i8(w: torch.Tensor, stream=None):
    """Per-row int8 (s = amax/127, round half away): w bf16 [N, K] -> (q int8 [N, K], s fp32 [N])."""
    _bf16_weight(w, "quantize_rows_i8")
    w2 = w.reshape(-1, w.shape[-1]).contiguous()
    N, K = w2.shape
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    s = torch.empty(N, dtype=torch.float32, device=w.device)
    check(_lib.lib().q36_quant_rows_i8(ptr(w2), N, K, ptr(q), ptr(s), _lib.stream_handle(stream)),
          "q36_quant_rows_i8")
    return q.view(w.shape), s.view(w.shape[:-1])


def quantize_blocks_e4m3(w: torch.Tensor, stream=None):
    """128x128 block e4m3: w bf16 [..., N, K] -> (q uint8 [..., N, K], s fp32 [..., N/128, K/128])."""
    _bf16_weight(w, "quantize_blocks_e4m3")
    N, K = w.shape[-2:]
    lead = w.shape[:-2]
    w2 = w.reshape(-1, K).contiguous()
    q = torch.empty(w2.shape, dtype=torch.uint8, device=w.device)
    s = torch.empty((w2.shape[0] // 128, K // 128), dtype=torch.float32, device=w.device)
    check(_lib.lib().q36_quant_blocks_e4m3(ptr(w2), w2.shape[0], K, ptr(q), ptr(s), _lib.stream_handle(stream)),
          "q36_quant_blocks_e4m3")
    return q.view(w.shape), s.view(*lead, N // 128, K // 128)


def pack_frag8(q: torch.Tensor, stream=None) -> torch.Tensor:
    """8-bit codes [..., N, K] row-major -> the MFMA fragment order of q36_pack_frag8 (same shape and
    bytes, reordered): 16-row tile t, 128-byte block b at (t * K/128 + b) * 2048; inside, byte
    h*1024 + 16*l + j holds row 16 t + l % 16, column 128 b + 32 (l / 16) + 16 h + j."""
    K = q.shape[-1]
    N = q.numel() // K
    out = torch.empty_like(q)
    check(_lib.lib().q36_pack_frag8(ptr(q), N, K, ptr(out), _lib.stream_handle(stream)), "q36_pack_frag8")
    return out


def unpack_frag8_np(p):
    """Host inverse of pack_frag8 (numpy array [..., N, K] in fragment order -> row-major)."""
    shape = p.shape
    K = shape[-1]
    N = p.size // K
    a = p.reshape(N // 16, K // 128, 2, 4, 16, 16)  # tile, block, half h, lane group, lane row, byte
    return a.transpose(0, 4, 1, 3, 2, 5).reshape(shape)


def prepare_experts(w13: torch.Tensor, w2: torch.Tensor, sw13: torch.Tensor, sw2: torch.Tensor,
                    dtype: int) -> ExpertWeights:
    """Quantize bf16 expert weights once (prepare time) and store the codes in MFMA fragment order.
    w13 [E,2I,H], w2 [E,H,I], shared [2I,H], [H,I]."""
    if dtype == Q36_MOE_INT8:
        q13, s13 = quantize_rows_i8(w13)
        q2, s2 = quantize_rows_i8(w2)
        qs13, ss13 = quantize_rows_i8(sw13)
        qs2, ss2 = quantize_rows_i8(sw2)
    elif dtype == Q36_MOE_FP8:
        q13, s13 = quantize_blocks_e4m3(w13)
        q2, s2 = quantize_blocks_e4m3(w2)
        qs13, ss13 = quantize_blocks_e4m3(sw13)
        qs2, ss2 = quantize_blocks_e4m3(sw2)
    else:
        raise ValueError(f"unknown MoE dtype {dtype}")
    return ExpertWeights(dtype, pack_frag8(q13), s13, pack_frag8(q2), s2, pack_frag8(qs13), ss13, pack_frag8(qs2), ss2)


def prepare_experts_q8_block_v1(blocks: torch.Tensor, H: int, I: int, sw13: torch.Tensor,  # noqa: E741
                                sw2: torch.Tensor) -> ExpertWeights:
    """The routed experts from the reference's channel-mode q8-block-v1 copy (L/i8x_kernels.py:69-141),
    read as they are (no re-quantization: the int8 codes and fp16 scales are the copy's); the shared
    expert, which the copy does not hold, quantized per channel as prepare_experts does."""
    from .formats import import_q8_block_v1
    w13, s13, w2, s2 = import_q8_block_v1(blocks, H, I)
    qs13, ss13 = quantize_rows_i8(sw13)
    qs2, ss2 = quantize_rows_i8(sw2)
    return ExpertWeights(Q36_MOE_INT8, w13, s13, w2, s2, pack_frag8(qs13), ss13, pack_frag8(qs2), ss2)


def prepare_experts_fp8_blocks(q13, s13, q2, s2, qs13, ss13, qs2, ss2) -> ExpertWeights:
    """The experts from already-quantized e4m3 128x128 blocks (an fp8 checkpoint's weight and
    weight_scale_inv: codes uint8 / float8_e4m3fn [.., N, K], fp32 scales [.., N/128, K/128]); only the
    codes are reordered for the MFMA."""
    def codes(t):
        return (t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t).contiguous()
    return ExpertWeights(Q36_MOE_FP8, pack_frag8(codes(q13)), s13.float().contiguous(), pack_frag8(codes(q2)),
                         s2.float().contiguous(), pack_frag8(codes(qs13)), ss13.float().contiguous(),
                         pack_frag8(codes(qs2)), ss2.float().contiguous())


def workspace_layout(M: int, E: int, H: int, I: int, topk: int, dtype: int) -> MoeWsLayout:  # noqa: E741
    L = MoeWsLayout()
    check(_lib.lib().q36_moe_workspace_layout(M, E, H, I, topk, dtype, C.byref(L)), "q36_moe_workspace_layout")
    return L


class Workspace:
    """Persistent per-device scratch for row batches of up to max_tokens rows (zeroed once)."""

    def __init__(self, E: int, H: int, I: int, topk: int, dtype: int, device, max_tokens: int = MAX_TOKENS):  # noqa: E741
        self.E, self.H, self.I, self.topk, self.dtype, self.max_tokens = E, H, I, topk, dtype, max_tokens
        nbytes = _lib.lib().q36_moe_workspace_bytes(max_tokens, E, H, I, topk, dtype)
        self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)

    def views(self, M: int) -> dict:
        """Typed views of the lists written by the last call with M rows (for tests and callers)."""
        L = workspace_layout(M, self.E, self.H, self.I, self.topk, self.dtype)
        b, E, k, S = self.buf, self.E, self.topk, M * self.topk

        def v(off, n, dt):
            nbytes = n * torch.empty((), dtype=dt).element_size()
            return b[off:off + nbytes].view(dt)
        ng = self.H // 128 if self.dtype == Q36_MOE_FP8 else 1
        return dict(
            logits=v(L.logits, M * E, torch.float32).view(M, E), ids=v(L.ids, S, torch.int32).view(M, k),
            wts=v(L.wts, S, torch.float32).view(M, k), counts=v(L.counts, E, torch.int32),
            offsets=v(L.offsets, E + 1, torch.int32), perm=v(L.perm, S, torch.int32),
            inv_perm=v(L.inv_perm, S, torch.int32), active=v(L.active, E, torch.int32),
            ctl=v(L.ctl, 64, torch.int32), xq=v(L.xq, M * self.H, torch.uint8).view(M, self.H),
            xs=v(L.xs, M * ng, torch.float32).view(M, ng),
            h=v(L.h, (S + M) * self.I, torch.bfloat16).view(S + M, self.I),
            y=v(L.y, (S + M) * self.H, torch.bfloat16).view(S + M, self.H))


def _args(x, positions, router_w, gate_w, ew, topk, ws: Workspace, out, router_bias, debug, norm=None, norm_q8=None,
          pre_norm=None):
    M, H = (x if x is not None else pre_norm[0]).shape
    if M > ws.max_tokens:
        raise ValueError(f"moe_row_batch: {M} rows exceed the workspace's {ws.max_tokens}")
    for name, t in (("x", x), ("router_w", router_w), ("gate_w", gate_w)):
        if t is not None and (t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError(f"moe_row_batch: {name} must be contiguous bfloat16")
    if positions is not None and (positions.dtype != torch.int32 or not positions.is_contiguous()):
        raise ValueError("moe_row_batch: positions must be contiguous int32")
    if router_bias is not None and (router_bias.dtype != torch.float32 or not router_bias.is_contiguous()):
        raise ValueError("moe_row_batch: router_bias must be contiguous float32")
    dbg = debug or {}
    w = [None] * 8 if ew is None else [ew.w13, ew.s13, ew.w2, ew.s2, ew.sw13, ew.ss13, ew.sw2, ew.ss2]
    resid = norm_w = norm_out = None
    eps = 0.0
    if norm is not None:
        resid, norm_w, eps, norm_out = norm
        for name, t in (("resid", resid), ("norm_out", norm_out)):
            if t.dtype != torch.bfloat16 or not t.is_contiguous() or tuple(t.shape) != (M, H):
                raise ValueError(f"moe_row_batch: {name} must be contiguous bfloat16 {(M, H)}")
        if norm_w.dtype != torch.bfloat16 or not norm_w.is_contiguous() or norm_w.numel() != H:
            raise ValueError(f"moe_row_batch: norm_w must be contiguous bfloat16 [{H}]")
    delta = r_in = r_out = in_w = None
    in_eps = 0.0
    if pre_norm is not None:
        delta, r_in, r_out, in_w, in_eps = pre_norm
        for name, t in (("delta", delta), ("resid_in", r_in), ("resid_out", r_out)):
            if t.dtype != torch.bfloat16 or not t.is_contiguous() or tuple(t.shape) != (M, H):
                raise ValueError(f"moe_row_batch: pre_norm {name} must be contiguous bfloat16 {(M, H)}")
        if in_w.dtype != torch.bfloat16 or not in_w.is_contiguous() or in_w.numel() != H:
            raise ValueError(f"moe_row_batch: pre_norm norm_w must be contiguous bfloat16 [{H}]")
    return MoeArgs(M, router_w.shape[0], H, ws.I, topk, ws.dtype, ptr(x), ptr(router_w), ptr(router_bias),
                   ptr(positions), *(ptr(t) for t in w), ptr(gate_w), ptr(out), ptr(ws.buf), ws.buf.numel(),
                   ptr(dbg.get("acc13")), ptr(dbg.get("acc2")), ptr(dbg.get("h")), ptr(resid), ptr(norm_w),
                   float(eps), ptr(norm_out), ptr(None if norm_q8 is None else norm_q8.codes),
                   ptr(None if norm_q8 is None else norm_q8.scales), int(norm_q8 is not None and norm_q8.frag),
                   ptr(delta), ptr(r_in), ptr(r_out), ptr(in_w), float(in_eps))


def route(x, positions, router_w, topk: int, ws: Workspace, router_bias=None, stream=None):
    """Routing only (ids, weights, expert lists and quantized x in the workspace); returns ws.views(M)."""
    a = _args(x, positions, router_w, None, None, topk, ws, None, router_bias, None)
    check(_lib.lib().q36_moe_route(C.byref(a), _lib.stream_handle(stream)), "q36_moe_route")
    return ws.views(x.shape[0])


def moe_row_batch(x, positions, router_w, gate_w, ew: ExpertWeights, topk: int, ws: Workspace, out=None,
                  router_bias=None, debug=None, stream=None, norm=None, norm_q8=None, pre_norm=None):
    """out[M, H] = shared_gate * shared_expert(x) + sum_j w_j * expert_{id_j}(x)  (bf16).

    norm = (resid, norm_w, eps, norm_out) fuses the next block's input add-norm into the combine:
    resid <- bf16(out + resid) in place and norm_out = its Gemma RMSNorm, the same bits as
    glue.add_rmsnorm(out, resid, norm_w, eps) after the block (L/qk_route.cu:630-820 combine_norm).
    norm_q8 (attn_fused.QuantRows, with norm): norm_out's e4m3 codes for the next projection.
    pre_norm = (delta, resid_in, resid_out, norm_w, eps) runs this block's own input add-norm in the
    route kernel: resid_out <- bf16(delta + resid_in) and x = its Gemma RMSNorm, the same bits as
    glue.add_rmsnorm(delta, resid, norm_w, eps, out=x) before the block; x is then an optional
    output (None, or a tensor that receives those rows).  resid_out must be another buffer than
    resid_in and delta (the route reads them while it writes)."""
    if ew.E != router_w.shape[0] or ew.I != ws.I or ew.dtype != ws.dtype or ew.E != ws.E:
        raise ValueError("moe_row_batch: expert weights, router and workspace disagree on E / I / dtype")
    if x is None and pre_norm is None:
        raise ValueError("moe_row_batch: x is required without pre_norm")
    shape_src = x if x is not None else pre_norm[0]
    if out is None:
        out = torch.empty_like(shape_src)
    if norm_q8 is not None and (norm is None or norm_q8.T != shape_src.shape[0]):
        raise ValueError("moe_row_batch: norm_q8 needs the fused add-norm and one row per token")
    a = _args(x, positions, router_w, gate_w, ew, topk, ws, out, router_bias, debug, norm, norm_q8, pre_norm)
    check(_lib.lib().q36_moe_forward(C.byref(a), _lib.stream_handle(stream)), "q36_moe_forward")
    return out


def moe_phases(x, positions, router_w, gate_w, ew: ExpertWeights, topk: int, ws: Workspace, out, router_bias=None,
               stream=None):
    """The same block as moe_row_batch as four separately launched phases (route, up, down, combine);
    returns the list of (name, callable) so a caller can schedule or time each one."""
    a = _args(x, positions, router_w, gate_w, ew, topk, ws, out, router_bias, None)
    L = _lib.lib()
    # the argument struct holds raw device addresses: the callables keep the tensors they point into
    # alive, so a caller that drops its own references does not leave them pointing at freed memory
    keep = (x, positions, router_w, gate_w, ew, ws, out, router_bias)

    def call(fn, name):
        def run(_keep=keep):
            check(fn(C.byref(a), _lib.stream_handle(stream)), name)
        return run
    return [("route", call(L.q36_moe_route, "q36_moe_route")), ("up", call(L.q36_moe_up, "q36_moe_up")),
            ("down", call(L.q36_moe_down, "q36_moe_down")), ("combine", call(L.q36_moe_combine, "q36_moe_combine"))]
