"""The hybrid layer's glue on libq36: the e4m3 block-scaled linear with column-segmented outputs
(q36_fp8_linear), the W8A16 linear on DENSE8 int8 copies (q36_dense8_linear) and the fused residual
add + Gemma RMSNorm (q36_add_rmsnorm).

Mirrors the reference's decode projections and add-norm (R = qwen36_nodes_kb34, L = R/qwen36_layer):
gdn_in_proj / qkv_proj with their outputs split by column (L/qk_proj_decode.cu:409,434; the DENSE8
seg kernel L/qk_proj_decode.cu:483-1102, L/dense8.py:317-353), the out_proj / o_proj before the
add-norm and the add-norm itself (L/proj.py:60-112 project_add_norm).  The weights are e4m3 with
128x128 block scales (the configuration's format), prepared once by prepare_fp8_weight.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from .. import _lib
from .._lib import AddNormArgs, Dense8LinearArgs, Fp8LinearArgs, check, ptr
from .moe import pack_frag8, quantize_blocks_e4m3


@dataclass
class Fp8Weight:
    q: torch.Tensor    # e4m3 codes [N_pad, K] row-major (rows past n are zero)
    s: torch.Tensor    # fp32 [N_pad / 128, K / 128]
    qp: torch.Tensor   # the same codes in MFMA fragment order (what the kernel reads)
    n: int             # output columns (rows of the unpadded weight)


def prepare_fp8_weight(w: torch.Tensor) -> Fp8Weight:
    """bf16 [N, K] -> e4m3 128x128 blocks, rows padded with zeros to a multiple of 128."""
    N, K = w.shape
    npad = (N + 127) // 128 * 128
    if npad != N:
        w = torch.cat([w, torch.zeros((npad - N, K), dtype=w.dtype, device=w.device)], dim=0)
    q, s = quantize_blocks_e4m3(w.contiguous())
    return Fp8Weight(q, s, pack_frag8(q), N)


def fp8_weight_from_blocks(q: torch.Tensor, s: torch.Tensor) -> Fp8Weight:
    """An fp8 checkpoint's e4m3 weight [N, K] (uint8 codes or float8_e4m3fn) and its 128x128 block
    weight_scale_inv [ceil(N/128), K/128] as they are (the same pair prepare_fp8_weight makes from bf16);
    rows padded with zero codes to a multiple of 128, the codes reordered for the MFMA."""
    q = q.view(torch.uint8) if q.dtype == torch.float8_e4m3fn else q
    N, K = q.shape
    npad = (N + 127) // 128 * 128
    if q.dtype != torch.uint8 or K % 128 or tuple(s.shape) != (npad // 128, K // 128):
        raise ValueError(f"fp8_weight_from_blocks: codes [N, K] and scales [N/128, K/128], got {tuple(q.shape)} "
                         f"{q.dtype} / {tuple(s.shape)}")
    if npad != N:
        q = torch.cat([q, torch.zeros((npad - N, K), dtype=torch.uint8, device=q.device)], dim=0)
    q = q.contiguous()
    return Fp8Weight(q, s.float().contiguous(), pack_frag8(q), N)


class LinearWorkspace:
    """The activation codes and scales of q36_fp8_linear for up to T_max tokens of width K."""

    def __init__(self, T_max: int, K: int, device):
        self.T_max, self.K = T_max, K
        self.buf = torch.empty(_lib.lib().q36_fp8_linear_workspace_bytes(T_max, K), dtype=torch.uint8, device=device)


def linear_rows(T: int, K: int, device):
    """Buffers for fp8_linear's pre-quantized input of T tokens of width K, in the layout it reads
    (q36_fp8_linear_act_frag); a producer (add_rmsnorm, the MoE's fused add-norm) fills them."""
    from .attn_fused import QuantRows
    return QuantRows.alloc(T, K, bool(_lib.lib().q36_fp8_linear_act_frag(T, K)), device)


def fp8_linear(x: torch.Tensor, w: Fp8Weight, ws: LinearWorkspace, segments=None, stream=None, xq=None):
    """y = x . W^T (bf16), x bf16 [T, K].

    segments: None (returns one [T, n] tensor) or a list of (col0, out) with out a bf16 [T, width]
    view whose rows may be strided (row stride = out.stride(0)); columns col0 .. col0 + width of y
    land in it.  The segments must tile [0, n) in order.  xq (linear_rows): x already quantized by its
    producer; x is then not read (may be None), with the same output bits.
    """
    if x is None:
        T, K = xq.T, xq.codes.shape[1]
    else:
        T, K = x.shape
    if xq is not None and (xq.T != T or xq.codes.shape[1] != K or
                           xq.frag != bool(_lib.lib().q36_fp8_linear_act_frag(T, K))):
        raise ValueError("fp8_linear: xq was not made for this input (linear_rows)")
    if T > ws.T_max or K != ws.K:
        raise ValueError(f"fp8_linear: [{T}, {K}] does not fit the workspace ({ws.T_max}, {ws.K})")
    if segments is None:
        out = torch.empty((T, w.n), dtype=torch.bfloat16, device=w.qp.device)
        segments, ret = [(0, out)], out
    else:
        ret = None
    segs = _segments("fp8_linear", T, w.n, segments)
    a = Fp8LinearArgs(T, w.qp.shape[0], K, w.n, ptr(x), ptr(w.qp), ptr(w.s), len(segments), segs,
                      ptr(ws.buf), ws.buf.numel(), ptr(None if xq is None else xq.codes),
                      ptr(None if xq is None else xq.scales))
    check(_lib.lib().q36_fp8_linear(C.byref(a), _lib.stream_handle(stream)), "q36_fp8_linear")
    return ret


def _segments(fn: str, T: int, n: int, segments):
    if not 1 <= len(segments) <= 4:
        raise ValueError(f"{fn}: 1 to 4 segments")
    end = 0
    segs = (_lib.LinearSeg * 4)()
    for i, (c0, o) in enumerate(segments):
        if c0 != end or o.dtype != torch.bfloat16 or o.shape[0] != T or o.stride(1) != 1:
            raise ValueError(f"{fn}: segment {i} (col0 {c0}) must continue at column {end} as bf16 [T, w]")
        segs[i] = _lib.LinearSeg(c0, o.stride(0), o.data_ptr())
        end = c0 + o.shape[1]
    if end != n:
        raise ValueError(f"{fn}: segments cover {end} of {n} columns")
    return segs


def dense8_linear(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, segments=None, stream=None, tiled=False):
    """y = x . dequant(q, s)^T (bf16) on a DENSE8 copy (formats.quant_dense8: q int8 [N, K], s fp16
    [K/128, >= N] group-major, possibly a column block of a wider buffer), x bf16 [T, K], T <= 64.
    segments as fp8_linear's.  The reference's decode W8A16 projections (L/dense8.py:229-265).
    tiled: q is formats.tile_w16's reordering of the copy (same bits out, 1 KB contiguous loads)."""
    T, K = x.shape
    N = q.shape[0]
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("dense8_linear: x must be contiguous bf16 [T, K]")
    if (q.dtype != torch.int8 or not q.is_contiguous() or q.shape[1] != K or s.dtype != torch.float16
            or s.dim() != 2 or s.shape[0] != K // 128 or s.shape[1] < N or s.stride(1) != 1):
        raise ValueError(f"dense8_linear: the copy must be q int8 [N, {K}] and s fp16 [{K // 128}, >= N]")
    if segments is None:
        out = torch.empty((T, N), dtype=torch.bfloat16, device=x.device)
        segments, ret = [(0, out)], out
    else:
        ret = None
    segs = _segments("dense8_linear", T, N, segments)
    a = Dense8LinearArgs(T, N, K, N, ptr(x), ptr(q), ptr(s), s.stride(0), len(segments), segs, int(bool(tiled)))
    check(_lib.lib().q36_dense8_linear(C.byref(a), _lib.stream_handle(stream)), "q36_dense8_linear")
    return ret


def add_rmsnorm(delta, residual: torch.Tensor, norm_w: torch.Tensor, eps: float, out=None, stream=None, q8=None):
    """residual += delta (bf16, in place; delta None: residual unchanged); returns the Gemma-normalised
    rows bf16((z * rstd) * (1 + w)) of z = delta + residual in fp32.  q8 (attn_fused.QuantRows of T
    rows): the rows' e4m3 codes also go there, as the next projection reads them."""
    T, H = residual.shape
    out = torch.empty_like(residual) if out is None else out
    if q8 is not None and (q8.T != T or q8.codes.shape[1] != H):
        raise ValueError("add_rmsnorm: q8 rows do not match the residual")
    a = AddNormArgs(T, H, ptr(delta), ptr(residual), ptr(norm_w), eps, ptr(out),
                    ptr(None if q8 is None else q8.codes), ptr(None if q8 is None else q8.scales),
                    int(q8 is not None and q8.frag))
    check(_lib.lib().q36_add_rmsnorm(C.byref(a), _lib.stream_handle(stream)), "q36_add_rmsnorm")
    return out
