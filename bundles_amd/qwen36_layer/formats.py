"""The reference's prepare-time int8 weight formats on libq36, and the bridges into this build's nodes.

Mirrors (R = qwen36_nodes_kb34, L = R/qwen36_layer):
  quant_q8_block_v1   <- i8x_kernels.make_copy / fill_layer / quantize_channel (L/i8x_kernels.py:12,69-141):
                         the q8-block-v1 expert copy, one block per routed expert
  q8_block_parts      <- i8x_kernels.block_parts (L/i8x_kernels.py:99-103)
  import_q8_block_v1  <- the copy read back as the decode MoE's int8 experts (q36_import_q8_block_v1)
  quant_dense8        <- dense8.quantize (L/dense8.py:168-188): int8 rows + group-major fp16 scales
The fp8 128x128 block format needs no converter: an e4m3 checkpoint's (weight, weight_scale_inv)
pair is the (codes, scales) pair the fp8 nodes take; moe.prepare_experts_fp8_blocks and
glue.fp8_weight_from_blocks only reorder the codes for the MFMA.
"""
from __future__ import annotations

import torch

from .. import _lib
from .._lib import check, ptr

GROUP = 128


def q8_block_v1_bytes(H: int, I: int) -> int:  # noqa: E741
    return int(_lib.lib().q36_q8_block_v1_bytes(H, I))


def quant_q8_block_v1(w13: torch.Tensor, w2: torch.Tensor, channel: bool = True, out=None, stream=None):
    """bf16 w13 [E, 2I, H], w2 [E, H, I] -> uint8 blocks [E, q8_block_v1_bytes(H, I)]."""
    E, I2, H = w13.shape
    I = I2 // 2  # noqa: E741
    if w13.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16 or tuple(w2.shape) != (E, H, I):
        raise ValueError(f"quant_q8_block_v1: bf16 w13 [E, 2I, H] and w2 [E, H, I], got {tuple(w13.shape)} / "
                         f"{tuple(w2.shape)}")
    w13, w2 = w13.contiguous(), w2.contiguous()
    out = torch.empty((E, q8_block_v1_bytes(H, I)), dtype=torch.uint8, device=w13.device) if out is None else out
    check(_lib.lib().q36_quant_q8_block_v1(ptr(w13), ptr(w2), E, H, I, int(channel), ptr(out),
                                           _lib.stream_handle(stream)), "q36_quant_q8_block_v1")
    return out


def q8_block_parts(block: torch.Tensor, H: int, I: int):  # noqa: E741
    """Views (q13 int8 [2I, H], q2 int8 [H, I], c13 fp16 [2I, H/128], c2 fp16 [H, I/128]) of one block."""
    o2, oc13 = 2 * I * H, 3 * I * H
    oc2 = oc13 + 2 * I * (H // GROUP) * 2
    eb = q8_block_v1_bytes(H, I)
    return (block[:o2].view(torch.int8).view(2 * I, H), block[o2:oc13].view(torch.int8).view(H, I),
            block[oc13:oc2].view(torch.float16).view(2 * I, H // GROUP),
            block[oc2:eb].view(torch.float16).view(H, I // GROUP))


def import_q8_block_v1(blocks: torch.Tensor, H: int, I: int, stream=None):  # noqa: E741
    """A channel-mode q8-block-v1 copy -> (w13, s13, w2, s2) of the decode MoE's int8 experts: codes in
    MFMA fragment order, fp32 per-channel scales."""
    E = blocks.shape[0]
    if blocks.dtype != torch.uint8 or blocks.dim() != 2 or blocks.shape[1] != q8_block_v1_bytes(H, I) or \
            not blocks.is_contiguous():
        raise ValueError("import_q8_block_v1: blocks must be contiguous uint8 [E, q8_block_v1_bytes(H, I)]")
    dev = blocks.device
    w13 = torch.empty((E, 2 * I, H), dtype=torch.int8, device=dev)
    w2 = torch.empty((E, H, I), dtype=torch.int8, device=dev)
    s13 = torch.empty((E, 2 * I), dtype=torch.float32, device=dev)
    s2 = torch.empty((E, H), dtype=torch.float32, device=dev)
    check(_lib.lib().q36_import_q8_block_v1(ptr(blocks), E, H, I, ptr(w13), ptr(s13), ptr(w2), ptr(s2),
                                            _lib.stream_handle(stream)), "q36_import_q8_block_v1")
    return w13, s13, w2, s2


def quant_dense8(w: torch.Tensor, q=None, s=None, stream=None):
    """bf16 w [N, K] -> (q int8 [N, K], s fp16 [K/128, N]); s may be a column block of a wider buffer
    (its row stride is taken from s.stride(0)), as the reference stacks the GDN in_proj copies."""
    N, K = w.shape
    if w.dtype != torch.bfloat16 or not w.is_contiguous():
        raise ValueError(f"quant_dense8: w must be contiguous bf16 [N, K], got {w.dtype} {tuple(w.shape)}")
    q = torch.empty((N, K), dtype=torch.int8, device=w.device) if q is None else q
    s = torch.empty((K // GROUP, N), dtype=torch.float16, device=w.device) if s is None else s
    if tuple(q.shape) != (N, K) or q.dtype != torch.int8 or not q.is_contiguous() or \
            tuple(s.shape) != (K // GROUP, N) or s.dtype != torch.float16 or s.stride(1) != 1:
        raise ValueError("quant_dense8: q/s buffers have the wrong shape, dtype or layout")
    check(_lib.lib().q36_quant_dense8(ptr(w), N, K, ptr(q), ptr(s), s.stride(0), _lib.stream_handle(stream)),
          "q36_quant_dense8")
    return q, s


def tile_w16(q: torch.Tensor, stream=None) -> torch.Tensor:
    """A DENSE8 copy's int8 rows [N, K] reordered into the W8A16 kernel's tile order (q36_tile_w16):
    each 16-row x 64-column piece the kernel loads at once becomes 1 KB contiguous.  The scales keep
    their group-major layout; glue.dense8_linear(..., tiled=True) reads the result."""
    N, K = q.shape
    if q.dtype != torch.int8 or not q.is_contiguous():
        raise ValueError("tile_w16: q must be contiguous int8 [N, K]")
    out = torch.empty_like(q)
    check(_lib.lib().q36_tile_w16(ptr(q), N, K, ptr(out), _lib.stream_handle(stream)), "q36_tile_w16")
    return out
