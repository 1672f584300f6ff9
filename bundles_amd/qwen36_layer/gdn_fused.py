"""GDN speculative verify on libq36.

Mirrors the reference's glue (R = qwen36_nodes_kb34, L = R/qwen36_layer): gdn_verify_fused
(L/gdn_fused.py:37-57 -> L/qk_gdn_verify.cu:841).  Two forms:
  gdn_verify_fused  (q36_gdn_verify)      every position's fp32 state (snapshots) and the rolled
                                           conv state out of place;
  gdn_verify_ring   (q36_gdn_verify_ring) the served ReplaySSM form: a read-only checkpoint plus
                                           the 16-entry (d, k, g) ring, conv state rolled in place,
                                           with the reference kernel's argument list.
"""
from __future__ import annotations

import ctypes as C

import torch

from .. import _lib
from .._lib import GdnArgs, GdnRingArgs, check, ptr

HEAD_K, HEAD_V, N_K_HEADS, N_V_HEADS = 128, 128, 16, 32
QKV_DIM = 2 * N_K_HEADS * HEAD_K + N_V_HEADS * HEAD_V  # 8192


def _req(t, name, dtype, shape):
    if t.dtype != dtype or not t.is_contiguous() or tuple(t.shape) != tuple(shape):
        raise ValueError(f"gdn_verify_fused: {name} must be contiguous {dtype} {tuple(shape)}, got "
                         f"{t.dtype} {tuple(t.shape)}")


def gdn_verify_fused(mixed, z, a, b, conv_state, conv_w, A_log, dt_bias, S0, norm_w, eps: float = 1e-6,
                     T: int | None = None, out=None, snaps=None, conv_state_out=None, stream=None):
    """One verify step over B sequences x T positions.

    Returns (out bf16 [B*T, 4096], snaps fp32 [B, T, 32, 128, 128], conv_state_out bf16 [B, 8192, 3])."""
    B = S0.shape[0]
    T = T if T is not None else mixed.shape[0] // B
    R = B * T
    _req(mixed, "mixed", torch.bfloat16, (R, QKV_DIM))
    _req(z, "z", torch.bfloat16, (R, N_V_HEADS * HEAD_V))
    _req(a, "a", torch.bfloat16, (R, N_V_HEADS))
    _req(b, "b", torch.bfloat16, (R, N_V_HEADS))
    _req(conv_state, "conv_state", torch.bfloat16, (B, QKV_DIM, 3))
    _req(conv_w, "conv_w", torch.bfloat16, (QKV_DIM, 4))
    _req(A_log, "A_log", torch.float32, (N_V_HEADS,))
    _req(dt_bias, "dt_bias", torch.float32, (N_V_HEADS,))
    _req(S0, "S0", torch.float32, (B, N_V_HEADS, HEAD_V, HEAD_K))
    _req(norm_w, "norm_w", torch.bfloat16, (HEAD_V,))
    dev = mixed.device
    out = torch.empty((R, N_V_HEADS * HEAD_V), dtype=torch.bfloat16, device=dev) if out is None else out
    snaps = torch.empty((B, T, N_V_HEADS, HEAD_V, HEAD_K), dtype=torch.float32, device=dev) if snaps is None \
        else snaps
    conv_state_out = torch.empty_like(conv_state) if conv_state_out is None else conv_state_out
    args = GdnArgs(B, T, ptr(mixed), ptr(z), ptr(a), ptr(b), ptr(conv_state), ptr(conv_state_out), ptr(conv_w),
                   ptr(A_log), ptr(dt_bias), ptr(S0), ptr(norm_w), eps, ptr(out), ptr(snaps))
    check(_lib.lib().q36_gdn_verify(C.byref(args), _lib.stream_handle(stream)), "q36_gdn_verify")
    return out, snaps, conv_state_out


RING = 16


def _pool(t, name, dtype, tail, inner_strides):
    """A slot pool [slots, *tail] with the given innermost strides (the slot stride is free but a
    multiple of 8 elements), as the reference's host checks require (L/qk_gdn_verify.cu:872-904)."""
    if t.dtype != dtype or t.dim() != 1 + len(tail) or tuple(t.shape[1:]) != tuple(tail) or \
            tuple(t.stride()[1:]) != tuple(inner_strides) or t.stride(0) % 8 != 0:
        raise ValueError(f"gdn_verify_ring: {name} must be a {dtype} [slots, {', '.join(map(str, tail))}] pool with "
                         f"contiguous heads, got {t.dtype} {tuple(t.shape)} strides {t.stride()}")


def _idx(t, name, n):
    if t.dim() != 1 or t.numel() < n or not t.is_contiguous() or t.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"gdn_verify_ring: {name} must hold at least {n} int32/int64 indices")
    return 1 if t.dtype == torch.int64 else 0


def gdn_verify_ring(mixed, z, a, b, conv_state, conv_w, window, A_log, dt_bias, h0, d_ring, dlo_ring, k_ring,
                    klo_ring, g_ring, qsl, state_idx, replay_idx, win_idx, write_pos, cache_base, norm_w,
                    eps: float = 1e-6, scale: float = HEAD_K ** -0.5, pf_weight=None, *, T: int = 4, out=None,
                    stream=None, oq=None):
    """out_proj's input [rows, 4096] for a verify batch over the ReplaySSM ring.

    The argument list is the reference kernel's (L/qk_gdn_verify.cu:841-849).  rows = B * T with T the
    draft window (the reference serves T = 4); request r owns rows qsl[r] .. qsl[r] + T - 1.
    conv_state, window and the five rings are updated in place; h0 is read only.  window is either
    the [wslots, 8192, T + 2] record pool or the reference's deduplicated [wslots, T, 8192, 3] view
    of it.  pf_weight is the reference's L2-prefetch hint (no effect on results) and is ignored.
    oq (glue.linear_rows(rows, 4096)): out's e4m3 codes also go there, the out_proj's pre-quantized input.
    Raises ValueError on a layout the kernel does not serve, RuntimeError when the library
    rejects the call."""
    rows = mixed.shape[0]
    if not 1 <= T <= 8 or rows % T:
        raise ValueError(f"gdn_verify_ring: {rows} verify rows are not a multiple of the draft window {T} (1..8)")
    B = rows // T
    _req(mixed, "mixed_qkv", torch.bfloat16, (rows, QKV_DIM))
    if z.dtype != torch.bfloat16 or z.numel() != rows * N_V_HEADS * HEAD_V or not z.is_contiguous():
        raise ValueError("gdn_verify_ring: z must be contiguous bf16 [rows, 32, 128]")
    _req(a, "a", torch.bfloat16, (rows, N_V_HEADS))
    _req(b, "b", torch.bfloat16, (rows, N_V_HEADS))
    _pool(conv_state, "conv_state", torch.bfloat16, (QKV_DIM, 3), (3, 1))
    _req(conv_w, "conv_weights", torch.bfloat16, (QKV_DIM, 4))
    if window.dim() == 4:  # the deduplicated [wslots, T, 8192, 3] view of [wslots, 8192, T + 2]
        if tuple(window.shape[1:]) != (T, QKV_DIM, 3) or tuple(window.stride()[1:]) != (1, T + 2, 1):
            raise ValueError("gdn_verify_ring: conv windows must be the deduplicated [slots, T, 8192, 3] view of "
                             "[slots, 8192, T + 2]")
        if window.stride(0) % 8:
            raise ValueError("gdn_verify_ring: the window slot stride must be a multiple of 8")
    else:
        _pool(window, "intermediate_conv_window", torch.bfloat16, (QKV_DIM, T + 2), (T + 2, 1))
    _req(A_log, "A_log", torch.float32, (N_V_HEADS,))
    if dt_bias.dtype not in (torch.float32, torch.bfloat16) or dt_bias.numel() != N_V_HEADS or \
            not dt_bias.is_contiguous():
        raise ValueError("gdn_verify_ring: dt_bias must hold 32 fp32 or bf16 values")
    if h0.dtype != torch.float32 or h0.dim() != 4 or tuple(h0.shape[1:]) != (N_V_HEADS, HEAD_V, HEAD_K) or \
            not h0.is_contiguous():
        raise ValueError("gdn_verify_ring: the checkpoint must be a contiguous fp32 [slots, 32, 128, 128] pool")
    for t, n in ((d_ring, "d ring"), (dlo_ring, "d ring (low parts)")):
        _pool(t, n, torch.bfloat16, (N_V_HEADS, RING, HEAD_V), (RING * HEAD_V, HEAD_V, 1))
    for t, n in ((k_ring, "k ring"), (klo_ring, "k ring (low parts)")):
        _pool(t, n, torch.bfloat16, (N_K_HEADS, RING, HEAD_K), (RING * HEAD_K, HEAD_K, 1))
    if g_ring.dtype != torch.float32 or tuple(g_ring.shape[1:]) != (N_V_HEADS, RING) or \
            tuple(g_ring.stride()[1:]) != (RING, 1) or g_ring.stride(0) % 4:
        raise ValueError("gdn_verify_ring: g ring must be an fp32 [slots, 32, 16] pool")
    if qsl.dtype != torch.int32 or qsl.numel() < B + 1 or not qsl.is_contiguous():
        raise ValueError("gdn_verify_ring: query_start_loc must hold B + 1 int32 offsets")
    flags = (_idx(state_idx, "mamba_cache_indices", B) | _idx(replay_idx, "req_pool_indices", B) << 1 |
             _idx(win_idx, "verify_intermediate_state_indices", B) << 2)
    rslots = min(d_ring.shape[0], dlo_ring.shape[0], k_ring.shape[0], klo_ring.shape[0], g_ring.shape[0])
    for t, n in ((write_pos, "write_pos"), (cache_base, "cache_base")):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.numel() < rslots:
            raise ValueError(f"gdn_verify_ring: ring cursor {n} must be contiguous int32 [ring slots]")
    _req(norm_w, "norm weight", torch.bfloat16, (HEAD_V,))
    out = torch.empty((rows, N_V_HEADS * HEAD_V), dtype=torch.bfloat16, device=mixed.device) if out is None else out
    _req(out, "out", torch.bfloat16, (rows, N_V_HEADS * HEAD_V))
    if oq is not None and (oq.T != rows or oq.frag or oq.codes.shape[1] != N_V_HEADS * HEAD_V):
        raise ValueError("gdn_verify_ring: oq must be row-major rows of the verify batch (glue.linear_rows)")
    args = GdnRingArgs(
        B, T, rows, min(conv_state.shape[0], h0.shape[0]), rslots, window.shape[0],
        ptr(mixed), ptr(z), ptr(a), ptr(b), ptr(conv_state), conv_state.stride(0), ptr(conv_w), ptr(window),
        window.stride(0), ptr(A_log), ptr(dt_bias), int(dt_bias.dtype == torch.float32), ptr(h0),
        ptr(d_ring), ptr(dlo_ring), d_ring.stride(0), dlo_ring.stride(0), ptr(k_ring), ptr(klo_ring),
        k_ring.stride(0), klo_ring.stride(0), ptr(g_ring), g_ring.stride(0), ptr(qsl), ptr(state_idx),
        ptr(replay_idx), ptr(win_idx), flags, ptr(write_pos), ptr(cache_base), ptr(norm_w), eps, scale, ptr(out),
        ptr(None if oq is None else oq.codes), ptr(None if oq is None else oq.scales))
    check(_lib.lib().q36_gdn_verify_ring(C.byref(args), _lib.stream_handle(stream)), "q36_gdn_verify_ring")
    return out
