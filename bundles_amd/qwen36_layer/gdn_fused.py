"""GDN speculative verify on libq36 (q36_gdn_verify).

Mirrors the reference's glue (R = qwen36_nodes_kb34, L = R/qwen36_layer): gdn_verify_fused
(L/gdn_fused.py:37-57 -> L/qk_gdn_verify.cu:841).  The reference keeps a replay ring; this node
returns every position's fp32 state (snapshots) and the rolled conv state out of place.
"""
from __future__ import annotations

import ctypes as C

import torch

from .. import _lib
from .._lib import GdnArgs, check, ptr

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
