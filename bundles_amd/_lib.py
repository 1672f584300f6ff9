"""ctypes binding of libq36.so, the extern "C" boundary declared in include/q36_abi.h.

The structures below mirror the header field for field; tests check their sizes against the
library's own sizeof.  Every call raises RuntimeError with q36_last_error() on a non-zero
return code.  There is no fallback: a missing library is an ImportError-like failure.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq36.so")

Q36_OK, Q36_EINVAL, Q36_ELAUNCH = 0, 1, 2
Q36_MOE_INT8, Q36_MOE_FP8 = 0, 1
Q36_LMH_W8A8, Q36_LMH_W8A8X2, Q36_LMH_W8A16 = 0, 1, 2

P = C.c_void_p
I32 = C.c_int32
SZ = C.c_size_t


class MoeArgs(C.Structure):
    _fields_ = [("M", I32), ("E", I32), ("H", I32), ("I", I32), ("topk", I32), ("dtype", I32),
                ("x", P), ("router_w", P), ("router_bias", P), ("positions", P),
                ("w13", P), ("s13", P), ("w2", P), ("s2", P), ("sw13", P), ("ss13", P), ("sw2", P), ("ss2", P),
                ("gate_w", P), ("out", P), ("workspace", P), ("workspace_bytes", SZ),
                ("dbg_acc13", P), ("dbg_acc2", P), ("dbg_h", P),
                ("resid", P), ("norm_w", P), ("norm_eps", C.c_float), ("norm_out", P),
                ("norm_q8", P), ("norm_q8s", P), ("norm_q8_frag", I32),
                ("in_delta", P), ("in_resid", P), ("in_resid_out", P), ("in_norm_w", P), ("in_norm_eps", C.c_float)]


class MoeWsLayout(C.Structure):
    _fields_ = [(n, SZ) for n in ("logits", "gate", "ids", "wts", "counts", "offsets", "perm", "inv_perm", "active", "ctl",
                                  "xq", "xs", "h", "y", "ecount", "eact", "elist", "total")]


class GdnArgs(C.Structure):
    _fields_ = [("B", I32), ("T", I32), ("mixed", P), ("z", P), ("a", P), ("b", P), ("conv_state", P),
                ("conv_state_out", P), ("conv_w", P), ("A_log", P), ("dt_bias", P), ("S0", P), ("norm_w", P),
                ("eps", C.c_float), ("out", P), ("snaps", P)]


I64 = C.c_int64


class GdnRingArgs(C.Structure):
    _fields_ = [("B", I32), ("T", I32), ("rows", I32), ("slots", I32), ("rslots", I32), ("wslots", I32),
                ("mixed", P), ("z", P), ("a", P), ("b", P), ("conv_state", P), ("cs_slot", I64), ("conv_w", P),
                ("window", P), ("win_slot", I64), ("A_log", P), ("dt_bias", P), ("dt_f32", I32), ("h0", P),
                ("d_ring", P), ("dlo_ring", P), ("d_slot", I64), ("dlo_slot", I64), ("k_ring", P), ("klo_ring", P),
                ("k_slot", I64), ("klo_slot", I64), ("g_ring", P), ("g_slot", I64), ("qsl", P), ("state_idx", P),
                ("replay_idx", P), ("win_idx", P), ("idx_i64", I32), ("write_pos", P), ("cache_base", P),
                ("norm_w", P), ("eps", C.c_float), ("scale", C.c_float), ("out", P), ("oq", P), ("oqs", P)]


class AttnArgs(C.Structure):
    _fields_ = [("T", I32), ("max_pos", I32), ("x", P), ("wqkv", P), ("sqkv", P), ("q_norm_w", P),
                ("k_norm_w", P), ("eps", C.c_float), ("cos_sin", P), ("positions", P), ("q", P), ("gate", P),
                ("k", P), ("v", P), ("k8", P), ("v8", P), ("workspace", P), ("workspace_bytes", SZ),
                ("xq", P), ("xqs", P), ("out_loc", P), ("k_cache", P), ("v_cache", P), ("num_slots", C.c_int64)]


class OprojArgs(C.Structure):
    _fields_ = [("T", I32), ("attn", P), ("gate", P), ("wo", P), ("so", P), ("out", P), ("workspace", P),
                ("workspace_bytes", SZ), ("aq", P), ("aqs", P)]


class LmheadArgs(C.Structure):
    _fields_ = [("R", I32), ("H", I32), ("V", I32), ("h", P), ("norm_w", P), ("eps", C.c_float), ("wq", P),
                ("ws", P), ("ids", P), ("logits", P), ("workspace", P), ("workspace_bytes", SZ), ("mode", I32),
                ("logits_f32", I32), ("wq_t", P)]


class LinearSeg(C.Structure):
    _fields_ = [("col0", I32), ("ld", I32), ("out", P)]


class Fp8LinearArgs(C.Structure):
    _fields_ = [("T", I32), ("N", I32), ("K", I32), ("n_out", I32), ("x", P), ("w", P), ("ws", P), ("nseg", I32),
                ("seg", LinearSeg * 4), ("workspace", P), ("workspace_bytes", SZ), ("xq", P), ("xqs", P)]


class Dense8LinearArgs(C.Structure):
    _fields_ = [("T", I32), ("N", I32), ("K", I32), ("n_out", I32), ("x", P), ("q", P), ("s", P),
                ("s_ld", C.c_int64), ("nseg", I32), ("seg", LinearSeg * 4), ("tiled", I32)]


class AddNormArgs(C.Structure):
    _fields_ = [("T", I32), ("H", I32), ("delta", P), ("residual", P), ("norm_w", P), ("eps", C.c_float), ("out", P),
                ("q8", P), ("q8s", P), ("q8_frag", I32)]


class DecodeArgs(C.Structure):
    _fields_ = [("B", I32), ("NT", I32), ("HQ", I32), ("HKV", I32), ("D", I32), ("splits", I32), ("q", P),
                ("k_cache", P), ("v_cache", P), ("num_slots", C.c_int64), ("page_table", P), ("pt_stride", I32),
                ("seqlens", P), ("out_loc", P), ("k_new", P), ("v_new", P), ("scale", C.c_float), ("out", P),
                ("workspace", P), ("workspace_bytes", SZ), ("gate", P), ("oq", P), ("oqs", P)]


_lib = None

# (name, restype, argtypes) of every exported symbol; tests check that each one resolves.
SYMBOLS = [
    ("q36_abi_version", I32, []),
    ("q36_last_error", C.c_char_p, []),
    ("q36_moe_workspace_bytes", SZ, [I32, I32, I32, I32, I32, I32]),
    ("q36_moe_workspace_layout", I32, [I32, I32, I32, I32, I32, I32, C.POINTER(MoeWsLayout)]),
    ("q36_moe_route", I32, [C.POINTER(MoeArgs), P]),
    ("q36_moe_up", I32, [C.POINTER(MoeArgs), P]),
    ("q36_moe_down", I32, [C.POINTER(MoeArgs), P]),
    ("q36_moe_combine", I32, [C.POINTER(MoeArgs), P]),
    ("q36_moe_forward", I32, [C.POINTER(MoeArgs), P]),
    ("q36_moe_forward_static", I32, [C.POINTER(MoeArgs), P]),
    ("q36_gdn_verify", I32, [C.POINTER(GdnArgs), P]),
    ("q36_gdn_verify_ring", I32, [C.POINTER(GdnRingArgs), P]),
    ("q36_attn_act_frag", I32, [I32]),
    ("q36_attn_workspace_bytes", SZ, [I32]),
    ("q36_oproj_workspace_bytes", SZ, [I32]),
    ("q36_attn_proj", I32, [C.POINTER(AttnArgs), P]),
    ("q36_attn_oproj", I32, [C.POINTER(OprojArgs), P]),
    ("q36_fp8_linear_act_frag", I32, [I32, I32]),
    ("q36_fp8_linear_workspace_bytes", SZ, [I32, I32]),
    ("q36_fp8_linear", I32, [C.POINTER(Fp8LinearArgs), P]),
    ("q36_add_rmsnorm", I32, [C.POINTER(AddNormArgs), P]),
    ("q36_dense8_linear", I32, [C.POINTER(Dense8LinearArgs), P]),
    ("q36_tile_w16", I32, [P, C.c_int64, I32, P, P]),
    ("q36_attn_decode_workspace_bytes", SZ, [I32, I32]),
    ("q36_attn_decode", I32, [C.POINTER(DecodeArgs), P]),
    ("q36_lmhead_workspace_bytes", SZ, [I32]),
    ("q36_lmhead_argmax", I32, [C.POINTER(LmheadArgs), P]),
    ("q36_quant_rows_i8", I32, [P, C.c_int64, I32, P, P, P]),
    ("q36_q8_block_v1_bytes", SZ, [I32, I32]),
    ("q36_quant_q8_block_v1", I32, [P, P, I32, I32, I32, I32, P, P]),
    ("q36_import_q8_block_v1", I32, [P, I32, I32, I32, P, P, P, P, P]),
    ("q36_quant_dense8", I32, [P, C.c_int64, I32, P, P, C.c_int64, P]),
    ("q36_quant_blocks_e4m3", I32, [P, C.c_int64, I32, P, P, P]),
    ("q36_pack_frag8", I32, [P, C.c_int64, I32, P, P]),
]
OPTIONAL_SYMBOLS: list = []


def lib():
    """Load libq36.so (built by bundles_amd.build); raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libq36.so is not built ({LIB_PATH}); run bundles_amd.build.build() first")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SYMBOLS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != Q36_OK:
        msg = lib().q36_last_error().decode(errors="replace")
        kind = "invalid argument" if rc == Q36_EINVAL else "launch failure"
        raise RuntimeError(f"{what}: {kind}: {msg}")


def ptr(t) -> int | None:
    """Device (or host) address of a torch tensor, None for None."""
    return None if t is None else t.data_ptr()


def stream_handle(stream=None) -> int | None:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream
