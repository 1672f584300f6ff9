"""ctypes front end of oracle/liboracle.so (the C restatement in q36_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against and the CPU
baseline bench.py times.  Arrays are numpy; bf16 travels as uint16 bit patterns and e4m3fn
as uint8 codes.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
I32 = C.c_int


class MoeArgs(C.Structure):
    _fields_ = [("mode", I32), ("M", I32), ("E", I32), ("H", I32), ("I", I32), ("k", I32),
                ("x", P), ("wr", P), ("bias", P), ("pos", P), ("w13", P), ("s13", P), ("w2", P),
                ("s2", P), ("sw13", P), ("ss13", P), ("sw2", P), ("ss2", P), ("gate_w", P), ("out", P),
                ("ids", P), ("wts", P), ("acc13", P), ("acc2", P), ("h", P), ("n_threads", I32),
                ("h_in", P), ("y_in", P), ("y", P)]


class GdnArgs(C.Structure):
    _fields_ = [("B", I32), ("T", I32), ("mixed", P), ("z", P), ("a", P), ("b", P), ("conv_state", P),
                ("conv_w", P), ("A_log", P), ("dt_bias", P), ("S0", P), ("norm_w", P), ("eps", C.c_float),
                ("out", P), ("snaps", P), ("use_f64", I32), ("n_threads", I32)]


class GdnRingArgs(C.Structure):
    _fields_ = [("B", I32), ("T", I32), ("mixed", P), ("z", P), ("a", P), ("b", P), ("conv_state", P),
                ("conv_w", P), ("window", P), ("A_log", P), ("dt_bias", P), ("h0", P), ("d_ring", P),
                ("dlo_ring", P), ("k_ring", P), ("klo_ring", P), ("g_ring", P), ("qsl", P), ("state_idx", P),
                ("replay_idx", P), ("win_idx", P), ("write_pos", P), ("cache_base", P), ("norm_w", P),
                ("eps", C.c_float), ("scale", C.c_float), ("out", P), ("use_f64", I32), ("n_threads", I32)]


class AttnArgs(C.Structure):
    _fields_ = [("T", I32), ("x", P), ("wqg", P), ("sqg", P), ("wk", P), ("sk", P), ("wv", P), ("sv", P),
                ("q_norm_w", P), ("k_norm_w", P), ("eps", C.c_float), ("cos_sin", P), ("positions", P),
                ("q", P), ("gate", P), ("k", P), ("v", P), ("k8", P), ("v8", P), ("n_threads", I32)]


class OprojArgs(C.Structure):
    _fields_ = [("T", I32), ("attn", P), ("gate", P), ("wo", P), ("so", P), ("out", P), ("n_threads", I32)]


class DecodeArgs(C.Structure):
    _fields_ = [("B", I32), ("NT", I32), ("HQ", I32), ("HKV", I32), ("D", I32), ("q", P), ("kcache", P),
                ("vcache", P), ("page_table", P), ("pt_stride", I32), ("seqlens", P), ("scale", C.c_float),
                ("out", P), ("n_threads", I32)]


class LmheadArgs(C.Structure):
    _fields_ = [("R", I32), ("H", I32), ("V", I32), ("h", P), ("norm_w", P), ("eps", C.c_float), ("wq", P),
                ("ws", P), ("ids", P), ("logits", P), ("n_threads", I32), ("mode", I32)]


def _declare(L):
    L.q36o_f32_to_bf16.restype = C.c_uint16
    L.q36o_f32_to_bf16.argtypes = [C.c_float]
    L.q36o_bf16_to_f32.restype = C.c_float
    L.q36o_bf16_to_f32.argtypes = [C.c_uint16]
    L.q36o_f32_to_e4m3.restype = C.c_uint8
    L.q36o_f32_to_e4m3.argtypes = [C.c_float]
    L.q36o_e4m3_to_f32.restype = C.c_float
    L.q36o_e4m3_to_f32.argtypes = [C.c_uint8]
    L.q36o_expf.restype = C.c_float
    L.q36o_expf.argtypes = [C.c_float]
    L.q36o_f32_to_f16.restype = C.c_uint16
    L.q36o_f32_to_f16.argtypes = [C.c_float]
    L.q36o_f16_to_f32.restype = C.c_float
    L.q36o_f16_to_f32.argtypes = [C.c_uint16]
    L.q36o_q8_block_bytes.restype = C.c_size_t
    L.q36o_q8_block_bytes.argtypes = [I32, I32]
    L.q36o_quant_q8_block_v1.argtypes = [P, P, I32, I32, I32, I32, P]
    L.q36o_quant_dense8.argtypes = [P, I32, I32, P, P, I32]
    L.q36o_f16_round.restype = C.c_float
    L.q36o_f16_round.argtypes = [C.c_float]
    L.q36o_dot_canon.restype = C.c_float
    L.q36o_dot_canon.argtypes = [P, P, I32]
    L.q36o_quant_rows_i8.argtypes = [P, I32, I32, P, P]
    L.q36o_quant_groups_e4m3.argtypes = [P, I32, I32, I32, P, P]
    L.q36o_quant_blocks_e4m3.argtypes = [P, I32, I32, P, P]
    L.q36o_fp8_linear.restype = I32
    L.q36o_fp8_linear.argtypes = [I32, I32, I32, P, P, P, P, I32]
    L.q36o_dense8_linear.restype = I32
    L.q36o_dense8_linear.argtypes = [I32, I32, I32, P, P, P, C.c_int64, P, I32]
    L.q36o_add_rmsnorm.restype = I32
    L.q36o_add_rmsnorm.argtypes = [I32, I32, P, P, P, C.c_float, P]
    L.q36o_route.restype = I32
    L.q36o_route.argtypes = [P, P, P, P, I32, I32, I32, I32, P, P, P, P, P, P, P, P, P]
    for fn, st in (("q36o_moe", MoeArgs), ("q36o_gdn_verify", GdnArgs), ("q36o_gdn_verify_ring", GdnRingArgs),
                   ("q36o_attn_proj", AttnArgs),
                   ("q36o_attn_oproj", OprojArgs), ("q36o_lmhead", LmheadArgs), ("q36o_attn_decode", DecodeArgs)):
        f = getattr(L, fn)
        f.restype = I32
        f.argtypes = [C.POINTER(st)]


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---------------------------------------------------------------- scalar / codec helpers
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16), vectorised like the C codec."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_lut() -> np.ndarray:
    L = lib()
    return np.array([L.q36o_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """Element-wise q36o_f32_to_e4m3 (RNE, satfinite); for small arrays."""
    enc = lib().q36o_f32_to_e4m3
    x = np.asarray(x, np.float32)
    return np.fromiter((enc(float(v)) for v in x.reshape(-1)), np.uint8, x.size).reshape(x.shape)


def e4m3_to_f32(b: np.ndarray) -> np.ndarray:
    return e4m3_lut()[np.asarray(b, dtype=np.uint8)]


def expf(x: float) -> float:
    return lib().q36o_expf(float(x))


def dot_canon(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().q36o_dot_canon(_p(a), _p(b), a.size)


# ---------------------------------------------------------------- quantizers
def quant_rows_i8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, K = x.shape
    q = np.empty((rows, K), np.int8)
    s = np.empty(rows, np.float32)
    lib().q36o_quant_rows_i8(_p(x), rows, K, _p(q), _p(s))
    return q, s


def quant_groups_e4m3(x: np.ndarray, group: int = 128):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, K = x.shape
    q = np.empty((rows, K), np.uint8)
    s = np.empty((rows, K // group), np.float32)
    lib().q36o_quant_groups_e4m3(_p(x), rows, K, group, _p(q), _p(s))
    return q, s


def quant_blocks_e4m3(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty((N // 128, K // 128), np.float32)
    lib().q36o_quant_blocks_e4m3(_p(w), N, K, _p(q), _p(s))
    return q, s


# ---------------------------------------------------------------- routing
def route(x_bf16, wr_bf16, k, bias=None, pos=None):
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    wr_bf16 = np.ascontiguousarray(wr_bf16, np.uint16)
    M, H = x_bf16.shape
    E = wr_bf16.shape[0]
    out = dict(logits=np.empty((M, E), np.float32), ids=np.empty((M, k), np.int32),
               wts=np.empty((M, k), np.float32), counts=np.empty(E, np.int32),
               offsets=np.empty(E + 1, np.int32), perm=np.empty(M * k, np.int32),
               inv_perm=np.empty(M * k, np.int32), active=np.zeros(E, np.int32))
    nact = C.c_int32(0)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ps = None if pos is None else np.ascontiguousarray(pos, np.int32)
    rc = lib().q36o_route(_p(x_bf16), _p(wr_bf16), _p(b), _p(ps), M, E, H, k, _p(out["logits"]), _p(out["ids"]),
                          _p(out["wts"]), _p(out["counts"]), _p(out["offsets"]), _p(out["perm"]),
                          _p(out["inv_perm"]), _p(out["active"]), C.addressof(nact))
    if rc:
        raise ValueError("q36o_route rejected the shapes")
    out["n_active"] = nact.value
    return out


# ---------------------------------------------------------------- MoE
def moe(mode, x, wr, w13, s13, w2, s2, sw13, ss13, sw2, ss2, gate_w, k, bias=None, pos=None, debug=False,
        n_threads=0, h_in=None, y_in=None):
    """mode 0: int8 W8A8, mode 1: fp8 e4m3 block-scaled.  Returns dict(out, ids, wts[, acc13, acc2, h, y]).
    h_in / y_in (bf16 bits [M*k+M, I] / [M*k+M, H]) feed the down stage / the combine with another
    implementation's intermediate rows (teacher forcing)."""
    x = np.ascontiguousarray(x, np.uint16)
    M, H = x.shape
    E = wr.shape[0]
    I = w13.shape[1] // 2
    S = M * k
    res = dict(out=np.empty((M, H), np.uint16), ids=np.empty((M, k), np.int32), wts=np.empty((M, k), np.float32))
    if debug:
        res["h"] = np.zeros((S + M, I), np.uint16)
        res["y"] = np.zeros((S + M, H), np.uint16)
        if mode == 0:
            res["acc13"] = np.zeros((S + M, 2 * I), np.int32)
            res["acc2"] = np.zeros((S + M, H), np.int32)
    keep = [np.ascontiguousarray(v) for v in (wr, w13, s13, w2, s2, sw13, ss13, sw2, ss2, gate_w)]
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ps = None if pos is None else np.ascontiguousarray(pos, np.int32)
    hin = None if h_in is None else np.ascontiguousarray(h_in, np.uint16).reshape(S + M, I)
    yin = None if y_in is None else np.ascontiguousarray(y_in, np.uint16).reshape(S + M, H)
    a = MoeArgs(mode, M, E, H, I, k, _p(x), *(_p(v) for v in keep[:1]), _p(b), _p(ps),
                *(_p(v) for v in keep[1:]), _p(res["out"]), _p(res["ids"]), _p(res["wts"]),
                _p(res.get("acc13")), _p(res.get("acc2")), _p(res.get("h")), n_threads, _p(hin), _p(yin),
                _p(res.get("y")))
    rc = lib().q36o_moe(C.byref(a))
    if rc:
        raise ValueError("q36o_moe rejected the shapes")
    return res


# ---------------------------------------------------------------- reference weight formats
def f32_to_f16_bits(x) -> np.ndarray:
    """float32 -> IEEE binary16 bit patterns (uint16) through the oracle's codec."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    f = lib().q36o_f32_to_f16
    return np.array([f(float(v)) for v in x], dtype=np.uint16)


def q8_block_bytes(H: int, I: int) -> int:  # noqa: E741
    return int(lib().q36o_q8_block_bytes(H, I))


def quant_q8_block_v1(w13, w2, channel=True):
    """q8-block-v1 expert blocks uint8 [E, block_bytes] from float32 w13 [E, 2I, H], w2 [E, H, I]."""
    w13 = np.ascontiguousarray(w13, np.float32)
    w2 = np.ascontiguousarray(w2, np.float32)
    E, I2, H = w13.shape
    out = np.zeros((E, q8_block_bytes(H, I2 // 2)), np.uint8)
    lib().q36o_quant_q8_block_v1(_p(w13), _p(w2), E, H, I2 // 2, int(channel), _p(out))
    return out


def q8_block_parts(block, H: int, I: int):  # noqa: E741
    """(q13 int8 [2I, H], q2 int8 [H, I], c13 fp16 bits [2I, H/128], c2 fp16 bits [H, I/128]) of one block."""
    o2, oc13 = 2 * I * H, 3 * I * H
    oc2 = oc13 + 2 * I * (H // 128) * 2
    eb = q8_block_bytes(H, I)
    return (block[:o2].view(np.int8).reshape(2 * I, H), block[o2:oc13].view(np.int8).reshape(H, I),
            block[oc13:oc2].view(np.uint16).reshape(2 * I, H // 128), block[oc2:eb].view(np.uint16).reshape(H, I // 128))


def quant_dense8(w, s_stride=None):
    """DENSE8 copy of float32 w [N, K]: (q int8 [N, K], s fp16 bits [K/128, s_stride])."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    s_stride = N if s_stride is None else s_stride
    q = np.zeros((N, K), np.int8)
    s = np.zeros((K // 128, s_stride), np.uint16)
    lib().q36o_quant_dense8(_p(w), N, K, _p(q), _p(s), s_stride)
    return q, s


# ---------------------------------------------------------------- GDN
def gdn_verify(B, T, mixed, z, a, b, conv_state, conv_w, A_log, dt_bias, S0, norm_w, eps=1e-6, use_f64=False,
               n_threads=0):
    """Returns (out bf16 [B*T,4096], snaps fp32 [B,T,32,128,128], rolled conv_state copy)."""
    cs = np.array(conv_state, dtype=np.uint16, copy=True, order="C")
    out = np.empty((B * T, 4096), np.uint16)
    snaps = np.empty((B, T, 32, 128, 128), np.float32)
    keep = [np.ascontiguousarray(v) for v in (mixed, z, a, b)]
    cw = np.ascontiguousarray(conv_w, np.uint16)
    al = np.ascontiguousarray(A_log, np.float32)
    dt = np.ascontiguousarray(dt_bias, np.float32)
    s0 = np.ascontiguousarray(S0, np.float32)
    nw = np.ascontiguousarray(norm_w, np.uint16)
    args = GdnArgs(B, T, *(_p(v) for v in keep), _p(cs), _p(cw), _p(al), _p(dt), _p(s0), _p(nw), eps, _p(out),
                   _p(snaps), int(use_f64), n_threads)
    rc = lib().q36o_gdn_verify(C.byref(args))
    if rc:
        raise ValueError("q36o_gdn_verify rejected the shapes")
    return out, snaps, cs


def gdn_verify_ring(B, T, mixed, z, a, b, conv_state, conv_w, window, A_log, dt_bias, h0, d_ring, dlo_ring,
                    k_ring, klo_ring, g_ring, qsl, state_idx, replay_idx, win_idx, write_pos, cache_base, norm_w,
                    eps=1e-6, scale=128 ** -0.5, use_f64=False, n_threads=0):
    """The ring verify (q36o_gdn_verify_ring) on copies of the mutable pools.

    Returns a dict: out bf16 [rows, 4096] and the updated conv_state, window, d/dlo/k/klo/g rings."""
    res = {k: np.array(v, copy=True, order="C") for k, v in (
        ("conv_state", conv_state), ("window", window), ("d_ring", d_ring), ("dlo_ring", dlo_ring),
        ("k_ring", k_ring), ("klo_ring", klo_ring), ("g_ring", g_ring))}
    rows = np.ascontiguousarray(mixed).shape[0]
    res["out"] = np.empty((rows, 4096), np.uint16)
    keep = {k: np.ascontiguousarray(v) for k, v in (("mixed", mixed), ("z", z), ("a", a), ("b", b))}
    cw = np.ascontiguousarray(conv_w, np.uint16)
    al = np.ascontiguousarray(A_log, np.float32)
    dt = np.ascontiguousarray(dt_bias, np.float32)
    hh = np.ascontiguousarray(h0, np.float32)
    nw = np.ascontiguousarray(norm_w, np.uint16)
    q = np.ascontiguousarray(qsl, np.int32)
    si, ri, wi = (np.ascontiguousarray(v, np.int64) for v in (state_idx, replay_idx, win_idx))
    wpos = np.ascontiguousarray(write_pos, np.int32)
    cbase = np.ascontiguousarray(cache_base, np.int32)
    args = GdnRingArgs(B, T, _p(keep["mixed"]), _p(keep["z"]), _p(keep["a"]), _p(keep["b"]), _p(res["conv_state"]),
                       _p(cw), _p(res["window"]), _p(al), _p(dt), _p(hh), _p(res["d_ring"]), _p(res["dlo_ring"]),
                       _p(res["k_ring"]), _p(res["klo_ring"]), _p(res["g_ring"]), _p(q), _p(si), _p(ri), _p(wi),
                       _p(wpos), _p(cbase), _p(nw), eps, scale, _p(res["out"]), int(use_f64), n_threads)
    rc = lib().q36o_gdn_verify_ring(C.byref(args))
    if rc:
        raise ValueError("q36o_gdn_verify_ring rejected the shapes")
    return res


# ---------------------------------------------------------------- attention projections
def attn_proj(x, wqg, sqg, wk, sk, wv, sv, q_norm_w, k_norm_w, eps, cos_sin, positions, n_threads=0):
    x = np.ascontiguousarray(x, np.uint16)
    T = x.shape[0]
    res = dict(q=np.empty((T, 16, 256), np.uint16), gate=np.empty((T, 16, 256), np.uint16),
               k=np.empty((T, 2, 256), np.uint16), v=np.empty((T, 2, 256), np.uint16),
               k8=np.empty((T, 2, 256), np.uint8), v8=np.empty((T, 2, 256), np.uint8))
    keep = [np.ascontiguousarray(v) for v in (wqg, sqg, wk, sk, wv, sv, q_norm_w, k_norm_w)]
    cs = np.ascontiguousarray(cos_sin, np.float32)
    ps = np.ascontiguousarray(positions, np.int32)
    a = AttnArgs(T, _p(x), *(_p(v) for v in keep), eps, _p(cs), _p(ps), _p(res["q"]), _p(res["gate"]),
                 _p(res["k"]), _p(res["v"]), _p(res["k8"]), _p(res["v8"]), n_threads)
    if lib().q36o_attn_proj(C.byref(a)):
        raise ValueError("q36o_attn_proj failed")
    return res


def attn_oproj(attn, gate, wo, so, n_threads=0):
    attn = np.ascontiguousarray(attn, np.uint16).reshape(-1, 4096)
    gate = np.ascontiguousarray(gate, np.uint16).reshape(-1, 4096)
    T = attn.shape[0]
    out = np.empty((T, 2048), np.uint16)
    wo = np.ascontiguousarray(wo)
    so = np.ascontiguousarray(so, np.float32)
    a = OprojArgs(T, _p(attn), _p(gate), _p(wo), _p(so), _p(out), n_threads)
    if lib().q36o_attn_oproj(C.byref(a)):
        raise ValueError("q36o_attn_oproj failed")
    return out


# ---------------------------------------------------------------- lm_head
def dense8_linear(x, q, s, n_threads=0):
    """x bf16 bits [T, K]; q int8 [N, K]; s fp16 bits (uint16) or float16 [K/128, >= N], group-major
    (the layout quant_dense8 writes) -> bf16 bits [T, N]."""
    x = np.ascontiguousarray(x, np.uint16)
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s).view(np.uint16) if s.dtype == np.float16 else np.ascontiguousarray(s, np.uint16)
    T, K = x.shape
    N = q.shape[0]
    out = np.empty((T, N), np.uint16)
    if lib().q36o_dense8_linear(T, N, K, _p(x), _p(q), _p(s), C.c_int64(s.shape[1]), _p(out), n_threads):
        raise ValueError("q36o_dense8_linear failed")
    return out


def lmhead(h, norm_w, eps, wq, ws, want_logits=False, n_threads=0, two_term=False, w8a16=False):
    h = np.ascontiguousarray(h, np.uint16)
    R, H = h.shape
    V = wq.shape[0]
    ids = np.empty(R, np.int32)
    logits = np.empty((R, V), np.uint16) if want_logits else None
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, np.uint16)
    wq = np.ascontiguousarray(wq, np.int8)
    ws = np.ascontiguousarray(ws, np.float32)
    a = LmheadArgs(R, H, V, _p(h), _p(nw), eps, _p(wq), _p(ws), _p(ids), _p(logits), n_threads,
                   2 if w8a16 else int(two_term))
    if lib().q36o_lmhead(C.byref(a)):
        raise ValueError("q36o_lmhead failed")
    return ids, logits


# ---------------------------------------------------------------- hybrid-layer glue
def fp8_linear(x, wq, ws, n_threads=0):
    """x bf16 bits [T, K]; wq e4m3 codes [N, K] row-major; ws fp32 [N/128, K/128] -> bf16 bits [T, N]."""
    x = np.ascontiguousarray(x, np.uint16)
    wq = np.ascontiguousarray(wq, np.uint8)
    ws = np.ascontiguousarray(ws, np.float32)
    T, K = x.shape
    N = wq.shape[0]
    out = np.empty((T, N), np.uint16)
    if lib().q36o_fp8_linear(T, N, K, _p(x), _p(wq), _p(ws), _p(out), n_threads):
        raise ValueError("q36o_fp8_linear failed")
    return out


def add_rmsnorm(delta, residual, w, eps):
    """delta (or None), residual bf16 bits [T, H], w bf16 bits [H] -> (out, new residual) bf16 bits."""
    residual = np.array(residual, np.uint16, copy=True, order="C")
    d = None if delta is None else np.ascontiguousarray(delta, np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    T, H = residual.shape
    out = np.empty_like(residual)
    if lib().q36o_add_rmsnorm(T, H, _p(d), _p(residual), _p(w), eps, _p(out)):
        raise ValueError("q36o_add_rmsnorm failed")
    return out, residual


# ---------------------------------------------------------------- decode attention
def attn_decode(q, kcache, vcache, page_table, seqlens, NT, scale, n_threads=0):
    """q bf16 bits [B*NT, HQ, D]; caches e4m3 codes [slots, HKV, D]; page_table int32 [B, L];
    seqlens int32 [B] -> bf16 bits [B*NT, HQ, D]."""
    q = np.ascontiguousarray(q, np.uint16)
    kcache = np.ascontiguousarray(kcache, np.uint8)
    vcache = np.ascontiguousarray(vcache, np.uint8)
    page_table = np.ascontiguousarray(page_table, np.int32)
    seqlens = np.ascontiguousarray(seqlens, np.int32)
    T, HQ, D = q.shape
    B = seqlens.shape[0]
    HKV = kcache.shape[1]
    out = np.empty_like(q)
    a = DecodeArgs(B, NT, HQ, HKV, D, _p(q), _p(kcache), _p(vcache), _p(page_table), page_table.shape[1],
                   _p(seqlens), scale, _p(out), n_threads)
    if lib().q36o_attn_decode(C.byref(a)):
        raise ValueError("q36o_attn_decode failed")
    return out


def f16_round(x):
    L = lib()
    return np.array([L.q36o_f16_round(float(v)) for v in np.ravel(x)], np.float32).reshape(np.shape(x))
