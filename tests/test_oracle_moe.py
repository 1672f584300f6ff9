"""Pins of the oracle's MoE block against a float64 restatement and exact integer products (CPU).

The float64 restatement quantizes activations at the same points (the reference rules) but does
every product and sum in float64 with dequantized operands; the integer accumulators of the W8A8
path are checked exactly against numpy int64 matrix products.
"""
import numpy as np
import pytest

from helpers import assert_bf16_close
from test_oracle_quant import torch_quant_rows_i8


def _bf(O, x):
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(x, np.float32)))


def _quant_e4m3_groups(O, x, group=128):
    q, s = O.quant_groups_e4m3(np.ascontiguousarray(x, np.float32), group)
    return O.e4m3_to_f32(q).astype(np.float64) * np.repeat(s, group, axis=1).astype(np.float64)


def _weights(O, mode, E, H, I, rng):
    if mode == 0:
        w13 = rng.integers(-127, 128, (E, 2 * I, H), dtype=np.int8)
        w2 = rng.integers(-127, 128, (E, H, I), dtype=np.int8)
        s13 = (rng.random((E, 2 * I)) * 2e-4 + 1e-5).astype(np.float32)
        s2 = (rng.random((E, H)) * 2e-4 + 1e-5).astype(np.float32)
    else:
        finite = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
        w13 = rng.choice(finite, (E, 2 * I, H)).astype(np.uint8)
        w2 = rng.choice(finite, (E, H, I)).astype(np.uint8)
        s13 = (rng.random((E, 2 * I // 128, H // 128)) * 2e-5 + 1e-6).astype(np.float32)
        s2 = (rng.random((E, H // 128, I // 128)) * 2e-5 + 1e-6).astype(np.float32)
    return w13, s13, w2, s2


def _deq(O, mode, w, s):
    if mode == 0:
        return w.astype(np.float64) * s[..., :, None]
    lut = O.e4m3_lut().astype(np.float64)
    return lut[w] * np.repeat(np.repeat(s, 128, axis=-2), 128, axis=-1).astype(np.float64)


def _expert64(O, mode, xd, W13, W2, I):
    g = _bf(O, W13[:I] @ xd)
    u = _bf(O, W13[I:] @ xd)
    h = _bf(O, (g / (1.0 + np.exp(-g.astype(np.float64)))) * u).astype(np.float32)
    if mode == 0:
        hq, hs = torch_quant_rows_i8(h[None])
        hd = hq[0].astype(np.float64) * hs[0]
    else:
        hd = _quant_e4m3_groups(O, h[None])[0]
    return W2 @ hd, h


@pytest.mark.parametrize("mode", [0, 1])
def test_moe_against_float64(oracle_mod, mode):
    O = oracle_mod
    rng = np.random.default_rng(40 + mode)
    M, E, H, I, k = 4, 64, 2048, 512, 6
    x = O.f32_to_bf16(rng.standard_normal((M, H)).astype(np.float32))
    wr = O.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    gw = O.f32_to_bf16((rng.standard_normal(H) * 0.02).astype(np.float32))
    w13, s13, w2, s2 = _weights(O, mode, E, H, I, rng)
    sw13, ss13, sw2, ss2 = (a[0].copy() for a in _weights(O, mode, 1, H, I, rng))
    r = O.moe(mode, x, wr, w13, s13, w2, s2, sw13, ss13, sw2, ss2, gw, k, debug=True)
    xf = O.bf16_to_f32(x)
    if mode == 0:
        xq, xs = torch_quant_rows_i8(xf)
        xd = xq.astype(np.float64) * xs[:, None]
    else:
        xd = _quant_e4m3_groups(O, xf)
    ref = np.zeros((M, H))
    for t in range(M):
        acc = np.zeros(H)
        for j in range(k):
            e = r["ids"][t, j]
            y, _ = _expert64(O, mode, xd[t], _deq(O, mode, w13[e], s13[e]), _deq(O, mode, w2[e], s2[e]), I)
            acc += _bf(O, y * r["wts"][t, j])
        ysh, _ = _expert64(O, mode, xd[t], _deq(O, mode, sw13, ss13), _deq(O, mode, sw2, ss2), I)
        gate = 1.0 / (1.0 + np.exp(-np.dot(xf[t].astype(np.float64), O.bf16_to_f32(gw).astype(np.float64))))
        ref[t] = acc + gate * _bf(O, ysh)
    assert_bf16_close(r["out"], O.f32_to_bf16(ref.astype(np.float32)), 1e-2, f"moe mode {mode}")
    if mode == 0:
        # the int32 accumulators before scaling, exactly
        S = M * k
        for t in range(M):
            for j in list(range(k)) + [None]:
                slot = S + t if j is None else t * k + j
                wq = sw13 if j is None else w13[r["ids"][t, j]]
                a13 = wq.astype(np.int64) @ xq[t].astype(np.int64)
                assert np.array_equal(r["acc13"][slot], a13)
                hq, _ = torch_quant_rows_i8(O.bf16_to_f32(r["h"][slot])[None])
                wq2 = sw2 if j is None else w2[r["ids"][t, j]]
                assert np.array_equal(r["acc2"][slot], wq2.astype(np.int64) @ hq[0].astype(np.int64))


def test_moe_padding_rows_are_zero(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(7)
    M, E, H, I, k = 3, 64, 2048, 512, 4
    x = O.f32_to_bf16(rng.standard_normal((M, H)).astype(np.float32))
    wr = O.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    gw = O.f32_to_bf16((rng.standard_normal(H) * 0.02).astype(np.float32))
    w13, s13, w2, s2 = _weights(O, 0, E, H, I, rng)
    sw13, ss13, sw2, ss2 = (a[0].copy() for a in _weights(O, 0, 1, H, I, rng))
    pos = np.array([3, 0, 9], np.int32)
    r = O.moe(0, x, wr, w13, s13, w2, s2, sw13, ss13, sw2, ss2, gw, k, pos=pos)
    assert not r["out"][1].any() and r["out"][0].any() and r["out"][2].any()
    assert np.all(r["ids"][1] == -1)


@pytest.mark.parametrize("mode", [0, 1])
def test_moe_teacher_forcing(oracle_mod, mode):
    """The oracle's teacher-forced stages: fed its own h and y it reproduces itself bit for bit; a
    changed h row moves only its own slot's y (and its token's output); a changed y row moves only its
    token's output, by the float64 sum the combine restates."""
    O = oracle_mod
    rng = np.random.default_rng(60 + mode)
    M, E, H, I, k = 3, 64, 2048, 512, 4
    x = O.f32_to_bf16(rng.standard_normal((M, H)).astype(np.float32))
    wr = O.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    gw = O.f32_to_bf16((rng.standard_normal(H) * 0.02).astype(np.float32))
    w13, s13, w2, s2 = _weights(O, mode, E, H, I, rng)
    sw13, ss13, sw2, ss2 = (a[0].copy() for a in _weights(O, mode, 1, H, I, rng))
    args = (mode, x, wr, w13, s13, w2, s2, sw13, ss13, sw2, ss2, gw, k)
    r = O.moe(*args, debug=True)
    r_h = O.moe(*args, debug=True, h_in=r["h"])
    r_y = O.moe(*args, debug=True, y_in=r["y"])
    for key in ("out", "y"):
        assert np.array_equal(r_h[key], r[key]) and np.array_equal(r_y[key], r[key]), key
    h2 = r["h"].copy()
    slot = 1 * k + 2  # token 1, pick 2
    h2[slot] = O.f32_to_bf16(O.bf16_to_f32(h2[slot]) * np.float32(1.5))
    r2 = O.moe(*args, debug=True, h_in=h2)
    changed = np.any(r2["y"] != r["y"], axis=1)
    assert changed[slot] and changed.sum() == 1
    assert np.array_equal(r2["out"][[0, 2]], r["out"][[0, 2]]) and np.any(r2["out"][1] != r["out"][1])
    y2 = r["y"].copy()
    y2[0 * k + 1] = O.f32_to_bf16(O.bf16_to_f32(y2[0 * k + 1]) + np.float32(0.25))
    r3 = O.moe(*args, debug=True, y_in=y2)
    assert np.array_equal(r3["out"][1:], r["out"][1:])
    yf = O.bf16_to_f32(y2).astype(np.float64)
    gate = 1.0 / (1.0 + np.exp(-np.dot(O.bf16_to_f32(x[0]).astype(np.float64), O.bf16_to_f32(gw).astype(np.float64))))
    ref0 = yf[0:k].sum(0) + gate * yf[M * k + 0]
    assert_bf16_close(r3["out"][:1], O.f32_to_bf16(ref0[None].astype(np.float32)), 1e-2, "combine of y_in")
