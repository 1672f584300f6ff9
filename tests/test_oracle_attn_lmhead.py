"""Pins of the oracle's attention projections and int8 lm_head (CPU).

lm_head: the int32 accumulators by exact numpy integer products, the logits by the closed form
bf16((acc * xs) * ws) in float32, the ids by the first index of the row maximum (numpy's argmax
order), the activation quantizer by the torch restatement of H/lmhead8.py:129-143; the final norm
against a float64 RMSNorm within tolerance.
Attention: the projections against a float64 product of the dequantized e4m3 operands, the head norm
and RoPE against a float64 restatement (rotation by position * theta^(-2i/64) of the pairs
(i, i + 32)); RoPE invariants: dims 64..255 do not depend on the position, each pair's length is
kept, and the pair turns by +position * inv_freq (a sign or pairing mistake fails this).  The cache
codes are the e4m3 encodings of the bf16 k and v.
"""
import numpy as np
import pytest

from helpers import assert_bf16_close
from test_oracle_quant import torch_quant_rows_i8


def _bf(O, x):
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(x, np.float32)))


def _lmhead_inputs(O, R, V, seed):
    rng = np.random.default_rng(seed)
    h = O.f32_to_bf16(rng.standard_normal((R, 2048)).astype(np.float32))
    wq = rng.integers(-127, 128, (V, 2048), dtype=np.int8)
    ws = (rng.random(V) * 2e-4 + 1e-5).astype(np.float32)
    return h, wq, ws


def test_lmhead_exact_without_norm(oracle_mod):
    O = oracle_mod
    R, V = 6, 1536
    h, wq, ws = _lmhead_inputs(O, R, V, 1)
    ids, logits = O.lmhead(h, None, 1e-6, wq, ws, want_logits=True)
    xq, xs = torch_quant_rows_i8(O.bf16_to_f32(h))
    acc = xq.astype(np.int64) @ wq.astype(np.int64).T
    assert np.abs(acc).max() < 2 ** 31
    ref = O.f32_to_bf16((acc.astype(np.float32) * xs[:, None].astype(np.float32)) * ws[None, :])
    assert np.array_equal(logits, ref)
    assert np.array_equal(ids, np.argmax(O.bf16_to_f32(ref), axis=1))


def torch_quant_two_term(y):
    """The reference's two-term activation rule (H/w8a8.py:25-37) restated: the int8 rule on y, then on
    the residual y - q1 s1 formed in float64 (q1 s1 and the difference are exact there) and rounded once
    to float32, which is what one fused multiply-add gives."""
    q1, s1 = torch_quant_rows_i8(y)
    res = (y.astype(np.float64) - q1.astype(np.float64) * s1[:, None].astype(np.float64)).astype(np.float32)
    q2, s2 = torch_quant_rows_i8(res)
    return q1, s1, q2, s2, res


def test_lmhead_two_term_exact(oracle_mod):
    """Two terms: the int32 accumulators of both terms exactly (numpy int64), the epilogue
    fma(acc1, s1, acc2 * s2) * ws (float64 fma then one float32 rounding, the multiply by ws rounded
    again), the bf16 logits and ids bit for bit; the two terms reconstruct y to within s2 / 2."""
    O = oracle_mod
    R, V = 5, 1280
    h, wq, ws = _lmhead_inputs(O, R, V, 4)
    ids, logits = O.lmhead(h, None, 1e-6, wq, ws, want_logits=True, two_term=True)
    y = O.bf16_to_f32(h)
    q1, s1, q2, s2, res = torch_quant_two_term(y)
    recon = q1.astype(np.float64) * s1[:, None] + q2.astype(np.float64) * s2[:, None]
    assert np.all(np.abs(recon - y) <= s2[:, None] * 0.5 * (1 + 1e-5) + 1e-12)  # ties land on s2 / 2
    assert np.all(s2 <= s1 * 0.5 * (1 + 1e-6))  # the residual is at most half a step of term 1
    a1 = q1.astype(np.int64) @ wq.astype(np.int64).T
    a2 = q2.astype(np.int64) @ wq.astype(np.int64).T
    inner = (a2.astype(np.float32) * s2[:, None]).astype(np.float64)
    f = (a1.astype(np.float64) * s1[:, None].astype(np.float64) + inner).astype(np.float32)  # one rounding
    ref = O.f32_to_bf16(f * ws[None, :])
    assert np.array_equal(logits, ref)
    assert np.array_equal(ids, np.argmax(O.bf16_to_f32(ref), axis=1))
    # the second term brings the logits closer to the unquantized activations' than one term does
    exact = y.astype(np.float64) @ (wq.astype(np.float64) * ws[:, None]).T
    _, one = O.lmhead(h, None, 1e-6, wq, ws, want_logits=True)
    e1 = np.abs(O.bf16_to_f32(one) - exact).mean()
    e2 = np.abs(O.bf16_to_f32(logits) - exact).mean()
    assert e2 < 0.5 * e1, (e1, e2)


def test_lmhead_ties_take_the_first_index(oracle_mod):
    O = oracle_mod
    R, V = 2, 512
    h, wq, ws = _lmhead_inputs(O, R, V, 2)
    wq[300] = wq[100]
    ws[300] = ws[100]
    wq[100] = 127 * np.sign(O.bf16_to_f32(h[0])).astype(np.int8)  # row 0's best column, twice
    wq[300] = wq[100]
    ids, logits = O.lmhead(h, None, 1e-6, wq, ws, want_logits=True)
    assert logits[0, 100] == logits[0, 300] and ids[0] == 100


def test_lmhead_norm_against_float64(oracle_mod):
    O = oracle_mod
    R, V = 4, 1024
    h, wq, ws = _lmhead_inputs(O, R, V, 3)
    nw = O.f32_to_bf16((np.random.default_rng(4).standard_normal(2048) * 0.1).astype(np.float32))
    _, logits = O.lmhead(h, nw, 1e-6, wq, ws, want_logits=True)
    x = O.bf16_to_f32(h).astype(np.float64)
    y = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-6) * (1.0 + O.bf16_to_f32(nw).astype(np.float64))
    yq, ys = torch_quant_rows_i8(_bf(O, y.astype(np.float32)))  # the node quantizes the bf16 norm output
    ref = (yq.astype(np.float64) * ys[:, None]) @ (wq.astype(np.float64) * ws[:, None].astype(np.float64)).T
    assert_bf16_close(logits, O.f32_to_bf16(ref.astype(np.float32)), 1e-2, "lm_head with norm")


def _attn_setup(O, T, seed):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16(rng.standard_normal((T, 2048)).astype(np.float32))
    w = (rng.standard_normal((9216, 2048)) * 0.02).astype(np.float32)
    q, s = O.quant_blocks_e4m3(w)
    qn = O.f32_to_bf16((rng.standard_normal(256) * 0.1).astype(np.float32))
    kn = O.f32_to_bf16((rng.standard_normal(256) * 0.1).astype(np.float32))
    return x, q, s, qn, kn


def _cos_sin(max_pos, theta=1e7):
    inv = theta ** (-np.arange(0, 64, 2, dtype=np.float64) / 64)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32), inv


def _run(O, x, q, s, qn, kn, cs, pos):
    return O.attn_proj(x, q[:8192], s[:64], q[8192:8704], s[64:68], q[8704:], s[68:72], qn, kn, 1e-6, cs, pos)


def test_attn_proj_against_float64(oracle_mod):
    O = oracle_mod
    T = 3
    x, q, s, qn, kn = _attn_setup(O, T, 5)
    cs, inv = _cos_sin(40000)
    pos = np.array([0, 17, 32767], np.int32)
    r = _run(O, x, q, s, qn, kn, cs, pos)
    xq, xs = O.quant_groups_e4m3(O.bf16_to_f32(x), 128)
    xd = O.e4m3_to_f32(xq).astype(np.float64) * np.repeat(xs, 128, axis=1)
    wd = O.e4m3_to_f32(q).astype(np.float64) * np.repeat(np.repeat(s, 128, axis=0), 128, axis=1)
    qkv = _bf(O, (xd @ wd.T).astype(np.float32)).astype(np.float64)

    def norm_rope(v, w, p):
        v = v / np.sqrt((v * v).mean() + 1e-6) * (1.0 + O.bf16_to_f32(w).astype(np.float64))
        c, sn = np.cos(p * inv), np.sin(p * inv)
        out = v.copy()
        out[:32] = v[:32] * c - v[32:64] * sn
        out[32:64] = v[32:64] * c + v[:32] * sn
        return out

    for t in range(T):
        qr = np.stack([norm_rope(qkv[t, h * 512:h * 512 + 256], qn, pos[t]) for h in range(16)])
        gr = np.stack([qkv[t, h * 512 + 256:h * 512 + 512] for h in range(16)])
        kr = np.stack([norm_rope(qkv[t, 8192 + h * 256:8192 + h * 256 + 256], kn, pos[t]) for h in range(2)])
        vr = np.stack([qkv[t, 8704 + h * 256:8704 + h * 256 + 256] for h in range(2)])
        for name, ref in (("q", qr), ("gate", gr), ("k", kr), ("v", vr)):
            assert_bf16_close(r[name][t], O.f32_to_bf16(ref.astype(np.float32)), 1e-2, f"{name}[{t}]")
    assert np.array_equal(r["k8"], O.f32_to_e4m3(O.bf16_to_f32(r["k"])))
    assert np.array_equal(r["v8"], O.f32_to_e4m3(O.bf16_to_f32(r["v"])))


def test_rope_invariants(oracle_mod):
    O = oracle_mod
    x, q, s, qn, kn = _attn_setup(O, 1, 6)
    cs, inv = _cos_sin(40000)
    r0 = _run(O, x, q, s, qn, kn, cs, np.array([0], np.int32))
    p = 5
    r1 = _run(O, x, q, s, qn, kn, cs, np.array([p], np.int32))
    for name in ("q", "k"):
        a0 = O.bf16_to_f32(r0[name][0]).astype(np.float64)
        a1 = O.bf16_to_f32(r1[name][0]).astype(np.float64)
        assert np.array_equal(r0[name][0][:, 64:], r1[name][0][:, 64:]), "dims 64.. moved with the position"
        z0 = a0[:, :32] + 1j * a0[:, 32:64]
        z1 = a1[:, :32] + 1j * a1[:, 32:64]
        assert np.allclose(np.abs(z1), np.abs(z0), rtol=2e-2, atol=1e-2)
        big = np.abs(z0) > 0.5
        turn = np.angle(z1[big] / z0[big])
        want = np.angle(np.exp(1j * p * np.broadcast_to(inv, z0.shape)[big]))
        assert np.allclose(np.angle(np.exp(1j * (turn - want))), 0, atol=2e-2)


def test_oproj_against_float64(oracle_mod):
    O = oracle_mod
    T = 2
    rng = np.random.default_rng(7)
    attn = O.f32_to_bf16(rng.standard_normal((T, 4096)).astype(np.float32))
    gate = O.f32_to_bf16((rng.standard_normal((T, 4096)) * 2).astype(np.float32))
    wo = (rng.standard_normal((2048, 4096)) * 0.02).astype(np.float32)
    qo, so = O.quant_blocks_e4m3(wo)
    out = O.attn_oproj(attn, gate, qo, so)
    g = O.bf16_to_f32(attn).astype(np.float64) / (1.0 + np.exp(-O.bf16_to_f32(gate).astype(np.float64)))
    gq, gs = O.quant_groups_e4m3(_bf(O, g.astype(np.float32)), 128)
    gd = O.e4m3_to_f32(gq).astype(np.float64) * np.repeat(gs, 128, axis=1)
    wd = O.e4m3_to_f32(qo).astype(np.float64) * np.repeat(np.repeat(so, 128, axis=0), 128, axis=1)
    assert_bf16_close(out, O.f32_to_bf16((gd @ wd.T).astype(np.float32)), 1e-2, "oproj")
