"""Pins of the oracle's W8A16 forms (CPU): bf16 rows times int8 weights, products exact in fp32.

DENSE8 linear (L/dense8.py:229-265 _w8_seg_kernel): y = bf16(sum over 128-column groups of
dot_g * s_g), accumulated group by group.  lm_head W8A16 (H/lmhead8.py:57-91): logit =
bf16(dot * ws[n]), first index of the row maximum.
Exact cases: integer-valued activations and power-of-two scales make every dot, product and partial
sum exact, so the outputs equal the float64 closed form rounded once to bf16 (a wrong group index,
a transposed weight or a dropped group fails them).  Random cases: within the bf16 bar of the float64
product of the dequantized operands.  Round trip: quant_dense8 then the linear reproduces x @ w.T
within the quantization bound sum |x| s / 2.
"""
import numpy as np

from helpers import assert_bf16_close


def _bf(O, x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


def _pow2_scales(rng, G, N):
    return (2.0 ** rng.integers(-4, 3, (G, N))).astype(np.float16)


def test_dense8_linear_exact_on_integer_inputs(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(0)
    T, N, K = 5, 40, 512
    x = rng.integers(-8, 9, (T, K)).astype(np.float32)
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = _pow2_scales(rng, K // 128, N)
    y = O.dense8_linear(_bf(O, x), q, s)
    deq = q.astype(np.float64) * np.repeat(s.astype(np.float64).T, 128, axis=1)  # [N, K]
    ref = x.astype(np.float64) @ deq.T
    assert np.array_equal(y, _bf(O, ref))
    # the scale row of each group matters: shifting the groups by one changes the result
    assert not np.array_equal(O.dense8_linear(_bf(O, x), q, np.roll(s, 1, axis=0)), y)


def test_dense8_linear_wide_scale_buffer_and_random(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(1)
    T, N, K = 7, 96, 1024
    x = _bf(O, rng.standard_normal((T, K)))
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    wide = (rng.random((K // 128, N + 24)) * 1e-3 + 1e-5).astype(np.float16)
    y = O.dense8_linear(x, q, wide[:, :N].copy())
    y_wide = O.dense8_linear(x, q, wide)  # a column block of a wider buffer: only the first N columns are read
    assert np.array_equal(y, y_wide)
    deq = q.astype(np.float64) * np.repeat(wide[:, :N].astype(np.float64).T, 128, axis=1)
    ref = O.bf16_to_f32(x).astype(np.float64) @ deq.T
    assert_bf16_close(y, _bf(O, ref), 8e-3, "dense8 linear vs float64")


def test_dense8_quantize_then_linear_round_trip(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(2)
    T, N, K = 4, 64, 2048
    w = O.bf16_to_f32(_bf(O, rng.standard_normal((N, K)) * 0.02))
    q, s = O.quant_dense8(w)
    x = O.bf16_to_f32(_bf(O, rng.standard_normal((T, K))))
    y = O.bf16_to_f32(O.dense8_linear(_bf(O, x), q, s)).astype(np.float64)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    sf = s.view(np.float16).astype(np.float64)                      # [K/128, N]
    bound = np.abs(x).reshape(T, K // 128, 128).sum(axis=2) @ (sf / 2)  # sum |x| s / 2 per output
    assert np.all(np.abs(y - exact) <= bound + np.abs(exact) * 2 ** -8 + 1e-6)


def test_lmhead_w8a16_exact_on_integer_rows(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(3)
    R, V = 6, 1024
    h = _bf(O, rng.integers(-6, 7, (R, 2048)))
    wq = rng.integers(-127, 128, (V, 2048), dtype=np.int8)
    ws = (rng.random(V) * 2e-4 + 1e-5).astype(np.float32)
    ids, logits = O.lmhead(h, None, 1e-6, wq, ws, want_logits=True, w8a16=True)
    acc = O.bf16_to_f32(h).astype(np.int64) @ wq.astype(np.int64).T    # exact integers, < 2^24
    assert np.abs(acc).max() < 2 ** 24
    ref = _bf(O, acc.astype(np.float32) * ws[None, :])
    assert np.array_equal(logits, ref)
    assert np.array_equal(ids, np.argmax(O.bf16_to_f32(ref), axis=1))


def test_lmhead_w8a16_norm_and_ties(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(4)
    R, V = 4, 1024
    h = _bf(O, rng.standard_normal((R, 2048)))
    wq = rng.integers(-127, 128, (V, 2048), dtype=np.int8)
    ws = (rng.random(V) * 2e-4 + 1e-5).astype(np.float32)
    nw = _bf(O, rng.standard_normal(2048) * 0.1)
    wq[700], ws[700] = wq[200], ws[200]
    ids, logits = O.lmhead(h, nw, 1e-6, wq, ws, want_logits=True, w8a16=True)
    x = O.bf16_to_f32(h).astype(np.float64)
    y = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-6) * (1.0 + O.bf16_to_f32(nw).astype(np.float64))
    yb = O.bf16_to_f32(_bf(O, y)).astype(np.float64)                     # the node feeds the bf16 norm output
    ref = yb @ (wq.astype(np.float64) * ws[:, None].astype(np.float64)).T
    assert_bf16_close(logits, _bf(O, ref), 8e-3, "lm_head W8A16 with norm")
    assert np.array_equal(logits[:, 700], logits[:, 200])
    lg = O.bf16_to_f32(logits)
    assert np.array_equal(ids, np.argmax(lg, axis=1))
    # W8A16 keeps the activations unquantized: closer to the float64 product than the one-term int8 form
    _, one = O.lmhead(h, nw, 1e-6, wq, ws, want_logits=True)
    e16 = np.abs(lg - ref).mean()
    e8 = np.abs(O.bf16_to_f32(one) - ref).mean()
    assert e16 < 0.5 * e8, (e16, e8)
