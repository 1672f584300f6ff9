"""Pins of the oracle's hybrid-layer glue: the e4m3 block-scaled linear and the add + Gemma RMSNorm
(L/proj.py:60-81).  Each is checked against an independent numpy restatement and closed forms."""
import numpy as np
import pytest

from oracle import oracle as O


def _bf(x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


def test_add_rmsnorm_residual_is_the_exact_bf16_sum():
    rng = np.random.default_rng(0)
    d = _bf(rng.standard_normal((5, 2048)))
    r = _bf(rng.standard_normal((5, 2048)) * 3)
    w = _bf(rng.standard_normal(2048) * 0.1)
    out, res = O.add_rmsnorm(d, r, w, 1e-6)
    want = O.f32_to_bf16(O.bf16_to_f32(d) + O.bf16_to_f32(r))  # one float32 add, one rounding
    assert np.array_equal(res, want)
    # the normalised rows against float64 (the canonical sum order is a rounding difference)
    z = (O.bf16_to_f32(d) + O.bf16_to_f32(r)).astype(np.float64)
    rstd = 1.0 / np.sqrt((z * z).mean(1, keepdims=True) + 1e-6)
    ref = z * rstd * (1.0 + O.bf16_to_f32(w).astype(np.float64))
    got = O.bf16_to_f32(out).astype(np.float64)
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-3)) < 2 ** -7


def test_add_rmsnorm_without_delta_keeps_the_residual():
    rng = np.random.default_rng(1)
    r = _bf(rng.standard_normal((3, 2048)))
    w = np.zeros(2048, np.uint16)
    out, res = O.add_rmsnorm(None, r, w, 0.0)
    assert np.array_equal(res, r)
    # w = 0 gives unit mean square (to bf16 rounding)
    y = O.bf16_to_f32(out).astype(np.float64)
    assert np.allclose((y * y).mean(1), 1.0, atol=1e-2)


def test_add_rmsnorm_constant_row_closed_form():
    r = np.full((1, 2048), _bf(np.float32(0.75)), np.uint16)
    w = np.full(2048, _bf(np.float32(0.5)), np.uint16)
    out, _ = O.add_rmsnorm(None, r, w, 0.0)
    # z = 0.75 everywhere: rstd = 1/0.75, y = 1 * 1.5
    assert np.all(O.bf16_to_f32(out) == np.float32(1.5))


@pytest.mark.parametrize("K", [2048, 4096])
def test_fp8_linear_against_float64(K):
    rng = np.random.default_rng(K)
    T, N = 3, 256
    x = _bf(rng.standard_normal((T, K)))
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq = np.empty((N, K), np.uint8)
    ws = np.empty((N // 128, K // 128), np.float32)
    O.lib().q36o_quant_blocks_e4m3(O._p(wf), N, K, O._p(wq), O._p(ws))
    got = O.bf16_to_f32(O.fp8_linear(x, wq, ws)).astype(np.float64)
    # independent restatement: the same quantization points, exact float64 products
    lut = O.e4m3_lut().astype(np.float64)
    xf = O.bf16_to_f32(x)
    xq = np.empty((T, K), np.uint8)
    xs = np.empty((T, K // 128), np.float32)
    O.lib().q36o_quant_groups_e4m3(O._p(np.ascontiguousarray(xf)), T, K, 128, O._p(xq), O._p(xs))
    xd = lut[xq] * np.repeat(xs.astype(np.float64), 128, axis=1)
    wd = lut[wq] * np.repeat(np.repeat(ws.astype(np.float64), 128, axis=0), 128, axis=1)
    ref = xd @ wd.T
    err = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert err.max() < 4e-3
    # and the quantization itself stays close to the unquantized product
    full = xf.astype(np.float64) @ wf.astype(np.float64).T
    assert (np.linalg.norm(got - full, axis=1) / np.linalg.norm(full, axis=1)).max() < 0.08


def test_fp8_linear_exact_on_exact_inputs():
    # amax 1.75 = 448 * 2^-8 and 0.4375 = 448 * 2^-10: power-of-two scales, code 448 (0x7e) for the
    # nonzero values, so every quantization, block sum and scale product is exact
    T, N, K = 2, 128, 2048
    x = np.zeros((T, K), np.float32)
    x[0, :128] = 1.75
    x[1, 128:256] = 1.75
    wf = np.zeros((N, K), np.float32)
    wf[:, :128] = 0.4375
    for n in range(N):
        wf[n, 128:128 + 2 ** (n % 4)] = 0.4375
    wq = np.empty((N, K), np.uint8)
    ws = np.empty((1, K // 128), np.float32)
    O.lib().q36o_quant_blocks_e4m3(O._p(wf), N, K, O._p(wq), O._p(ws))
    assert ws[0, 0] == 2.0 ** -10 and ws[0, 1] == 2.0 ** -10
    got = O.bf16_to_f32(O.fp8_linear(_bf(x), wq, ws))
    assert np.all(got[0] == np.float32(128 * 1.75 * 0.4375))
    assert np.array_equal(got[1], np.float32(1.75 * 0.4375) * (2.0 ** (np.arange(N) % 4)).astype(np.float32))
