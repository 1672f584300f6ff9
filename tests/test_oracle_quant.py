"""Pins of the oracle's quantizers against torch restatements of the reference's formulas (CPU).

int8 rule: H/lmhead8.py:129-143 quantize_rows_torch (s = amax/127, round half away, clamp);
e4m3 rule: the per-token x 128-group rule of L/qk_moe_prefill_i8.cu:3671-3705 with 448 for 127.
"""
import numpy as np
import torch


def torch_quant_rows_i8(w):
    wf = torch.from_numpy(w).double().float()
    s = wf.abs().amax(dim=1) / 127.0
    v = wf / torch.where(s > 0, s, torch.ones_like(s)).unsqueeze(1)
    r = torch.sign(v) * torch.floor(v.abs() + 0.5)
    return r.clamp(-127, 127).to(torch.int8).numpy(), s.numpy()


def torch_quant_e4m3(x, amax):
    inv = torch.where(amax > 0, 448.0 / amax, torch.zeros_like(amax))
    return (x * inv).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8), amax / 448.0


def test_quant_rows_i8_matches_reference_formula(oracle_mod):
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((257, 2048)) * 0.02).astype(np.float32)
    w[3] = 0.0
    w[4, :] = 0.0
    w[4, 7] = -1.5
    w[5, :8] = np.array([127, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 126.5], np.float32)  # exact .5 ties
    q, s = oracle_mod.quant_rows_i8(w)
    qr, sr = torch_quant_rows_i8(w)
    assert np.array_equal(q, qr) and np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    assert s[3] == 0 and not q[3].any()
    assert list(q[5, :8]) == [127, 64, -64, 1, -1, 2, -3, 127]  # half away from zero
    deq = q.astype(np.float64) * s[:, None]
    assert np.all(np.abs(deq - w) <= s[:, None] * 0.5 + 1e-12)


def test_quant_groups_e4m3_matches_torch(oracle_mod):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((33, 2048)).astype(np.float32) * np.float32(3)
    x[2, :128] = 0.0
    q, s = oracle_mod.quant_groups_e4m3(x, 128)
    xt = torch.from_numpy(x).view(33, 16, 128)
    qr, sr = torch_quant_e4m3(xt, xt.abs().amax(dim=2, keepdim=True))
    assert np.array_equal(q, qr.reshape(33, 2048).numpy())
    assert np.array_equal(s.view(np.uint32), sr.reshape(33, 16).numpy().view(np.uint32))
    assert s[2, 0] == 0 and not q[2, :128].any()
    # every group's largest magnitude lands on the 448 code
    assert np.all(np.abs(oracle_mod.e4m3_to_f32(q)).reshape(33, 16, 128).max(axis=2)[s > 0] == 448)


def test_quant_blocks_e4m3_matches_torch(oracle_mod):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    q, s = oracle_mod.quant_blocks_e4m3(w)
    wt = torch.from_numpy(w).view(2, 128, 3, 128).permute(0, 2, 1, 3)
    amax = wt.abs().amax(dim=(2, 3), keepdim=True)
    qr, sr = torch_quant_e4m3(wt, amax)
    qr = qr.permute(0, 2, 1, 3).reshape(256, 384).numpy()
    assert np.array_equal(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.reshape(2, 3).numpy().view(np.uint32))
    sb = np.broadcast_to(s[:, None, :, None], (2, 128, 3, 128)).reshape(256, 384)
    deq = oracle_mod.e4m3_to_f32(q) * sb
    # half a step of the e4m3 grid: 2^-4 relative in the normal range, 2^-10 * s in the subnormal one
    assert np.all(np.abs(deq - w) <= 2 ** -4 * np.abs(w) + sb * 2 ** -10 * (1 + 1e-6))
