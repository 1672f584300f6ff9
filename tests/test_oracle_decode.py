"""Pins for the decode / verify attention oracle (q36o_attn_decode): the f16 rounding of the softmax
weights against torch, closed forms (one visible key, uniform scores), the causal rule among the
new tokens, the grouped-query head mapping, order independence, and an independent float64
restatement built on torch's e4m3 / f16 conversions."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def _inputs(B, NT, L, seed, slots=None, q_scale=1.0):
    rng = np.random.default_rng(seed)
    HQ, HKV, D = 16, 2, 256
    slots = slots or B * L + 7
    q = torch.from_numpy(rng.standard_normal((B * NT, HQ, D)).astype(np.float32) * q_scale).to(torch.bfloat16)
    kc = torch.from_numpy(rng.standard_normal((slots, HKV, D)).astype(np.float32)).to(torch.float8_e4m3fn)
    vc = torch.from_numpy(rng.standard_normal((slots, HKV, D)).astype(np.float32)).to(torch.float8_e4m3fn)
    pt = np.stack([rng.permutation(slots)[:L] for _ in range(B)]).astype(np.int32)
    return q.view(torch.int16).numpy().view(np.uint16), kc.view(torch.uint8).numpy(), vc.view(torch.uint8).numpy(), pt


def test_f16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32), rng.uniform(0, 1e-4, 50000).astype(np.float32),
                        np.array([0.0, -0.0, 1.0, 2 ** -24, 2 ** -25, 3 * 2 ** -25, 65504.0, 1 + 2 ** -11, 1 + 3 * 2 ** -11],
                                 np.float32)])
    ref = torch.from_numpy(x).to(torch.float16).to(torch.float32).numpy()
    assert np.array_equal(O.f16_round(x).view(np.uint32), ref.view(np.uint32))


def test_one_visible_key_returns_its_value():
    B, NT, L = 2, 1, 8
    q, kc, vc, pt = _inputs(B, NT, L, 1)
    seq = np.array([1, 1], np.int32)  # one key: p = 1, out = bf16(v)
    out = O.attn_decode(q, kc, vc, pt, seq, NT, 1 / 16)
    v = torch.from_numpy(vc).view(torch.float8_e4m3fn).float()
    for r in range(B):
        for i in range(16):
            ref = v[pt[r, 0], i // 8].to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(out[r, i], ref)


def test_uniform_scores_give_the_mean_value():
    B, NT, L = 2, 2, 37
    q, kc, vc, pt = _inputs(B, NT, L, 2)
    q[:] = 0  # every score 0: p = 1 for all visible keys
    seq = np.array([37, 20], np.int32)
    out = O.attn_decode(q, kc, vc, pt, seq, NT, 1 / 16)
    v = torch.from_numpy(vc).view(torch.float8_e4m3fn).double()
    for r in range(B):
        for t in range(NT):
            nk = seq[r] - NT + t + 1
            for i in (0, 7, 8, 15):
                mean = v[torch.from_numpy(pt[r, :nk]).long(), i // 8].mean(0)
                ref = mean.float().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
                assert np.array_equal(out[r * NT + t, i], ref)


def test_causal_rule_and_head_mapping():
    B, NT, L = 1, 4, 50
    q, kc, vc, pt = _inputs(B, NT, L, 3)
    seq = np.array([50], np.int32)
    base = O.attn_decode(q, kc, vc, pt, seq, NT, 1 / 16)
    # keys after a token's last visible position change nothing for it (token t sees 0 .. 46 + t)
    kc2, vc2 = kc.copy(), vc.copy()
    for pos in (48, 49):
        kc2[pt[0, pos]] ^= 0x11
        vc2[pt[0, pos]] ^= 0x22
    out = O.attn_decode(q, kc2, vc2, pt, seq, NT, 1 / 16)
    assert np.array_equal(out[:2], base[:2])          # tokens 0, 1 see positions <= 47
    assert not np.array_equal(out[3], base[3])        # token 3 sees 49
    # q heads 0..7 read kv head 0 only, 8..15 kv head 1 only
    vc3 = vc.copy()
    vc3[:, 1] ^= 0x33
    out3 = O.attn_decode(q, kc, vc3, pt, seq, NT, 1 / 16)
    assert np.array_equal(out3[:, :8], base[:, :8]) and not np.array_equal(out3[:, 8:], base[:, 8:])


def test_key_order_does_not_matter():
    B, NT, L = 1, 1, 64
    q, kc, vc, pt = _inputs(B, NT, L, 4)
    seq = np.array([64], np.int32)
    a = O.attn_decode(q, kc, vc, pt, seq, NT, 1 / 16)
    perm = np.random.default_rng(9).permutation(64)
    b = O.attn_decode(q, kc, vc, pt[:, perm], seq, NT, 1 / 16)
    fa = a.astype(np.uint32) << 16
    fb = b.astype(np.uint32) << 16
    np.testing.assert_allclose(fa.view(np.float32), fb.view(np.float32), rtol=1e-2, atol=1e-6)


@pytest.mark.parametrize("NT", [1, 4])
def test_against_float64_restatement(NT):
    B, L = 2, 70
    q, kc, vc, pt = _inputs(B, NT, L, 5 + NT, q_scale=2.0)
    seq = np.array([70, 33], np.int32)
    out = O.attn_decode(q, kc, vc, pt, seq, NT, 1 / 16)
    qd = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).float().to(torch.float8_e4m3fn).double()
    kd = torch.from_numpy(kc).view(torch.float8_e4m3fn).double()
    vd = torch.from_numpy(vc).view(torch.float8_e4m3fn).double()
    got = torch.from_numpy((out.astype(np.uint32) << 16).view(np.float32)).double()
    for r in range(B):
        for t in range(NT):
            nk = int(seq[r]) - NT + t + 1
            idx = torch.from_numpy(pt[r, :nk]).long()
            for i in range(16):
                s = (kd[idx, i // 8] @ qd[r * NT + t, i]) / 16
                p = torch.exp(s - s.max())
                p16 = p.float().to(torch.float16).double()
                ref = (p16 @ vd[idx, i // 8]) / p.sum()
                err = (got[r * NT + t, i] - ref).norm() / ref.norm()
                assert err < 4e-3, (r, t, i, float(err))
