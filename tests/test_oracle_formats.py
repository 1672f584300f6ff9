"""Pins of the oracle's restatement of the reference's prepare-time weight formats (CPU).

q8-block-v1 expert copies (L/i8x_kernels.py:12,69-141) and DENSE8 copies (L/dense8.py:140-188) share
one rule: s16 = fp16(fp32(amax / 127) * (1 + 2^-10)), q = clamp(round_half_away(w / s16), +-127).  It is
pinned against torch's own float16 conversion and a torch restatement written from the reference's
torch reference (quantize_torch, L/dense8.py:168-183), against the bound |w - q s| <= s / 2, against
amax = 0 rows and exact .5 ties, and the block layout against its byte offsets.
"""
import numpy as np
import pytest
import torch


def test_f16_codec_matches_torch(oracle_mod):
    O = oracle_mod
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(20000, generator=g) * s for s in (1e-8, 1e-5, 1e-3, 1, 100, 3e4)])
    edge = torch.tensor([0.0, -0.0, 65504.0, 65519.9, 65520.0, 7e4, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 2 ** -14,
                         2 ** -14 * (1 - 2 ** -11), float("inf"), -float("inf")])
    x = torch.cat([x, edge, -edge])
    got = O.f32_to_f16_bits(x.numpy())
    want = x.to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    back = np.array([O.lib().q36o_f16_to_f32(int(b)) for b in want[:5000]], np.float32)
    assert np.array_equal(back, torch.from_numpy(want[:5000].view(np.int16)).view(torch.float16).float().numpy())


def _torch_rule(w: torch.Tensor, group: int):
    """The reference's torch quantizer restated (L/dense8.py:168-183) on float32 rows of `group` columns."""
    N, K = w.shape
    wf = w.view(N, K // group, group)
    amax = wf.abs().amax(dim=2)
    s16 = ((amax / 127.0) * 1.0009765625).to(torch.float16)
    sf = s16.float()
    v = wf / torch.where(sf > 0, sf, torch.ones_like(sf)).unsqueeze(2)
    r = torch.sign(v) * torch.floor(v.abs() + 0.5)
    return r.clamp(-127, 127).to(torch.int8).view(N, K), s16


def test_dense8_matches_reference_rule_and_bounds(oracle_mod):
    O = oracle_mod
    g = torch.Generator().manual_seed(1)
    N, K = 96, 512
    w = (torch.randn((N, K), generator=g) * 0.02).to(torch.bfloat16).float()
    w[3] = 0.0                                           # amax = 0: zero codes, zero scale
    w[5, :128] = torch.arange(128) * 0.5                 # exact .5 ties in the first group
    q, s = O.quant_dense8(w.numpy(), s_stride=N + 8)     # a column block of a wider scale buffer
    rq, rs = _torch_rule(w, 128)
    assert np.array_equal(q, rq.numpy())
    assert np.array_equal(s[:, :N], rs.t().contiguous().view(torch.int16).numpy().view(np.uint16))
    assert not np.any(s[:, N:]), "columns past N of the scale buffer are not written"
    assert not np.any(q[3]) and not np.any(s[:, 3])
    sf = torch.from_numpy(s[:, :N].view(np.int16)).view(torch.float16).float().t().numpy()
    deq = q.reshape(N, K // 128, 128).astype(np.float64) * sf[:, :, None]
    err = np.abs(deq - w.numpy().reshape(N, K // 128, 128))
    assert np.all(err <= sf[:, :, None] / 2 + 1e-12), "|w - q s| <= s / 2 (no element clamped)"


@pytest.mark.parametrize("channel", [True, False])
def test_q8_block_v1_layout_and_rule(oracle_mod, channel):
    O = oracle_mod
    g = torch.Generator().manual_seed(2)
    E, H, I = 3, 256, 128
    w13 = (torch.randn((E, 2 * I, H), generator=g) * 0.02).to(torch.bfloat16).float()
    w2 = (torch.randn((E, H, I), generator=g) * 0.02).to(torch.bfloat16).float()
    blocks = O.quant_q8_block_v1(w13.numpy(), w2.numpy(), channel=channel)
    # byte offsets of the layout (L/i8x_kernels.py:69-74): int8 w13 | int8 w2 | fp16 c13 | fp16 c2
    assert blocks.shape[1] == 2 * I * H + H * I + 2 * I * (H // 128) * 2 + H * (I // 128) * 2
    for e in range(E):
        q13, q2, c13, c2 = O.q8_block_parts(blocks[e], H, I)
        for q, c, w, K in ((q13, c13, w13[e], H), (q2, c2, w2[e], I)):
            rq, rs = _torch_rule(w, K if channel else 128)
            assert np.array_equal(q, rq.numpy())
            rbits = rs.view(torch.int16).numpy().view(np.uint16)
            want = np.repeat(rbits, K // 128, axis=1) if channel else rbits
            assert np.array_equal(c, want), "scales: one per row replicated (channel) or one per group"
