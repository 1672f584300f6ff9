"""GPU parity of the ReplaySSM GDN verify (q36_gdn_verify_ring through the C-ABI) against the oracle.

Bar: conv state pool and window records bit-exact; bf16 outputs within 1e-2 relative (per-row
norm); the appended d entries (high + low parts) within 1e-4 of the oracle's, keys within 4e-5
(two bf16 parts hold 16 bits), gates within 1e-5; every ring entry the call must not write is unchanged bit for bit.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, assert_f32_close, bf16_f32, bits16, np_

pytestmark = pytest.mark.gpu

POOLS = ("conv_state", "window", "d_ring", "dlo_ring", "k_ring", "klo_ring", "g_ring")


@pytest.fixture(scope="module")
def gdn():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import gdn_fused
    return gdn_fused


def _host(t):
    return bits16(t) if t.dtype == torch.bfloat16 else np_(t)


def _case(gdn, O, dev, B, T, seed, wp=None, padded=(), idx32=False, dt_bf16=False, view4=False):
    from bundles_amd import synth
    print(f"gdn ring B={B} T={T} seed={seed} wp={wp} padded={padded} idx32={idx32} dt_bf16={dt_bf16} "
          f"view4={view4}", flush=True)
    d = synth.gdn_ring_inputs(B, T, dev, seed=seed, wp=wp, padded=padded)
    if idx32:
        for k in ("state_idx", "replay_idx", "win_idx"):
            d[k] = d[k].to(torch.int32)
    if dt_bf16:
        d["dt_bias"] = d["dt_bias"].to(torch.bfloat16)
    host = {k: _host(v) for k, v in d.items() if isinstance(v, torch.Tensor)}
    if dt_bf16:
        host["dt_bias"] = bf16_f32(host["dt_bias"])
    before = {k: host[k].copy() for k in POOLS}
    win = d["window"]
    if view4:  # the reference's deduplicated [slots, T, 8192, 3] view of the [slots, 8192, T + 2] records
        win = torch.as_strided(win, (win.shape[0], T, 8192, 3), (win.stride(0), 1, T + 2, 1))
    out = gdn.gdn_verify_ring(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"], win, d["A_log"],
                              d["dt_bias"], d["h0"], d["d_ring"], d["dlo_ring"], d["k_ring"], d["klo_ring"],
                              d["g_ring"], d["qsl"], d["state_idx"], d["replay_idx"], d["win_idx"], d["write_pos"],
                              d["cache_base"], d["norm_w"], 1e-6, d["scale"], T=T)
    torch.cuda.synchronize()
    ref = O.gdn_verify_ring(B, T, host["mixed"], host["z"], host["a"], host["b"], before["conv_state"],
                            host["conv_w"], before["window"], host["A_log"], host["dt_bias"], host["h0"],
                            before["d_ring"], before["dlo_ring"], before["k_ring"], before["klo_ring"],
                            before["g_ring"], host["qsl"], host["state_idx"], host["replay_idx"], host["win_idx"],
                            host["write_pos"], host["cache_base"], host["norm_w"], 1e-6, d["scale"])
    got = {k: _host(d[k]) for k in POOLS}
    worst = assert_bf16_close(bits16(out), ref["out"], 1e-2, "ring verify out")
    assert np.array_equal(got["conv_state"], ref["conv_state"]), "conv state pool"
    assert np.array_equal(got["window"], ref["window"]), "window records"
    # appended entries: values against the oracle; everything else untouched
    written = {k: np.zeros(ref[k].shape[:3], bool) for k in ("d_ring", "k_ring", "g_ring")}
    si, rp_all = host["state_idx"], host["replay_idx"]
    for r in range(B):
        if si[r] < 0:
            continue
        rp = rp_all[r]
        n = int(np.clip(host["write_pos"][rp], 0, 16))
        for t in range(T):
            if n + t >= 16:
                break
            p = (int(host["cache_base"][rp]) + n + t) & 15
            written["d_ring"][rp, :, p] = True
            written["k_ring"][rp, :, p] = True
            written["g_ring"][rp, :, p] = True
            gd = bf16_f32(got["d_ring"][rp, :, p]).astype(np.float64) + bf16_f32(got["dlo_ring"][rp, :, p])
            rd = bf16_f32(ref["d_ring"][rp, :, p]).astype(np.float64) + bf16_f32(ref["dlo_ring"][rp, :, p])
            assert_f32_close(gd, rd, 1e-4, f"d entry r={r} t={t}")
            gk = bf16_f32(got["k_ring"][rp, :, p]).astype(np.float64) + bf16_f32(got["klo_ring"][rp, :, p])
            rk = bf16_f32(ref["k_ring"][rp, :, p]).astype(np.float64) + bf16_f32(ref["klo_ring"][rp, :, p])
            # high + low bf16 parts hold 16 significant bits (2^-16 ~ 1.5e-5 of an element): a last-bit
            # difference in the unit key (its norm's summation order) can move the split by that much
            assert_f32_close(gk, rk, 4e-5, f"k entry r={r} t={t}")
            assert np.allclose(got["g_ring"][rp, :, p], ref["g_ring"][rp, :, p], rtol=1e-5, atol=0), f"g r={r} t={t}"
    for k, kl in (("d_ring", "dlo_ring"), ("k_ring", "klo_ring"), ("g_ring", None)):
        keep = ~written[k]
        assert np.array_equal(got[k][keep], before[k][keep]), f"{k}: an entry outside the appends changed"
        if kl:
            assert np.array_equal(got[kl][keep], before[kl][keep]), f"{kl}: an entry outside the appends changed"
    for r in padded:
        assert not np.any(bits16(out)[r * T:(r + 1) * T]), "padded rows are zero"
    return worst


def test_ring_bench_shape(gdn, oracle_mod, dev):
    """32 requests x 4 drafts (the reference's window), random committed history 0 .. 12."""
    w = _case(gdn, oracle_mod, dev, 32, 4, seed=1)
    print("worst row / elem / exact:", w)


def test_ring_config3_window_partial_appends(gdn, oracle_mod, dev):
    """1 + 4 positions (config 3's window) with 13 committed entries: only three appends fit."""
    _case(gdn, oracle_mod, dev, 8, 5, seed=2, wp=13)


@pytest.mark.parametrize("T,wp", [(1, 16), (8, 0), (2, 15)])
def test_ring_edges(gdn, oracle_mod, dev, T, wp):
    _case(gdn, oracle_mod, dev, 4, T, seed=3 + T, wp=wp)


def test_ring_int32_indices_bf16_dt_padding_and_window_view(gdn, oracle_mod, dev):
    _case(gdn, oracle_mod, dev, 6, 4, seed=9, padded=(0, 4), idx32=True, dt_bf16=True, view4=True)


def test_empty_ring_matches_snapshot_kernel(gdn, dev):
    """write_pos 0: the ring kernel starts from the checkpoint itself, so its output is the snapshot
    kernel's (q36_gdn_verify) on the same inputs, within the bf16 bar."""
    from bundles_amd import synth
    B, T = 16, 5
    d = synth.gdn_ring_inputs(B, T, dev, seed=12, wp=0)
    si = d["state_idx"]
    snap_out, _, cs_out = gdn.gdn_verify_fused(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"][si].contiguous(),
                                               d["conv_w"], d["A_log"], d["dt_bias"], d["h0"][si].contiguous(),
                                               d["norm_w"], 1e-6, T=T)
    out = gdn.gdn_verify_ring(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"], d["window"],
                              d["A_log"], d["dt_bias"], d["h0"], d["d_ring"], d["dlo_ring"], d["k_ring"],
                              d["klo_ring"], d["g_ring"], d["qsl"], d["state_idx"], d["replay_idx"], d["win_idx"],
                              d["write_pos"], d["cache_base"], d["norm_w"], 1e-6, d["scale"], T=T)
    torch.cuda.synchronize()
    assert_bf16_close(bits16(out), bits16(snap_out), 1e-2, "ring vs snapshot kernel")
    assert torch.equal(d["conv_state"][si], cs_out), "both roll the conv state the same way"


def test_ring_rejects_bad_layouts(gdn, dev):
    from bundles_amd import synth
    d = synth.gdn_ring_inputs(2, 4, dev, seed=0)
    args = [d[k] for k in ("mixed", "z", "a", "b", "conv_state", "conv_w", "window", "A_log", "dt_bias", "h0",
                           "d_ring", "dlo_ring", "k_ring", "klo_ring", "g_ring", "qsl", "state_idx", "replay_idx",
                           "win_idx", "write_pos", "cache_base", "norm_w")]
    with pytest.raises(ValueError, match="multiple of the draft window"):
        gdn.gdn_verify_ring(*args, T=3)
    bad = list(args)
    bad[10] = d["d_ring"][:, :, :8]  # an 8-entry ring is not the served layout
    with pytest.raises(ValueError, match="d ring"):
        gdn.gdn_verify_ring(*bad, T=4)


@pytest.mark.parametrize("padded", [(), (1,)])
def test_ring_out_proj_codes(gdn, dev, padded):
    """The verify kernel's e4m3 codes of its output (oq) drive the out_proj (q36_fp8_linear, K = 4096)
    to the same bits as the bf16 output does; a padded request's rows get zero codes and scales."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import glue
    B, T = 4, 5
    print(f"gdn ring out_proj codes padded={padded}", flush=True)
    d = synth.gdn_ring_inputs(B, T, dev, seed=41, padded=padded)
    pools = {k: d[k].clone() for k in POOLS}

    def run(oq):
        for k in POOLS:
            d[k].copy_(pools[k])
        return gdn.gdn_verify_ring(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"], d["window"],
                                   d["A_log"], d["dt_bias"], d["h0"], d["d_ring"], d["dlo_ring"], d["k_ring"],
                                   d["klo_ring"], d["g_ring"], d["qsl"], d["state_idx"], d["replay_idx"],
                                   d["win_idx"], d["write_pos"], d["cache_base"], d["norm_w"], 1e-6, d["scale"],
                                   T=T, oq=oq)
    out1 = run(None).clone()
    oq = glue.linear_rows(B * T, 4096, dev)
    oq.codes.fill_(0x7F)
    oq.scales.fill_(float("nan"))
    out2 = run(oq)
    g = torch.Generator(device=dev).manual_seed(3)
    w = glue.prepare_fp8_weight((torch.randn((2048, 4096), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    ws = glue.LinearWorkspace(B * T, 4096, dev)
    y1 = glue.fp8_linear(out1, w, ws)
    y2 = glue.fp8_linear(None, w, ws, xq=oq)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert (oq.codes != 0x7F).all() and torch.isfinite(oq.scales).all()
    for r in padded:
        rows = slice(int(d["qsl"][r]), int(d["qsl"][r]) + T)
        assert not oq.codes[rows].any() and not oq.scales[rows].any()
