"""Pins of the oracle's GDN verify over the ReplaySSM ring (CPU).

The ring oracle is pinned by what is independent of its own code:
  * an empty ring (write_pos 0) is the snapshot verify from the checkpoint: bit-identical output,
    rolled state and gates, and the appended (d, k) entries rebuild every snapshot state through
    S_t = e^{g_t} S_{t-1} + d_t k_t^T (high + low parts, so to ~2^-16);
  * a float64 matrix-form restatement (S_t = e^{g_t} S_{t-1} (I - beta k k^T) + beta v k^T) from the
    history state td h0 + sum_c decay_c dhat_c khat_c^T, decay from the suffix sums of the gates;
  * two chained windows (the first appends T entries, all accepted, the second reads them back)
    against one snapshot verify over 2T positions: the ReplaySSM invariant, within the bf16 bar
    (the verify reads only the entries' high parts);
  * rotating the ring's physical slots with cache_base changes nothing; padded requests write
    zeros and nothing else; the window record is [s1 s2 x0 .. x_{T-1}].
"""
import numpy as np
import pytest

from helpers import assert_bf16_close, assert_f32_close, bf16_f32


def _np(d):
    import torch
    out = {}
    for k, v in d.items():
        if isinstance(v, (int, float)):
            out[k] = v
        elif v.dtype == torch.bfloat16:
            out[k] = v.contiguous().view(torch.int16).numpy().view(np.uint16)
        else:
            out[k] = v.contiguous().numpy()
    return out


def _inputs(B, T, seed, **kw):
    from bundles_amd import synth
    return _np(synth.gdn_ring_inputs(B, T, "cpu", seed=seed, **kw))


def _ring(O, d, B, T, use_f64=False, **over):
    a = dict(d, **over)
    return O.gdn_verify_ring(B, T, a["mixed"], a["z"], a["a"], a["b"], a["conv_state"], a["conv_w"], a["window"],
                             a["A_log"], a["dt_bias"], a["h0"], a["d_ring"], a["dlo_ring"], a["k_ring"],
                             a["klo_ring"], a["g_ring"], a["qsl"], a["state_idx"], a["replay_idx"], a["win_idx"],
                             a["write_pos"], a["cache_base"], a["norm_w"], 1e-6, a["scale"], use_f64=use_f64)


def _snap(O, d, B, T, mixed=None, z=None, a=None, b=None, conv_state=None):
    """The snapshot verify (q36o_gdn_verify) of the same requests from their checkpoints."""
    si = d["state_idx"]
    S0 = np.ascontiguousarray(d["h0"][si])
    cs = np.ascontiguousarray(d["conv_state"][si] if conv_state is None else conv_state)
    return O.gdn_verify(B, T, d["mixed"] if mixed is None else mixed, d["z"] if z is None else z,
                        d["a"] if a is None else a, d["b"] if b is None else b, cs, d["conv_w"], d["A_log"],
                        d["dt_bias"], S0, d["norm_w"], 1e-6)


def _phys(d, r, c):
    rp = d["replay_idx"][r]
    return (int(d["cache_base"][rp]) + c) & 15


def test_empty_ring_is_the_snapshot_verify(oracle_mod):
    O = oracle_mod
    B, T = 3, 4
    d = _inputs(B, T, seed=5, wp=0)
    res = _ring(O, d, B, T)
    out, snaps, cs = _snap(O, d, B, T)
    assert np.array_equal(res["out"], out), "empty ring: output must equal the snapshot verify bit for bit"
    si = d["state_idx"]
    assert np.array_equal(res["conv_state"][si], cs), "rolled conv state"
    conv_in = np.concatenate([bf16_f32(d["conv_state"][si]),
                              bf16_f32(d["mixed"]).reshape(B, T, 8192).transpose(0, 2, 1)], axis=2)
    assert np.array_equal(bf16_f32(res["window"][d["win_idx"]]), conv_in[:, :, 1:]), "window record"
    a = bf16_f32(d["a"]).reshape(B, T, 32)
    for r in range(B):
        rp = d["replay_idx"][r]
        H = d["h0"][si[r]].astype(np.float64)
        for t in range(T):
            p = _phys(d, r, t)
            dd = bf16_f32(res["d_ring"][rp, :, p]).astype(np.float64) + bf16_f32(res["dlo_ring"][rp, :, p])
            kk = bf16_f32(res["k_ring"][rp, :, p]).astype(np.float64) + bf16_f32(res["klo_ring"][rp, :, p])
            g = res["g_ring"][rp, :, p].astype(np.float64)
            xg = a[r, t].astype(np.float64) + d["dt_bias"]
            # the reference's softplus is fp32 log(1 + e^x): 1 + e^x is rounded to fp32 first (for x << 0
            # that rounding is most of the error), the rest is float64 here
            onep = (1.0 + np.exp(xg)).astype(np.float32).astype(np.float64)
            gref = -np.exp(d["A_log"].astype(np.float64)) * np.where(xg <= 20, np.log(onep), xg)
            assert np.allclose(g, gref, rtol=2e-5, atol=1e-9), "g ring entries are the gates"
            H = np.exp(g)[:, None, None] * H + dd[:, :, None] * np.repeat(kk, 2, axis=0)[:, None, :]
            assert_f32_close(H.reshape(32, -1), snaps[r, t].reshape(32, -1), 1e-4, f"rebuilt state r={r} t={t}")


def _ref64(O, d, B, T):
    """float64 restatement from the ring's history, matrix form of the delta rule."""
    from test_oracle_gdn import _front
    si = d["state_idx"]
    f = dict(d, conv_state=d["conv_state"][si])
    conv, _ = _front(O, f, B, T)
    out = np.zeros((B * T, 4096))
    dnew = np.zeros((B, T, 32, 128))
    nw = bf16_f32(d["norm_w"]).astype(np.float64)
    z = bf16_f32(d["z"]).astype(np.float64)
    a = bf16_f32(d["a"])
    b = bf16_f32(d["b"])
    for r in range(B):
        rp = d["replay_idx"][r]
        n = int(np.clip(d["write_pos"][rp], 0, 16))
        for hv in range(32):
            hk = hv // 2
            phys = [_phys(d, r, c) for c in range(n)]
            g = d["g_ring"][rp, hv, phys].astype(np.float64)
            S = np.exp(g.sum()) * d["h0"][si[r], hv].astype(np.float64)
            for c in range(n):
                dec = np.exp(g[c + 1:].sum())
                S += dec * np.outer(bf16_f32(d["d_ring"][rp, hv, phys[c]]), bf16_f32(d["k_ring"][rp, hk, phys[c]]))
            for t in range(T):
                row = r * T + t
                q = conv[r, t, hk * 128:(hk + 1) * 128].astype(np.float64)
                k = conv[r, t, 2048 + hk * 128:2048 + (hk + 1) * 128].astype(np.float64)
                v = conv[r, t, 4096 + hv * 128:4096 + (hv + 1) * 128].astype(np.float64)
                q = q / np.sqrt(np.sum(q * q) + 1e-6) * d["scale"]
                k = k / np.sqrt(np.sum(k * k) + 1e-6)
                xg = float(a[row, hv]) + float(d["dt_bias"][hv])
                eg = np.exp(-np.exp(float(d["A_log"][hv])) * (np.log1p(np.exp(xg)) if xg <= 20 else xg))
                beta = 1.0 / (1.0 + np.exp(-float(b[row, hv])))
                dnew[r, t, hv] = beta * (v - eg * (S @ k))
                S = eg * S @ (np.eye(128) - beta * np.outer(k, k)) + beta * np.outer(v, k)
                o = bf16_f32(O.f32_to_bf16((S @ q).astype(np.float32))).astype(np.float64)
                rstd = 1.0 / np.sqrt(np.mean(o * o) + 1e-6)
                zz = z[row, hv * 128:(hv + 1) * 128]
                out[row, hv * 128:(hv + 1) * 128] = o * rstd * nw * (zz / (1.0 + np.exp(-zz)))
    return out, dnew


@pytest.mark.parametrize("T,wp", [(4, 7), (5, 11), (1, 16), (3, 3)])
def test_ring_history_against_float64(oracle_mod, T, wp):
    O = oracle_mod
    B = 2
    d = _inputs(B, T, seed=20 + T, wp=wp)
    res = _ring(O, d, B, T)
    rout, dnew = _ref64(O, d, B, T)
    assert_bf16_close(res["out"], O.f32_to_bf16(rout.astype(np.float32)), 1e-2, "ring verify out")
    n = min(wp, 16)
    for r in range(B):
        rp = d["replay_idx"][r]
        for t in range(T):
            p = _phys(d, r, n + t)
            got = bf16_f32(res["d_ring"][rp, :, p]).astype(np.float64) + bf16_f32(res["dlo_ring"][rp, :, p])
            if n + t < 16:
                assert_f32_close(got, dnew[r, t], 1e-4, f"d entry r={r} t={t}")
            else:  # a full ring takes no appends
                assert np.array_equal(res["d_ring"][rp, :, p], d["d_ring"][rp, :, p])
    # the double-precision variant of the oracle agrees with its fp32 path
    res64 = _ring(O, d, B, T, use_f64=True)
    assert_bf16_close(res["out"], res64["out"], 1e-2, "f32 vs f64")


def test_two_windows_equal_one_long_window(oracle_mod):
    """Window 1 appends T entries to an empty ring; with all of them accepted (write_pos = T) window 2
    reads them back.  Its outputs must equal the snapshot verify over 2T positions at positions
    T .. 2T-1, to the bf16 precision of the entries' high parts."""
    O = oracle_mod
    B, T = 2, 4
    d = _inputs(B, 2 * T, seed=41, wp=0)
    mix = d["mixed"].reshape(B, 2 * T, -1)
    zz = d["z"].reshape(B, 2 * T, -1)
    aa = d["a"].reshape(B, 2 * T, -1)
    bb = d["b"].reshape(B, 2 * T, -1)

    def half(x, h):
        return np.ascontiguousarray(x[:, h * T:(h + 1) * T].reshape(B * T, -1))

    qsl = np.arange(0, (B + 1) * T, T, dtype=np.int32)
    win = np.zeros((d["window"].shape[0], 8192, T + 2), np.uint16)
    first = _ring(O, d, B, T, mixed=half(mix, 0), z=half(zz, 0), a=half(aa, 0), b=half(bb, 0), qsl=qsl, window=win)
    wpos = d["write_pos"].copy()
    wpos[d["replay_idx"]] = T
    second = _ring(O, dict(d, **{k: first[k] for k in ("conv_state", "d_ring", "dlo_ring", "k_ring", "klo_ring",
                                                       "g_ring")}), B, T,
                   mixed=half(mix, 1), z=half(zz, 1), a=half(aa, 1), b=half(bb, 1), qsl=qsl, window=win,
                   write_pos=wpos)
    out, _, _ = _snap(O, d, B, 2 * T)
    ref = out.reshape(B, 2 * T, -1)[:, T:].reshape(B * T, -1)
    assert_bf16_close(second["out"], np.ascontiguousarray(ref), 1e-2, "second window vs one long window")
    assert np.array_equal(first["out"], np.ascontiguousarray(out.reshape(B, 2 * T, -1)[:, :T].reshape(B * T, -1)))


def test_cache_base_rotation_and_padding(oracle_mod):
    O = oracle_mod
    B, T = 3, 4
    d = _inputs(B, T, seed=9, wp=9, padded=(1,))
    res = _ring(O, d, B, T)
    assert not np.any(res["out"][T:2 * T]), "a padded request's rows are zero"
    # rotate every ring's physical slots by 5 and move cache_base with them
    rot = {k: np.ascontiguousarray(np.roll(d[k], 5, axis=2)) for k in ("d_ring", "dlo_ring", "k_ring", "klo_ring",
                                                                        "g_ring")}
    res2 = _ring(O, dict(d, **rot), B, T, cache_base=((d["cache_base"] + 5) & 15).astype(np.int32))
    assert np.array_equal(res["out"], res2["out"]), "the ring's physical rotation must not matter"
    for k in rot:
        assert np.array_equal(np.roll(res[k], 5, axis=2), res2[k]), k
    # the padded request touched nothing
    r = 1
    rp = d["replay_idx"][r]
    for k in ("d_ring", "dlo_ring", "k_ring", "klo_ring", "g_ring"):
        assert np.array_equal(res[k][rp], d[k][rp]), k
    assert np.array_equal(res["window"][d["win_idx"][r]], d["window"][d["win_idx"][r]])
