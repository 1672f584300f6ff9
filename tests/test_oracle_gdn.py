"""Pins of the oracle's GDN verify step (CPU).

The recurrence is checked against its matrix form S_t = e^{g_t} S_{t-1} (I - beta_t k_t k_t^T) +
beta_t v_t k_t^T in float64 (a different algebra from the oracle's row-wise delta update), the
front (conv taps with bf16 products, SiLU, L2 norms, gates) against a numpy float32 restatement,
and the delta-rule invariant S_t k_t = v_t at beta = 1, g = 0.
"""
import numpy as np
import pytest

from helpers import assert_bf16_close, assert_f32_close


def _inputs(B, T, seed):
    import torch
    from bundles_amd import synth
    d = synth.gdn_inputs(B, T, "cpu", seed=seed)
    out = {}
    for k, v in d.items():
        if isinstance(v, int):
            out[k] = v
        elif v.dtype == torch.bfloat16:
            out[k] = v.contiguous().view(torch.int16).numpy().view(np.uint16)
        else:
            out[k] = v.contiguous().numpy()
    return out


def _run(O, d, B, T, use_f64=False):
    return O.gdn_verify(B, T, d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"], d["A_log"],
                        d["dt_bias"], d["S0"], d["norm_w"], 1e-6, use_f64=use_f64)


def _front(O, d, B, T):
    """conv + SiLU (bf16 tap products, fp32 sum oldest first) -> [B, T, 8192] float32."""
    bf = lambda x: O.bf16_to_f32(O.f32_to_bf16(np.asarray(x, np.float32)))
    ex = np.vectorize(lambda v: O.expf(float(v)), otypes=[np.float32])
    win = np.concatenate([O.bf16_to_f32(d["conv_state"]), O.bf16_to_f32(d["mixed"]).reshape(B, T, 8192)
                          .transpose(0, 2, 1)], axis=2)  # [B, 8192, 3 + T]
    cw = O.bf16_to_f32(d["conv_w"])
    out = np.empty((B, T, 8192), np.float32)
    for t in range(T):
        acc = bf(win[:, :, t] * cw[:, 0])
        for i in range(1, 4):
            acc = (acc + bf(win[:, :, t + i] * cw[:, i])).astype(np.float32)
        out[:, t] = bf(acc / (np.float32(1) + ex(-acc)))
    return out, win[:, :, T:]


def _ref64(O, d, B, T):
    conv, new_state = _front(O, d, B, T)
    S = d["S0"].astype(np.float64).copy()
    snaps = np.empty((B, T, 32, 128, 128))
    out = np.empty((B * T, 4096))
    nw = O.bf16_to_f32(d["norm_w"]).astype(np.float64)
    z = O.bf16_to_f32(d["z"]).astype(np.float64)
    a = O.bf16_to_f32(d["a"])
    b = O.bf16_to_f32(d["b"])
    for bq in range(B):
        for hv in range(32):
            hk = hv // 2
            for t in range(T):
                r = bq * T + t
                q = conv[bq, t, hk * 128:(hk + 1) * 128].astype(np.float64)
                k = conv[bq, t, 2048 + hk * 128:2048 + (hk + 1) * 128].astype(np.float64)
                v = conv[bq, t, 4096 + hv * 128:4096 + (hv + 1) * 128].astype(np.float64)
                q = q / np.sqrt(np.sum(q * q) + 1e-6) / np.sqrt(128.0)
                k = k / np.sqrt(np.sum(k * k) + 1e-6)
                xg = float(a[r, hv]) + float(d["dt_bias"][hv])
                sp = np.log1p(np.exp(xg)) if xg <= 20 else xg
                eg = np.exp(-np.exp(float(d["A_log"][hv])) * sp)
                beta = 1.0 / (1.0 + np.exp(-float(b[r, hv])))
                S[bq, hv] = eg * S[bq, hv] @ (np.eye(128) - beta * np.outer(k, k)) + beta * np.outer(v, k)
                snaps[bq, t, hv] = S[bq, hv]
                o = O.bf16_to_f32(O.f32_to_bf16((S[bq, hv] @ q).astype(np.float32))).astype(np.float64)
                rstd = 1.0 / np.sqrt(np.mean(o * o) + 1e-6)
                zz = z[r, hv * 128:(hv + 1) * 128]
                out[r, hv * 128:(hv + 1) * 128] = o * rstd * nw * (zz / (1.0 + np.exp(-zz)))
    return out, snaps, new_state


@pytest.mark.parametrize("B,T", [(1, 1), (2, 5)])
def test_gdn_against_matrix_form(oracle_mod, B, T):
    O = oracle_mod
    d = _inputs(B, T, seed=3 + T)
    out, snaps, cs = _run(O, d, B, T)
    rout, rsnaps, rstate = _ref64(O, d, B, T)
    assert np.array_equal(O.bf16_to_f32(cs), rstate), "rolled conv state must be the last three inputs"
    assert_f32_close(snaps.reshape(B * T * 32, -1), rsnaps.reshape(B * T * 32, -1), 1e-4, "state")
    assert_bf16_close(out, O.f32_to_bf16(rout.astype(np.float32)), 1e-2, "gdn out")
    # the float64 variant of the oracle agrees with its fp32 path
    _, snaps64, _ = _run(O, d, B, T, use_f64=True)
    assert_f32_close(snaps.reshape(B * T * 32, -1), snaps64.reshape(B * T * 32, -1), 1e-4, "f32 vs f64")


def test_delta_rule_writes_v_at_k(oracle_mod):
    """beta = 1 and g = 0 (A_log very negative): after position t, S_t k_t = v_t for unit k_t."""
    O = oracle_mod
    B, T = 1, 3
    d = _inputs(B, T, seed=11)
    d["b"] = O.f32_to_bf16(np.full(d["b"].shape, 60.0, np.float32))   # sigmoid -> 1
    d["A_log"] = np.full(32, -60.0, np.float32)                        # g = -exp(-60) * sp ~ 0
    _, snaps, _ = _run(O, d, B, T)
    conv, _ = _front(O, d, B, T)
    for t in range(T):
        for hv in (0, 5, 31):
            hk = hv // 2
            k = conv[0, t, 2048 + hk * 128:2048 + (hk + 1) * 128].astype(np.float64)
            k = k / np.sqrt(np.sum(k * k) + 1e-6)
            v = conv[0, t, 4096 + hv * 128:4096 + (hv + 1) * 128].astype(np.float64)
            sk = snaps[0, t, hv].astype(np.float64) @ k
            assert np.allclose(sk, v, atol=2e-4 * (1 + np.abs(v).max())), (t, hv)
