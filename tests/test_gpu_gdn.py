"""GPU parity of the GDN verify step (libq36 through the C-ABI) against the CPU oracle.

Bar: conv state bit-exact; per-position fp32 states within 1e-4 relative (per (seq, pos, head)
matrix, against its largest entry); bf16 outputs within 1e-2 relative (per-row norm).
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, assert_f32_close, bits16, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gdn():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import gdn_fused
    return gdn_fused


def _run(gdn, O, dev, B, T, seed):
    from bundles_amd import synth
    print(f"gdn B={B} T={T} seed={seed}", flush=True)
    d = synth.gdn_inputs(B, T, dev, seed=seed)
    out, snaps, cs_out = gdn.gdn_verify_fused(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"],
                                              d["A_log"], d["dt_bias"], d["S0"], d["norm_w"], 1e-6, T=T)
    torch.cuda.synchronize()
    r_out, r_snaps, r_cs = O.gdn_verify(B, T, bits16(d["mixed"]), bits16(d["z"]), bits16(d["a"]), bits16(d["b"]),
                                        bits16(d["conv_state"]), bits16(d["conv_w"]), np_(d["A_log"]),
                                        np_(d["dt_bias"]), np_(d["S0"]), bits16(d["norm_w"]), 1e-6)
    return out, snaps, cs_out, r_out, r_snaps, r_cs, d


@pytest.mark.parametrize("B,T", [(1, 1), (2, 5), (3, 8), (4, 2)])
def test_gdn_small(gdn, oracle_mod, dev, B, T):
    out, snaps, cs_out, r_out, r_snaps, r_cs, _ = _run(gdn, oracle_mod, dev, B, T, seed=10 * B + T)
    assert np.array_equal(bits16(cs_out), r_cs), "rolled conv state differs"
    ws = assert_f32_close(np_(snaps).reshape(B * T * 32, -1), r_snaps.reshape(B * T * 32, -1), 1e-4, "state")
    wo, ao, eo = assert_bf16_close(bits16(out), r_out, 1e-2, "gdn out")
    print(f"state worst rel {ws:.2e}; out row err {wo:.2e} elem {ao:.2e} exact {eo:.4f}", flush=True)


def test_gdn_config3_full(gdn, oracle_mod, dev):
    """Config 3: 32 sequences x (1 + 4) positions, 16 QK heads x 128, 32 V heads x 128."""
    B, T = 32, 5
    out, snaps, cs_out, r_out, r_snaps, r_cs, _ = _run(gdn, oracle_mod, dev, B, T, seed=0)
    assert np.array_equal(bits16(cs_out), r_cs)
    ws = assert_f32_close(np_(snaps).reshape(B * T * 32, -1), r_snaps.reshape(B * T * 32, -1), 1e-4, "state")
    wo, ao, eo = assert_bf16_close(bits16(out), r_out, 1e-2, "gdn out")
    print(f"config 3: state worst rel {ws:.2e}; out row err {wo:.2e} exact {eo:.4f}", flush=True)


def test_gdn_rejects_aliasing(gdn, dev):
    from bundles_amd import synth
    d = synth.gdn_inputs(1, 2, dev, seed=1)
    with pytest.raises(RuntimeError, match="alias"):
        gdn.gdn_verify_fused(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"], d["A_log"],
                             d["dt_bias"], d["S0"], d["norm_w"], T=2, conv_state_out=d["conv_state"])
