"""GPU parity of config 5's hybrid node with the GDN verify in the served ReplaySSM ring form
(q36_gdn_verify_ring) against the CPU oracle, stage by stage on the GPU's own inputs: the add-norms
and the lm_head ids bit-exact; each GDN layer's output within 1e-2 relative per row, its rolled conv
state and window records bit-exact, its appended ring entries within 1e-4 (d) and 4e-5 (k) of the
oracle's ring verify on the same pools; the other stages as in the snapshot form's tests."""
import numpy as np
import pytest
import torch

import test_gpu_hybrid as H
from helpers import assert_bf16_close, assert_f32_close, bf16_f32, bits16, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def run(dev):
    from bundles_amd import _lib, synth
    _lib.lib()
    from bundles_amd.qwen36_layer import hybrid
    w = hybrid.make_weights(dev, seed=3, E=H.E, V=H.V)
    st = hybrid.make_state(H.B, H.T, H.CTX, dev, seed=4, gdn_form="ring", ring_wp=6)
    ws = hybrid.HybridWorkspace(H.B, H.T, H.E, dev, snapshots=False)
    x = synth.randn((H.B * H.T, 2048), synth.gen(dev, 5), dev)
    kc0, vc0 = st.k_cache.clone(), st.v_cache.clone()
    trace = {}
    ids = hybrid.forward(x, w, st, ws, trace=trace)
    torch.cuda.synchronize()
    return dict(hybrid=hybrid, w=w, st=st, trace=trace, ids=ids, kc0=kc0, vc0=vc0)


def test_add_norms_are_bit_exact(run, oracle_mod):
    H.test_add_norms_are_bit_exact(run, oracle_mod)


def test_gdn_ring_layers(run, oracle_mod):
    O, tr, w, st = oracle_mod, run["trace"], run["w"], run["st"]
    gi = 0
    for i, L in enumerate(w.layers):
        if L.kind != "gdn":
            continue
        g, R = L.mixer, st.ring[gi]
        print(f"GDN ring layer {i}", flush=True)
        ref = O.gdn_verify_ring(
            H.B, H.T, bits16(tr[f"L{i}.mixed"]), bits16(tr[f"L{i}.z"]), bits16(tr[f"L{i}.a"]), bits16(tr[f"L{i}.b"]),
            bits16(tr[f"L{i}.conv_state_in"]), bits16(g.conv_w), np.zeros(R["window"].shape, np.uint16),
            np_(g.A_log), np_(g.dt_bias), np_(st.S[gi]), *(bits16(tr[f"L{i}.ring_{k}_in"]) for k in ("d", "dlo", "k", "klo")),
            np_(tr[f"L{i}.ring_g_in"]), np_(R["qsl"]), np_(R["idx"]), np_(R["idx"]), np_(R["idx"]), np_(R["wp"]),
            np_(R["cb"]), bits16(g.norm_w), w.eps, 128 ** -0.5)
        assert_bf16_close(bits16(tr[f"L{i}.gout"]), ref["out"], 1e-2, f"L{i} gdn ring")
        assert np.array_equal(bits16(st.conv_state[gi]), ref["conv_state"]), f"L{i} conv state"
        assert np.array_equal(bits16(R["window"]), ref["window"]), f"L{i} window records"
        got_d = bf16_f32(bits16(R["d"])).astype(np.float64) + bf16_f32(bits16(R["dlo"]))
        want_d = bf16_f32(ref["d_ring"]).astype(np.float64) + bf16_f32(ref["dlo_ring"])
        assert_f32_close(got_d.reshape(-1, 128), want_d.reshape(-1, 128), 1e-4, f"L{i} d ring")
        got_k = bf16_f32(bits16(R["k"])).astype(np.float64) + bf16_f32(bits16(R["klo"]))
        want_k = bf16_f32(ref["k_ring"]).astype(np.float64) + bf16_f32(ref["klo_ring"])
        assert_f32_close(got_k.reshape(-1, 128), want_k.reshape(-1, 128), 4e-5, f"L{i} k ring")
        gi += 1


def test_attention_layer(run, oracle_mod):
    H.test_attention_layer(run, oracle_mod)


def test_moe_blocks(run, oracle_mod):
    H.test_moe_blocks(run, oracle_mod)


def test_lmhead_ids_bit_exact(run, oracle_mod):
    H.test_lmhead_ids_bit_exact(run, oracle_mod)
