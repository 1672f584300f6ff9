"""Config 5's hybrid node at its full size on the GPU, checked stage by stage against the CPU oracle.

The workload is the bench's: 64 requests x 4 verify tokens (256 rows a step) over 4096 cached e4m3 keys
per request, 512 experts top-10 in every MoE block, the GDN layers in the served ReplaySSM ring form, and
the int8 lm_head over the 151936-token vocabulary.  Every stage runs on all 256 rows; the oracle checks
each stage on the inputs the GPU gave it (teacher forcing) for a 16-row subset (requests 0..3), to that
stage's bar: add-norms (all rows) and lm_head ids bit-exact; fp8 projections, GDN, attention and MoE
within 1e-2 relative per row; the GDN conv state and window records of the subset bit-exact, its ring
appends within 1e-4 (d) and 4e-5 (k)."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, assert_f32_close, bf16_f32, bits16, bits8, np_

pytestmark = pytest.mark.gpu

B, T, CTX, E, V = 64, 4, 4096, 512, 151936
NS = 4            # requests in the checked subset
ROWS = NS * T     # their rows: 0 .. 15


@pytest.fixture(scope="module")
def run(dev):
    from bundles_amd import _lib, synth
    _lib.lib()
    from bundles_amd.qwen36_layer import hybrid
    print(f"hybrid full size: B={B} T={T} ctx={CTX} E={E} V={V}", flush=True)
    w = hybrid.make_weights(dev, seed=13, E=E, V=V)
    st = hybrid.make_state(B, T, CTX, dev, seed=14, gdn_form="ring", ring_wp=7)
    ws = hybrid.HybridWorkspace(B, T, E, dev, snapshots=False)
    x = synth.randn((B * T, 2048), synth.gen(dev, 15), dev)
    kc0, vc0 = st.k_cache.clone(), st.v_cache.clone()
    trace = {}
    ids = hybrid.forward(x, w, st, ws, trace=trace)
    torch.cuda.synchronize()
    return dict(w=w, st=st, trace=trace, ids=ids, kc0=kc0, vc0=vc0)


def _frag_rm(t):
    from bundles_amd.qwen36_layer import moe
    return moe.unpack_frag8_np(np_(t))


def _sub(t):
    return bits16(t[:ROWS])


def test_add_norms_are_bit_exact(run, oracle_mod):
    O, tr, w = oracle_mod, run["trace"], run["w"]
    h0, _ = O.add_rmsnorm(None, bits16(tr["x"]), bits16(w.layers[0].input_norm_w), w.eps)
    assert np.array_equal(h0, bits16(tr["h0"]))
    for i, L in enumerate(w.layers):
        post, res_mid = O.add_rmsnorm(bits16(tr[f"L{i}.o"]), bits16(tr[f"L{i}.res_in"]), bits16(L.post_norm_w), w.eps)
        assert np.array_equal(post, bits16(tr[f"L{i}.post"])), f"layer {i} post norm"
        # the residual after the mixer lives only inside the MoE call (its route writes it, its combine
        # adds to it in place): checked through the residual after the MoE, formed from the oracle's
        # res_mid below, and directly by test_moe_input_add_norm
        nxt = w.layers[i + 1].input_norm_w if i + 1 < len(w.layers) else w.final_norm_w
        hn, res_out = O.add_rmsnorm(bits16(tr[f"L{i}.moe"]), res_mid, bits16(nxt), w.eps)
        want = tr[f"L{i + 1}.in"] if i + 1 < len(w.layers) else tr["final"]
        assert np.array_equal(hn, bits16(want)), f"layer {i} next norm"
        assert np.array_equal(res_out, bits16(tr[f"L{i}.res_out"])), f"layer {i} residual after the MoE"


def test_gdn_ring_layers(run, oracle_mod):
    O, tr, w, st = oracle_mod, run["trace"], run["w"], run["st"]
    gi = 0
    for i, L in enumerate(w.layers):
        if L.kind != "gdn":
            continue
        g, R = L.mixer, st.ring[gi]
        print(f"GDN ring layer {i} (requests 0..{NS - 1})", flush=True)
        ref = O.fp8_linear(_sub(tr[f"L{i}.in"]), np_(g.in_proj.q), np_(g.in_proj.s))
        got = np.concatenate([_sub(tr[f"L{i}.{k}"]) for k in ("mixed", "z", "b", "a")], axis=1)
        assert_bf16_close(got, ref[:, :got.shape[1]], 1e-2, f"L{i} in_proj")
        ref = O.gdn_verify_ring(
            NS, T, _sub(tr[f"L{i}.mixed"]), _sub(tr[f"L{i}.z"]), _sub(tr[f"L{i}.a"]), _sub(tr[f"L{i}.b"]),
            bits16(tr[f"L{i}.conv_state_in"]), bits16(g.conv_w), np.zeros(R["window"].shape, np.uint16),
            np_(g.A_log), np_(g.dt_bias), np_(st.S[gi]),
            *(bits16(tr[f"L{i}.ring_{k}_in"]) for k in ("d", "dlo", "k", "klo")), np_(tr[f"L{i}.ring_g_in"]),
            np_(R["qsl"])[:NS + 1], np_(R["idx"])[:NS], np_(R["idx"])[:NS], np_(R["idx"])[:NS], np_(R["wp"]),
            np_(R["cb"]), bits16(g.norm_w), w.eps, 128 ** -0.5)
        assert_bf16_close(_sub(tr[f"L{i}.gout"]), ref["out"], 1e-2, f"L{i} gdn ring")
        assert np.array_equal(bits16(st.conv_state[gi])[:NS], ref["conv_state"][:NS]), f"L{i} conv state"
        assert np.array_equal(bits16(R["window"])[:NS], ref["window"][:NS]), f"L{i} window records"
        got_d = bf16_f32(bits16(R["d"])[:NS]).astype(np.float64) + bf16_f32(bits16(R["dlo"])[:NS])
        want_d = bf16_f32(ref["d_ring"][:NS]).astype(np.float64) + bf16_f32(ref["dlo_ring"][:NS])
        assert_f32_close(got_d.reshape(-1, 128), want_d.reshape(-1, 128), 1e-4, f"L{i} d ring")
        got_k = bf16_f32(bits16(R["k"])[:NS]).astype(np.float64) + bf16_f32(bits16(R["klo"])[:NS])
        want_k = bf16_f32(ref["k_ring"][:NS]).astype(np.float64) + bf16_f32(ref["klo_ring"][:NS])
        assert_f32_close(got_k.reshape(-1, 128), want_k.reshape(-1, 128), 4e-5, f"L{i} k ring")
        ref = O.fp8_linear(_sub(tr[f"L{i}.gout"]), np_(g.out_proj.q), np_(g.out_proj.s))
        assert_bf16_close(_sub(tr[f"L{i}.o"]), ref, 1e-2, f"L{i} out_proj")
        gi += 1


def test_attention_layer(run, oracle_mod):
    O, tr, w, st = oracle_mod, run["trace"], run["w"], run["st"]
    i = [k for k, L in enumerate(w.layers) if L.kind == "attn"][0]
    a = w.layers[i].mixer
    print(f"attention layer {i}: {CTX} keys, requests 0..{NS - 1}", flush=True)
    q, s = np_(a.w.wqkv).astype(np.uint8), np_(a.w.sqkv)
    r = O.attn_proj(_sub(tr[f"L{i}.in"]), q[:8192], s[:64], q[8192:8704], s[64:68], q[8704:], s[68:72],
                    bits16(a.q_norm_w), bits16(a.k_norm_w), w.eps, np_(st.cos_sin), np_(st.positions)[:ROWS])
    for k in ("q", "gate"):
        assert_bf16_close(_sub(tr[f"L{i}.{k}"]).reshape(ROWS, -1), r[k].reshape(ROWS, -1), 1e-2, f"attn {k}")
    kc, vc = bits8(st.k_cache), bits8(st.v_cache)
    loc = np_(st.out_loc)
    assert np.array_equal(kc[loc], bits8(tr[f"L{i}.k8"])) and np.array_equal(vc[loc], bits8(tr[f"L{i}.v8"]))
    keep = np.ones(kc.shape[0], bool)
    keep[loc] = False
    assert np.array_equal(kc[keep], bits8(run["kc0"])[keep]) and np.array_equal(vc[keep], bits8(run["vc0"])[keep])
    ref = O.attn_decode(_sub(tr[f"L{i}.q"]), kc, vc, np_(st.page_table)[:NS], np_(st.seqlens)[:NS], T, 1.0 / 16.0)
    assert_bf16_close(_sub(tr[f"L{i}.attn"]).reshape(-1, 256), ref.reshape(-1, 256), 1e-2, "attn core")
    ref = O.attn_oproj(_sub(tr[f"L{i}.attn"]), _sub(tr[f"L{i}.gate"]), np_(a.w.wo).astype(np.uint8), np_(a.w.so))
    assert_bf16_close(_sub(tr[f"L{i}.o"]), ref, 1e-2, "attn o_proj")


def test_moe_blocks(run, oracle_mod):
    O, tr, w = oracle_mod, run["trace"], run["w"]
    for i, L in enumerate(w.layers):
        ew = L.experts
        r = O.moe(1, _sub(tr[f"L{i}.post"]), bits16(L.router_w), _frag_rm(ew.w13), np_(ew.s13), _frag_rm(ew.w2),
                  np_(ew.s2), _frag_rm(ew.sw13), np_(ew.ss13), _frag_rm(ew.sw2), np_(ew.ss2), bits16(L.gate_w), 10,
                  bias=np_(L.router_bias))
        wr, ar, er = assert_bf16_close(_sub(tr[f"L{i}.moe"]), r["out"], 1e-2, f"L{i} moe")
        print(f"layer {i} MoE (512 experts) row error {wr:.2e}, elementwise {ar:.2e}, exact {er:.3f}", flush=True)


def test_lmhead_ids_bit_exact(run, oracle_mod):
    """The node's arithmetic for the step's 256 rows is the two-term W8A8 form: ids bit-exact."""
    from bundles_amd.qwen36_layer import hybrid
    O, tr, w = oracle_mod, run["trace"], run["w"]
    mode = hybrid.lm_mode(run["ids"].shape[0], w.lm_q.shape[0])
    assert mode == "two_term"
    ids, _ = O.lmhead(_sub(tr["final"]), None, w.eps, np_(w.lm_q), np_(w.lm_s), two_term=True)
    assert np.array_equal(ids, np_(run["ids"])[:ROWS])
