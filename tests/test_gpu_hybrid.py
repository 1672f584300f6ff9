"""GPU parity of config 5's hybrid node (three GDN layers + one attention layer, each + fp8 MoE, the
add-norms, final norm, int8 lm_head + argmax) against the CPU oracle, stage by stage.

Every stage is checked on the inputs the GPU gave it (teacher forcing), to that stage's own bar:
the add-norms and the lm_head ids bit-exact, the fp8 projections / GDN / attention / MoE within
1e-2 relative per row.  The end-to-end hidden state is also compared with the oracle run free from
the embedded tokens alone (routing flips make the free-running pipelines drift: reported, bounded
loosely)."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bf16_f32, bits16, bits8, np_

pytestmark = pytest.mark.gpu

B, T, CTX, E, V = 2, 4, 40, 64, 4096


@pytest.fixture(scope="module")
def run(dev):
    from bundles_amd import _lib, synth
    _lib.lib()
    from bundles_amd.qwen36_layer import hybrid
    w = hybrid.make_weights(dev, seed=3, E=E, V=V)
    st = hybrid.make_state(B, T, CTX, dev, seed=4)
    ws = hybrid.HybridWorkspace(B, T, E, dev)
    x = synth.randn((B * T, 2048), synth.gen(dev, 5), dev)
    kc0, vc0 = st.k_cache.clone(), st.v_cache.clone()
    trace = {}
    ids = hybrid.forward(x, w, st, ws, trace=trace)
    torch.cuda.synchronize()
    return dict(hybrid=hybrid, w=w, st=st, trace=trace, ids=ids, kc0=kc0, vc0=vc0)


def _frag_rm(t):
    from bundles_amd.qwen36_layer import moe
    return moe.unpack_frag8_np(np_(t))


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


def test_gdn_layers(run, oracle_mod):
    O, tr, w, st = oracle_mod, run["trace"], run["w"], run["st"]
    gi = 0
    for i, L in enumerate(w.layers):
        if L.kind != "gdn":
            continue
        g = L.mixer
        print(f"GDN layer {i}", flush=True)
        ref = O.fp8_linear(bits16(tr[f"L{i}.in"]), np_(g.in_proj.q), np_(g.in_proj.s))
        got = np.concatenate([bits16(tr[f"L{i}.{k}"]) for k in ("mixed", "z", "b", "a")], axis=1)
        assert_bf16_close(got, ref[:, :got.shape[1]], 1e-2, f"L{i} in_proj")
        out, _, _ = O.gdn_verify(B, T, bits16(tr[f"L{i}.mixed"]), bits16(tr[f"L{i}.z"]), bits16(tr[f"L{i}.a"]),
                                 bits16(tr[f"L{i}.b"]), bits16(st.conv_state[gi]), bits16(g.conv_w), np_(g.A_log),
                                 np_(g.dt_bias), np_(st.S[gi]), bits16(g.norm_w), w.eps)
        assert_bf16_close(bits16(tr[f"L{i}.gout"]), out, 1e-2, f"L{i} gdn")
        ref = O.fp8_linear(bits16(tr[f"L{i}.gout"]), np_(g.out_proj.q), np_(g.out_proj.s))
        assert_bf16_close(bits16(tr[f"L{i}.o"]), ref, 1e-2, f"L{i} out_proj")
        gi += 1


def test_attention_layer(run, oracle_mod):
    O, tr, w, st = oracle_mod, run["trace"], run["w"], run["st"]
    i = [k for k, L in enumerate(w.layers) if L.kind == "attn"][0]
    a = w.layers[i].mixer
    q, s = np_(a.w.wqkv).astype(np.uint8), np_(a.w.sqkv)
    r = O.attn_proj(bits16(tr[f"L{i}.in"]), q[:8192], s[:64], q[8192:8704], s[64:68], q[8704:], s[68:72],
                    bits16(a.q_norm_w), bits16(a.k_norm_w), w.eps, np_(st.cos_sin), np_(st.positions))
    for k in ("q", "gate"):
        assert_bf16_close(bits16(tr[f"L{i}.{k}"]).reshape(B * T, -1), r[k].reshape(B * T, -1), 1e-2, f"attn {k}")
    # the new rows landed in the pool at out_loc, the rest of the pool is unchanged
    kc, vc = bits8(st.k_cache), bits8(st.v_cache)
    loc = np_(st.out_loc)
    assert np.array_equal(kc[loc], bits8(tr[f"L{i}.k8"])) and np.array_equal(vc[loc], bits8(tr[f"L{i}.v8"]))
    keep = np.ones(kc.shape[0], bool)
    keep[loc] = False
    assert np.array_equal(kc[keep], bits8(run["kc0"])[keep]) and np.array_equal(vc[keep], bits8(run["vc0"])[keep])
    ref = O.attn_decode(bits16(tr[f"L{i}.q"]), kc, vc, np_(st.page_table), np_(st.seqlens), T, 1.0 / 16.0)
    assert_bf16_close(bits16(tr[f"L{i}.attn"]).reshape(-1, 256), ref.reshape(-1, 256), 1e-2, "attn core")
    ref = O.attn_oproj(bits16(tr[f"L{i}.attn"]), bits16(tr[f"L{i}.gate"]), np_(a.w.wo).astype(np.uint8),
                       np_(a.w.so))
    assert_bf16_close(bits16(tr[f"L{i}.o"]), ref, 1e-2, "attn o_proj")


def test_moe_blocks(run, oracle_mod):
    O, tr, w = oracle_mod, run["trace"], run["w"]
    for i, L in enumerate(w.layers):
        ew = L.experts
        r = O.moe(1, bits16(tr[f"L{i}.post"]), bits16(L.router_w), _frag_rm(ew.w13), np_(ew.s13), _frag_rm(ew.w2),
                  np_(ew.s2), _frag_rm(ew.sw13), np_(ew.ss13), _frag_rm(ew.sw2), np_(ew.ss2), bits16(L.gate_w), 10,
                  bias=np_(L.router_bias))
        wr, _, _ = assert_bf16_close(bits16(tr[f"L{i}.moe"]), r["out"], 1e-2, f"L{i} moe")
        print(f"layer {i} MoE row error {wr:.2e}", flush=True)


def check_lmhead_ids(run, oracle_mod, final_bits, rows=None):
    """The node's lm_head arithmetic for the step's row count: W8A8 ids bit-exact (one or two terms);
    W8A16 (below 64 rows) ids pick a logit within one bf16 step of the oracle's row maximum."""
    from bundles_amd.qwen36_layer import hybrid
    O, w = oracle_mod, run["w"]
    got = np_(run["ids"]) if rows is None else np_(run["ids"])[rows]
    mode = hybrid.lm_mode(run["ids"].shape[0], w.lm_q.shape[0])
    ids, lg = O.lmhead(final_bits, None, w.eps, np_(w.lm_q), np_(w.lm_s), want_logits=True,
                       two_term=mode == "two_term", w8a16=mode == "w8a16")
    if mode != "w8a16":
        assert np.array_equal(ids, got), f"lm_head ({mode}) ids differ"
        return
    r = bf16_f32(lg)
    rmax = r.max(axis=1)
    picked = r[np.arange(r.shape[0]), got]
    assert np.all(rmax - picked <= np.abs(rmax) * 2 ** -7 + 1e-6), "a W8A16 id's logit is below the oracle maximum"


def test_lmhead_ids_bit_exact(run, oracle_mod):
    check_lmhead_ids(run, oracle_mod, bits16(run["trace"]["final"]))


def test_end_to_end_against_the_free_running_oracle(run, oracle_mod):
    """The oracle composed from the embedded tokens alone (no GPU intermediates).  Not a parity bar:
    a 1e-2 difference at a router input flips some of a row's top-10 picks among 64 near-tied
    logits, and the greedy argmax over random-weight logits is as fragile, so the two free-running
    pipelines drift apart by a few percent (measured 4.5e-2, 62 % equal ids at this seed).  The
    stage tests above are the parity claim; this one bounds the drift and reports it."""
    O, tr, w, st = oracle_mod, run["trace"], run["w"], run["st"]
    res = bits16(tr["x"])
    h, _ = O.add_rmsnorm(None, res, bits16(w.layers[0].input_norm_w), w.eps)
    kc, vc = bits8(run["kc0"]).copy(), bits8(run["vc0"]).copy()
    gi = 0
    for i, L in enumerate(w.layers):
        if L.kind == "gdn":
            g = L.mixer
            y = O.fp8_linear(h, np_(g.in_proj.q), np_(g.in_proj.s))
            mixed, z, bb, aa = y[:, :8192], y[:, 8192:12288], y[:, 12288:12320], y[:, 12320:12352]
            out, _, _ = O.gdn_verify(B, T, mixed, z, aa, bb, bits16(st.conv_state[gi]), bits16(g.conv_w),
                                     np_(g.A_log), np_(g.dt_bias), np_(st.S[gi]), bits16(g.norm_w), w.eps)
            o = O.fp8_linear(out, np_(g.out_proj.q), np_(g.out_proj.s))
            gi += 1
        else:
            a = L.mixer
            q, s = np_(a.w.wqkv).astype(np.uint8), np_(a.w.sqkv)
            r = O.attn_proj(h, q[:8192], s[:64], q[8192:8704], s[64:68], q[8704:], s[68:72], bits16(a.q_norm_w),
                            bits16(a.k_norm_w), w.eps, np_(st.cos_sin), np_(st.positions))
            loc = np_(st.out_loc)
            kc[loc], vc[loc] = r["k8"], r["v8"]
            at = O.attn_decode(r["q"], kc, vc, np_(st.page_table), np_(st.seqlens), T, 1.0 / 16.0)
            o = O.attn_oproj(at, r["gate"], np_(a.w.wo).astype(np.uint8), np_(a.w.so))
        h, res = O.add_rmsnorm(o, res, bits16(L.post_norm_w), w.eps)
        ew = L.experts
        m = O.moe(1, h, bits16(L.router_w), _frag_rm(ew.w13), np_(ew.s13), _frag_rm(ew.w2), np_(ew.s2),
                  _frag_rm(ew.sw13), np_(ew.ss13), _frag_rm(ew.sw2), np_(ew.ss2), bits16(L.gate_w), 10,
                  bias=np_(L.router_bias))["out"]
        nxt = w.layers[i + 1].input_norm_w if i + 1 < len(w.layers) else w.final_norm_w
        h, res = O.add_rmsnorm(m, res, bits16(nxt), w.eps)
    wr, ar, er = assert_bf16_close(bits16(tr["final"]), h, 0.25, "end to end")
    from bundles_amd.qwen36_layer import hybrid
    mode = hybrid.lm_mode(h.shape[0], w.lm_q.shape[0])
    ids, _ = O.lmhead(h, None, w.eps, np_(w.lm_q), np_(w.lm_s), two_term=mode == "two_term", w8a16=mode == "w8a16")
    agree = float(np.mean(ids == np_(run["ids"])))
    print(f"end to end: final hidden row error {wr:.2e}, greedy ids agree on {agree:.2f} of rows", flush=True)


def test_producer_quantized_rows_change_no_bit(run, dev):
    """The step with every projection quantizing its own input (prequant=False) gives the same bits at
    every stage as the default, where the add-norms, the MoE's fused add-norm and the attention
    epilogue write the e4m3 rows (the KV cache rows it rewrites are the same values)."""
    from bundles_amd import synth
    hybrid, w, st = run["hybrid"], run["w"], run["st"]
    ws = hybrid.HybridWorkspace(B, T, E, dev, prequant=False)
    x = synth.randn((B * T, 2048), synth.gen(dev, 5), dev)
    trace = {}
    ids = hybrid.forward(x, w, st, ws, trace=trace)
    torch.cuda.synchronize()
    assert torch.equal(ids, run["ids"])
    for k, v in run["trace"].items():
        if isinstance(v, torch.Tensor):
            assert torch.equal(trace[k].view(torch.uint8), v.view(torch.uint8)), k
