"""Graph capture of the entry points: a call recorded into a CUDA graph (torch.cuda.graph, a hipGraph)
and replayed several times gives the eager call's bits on every replay.

The library records no memset node.  The workspace words that must start at zero (the MoE tickets and
expert counters, the lm_head's argmax keys) are reset by the library's own kernels, so a replay
starts from whatever the previous call on that workspace left.  Between replays the same entry runs
eagerly on the same workspace with other inputs, and the stream is synchronized, so every replay
after the first starts from a foreign call's leftovers.  The ring GDN verify updates its pools in
place: they are restored eagerly before each replay and compared after it.  Every output is
overwritten with a byte pattern before each replay, so a replay that wrote nothing would fail.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

REPLAYS = 4


@pytest.fixture(scope="module")
def lib():
    from bundles_amd import _lib
    _lib.lib()


def _bits(t: torch.Tensor) -> torch.Tensor:
    if t.dtype in (torch.bfloat16, torch.float16, torch.int16):
        return t.view(torch.int16)
    if t.dtype in (torch.float32, torch.int32):
        return t.view(torch.int32)
    return t


def _check_replays(what, call, outs_of, other=None, restore=None, state=()):
    """call() launches the entry and returns its result; outs_of(result) lists the tensors to compare;
    other() runs the same entry eagerly with other inputs; restore() resets in-place state; state lists
    tensors updated in place that must match the eager call's too."""
    print(f"graph: {what}", flush=True)
    if restore:
        restore()
    ref = [o.clone() for o in outs_of(call())] + [s.clone() for s in state]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    if restore:
        restore()
    with torch.cuda.graph(g):
        res = call()
    fresh = list(outs_of(res))
    outs = fresh + list(state)
    for i in range(REPLAYS):
        if restore:
            restore()
        for o in fresh:  # the replay must write every output again, not leave an earlier call's bits
            o.view(torch.uint8).fill_(0xA5)
        g.replay()
        torch.cuda.synchronize()
        for k, (a, b) in enumerate(zip(outs, ref)):
            assert torch.equal(_bits(a), _bits(b)), f"{what}: replay {i}, output {k} differs from the eager call"
        if other:
            other()
            torch.cuda.synchronize()
    del g


@pytest.mark.parametrize("dtype_name,M", [("Q36_MOE_FP8", 64), ("Q36_MOE_INT8", 37)])
def test_graph_moe_forward(lib, dev, dtype_name, M):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import moe
    dtype = getattr(moe, dtype_name)
    d = synth.moe_inputs(M, dev, seed=11, E=64, zipf=1.1)
    d2 = synth.moe_inputs(M + 3, dev, seed=12, E=64, zipf=1.1)
    ew = moe.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], dtype)
    ws = moe.Workspace(64, 2048, 512, 10, dtype, dev, max_tokens=128)
    out = torch.empty((M, 2048), dtype=torch.bfloat16, device=dev)

    def call():
        return moe.moe_row_batch(d["x"], None, d["router_w"], d["gate_w"], ew, 10, ws, out=out,
                                 router_bias=d["router_bias"])

    def other():
        moe.moe_row_batch(d2["x"], None, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"])

    _check_replays(f"moe {dtype_name} M={M}", call, lambda r: [r], other)


@pytest.mark.parametrize("R,mode,logits", [(300, "w8a8", None), (200, "x2", "bf16"), (16, "w8a16", "f32")])
def test_graph_lmhead_argmax(lib, dev, R, mode, logits):
    from bundles_amd import synth
    from bundles_amd.qwen36_lmhead8 import lmhead8 as lmh
    V = 8192
    d = synth.lmhead_inputs(R, V, dev, seed=R)
    h2 = torch.randn((R, 2048), device=dev).to(torch.bfloat16)
    q, s = lmh.quantize_rows(d["w"])
    qt = lmh.tile_rows_w16(q)
    ws = lmh.Workspace(R, dev)
    ids = torch.full((R,), -1, dtype=torch.int32, device=dev)
    out = None if logits is None else torch.empty(
        (R, V), dtype=torch.float32 if logits == "f32" else torch.bfloat16, device=dev)
    kw = dict(two_term=mode == "x2", w8a16=mode == "w8a16", q_t=qt, norm_w=d["norm_w"], eps=1e-6)

    def call():
        lmh.w8a8_lmhead_argmax(d["h"], None, s, ws, ids=ids, logits=out, **kw)
        return [ids] + ([] if out is None else [out])

    def other():
        lmh.w8a8_lmhead_argmax(h2, None, s, ws, **kw)

    _check_replays(f"lm_head {mode} R={R} logits={logits}", call, lambda r: r, other)


@pytest.mark.parametrize("T,N,K", [(37, 4096, 2048), (200, 2304, 2048), (16, 2048, 4096)])
def test_graph_fp8_linear(lib, dev, T, N, K):
    from bundles_amd.qwen36_layer import glue
    g = torch.Generator(device=dev).manual_seed(T + N)
    w = glue.prepare_fp8_weight((torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    x = torch.randn((T, K), generator=g, device=dev).to(torch.bfloat16)
    x2 = torch.randn((T, K), generator=g, device=dev).to(torch.bfloat16)
    ws = glue.LinearWorkspace(T, K, dev)
    _check_replays(f"fp8_linear T={T} N={N} K={K}", lambda: glue.fp8_linear(x, w, ws), lambda r: [r],
                   lambda: glue.fp8_linear(x2, w, ws))


@pytest.mark.parametrize("T,N,K,tiled", [(4, 12352, 2048, True), (32, 2048, 4096, False)])
def test_graph_dense8_linear(lib, dev, T, N, K, tiled):
    from bundles_amd.qwen36_layer import formats, glue
    g = torch.Generator(device=dev).manual_seed(T + N)
    q, s = formats.quant_dense8((torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    if tiled:
        q = formats.tile_w16(q)
    x = torch.randn((T, K), generator=g, device=dev).to(torch.bfloat16)
    x2 = torch.randn((T, K), generator=g, device=dev).to(torch.bfloat16)
    _check_replays(f"dense8_linear T={T} N={N} K={K} tiled={tiled}",
                   lambda: glue.dense8_linear(x, q, s, tiled=tiled), lambda r: [r],
                   lambda: glue.dense8_linear(x2, q, s, tiled=tiled))


def test_graph_attn_decode_with_new_rows(lib, dev):
    """Verify form (4 new tokens a request) with the new K/V rows written into the cache inside the
    graph: every replay writes the same rows to the same slots, then attends over them."""
    from bundles_amd.qwen36_layer import attn_fused
    B, NT = 16, 4
    g = torch.Generator().manual_seed(21)
    seqlens = torch.randint(NT, 700, (B,), generator=g, dtype=torch.int32)
    slots = int(seqlens.sum()) + 8
    e4 = lambda t: t.to(torch.float8_e4m3fn).view(torch.uint8)
    kc = e4(torch.randn((slots, 2, 256), generator=g)).to(dev)
    vc = e4(torch.randn((slots, 2, 256), generator=g)).to(dev)
    perm = torch.randperm(slots, generator=g).to(torch.int32)
    pt = torch.zeros((B, int(seqlens.max()) + 2), dtype=torch.int32)
    loc = torch.empty((B * NT,), dtype=torch.int64)
    o = 0
    for b in range(B):
        n = int(seqlens[b])
        pt[b, :n] = perm[o:o + n]
        loc[b * NT:(b + 1) * NT] = pt[b, n - NT:n].long()
        o += n
    pt, seqlens, loc = pt.to(dev), seqlens.to(dev), loc.to(dev)
    q = torch.randn((B * NT, 16, 256), generator=g).to(torch.bfloat16).to(dev)
    q2 = torch.randn((B * NT, 16, 256), generator=g).to(torch.bfloat16).to(dev)
    kn = e4(torch.randn((B * NT, 2, 256), generator=g)).to(dev)
    vn = e4(torch.randn((B * NT, 2, 256), generator=g)).to(dev)
    ws = attn_fused.DecodeWorkspace(B, dev)

    def call():
        return attn_fused.attn_decode(q, kc, vc, pt, seqlens, NT, 1.0 / 16.0, ws, out_loc=loc, k_new=kn, v_new=vn)

    _check_replays("attn_decode B=16 NT=4 with new rows", call, lambda r: [r],
                   lambda: attn_fused.attn_decode(q2, kc, vc, pt, seqlens, NT, 1.0 / 16.0, ws), state=(kc, vc))


def test_graph_gdn_verify_ring(lib, dev):
    """The served GDN verify updates its pools in place (conv state rolled, ring appends, window
    records); with the pools restored before each replay, every replay gives the eager output and pools."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import gdn_fused
    pools = ("conv_state", "window", "d_ring", "dlo_ring", "k_ring", "klo_ring", "g_ring")
    B, T = 8, 5
    d = synth.gdn_ring_inputs(B, T, dev, seed=31)
    saved = {k: d[k].clone() for k in pools}

    def restore():
        for k in pools:
            d[k].copy_(saved[k])

    def call():
        return gdn_fused.gdn_verify_ring(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"],
                                         d["window"], d["A_log"], d["dt_bias"], d["h0"], d["d_ring"], d["dlo_ring"],
                                         d["k_ring"], d["klo_ring"], d["g_ring"], d["qsl"], d["state_idx"],
                                         d["replay_idx"], d["win_idx"], d["write_pos"], d["cache_base"], d["norm_w"],
                                         1e-6, d["scale"], T=T)

    _check_replays("gdn ring B=8 T=5", call, lambda r: [r], restore=restore, state=[d[k] for k in pools])


@pytest.mark.parametrize("form", ["snapshot", "ring"])
def test_graph_hybrid_step(lib, dev, form):
    """The whole hybrid verify step (3 GDN + 1 attention layer, each with its MoE, the add-norms, the
    final norm and the int8 lm_head), captured as the bench runs it: with the KV cache, conv states and
    ring pools restored before each replay, every replay gives the eager step's ids and state."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import hybrid
    B, T, CTX, E, V = 2, 4, 40, 64, 4096
    w = hybrid.make_weights(dev, seed=3, E=E, V=V)
    st = hybrid.make_state(B, T, CTX, dev, seed=4, gdn_form=form)
    ws = hybrid.HybridWorkspace(B, T, E, dev)
    x = synth.randn((B * T, 2048), synth.gen(dev, 5), dev)
    x2 = synth.randn((B * T, 2048), synth.gen(dev, 6), dev)
    state = [st.k_cache, st.v_cache] + list(st.conv_state) + list(st.S)
    for r in st.ring or []:
        state += [t for t in r.values() if isinstance(t, torch.Tensor)]
    saved = [t.clone() for t in state]

    def restore():
        for t, s in zip(state, saved):
            t.copy_(s)

    _check_replays(f"hybrid step {form}", lambda: hybrid.forward(x, w, st, ws), lambda r: [r],
                   other=lambda: hybrid.forward(x2, w, st, ws), restore=restore, state=state)
