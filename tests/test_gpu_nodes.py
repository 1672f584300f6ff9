"""The node shims (prepare / forward) on the GPU: the layer node's decode row batch is the libq36 MoE
path bit for bit, the served module is left untouched, non-decode calls go to stock, and the
lm_head node returns the int8 path's logits and ids."""
import types

import pytest
import torch

pytestmark = pytest.mark.gpu


class _Holder(torch.nn.Module):
    def __init__(self, **tensors):
        super().__init__()
        for k, v in tensors.items():
            setattr(self, k, torch.nn.Parameter(v, requires_grad=False))


class _Block(torch.nn.Module):
    """Stand-in for the served sparse MoE block (stock forward marks the call)."""

    def __init__(self, d):
        super().__init__()
        self.gate = _Holder(weight=d["router_w"])
        self.gate.bias = None
        self.experts = _Holder(w13_weight=d["w13"], w2_weight=d["w2"])
        self.shared_expert = torch.nn.Module()
        self.shared_expert.gate_up_proj = _Holder(weight=d["sw13"])
        self.shared_expert.down_proj = _Holder(weight=d["sw2"])
        self.shared_expert_gate = _Holder(weight=d["gate_w"].reshape(1, -1))
        self.stock_calls = 0

    def forward(self, hidden_states, forward_batch=None, defer_finalize=False):
        self.stock_calls += 1
        return torch.zeros_like(hidden_states)


class _Layer(torch.nn.Module):
    def __init__(self, block):
        super().__init__()
        self.mlp = block

    def forward(self, positions, hidden_states, residual, forward_batch):
        return self.mlp(hidden_states, forward_batch), residual


class _Mode:
    """Stand-in for the engine's ForwardMode: one of decode, target_verify, extend, idle."""

    def __init__(self, name):
        self.name = name

    def is_decode(self):
        return self.name == "decode"

    def is_target_verify(self):
        return self.name == "target_verify"

    def is_extend(self):
        return self.name in ("extend", "target_verify")

    def is_idle(self):
        return self.name == "idle"


def _batch(mode, positions, **kw):
    return types.SimpleNamespace(forward_mode=_Mode(mode), positions=positions, **kw)


@pytest.mark.parametrize("dtype", [0, 1])
def test_layer_node_runs_the_moe_row_batch(dev, dtype):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import formats, layer, moe
    M, E = 16, 64
    print(f"layer node MoE dtype={dtype}", flush=True)
    d = synth.moe_inputs(M, dev, seed=5, E=E)
    served = _Layer(_Block(d))
    mlp_before = served._modules["mlp"]
    node = layer.prepare(served, dtype=dtype)
    assert served._modules["mlp"] is mlp_before and served.mlp.forward.__self__ is mlp_before
    pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
    resid = torch.randn((M, 2048), device=dev).to(torch.bfloat16)
    if dtype == moe.Q36_MOE_INT8:  # the node runs on the reference's own q8-block-v1 codes
        blocks = formats.quant_q8_block_v1(d["w13"], d["w2"], channel=True)
        ew = moe.prepare_experts_q8_block_v1(blocks, 2048, 512, d["sw13"], d["sw2"])
    else:
        ew = moe.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], dtype)
    ws = moe.Workspace(E, 2048, 512, 10, dtype, dev)
    ref = moe.moe_row_batch(d["x"], pos, d["router_w"], d["gate_w"], ew, 10, ws)
    for mode in ("decode", "target_verify"):
        out, r = layer.forward(node, pos, d["x"], resid, _batch(mode, pos))
        assert r is resid
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), mode
    assert mlp_before.stock_calls == 0
    # a prefill chunk (its first row at position 0), an idle batch, a batch without positions or without a
    # mode: all go to the stock block
    pre = torch.arange(0, M, dtype=torch.int32, device=dev)
    calls = 0
    for fb in (_batch("extend", pre), _batch("idle", pos), _batch("decode", None),
               types.SimpleNamespace(positions=pos)):
        out2, _ = layer.forward(node, pos, d["x"], resid, fb)
        calls += 1
        assert mlp_before.stock_calls == calls and not out2.any()


# ---- the mixers: stand-ins of the served GDN and attention layers with an engine view ---------------
class _Lin(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.weight = torch.nn.Parameter(w, requires_grad=False)
        self.bias = None


class _GdnCore(torch.nn.Module):
    def __init__(self, f, layer_id):
        super().__init__()
        self.conv_weights, self.A_log, self.dt_bias = f["conv_w"], f["A_log"], f["dt_bias"]
        self.head_k_dim, self.layer_id = 128, layer_id


class _LinearAttn(torch.nn.Module):
    """Stand-in of the served recurrent mixer: stock forward marks the call."""

    def __init__(self, f, w_qkvz, w_ba, w_out, layer_id):
        super().__init__()
        self.in_proj_qkvz, self.in_proj_ba, self.out_proj = _Lin(w_qkvz), _Lin(w_ba), _Lin(w_out)
        self.attn = _GdnCore(f, layer_id)
        self.norm = types.SimpleNamespace(weight=f["norm_w"], eps=1e-6)
        self.stock_calls = 0

    def forward(self, hidden_states, forward_batch):
        self.stock_calls += 1
        return torch.zeros_like(hidden_states)


class _GdnLayer(torch.nn.Module):
    def __init__(self, block, lin):
        super().__init__()
        self.mlp, self.linear_attn = block, lin

    def forward(self, positions, hidden_states, residual, forward_batch):
        return self.linear_attn(hidden_states, forward_batch), residual


class _View:
    """An EngineView over pools the test owns."""

    def __init__(self, gdn=None, kv=None):
        self.gdn, self.kv = gdn, kv

    def gdn_pools(self, layer_id, forward_batch):
        return self.gdn

    def kv_view(self, layer_id, forward_batch):
        return self.kv


@pytest.mark.parametrize("B", [6, 10])
def test_layer_node_gdn_verify(dev, B):
    """24 rows project through the DENSE8 copies (at most 32 rows, the reference's rule), 40 rows through
    the e4m3 blocks; either way the node's step equals the same entries composed by hand."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import engine, formats, gdn_fused, glue, layer
    T = 4
    print(f"layer node GDN mixer B={B}", flush=True)
    f = synth.gdn_ring_inputs(B, T, dev, seed=21)
    g = synth.gen(dev, 22)
    x = synth.randn((B * T, 2048), g, dev)
    w_qkvz, w_ba = synth.randn((12288, 2048), g, dev, 0.02), synth.randn((64, 2048), g, dev, 0.02)
    w_out = synth.randn((2048, 4096), g, dev, 0.02)
    lin = _LinearAttn(f, w_qkvz, w_ba, w_out, layer_id=3)
    served = _GdnLayer(_Block(synth.moe_inputs(1, dev, seed=5, E=64)), lin)

    def pools(src):
        return engine.GdnPools(src["conv_state"], src["window"], src["h0"], src["d_ring"], src["dlo_ring"],
                               src["k_ring"], src["klo_ring"], src["g_ring"], src["qsl"], src["state_idx"],
                               src["replay_idx"], src["win_idx"], src["write_pos"], src["cache_base"], T)
    mine = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in f.items()}
    node = layer.prepare(served, engine=_View(gdn=pools(mine)))
    assert served._modules["linear_attn"] is lin
    pos = torch.arange(100, 100 + B * T, dtype=torch.int32, device=dev)
    out, _ = layer.forward(node, pos, x, None, _batch("target_verify", pos))
    # the same step composed from the entries by hand
    dense8 = B * T <= layer.DENSE8_ROWS
    e = dict(dtype=torch.bfloat16, device=dev)
    mixed, z = torch.empty((B * T, 8192), **e), torch.empty((B * T, 4096), **e)
    b, a = torch.empty((B * T, 32), **e), torch.empty((B * T, 32), **e)
    segs = [(0, mixed), (8192, z), (12288, b), (12320, a)]
    if dense8:
        in8, out8 = formats.quant_dense8(torch.cat([w_qkvz, w_ba])), formats.quant_dense8(w_out)
        glue.dense8_linear(x, *in8, segments=segs)
    else:
        inw, outw = glue.prepare_fp8_weight(torch.cat([w_qkvz, w_ba])), glue.prepare_fp8_weight(w_out)
        glue.fp8_linear(x, inw, glue.LinearWorkspace(B * T, 2048, dev), segs)
    core = gdn_fused.gdn_verify_ring(mixed, z, a, b, f["conv_state"], f["conv_w"], f["window"], f["A_log"],
                                     f["dt_bias"], f["h0"], f["d_ring"], f["dlo_ring"], f["k_ring"], f["klo_ring"],
                                     f["g_ring"], f["qsl"], f["state_idx"], f["replay_idx"], f["win_idx"],
                                     f["write_pos"], f["cache_base"], f["norm_w"], 1e-6, 128 ** -0.5, T=T)
    ref = glue.dense8_linear(core, *out8) if dense8 else glue.fp8_linear(core, outw, glue.LinearWorkspace(B * T, 4096, dev))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    for k in ("conv_state", "window", "d_ring", "dlo_ring", "k_ring", "klo_ring", "g_ring"):
        assert torch.equal(mine[k].view(torch.uint8), f[k].view(torch.uint8)), k
    # stock runs on the replica's private mixer (a shallow copy: its own call counter)
    rl = node.replica.linear_attn
    assert rl is not lin and rl.stock_calls == 0 and lin.stock_calls == 0
    # decode and extend batches, and a view that does not serve the batch, run the stock mixer
    layer.forward(node, pos, x, None, _batch("decode", pos))
    layer.forward(node, pos, x, None, _batch("extend", pos))
    assert rl.stock_calls == 2
    node2 = layer.prepare(served, engine=_View())
    layer.forward(node2, pos, x, None, _batch("target_verify", pos))
    assert node2.replica.linear_attn.stock_calls == 1 and lin.stock_calls == 0


class _AttnLayer(torch.nn.Module):
    """Stand-in of the served gated-attention decoder layer (stock self_attention marks the call)."""

    def __init__(self, block, w_qkv, w_o, qn, kn, cos_sin):
        super().__init__()
        self.mlp = block
        self.qkv_proj, self.o_proj = _Lin(w_qkv), _Lin(w_o)
        self.q_norm = types.SimpleNamespace(weight=qn, variance_epsilon=1e-6)
        self.k_norm = types.SimpleNamespace(weight=kn, variance_epsilon=1e-6)
        self.rotary_emb = types.SimpleNamespace(cos_sin_cache=cos_sin, rotary_dim=64)
        self.attn = types.SimpleNamespace(layer_id=7, scaling=1.0 / 16)
        self.num_heads, self.num_kv_heads, self.head_dim = 16, 2, 256
        self.stock_calls = 0

    def self_attention(self, positions, hidden_states, forward_batch):
        self.stock_calls += 1
        return torch.zeros_like(hidden_states)

    def forward(self, positions, hidden_states, residual, forward_batch):
        return self.self_attention(positions, hidden_states, forward_batch), residual


def test_layer_node_attention_verify(dev):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import attn_fused, engine, layer
    B, T, ctx = 5, 4, 300
    print("layer node attention mixer", flush=True)
    ai = synth.attn_inputs(B * T, dev, seed=31, max_pos=ctx + T + 1)
    w_qkv = torch.cat([ai["wqg"], ai["wk"], ai["wv"]]).contiguous()
    served = _AttnLayer(_Block(synth.moe_inputs(1, dev, seed=5, E=64)), w_qkv, ai["wo"], ai["q_norm_w"],
                        ai["k_norm_w"], ai["cos_sin"])
    g = synth.gen(dev, 32)
    slots = B * (ctx + T) + 16
    kc = torch.randn((slots, 2, 256), generator=g, device=dev).to(torch.float8_e4m3fn).view(torch.uint8)
    vc = torch.randn((slots, 2, 256), generator=g, device=dev).to(torch.float8_e4m3fn).view(torch.uint8)
    pt = torch.randperm(slots, generator=g, device=dev)[:B * (ctx + T)].to(torch.int32).reshape(B, ctx + T)
    seqlens = torch.full((B,), ctx + T, dtype=torch.int32, device=dev)
    out_loc = pt[:, ctx:].reshape(-1).to(torch.int64).contiguous()
    pos = (ctx + torch.arange(T, device=dev, dtype=torch.int32)).repeat(B)
    kc2, vc2 = kc.clone(), vc.clone()
    node = layer.prepare(served, engine=_View(kv=engine.KvView(kc2, vc2, pt, seqlens, out_loc, T)))
    out, _ = layer.forward(node, pos.to(torch.int64), ai["x"], None, _batch("target_verify", pos))
    w = attn_fused.prepare_weights(ai["wqg"], ai["wk"], ai["wv"], ai["wo"])
    ws = attn_fused.Workspace(B * T, dev)
    p = attn_fused.attn_proj(ai["x"], w, ai["q_norm_w"], ai["k_norm_w"], 1e-6, ai["cos_sin"], pos, ws)
    o = attn_fused.attn_decode(p["q"], kc, vc, pt, seqlens, T, 1.0 / 16, attn_fused.DecodeWorkspace(B, dev),
                               out_loc=out_loc, k_new=p["k8"], v_new=p["v8"])
    ref = attn_fused.attn_oproj(o.view(B * T, -1), p["gate"].view(B * T, -1), w, ws)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc)  # the new rows landed in the same slots
    assert node.replica.stock_calls == 0 and served.stock_calls == 0
    layer.forward(node, pos, ai["x"], None, _batch("decode", pos))
    layer.forward(node, pos, ai["x"], None, _batch("extend", pos))
    assert node.replica.stock_calls == 2 and served.stock_calls == 0


class _Processor(torch.nn.Module):
    """Stand-in for the served logits processor: logits = lm_head.quant_method.apply(...); in decode
    and verify modes the logits are then copied into the metadata's fp32 buffer when the shapes match
    (stock's _copy_logits_to_buffer), and the buffer is what the processor returns."""

    def __init__(self, vocab_size=None):
        super().__init__()
        self.vocab_size = vocab_size
        self.logit_scale = None

    def forward(self, input_ids, hidden_states, lm_head, logits_metadata=None):
        qm = getattr(lm_head, "quant_method", None)
        if qm is not None:
            logits = qm.apply(lm_head, hidden_states)
        else:
            logits = torch.matmul(hidden_states, lm_head.weight.T)
        buf = getattr(logits_metadata, "next_token_logits_buffer", None)
        if buf is not None and buf.shape == logits.shape:
            buf.copy_(logits)
            return buf
        return logits


@pytest.mark.parametrize("R", [8, 64, 100, 300])
def test_lmhead_node_logits_and_ids(dev, R):
    """The node's logits and greedy ids are the int8 path's: W8A16 below 64 rows, the two-term form up
    to 256 rows, one term above; the served head is not modified."""
    from bundles_amd.qwen36_lmhead8 import lmhead8, node
    V = 4096
    g = torch.Generator(device=dev).manual_seed(3 + R)
    h = torch.randn((R, 2048), generator=g, device=dev).to(torch.bfloat16)
    head = _Holder(weight=(torch.randn((V, 2048), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    w_before = head.weight.detach().clone()
    proc = _Processor()
    prepared = node.prepare(proc)
    logits = node.forward(prepared, None, h, head)
    q, s = lmhead8.quantize_rows(head.weight.data)
    ws = lmhead8.Workspace(R, dev)
    mode = node.row_mode(R, V)
    assert mode == ("w8a16" if R < 64 else "two_term" if R <= 256 else "one_term")
    ids, ref = lmhead8.w8a8_lmhead_argmax(h, q, s, ws, want_logits=True, two_term=mode == "two_term",
                                          w8a16=mode == "w8a16")
    torch.cuda.synchronize()
    assert torch.equal(logits.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(prepared.last_ids, ids)
    assert torch.equal(head.weight, w_before)
    # the copy is reused while the weight is unchanged, rebuilt after an in-place update
    c0 = prepared.copy
    node.forward(prepared, None, h, head)
    assert prepared.copy is c0
    with torch.no_grad():
        head.weight.mul_(2)
    node.forward(prepared, None, h, head)
    assert prepared.copy is not c0
    # an embedding bias is not on the int8 path: the stock product of the served weight
    out = node.Int8Head(prepared, head).apply(None, h, embedding_bias=torch.zeros(V, device=dev))
    assert out.dtype == torch.bfloat16 and prepared.last_ids is None
    # a head the node does not serve (fp32 weight) reaches the processor unchanged
    head32 = _Holder(weight=torch.randn((V, 2048), generator=g, device=dev))
    assert not node.Int8Head.serves(head32)
    out = node.forward(prepared, None, h.float(), head32)
    assert out.dtype == torch.float32


@pytest.mark.parametrize("R", [8, 16, 64, 300])
def test_lmhead_node_writes_the_fp32_logits_buffer(dev, R):
    """A decode call with stock's fp32 next_token_logits_buffer of exactly [rows, vocab]: from 16 rows the
    int8 head writes the bf16-rounded logits into it directly (stock's copy is then of the buffer onto
    itself); below 16 rows a bf16 tensor comes back and stock copies it.  The buffer ends holding the
    same values either way (H/node.py:68-88,136-149)."""
    from bundles_amd.qwen36_lmhead8 import lmhead8, node
    V = 4096
    print(f"lmhead node fp32 buffer R={R}", flush=True)
    g = torch.Generator(device=dev).manual_seed(40 + R)
    h = torch.randn((R, 2048), generator=g, device=dev).to(torch.bfloat16)
    head = _Holder(weight=(torch.randn((V, 2048), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    prepared = node.prepare(_Processor(vocab_size=V))
    buf = torch.full((R, V), float("nan"), dtype=torch.float32, device=dev)
    meta = types.SimpleNamespace(forward_mode=_Mode("decode"), next_token_logits_buffer=buf)
    seen = []
    apply0 = node.Int8Head.apply

    def spy(self, layer, hidden_states, embedding_bias=None):
        out = apply0(self, layer, hidden_states, embedding_bias)
        seen.append(out)
        return out
    node.Int8Head.apply = spy
    try:
        out = node.forward(prepared, None, h, head, meta)
    finally:
        node.Int8Head.apply = apply0
    q, s = lmhead8.quantize_rows(head.weight.data)
    mode = node.row_mode(R, V)
    ids, ref = lmhead8.w8a8_lmhead_argmax(h, q, s, lmhead8.Workspace(R, dev), want_logits=True,
                                          two_term=mode == "two_term", w8a16=mode == "w8a16")
    torch.cuda.synchronize()
    assert out.data_ptr() == buf.data_ptr() and torch.equal(buf, ref.float())
    assert (seen[0].data_ptr() == buf.data_ptr()) is (R >= node.LOGITS_BUF_MIN_ROWS)
    assert torch.equal(prepared.last_ids, ids)
    # a prefill (extend) call gets no buffer: a fresh bf16 tensor comes back
    meta_x = types.SimpleNamespace(forward_mode=_Mode("extend"), next_token_logits_buffer=None)
    out_x = node.forward(prepared, None, h, head, meta_x)
    assert out_x.dtype == torch.bfloat16 and torch.equal(out_x, ref)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the decision capture launches nothing
def test_lmhead_node_under_graph_capture(dev):
    """Under capture the node builds neither its int8 copy nor its workspace (both allocate and launch
    work of their own), so a batch captured before any eager call goes to the stock product.  Once an
    eager call has made them, a captured call runs the int8 path, and its replays give the eager
    logits and ids."""
    from bundles_amd.qwen36_lmhead8 import node
    R, V = 100, 4096
    g = torch.Generator(device=dev).manual_seed(77)
    h = torch.randn((R, 2048), generator=g, device=dev).to(torch.bfloat16)
    head = _Holder(weight=(torch.randn((V, 2048), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    prepared = node.prepare(_Processor())
    print("lmhead node under capture: decisions", flush=True)
    empty = torch.cuda.CUDAGraph()
    with torch.cuda.graph(empty):  # nothing is launched inside: only the decisions are checked
        no_copy = prepared.copy_for(head.weight)
        no_ws = prepared.workspace_for(h.device)
    assert no_copy is None and no_ws is None
    assert prepared.copy is None and prepared.workspace is None
    del empty
    print("lmhead node under capture: int8 path", flush=True)
    ref = node.forward(prepared, None, h, head).clone()
    ids = prepared.last_ids.clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = node.forward(prepared, None, h, head)
    got_ids = prepared.last_ids
    for _ in range(3):
        out.fill_(0)
        got_ids.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(got_ids, ids)
        node.forward(prepared, None, torch.randn((R, 2048), device=dev).to(torch.bfloat16), head)
        torch.cuda.synchronize()
