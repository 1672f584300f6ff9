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


def test_layer_node_runs_the_moe_row_batch(dev):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import layer, moe
    M, E = 16, 64
    d = synth.moe_inputs(M, dev, seed=5, E=E)
    served = _Layer(_Block(d))
    mlp_before = served._modules["mlp"]
    node = layer.prepare(served, dtype=moe.Q36_MOE_FP8)
    assert served._modules["mlp"] is mlp_before and served.mlp.forward.__self__ is mlp_before
    pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
    fb = types.SimpleNamespace(positions=pos)
    resid = torch.randn((M, 2048), device=dev).to(torch.bfloat16)
    out, r = layer.forward(node, pos, d["x"], resid, fb)
    assert r is resid
    ew = moe.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], moe.Q36_MOE_FP8)
    ws = moe.Workspace(E, 2048, 512, 10, moe.Q36_MOE_FP8, dev)
    ref = moe.moe_row_batch(d["x"], pos, d["router_w"], d["gate_w"], ew, 10, ws)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert mlp_before.stock_calls == 0
    # a call without positions (prefill-shaped) goes to the stock block
    out2, _ = layer.forward(node, pos, d["x"], resid, types.SimpleNamespace(positions=None))
    assert mlp_before.stock_calls == 1 and not out2.any()


class _Processor(torch.nn.Module):
    """Stand-in for the served logits processor: logits = lm_head.quant_method.apply(...)."""

    def forward(self, input_ids, hidden_states, lm_head, logits_metadata=None):
        qm = getattr(lm_head, "quant_method", None)
        if qm is not None:
            return qm.apply(lm_head, hidden_states)
        return torch.matmul(hidden_states, lm_head.weight.T)


def test_lmhead_node_logits_and_ids(dev):
    from bundles_amd.qwen36_lmhead8 import lmhead8, node
    R, V = 8, 4096
    g = torch.Generator(device=dev).manual_seed(3)
    h = torch.randn((R, 2048), generator=g, device=dev).to(torch.bfloat16)
    head = _Holder(weight=(torch.randn((V, 2048), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    proc = _Processor()
    prepared = node.prepare(proc)
    logits = node.forward(prepared, None, h, head)
    q, s = lmhead8.quantize_rows(head.weight.data)
    ws = lmhead8.Workspace(R, dev)
    ids, ref = lmhead8.w8a8_lmhead_argmax(h, q, s, ws, want_logits=True)
    torch.cuda.synchronize()
    assert torch.equal(logits.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(prepared.last_ids, ids)
    # an embedding bias is not on the int8 path: stock matmul
    out = prepared.logits(head, h, embedding_bias=torch.zeros(V, device=dev))
    assert out.dtype == torch.bfloat16 and prepared.last_ids is None
