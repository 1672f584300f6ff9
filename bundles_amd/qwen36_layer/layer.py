"""Decoder-layer node: prepare(module) / forward(prepared, *args, **kwargs).

Mirrors the reference's layer entry (R = qwen36_nodes_kb34, L = R/qwen36_layer):
  prepare  <- L/layer.py:486-531: compose a replica of the served layer (never mutate the served
              module), give it a private MoE block whose decode row batch runs the libq36 path,
              and return a callable that runs the stock layer forward on the replica.
  forward  <- the manifest entry: forward(prepared, *args, **kwargs) = prepared(*args, **kwargs).
The MoE block is validated the way L/layer.py:386-411 does (Qwen sparse MoE, separate shared
expert with a sigmoid gate, plain softmax top-k with renormalisation, bias-free router), its
weights are quantized once here (int8 per channel or e4m3 128x128 blocks, the choice the caller
passes, as the reference's i8x copy is built at prepare time, L/i8x_reloc.py:193-241), and the
decode row batch (positions given, at most MAX_TOKENS rows) runs q36_moe_forward.  Everything
else (prefill, mixed batches, deferred finalize) goes to the stock block.forward, as in the
reference (L/layer.py:435-445).  The GDN verify and attention projection nodes are exposed as the
kernel calls the reference's glue makes (gdn_fused.gdn_verify_fused, attn_fused.attn_proj /
attn_oproj), not installed here: the served modules they replace (the linear-attention and
attention blocks with their cache pools) belong to the serving engine.
"""
from __future__ import annotations

import copy

import torch

from . import moe

HIDDEN, EXPERTS, INTERMEDIATE, TOPK = 2048, 512, 512, 10


def _check(name: str, t: torch.Tensor, shape) -> None:
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name}: shape {tuple(t.shape)} != {tuple(shape)}")


def _topk_ok(block, topk: int) -> bool:
    cfg = getattr(getattr(block, "topk", None), "topk_config", None)
    if cfg is None:
        return True  # a block without a topk config object: the shapes below decide
    return (cfg.top_k == topk and cfg.renormalize and getattr(cfg, "scoring_func", "softmax") == "softmax"
            and getattr(cfg, "correction_bias", None) is None and not getattr(cfg, "use_grouped_topk", False)
            and getattr(cfg, "custom_routing_function", None) is None)


class _MoeNode:
    """The replica's private MoE block: decode row batches on libq36, the rest on stock."""

    def __init__(self, block, dtype: int, topk: int, max_tokens: int):
        experts, shared = block.experts, block.shared_expert
        self.block = block
        self.topk = topk
        self.router_w = block.gate.weight
        self.gate_w = block.shared_expert_gate.weight.reshape(-1)
        E, H = self.router_w.shape
        I = experts.w2_weight.shape[2]  # noqa: E741
        _check("experts.w13_weight", experts.w13_weight, (E, 2 * I, H))
        _check("experts.w2_weight", experts.w2_weight, (E, H, I))
        _check("shared_expert.gate_up_proj.weight", shared.gate_up_proj.weight, (2 * I, H))
        _check("shared_expert.down_proj.weight", shared.down_proj.weight, (H, I))
        _check("shared_expert_gate.weight", self.gate_w, (H,))
        with torch.no_grad():
            self.ew = moe.prepare_experts(experts.w13_weight, experts.w2_weight, shared.gate_up_proj.weight,
                                          shared.down_proj.weight, dtype)
        self.ws = moe.Workspace(E, H, I, topk, dtype, self.router_w.device, max_tokens=max_tokens)
        self.max_tokens = max_tokens

    def __call__(self, hidden_states, forward_batch=None, defer_finalize=False):
        n = hidden_states.shape[0]
        positions = getattr(forward_batch, "positions", None)
        if (defer_finalize or forward_batch is None or n == 0 or n > self.max_tokens or positions is None
                or positions.shape[0] != n):
            return self.block.forward(hidden_states, forward_batch, defer_finalize=defer_finalize)
        x = hidden_states.reshape(-1, self.router_w.shape[1]).contiguous()
        return moe.moe_row_batch(x, positions.to(torch.int32), self.router_w, self.gate_w, self.ew, self.topk,
                                 self.ws)


def prepare(module, dtype: int = moe.Q36_MOE_FP8, topk: int = TOPK, max_tokens: int = moe.MAX_TOKENS):
    """Replica of the served decoder layer with the libq36 MoE decode path (the served module and
    its submodule dict are left untouched)."""
    block = module.mlp
    if (getattr(block, "shared_expert", None) is None or getattr(block, "shared_expert_gate", None) is None
            or not hasattr(block, "experts") or not _topk_ok(block, topk)):
        raise RuntimeError("this node serves the sparse MoE layer with a separate gated shared expert and "
                           f"plain softmax top-{topk} routing")
    if getattr(block.gate, "bias", None) is not None:
        raise RuntimeError("this node serves a bias-free router")
    replica = copy.copy(module)
    replica._modules = dict(module._modules)
    private = copy.copy(block)
    private.forward = _MoeNode(block, dtype, topk, max_tokens)
    replica._modules["mlp"] = private
    stock_forward = type(module).forward

    def layer(*args, **kwargs):
        return stock_forward(replica, *args, **kwargs)

    layer.replica = replica
    layer.moe = private.forward
    return layer


def forward(prepared, *args, **kwargs):
    return prepared(*args, **kwargs)
