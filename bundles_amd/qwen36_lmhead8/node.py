"""lm_head node: prepare(module) / forward(prepared, *args, **kwargs).

Mirrors the reference's logits-processor node (R = qwen36_nodes_kb34, H = R/qwen36_lmhead8):
  prepare  <- H/node.py:169-170: wrap the served logits processor.
  forward  <- H/node.py:172-173: run the stock processor with the lm_head swapped for a stand-in
              whose apply() computes the logits on the int8 path (H/node.py:100-110, :154-167).
The int8 copy of the head weight is built once per weight (H/node.py:123-134: keyed on the
weight's pointer, shape, dtype and device, never while a graph is being captured), rows are
quantized per row at call time, and the logits come from q36_lmhead_argmax with the logits
output enabled (bf16, as the reference's w8a8_linear returns them).  The greedy ids of the same
launch are kept on the node (last_ids) for a sampler that reads them instead of taking the
argmax again.  Anything the int8 path does not cover (an embedding bias, non-bf16 or strided
hidden states, more rows than MAX_ROWS, a weight shape other than [V, 2048]) goes to the stock
matmul, as in the reference (H/node.py:150-151).
"""
from __future__ import annotations

import torch

from . import lmhead8

MAX_ROWS = 4096
HIDDEN = 2048


class _Apply:
    __slots__ = ("node", "lm_head")

    def __init__(self, node, lm_head):
        self.node, self.lm_head = node, lm_head

    def apply(self, _stand_in, hidden_states, embedding_bias=None):
        return self.node.logits(self.lm_head, hidden_states, embedding_bias)


class _StandInHead:
    __slots__ = ("quant_method",)

    def __init__(self, apply):
        self.quant_method = apply


def _plain_head(lm_head) -> bool:
    w = getattr(lm_head, "weight", None)
    return isinstance(w, torch.Tensor) and w.dim() == 2


class _Node:
    def __init__(self, module):
        self.module = module
        self.stock_forward = type(module).forward
        self.q = self.scale = None
        self.source = None
        self.ws = None
        self.last_ids = None

    def _ready(self, weight) -> bool:
        key = (weight.data_ptr(), tuple(weight.shape), weight.dtype, weight.device)
        if self.q is not None and self.source == key:
            return True
        if torch.cuda.is_current_stream_capturing():
            return False
        with torch.no_grad():
            self.q, self.scale = lmhead8.quantize_rows(weight.to(torch.bfloat16).contiguous())
        self.source = key
        return True

    def logits(self, lm_head, hidden_states, embedding_bias=None):
        weight = lm_head.weight
        rows = hidden_states.shape[0] if hidden_states.dim() == 2 else 0
        if (embedding_bias is None and hidden_states.dtype == torch.bfloat16 and 0 < rows <= MAX_ROWS
                and hidden_states.shape[1] == HIDDEN == weight.shape[1] and weight.shape[0] % 16 == 0
                and hidden_states.stride(1) == 1 and hidden_states.device == weight.device
                and weight.device.type == "cuda" and self._ready(weight)):
            if self.ws is None or self.ws.R_max < rows:
                if torch.cuda.is_current_stream_capturing():
                    return torch.matmul(hidden_states.to(weight.dtype), weight.T)
                self.ws = lmhead8.Workspace(MAX_ROWS, hidden_states.device)
            ids, out = lmhead8.w8a8_lmhead_argmax(hidden_states.contiguous(), self.q, self.scale, self.ws,
                                                  want_logits=True)
            self.last_ids = ids
            return out
        self.last_ids = None
        return torch.matmul(hidden_states.to(weight.dtype), weight.T)

    def __call__(self, *args, **kwargs):
        if "lm_head" in kwargs:
            if _plain_head(kwargs["lm_head"]):
                kwargs = {**kwargs, "lm_head": _StandInHead(_Apply(self, kwargs["lm_head"]))}
        elif len(args) > 2 and _plain_head(args[2]):
            args = (*args[:2], _StandInHead(_Apply(self, args[2])), *args[3:])
        return self.stock_forward(self.module, *args, **kwargs)


def prepare(module):
    return _Node(module)


def forward(prepared, *args, **kwargs):
    return prepared(*args, **kwargs)
