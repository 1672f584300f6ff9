"""Logits-processor node: prepare(module) / forward(prepared, *args, **kwargs).

The slot (R = qwen36_nodes_kb34, H = R/qwen36_lmhead8; entries H/node.py:169-173) wraps the served
logits processor.  The processor computes logits through its lm_head argument: a head with a dense
`weight` is multiplied directly, any other head through `head.quant_method.apply(head, hidden_states,
embedding_bias)`.  The node hands the processor an Int8Head in place of a plain bf16 head: an object
without a `weight` whose quant_method is itself, so the processor's own code calls Int8Head.apply,
which runs q36_lmhead_argmax on an int8 copy of the served weight.  Everything else the processor does
(pruning, gathering, sampling metadata) is untouched.

Design:
  HeadCopy     the int8 copy of one served weight (codes + per-row fp32 scales, H/lmhead8.py:95-143),
               built on the first eligible call outside graph capture and rebuilt only when the served
               weight's storage, shape or version changes.
  row policy   the arithmetic follows the reference's choice by row count (H/node.py:9-11,144-151):
               fewer than W8A16_BELOW rows run W8A16 (bf16 rows, int8 weights; H/lmhead8.py:57-91),
               up to MAX_TWO_TERM rows the two-term W8A8 form (H/w8a8.py:25-37); more rows, up to
               MAX_ROWS, run the one-term W8A8 form (config 5's int8 lm_head over 2048 rows; the
               reference hands more than 256 rows to a bf16 matmul).
  greedy ids   the same launch finds each row's first largest logit; Int8Head keeps them on the node
               (last_ids) for a sampler that reads them instead of taking the argmax again.
  logits buffer for a decode or target-verify call of at least LOGITS_BUF_MIN_ROWS rows, the logits go
               straight into the processor's fp32 next_token_logits_buffer (bf16-rounded values) when
               its shape is exactly [rows, vocab]: stock then copies that tensor onto itself, a no-op
               (H/node.py:68-88,136-149); otherwise a fresh bf16 tensor is returned.
Heads the int8 path does not serve reach the processor as they came, so its stock code runs
(H/node.py:34-56): a processor that wants fp32 logits, an RL on-policy target or a tensor-parallel
all-gather of the logits; LoRA-wrapped heads; pre-quantized heads (a quant method other than the
unquantized one) and heads on the Intel AMX backend; no dense 2-D bf16 CUDA weight of width 2048; an
embedding bias, strided or non-bf16 hidden states, more than MAX_ROWS rows.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import lmhead8

HIDDEN = 2048
MAX_ROWS = 4096       # rows a call may carry on the int8 path (the workspace is sized once for this)
MAX_TWO_TERM = 256    # row batches up to this size take the two-term activation form
W8A16_BELOW = 64      # row batches below this size keep the activations in bf16
LOGITS_BUF_MIN_ROWS = 16  # row batches from this size write stock's fp32 logits buffer directly


def row_mode(rows: int, vocab: int = 151936) -> str:
    """The arithmetic for a row batch of `rows` rows: 'w8a16', 'two_term' or 'one_term'."""
    if rows < W8A16_BELOW and vocab % 32 == 0:
        return "w8a16"
    return "two_term" if rows <= MAX_TWO_TERM else "one_term"


def _servable_weight(w) -> bool:
    return (isinstance(w, torch.Tensor) and w.dim() == 2 and w.is_cuda and w.dtype == torch.bfloat16
            and w.shape[1] == HIDDEN and w.shape[0] % 16 == 0 and w.stride(1) == 1)


def _stock_logits_module():
    try:
        from sglang.srt.layers import logits_processor as stock_logits
    except ImportError:
        return None
    return stock_logits


def _prequantized(head) -> bool:
    """A head whose logits come from its own quant method (a quantized checkpoint's lm_head): the
    processor's own rule when SGLang is importable, else any quant method other than the unquantized
    one."""
    qm = getattr(head, "quant_method", None)
    stock = _stock_logits_module()
    if stock is not None and hasattr(stock, "should_apply_lm_head_quant_method"):
        return bool(stock.should_apply_lm_head_quant_method(head, qm))
    return qm is not None and not type(qm).__name__.startswith("Unquantized")


def _amx(head) -> bool:
    stock = _stock_logits_module()
    probe = getattr(stock, "use_intel_amx_backend", None) if stock is not None else None
    if callable(probe):
        return bool(probe(head))
    return bool(getattr(head, "use_intel_amx_backend", False))


def processor_refusal(processor) -> str | None:
    """Why the int8 head cannot stand in for this processor's lm_head (None: it can; H/node.py:34-38)."""
    if getattr(processor, "use_fp32_lm_head", False):
        return "fp32 lm_head"
    if getattr(processor, "rl_on_policy_target", None) is not None:
        return "RL on-policy target"
    if getattr(processor, "do_tensor_parallel_all_gather", False) or \
            getattr(processor, "do_tensor_parallel_all_gather_dp_attn", False):
        return "tensor-parallel all-gather of the logits"
    return None


def _meta(args, kwargs):
    return kwargs["logits_metadata"] if "logits_metadata" in kwargs else args[3] if len(args) > 3 else None


def logits_buffer(processor, args, kwargs) -> torch.Tensor | None:
    """Stock's fp32 next_token_logits_buffer for a decode / target-verify call, else None.  In those
    modes the processor computes logits once and copies them into this buffer when the shapes match;
    writing the bf16-rounded logits into it directly makes that copy a no-op with the same bytes
    (H/node.py:68-88).  A processor that scales its logits afterwards gets no buffer."""
    meta = _meta(args, kwargs)
    mode = getattr(meta, "forward_mode", None)
    is_decode, is_verify = getattr(mode, "is_decode", None), getattr(mode, "is_target_verify", None)
    if not (callable(is_decode) and callable(is_verify)) or not (is_decode() or is_verify()):
        return None
    if getattr(processor, "logit_scale", None) is not None:
        return None
    buf = getattr(meta, "next_token_logits_buffer", None)
    if not isinstance(buf, torch.Tensor) or buf.dtype != torch.float32 or buf.dim() != 2 or not buf.is_contiguous():
        return None
    return buf


def _version(w: torch.Tensor):
    try:
        return w._version
    except RuntimeError:  # inference tensors track no version; storage, shape and device still bind
        return None


@dataclass
class HeadCopy:
    q: torch.Tensor        # int8 [V, 2048] codes in the tile order (lmhead8.tile_rows_w16), what every form reads
    scale: torch.Tensor    # fp32 [V]
    ident: tuple           # (storage pointer, shape, device, version) of the weight it was built from

    @staticmethod
    def ident_of(w: torch.Tensor) -> tuple:
        return (w.data_ptr(), tuple(w.shape), w.device, _version(w))


class LogitsNode:
    """The prepared node: call it as the served processor would be called."""

    def __init__(self, processor):
        self.processor = processor
        self.stock_forward = type(processor).forward
        self.copy: HeadCopy | None = None
        self.workspace: lmhead8.Workspace | None = None
        self.last_ids: torch.Tensor | None = None
        self.out_buf: torch.Tensor | None = None  # this call's fp32 logits buffer (set by __call__)

    # -- the int8 copy and scratch, made outside capture only --
    def copy_for(self, w: torch.Tensor) -> HeadCopy | None:
        ident = HeadCopy.ident_of(w)
        if self.copy is not None and self.copy.ident == ident:
            return self.copy
        if torch.cuda.is_current_stream_capturing():
            return None
        self.copy = None  # free the stale copy before building the new one
        with torch.no_grad():
            q, s = lmhead8.quantize_rows(w.contiguous())
            q = lmhead8.tile_rows_w16(q)  # the row-major codes are freed: one copy of V x 2048 bytes
        self.copy = HeadCopy(q, s, ident)
        return self.copy

    def workspace_for(self, device) -> lmhead8.Workspace | None:
        if self.workspace is None:
            if torch.cuda.is_current_stream_capturing():
                return None
            self.workspace = lmhead8.Workspace(MAX_ROWS, device)
        return self.workspace

    # -- one call of the int8 head; None: not served here --
    def int8_logits(self, weight, hidden_states, embedding_bias):
        self.last_ids = None
        h = hidden_states
        if (embedding_bias is not None or not isinstance(h, torch.Tensor) or h.dim() != 2
                or h.dtype != torch.bfloat16 or h.shape[1] != HIDDEN or not 0 < h.shape[0] <= MAX_ROWS
                or h.device != weight.device or h.stride(1) != 1):
            return None
        hc = self.copy_for(weight)
        ws = self.workspace_for(h.device) if hc is not None else None
        if ws is None:
            return None
        rows, vocab = h.shape[0], hc.q.shape[0]
        mode = row_mode(rows, vocab)
        buf = self.out_buf
        out = (buf if buf is not None and rows >= LOGITS_BUF_MIN_ROWS and tuple(buf.shape) == (rows, vocab)
               and vocab == getattr(self.processor, "vocab_size", -1) and buf.device == weight.device else None)
        ids, logits = lmhead8.w8a8_lmhead_argmax(h.contiguous(), None, hc.scale, ws, want_logits=True, logits=out,
                                                 two_term=mode == "two_term", w8a16=mode == "w8a16", q_t=hc.q)
        self.last_ids = ids
        return logits

    def serves(self, head) -> bool:
        """Whether the int8 head stands in for `head` in this processor (H/node.py:34-56)."""
        return processor_refusal(self.processor) is None and Int8Head.serves(head)

    def __call__(self, *args, **kwargs):
        if "lm_head" in kwargs:
            head = kwargs["lm_head"]
            if self.serves(head):
                kwargs = dict(kwargs, lm_head=Int8Head(self, head))
        elif len(args) > 2 and self.serves(args[2]):
            args = args[:2] + (Int8Head(self, args[2]),) + args[3:]
        self.out_buf = logits_buffer(self.processor, args, kwargs)
        try:
            return self.stock_forward(self.processor, *args, **kwargs)
        finally:
            self.out_buf = None


class Int8Head:
    """Stands in for the served head inside one processor call: no `weight`, and quant_method is the
    object itself, whose apply() the processor calls with the hidden rows."""

    def __init__(self, node: LogitsNode, served):
        self.node, self.served = node, served
        self.quant_method = self

    @staticmethod
    def serves(head) -> bool:
        """The head-side rules: no LoRA wrapper, not pre-quantized, not on AMX, a dense bf16 weight."""
        if head is None or (hasattr(head, "set_lora") and hasattr(head, "apply_lora")):
            return False
        if _prequantized(head) or _amx(head):
            return False
        return _servable_weight(getattr(head, "weight", None))

    def apply(self, layer, hidden_states, embedding_bias=None):
        w = self.served.weight
        out = self.node.int8_logits(w, hidden_states, embedding_bias)
        if out is None:  # the stock product of the served weight (what the processor does for a dense head)
            out = torch.matmul(hidden_states.to(w.dtype), w.T)
            if embedding_bias is not None:
                out += embedding_bias  # in place: the logits keep the head's dtype
        return out


def prepare(module):
    return LogitsNode(module)


def forward(prepared, *args, **kwargs):
    return prepared(*args, **kwargs)
