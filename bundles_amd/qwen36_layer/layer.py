"""Decoder-layer node: prepare(module) / forward(prepared, *args, **kwargs).

The reference's layer entry (R = qwen36_nodes_kb34, L = R/qwen36_layer) builds a private replica of the
served decoder layer (L/layer.py:486-531) and swaps its hot sub-paths for its kernels, leaving the
served module and its submodule dict untouched.  This node does the same with libq36:

  MoE block      <- _replace_moe (L/layer.py:387-483): the decode / target-verify row batch (at most
                    MAX_TOKENS rows, positions given) runs q36_moe_forward; prefill, mixed and idle
                    batches and deferred finalize run the stock block.
  GDN mixer      <- _replace_gdn_prefill's target-verify branch (L/layer.py:289-309) with
                    gdn_verify_fused (L/gdn_fused.py:37-57): in_proj, the verify over the ReplaySSM ring
                    with its gated norm, and out_proj, on a verify batch; stock otherwise.  A batch of at
                    most DENSE8_ROWS rows projects through DENSE8 int8 copies of the served weights
                    (W8A16, L/layer.py:13-17, L/dense8_store.py:8-13), wider ones through the e4m3 copies.
  attention      <- attn_fused.install (L/attn_fused.py:213-273): the q/gate/k/v projection with the q/k
                    norm, partial RoPE and the e4m3 KV write, the verify attention over the KV cache, and
                    the gated o_proj, on a verify batch; stock otherwise.
The row-batch rule is the reference's (L/layer.py:174-189): forward_mode.is_decode() or
is_target_verify(); every other call, including a prefill chunk whose first row sits at position 0,
goes to stock code.  (The libq36 MoE treats position-0 rows as padding, so it must never see prefill.)

Weights are prepared once here, never on the hot path: the MoE experts in the caller's format (e4m3
128x128 blocks, or int8 per channel built as the reference's q8-block-v1 copy, L/i8x_kernels.py:69-141,
L/i8x_reloc.py:193-241), the projections of the mixers as e4m3 128x128 blocks.  The mixers' pools come
from an EngineView (engine.py); without one that serves the batch, the mixers run stock.
"""
from __future__ import annotations

import copy

import torch

from . import attn_fused, gdn_fused, moe
from .engine import EngineView, SglangView
from .formats import quant_dense8, tile_w16
from .glue import LinearWorkspace, dense8_linear, fp8_linear, linear_rows, prepare_fp8_weight

HIDDEN, EXPERTS, INTERMEDIATE, TOPK = 2048, 512, 512, 10
MAX_TOKENS = moe.MAX_TOKENS
GDN_QKV, GDN_Z, GDN_HV = gdn_fused.QKV_DIM, gdn_fused.N_V_HEADS * gdn_fused.HEAD_V, gdn_fused.N_V_HEADS
PROJ_IN = 4096
DENSE8_ROWS = 32  # the reference's DENSE8 row limit for the recurrent block's projections


def _mode_is(forward_batch, *names) -> bool:
    mode = getattr(forward_batch, "forward_mode", None)
    if mode is None:
        return False
    return any(bool(getattr(mode, n)()) for n in names if callable(getattr(mode, n, None)))


def row_batch(forward_batch) -> bool:
    """Plain decode or MTP target-verify: the engine's per-token calls (L/layer.py:174-185)."""
    return _mode_is(forward_batch, "is_decode", "is_target_verify")


def verify_batch(forward_batch) -> bool:
    return _mode_is(forward_batch, "is_target_verify")


def _check(name: str, t: torch.Tensor, shape) -> None:
    """The served tensors this node reads: bf16, contiguous, of the model's shape."""
    if tuple(t.shape) != tuple(shape) or t.dtype != torch.bfloat16 or not t.is_contiguous():
        raise RuntimeError(f"{name} is {tuple(t.shape)} {t.dtype}"
                           f"{'' if t.is_contiguous() else ' (strided)'}; this node serves bf16 {tuple(shape)}")


def _topk_ok(block, topk: int) -> bool:
    cfg = getattr(getattr(block, "topk", None), "topk_config", None)
    if cfg is None:
        return True  # a block without a topk config object: the shapes below decide
    return (cfg.top_k == topk and cfg.renormalize and getattr(cfg, "scoring_func", "softmax") == "softmax"
            and getattr(cfg, "correction_bias", None) is None and not getattr(cfg, "use_grouped_topk", False)
            and getattr(cfg, "custom_routing_function", None) is None)


class _Scratch:
    """Per-device buffers shared by every layer node on the device: the calls are stream ordered, one
    layer after another, so one set serves them all."""

    _by_device: dict = {}

    @classmethod
    def get(cls, device, rows: int):
        s = cls._by_device.get(device)
        if s is None or s.rows < rows:
            s = cls._by_device[device] = cls(device, max(rows, MAX_TOKENS))
        return s

    def __init__(self, device, rows: int):
        self.rows = rows
        self.lin2048 = LinearWorkspace(rows, HIDDEN, device)
        self.lin4096 = LinearWorkspace(rows, PROJ_IN, device)
        self.attn = attn_fused.Workspace(rows, device)
        self.decode = attn_fused.DecodeWorkspace(rows, device)


# ---- MoE ---------------------------------------------------------------------------------------------
class _MoeNode:
    """The replica's private MoE block: row batches on libq36, the rest on stock."""

    def __init__(self, block, dtype: int, topk: int, max_tokens: int):
        experts, shared = block.experts, block.shared_expert
        self.block = block
        self.topk = topk
        self.router_w = block.gate.weight
        self.gate_w = block.shared_expert_gate.weight.reshape(-1)
        E, H = self.router_w.shape
        I = experts.w2_weight.shape[2]  # noqa: E741
        _check("gate.weight", self.router_w, (E, H))
        _check("experts.w13_weight", experts.w13_weight, (E, 2 * I, H))
        _check("experts.w2_weight", experts.w2_weight, (E, H, I))
        _check("shared_expert.gate_up_proj.weight", shared.gate_up_proj.weight, (2 * I, H))
        _check("shared_expert.down_proj.weight", shared.down_proj.weight, (H, I))
        _check("shared_expert_gate.weight", self.gate_w, (H,))
        with torch.no_grad():
            if dtype == moe.Q36_MOE_INT8:
                # the reference's own int8 codes: the channel-mode q8-block-v1 copy, read back as they are
                from .formats import quant_q8_block_v1
                blocks = quant_q8_block_v1(experts.w13_weight, experts.w2_weight, channel=True)
                self.ew = moe.prepare_experts_q8_block_v1(blocks, H, I, shared.gate_up_proj.weight,
                                                          shared.down_proj.weight)
                del blocks
            else:
                self.ew = moe.prepare_experts(experts.w13_weight, experts.w2_weight, shared.gate_up_proj.weight,
                                              shared.down_proj.weight, dtype)
        self.ws = moe.Workspace(E, H, I, topk, dtype, self.router_w.device, max_tokens=max_tokens)
        self.max_tokens = max_tokens

    def served(self, hidden_states, forward_batch) -> bool:
        n = hidden_states.shape[0]
        positions = getattr(forward_batch, "positions", None)
        return (row_batch(forward_batch) and 0 < n <= self.max_tokens and hidden_states.dtype == torch.bfloat16
                and positions is not None and positions.shape[0] == n)

    def __call__(self, hidden_states, forward_batch=None, defer_finalize=False):
        if defer_finalize or forward_batch is None or not self.served(hidden_states, forward_batch):
            return self.block.forward(hidden_states, forward_batch, defer_finalize=defer_finalize)
        x = hidden_states.reshape(-1, self.router_w.shape[1]).contiguous()
        return moe.moe_row_batch(x, forward_batch.positions.to(torch.int32), self.router_w, self.gate_w, self.ew,
                                 self.topk, self.ws)


def _moe_block(module, topk):
    """The served sparse MoE block, if it is the kind this node serves (raises otherwise)."""
    block = getattr(module, "mlp", None)
    if (getattr(block, "shared_expert", None) is None or getattr(block, "shared_expert_gate", None) is None
            or not hasattr(block, "experts") or not _topk_ok(block, topk)):
        raise RuntimeError("this node serves the sparse MoE layer with a separate gated shared expert and "
                           f"plain softmax top-{topk} routing")
    if getattr(block.gate, "bias", None) is not None:
        raise RuntimeError("this node serves a bias-free router")
    return block


def _install_moe(module, replica, dtype, topk, max_tokens):
    block = _moe_block(module, topk)
    private = copy.copy(block)
    private.forward = _MoeNode(block, dtype, topk, max_tokens)
    replica._modules["mlp"] = private
    return private.forward


# ---- GDN mixer -----------------------------------------------------------------------------------------
def _tiled_dense8(w: torch.Tensor):
    """The reference's DENSE8 copy of w (L/dense8.py:168-188) with its rows tiled for the W8A16 kernel."""
    q, s = quant_dense8(w)
    return tile_w16(q), s


def gdn_layer_refusal(core, norm) -> str | None:
    """Why the ring verify cannot serve this recurrent layer (None: it can): the layer half of the
    reference's served-layout check (L/gdn_fused.py:30-34), a bias-free SiLU conv and the swish-gated
    RMSNorm applied before the gate over whole heads.  Attributes a module does not have are taken as
    the served model's."""
    if getattr(core, "bias", None) is not None or getattr(core, "activation", "silu") not in ("silu", "swish"):
        return "a conv with a bias or a non-SiLU activation"
    if (getattr(norm, "norm_before_gate", True) is not True
            or getattr(norm, "group_size", None) not in (None, norm.weight.numel())
            or getattr(norm, "activation", "silu") not in ("silu", "swish") or getattr(norm, "bias", None) is not None):
        return "a gated norm other than the swish-gated RMSNorm"
    return None


class _GdnMixer:
    """The recurrent mixer's target-verify step: in_proj (e4m3 blocks, columns split q|k|v, z, b, a),
    q36_gdn_verify_ring over the engine's pools (conv, delta rule, ring appends, gated norm), out_proj."""

    def __init__(self, lin, replica_lin, engine: EngineView, max_tokens: int, dense8_rows: int = DENSE8_ROWS):
        w_qkvz, w_ba, w_out = lin.in_proj_qkvz.weight, lin.in_proj_ba.weight, lin.out_proj.weight
        core, norm = lin.attn, lin.norm
        _check("linear_attn.in_proj_qkvz.weight", w_qkvz, (GDN_QKV + GDN_Z, HIDDEN))
        _check("linear_attn.in_proj_ba.weight", w_ba, (2 * GDN_HV, HIDDEN))
        _check("linear_attn.out_proj.weight", w_out, (HIDDEN, GDN_Z))
        _check("linear_attn.attn.conv_weights", core.conv_weights, (GDN_QKV, 4))
        _check("linear_attn.norm.weight", norm.weight, (gdn_fused.HEAD_V,))
        for b in (lin.in_proj_qkvz, lin.in_proj_ba, lin.out_proj):
            if getattr(b, "bias", None) is not None:
                raise RuntimeError("this node serves bias-free GDN projections")
        if core.A_log.dtype != torch.float32 or core.A_log.numel() != GDN_HV:
            raise RuntimeError("linear_attn.attn.A_log must be fp32 [32]")
        self.lin, self.replica, self.engine, self.max_tokens = lin, replica_lin, engine, max_tokens
        # a layer outside the served layout keeps the stock mixer for every batch
        self.refusal = gdn_layer_refusal(core, norm)
        self.layer_id = int(getattr(core, "layer_id", getattr(lin, "layer_id", -1)))
        self.stock = type(lin).forward
        self.conv_w, self.A_log, self.dt_bias = core.conv_weights, core.A_log, core.dt_bias.contiguous()
        self.norm_w, self.eps = norm.weight, float(getattr(norm, "eps", getattr(norm, "variance_epsilon", 1e-6)))
        self.scale = float(getattr(core, "head_k_dim", gdn_fused.HEAD_K)) ** -0.5
        self.dense8_rows = min(int(dense8_rows), 64)
        with torch.no_grad():
            w_in = torch.cat([w_qkvz, w_ba], dim=0)
            self.in_proj = prepare_fp8_weight(w_in)
            self.out_proj = prepare_fp8_weight(w_out)
            # the DENSE8 copies (int8 rows, fp16 scales per 128 columns) for the narrow batches, their rows
            # in the W8A16 kernel's tile order (1 KB contiguous loads; the same results)
            self.in8 = _tiled_dense8(w_in) if self.dense8_rows > 0 else None
            self.out8 = _tiled_dense8(w_out.contiguous()) if self.dense8_rows > 0 else None

    def __call__(self, hidden_states, forward_batch):
        x = hidden_states
        rows = x.shape[0] if isinstance(x, torch.Tensor) and x.dim() == 2 else 0
        pools = (self.engine.gdn_pools(self.layer_id, forward_batch)
                 if self.refusal is None and verify_batch(forward_batch) and 0 < rows <= self.max_tokens
                 and x.dtype == torch.bfloat16 else None)
        if pools is None or rows % pools.draft:
            return self.stock(self.replica, hidden_states, forward_batch)
        sc = _Scratch.get(x.device, rows)
        x = x.contiguous()
        e = dict(dtype=torch.bfloat16, device=x.device)
        mixed, z = torch.empty((rows, GDN_QKV), **e), torch.empty((rows, GDN_Z), **e)
        b, a = torch.empty((rows, GDN_HV), **e), torch.empty((rows, GDN_HV), **e)
        segs = [(0, mixed), (GDN_QKV, z), (GDN_QKV + GDN_Z, b), (GDN_QKV + GDN_Z + GDN_HV, a)]
        dense8 = rows <= self.dense8_rows
        if dense8:
            dense8_linear(x, *self.in8, segments=segs, tiled=True)
        else:
            fp8_linear(x, self.in_proj, sc.lin2048, segments=segs)
        p = pools
        # the e4m3 out_proj input comes from the verify kernel's epilogue (same bits as quantizing core)
        oq = None if dense8 else linear_rows(rows, PROJ_IN, x.device)
        core = gdn_fused.gdn_verify_ring(mixed, z, a, b, p.conv_state, self.conv_w, p.window, self.A_log,
                                         self.dt_bias, p.h0, p.d, p.dlo, p.k, p.klo, p.g, p.qsl, p.state_idx,
                                         p.replay_idx, p.win_idx, p.write_pos, p.cache_base, self.norm_w, self.eps,
                                         self.scale, T=p.draft, oq=oq)
        out = torch.empty((rows, HIDDEN), **e)
        if dense8:
            dense8_linear(core, *self.out8, segments=[(0, out)], tiled=True)
        else:
            fp8_linear(core, self.out_proj, sc.lin4096, segments=[(0, out)], xq=oq)
        return out


def _install_gdn(module, replica, engine, max_tokens, dense8_rows):
    lin = module.linear_attn
    private = copy.copy(lin)
    private._modules = dict(lin._modules)
    mixer = _GdnMixer(lin, private, engine, max_tokens, dense8_rows)
    private.forward = mixer
    replica._modules["linear_attn"] = private
    return mixer


# ---- attention mixer --------------------------------------------------------------------------------------
def attn_layer_refusal(module) -> str | None:
    """Why the verify attention cannot serve this attention layer (None: it can): the layer half of the
    reference's served-layout check (L/attn_fused.py:48-60), an output gate, one q/k norm epsilon, an
    unscaled e4m3 cache, full causal self-attention (no sliding window, no cross-attention, no logit
    cap).  Attributes a module does not have are taken as the served model's."""
    attn = getattr(module, "attn", None)
    if not getattr(module, "attn_output_gate", True):
        return "no output gate"
    if float(module.q_norm.variance_epsilon) != float(module.k_norm.variance_epsilon):
        return "different q and k norm epsilons"
    if getattr(attn, "k_scale", None) is not None or getattr(attn, "v_scale", None) is not None:
        return "a scaled KV cache"
    sw = getattr(attn, "sliding_window_size", None)
    if sw is not None and sw > -1:
        return "a sliding window"
    if getattr(attn, "is_cross_attention", False):
        return "cross-attention"
    if getattr(attn, "logit_cap", None) not in (None, 0, 0.0):
        return "a logit cap"
    return None


class _AttnMixer:
    """The gated attention mixer's target-verify step: q36_attn_proj (q/gate/k/v, q/k norm, partial
    RoPE, the new e4m3 K/V rows written into the engine's KV cache at out_cache_loc), q36_attn_decode
    over that cache, and q36_attn_oproj (sigmoid gate, o_proj)."""

    def __init__(self, module, replica, engine: EngineView, max_tokens: int):
        w_qkv, w_o = module.qkv_proj.weight, module.o_proj.weight
        nq, nkv, d = attn_fused.N_Q_HEADS, attn_fused.N_KV_HEADS, attn_fused.HEAD_DIM
        _check("qkv_proj.weight", w_qkv, (attn_fused.QKV_ROWS, HIDDEN))
        _check("o_proj.weight", w_o, (HIDDEN, nq * d))
        _check("q_norm.weight", module.q_norm.weight, (d,))
        _check("k_norm.weight", module.k_norm.weight, (d,))
        if getattr(module.qkv_proj, "bias", None) is not None or getattr(module.o_proj, "bias", None) is not None:
            raise RuntimeError("this node serves bias-free attention projections")
        if int(getattr(module, "num_heads", nq)) != nq or int(getattr(module, "num_kv_heads", nkv)) != nkv or \
                int(getattr(module, "head_dim", d)) != d:
            raise RuntimeError("this node serves 16 x 256 query heads over 2 KV heads")
        rot = module.rotary_emb
        if int(getattr(rot, "rotary_dim", 64)) != 64 or rot.cos_sin_cache.shape[-1] != 64:
            raise RuntimeError("this node serves RoPE on the first 64 dims of each head")
        self.replica, self.engine, self.max_tokens = replica, engine, max_tokens
        # a layer outside the served layout keeps the stock attention for every batch
        self.refusal = attn_layer_refusal(module)
        self.layer_id = int(getattr(module.attn, "layer_id", getattr(module, "layer_id", -1)))
        self.stock = type(module).self_attention
        self.scale = float(getattr(module.attn, "scaling", d ** -0.5))
        self.eps = float(module.q_norm.variance_epsilon)
        self.q_norm_w, self.k_norm_w = module.q_norm.weight, module.k_norm.weight
        with torch.no_grad():
            self.cos_sin = rot.cos_sin_cache.to(torch.float32).contiguous()
            qg = nq * 2 * d
            self.w = attn_fused.prepare_weights(w_qkv[:qg], w_qkv[qg:qg + nkv * d], w_qkv[qg + nkv * d:], w_o)

    def __call__(self, positions, hidden_states, forward_batch):
        x = hidden_states
        rows = x.shape[0] if isinstance(x, torch.Tensor) and x.dim() == 2 else 0
        kv = (self.engine.kv_view(self.layer_id, forward_batch)
              if self.refusal is None and verify_batch(forward_batch) and 0 < rows <= self.max_tokens
              and x.dtype == torch.bfloat16 else None)
        if kv is None or rows % kv.draft or not 1 <= kv.draft <= 4:
            return self.stock(self.replica, positions, hidden_states, forward_batch)
        sc = _Scratch.get(x.device, rows)
        pos = positions.to(torch.int32).contiguous()
        p = attn_fused.attn_proj(x.contiguous(), self.w, self.q_norm_w, self.k_norm_w, self.eps, self.cos_sin, pos,
                                 sc.attn, cache=(kv.k_cache, kv.v_cache, kv.out_loc.to(torch.int64).contiguous()))
        # the o_proj's e4m3 input comes from the attention's epilogue (same bits as quantizing o * sigmoid(gate))
        aq = attn_fused.oproj_rows(rows, x.device)
        gate = p["gate"].view(rows, -1)
        o = attn_fused.attn_decode(p["q"], kv.k_cache, kv.v_cache, kv.page_table, kv.seqlens, kv.draft, self.scale,
                                   sc.decode, gate=gate, oq=aq)
        return attn_fused.attn_oproj(o.view(rows, -1), gate, self.w, sc.attn, aq=aq)


def _install_attention(module, replica, engine, max_tokens):
    mixer = _AttnMixer(module, replica, engine, max_tokens)
    # an instance attribute of the replica shadows the class's method; the served module keeps its own
    replica.self_attention = mixer
    return mixer


# ---- entry --------------------------------------------------------------------------------------------
def prepare(module, dtype: int = moe.Q36_MOE_FP8, topk: int = TOPK, max_tokens: int = MAX_TOKENS,
            engine: EngineView | None = None, mixers: bool = True, dense8_rows: int = DENSE8_ROWS):
    """Replica of the served decoder layer with the libq36 paths installed; the served module and its
    submodule dict are left untouched.  engine: where the mixers find the verify batch's pools
    (default: SGLang's attention backend, absent here); mixers=False installs the MoE only;
    dense8_rows: verify batches up to this many rows run the recurrent block's projections on DENSE8
    copies (0: never)."""
    _moe_block(module, topk)
    replica = copy.copy(module)
    replica._modules = dict(module._modules)
    node_moe = _install_moe(module, replica, dtype, topk, max_tokens)
    engine = engine if engine is not None else SglangView()
    mixer = None
    if mixers:
        if hasattr(module, "linear_attn"):
            mixer = _install_gdn(module, replica, engine, max_tokens, dense8_rows)
        elif hasattr(module, "qkv_proj") and hasattr(module, "o_proj"):
            mixer = _install_attention(module, replica, engine, max_tokens)
    stock_forward = type(module).forward

    def layer(*args, **kwargs):
        return stock_forward(replica, *args, **kwargs)

    layer.replica = replica
    layer.moe = node_moe
    layer.mixer = mixer
    return layer


def forward(prepared, *args, **kwargs):
    return prepared(*args, **kwargs)
