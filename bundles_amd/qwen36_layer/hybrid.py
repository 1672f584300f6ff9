"""Config 5's hybrid decoder node on libq36: three gated-delta-net layers and one gated full-attention
layer, each followed by the fp8 512-expert MoE block, the add-norms between the blocks, then the
final norm and the int8 lm_head + greedy argmax.  One verify step of B requests x T tokens.

Mirrors the reference's composition (R = qwen36_nodes_kb34, L = R/qwen36_layer, H = R/qwen36_lmhead8):
the stock decoder layer the node replicates (L/layer.py:486-531): input add-norm, mixer, post add-norm,
MoE; the projection + add-norm around the mixers (L/proj.py:60-112); the GDN mixer's in_proj split
and verify (L/proj_fused.py:1-20, L/gdn_fused.py:37-57); the attention verify (L/attn_fused.py:110-124,
232-273); the lm_head node with the greedy sampler (H/node.py:136-151).  Each layer's input norm is the
add-norm fed by the previous layer's MoE output, folded into that MoE's combine launch as the
reference folds it (L/layer.py:66-145, L/qk_route.cu:630-820).  Every launch is a libq36 entry;
nothing here computes.

The projections are e4m3 with 128x128 block scales (the configuration's weight format), the KV
cache e4m3 with one-token pages, the lm_head int8 per channel with the lm_head node's arithmetic by
row count (lm_mode: W8A16 below 64 rows, two-term W8A8 up to 256, one-term above; H/node.py:9-11,
144-151).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .. import synth
from ..qwen36_lmhead8 import lmhead8, node as lm_node
from . import attn_fused, gdn_fused, moe
from .glue import Fp8Weight, LinearWorkspace, add_rmsnorm, fp8_linear, linear_rows, prepare_fp8_weight

KINDS = ("gdn", "gdn", "gdn", "attn")
HIDDEN, TOPK = 2048, 10
GDN_QKV, GDN_Z, GDN_HV = 8192, 4096, 32
IN_PROJ_N = GDN_QKV + GDN_Z + 2 * GDN_HV  # q|k|v, z, b, a = 12352 columns
ATTN_SCALE = 1.0 / 16.0  # 1 / sqrt(256)


@dataclass
class GdnLayer:
    in_proj: Fp8Weight   # [12352 (padded to 12416), 2048]
    out_proj: Fp8Weight  # [2048, 4096]
    conv_w: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    norm_w: torch.Tensor


@dataclass
class AttnLayer:
    w: attn_fused.AttnWeights
    q_norm_w: torch.Tensor
    k_norm_w: torch.Tensor


@dataclass
class Layer:
    kind: str
    input_norm_w: torch.Tensor
    post_norm_w: torch.Tensor
    mixer: object
    experts: moe.ExpertWeights
    router_w: torch.Tensor
    router_bias: torch.Tensor
    gate_w: torch.Tensor


@dataclass
class HybridWeights:
    layers: list
    final_norm_w: torch.Tensor
    lm_q: torch.Tensor   # int8 [V, 2048] row-major (the reference layout; what the oracle checks read)
    lm_s: torch.Tensor
    E: int
    lm_qt: torch.Tensor | None = None  # the same codes in the tile order (what the lm_head reads)
    eps: float = 1e-6


@dataclass
class HybridState:
    """One verify step's inputs beside the hidden rows: B requests x T new tokens."""
    B: int
    T: int
    conv_state: list          # per GDN layer bf16 [B, 8192, 3]
    S: list                   # per GDN layer fp32 [B, 32, 128, 128]
    k_cache: torch.Tensor     # e4m3 [slots, 2, 256]
    v_cache: torch.Tensor
    page_table: torch.Tensor  # int32 [B, stride]
    seqlens: torch.Tensor     # int32 [B], keys including the T new tokens
    out_loc: torch.Tensor     # int64 [B*T]: the new tokens' cache slots
    positions: torch.Tensor   # int32 [B*T]
    cos_sin: torch.Tensor     # fp32 [max_pos, 64]
    # "snapshot": the GDN verify writes every position's state (q36_gdn_verify, config 3's form);
    # "ring": the served ReplaySSM form (q36_gdn_verify_ring): S is the read-only checkpoint, conv_state
    # rolls in place, and each GDN layer has the ring pools in `ring` (request r on slot r)
    gdn_form: str = "snapshot"
    ring: list | None = None


def make_weights(device, seed: int = 0, E: int = synth.E, V: int = 151936, zipf: float = 1.1) -> HybridWeights:
    """Random-init weights of the architecture (no checkpoints), quantized once as the node prepares them."""
    g = synth.gen(device, seed)
    layers = []
    for i, kind in enumerate(KINDS):
        if kind == "gdn":
            gi = synth.gdn_inputs(1, 1, device, seed=seed * 16 + i)
            mixer = GdnLayer(prepare_fp8_weight(synth.randn((IN_PROJ_N, HIDDEN), g, device, 0.02)),
                             prepare_fp8_weight(synth.randn((HIDDEN, GDN_Z), g, device, 0.02)),
                             gi["conv_w"], gi["A_log"], gi["dt_bias"], gi["norm_w"])
        else:
            ai = synth.attn_inputs(1, device, seed=seed * 16 + i)
            mixer = AttnLayer(attn_fused.prepare_weights(ai["wqg"], ai["wk"], ai["wv"], ai["wo"]), ai["q_norm_w"],
                              ai["k_norm_w"])
        mi = synth.moe_inputs(1, device, seed=seed * 16 + 8 + i, E=E, zipf=zipf)
        ew = moe.prepare_experts(mi["w13"], mi["w2"], mi["sw13"], mi["sw2"], moe.Q36_MOE_FP8)
        del mi["w13"], mi["w2"]
        layers.append(Layer(kind, synth.randn((HIDDEN,), g, device, 0.1), synth.randn((HIDDEN,), g, device, 0.1),
                            mixer, ew, mi["router_w"], mi["router_bias"], mi["gate_w"]))
    lw = synth.randn((V, HIDDEN), g, device, 0.02)
    lm_q, lm_s = lmhead8.quantize_rows(lw)
    del lw
    return HybridWeights(layers, synth.randn((HIDDEN,), g, device, 0.1), lm_q, lm_s, E, lmhead8.tile_rows_w16(lm_q))


def _ring_pools(B: int, T: int, device, g, wp: int) -> dict:
    """One GDN layer's ReplaySSM pools for B requests on slots 0..B-1: a committed history of wp entries
    per request at a random cache base (d ~ N(0, 0.3), unit keys, gates of a typical magnitude, each
    bf16 value with its low part), the draft-window records, the cursors and the request indices."""
    d32 = torch.randn((B, GDN_HV, 16, 128), generator=g, device=device) * 0.3
    k32 = torch.randn((B, GDN_HV // 2, 16, 128), generator=g, device=device)
    k32 = k32 / k32.norm(dim=-1, keepdim=True)
    dh, kh = d32.to(torch.bfloat16), k32.to(torch.bfloat16)
    return dict(
        window=torch.zeros((B, GDN_QKV, T + 2), dtype=torch.bfloat16, device=device),
        d=dh, dlo=(d32 - dh.float()).to(torch.bfloat16), k=kh, klo=(k32 - kh.float()).to(torch.bfloat16),
        g=(-0.05 * torch.rand((B, GDN_HV, 16), generator=g, device=device)).contiguous(),
        wp=torch.full((B,), wp, dtype=torch.int32, device=device),
        cb=torch.randint(0, 16, (B,), generator=g, device=device, dtype=torch.int32),
        qsl=torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=device),
        idx=torch.arange(B, dtype=torch.int64, device=device))


def make_state(B: int, T: int, ctx: int, device, seed: int = 0, extra_slots: int = 64, gdn_form: str = "snapshot",
               ring_wp: int = 8) -> HybridState:
    """The node's state for one verify step: GDN conv / recurrent states, and an e4m3 KV pool holding
    ctx cached keys per request (values N(0,1) scaled per KV head) at random one-token slots, with the
    T new tokens' slots already in the page table (as the engine assigns them).  gdn_form "ring" adds
    each GDN layer's ReplaySSM pools with ring_wp committed entries per request."""
    if gdn_form not in ("snapshot", "ring"):
        raise ValueError(f"gdn_form must be 'snapshot' or 'ring', not {gdn_form!r}")
    g = synth.gen(device, seed)
    n_gdn = KINDS.count("gdn")
    conv = [synth.randn((B, GDN_QKV, 3), g, device) for _ in range(n_gdn)]
    S = [torch.randn((B, GDN_HV, 128, 128), generator=g, device=device) * 0.1 for _ in range(n_gdn)]
    slots = B * (ctx + T) + extra_slots
    hs = 0.5 + 1.5 * torch.rand((1, 2, 1), generator=g, device=device)
    kc = (torch.randn((slots, 2, 256), generator=g, device=device) * hs).to(torch.float8_e4m3fn).view(torch.uint8)
    vc = (torch.randn((slots, 2, 256), generator=g, device=device) * hs).to(torch.float8_e4m3fn).view(torch.uint8)
    perm = torch.randperm(slots, generator=g, device=device)[:B * (ctx + T)].to(torch.int32)
    pt = perm.reshape(B, ctx + T).contiguous()
    seqlens = torch.full((B,), ctx + T, dtype=torch.int32, device=device)
    out_loc = pt[:, ctx:].reshape(-1).to(torch.int64).contiguous()
    positions = (ctx + torch.arange(T, device=device, dtype=torch.int32)).repeat(B).contiguous()
    ring = [_ring_pools(B, T, device, g, ring_wp) for _ in range(n_gdn)] if gdn_form == "ring" else None
    return HybridState(B, T, conv, S, kc, vc, pt, seqlens, out_loc, positions,
                       synth.rope_cos_sin(ctx + T + 1, device=device), gdn_form, ring)


@dataclass
class HybridWorkspace:
    """Every intermediate of one step of M = B*T rows (allocated once, reused by every step).  With
    snapshots=False (the ring form) the per-position GDN state buffers are not allocated.  With
    prequant (the default) every projection that follows an add-norm or the attention reads e4m3 rows
    its producer wrote (the add-norm, the MoE's fused add-norm, the attention epilogue) instead of
    quantizing them in a launch of its own; the outputs are the same bits either way."""
    B: int
    T: int
    E: int
    device: object
    bufs: dict = field(default_factory=dict)
    snapshots: bool = True
    prequant: bool = True

    def __post_init__(self):
        M, dev, bf = self.B * self.T, self.device, torch.bfloat16

        def e(*shape, dtype=bf):
            return torch.empty(shape, dtype=dtype, device=dev)
        n_gdn = KINDS.count("gdn")
        self.bufs = dict(
            residual=e(M, HIDDEN), residual2=e(M, HIDDEN), h=e(M, HIDDEN), h2=e(M, HIDDEN), o=e(M, HIDDEN), m=e(M, HIDDEN),
            mixed=e(M, GDN_QKV), z=e(M, GDN_Z), b=e(M, GDN_HV), a=e(M, GDN_HV), gout=e(M, GDN_Z),
            snaps=[e(self.B, self.T, GDN_HV, 128, 128, dtype=torch.float32) for _ in range(n_gdn)] if self.snapshots
            else None,
            conv_out=[e(self.B, GDN_QKV, 3) for _ in range(n_gdn)],
            attn=dict(q=e(M, 16, 256), gate=e(M, 16, 256), k=e(M, 2, 256), v=e(M, 2, 256),
                      k8=e(M, 2, 256, dtype=torch.uint8), v8=e(M, 2, 256, dtype=torch.uint8)),
            attn_out=e(M, 16, 256), ids=e(M, dtype=torch.int32))
        # producer-quantized rows for the layers' first projections (GDN in_proj, attention QKV) and the o_proj
        self.q8_gdn = linear_rows(M, HIDDEN, dev)
        self.q8_attn = attn_fused.proj_rows(M, dev)
        self.q8_o = attn_fused.oproj_rows(M, dev)
        self.q8_gout = linear_rows(M, 4096, dev)  # the ring verify's output codes for the out_proj
        self.lin2048 = LinearWorkspace(M, 2048, dev)
        self.lin4096 = LinearWorkspace(M, 4096, dev)
        self.attn = attn_fused.Workspace(M, dev)
        self.decode = attn_fused.DecodeWorkspace(self.B, dev)
        self.moe = moe.Workspace(self.E, HIDDEN, 512, TOPK, moe.Q36_MOE_FP8, dev, max_tokens=max(M, 1))
        self.lmhead = lmhead8.Workspace(M, dev)


def lm_mode(rows: int, vocab: int) -> str:
    """The lm_head arithmetic the node uses for a row batch: 'w8a16', 'two_term' or 'one_term'."""
    return lm_node.row_mode(rows, vocab)


def forward(x: torch.Tensor, w: HybridWeights, st: HybridState, ws: HybridWorkspace, trace: dict | None = None,
            stream=None) -> torch.Tensor:
    """x bf16 [B*T, 2048] (the embedded tokens) -> greedy ids int32 [B*T].  With trace (a dict), the
    inputs and outputs of every stage are kept there (copies) for stage-by-stage checks."""
    b = ws.bufs
    M = st.B * st.T
    if x.shape != (M, HIDDEN):
        raise ValueError(f"hybrid.forward: x must be [{M}, {HIDDEN}]")

    def keep(name, t):
        if trace is not None:
            trace[name] = t.clone() if isinstance(t, torch.Tensor) else t

    def rows_for(i):  # the e4m3 rows layer i's first projection reads (None: it quantizes its own)
        if not ws.prequant or i >= len(w.layers):
            return None
        return ws.q8_gdn if w.layers[i].kind == "gdn" else ws.q8_attn

    res, res_alt, h, h_next = b["residual"], b["residual2"], b["h"], b["h2"]
    res.copy_(x)
    add_rmsnorm(None, res, w.layers[0].input_norm_w, w.eps, out=h, stream=stream, q8=rows_for(0))
    keep("x", x)
    keep("h0", h)
    gi = 0
    for i, L in enumerate(w.layers):
        keep(f"L{i}.in", h)
        if L.kind == "gdn":
            g = L.mixer
            fp8_linear(h, g.in_proj, ws.lin2048, segments=[(0, b["mixed"]), (GDN_QKV, b["z"]),
                                                           (GDN_QKV + GDN_Z, b["b"]),
                                                           (GDN_QKV + GDN_Z + GDN_HV, b["a"])], stream=stream,
                       xq=rows_for(i))
            keep(f"L{i}.mixed", b["mixed"]), keep(f"L{i}.z", b["z"]), keep(f"L{i}.a", b["a"]), keep(f"L{i}.b", b["b"])
            if st.gdn_form == "ring":
                R = st.ring[gi]
                keep(f"L{i}.conv_state_in", st.conv_state[gi])
                for k in ("d", "dlo", "k", "klo", "g"):
                    keep(f"L{i}.ring_{k}_in", R[k])
                gdn_fused.gdn_verify_ring(b["mixed"], b["z"], b["a"], b["b"], st.conv_state[gi], g.conv_w, R["window"],
                                          g.A_log, g.dt_bias, st.S[gi], R["d"], R["dlo"], R["k"], R["klo"], R["g"],
                                          R["qsl"], R["idx"], R["idx"], R["idx"], R["wp"], R["cb"], g.norm_w, w.eps,
                                          128 ** -0.5, T=st.T, out=b["gout"], stream=stream,
                                          oq=ws.q8_gout if ws.prequant else None)
                gq = ws.q8_gout if ws.prequant else None
            else:
                gdn_fused.gdn_verify_fused(b["mixed"], b["z"], b["a"], b["b"], st.conv_state[gi], g.conv_w, g.A_log,
                                           g.dt_bias, st.S[gi], g.norm_w, w.eps, T=st.T, out=b["gout"],
                                           snaps=b["snaps"][gi], conv_state_out=b["conv_out"][gi], stream=stream)
                gq = None
            keep(f"L{i}.gout", b["gout"])
            fp8_linear(b["gout"], g.out_proj, ws.lin4096, segments=[(0, b["o"])], stream=stream, xq=gq)
            gi += 1
        else:
            a = L.mixer
            # the new tokens' K / V rows go into the cache in the projection's norm / RoPE step
            p = attn_fused.attn_proj(h, a.w, a.q_norm_w, a.k_norm_w, w.eps, st.cos_sin, st.positions, ws.attn,
                                     out=b["attn"], stream=stream, xq=rows_for(i),
                                     cache=(st.k_cache, st.v_cache, st.out_loc))
            oq = ws.q8_o if ws.prequant else None
            for k in ("q", "gate", "k8", "v8"):
                keep(f"L{i}.{k}", p[k])
            attn_fused.attn_decode(p["q"], st.k_cache, st.v_cache, st.page_table, st.seqlens, st.T, ATTN_SCALE,
                                   ws.decode, out=b["attn_out"], stream=stream,
                                   gate=p["gate"].view(M, 4096) if oq is not None else None, oq=oq)
            keep(f"L{i}.attn", b["attn_out"])
            attn_fused.attn_oproj(b["attn_out"].view(M, 4096), p["gate"].view(M, 4096), a.w, ws.attn, out=b["o"],
                                  stream=stream, aq=oq)
        keep(f"L{i}.o", b["o"])
        keep(f"L{i}.res_in", res)
        # the MoE block's input add-norm runs in its route kernel, the next block's in its combine
        # (the same bits as add_rmsnorm before and after the block); the residual moves to the other
        # buffer (the route reads the old one while it writes the new one)
        nxt = w.layers[i + 1].input_norm_w if i + 1 < len(w.layers) else w.final_norm_w
        moe.moe_row_batch(h if trace is not None else None, None, L.router_w, L.gate_w, L.experts, TOPK, ws.moe,
                          out=b["m"], router_bias=L.router_bias, stream=stream,
                          norm=(res_alt, nxt, w.eps, h_next), norm_q8=rows_for(i + 1),
                          pre_norm=(b["o"], res, res_alt, L.post_norm_w, w.eps))
        keep(f"L{i}.post", h)
        res, res_alt = res_alt, res
        h, h_next = h_next, h
        keep(f"L{i}.moe", b["m"])
        keep(f"L{i}.res_out", res)
    keep("final", h)
    mode = lm_mode(M, w.lm_q.shape[0])
    lmhead8.w8a8_lmhead_argmax(h, w.lm_q if w.lm_qt is None else None, w.lm_s, ws.lmhead, norm_w=None, eps=w.eps,
                               ids=b["ids"], q_t=w.lm_qt, stream=stream,
                               two_term=mode == "two_term", w8a16=mode == "w8a16")
    keep("ids", b["ids"])
    return b["ids"]
