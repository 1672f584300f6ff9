"""Where a verify batch's recurrent and attention state lives in the serving engine.

The layer node's GDN and attention paths need the engine's pools: the ReplaySSM checkpoint, rings,
conv states and draft windows of a recurrent layer, and the e4m3 KV cache, page table and key counts
of an attention layer.  The reference reads them through SGLang's attention backend
(R = qwen36_nodes_kb34, L = R/qwen36_layer):
  recurrent pools  <- L/gdn_fused.py:37-57 (get_attn_backend().linear_attn_backend, the mamba pool of
                      the layer, the forward metadata's query_start_loc / mamba_cache_indices, the
                      request pool indices, verify_intermediate_state_indices, the ring cursors)
  attention cache  <- L/attn_fused.py:70-75,110-124 (get_attn_backend().full_attn_backend, its KV
                      pool's buffers for the layer, page_table, cache_seqlens_int32, out_cache_loc)
Here that lookup is one object, an EngineView, handed to prepare(): SglangView reads the engine's
structures under the reference's attribute names; a test or another engine passes its own view.  A
view returns None when it cannot serve a batch, and the node then runs the stock module.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class GdnPools:
    """One recurrent layer's ReplaySSM pools and the batch's indices into them (q36_gdn_verify_ring)."""
    conv_state: torch.Tensor   # bf16 [slots, 8192, 3], rolled in place
    window: torch.Tensor       # bf16 [wslots, 8192, T + 2] (or its deduplicated [wslots, T, 8192, 3] view)
    h0: torch.Tensor           # fp32 [slots, 32, 128, 128], read only
    d: torch.Tensor            # bf16 [rslots, 32, 16, 128] (high parts)
    dlo: torch.Tensor          # bf16 [rslots, 32, 16, 128] (low parts)
    k: torch.Tensor            # bf16 [rslots, 16, 16, 128]
    klo: torch.Tensor          # bf16 [rslots, 16, 16, 128]
    g: torch.Tensor            # fp32 [rslots, 32, 16]
    qsl: torch.Tensor          # int32 [B + 1] first row of each request
    state_idx: torch.Tensor    # int32 / int64 [B] checkpoint and conv-state slot (< 0: padded request)
    replay_idx: torch.Tensor   # int32 / int64 [B] ring slot
    win_idx: torch.Tensor      # int32 / int64 [B] draft-window slot
    write_pos: torch.Tensor    # int32 [rslots] committed ring entries
    cache_base: torch.Tensor   # int32 [rslots] physical slot of logical ring entry 0
    draft: int = 4             # verify tokens per request


@dataclass
class KvView:
    """The attention layer's e4m3 KV cache (one-token pages) for one verify batch (q36_attn_decode)."""
    k_cache: torch.Tensor      # uint8 (e4m3 codes) [slots, 2, 256]
    v_cache: torch.Tensor
    page_table: torch.Tensor   # int32 [B, stride]: cache slot of each key position
    seqlens: torch.Tensor      # int32 [B]: key positions including the new tokens
    out_loc: torch.Tensor      # int64 [B * draft]: the new tokens' slots
    draft: int = 4


class EngineView:
    """The engine lookups the layer node makes; every method may return None (run stock)."""

    def gdn_pools(self, layer_id: int, forward_batch) -> GdnPools | None:
        return None

    def kv_view(self, layer_id: int, forward_batch) -> KvView | None:
        return None


RING_ENTRIES = 16  # the ring verify serves the 16-entry compact circular ReplaySSM ring
MAX_DRAFT = 8     # verify tokens per request the ring kernel serves


def gdn_pool_refusal(lin, pool, params, forward_batch) -> str | None:
    """Why the ring verify cannot serve this engine's recurrent pools (None: it can).  The served layout
    the reference requires before its verify kernel runs (L/gdn_fused.py:19-34): no multi-item scoring,
    the compact circular ReplaySSM ring (ring pools present, no spec-fold layout, not KDA, no beta ring,
    16 entries); here any of these sends the batch to the stock mixer instead of raising."""
    if getattr(lin, "mis_metadata", None) is not None:
        return "multi-item scoring"
    if (getattr(params, "replayssm_d", None) is None or getattr(params, "replayssm_rawv", None) is None
            or getattr(params, "replayssm_rawk", None) is None or getattr(pool, "replayssm_cache_base", None) is None):
        return "no ReplaySSM ring pools"
    if getattr(pool, "replayssm_spec_fold", True):
        return "spec-fold ring layout"
    if getattr(pool, "replayssm_is_kda", False):
        return "KDA ring"
    if getattr(params, "replayssm_beta", None) is not None:
        return "ring with a beta pool"
    if params.replayssm_d.shape[-2] != RING_ENTRIES:
        return f"{params.replayssm_d.shape[-2]}-entry ring"
    spec = getattr(forward_batch, "spec_info", None)
    draft = getattr(spec, "draft_token_num", None)
    if draft is None or not 1 <= int(draft) <= MAX_DRAFT:
        return f"{draft}-token drafts"
    return None


def kv_backend_refusal(full) -> str | None:
    """Why the verify attention cannot serve this attention backend (None: it can): one-token pages,
    chain drafts, no MLA (the backend half of L/attn_fused.py:48-60; the layer half is checked when the
    node is prepared)."""
    if getattr(full, "page_size", 1) != 1:
        return f"page size {getattr(full, 'page_size', None)}"
    if int(getattr(full, "topk", 1) or 1) > 1:
        return "tree drafts (topk > 1)"
    if getattr(full, "use_mla", False):
        return "MLA"
    return None


def _e4m3_codes(t: torch.Tensor) -> torch.Tensor | None:
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)
    return t if t.dtype == torch.uint8 else None


class SglangView(EngineView):
    """SGLang's hybrid attention backend, read under the attribute names the reference's glue uses.
    Absent SGLang (this image), every lookup returns None."""

    def _backend(self):
        try:
            from sglang.srt.model_executor.forward_context import get_attn_backend
        except ImportError:
            return None
        return get_attn_backend()

    def gdn_pools(self, layer_id, forward_batch):
        be = self._backend()
        lin = getattr(be, "linear_attn_backend", None)
        if lin is None:
            return None
        fm, pool = lin.forward_metadata, lin.req_to_token_pool.mamba_pool
        p = lin.req_to_token_pool.mamba2_layer_cache(layer_id)
        if getattr(fm, "retrieve_next_token", None) is not None or getattr(fm, "retrieve_next_sibling", None) is not None:
            return None  # tree drafts: the kernel serves chain verification only
        if gdn_pool_refusal(lin, pool, p, forward_batch) is not None:
            return None
        return GdnPools(p.conv[0], p.intermediate_conv_window[0], p.temporal, p.replayssm_d, p.replayssm_rawv,
                        p.replayssm_k, p.replayssm_rawk, p.replayssm_g, fm.query_start_loc, fm.mamba_cache_indices,
                        forward_batch.req_pool_indices, lin.verify_intermediate_state_indices,
                        pool.replayssm_spec_write_pos, pool.replayssm_cache_base,
                        int(forward_batch.spec_info.draft_token_num))

    def kv_view(self, layer_id, forward_batch):
        be = self._backend()
        full = getattr(be, "full_attn_backend", None)
        if full is None or kv_backend_refusal(full) is not None:
            return None
        k, v = full.token_to_kv_pool.get_kv_buffer(layer_id)
        k8, v8 = _e4m3_codes(k), _e4m3_codes(v)
        if k8 is None or v8 is None:
            return None
        md = full.forward_metadata
        return KvView(k8, v8, md.page_table, md.cache_seqlens_int32, forward_batch.out_cache_loc,
                      int(forward_batch.spec_info.draft_token_num))
