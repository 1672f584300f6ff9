"""The nodes' served-layout rules on the CPU (no GPU): every engine, layer or processor the kernels do
not serve sends the batch to stock code, and the logits node writes stock's fp32 logits buffer only when
the reference would (R = qwen36_nodes_kb34: L/gdn_fused.py:19-34, L/attn_fused.py:48-60,
H/node.py:34-88)."""
import gc
import types
import weakref

import pytest
import torch

NS = types.SimpleNamespace


class _Mode:
    def __init__(self, name):
        self.name = name

    def is_decode(self):
        return self.name == "decode"

    def is_target_verify(self):
        return self.name == "target_verify"

    def is_extend(self):
        return self.name in ("extend", "target_verify")


# ---- recurrent pools --------------------------------------------------------------------------------------
def _gdn_backend(**over):
    """A SimpleNamespace SGLang backend whose recurrent pools are the served layout, with `over` applied:
    keys 'lin.X', 'pool.X', 'params.X', 'fm.X' set attribute X of that object."""
    t = torch.zeros
    params = NS(conv=[t(4, 8192, 3)], intermediate_conv_window=[t(4, 8192, 6)], temporal=t(4, 32, 128, 128),
                replayssm_d=t(4, 32, 16, 128), replayssm_rawv=t(4, 32, 16, 128), replayssm_k=t(4, 16, 16, 128),
                replayssm_rawk=t(4, 16, 16, 128), replayssm_g=t(4, 32, 16), replayssm_beta=None)
    pool = NS(replayssm_spec_write_pos=t(4, dtype=torch.int32), replayssm_cache_base=t(4, dtype=torch.int32),
              replayssm_spec_fold=False, replayssm_is_kda=False)
    fm = NS(retrieve_next_token=None, retrieve_next_sibling=None, query_start_loc=t(3, dtype=torch.int32),
            mamba_cache_indices=t(2, dtype=torch.int32))
    lin = NS(forward_metadata=fm, mis_metadata=None, verify_intermediate_state_indices=t(2, dtype=torch.int32),
             req_to_token_pool=NS(mamba_pool=pool, mamba2_layer_cache=lambda layer_id: params))
    objs = {"lin": lin, "pool": pool, "params": params, "fm": fm}
    for k, v in over.items():
        obj, attr = k.split(".")
        setattr(objs[obj], attr, v)
    return NS(linear_attn_backend=lin)


def _view(backend):
    from bundles_amd.qwen36_layer.engine import SglangView

    class View(SglangView):
        def _backend(self):
            return backend
    return View()


def _verify_batch(draft=4, rows=8):
    return NS(forward_mode=_Mode("target_verify"), spec_info=NS(draft_token_num=draft),
              req_pool_indices=torch.zeros(rows // max(draft, 1), dtype=torch.int32),
              out_cache_loc=torch.zeros(rows, dtype=torch.int64), positions=torch.arange(1, rows + 1))


GDN_VIOLATIONS = {
    "multi-item scoring": {"lin.mis_metadata": object()},
    "tree drafts": {"fm.retrieve_next_token": torch.zeros(2)},
    "spec-fold ring": {"pool.replayssm_spec_fold": True},
    "spec-fold unknown": {},  # the pool has no replayssm_spec_fold attribute (deleted in the test)
    "KDA ring": {"pool.replayssm_is_kda": True},
    "beta ring": {"params.replayssm_beta": torch.zeros(4, 32, 16)},
    "no ring": {"params.replayssm_d": None},
    "no raw v": {"params.replayssm_rawv": None},
    "no cache base": {"pool.replayssm_cache_base": None},
    "8-entry ring": {"params.replayssm_d": torch.zeros(4, 32, 8, 128)},
}


def test_gdn_pools_served_layout():
    pools = _view(_gdn_backend()).gdn_pools(3, _verify_batch())
    assert pools is not None and pools.draft == 4 and pools.d.shape == (4, 32, 16, 128)


@pytest.mark.parametrize("case", sorted(GDN_VIOLATIONS))
def test_gdn_pools_refuse_unserved_layouts(case):
    over = dict(GDN_VIOLATIONS[case])
    if case == "spec-fold unknown":  # an attribute the pool does not have counts as spec-fold (the reference)
        b = _gdn_backend()
        del b.linear_attn_backend.req_to_token_pool.mamba_pool.replayssm_spec_fold
    else:
        b = _gdn_backend(**over)
    assert _view(b).gdn_pools(3, _verify_batch()) is None


@pytest.mark.parametrize("draft", [0, 9])
def test_gdn_pools_refuse_draft_lengths_out_of_range(draft):
    assert _view(_gdn_backend()).gdn_pools(3, _verify_batch(draft=draft, rows=8)) is None


# ---- attention backend ----------------------------------------------------------------------------------------
def _kv_backend(**over):
    k = torch.zeros((64, 2, 256), dtype=torch.float8_e4m3fn)
    full = NS(page_size=1, topk=1, use_mla=False, token_to_kv_pool=NS(get_kv_buffer=lambda layer_id: (k, k)),
              forward_metadata=NS(page_table=torch.zeros((2, 16), dtype=torch.int32),
                                  cache_seqlens_int32=torch.full((2,), 8, dtype=torch.int32)))
    for a, v in over.items():
        setattr(full, a, v)
    return NS(full_attn_backend=full)


def test_kv_view_served_layout():
    kv = _view(_kv_backend()).kv_view(7, _verify_batch())
    assert kv is not None and kv.k_cache.dtype == torch.uint8 and kv.draft == 4


@pytest.mark.parametrize("over", [{"page_size": 16}, {"topk": 2}, {"use_mla": True}], ids=str)
def test_kv_view_refuses_unserved_backends(over):
    assert _view(_kv_backend(**over)).kv_view(7, _verify_batch()) is None


def test_kv_view_refuses_a_non_e4m3_cache():
    b = _kv_backend()
    kb = torch.zeros((64, 2, 256), dtype=torch.bfloat16)
    b.full_attn_backend.token_to_kv_pool = NS(get_kv_buffer=lambda layer_id: (kb, kb))
    assert _view(b).kv_view(7, _verify_batch()) is None


# ---- layer-side rules and the mixers' stock path -------------------------------------------------------------
def test_gdn_layer_refusal():
    from bundles_amd.qwen36_layer.layer import gdn_layer_refusal
    w = torch.zeros(128)
    ok_core, ok_norm = NS(bias=None, activation="silu"), NS(weight=w, norm_before_gate=True, group_size=None,
                                                            activation="swish", bias=None)
    assert gdn_layer_refusal(ok_core, ok_norm) is None
    assert gdn_layer_refusal(NS(), NS(weight=w)) is None  # plain modules: the served model's defaults
    assert gdn_layer_refusal(NS(bias=w, activation="silu"), ok_norm)
    assert gdn_layer_refusal(NS(bias=None, activation="gelu"), ok_norm)
    for bad in ({"norm_before_gate": False}, {"group_size": 64}, {"activation": "sigmoid"}, {"bias": w}):
        assert gdn_layer_refusal(ok_core, NS(**{**vars(ok_norm), **bad})), bad
    assert gdn_layer_refusal(ok_core, NS(**{**vars(ok_norm), "group_size": 128})) is None


def _attn_module(**attn_over):
    attn = NS(k_scale=None, v_scale=None, sliding_window_size=-1, is_cross_attention=False, logit_cap=0.0)
    for a, v in attn_over.items():
        setattr(attn, a, v)
    return NS(attn=attn, attn_output_gate=True, q_norm=NS(variance_epsilon=1e-6), k_norm=NS(variance_epsilon=1e-6))


def test_attn_layer_refusal():
    from bundles_amd.qwen36_layer.layer import attn_layer_refusal
    assert attn_layer_refusal(_attn_module()) is None
    assert attn_layer_refusal(_attn_module(sliding_window_size=None, logit_cap=None)) is None
    for bad in ({"k_scale": 1.0}, {"v_scale": torch.ones(1)}, {"sliding_window_size": 4096},
                {"is_cross_attention": True}, {"logit_cap": 30.0}):
        assert attn_layer_refusal(_attn_module(**bad)), bad
    m = _attn_module()
    m.attn_output_gate = False
    assert attn_layer_refusal(m)
    m = _attn_module()
    m.k_norm = NS(variance_epsilon=1e-5)
    assert attn_layer_refusal(m)


class _Stock:
    def __init__(self):
        self.calls = 0

    def __call__(self, *args):
        self.calls += 1
        return "stock"


def _bare(cls, **attrs):
    """A mixer object with only the attributes its dispatch reads (its weights need a GPU to prepare)."""
    m = object.__new__(cls)
    for k, v in attrs.items():
        setattr(m, k, v)
    return m


def test_gdn_mixer_sends_refused_layers_and_pools_to_stock():
    from bundles_amd.qwen36_layer.layer import _GdnMixer
    x = torch.zeros((8, 2048), dtype=torch.bfloat16)
    asked = []

    class Engine:
        def gdn_pools(self, layer_id, fb):
            asked.append(layer_id)
            return None
    stock = _Stock()
    # a refused layer never asks the engine
    m = _bare(_GdnMixer, refusal="a conv with a bias", engine=Engine(), stock=stock, replica=None, max_tokens=256,
              layer_id=2)
    assert m(x, _verify_batch()) == "stock" and stock.calls == 1 and asked == []
    # a served layer whose engine refuses its pools (each engine-side violation above returns None)
    for case in sorted(GDN_VIOLATIONS):
        if case == "spec-fold unknown":
            continue
        m = _bare(_GdnMixer, refusal=None, engine=_view(_gdn_backend(**GDN_VIOLATIONS[case])), stock=stock,
                  replica=None, max_tokens=256, layer_id=2)
        assert m(x, _verify_batch()) == "stock", case
    assert stock.calls == 1 + len(GDN_VIOLATIONS) - 1


def test_attn_mixer_sends_refused_layers_and_backends_to_stock():
    from bundles_amd.qwen36_layer.layer import _AttnMixer
    x = torch.zeros((8, 2048), dtype=torch.bfloat16)
    pos = torch.arange(1, 9)
    stock = _Stock()
    m = _bare(_AttnMixer, refusal="a sliding window", engine=_view(_kv_backend()), stock=stock, replica=None,
              max_tokens=256, layer_id=7)
    assert m(pos, x, _verify_batch()) == "stock" and stock.calls == 1
    for over in ({"page_size": 16}, {"topk": 2}, {"use_mla": True}):
        m = _bare(_AttnMixer, refusal=None, engine=_view(_kv_backend(**over)), stock=stock, replica=None,
                  max_tokens=256, layer_id=7)
        assert m(pos, x, _verify_batch()) == "stock", over
    assert stock.calls == 4


# ---- logits processor --------------------------------------------------------------------------------------
class _Proc:
    """Stand-in for the served logits processor: records the head it was handed."""

    def __init__(self, **attrs):
        self.heads = []
        for k, v in attrs.items():
            setattr(self, k, v)

    def forward(self, input_ids, hidden_states, lm_head, logits_metadata=None):
        self.heads.append(lm_head)
        return None


def _head(**attrs):
    return NS(weight=torch.zeros((4096, 2048), dtype=torch.bfloat16), **attrs)


@pytest.mark.parametrize("attrs,served", [
    ({}, True),
    ({"use_fp32_lm_head": True}, False),
    ({"rl_on_policy_target": "x"}, False),
    ({"do_tensor_parallel_all_gather": True}, False),
    ({"do_tensor_parallel_all_gather_dp_attn": True}, False),
], ids=lambda v: str(v))
def test_logits_node_processor_refusals(monkeypatch, attrs, served):
    from bundles_amd.qwen36_lmhead8 import node
    monkeypatch.setattr(node, "_servable_weight", lambda w: True)  # CPU weights: the rule under test decides
    proc = _Proc(**attrs)
    prepared = node.prepare(proc)
    head = _head()
    node.forward(prepared, None, torch.zeros((8, 2048)), head)
    assert isinstance(proc.heads[-1], node.Int8Head) is served
    if not served:
        assert proc.heads[-1] is head


class UnquantizedEmbeddingMethod:
    pass


class Fp8LinearMethod:
    pass


@pytest.mark.parametrize("head,served", [
    (_head(), True),
    (_head(quant_method=UnquantizedEmbeddingMethod()), True),
    (_head(quant_method=Fp8LinearMethod()), False),
    (_head(use_intel_amx_backend=True), False),
    (_head(set_lora=lambda *a: None, apply_lora=lambda *a: None), False),
    (None, False),
], ids=["plain", "unquantized-method", "pre-quantized", "amx", "lora", "none"])
def test_int8_head_refusals(monkeypatch, head, served):
    from bundles_amd.qwen36_lmhead8 import node
    monkeypatch.setattr(node, "_servable_weight", lambda w: True)
    assert node.Int8Head.serves(head) is served


def test_logits_buffer_rule():
    from bundles_amd.qwen36_lmhead8 import node
    buf = torch.zeros((16, 4096), dtype=torch.float32)
    proc = NS(logit_scale=None)
    meta = lambda mode, b=buf: NS(forward_mode=_Mode(mode), next_token_logits_buffer=b)  # noqa: E731
    assert node.logits_buffer(proc, (None, None, None, meta("decode")), {}) is buf
    assert node.logits_buffer(proc, (None, None, None), {"logits_metadata": meta("target_verify")}) is buf
    assert node.logits_buffer(proc, (None, None, None, meta("extend")), {}) is None
    assert node.logits_buffer(NS(logit_scale=0.5), (None, None, None, meta("decode")), {}) is None
    for b in (buf.to(torch.bfloat16), buf[:, ::2], buf.reshape(-1), None):
        assert node.logits_buffer(proc, (None, None, None, meta("decode", b)), {}) is None
    assert node.logits_buffer(proc, (None, None, None), {}) is None


def test_logits_node_sets_the_buffer_only_inside_the_call(monkeypatch):
    from bundles_amd.qwen36_lmhead8 import node
    buf = torch.zeros((16, 4096), dtype=torch.float32)
    seen = []

    class Proc(_Proc):
        def forward(self, input_ids, hidden_states, lm_head, logits_metadata=None):
            seen.append(prepared.out_buf)
    proc = Proc(logit_scale=None)
    prepared = node.prepare(proc)
    meta = NS(forward_mode=_Mode("decode"), next_token_logits_buffer=buf)
    node.forward(prepared, None, torch.zeros((16, 2048)), _head(), meta)
    assert seen == [buf] and prepared.out_buf is None


# ---- the MoE phase callables keep their tensors alive ---------------------------------------------------------
def test_moe_phases_keep_the_tensors_they_point_into():
    """The phase callables hold a struct of raw addresses: the tensors behind it must live as long as the
    callables, whatever the caller does with its own references (a caller that dropped them once left the
    struct pointing at freed memory)."""
    from bundles_amd.qwen36_layer import moe
    E, H, I, M, k = 8, 2048, 512, 4, 2
    u8 = dict(dtype=torch.uint8)
    ew = moe.ExpertWeights(moe.Q36_MOE_INT8, torch.zeros((E, 2 * I, H), **u8), torch.zeros((E, 2 * I)),
                           torch.zeros((E, H, I), **u8), torch.zeros((E, H)), torch.zeros((2 * I, H), **u8),
                           torch.zeros(2 * I), torch.zeros((H, I), **u8), torch.zeros(H))
    ws = moe.Workspace(E, H, I, k, moe.Q36_MOE_INT8, "cpu", max_tokens=M)
    x = torch.zeros((M, H), dtype=torch.bfloat16)
    pos = torch.arange(1, M + 1, dtype=torch.int32)
    rw = torch.zeros((E, H), dtype=torch.bfloat16)
    gw = torch.zeros(H, dtype=torch.bfloat16)
    out = torch.empty_like(x)
    refs = [weakref.ref(t) for t in (x, pos, rw, gw, out, ws.buf, ew.w13, ew.ss2)]
    phases = moe.moe_phases(x, pos, rw, gw, ew, k, ws, out)
    del x, pos, rw, gw, out, ws, ew
    gc.collect()
    assert all(r() is not None for r in refs)
    assert [n for n, _ in phases] == ["route", "up", "down", "combine"]
    del phases
    gc.collect()
    assert all(r() is None for r in refs)
