"""libq36 against the committed golden fixtures (seeded inputs regenerated on the CPU, moved to the
GPU): the config-1 int8 MoE at its full 512 experts bit for bit (ids, weights, output), the small
lm_head bit for bit, attention and GDN within the fp tolerances (bf16 1e-2 per-row norm, fp32
state 1e-4)."""
import os

import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, assert_f32_close, bits16, bits8, np_

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _fx(name):
    return np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)


def test_moe_cfg1_full_experts(dev):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import moe
    print("golden moe cfg1 (8 tokens, 512 experts, int8)", flush=True)
    fx = _fx("moe_cfg1_int8_m8")
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in synth.moe_inputs(8, "cpu", seed=0).items()}
    ew = moe.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], moe.Q36_MOE_INT8)
    del d["w13"], d["w2"]
    ws = moe.Workspace(512, 2048, 512, 10, moe.Q36_MOE_INT8, dev)
    out = moe.moe_row_batch(d["x"], None, d["router_w"], d["gate_w"], ew, 10, ws)
    torch.cuda.synchronize()
    v = ws.views(8)
    assert np.array_equal(np_(v["ids"]), fx["ids"])
    assert np.array_equal(np_(v["wts"]).view(np.uint32), fx["wts"].view(np.uint32))
    assert np.array_equal(bits16(out), fx["out"])


def test_lmhead_small(dev):
    from bundles_amd import synth
    from bundles_amd.qwen36_lmhead8 import lmhead8
    fx = _fx("lmhead_r8_v4096")
    d = {k: v.to(dev) for k, v in synth.lmhead_inputs(8, 4096, "cpu", seed=0).items()}
    q, s = lmhead8.quantize_rows(d["w"])
    ws = lmhead8.Workspace(8, dev)
    ids, logits = lmhead8.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=d["norm_w"], eps=1e-6, want_logits=True)
    torch.cuda.synchronize()
    assert np.array_equal(np_(ids), fx["ids"])
    assert np.array_equal(bits16(logits), fx["logits"])


def test_attention_t4(dev):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import attn_fused as A
    fx = _fx("attn_t4")
    d = {k: v.to(dev) for k, v in synth.attn_inputs(4, "cpu", seed=0).items()}
    w = A.prepare_weights(d["wqg"], d["wk"], d["wv"], d["wo"])
    ws = A.Workspace(4, dev)
    o = A.attn_proj(d["x"], w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws)
    out = A.attn_oproj(d["attn"], o["gate"].reshape(4, 4096), w, ws)
    torch.cuda.synchronize()
    for key in ("q", "gate", "k", "v"):
        assert_bf16_close(bits16(o[key]).reshape(4, -1), fx[key].reshape(4, -1), 1e-2, key)
    assert_bf16_close(bits16(out), fx["oproj"], 1e-2, "oproj")


def test_gdn_b2(dev, oracle_mod):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import gdn_fused
    fx = _fx("gdn_b2_t5")
    B, T = 2, 5
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in synth.gdn_inputs(B, T, "cpu", seed=0).items()}
    out = torch.empty((B * T, 4096), dtype=torch.bfloat16, device=dev)
    snaps = torch.empty((B, T, 32, 128, 128), dtype=torch.float32, device=dev)
    cso = torch.empty_like(d["conv_state"])
    gdn_fused.gdn_verify_fused(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_w"], d["A_log"],
                               d["dt_bias"], d["S0"], d["norm_w"], 1e-6, T=T, out=out, snaps=snaps, conv_state_out=cso)
    torch.cuda.synchronize()
    assert_bf16_close(bits16(out), fx["out"], 1e-2, "gdn out")
    sn = np_(snaps)
    assert_f32_close(sn[:, :, [0, 17], :4, :].reshape(-1, 128), fx["snap_slice"].reshape(-1, 128), 1e-4, "snaps")
    assert np.allclose(sn.astype(np.float64).sum(axis=(3, 4)), fx["snap_sum"], rtol=1e-4, atol=1e-2)
    assert np.array_equal(bits16(cso), fx["conv_state"])
