"""The bundle files keep the reference's schema (R/manifest.toml, R/rebuild.json), name sources
that exist, and point at entries the node modules define (CPU, no GPU)."""
import json
import os
import types

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bundles_amd")


def _toml():
    try:
        import tomllib
    except ImportError:
        import tomli as tomllib
    with open(os.path.join(PKG, "manifest.toml"), "rb") as f:
        return tomllib.load(f)


def test_manifest_schema_and_sources():
    m = _toml()
    assert set(m) >= {"bundle_id", "abi_version", "competition", "ops"}
    assert m["abi_version"] == "cacheon-op-abi-v0"
    assert set(m["competition"]) == {"target", "mode", "arena"}
    slots = {op["slot"]: op for op in m["ops"]}
    assert set(slots) == {"model.layers.*", "logits_processor"}
    for op in m["ops"]:
        assert set(op) == {"slot", "source", "entry", "prepare", "dtypes", "architectures", "cuda_sources"}
        assert op["architectures"] == ["gfx950"] and op["dtypes"] == ["bfloat16"]
        assert os.path.exists(os.path.join(PKG, op["source"])), op["source"]
        for src in op["cuda_sources"]:
            assert os.path.exists(os.path.join(PKG, src)), src


def test_manifest_entries_exist():
    import importlib
    for op in _toml()["ops"]:
        mod = importlib.import_module("bundles_amd." + op["source"][:-3].replace("/", "."))
        assert callable(getattr(mod, op["entry"])) and callable(getattr(mod, op["prepare"]))


def test_rebuild_points_at_the_build_script():
    r = json.load(open(os.path.join(PKG, "rebuild.json")))
    (step,) = r["steps"]
    assert step["type"] == "repo_python" and os.path.exists(os.path.join(ROOT, step["path"]))


def test_layer_prepare_rejects_unsupported_blocks():
    from bundles_amd.qwen36_layer import layer

    class Block:
        shared_expert = None
    class Layer:
        mlp = Block()
    with pytest.raises(RuntimeError):
        layer.prepare(Layer())


def test_layer_prepare_rejects_non_bf16_experts():
    """An fp8 or strided expert tensor is refused before anything reads it (the quantizers read bf16)."""
    import torch
    from bundles_amd.qwen36_layer import layer

    def holder(**kw):
        return types.SimpleNamespace(**kw)
    E, H, I = 64, 2048, 512
    bf = torch.bfloat16
    for w13 in (torch.zeros((E, 2 * I, H), dtype=torch.float8_e4m3fn),
                torch.zeros((E, H, 2 * I), dtype=bf).transpose(1, 2)):
        block = holder(gate=holder(weight=torch.zeros((E, H), dtype=bf), bias=None),
                       experts=holder(w13_weight=w13, w2_weight=torch.zeros((E, H, I), dtype=bf)),
                       shared_expert=holder(gate_up_proj=holder(weight=torch.zeros((2 * I, H), dtype=bf)),
                                            down_proj=holder(weight=torch.zeros((H, I), dtype=bf))),
                       shared_expert_gate=holder(weight=torch.zeros((1, H), dtype=bf)))
        with pytest.raises(RuntimeError, match="bf16"):
            layer._MoeNode(block, 1, 10, 256)


def test_row_batch_rule():
    """Only decode and target-verify batches are row batches (the MoE path treats position-0 rows as
    padding, so a prefill chunk must never reach it)."""
    from bundles_amd.qwen36_layer import layer

    class Mode:
        def __init__(self, name):
            self.name = name

        def is_decode(self):
            return self.name == "decode"

        def is_target_verify(self):
            return self.name == "verify"
    for name, want in (("decode", True), ("verify", True), ("extend", False), ("idle", False)):
        fb = types.SimpleNamespace(forward_mode=Mode(name))
        assert layer.row_batch(fb) is want
        assert layer.verify_batch(fb) is (name == "verify")
    assert not layer.row_batch(types.SimpleNamespace(positions=None)) and not layer.row_batch(None)


def test_lmhead_row_policy():
    """The lm_head arithmetic by row count (H/node.py:9-11,144-151): W8A16 below 64 rows (when the
    vocabulary is a multiple of the W8A16 tile), two terms up to 256, one term above."""
    from bundles_amd.qwen36_lmhead8 import node
    assert [node.row_mode(r) for r in (1, 63, 64, 256, 257, 4096)] == \
        ["w8a16", "w8a16", "two_term", "two_term", "one_term", "one_term"]
    assert node.row_mode(8, vocab=4112) == "two_term"
