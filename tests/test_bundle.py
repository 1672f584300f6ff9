"""The bundle files keep the reference's schema (R/manifest.toml, R/rebuild.json), name sources
that exist, and point at entries the node modules define (CPU, no GPU)."""
import json
import os

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
