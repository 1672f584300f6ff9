"""Each manifest op links from its own cuda_sources list alone (CPU, no GPU).

A loader that builds one op from manifest.toml compiles the units the op lists and nothing else
(R/manifest.toml:149: one extension per op).  This test does that: it compiles every unit once for
gfx950, links each op's list with --no-undefined, and checks that the linked library defines every
q36_* entry the op's Python modules call, found by walking the op's source module and the modules
it imports from this package.
"""
import ast
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bundles_amd")

pytestmark = pytest.mark.skipif(not os.path.exists(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")),
                                reason="hipcc is not installed")


def _manifest():
    try:
        import tomllib
    except ImportError:
        import tomli as tomllib
    with open(os.path.join(PKG, "manifest.toml"), "rb") as f:
        return tomllib.load(f)


def _module_path(dotted: str) -> str | None:
    base = os.path.join(ROOT, *dotted.split("."))
    for cand in (base + ".py", os.path.join(base, "__init__.py")):
        if os.path.exists(cand):
            return cand
    return None


def _imports(path: str, dotted: str) -> set[str]:
    """Dotted names of the package modules `path` imports (relative or absolute, at any depth)."""
    pkg = dotted.rsplit(".", 1)[0] if not path.endswith("__init__.py") else dotted
    out = set()
    for node in ast.walk(ast.parse(open(path).read())):
        if isinstance(node, ast.ImportFrom):
            if node.level:
                parts = pkg.split(".")
                base = parts[:len(parts) - (node.level - 1)]
                mod = ".".join(base + ([node.module] if node.module else []))
            else:
                mod = node.module or ""
            if not mod.startswith("bundles_amd"):
                continue
            out.add(mod)
            for a in node.names:  # `from . import moe` names a module
                if _module_path(f"{mod}.{a.name}"):
                    out.add(f"{mod}.{a.name}")
        elif isinstance(node, ast.Import):
            out |= {a.name for a in node.names if a.name.startswith("bundles_amd")}
    return out


def op_symbols(source: str) -> set[str]:
    """q36_* attributes called by the op's module and every package module it reaches."""
    start = "bundles_amd." + source[:-3].replace("/", ".")
    seen, todo, syms = set(), [start], set()
    while todo:
        mod = todo.pop()
        if mod in seen:
            continue
        seen.add(mod)
        path = _module_path(mod)
        if path is None:
            continue
        tree = ast.parse(open(path).read())
        syms |= {n.attr for n in ast.walk(tree) if isinstance(n, ast.Attribute) and n.attr.startswith("q36_")}
        todo += sorted(_imports(path, mod) - seen)
    return syms | {"q36_abi_version", "q36_last_error"}


@pytest.fixture(scope="module")
def objects(tmp_path_factory):
    from bundles_amd import build
    out = tmp_path_factory.mktemp("objs")
    srcs = sorted({s for op in _manifest()["ops"] for s in op["cuda_sources"]})
    objs = build.compile_objects([os.path.join(PKG, s) for s in srcs], str(out))
    return dict(zip(srcs, objs)), out


def test_op_symbol_walk_finds_the_entries():
    ops = {op["slot"]: op for op in _manifest()["ops"]}
    lm = op_symbols(ops["logits_processor"]["source"])
    assert {"q36_lmhead_argmax", "q36_lmhead_workspace_bytes", "q36_quant_rows_i8"} <= lm
    assert not any(s.startswith("q36_moe") for s in lm)  # the logits op does not reach the MoE
    layer = op_symbols(ops["model.layers.*"]["source"])
    assert {"q36_moe_forward", "q36_gdn_verify_ring", "q36_attn_decode", "q36_dense8_linear",
            "q36_fp8_linear", "q36_add_rmsnorm", "q36_quant_blocks_e4m3"} <= layer


@pytest.mark.parametrize("slot", ["model.layers.*", "logits_processor"])
def test_op_links_from_its_own_sources(objects, slot):
    from bundles_amd import build
    objs, out = objects
    op = next(o for o in _manifest()["ops"] if o["slot"] == slot)
    lib = str(out / f"op_{slot.split('.')[0].replace('*', 'x')}.so")
    build.link([objs[s] for s in op["cuda_sources"]], lib)  # raises on an undefined symbol
    nm = shutil.which("nm") or "/usr/bin/nm"
    defined = subprocess.run([nm, "-D", "--defined-only", lib], check=True, capture_output=True, text=True).stdout
    have = {l.split()[-1] for l in defined.splitlines() if l.split() and l.split()[-1].startswith("q36_")}
    need = op_symbols(op["source"])
    assert need <= have, f"{slot}: {sorted(need - have)} not defined by {op['cuda_sources']}"


def test_full_library_is_the_union_of_the_ops():
    from bundles_amd import build
    listed = {s for op in _manifest()["ops"] for s in op["cuda_sources"]}
    assert {os.path.relpath(s, PKG) for s in build.sources()} == listed
