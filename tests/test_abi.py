"""The C-ABI boundary on the CPU: the library loads, exports every symbol include/q36_abi.h
declares, the ctypes structures match the C layout, and invalid arguments are rejected with
Q36_EINVAL and a message before anything is launched (no GPU needed)."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q36_abi.h")


@pytest.fixture(scope="module")
def L():
    from bundles_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from bundles_amd import build
        build.build()
    return _lib.lib()


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(q36_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported(L):
    from bundles_amd import _lib
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), f"{n} declared in q36_abi.h but not exported"
    bound = {s[0] for s in _lib.SYMBOLS}
    assert set(names) <= bound, f"not bound in _lib.SYMBOLS: {set(names) - bound}"
    assert L.q36_abi_version() == 7


def test_struct_layouts_match_header(tmp_path):
    from bundles_amd import _lib
    structs = {"q36_moe_args": _lib.MoeArgs, "q36_moe_ws_layout": _lib.MoeWsLayout, "q36_gdn_args": _lib.GdnArgs,
               "q36_gdn_ring_args": _lib.GdnRingArgs,
               "q36_attn_args": _lib.AttnArgs, "q36_oproj_args": _lib.OprojArgs, "q36_lmhead_args": _lib.LmheadArgs,
               "q36_decode_args": _lib.DecodeArgs, "q36_linear_seg": _lib.LinearSeg,
               "q36_fp8_linear_args": _lib.Fp8LinearArgs, "q36_add_norm_args": _lib.AddNormArgs,
               "q36_dense8_linear_args": _lib.Dense8LinearArgs}
    hdr = open(HEADER).read()
    structs = {k: v for k, v in structs.items() if f"typedef struct {k}" in hdr}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, st in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in st._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l}
    for cname, st in structs.items():
        assert got[(cname, "size")] == C.sizeof(st), cname
        for fname, _ in st._fields_:
            assert got[(cname, fname)] == getattr(st, fname).offset, f"{cname}.{fname}"


def test_invalid_arguments_are_rejected(L):
    from bundles_amd import _lib
    assert L.q36_moe_forward(None, None) == _lib.Q36_EINVAL
    a = _lib.MoeArgs()
    a.M, a.E, a.H, a.I, a.topk, a.dtype = 8, 512, 1024, 512, 10, 1
    assert L.q36_moe_forward(C.byref(a), None) == _lib.Q36_EINVAL
    assert b"H=1024" in L.q36_last_error()
    a.H, a.topk = 2048, 17
    assert L.q36_moe_route(C.byref(a), None) == _lib.Q36_EINVAL
    assert b"topk" in L.q36_last_error()
    a.topk, a.dtype = 10, 7
    assert L.q36_moe_forward(C.byref(a), None) == _lib.Q36_EINVAL
    a.dtype = 1
    assert L.q36_moe_forward(C.byref(a), None) == _lib.Q36_EINVAL  # null pointers
    # the route's input add-norm: its three row buffers are required, and what the route writes
    # (in_resid_out, x) must not overlap what it reads (host addresses: nothing is launched)
    a.router_w, a.workspace, a.in_norm_w = 0x10000, 0x20000, 0x30000
    assert L.q36_moe_route(C.byref(a), None) == _lib.Q36_EINVAL
    assert b"in_delta" in L.q36_last_error()
    a.in_delta, a.in_resid, a.in_resid_out = 0x100000, 0x200000, 0x100000 + 8 * 2048 * 2 - 16
    assert L.q36_moe_route(C.byref(a), None) == _lib.Q36_EINVAL
    assert b"overlap" in L.q36_last_error()
    a.in_resid_out, a.x = 0x300000, 0x200000 + 4096
    assert L.q36_moe_route(C.byref(a), None) == _lib.Q36_EINVAL
    assert b"overlap" in L.q36_last_error()
    g = _lib.GdnArgs()
    g.B, g.T = 2, 9
    assert L.q36_gdn_verify(C.byref(g), None) == _lib.Q36_EINVAL
    assert b"T=9" in L.q36_last_error()
    gr = _lib.GdnRingArgs()
    gr.B, gr.T = 2, 9
    assert L.q36_gdn_verify_ring(C.byref(gr), None) == _lib.Q36_EINVAL
    assert b"T=9" in L.q36_last_error()
    gr.T = 4
    assert L.q36_gdn_verify_ring(C.byref(gr), None) == _lib.Q36_EINVAL  # null pointers
    assert b"null" in L.q36_last_error()
    gr.B = 0
    assert L.q36_gdn_verify_ring(C.byref(gr), None) == _lib.Q36_OK  # an empty batch launches nothing
    d = _lib.DecodeArgs()
    d.B, d.NT, d.HQ, d.HKV, d.D = 4, 4, 32, 4, 128
    assert L.q36_attn_decode(C.byref(d), None) == _lib.Q36_EINVAL
    assert b"HQ=32" in L.q36_last_error()
    d.HQ, d.HKV, d.D, d.NT = 16, 2, 256, 5
    assert L.q36_attn_decode(C.byref(d), None) == _lib.Q36_EINVAL
    assert b"NT=5" in L.q36_last_error()
    d.NT = 4
    assert L.q36_attn_decode(C.byref(d), None) == _lib.Q36_EINVAL  # null pointers
    f = _lib.Fp8LinearArgs()
    f.T, f.N, f.K, f.n_out = 4, 256, 1024, 256
    assert L.q36_fp8_linear(C.byref(f), None) == _lib.Q36_EINVAL
    assert b"K=1024" in L.q36_last_error()
    f.K, f.N = 2048, 200
    assert L.q36_fp8_linear(C.byref(f), None) == _lib.Q36_EINVAL
    assert b"N=200" in L.q36_last_error()
    n = _lib.AddNormArgs()
    n.T, n.H = 4, 4096
    assert L.q36_add_rmsnorm(C.byref(n), None) == _lib.Q36_EINVAL
    assert b"H=4096" in L.q36_last_error()


def test_workspace_layout_is_consistent(L):
    from bundles_amd import _lib
    for M in (1, 8, 64, 256):
        lay = _lib.MoeWsLayout()
        assert L.q36_moe_workspace_layout(M, 512, 2048, 512, 10, 1, C.byref(lay)) == 0
        total = L.q36_moe_workspace_bytes(M, 512, 2048, 512, 10, 1)
        assert lay.total == total
        offs = [getattr(lay, f) for f, _ in lay._fields_ if f != "total"]
        assert all(o % 256 == 0 for o in offs) and max(offs) < total
        assert lay.ctl == 0
