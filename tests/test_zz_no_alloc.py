"""q36_moe_forward_static (the MoE entry that allocates nothing: its workspace is the library's own
device array) against q36_moe_forward with a caller workspace, through the C-ABI: bit for bit on two
calls in a row, the second with fewer rows, for the int8 and the fp8 experts; and its rejections."""
import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(fn, a):
    from bundles_amd import _lib
    return fn(C.byref(a), _lib.stream_handle())


@pytest.mark.parametrize("dtype", [0, 1])
def test_static_matches_workspace_entry(dev, dtype):
    from bundles_amd import _lib, synth
    from bundles_amd.qwen36_layer import moe
    L = _lib.lib()
    E = 128
    d = synth.moe_inputs(256, dev, seed=11 + dtype, E=E, zipf=1.1)
    ew = moe.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], dtype)
    ws = moe.Workspace(E, 2048, 512, 10, dtype, dev)
    for M in (200, 37):  # the second call is smaller: stale rows of the first must not leak
        x = d["x"][:M].contiguous()
        pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
        pos[M // 3] = 0  # one padding row
        ref = torch.empty_like(x)
        got = torch.full_like(x, float("nan"))
        a = moe._args(x, pos, d["router_w"], d["gate_w"], ew, 10, ws, ref, d["router_bias"], None)
        assert _call(L.q36_moe_forward, a) == 0
        b = moe._args(x, pos, d["router_w"], d["gate_w"], ew, 10, ws, got, d["router_bias"], None)
        b.workspace, b.workspace_bytes = None, 0
        rc = _call(L.q36_moe_forward_static, b)
        assert rc == 0, L.q36_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"M={M}"
        assert not got[M // 3].any()


def test_static_rejections(dev):
    from bundles_amd import _lib, synth
    from bundles_amd.qwen36_layer import moe
    L = _lib.lib()
    d = synth.moe_inputs(8, dev, seed=3, E=1024)
    ws = moe.Workspace(1024, 2048, 512, 10, 1, dev, max_tokens=8)
    out = torch.empty_like(d["x"])
    a = moe._args(d["x"], None, d["router_w"], d["gate_w"], None, 10, ws, out, None, None)
    a.dtype, a.M, a.topk = 1, 256, 16  # 256 rows x 17 slots need more than the static scratch
    a.workspace, a.workspace_bytes = None, 0
    assert _call(L.q36_moe_forward_static, a) == 1
    assert b"scratch" in L.q36_last_error()
    a.M = 8
    a.workspace, a.workspace_bytes = ws.buf.data_ptr(), ws.buf.numel()  # a caller workspace is refused
    assert _call(L.q36_moe_forward_static, a) == 1
