"""Two streams, two workspaces: the entries hold no state outside their arguments, so calls with
separate workspaces on two streams, launched alternately and running side by side, give the bits
each gives alone.  (Calls that share one workspace must be ordered by the caller; that case is not
run here.)  Both streams are created with the default priority.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

ROUNDS = 3


@pytest.fixture(scope="module")
def lib():
    from bundles_amd import _lib
    _lib.lib()


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t


def _side_by_side(what, make_call, n=2):
    """make_call(i) -> (call(stream) -> list of outputs) for job i; each job runs alone first, then
    the jobs run ROUNDS times on their own streams, launched alternately with no wait between."""
    print(f"streams: {what}", flush=True)
    calls = [make_call(i) for i in range(n)]
    alone = [[o.clone() for o in c(torch.cuda.current_stream())] for c in calls]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(n)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    results = [[] for _ in range(n)]
    for _ in range(ROUNDS):
        for i, (c, s) in enumerate(zip(calls, streams)):
            with torch.cuda.stream(s):
                results[i].append(c(s))
    torch.cuda.synchronize()
    for i in range(n):
        for r, outs in enumerate(results[i]):
            for k, (a, b) in enumerate(zip(outs, alone[i])):
                assert torch.equal(_bits(a), _bits(b)), f"{what}: job {i} round {r} output {k}"


def test_streams_moe_forward(lib, dev):
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import moe
    dt = moe.Q36_MOE_FP8
    d = synth.moe_inputs(64, dev, seed=51, E=64, zipf=1.1)
    ew = moe.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], dt)
    xs = [d["x"], torch.randn((48, 2048), device=dev).to(torch.bfloat16)]

    def make(i):
        ws = moe.Workspace(64, 2048, 512, 10, dt, dev, max_tokens=64)

        def call(s):
            return [moe.moe_row_batch(xs[i], None, d["router_w"], d["gate_w"], ew, 10, ws,
                                      router_bias=d["router_bias"], stream=s)]
        return call

    _side_by_side("moe fp8, 64 and 48 tokens", make)


def test_streams_lmhead_argmax(lib, dev):
    from bundles_amd import synth
    from bundles_amd.qwen36_lmhead8 import lmhead8 as lmh
    V = 8192
    d = synth.lmhead_inputs(256, V, dev, seed=52)
    q, s = lmh.quantize_rows(d["w"])
    qt = lmh.tile_rows_w16(q)
    hs = [d["h"], torch.randn((100, 2048), device=dev).to(torch.bfloat16)]

    def make(i):
        ws = lmh.Workspace(256, dev)

        def call(st):
            ids, logits = lmh.w8a8_lmhead_argmax(hs[i], None, s, ws, norm_w=d["norm_w"], eps=1e-6, q_t=qt,
                                                 two_term=i == 1, want_logits=True, stream=st)
            return [ids, logits]
        return call

    _side_by_side("lm_head one term 256 rows and two terms 100 rows", make)


def test_streams_decode_attention(lib, dev):
    from bundles_amd.qwen36_layer import attn_fused
    g = torch.Generator().manual_seed(53)
    B, NT = 8, 4
    seqlens = torch.randint(NT, 900, (B,), generator=g, dtype=torch.int32)
    slots = int(seqlens.sum())
    e4 = lambda t: t.to(torch.float8_e4m3fn).view(torch.uint8)
    kc = e4(torch.randn((slots, 2, 256), generator=g)).to(dev)
    vc = e4(torch.randn((slots, 2, 256), generator=g)).to(dev)
    perm = torch.randperm(slots, generator=g).to(torch.int32)
    pt = torch.zeros((B, int(seqlens.max())), dtype=torch.int32)
    o = 0
    for b in range(B):
        n = int(seqlens[b])
        pt[b, :n] = perm[o:o + n]
        o += n
    pt, seqlens = pt.to(dev), seqlens.to(dev)
    qs = [torch.randn((B * NT, 16, 256), generator=g).to(torch.bfloat16).to(dev) for _ in range(2)]

    def make(i):
        ws = attn_fused.DecodeWorkspace(B, dev)

        def call(s):
            return [attn_fused.attn_decode(qs[i], kc, vc, pt, seqlens, NT, 1.0 / 16.0, ws, stream=s)]
        return call

    _side_by_side("decode attention 8 x 4", make)
