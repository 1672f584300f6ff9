"""GPU parity of the decode / verify attention over the e4m3 KV cache (q36_attn_decode through the
C-ABI) against the CPU oracle.

Bar: bf16 outputs within 1e-2 relative (per-row norm, one row = one query head of one token); the
cache rows written from out_loc are bit-exact.  Cases follow what the reference's verify path
meets: 1-token decode and 4-token drafts, key counts that are not multiples of the 64-key tile,
requests shorter than a tile, more splits than tiles, scattered one-token pages, peaked softmax."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bits16, bits8

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 2, 256
SCALE = 1.0 / 16.0


@pytest.fixture(scope="module")
def attn():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import attn_fused
    return attn_fused


def _e4m3(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float8_e4m3fn).view(torch.uint8)


def _make(B, NT, seqlens, seed, qscale=1.0, extra_slots=16):
    """Host tensors: q bf16 [B*NT, 16, 256], caches e4m3 [slots, 2, 256], a page table that gives each
    request distinct slots in random order (so consecutive keys sit in unrelated cache rows)."""
    g = torch.Generator().manual_seed(seed)
    slots = int(sum(seqlens)) + extra_slots
    q = (torch.randn((B * NT, HQ, D), generator=g) * qscale).to(torch.bfloat16)
    kc = _e4m3(torch.randn((slots, HKV, D), generator=g))
    vc = _e4m3(torch.randn((slots, HKV, D), generator=g))
    perm = torch.randperm(slots, generator=g).to(torch.int32)
    L = max(seqlens) + 3
    pt = torch.zeros((B, L), dtype=torch.int32)
    o = 0
    for b, n in enumerate(seqlens):
        pt[b, :n] = perm[o:o + n]
        o += n
    return dict(q=q, kc=kc, vc=vc, pt=pt, seqlens=torch.tensor(seqlens, dtype=torch.int32), perm=perm, used=o)


def _run(attn, h, NT, dev, splits=0, **kw):
    B = h["seqlens"].shape[0]
    ws = attn.DecodeWorkspace(B, dev, splits=splits)
    d = {k: h[k].to(dev) for k in ("q", "kc", "vc", "pt", "seqlens")}
    out = attn.attn_decode(d["q"], d["kc"], d["vc"], d["pt"], d["seqlens"], NT, SCALE, ws, **kw)
    torch.cuda.synchronize()
    return out, d


def _oracle(O, h, NT):
    return O.attn_decode(bits16(h["q"]), bits8(h["kc"]), bits8(h["vc"]), h["pt"].numpy(), h["seqlens"].numpy(), NT,
                         SCALE)


def _check(out, ref, what):
    got = bits16(out).reshape(-1, D)
    wr, ar, er = assert_bf16_close(got, ref.reshape(-1, D), 1e-2, what)
    print(f"{what}: row err {wr:.2e} elem {ar:.2e} exact {er:.4f}", flush=True)
    return wr


@pytest.mark.parametrize("NT,seqlens,splits", [
    (1, [1, 63, 64, 65, 300], 0),
    (1, [4096], 0),
    (4, [4, 5, 67, 128, 1000], 0),
    (4, [4, 5, 67, 128, 1000], 1),
    (4, [4, 5, 67, 128, 1000], 3),
    (4, [4, 5, 67, 128, 1000], 64),
    (2, [2, 130, 777], 0),
    (3, [3, 64, 129], 5),
    # the one-row-tile form (NT <= 2, two stages) with splits: waves of zero, one or a few steps
    (1, [1, 2, 33, 97, 2049], 7),
    (2, [2, 3, 65, 4096], 64),
])
def test_decode_parity(attn, oracle_mod, dev, NT, seqlens, splits):
    print(f"attn_decode NT={NT} seqlens={seqlens} splits={splits}", flush=True)
    h = _make(len(seqlens), NT, seqlens, seed=7 * NT + len(seqlens) + splits)
    out, _ = _run(attn, h, NT, dev, splits=splits)
    _check(out, _oracle(oracle_mod, h, NT), f"decode NT={NT} splits={splits}")


def test_decode_peaked_softmax(attn, oracle_mod, dev):
    """Scores of std ~4 (q scaled by 4): the weights span many binades, so the online rescale and
    the f16 rounding of P matter."""
    print("attn_decode peaked", flush=True)
    h = _make(2, 4, [2000, 3001], seed=11, qscale=4.0)
    out, _ = _run(attn, h, 4, dev)
    _check(out, _oracle(oracle_mod, h, 4), "decode peaked")


def test_decode_peaked_softmax_one_row_tile(attn, oracle_mod, dev):
    """The peaked case in the one-row-tile form (NT = 1 and 2: two waves a SIMD, two stages), whose
    lazy rescale runs on its own accumulators."""
    for NT, seqlens in ((1, [1500, 2500, 4096]), (2, [700, 3001])):
        print(f"attn_decode peaked NT={NT}", flush=True)
        h = _make(len(seqlens), NT, seqlens, seed=13 + NT, qscale=4.0)
        out, _ = _run(attn, h, NT, dev)
        _check(out, _oracle(oracle_mod, h, NT), f"decode peaked NT={NT}")


def test_decode_bench_shape(attn, oracle_mod, dev):
    """The bench workload's shape: 32 requests x 4 draft tokens over 4096 cached keys each."""
    print("attn_decode B=32 NT=4 ctx=4096", flush=True)
    h = _make(32, 4, [4096] * 32, seed=5)
    out, _ = _run(attn, h, 4, dev)
    _check(out, _oracle(oracle_mod, h, 4), "decode bench shape")
    out2, _ = _run(attn, h, 4, dev)
    assert torch.equal(out, out2), "two runs of the same inputs differ"


def test_decode_config5_batch(attn, oracle_mod, dev):
    """The decode leg's literal batch: 256 sequences x 1 new token over 4096 cached keys each (1 Mi
    cache rows, 512 MB a cache, made on the GPU).  Every request runs; the oracle checks a strided
    sixteenth of them (requests 0, 16, .., 240 plus the last) on their own rows of the cache."""
    B, NT, L = 256, 1, 4096
    print(f"attn_decode B={B} NT={NT} ctx={L}", flush=True)
    g = torch.Generator(device=dev).manual_seed(55)
    slots = B * L + 64
    kc = torch.empty((slots, HKV, D), dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    for c in (kc, vc):
        for i in range(0, slots, 1 << 17):
            n = min(1 << 17, slots - i)
            c[i:i + n] = _e4m3(torch.randn((n, HKV, D), generator=g, device=dev))
    q = torch.randn((B * NT, HQ, D), generator=g, device=dev).to(torch.bfloat16)
    pt = torch.randperm(slots, generator=g, device=dev)[:B * L].to(torch.int32).view(B, L).contiguous()
    seqlens = torch.full((B,), L, dtype=torch.int32, device=dev)
    ws = attn.DecodeWorkspace(B, dev)
    out = attn.attn_decode(q, kc, vc, pt, seqlens, NT, SCALE, ws)
    torch.cuda.synchronize()
    sub = list(range(0, B, 16)) + [B - 1]
    rows = pt[sub].reshape(-1).long()
    h = dict(q=q.view(B, NT, HQ, D)[sub].reshape(-1, HQ, D).cpu(), kc=kc[rows].cpu(), vc=vc[rows].cpu(),
             pt=torch.arange(len(sub) * L, dtype=torch.int32).view(len(sub), L),
             seqlens=torch.full((len(sub),), L, dtype=torch.int32))
    ref = _oracle(oracle_mod, h, NT)
    got = out.view(B, NT, HQ, D)[sub].reshape(-1, HQ, D)
    _check(got, ref, f"decode B={B} ctx={L} (strided subset of {len(sub)})")
    assert torch.isfinite(out.float()).all()
    del kc, vc


def test_decode_writes_new_rows_first(attn, oracle_mod, dev):
    """out_loc: the new tokens' K/V rows land in their slots (bit-exact, other rows untouched) and
    the attention sees them; slots past the cache are skipped."""
    print("attn_decode out_loc", flush=True)
    NT, seqlens = 4, [4, 70, 513]
    h = _make(len(seqlens), NT, seqlens, seed=23)
    g = torch.Generator().manual_seed(24)
    T = len(seqlens) * NT
    k_new = _e4m3(torch.randn((T, HKV, D), generator=g))
    v_new = _e4m3(torch.randn((T, HKV, D), generator=g))
    loc = torch.cat([h["pt"][b, n - NT:n] for b, n in enumerate(seqlens)]).to(torch.int64)
    kc0, vc0 = h["kc"].clone(), h["vc"].clone()
    dev_new = dict(out_loc=loc.to(dev), k_new=k_new.to(dev), v_new=v_new.to(dev))
    out, d = _run(attn, h, NT, dev, **dev_new)
    kc1, vc1 = d["kc"].cpu(), d["vc"].cpu()
    kc0[loc], vc0[loc] = k_new, v_new
    assert torch.equal(kc1, kc0) and torch.equal(vc1, vc0), "cache after the scatter differs"
    h2 = dict(h, kc=kc0, vc=vc0)
    _check(out, _oracle(oracle_mod, h2, NT), "decode out_loc")
    # a slot outside the cache is skipped, the rest are written
    bad = loc.clone()
    bad[0] = h["kc"].shape[0] + 5
    out_b, d_b = _run(attn, h, NT, dev, out_loc=bad.to(dev), k_new=dev_new["k_new"], v_new=dev_new["v_new"])
    kcb = d_b["kc"].cpu()
    assert torch.equal(kcb[loc[1:]], k_new[1:]) and torch.equal(kcb[loc[0]], h["kc"][loc[0]])


def test_decode_split_counts_agree(attn, dev):
    """The split count changes only the order of the fp32 sums: outputs within 2e-3 of each other."""
    h = _make(3, 4, [900, 1500, 2100], seed=31)
    outs = [_run(attn, h, 4, dev, splits=s)[0] for s in (1, 2, 7, 64)]
    for o in outs[1:]:
        assert_bf16_close(bits16(o).reshape(-1, D), bits16(outs[0]).reshape(-1, D), 2e-3, "splits")


def test_decode_rejects_bad_shapes(attn, dev):
    h = _make(1, 4, [8], seed=1)
    ws = attn.DecodeWorkspace(1, dev)
    d = {k: h[k].to(dev) for k in ("q", "kc", "vc", "pt", "seqlens")}
    with pytest.raises(ValueError):
        attn.attn_decode(d["q"], d["kc"], d["vc"], d["pt"], d["seqlens"], 3, SCALE, ws)
    with pytest.raises(RuntimeError, match="NT=8"):
        q8 = torch.zeros((8, HQ, D), dtype=torch.bfloat16, device=dev)
        attn.attn_decode(q8, d["kc"], d["vc"], d["pt"], d["seqlens"], 8, SCALE, ws)
    with pytest.raises(RuntimeError, match="HQ=8"):
        attn.attn_decode(d["q"][:, :8].contiguous(), d["kc"], d["vc"], d["pt"], d["seqlens"], 4, SCALE, ws)
