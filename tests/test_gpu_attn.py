"""GPU parity of the fused attention projections (libq36 through the C-ABI) against the CPU oracle.

Bar: bf16 outputs (q, gate, k, v, o_proj out) within 1e-2 relative (per-row norm); the e4m3 cache
codes equal the e4m3 conversion of the kernel's own k / v rows, and decode within 2e-2 of the
oracle's (one e4m3 step is up to 1/8 relative, so a one-ulp difference in k can move a code)."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bits16, bits8, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def attn():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import attn_fused
    return attn_fused


def _setup(attn, dev, T, seed):
    from bundles_amd import synth
    d = synth.attn_inputs(T, dev, seed=seed)
    w = attn.prepare_weights(d["wqg"], d["wk"], d["wv"], d["wo"])
    d["positions"][0] = 0
    d["positions"][-1] = 32767
    return d, w


def _oracle_weights(w):
    q, s = np_(w.wqkv).astype(np.uint8), np_(w.sqkv)
    return dict(wqg=q[:8192], sqg=s[:64], wk=q[8192:8704], sk=s[64:68], wv=q[8704:], sv=s[68:72])


@pytest.mark.parametrize("T", [1, 37, 128])
def test_attn_proj_cache_append(attn, dev, T):
    """cache=(k_cache, v_cache, out_loc): the new tokens' K / V codes land in their slots, the same bytes
    as k8 / v8 (and as q36_attn_decode's out_loc would write); slots outside the cache are skipped and
    every other row is untouched; q, gate, k, v are the same bits as without the cache."""
    print(f"attn_proj cache append T={T}", flush=True)
    d, w = _setup(attn, dev, T, seed=40 + T)
    ws = attn.Workspace(T, dev)
    slots = 3 * T + 5
    g = torch.Generator(device="cpu").manual_seed(T)
    kc = torch.randint(0, 256, (slots, 2, 256), generator=g, dtype=torch.uint8).to(dev)
    vc = torch.randint(0, 256, (slots, 2, 256), generator=g, dtype=torch.uint8).to(dev)
    kc0, vc0 = kc.clone(), vc.clone()
    loc = torch.randperm(slots, generator=g)[:T].to(torch.int64)
    if T > 1:
        loc[1] = slots      # past the cache: skipped
        loc[-1] = -1        # padding: skipped
    ref = attn.attn_proj(d["x"], w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws)
    ref = {k: v.clone() for k, v in ref.items()}
    o = attn.attn_proj(d["x"], w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws,
                       cache=(kc, vc, loc.to(dev)))
    torch.cuda.synchronize()
    for key in ("q", "gate", "k", "v", "k8", "v8"):
        assert torch.equal(o[key], ref[key]), f"{key} changed with the cache append"
    ek, ev = kc0.clone(), vc0.clone()
    for t in range(T):
        s_ = int(loc[t])
        if 0 <= s_ < slots:
            ek[s_] = ref["k8"][t]
            ev[s_] = ref["v8"][t]
    assert torch.equal(kc, ek), "k_cache differs from the expected rows"
    assert torch.equal(vc, ev), "v_cache differs from the expected rows"


@pytest.mark.parametrize("T", [1, 37, 128, 256])
def test_attn_proj_parity(attn, oracle_mod, dev, T):
    O = oracle_mod
    print(f"attn_proj T={T}", flush=True)
    d, w = _setup(attn, dev, T, seed=T)
    ws = attn.Workspace(T, dev)
    o = attn.attn_proj(d["x"], w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws)
    torch.cuda.synchronize()
    ow = _oracle_weights(w)
    r = O.attn_proj(bits16(d["x"]), ow["wqg"], ow["sqg"], ow["wk"], ow["sk"], ow["wv"], ow["sv"],
                    bits16(d["q_norm_w"]), bits16(d["k_norm_w"]), 1e-6, np_(d["cos_sin"]), np_(d["positions"]))
    for key in ("q", "gate", "k", "v"):
        wr, ar, er = assert_bf16_close(bits16(o[key]).reshape(T, -1), r[key].reshape(T, -1), 1e-2, key)
        print(f"{key}: row err {wr:.2e} elem {ar:.2e} exact {er:.4f}", flush=True)
    for key, src in (("k8", "k"), ("v8", "v")):
        # the cache write is exact on the kernel's own bf16 row (e4m3 satfinite, round to nearest even)
        codes = bits8(o[key]).reshape(T, -1)
        own = O.f32_to_e4m3(O.bf16_to_f32(bits16(o[src]).reshape(T, -1)))
        assert np.array_equal(codes, own), f"{key}: codes differ from e4m3 of the kernel's own {src}"
        # against the oracle's codes: a one-ulp bf16 difference in a row can move a code by one e4m3 step
        # (up to 1/8 relative), so the decoded rows are held to 2e-2
        got = O.e4m3_to_f32(codes)
        ref = O.e4m3_to_f32(r[key].reshape(T, -1))
        assert_bf16_close(O.f32_to_bf16(got), O.f32_to_bf16(ref), 2e-2, key)
        print(f"{key}: exact codes {np.mean(codes == r[key].reshape(T, -1)):.4f}")


@pytest.mark.parametrize("T", [1, 37, 128])
def test_attn_oproj_parity(attn, oracle_mod, dev, T):
    O = oracle_mod
    print(f"attn_oproj T={T}", flush=True)
    d, w = _setup(attn, dev, T, seed=100 + T)
    ws = attn.Workspace(T, dev)
    gate = (torch.randn((T, 4096), device=dev) * 2).to(torch.bfloat16)
    out = attn.attn_oproj(d["attn"], gate, w, ws)
    torch.cuda.synchronize()
    r = O.attn_oproj(bits16(d["attn"]), bits16(gate), np_(w.wo).astype(np.uint8), np_(w.so))
    wr, ar, er = assert_bf16_close(bits16(out), r, 1e-2, "oproj")
    print(f"oproj: row err {wr:.2e} elem {ar:.2e} exact {er:.4f}", flush=True)


@pytest.mark.parametrize("T", [150, 256])
def test_attn_proj_rows_do_not_depend_on_the_batch(attn, dev, T):
    """The first 16 tokens of a T-token call equal a 16-token call (the streaming GEMM) bit for bit, q,
    gate, k, v and the cache codes: past 128 tokens the QKV takes the tiled GEMM (64-token groups at
    150, 128 at 256), whose sums run in the same order.  (From 32 to 128 tokens it takes the K-sliced
    GEMM, which adds its four K quarters apart, so its bits may differ.)  Likewise the o_proj."""
    print(f"attn_proj batch invariance T={T}", flush=True)
    d, w = _setup(attn, dev, T, seed=500 + T)
    o = attn.attn_proj(d["x"], w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"],
                       attn.Workspace(T, dev))
    o16 = attn.attn_proj(d["x"][:16].contiguous(), w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"],
                         d["positions"][:16].contiguous(), attn.Workspace(16, dev))
    gate = (torch.randn((T, 4096), device=dev) * 2).to(torch.bfloat16)
    out = attn.attn_oproj(d["attn"], gate, w, attn.Workspace(T, dev))
    out16 = attn.attn_oproj(d["attn"][:16].contiguous(), gate[:16].contiguous(), w, attn.Workspace(16, dev))
    torch.cuda.synchronize()
    for key in ("q", "gate", "k", "v", "k8", "v8"):
        assert torch.equal(o[key][:16], o16[key]), key
    assert torch.equal(out[:16], out16), "o_proj"


def test_pack_frag_layout(attn, dev):
    """q36_pack_frag8 against the documented byte map, on a ragged-looking shape."""
    N, K = 48, 384
    q = torch.randint(0, 256, (N, K), dtype=torch.uint8, device=dev)
    got = np_(attn.pack_frag(q))
    src = np_(q)
    ref = np.empty(N * K, np.uint8)
    nkb = K // 128
    for r in range(N // 16):
        for b in range(nkb):
            base = (r * nkb + b) * 2048
            for h in range(2):
                for l in range(64):
                    row, col = 16 * r + l % 16, 128 * b + 32 * (l // 16) + 16 * h
                    ref[base + h * 1024 + 16 * l: base + h * 1024 + 16 * l + 16] = src[row, col:col + 16]
    assert np.array_equal(got.reshape(-1), ref)


# ---- activations quantized by their producer kernels (the projections skip their own launch) -----------
def _same(a, b, what):
    assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b), what


@pytest.mark.parametrize("T", [1, 37, 128, 256])
def test_attn_proj_from_add_norm_codes(attn, dev, T):
    """q36_add_rmsnorm's e4m3 rows (q8) fed to q36_attn_proj (xq) give the same bits as the projection
    of the add-norm's bf16 output; the codes equal the projection's own quantization in either layout."""
    from bundles_amd.qwen36_layer import glue
    print(f"attn_proj from add-norm codes T={T}", flush=True)
    d, w = _setup(attn, dev, T, seed=300 + T)
    g = torch.Generator(device=dev).manual_seed(T)
    resid = torch.randn((T, 2048), generator=g, device=dev).to(torch.bfloat16)
    delta = torch.randn((T, 2048), generator=g, device=dev).to(torch.bfloat16)
    nw = (torch.randn(2048, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    r1, r2 = resid.clone(), resid.clone()
    h = glue.add_rmsnorm(delta, r1, nw, 1e-6)
    xq = attn.proj_rows(T, dev)
    xq.codes.fill_(0x7F)  # the padding rows must be written, not left as they were
    xq.scales.fill_(float("nan"))
    h2 = glue.add_rmsnorm(delta, r2, nw, 1e-6, q8=xq)
    ws = attn.Workspace(T, dev)
    ref = attn.attn_proj(h, w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws)
    ref = {k: v.clone() for k, v in ref.items()}
    got = attn.attn_proj(None, w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws, xq=xq)
    torch.cuda.synchronize()
    _same(h, h2, "add-norm out")
    _same(r1, r2, "residual")
    for k in ref:
        _same(got[k], ref[k], k)
    # every byte written (a quantized code is never the NaN pattern 0x7f), padding tokens' scales zero
    assert (xq.codes != 0x7F).all() and torch.isfinite(xq.scales).all() and (xq.scales[T:] == 0).all()


def test_attn_proj_from_moe_combine_codes(attn, dev):
    """The MoE's fused add-norm with norm_q8: its e4m3 rows drive q36_attn_proj to the same bits as its
    bf16 norm_out does (64 rows: fragment order)."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import moe
    M, E = 64, 64
    print("attn_proj from MoE combine codes", flush=True)
    md = synth.moe_inputs(M, dev, seed=8, E=E)
    ew = moe.prepare_experts(md["w13"], md["w2"], md["sw13"], md["sw2"], moe.Q36_MOE_FP8)
    mws = moe.Workspace(E, 2048, 512, 10, moe.Q36_MOE_FP8, dev)
    g = torch.Generator(device=dev).manual_seed(9)
    resid = torch.randn((M, 2048), generator=g, device=dev).to(torch.bfloat16)
    nw = (torch.randn(2048, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    n1, n2 = torch.empty_like(resid), torch.empty_like(resid)
    r1, r2 = resid.clone(), resid.clone()
    moe.moe_row_batch(md["x"], None, md["router_w"], md["gate_w"], ew, 10, mws, norm=(r1, nw, 1e-6, n1))
    xq = attn.proj_rows(M, dev)
    moe.moe_row_batch(md["x"], None, md["router_w"], md["gate_w"], ew, 10, mws, norm=(r2, nw, 1e-6, n2), norm_q8=xq)
    d, w = _setup(attn, dev, M, seed=77)
    ws = attn.Workspace(M, dev)
    ref = attn.attn_proj(n1, w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws)
    ref = {k: v.clone() for k, v in ref.items()}
    got = attn.attn_proj(None, w, d["q_norm_w"], d["k_norm_w"], 1e-6, d["cos_sin"], d["positions"], ws, xq=xq)
    torch.cuda.synchronize()
    _same(n1, n2, "norm_out")
    for k in ref:
        _same(got[k], ref[k], k)


@pytest.mark.parametrize("B,NT,splits", [(2, 4, 1), (4, 4, 0), (32, 1, 2)])
def test_oproj_from_decode_codes(attn, dev, B, NT, splits):
    """q36_attn_decode with the gate writes the o_proj's e4m3 input; q36_attn_oproj on it (aq) gives
    the same bits as on the bf16 attention output and gate (one split: the split kernel's epilogue;
    several: the combine's)."""
    print(f"oproj from decode codes B={B} NT={NT} splits={splits}", flush=True)
    T = B * NT
    g = torch.Generator(device=dev).manual_seed(B * 10 + NT)
    ctx = 300
    slots = B * ctx + 16
    q = torch.randn((T, 16, 256), generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn((slots, 2, 256), generator=g, device=dev).to(torch.float8_e4m3fn).view(torch.uint8)
    vc = torch.randn((slots, 2, 256), generator=g, device=dev).to(torch.float8_e4m3fn).view(torch.uint8)
    pt = torch.randperm(slots, generator=g, device=dev)[:B * ctx].to(torch.int32).view(B, ctx).contiguous()
    sl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    gate = (torch.randn((T, 4096), generator=g, device=dev) * 2).to(torch.bfloat16)
    dws = attn.DecodeWorkspace(B, dev, splits=splits)
    o1 = attn.attn_decode(q, kc, vc, pt, sl, NT, 1.0 / 16, dws)
    oq = attn.oproj_rows(T, dev)
    o2 = attn.attn_decode(q, kc, vc, pt, sl, NT, 1.0 / 16, dws, gate=gate, oq=oq)
    d, w = _setup(attn, dev, T, seed=5)
    ws = attn.Workspace(T, dev)
    ref = attn.attn_oproj(o1.view(T, -1), gate, w, ws)
    got = attn.attn_oproj(None, None, w, ws, aq=oq)
    torch.cuda.synchronize()
    _same(o1, o2, "attention out")
    _same(got, ref, "o_proj out")
