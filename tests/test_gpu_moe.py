"""GPU parity of the decode MoE block (libq36 through the C-ABI) against the CPU oracle.

Bar: expert ids, weights-free integer lists and int32 accumulators bit-exact; bf16 outputs within
1e-2 relative (and, by construction of the shared arithmetic, expected bit-exact for W8A8).
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bits16, bits8, elementwise_rel, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def q36():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import moe
    return moe


def _host_weights(ew):
    """Host copies for the oracle: the code tensors back in row-major order."""
    from bundles_amd.qwen36_layer.moe import unpack_frag8_np
    hw = {k: np_(getattr(ew, k)) for k in ("w13", "s13", "w2", "s2", "sw13", "ss13", "sw2", "ss2")}
    for k in ("w13", "w2", "sw13", "sw2"):
        hw[k] = unpack_frag8_np(hw[k])
    return hw


def test_quant_rows_i8_matches_oracle(q36, oracle_mod, dev):
    O = oracle_mod
    g = torch.Generator(device=dev).manual_seed(1)
    w = (torch.randn((300, 2048), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    w[7].zero_()
    w[8, 5] = 0.5 * w[8].abs().max()  # a tie at .5 after division lands exactly on the half-way rule
    q, s = q36.quantize_rows_i8(w)
    torch.cuda.synchronize()
    qo, so = O.quant_rows_i8(O.bf16_to_f32(bits16(w)))
    assert np.array_equal(np_(q), qo)
    assert np.array_equal(np_(s).view(np.uint32), so.view(np.uint32))
    assert np_(s)[7] == 0 and not np_(q)[7].any()


def test_quant_blocks_e4m3_matches_oracle(q36, oracle_mod, dev):
    O = oracle_mod
    g = torch.Generator(device=dev).manual_seed(2)
    w = (torch.randn((3, 256, 512), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    w[1, :128, :128] = 0
    q, s = q36.quantize_blocks_e4m3(w)
    torch.cuda.synchronize()
    for i in range(3):
        qo, so = O.quant_blocks_e4m3(O.bf16_to_f32(bits16(w[i])))
        assert np.array_equal(bits8(q[i]), qo)
        assert np.array_equal(np_(s[i]).view(np.uint32), so.view(np.uint32))


# past 128 rows the router takes eight experts a wave: 129 rows end in a partial 8-token group, 200 rows pad
ROUTE_CASES = [(1, False, False), (8, False, False), (64, True, False), (64, True, True), (256, False, True),
               (129, True, False), (200, True, True), (256, True, False)]


@pytest.mark.parametrize("M,zipf,padded", ROUTE_CASES)
def test_route_bit_exact(q36, oracle_mod, dev, M, zipf, padded):
    from bundles_amd import synth
    O = oracle_mod
    print(f"route M={M} zipf={zipf} padded={padded}", flush=True)
    d = synth.moe_inputs(M, dev, seed=10 + M, E=512, zipf=1.1 if zipf else None)
    pos = None
    if padded:
        pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
        pos[::5] = 0
    ws = q36.Workspace(512, 2048, 512, 10, q36.Q36_MOE_FP8, dev)
    v = q36.route(d["x"], pos, d["router_w"], 10, ws, router_bias=d["router_bias"])
    torch.cuda.synchronize()
    r = O.route(bits16(d["x"]), bits16(d["router_w"]), 10,
                bias=None if d["router_bias"] is None else np_(d["router_bias"]),
                pos=None if pos is None else np_(pos))
    assert np.array_equal(np_(v["logits"]).view(np.uint32), r["logits"].view(np.uint32))
    assert np.array_equal(np_(v["ids"]), r["ids"])
    assert np.array_equal(np_(v["wts"]).view(np.uint32), r["wts"].view(np.uint32))
    for key in ("counts", "offsets", "perm", "inv_perm"):
        assert np.array_equal(np_(v[key]), r[key]), key
    n_act = int(np_(v["ctl"])[1])
    assert n_act == r["n_active"]
    assert np.array_equal(np_(v["active"])[:n_act], r["active"][:n_act])
    assert int(np_(v["ctl"])[0]) == 0, "route ticket must be left at zero"


def test_route_tie_rule(q36, oracle_mod, dev):
    """Equal bf16 logits rank by id ascending (the tie rule of the top-k, logit desc then id asc): 13
    experts share one router row and one bias of +10, so their logits are bitwise equal and the largest
    of every token; the 10 picks of each token must be the 10 lowest of those ids in ascending order,
    as the oracle has them.  Padded rows (position 0) stay out of the lists."""
    from bundles_amd import synth
    O = oracle_mod
    M, E, k = 64, 512, 10
    print("route tie rule M=64", flush=True)
    d = synth.moe_inputs(M, dev, seed=77, E=E)
    tied = [511, 3, 300, 7, 256, 100, 255, 200, 301, 400, 450, 480, 500]
    rw = d["router_w"].clone()
    bias = torch.zeros(E, dtype=torch.float32, device=dev)
    for e in tied:
        rw[e].copy_(rw[42])
        bias[e] = 10.0
    pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
    pos[::7] = 0
    ws = q36.Workspace(E, 2048, 512, k, q36.Q36_MOE_FP8, dev)
    v = q36.route(d["x"], pos, rw, k, ws, router_bias=bias)
    torch.cuda.synchronize()
    r = O.route(bits16(d["x"]), bits16(rw), k, bias=np_(bias), pos=np_(pos))
    lg = np_(v["logits"])
    assert (lg[:, tied] == lg[:, tied[:1]]).all(), "the tied experts' logits are not equal"
    ids = np_(v["ids"])
    live = np_(pos) != 0
    assert (ids[live] == np.array(sorted(tied)[:k], dtype=np.int32)).all()
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(np_(v["wts"]).view(np.uint32), r["wts"].view(np.uint32))
    for key in ("counts", "offsets", "perm", "inv_perm"):
        assert np.array_equal(np_(v[key]), r[key]), key


def _run_moe(q36, O, dev, M, E, dtype, seed, zipf=None, padded=False, debug=True):
    from bundles_amd import synth
    d = synth.moe_inputs(M, dev, seed=seed, E=E, zipf=zipf)
    ew = q36.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], dtype)
    pos = None
    if padded:
        pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
        pos[1::4] = 0
    ws = q36.Workspace(E, 2048, 512, 10, dtype, dev)
    S = M * 10
    dbg = {"h": torch.zeros((S + M, 512), dtype=torch.bfloat16, device=dev)}
    if dtype == q36.Q36_MOE_INT8:
        dbg["acc13"] = torch.zeros((S + M, 1024), dtype=torch.int32, device=dev)
        dbg["acc2"] = torch.zeros((S + M, 2048), dtype=torch.int32, device=dev)
    out = q36.moe_row_batch(d["x"], pos, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"],
                            debug=dbg if debug else None)
    torch.cuda.synchronize()
    hw = _host_weights(ew)
    r = O.moe(dtype, bits16(d["x"]), bits16(d["router_w"]), hw["w13"], hw["s13"], hw["w2"], hw["s2"], hw["sw13"],
              hw["ss13"], hw["sw2"], hw["ss2"], bits16(d["gate_w"]), 10,
              bias=None if d["router_bias"] is None else np_(d["router_bias"]),
              pos=None if pos is None else np_(pos), debug=True)
    return out, ws.views(M), dbg, r, pos


MOE_CASES = [(1, 64, 0), (8, 64, 0), (37, 128, 0), (64, 64, 0), (1, 64, 1), (8, 64, 1), (37, 128, 1), (64, 64, 1),
             # int8 (bit-exact end to end) one token past the 16-, 32- and 64-token block edges of the expert
             # work items; the fp8 forms of such ragged batches are checked stage by stage below
             (17, 64, 0), (33, 128, 0), (65, 64, 0), (97, 64, 0)]


@pytest.mark.parametrize("M,E,dtype", MOE_CASES)
def test_moe_small_parity(q36, oracle_mod, dev, M, E, dtype):
    print(f"moe M={M} E={E} dtype={dtype}", flush=True)
    out, v, dbg, r, _ = _run_moe(q36, oracle_mod, dev, M, E, dtype, seed=100 + M)
    assert np.array_equal(np_(v["ids"]), r["ids"])
    valid = np.ones(M * 10 + M, bool)
    if dtype == q36.Q36_MOE_INT8:
        assert np.array_equal(np_(dbg["acc13"])[valid], r["acc13"][valid]), "up int32 accumulators differ"
        assert np.array_equal(bits16(dbg["h"]), r["h"]), "SwiGLU output differs"
        assert np.array_equal(np_(dbg["acc2"]), r["acc2"]), "down int32 accumulators differ"
        assert np.array_equal(bits16(out), r["out"]), "W8A8 output is expected bit-exact"
    else:
        wh, ah, eh = assert_bf16_close(bits16(dbg["h"]), r["h"], 1e-2, "fp8 h")
        wo, ao, eo = assert_bf16_close(bits16(out), r["out"], 1e-2, "fp8 out")
        print(f"fp8 h: row err {wh:.2e} elem {ah:.2e} exact {eh:.4f}; out: row err {wo:.2e} elem {ao:.2e} "
              f"exact {eo:.4f}", flush=True)


@pytest.mark.parametrize("dtype", [0, 1])
def test_moe_padded_rows(q36, oracle_mod, dev, dtype):
    out, v, dbg, r, pos = _run_moe(q36, oracle_mod, dev, 24, 64, dtype, seed=7, padded=True)
    p = np_(pos)
    assert np.array_equal(np_(v["ids"]), r["ids"])
    assert not bits16(out)[p == 0].any(), "padded rows must be zero"
    if dtype == 0:
        assert np.array_equal(bits16(out), r["out"])
    else:
        assert_bf16_close(bits16(out), r["out"], 1e-2, "fp8 out")


def test_moe_config1_int8_full(q36, oracle_mod, dev):
    """Config 1: int8 W8A8, 8 tokens, 512 experts top-10, seed 0 -- the CPU-runnable parity anchor."""
    out, v, dbg, r, _ = _run_moe(q36, oracle_mod, dev, 8, 512, 0, seed=0)
    assert np.array_equal(np_(v["ids"]), r["ids"])
    assert np.array_equal(np_(dbg["acc13"]), r["acc13"])
    assert np.array_equal(np_(dbg["acc2"]), r["acc2"])
    assert np.array_equal(bits16(out), r["out"])


@pytest.mark.parametrize("M,dtype", [(64, 1), (128, 0)])
def test_moe_unskewed_many_units(q36, oracle_mod, dev, M, dtype):
    """An unskewed router at 512 experts: several hundred active units (more active expert workgroups
    than the chip holds at once), int8 bit-exact and e4m3 within the bar."""
    print(f"moe unskewed M={M} dtype={dtype}", flush=True)
    out, v, dbg, r, _ = _run_moe(q36, oracle_mod, dev, M, 512, dtype, seed=11)
    assert np.array_equal(np_(v["ids"]), r["ids"])
    n_units = len(np.unique(r["ids"])) + 1
    assert n_units * 8 > 512, f"only {n_units} units: the case does not exceed one round of workgroups"
    _check_out(q36, dtype, dbg, out, r, "unskewed")


@pytest.mark.parametrize("M,dtype,padded", [(256, 0, False), (256, 1, False), (200, 0, True)])
def test_moe_hot_experts_many_blocks(q36, oracle_mod, dev, M, dtype, padded):
    """Zipf-skewed routing past 64 rows: the hot experts (and the shared expert) hold several 64-token
    blocks, each taken by its own expert workgroups."""
    print(f"moe hot experts M={M} dtype={dtype} padded={padded}", flush=True)
    out, v, dbg, r, pos = _run_moe(q36, oracle_mod, dev, M, 512, dtype, seed=21, zipf=1.1, padded=padded)
    assert np.array_equal(np_(v["ids"]), r["ids"])
    ids = r["ids"][r["ids"] >= 0]
    top = np.bincount(ids, minlength=512).max()
    assert top > 128, f"the hottest expert has {top} tokens: fewer than three 64-token blocks"
    if padded:
        assert not bits16(out)[np_(pos) == 0].any(), "padded rows must be zero"
    _check_out(q36, dtype, dbg, out, r, "hot experts", accs=not padded)


def _check_out(q36, dtype, dbg, out, r, what, accs=True):
    if dtype == q36.Q36_MOE_INT8:
        if accs:  # (padded rows' slots hold nothing on either side only for the output)
            assert np.array_equal(np_(dbg["acc13"]), r["acc13"]), "up int32 accumulators differ"
            assert np.array_equal(np_(dbg["acc2"]), r["acc2"]), "down int32 accumulators differ"
        assert np.array_equal(bits16(out), r["out"]), "W8A8 output is expected bit-exact"
    else:
        wo, ao, eo = assert_bf16_close(bits16(out), r["out"], 1e-2, "fp8 out")
        print(f"{what} fp8 out: row err {wo:.2e} elem {ao:.2e} exact fraction {eo:.4f}", flush=True)


def test_moe_config2_fp8_full(q36, oracle_mod, dev):
    """Config 2: e4m3 block-scaled, batch 64, 512 experts top-10, Zipf(1.1)-skewed router."""
    out, v, dbg, r, _ = _run_moe(q36, oracle_mod, dev, 64, 512, 1, seed=0, zipf=1.1)
    assert np.array_equal(np_(v["ids"]), r["ids"])
    wo, ao, eo = assert_bf16_close(bits16(out), r["out"], 1e-2, "config 2 out")
    print(f"config 2 out: row err {wo:.2e} elem {ao:.2e} exact fraction {eo:.4f}", flush=True)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_moe_config2_fp8_stages(q36, oracle_mod, dev, seed):
    """Config 2 stage by stage, three seeds: the x quantization bit-exact; the gate/up stage (h) and
    the down stage fed the GPU's own h (teacher forcing) each within the bf16 bar, with elementwise
    errors and the number of re-quantization group scales that differ reported; the combine fed the
    GPU's own weighted expert rows bit-exact; and the block end to end."""
    _fp8_stages(q36, oracle_mod, dev, 64, 512, seed, zipf=1.1, e2e=True)


@pytest.mark.parametrize("M,E,seed", [(33, 128, 133), (97, 64, 197), (17, 512, 5)])
def test_moe_fp8_stages_ragged(q36, oracle_mod, dev, M, E, seed):
    """Ragged fp8 batches (one token past a work item's 16-, 32- or 64-token edge), stage by stage with the
    same bars as config 2.  The end-to-end error is reported, not asserted: the down stage re-quantizes h
    to e4m3 per 128-group, so a one-ulp difference in h (2 % of its elements, from the MFMA's summation
    order) can move a 3-bit mantissa code or a group scale, and a row whose output nearly cancels then
    shows that step as a large relative error (33 x 128 experts, seed 133: 1.3e-2 end to end, while each
    stage alone is within its bar)."""
    _fp8_stages(q36, oracle_mod, dev, M, E, seed, zipf=None, e2e=False)


def _fp8_stages(q36, O, dev, M, E, seed, zipf, e2e):
    from bundles_amd import synth
    print(f"moe fp8 stages M={M} E={E} seed={seed}", flush=True)
    d = synth.moe_inputs(M, dev, seed=seed, E=E, zipf=zipf)
    ew = q36.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], q36.Q36_MOE_FP8)
    ws = q36.Workspace(E, 2048, 512, 10, q36.Q36_MOE_FP8, dev)
    S = M * 10
    dbg = {"h": torch.zeros((S + M, 512), dtype=torch.bfloat16, device=dev)}
    out = q36.moe_row_batch(d["x"], None, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"],
                            debug=dbg)
    torch.cuda.synchronize()
    v = ws.views(M)
    hw = _host_weights(ew)
    args = (1, bits16(d["x"]), bits16(d["router_w"]), hw["w13"], hw["s13"], hw["w2"], hw["s2"], hw["sw13"],
            hw["ss13"], hw["sw2"], hw["ss2"], bits16(d["gate_w"]), 10)
    kw = dict(bias=None if d["router_bias"] is None else np_(d["router_bias"]), debug=True)
    r = O.moe(*args, **kw)
    assert np.array_equal(np_(v["ids"]), r["ids"])
    # x quantization: e4m3 codes and per-(token, 128-group) scales
    xq, xs = O.quant_groups_e4m3(O.bf16_to_f32(bits16(d["x"])))
    assert np.array_equal(bits8(v["xq"]), xq) and np.array_equal(np_(v["xs"]).view(np.uint32), xs.view(np.uint32))
    # up + SwiGLU
    h_gpu, y_gpu = bits16(dbg["h"]), bits16(v["y"])
    up = assert_bf16_close(h_gpu, r["h"], 1e-2, "up stage h")
    # the down stage's re-quantization of h: scale of each (slot, 128-group)
    _, hs_gpu = O.quant_groups_e4m3(O.bf16_to_f32(h_gpu))
    _, hs_ref = O.quant_groups_e4m3(O.bf16_to_f32(r["h"]))
    n_scale = int(np.sum(hs_gpu.view(np.uint32) != hs_ref.view(np.uint32)))
    # down fed the GPU's h
    rd = O.moe(*args, **kw, h_in=h_gpu)
    dn = assert_bf16_close(y_gpu, rd["y"], 1e-2, "down stage y (teacher forced)")
    # combine fed the GPU's y: the same fp32 sums in the same order
    rc = O.moe(*args, **kw, y_in=y_gpu)
    assert np.array_equal(bits16(out), rc["out"]), "combine (teacher forced) must be bit-exact"
    if e2e:
        e2e = assert_bf16_close(bits16(out), r["out"], 1e-2, "config 2 out")
    else:
        g2, r2 = O.bf16_to_f32(bits16(out)).astype(np.float64), O.bf16_to_f32(r["out"]).astype(np.float64)
        row = np.linalg.norm(g2 - r2, axis=-1) / np.maximum(np.linalg.norm(r2, axis=-1), 1e-30)
        e2e = (float(row.max()), elementwise_rel(g2, r2), float(np.mean(bits16(out) == r["out"])))
    print(f"seed {seed}: h exact {up[2]:.4f} row {up[0]:.2e} elem {up[1]:.2e}; group scales differing "
          f"{n_scale}/{hs_ref.size}; down(tf) row {dn[0]:.2e} elem {dn[1]:.2e} exact {dn[2]:.4f}; "
          f"end-to-end row {e2e[0]:.2e} elem {e2e[1]:.2e} exact {e2e[2]:.4f}", flush=True)
    # elementwise bars (|g - r| / (|r| + rms of the row)): the stages one at a time are tight
    assert up[1] <= 2e-2 and dn[1] <= 2e-2, (up, dn)


@pytest.mark.parametrize("dtype", [0, 1])
def test_moe_fused_add_norm(q36, oracle_mod, dev, dtype):
    """The next block's add-norm fused into the combine gives the same bits as the block followed by
    q36_add_rmsnorm: the block output, the updated residual and the normalised rows (padding rows
    included), and matches the oracle's add-norm on the block output."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import glue
    O = oracle_mod
    M, E = 40, 64
    d = synth.moe_inputs(M, dev, seed=21 + dtype, E=E, zipf=1.1)
    ew = q36.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], dtype)
    ws = q36.Workspace(E, 2048, 512, 10, dtype, dev)
    pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
    pos[3::7] = 0
    g = synth.gen(dev, 77)
    resid0 = synth.randn((M, 2048), g, dev)
    nw = synth.randn((2048,), g, dev, 0.1)
    ref = q36.moe_row_batch(d["x"], pos, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"])
    r_ref = resid0.clone()
    y_ref = glue.add_rmsnorm(ref, r_ref, nw, 1e-6)
    r_got = resid0.clone()
    y_got = torch.empty_like(resid0)
    got = q36.moe_row_batch(d["x"], pos, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"],
                            norm=(r_got, nw, 1e-6, y_got))
    torch.cuda.synchronize()
    for a, b, what in ((got, ref, "out"), (r_got, r_ref, "residual"), (y_got, y_ref, "normed rows")):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), what
    hn, res = O.add_rmsnorm(bits16(got), bits16(resid0), bits16(nw), 1e-6)
    assert np.array_equal(bits16(y_got), hn) and np.array_equal(bits16(r_got), res)


@pytest.mark.parametrize("dtype,M", [(1, 1), (1, 2), (0, 5), (1, 24), (1, 40), (0, 64), (1, 256), (0, 131)])
def test_moe_input_add_norm(q36, oracle_mod, dev, dtype, M):
    """This block's own input add-norm run by the route kernel (pre_norm) gives the same bits as
    q36_add_rmsnorm followed by the block: the normed rows, the new residual, the block output (padding
    rows included), and with the next block's add-norm fused into the combine too, the hybrid node's
    form; the old residual is left as it was, and the oracle's add-norm agrees.  M covers every router
    shape (1, 2, 4 and 8 tokens a workgroup, two, four and eight experts a wave)."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import glue
    O = oracle_mod
    E = 512 if M in (1, 256) else 64
    d = synth.moe_inputs(M, dev, seed=31 + M, E=E, zipf=1.1)
    ew = q36.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], dtype)
    ws = q36.Workspace(E, 2048, 512, 10, dtype, dev)
    pos = torch.arange(1, M + 1, dtype=torch.int32, device=dev)
    pos[2::5] = 0
    g = synth.gen(dev, 91 + M)
    delta, resid0 = synth.randn((M, 2048), g, dev), synth.randn((M, 2048), g, dev)
    nw, nw2 = synth.randn((2048,), g, dev, 0.1), synth.randn((2048,), g, dev, 0.1)
    kw = dict(router_bias=d["router_bias"])
    r_ref = resid0.clone()
    x_ref = glue.add_rmsnorm(delta, r_ref, nw, 1e-6)
    ref = q36.moe_row_batch(x_ref, pos, d["router_w"], d["gate_w"], ew, 10, ws, **kw)
    r_in, r_out, x_got = resid0.clone(), torch.empty_like(resid0), torch.empty_like(resid0)
    got = q36.moe_row_batch(x_got, pos, d["router_w"], d["gate_w"], ew, 10, ws, **kw,
                            pre_norm=(delta, r_in, r_out, nw, 1e-6))
    r_out2 = torch.empty_like(resid0)
    got2 = q36.moe_row_batch(None, pos, d["router_w"], d["gate_w"], ew, 10, ws, **kw,
                             pre_norm=(delta, r_in, r_out2, nw, 1e-6))
    # both norms fused (the hybrid node's layer): then the next block's add-norm on the new residual
    r_ref2 = r_ref.clone()
    y_ref = glue.add_rmsnorm(ref, r_ref2, nw2, 1e-6)
    r_out3, y_got = torch.empty_like(resid0), torch.empty_like(resid0)
    got3 = q36.moe_row_batch(None, pos, d["router_w"], d["gate_w"], ew, 10, ws, **kw,
                             pre_norm=(delta, r_in, r_out3, nw, 1e-6), norm=(r_out3, nw2, 1e-6, y_got))
    torch.cuda.synchronize()
    eq = lambda a, b: torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert eq(x_got, x_ref), "normed rows"
    assert eq(r_out, r_ref) and eq(r_out2, r_ref), "new residual"
    assert eq(r_in, resid0), "the old residual is read only"
    assert eq(got, ref) and eq(got2, ref) and eq(got3, ref), "block output"
    assert eq(r_out3, r_ref2) and eq(y_got, y_ref), "the next block's add-norm after the fused one"
    hn, res = O.add_rmsnorm(bits16(delta), bits16(resid0), bits16(nw), 1e-6)
    assert np.array_equal(bits16(x_got), hn) and np.array_equal(bits16(r_out), res)


def test_moe_input_add_norm_rejects_overlap(q36, dev):
    """The route reads in_delta and in_resid while it writes in_resid_out and x: overlapping buffers
    are refused before anything is launched."""
    from bundles_amd import synth
    d = synth.moe_inputs(8, dev, seed=5, E=64, zipf=1.1)
    ew = q36.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], 1)
    ws = q36.Workspace(64, 2048, 512, 10, 1, dev)
    delta, resid = torch.zeros((8, 2048), dtype=torch.bfloat16, device=dev), torch.zeros((8, 2048), dtype=torch.bfloat16, device=dev)
    nw = torch.zeros(2048, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="overlap"):
        q36.moe_row_batch(None, None, d["router_w"], d["gate_w"], ew, 10, ws, pre_norm=(delta, resid, resid, nw, 1e-6))
    with pytest.raises(RuntimeError, match="overlap"):
        q36.moe_row_batch(delta, None, d["router_w"], d["gate_w"], ew, 10, ws,
                          pre_norm=(delta, resid, torch.empty_like(resid), nw, 1e-6))


def test_moe_repeat_deterministic(q36, dev):
    """Two calls on one workspace give identical bits (the self-resetting ticket, no races)."""
    from bundles_amd import synth
    d = synth.moe_inputs(64, dev, seed=3, E=64, zipf=1.1)
    ew = q36.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], q36.Q36_MOE_FP8)
    ws = q36.Workspace(64, 2048, 512, 10, q36.Q36_MOE_FP8, dev)
    outs = [q36.moe_row_batch(d["x"], None, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"])
            for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(outs[0].view(torch.int16), outs[2].view(torch.int16))


def test_pack_frag8_round_trip(q36, dev):
    """pack_frag8 then the host inverse gives the codes back, for int8 and e4m3 shapes of the experts."""
    from bundles_amd.qwen36_layer.moe import pack_frag8, unpack_frag8_np
    for shape in ((3, 1024, 2048), (2, 2048, 512), (48, 384)):
        q = torch.randint(-128, 128, shape, dtype=torch.int8, device=dev)
        p = pack_frag8(q)
        torch.cuda.synchronize()
        assert not torch.equal(p, q)
        assert np.array_equal(unpack_frag8_np(np_(p)), np_(q))
