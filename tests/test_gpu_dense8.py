"""GPU parity of the W8A16 GEMM (libq36 through the C-ABI) against the CPU oracle: the DENSE8 linear
(q36_dense8_linear) and the lm_head's W8A16 form (q36_lmhead_argmax, Q36_LMH_W8A16); and the lm_head on
the tile-order copy of its codes (q36_lmhead_args.wq_t) against the row-major codes, in every form.

Bar: the GPU sums the bf16 x int8 products (each exact in fp32) in fp32 in its MFMA order, the oracle
sums each 128-column group exactly and rounds once, so outputs agree within the bf16 bar (worst row
relative L2 error 4e-3, most elements bit-equal); the lm_head ids are each row's first largest GPU
logit, and the logit they pick is within one bf16 step of the oracle's row maximum.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bf16_f32, bits16, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import formats, glue
    from bundles_amd.qwen36_lmhead8 import lmhead8
    return formats, glue, lmhead8


def _copy(formats, N, K, dev, seed, s_pad=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wide = torch.zeros((K // 128, N + s_pad), dtype=torch.float16, device=dev)
    q, s = formats.quant_dense8(w, s=wide[:, :N] if s_pad else None)
    return q, (wide if s_pad else s)


@pytest.mark.parametrize("T,N,K", [(1, 2048, 2048), (4, 12352, 2048), (16, 2048, 4096), (37, 4096, 2048),
                                   (64, 12352, 2048), (64, 2048, 4096)])
def test_dense8_linear_vs_oracle(mods, oracle_mod, dev, T, N, K):
    formats, glue, _ = mods
    print(f"dense8 linear T={T} N={N} K={K}", flush=True)
    q, s = _copy(formats, N, K, dev, seed=T + N + K, s_pad=32 if T == 16 else 0)
    x = torch.randn((T, K), generator=torch.Generator(device=dev).manual_seed(T), device=dev).to(torch.bfloat16)
    y = glue.dense8_linear(x, q, s)
    torch.cuda.synchronize()
    ref = oracle_mod.dense8_linear(bits16(x), np_(q), np_(s).view(np.uint16))
    worst, _, exact = assert_bf16_close(bits16(y), ref, 4e-3, "dense8 linear")
    assert exact > 0.9, f"only {exact:.3f} of the outputs bit-equal"


def test_dense8_linear_segments_gdn_in_proj(mods, oracle_mod, dev):
    """The GDN in_proj split (8192 | 4096 | 32 | 32 columns) into strided views of one buffer."""
    formats, glue, _ = mods
    T, N, K = 24, 12352, 2048
    q, s = _copy(formats, N, K, dev, seed=7)
    x = torch.randn((T, K), generator=torch.Generator(device=dev).manual_seed(8), device=dev).to(torch.bfloat16)
    big = torch.full((T, N + 64), -7.0, dtype=torch.bfloat16, device=dev)
    cols = [0, 8192, 12288, 12320]
    widths = [8192, 4096, 32, 32]
    outs = [big[:, c + 16 * i:c + 16 * i + w_] for i, (c, w_) in enumerate(zip(cols, widths))]
    glue.dense8_linear(x, q, s, segments=list(zip(cols, outs)))
    whole = glue.dense8_linear(x, q, s)
    torch.cuda.synchronize()
    got = torch.cat(outs, dim=1)
    assert torch.equal(got, whole), "segmented and whole outputs differ"
    gaps = [big[:, c + 16 * i - 16:c + 16 * i] for i, c in enumerate(cols) if i]
    assert all(torch.all(gp == -7.0) for gp in gaps), "a store landed outside its segment"
    ref = oracle_mod.dense8_linear(bits16(x), np_(q), np_(s).view(np.uint16))
    assert_bf16_close(bits16(whole), ref, 4e-3, "dense8 segments")


def test_dense8_linear_rejects_bad_shapes(mods, dev):
    formats, glue, _ = mods
    q, s = _copy(formats, 64, 2048, dev, seed=1)
    with pytest.raises(RuntimeError, match="T=65"):
        glue.dense8_linear(torch.zeros((65, 2048), dtype=torch.bfloat16, device=dev), q, s)
    with pytest.raises(ValueError):
        glue.dense8_linear(torch.zeros((4, 1024), dtype=torch.bfloat16, device=dev), q, s)


# 1-8 rows take 32-row waves; 9-24 rows and 33-64 rows 64-row waves when V % 64 == 0 (4128 is not:
# 32-row waves); 25-32 rows 128-row waves when V % 128 == 0 (4160 is not: 64-row waves)
@pytest.mark.parametrize("R,V,norm", [(1, 4096, True), (16, 151936, True), (24, 8192, True), (12, 4128, False),
                                      (37, 8192, False), (64, 4096, True), (32, 8192, True), (29, 4160, False),
                                      (48, 4128, True)])
def test_lmhead_w8a16_vs_oracle(mods, oracle_mod, dev, R, V, norm):
    from bundles_amd import synth
    _, _, lmh = mods
    print(f"lmhead W8A16 R={R} V={V} norm={norm}", flush=True)
    d = synth.lmhead_inputs(R, V, dev, seed=R + V + 1)
    q, s = lmh.quantize_rows(d["w"])
    ws = lmh.Workspace(R, dev)
    nw = d["norm_w"] if norm else None
    ids, logits = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=nw, eps=1e-6, want_logits=True, w8a16=True)
    torch.cuda.synchronize()
    rid, rlog = oracle_mod.lmhead(bits16(d["h"]), bits16(nw) if norm else None, 1e-6, np_(q), np_(s),
                                  want_logits=True, w8a16=True)
    got = bits16(logits)
    _, _, exact = assert_bf16_close(got, rlog, 4e-3, "W8A16 logits")
    assert exact > 0.9, f"only {exact:.3f} of the logits bit-equal"
    g = bf16_f32(got)
    r = bf16_f32(rlog)
    assert np.array_equal(np_(ids), np.argmax(g, axis=1)), "ids are not the first largest GPU logit"
    rmax = r.max(axis=1)
    picked = r[np.arange(R), np_(ids)]
    assert np.all(rmax - picked <= np.abs(rmax) * 2 ** -7 + 1e-6), "an id's logit is below the oracle maximum"
    agree = np.mean(np_(ids) == rid)
    assert agree >= 0.9, f"ids agree on {agree:.2f} of the rows"


@pytest.mark.parametrize("R,V,norm", [(1, 151936, True), (16, 8192, False), (24, 8192, True), (37, 4128, True),
                                      (64, 4096, False), (32, 151936, True), (48, 8192, False)])
def test_lmhead_w8a16_tiled_copy_same_bits(mods, dev, R, V, norm):
    """The W8A16 lm_head on the tile-order copy (tile_rows_w16, what the logits node keeps) gives the
    row-major codes' ids and bf16 logits bit for bit, across the 32-, 64- and 128-row wave shapes; the copy
    is the stated permutation (a torch reshape of the same definition)."""
    from bundles_amd import synth
    _, _, lmh = mods
    print(f"lmhead W8A16 tiled R={R} V={V} norm={norm}", flush=True)
    d = synth.lmhead_inputs(R, V, dev, seed=3 * R + V)
    q, s = lmh.quantize_rows(d["w"])
    qt = lmh.tile_rows_w16(q)
    ws = lmh.Workspace(R, dev)
    nw = d["norm_w"] if norm else None
    ids, logits = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=nw, eps=1e-6, want_logits=True, w8a16=True)
    ids2, logits2 = lmh.w8a8_lmhead_argmax(d["h"], None, s, ws, norm_w=nw, eps=1e-6, want_logits=True, w8a16=True,
                                           q_t=qt)
    torch.cuda.synchronize()
    want = q.view(V // 16, 16, 2048 // 64, 4, 16).permute(0, 2, 3, 1, 4).reshape(V, 2048)
    assert torch.equal(qt, want), "tile order"
    assert torch.equal(ids, ids2)
    assert torch.equal(logits.view(torch.int16), logits2.view(torch.int16))


# the W8A8 GEMM forms on the tile-order copy: one term (ids only, bf16 and f32 logits) and two terms
@pytest.mark.parametrize("R,V,two_term,logits", [(256, 151936, False, None), (64, 4096, False, "bf16"),
                                                 (300, 8192, True, None), (128, 4160, False, "f32"),
                                                 (256, 8192, True, "bf16"), (2048, 4096, False, None)])
def test_lmhead_w8a8_tiled_copy_same_bits(mods, dev, R, V, two_term, logits):
    """Every W8A8 form reads the tile-order copy (q_t) in place of the row-major codes and gives the same ids
    and logits bit for bit (the same products summed in the same MFMA order); a copy of the wrong shape is
    refused before anything is launched."""
    from bundles_amd import synth
    _, _, lmh = mods
    print(f"lmhead W8A8 tiled R={R} V={V} two_term={two_term} logits={logits}", flush=True)
    d = synth.lmhead_inputs(R, V, dev, seed=5 * R + V)
    q, s = lmh.quantize_rows(d["w"])
    qt = lmh.tile_rows_w16(q)
    ws = lmh.Workspace(R, dev)

    def run(qq, qtt):
        out = None
        if logits is not None:
            out = torch.full((R, V), -3.0, device=dev,
                             dtype=torch.float32 if logits == "f32" else torch.bfloat16)
        ids = torch.full((R,), -1, dtype=torch.int32, device=dev)
        lmh.w8a8_lmhead_argmax(d["h"], qq, s, ws, norm_w=d["norm_w"], eps=1e-6, ids=ids, two_term=two_term,
                               logits=out, q_t=qtt)
        return ids, out

    ids, out = run(q, None)
    ids2, out2 = run(None, qt)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2), "ids"
    assert int(ids.min()) >= 0
    if logits is not None:
        iv = torch.int32 if logits == "f32" else torch.int16
        assert torch.equal(out.view(iv), out2.view(iv)), "logits"
    with pytest.raises(ValueError):
        lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, q_t=qt[: V - 32])


@pytest.mark.parametrize("T,N,K", [(1, 12352, 2048), (16, 2048, 4096), (37, 384, 2048)])
def test_dense8_tiled_copy_same_bits(dev, T, N, K):
    """formats.tile_w16 is the stated permutation of the rows (checked against a torch reshape of the
    same definition), and the linear on the tiled copy gives the row-major copy's bits."""
    from bundles_amd.qwen36_layer import formats, glue
    print(f"dense8 tiled T={T} N={N} K={K}", flush=True)
    g = torch.Generator(device=dev).manual_seed(N + T)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((T, K), generator=g, device=dev).to(torch.bfloat16)
    q, s = formats.quant_dense8(w)
    qt = formats.tile_w16(q)
    # piece (row tile i, column step j) at (i * K/64 + j) KB; row r, columns 16 g .. of it at 16 (r + 16 g)
    want = q.view(N // 16, 16, K // 64, 4, 16).permute(0, 2, 3, 1, 4).contiguous().view(N, K)
    y0 = glue.dense8_linear(x, q, s)
    y1 = glue.dense8_linear(x, qt, s, tiled=True)
    torch.cuda.synchronize()
    assert torch.equal(qt, want)
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
