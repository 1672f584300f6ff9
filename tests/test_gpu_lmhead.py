"""GPU parity of the int8 lm_head + argmax (libq36 through the C-ABI) against the CPU oracle.

Bar: int8 activations, logits (exact: int32 accumulation and two IEEE products; two terms: the int32
accumulators of both terms, one fma and one product) and argmax ids bit-exact.  The W8A16 form (fp32
accumulation of exact products in the MFMA's order) is judged in test_gpu_dense8.py."""
import numpy as np
import pytest
import torch

from helpers import bits16, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lmh():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_lmhead8 import lmhead8
    return lmhead8


def _setup(lmh, dev, R, V, seed):
    from bundles_amd import synth
    d = synth.lmhead_inputs(R, V, dev, seed=seed)
    q, s = lmh.quantize_rows(d["w"])
    return d, q, s


@pytest.mark.parametrize("R,V,norm", [(1, 2048, True), (37, 4096, True), (256, 8192, False), (300, 4112, True),
                                      (1024, 4112, True), (1536, 2320, False)])
def test_lmhead_logits_and_ids_exact(lmh, oracle_mod, dev, R, V, norm):
    O = oracle_mod
    print(f"lmhead R={R} V={V} norm={norm}", flush=True)
    d, q, s = _setup(lmh, dev, R, V, seed=R + V)
    ws = lmh.Workspace(R, dev)
    nw = d["norm_w"] if norm else None
    ids, logits = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=nw, eps=1e-6, want_logits=True)
    torch.cuda.synchronize()
    rid, rlog = O.lmhead(bits16(d["h"]), bits16(nw) if norm else None, 1e-6, np_(q), np_(s), want_logits=True)
    assert np.array_equal(bits16(logits), rlog), "logits differ"
    assert np.array_equal(np_(ids), rid), "argmax ids differ"


@pytest.mark.parametrize("R,V,norm", [(1, 2048, True), (64, 4096, True), (100, 4112, False), (256, 8192, True),
                                      (300, 2320, True)])
def test_lmhead_two_term_logits_and_ids_exact(lmh, oracle_mod, dev, R, V, norm):
    O = oracle_mod
    print(f"lmhead two-term R={R} V={V} norm={norm}", flush=True)
    d, q, s = _setup(lmh, dev, R, V, seed=3 * R + V)
    ws = lmh.Workspace(R, dev)
    nw = d["norm_w"] if norm else None
    ids, logits = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=nw, eps=1e-6, want_logits=True, two_term=True)
    torch.cuda.synchronize()
    rid, rlog = O.lmhead(bits16(d["h"]), bits16(nw) if norm else None, 1e-6, np_(q), np_(s), want_logits=True,
                         two_term=True)
    assert np.array_equal(bits16(logits), rlog), "two-term logits differ"
    assert np.array_equal(np_(ids), rid), "two-term argmax ids differ"


@pytest.mark.parametrize("R,two", [(64, False), (300, False), (100, True)])
def test_lmhead_full_vocab_logits(lmh, oracle_mod, dev, R, two):
    """The full 151936 vocabulary with the logits stored: each persistent workgroup walks several
    tiles (the next tile's loads in flight across the epilogue, the alternating scale buffers), and
    every logit and id is compared."""
    O = oracle_mod
    V = 151936
    print(f"lmhead full vocab logits R={R} two_term={two}", flush=True)
    d, q, s = _setup(lmh, dev, R, V, seed=R + 11)
    ws = lmh.Workspace(R, dev)
    ids, logits = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=d["norm_w"], eps=1e-6, want_logits=True,
                                         two_term=two)
    torch.cuda.synchronize()
    rid, rlog = O.lmhead(bits16(d["h"]), bits16(d["norm_w"]), 1e-6, np_(q), np_(s), want_logits=True, two_term=two)
    assert np.array_equal(bits16(logits), rlog), "logits differ"
    assert np.array_equal(np_(ids), rid), "argmax ids differ"


def test_lmhead_full_vocab(lmh, oracle_mod, dev):
    O = oracle_mod
    R, V = 64, 151936
    d, q, s = _setup(lmh, dev, R, V, seed=5)
    ws = lmh.Workspace(R, dev)
    ids = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=d["norm_w"], eps=1e-6)
    torch.cuda.synchronize()
    rid, _ = O.lmhead(bits16(d["h"]), bits16(d["norm_w"]), 1e-6, np_(q), np_(s))
    assert np.array_equal(np_(ids), rid)


def test_lmhead_config5_rows_subset(lmh, oracle_mod, dev):
    """Config 5: 2048 rows (256 sequences x 8 positions) x 151936; 64 rows checked on the CPU."""
    O = oracle_mod
    R, V = 2048, 151936
    d, q, s = _setup(lmh, dev, R, V, seed=0)
    ws = lmh.Workspace(R, dev)
    ids = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, norm_w=d["norm_w"], eps=1e-6)
    torch.cuda.synchronize()
    rows = np.concatenate([np.arange(0, 8), np.arange(R - 8, R), np.random.default_rng(0).choice(R, 48, False)])
    rid, _ = O.lmhead(np.ascontiguousarray(bits16(d["h"])[rows]), bits16(d["norm_w"]), 1e-6, np_(q), np_(s))
    assert np.array_equal(np_(ids)[rows], rid)


def test_lmhead_ties_pick_first_index(lmh, dev):
    R, V = 8, 2048
    d, q, s = _setup(lmh, dev, R, V, seed=9)
    q[1000] = q[17]
    s[1000] = s[17]
    q[2047] = q[17]
    s[2047] = s[17]
    ws = lmh.Workspace(R, dev)
    ids, logits = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, want_logits=True)
    torch.cuda.synchronize()
    lg = logits.float().cpu().numpy()
    assert np.array_equal(np_(ids), lg.argmax(axis=1))  # numpy argmax = first maximal index


@pytest.mark.parametrize("R,mode", [(16, "w8a16"), (64, "two_term"), (300, "one_term"), (300, "two_term")])
def test_lmhead_fp32_logits_buffer(lmh, dev, R, mode):
    """logits into an fp32 buffer (stock's next_token_logits_buffer, H/node.py:68-88): the same
    bf16-rounded values as the bf16 output, widened, and the same ids, in every arithmetic form."""
    V = 4096
    print(f"lmhead fp32 logits R={R} mode={mode}", flush=True)
    d, q, s = _setup(lmh, dev, R, V, seed=900 + R)
    ws = lmh.Workspace(R, dev)
    kw = dict(two_term=mode == "two_term", w8a16=mode == "w8a16")
    ids16, lg16 = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, want_logits=True, **kw)
    buf = torch.full((R, V), float("nan"), dtype=torch.float32, device=dev)
    ids32, lg32 = lmh.w8a8_lmhead_argmax(d["h"], q, s, ws, logits=buf, **kw)
    torch.cuda.synchronize()
    assert lg32.data_ptr() == buf.data_ptr()
    assert torch.equal(lg32, lg16.float()) and torch.equal(ids32, ids16)
