"""Pins of the oracle's routing (logits, top-k, weights, expert lists) against independent numpy (CPU).

Rule (L/i8x_decode.py:98-117; L/qk_route.cu:117-192): bf16 logits, softmax in fp32, top-k by
(logit desc, id asc), weights renormalised over the k picks; padded rows (position 0) stay out.
"""
import numpy as np
import pytest


def _inputs(M, E, seed, bias=False):
    from oracle import oracle as O
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16(rng.standard_normal((M, 2048)).astype(np.float32))
    wr = O.f32_to_bf16((rng.standard_normal((E, 2048)) * 0.02).astype(np.float32))
    b = None
    if bias:
        rank = rng.permutation(E) + 1.0
        p = rank ** -1.1
        b = np.log(p / p.sum()).astype(np.float32)
    return x, wr, b


@pytest.mark.parametrize("M,E,k,bias", [(8, 512, 10, False), (64, 512, 10, True), (5, 64, 8, False)])
def test_route_against_numpy(oracle_mod, M, E, k, bias):
    O = oracle_mod
    x, wr, b = _inputs(M, E, 10 + M, bias)
    r = O.route(x, wr, k, bias=b)
    xf = O.bf16_to_f32(x).astype(np.float64)
    wf = O.bf16_to_f32(wr).astype(np.float64)
    exact = xf @ wf.T + (0 if b is None else b.astype(np.float64)[None])
    # logits: the canonical fp32 order rounds to the float64 bf16 value, or to a neighbour
    l64 = O.bf16_to_f32(O.f32_to_bf16(exact.astype(np.float32)))
    lg = r["logits"]
    step = np.abs(l64) * 2 ** -7 + 1e-30
    assert np.all(np.abs(lg - l64) <= step)
    assert np.mean(lg == l64) > 0.99
    # ids: lexicographic (logit desc, id asc) on the oracle's own logits
    ids = np.stack([np.lexsort((np.arange(E), -lg[t]))[:k] for t in range(M)])
    assert np.array_equal(r["ids"], ids)
    # weights: float64 softmax over bf16 logits, renormalised over the picks
    p = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    pk = np.take_along_axis(p, ids, axis=1)
    w64 = pk / pk.sum(axis=1, keepdims=True)
    assert np.allclose(r["wts"], w64, rtol=2e-6, atol=1e-7)
    assert np.allclose(r["wts"].sum(axis=1), 1.0, atol=1e-6)
    # lists: counting sort by (expert, token, j)
    flat = ids.reshape(-1)
    assert np.array_equal(r["counts"], np.bincount(flat, minlength=E))
    assert np.array_equal(r["offsets"], np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    order = np.lexsort((np.arange(M * k), flat))
    assert np.array_equal(r["perm"], order)
    inv = np.empty(M * k, np.int64)
    inv[order] = np.arange(M * k)
    assert np.array_equal(r["inv_perm"], inv)
    act = np.nonzero(np.bincount(flat, minlength=E))[0]
    assert r["n_active"] == act.size and np.array_equal(r["active"][:act.size], act)


def test_route_padding_and_ties(oracle_mod):
    O = oracle_mod
    M, E, k = 6, 64, 4
    x, wr, _ = _inputs(M, E, 3)
    wr[10] = wr[3]  # identical rows: equal logits, the lower id must win
    pos = np.array([5, 0, 7, 0, 9, 1], np.int32)
    r = O.route(x, wr, k, pos=pos)
    assert np.all(r["ids"][pos == 0] == -1) and np.all(r["wts"][pos == 0] == 0)
    for t in np.nonzero(pos)[0]:
        row = list(r["ids"][t])
        if 10 in row:
            assert 3 in row and row.index(3) < row.index(10)
    assert r["offsets"][-1] == k * np.count_nonzero(pos)
    assert np.all(r["perm"][r["offsets"][-1]:] == -1)
    assert np.all(r["inv_perm"].reshape(M, k)[pos == 0] == -1)
