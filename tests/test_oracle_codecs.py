"""Pins of the oracle's scalar codecs and math against independent implementations (CPU)."""
import numpy as np
import torch


def test_bf16_round_matches_torch(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s for s in (1e-30, 1e-3, 1, 1e6, 1e30)])
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, 1.0039062, 1.0117188,
                                     1.00390625, 1.01171875], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16(x)
    assert np.array_equal(got, ref)
    assert all(O.lib().q36o_f32_to_bf16(float(v)) == r for v, r in zip(x[:2000], ref[:2000]))


def test_e4m3_decode_all_codes(oracle_mod):
    O = oracle_mod
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = O.e4m3_lut()
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin])) and set(codes[~fin]) == {0x7F, 0xFF}
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_e4m3_encode_rne_and_saturation(oracle_mod):
    O = oracle_mod
    enc = O.lib().q36o_f32_to_e4m3
    lut = O.e4m3_lut()
    fin = np.sort(np.unique(np.abs(lut[np.isfinite(lut)])))
    mids = ((fin[1:].astype(np.float64) + fin[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(1)
    xs = np.concatenate([fin, mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                         rng.uniform(-447, 447, 20000).astype(np.float32),
                         (rng.standard_normal(20000) * 1e-3).astype(np.float32)])
    xs = np.concatenate([xs, -xs])
    ref = torch.from_numpy(xs).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([enc(float(v)) for v in xs], np.uint8)
    assert np.array_equal(got, ref), "round-to-nearest-even disagrees with torch below the saturation point"
    # saturation (satfinite): everything at or above 448 in magnitude, inf included, maps to +-448
    for v in (448.0, 449.0, 463.9, 464.0, 480.0, 1e6, np.inf):
        assert enc(v) == 0x7E and enc(-v) == 0xFE
    assert enc(float("nan")) & 0x7F == 0x7F
    # round trip of every finite code
    for c in range(256):
        if c & 0x7F != 0x7F:
            assert enc(float(lut[c])) == c


def test_expf_within_two_ulp(oracle_mod):
    O = oracle_mod
    xs = np.concatenate([np.linspace(-103.9, 88.7, 200001), np.linspace(-1, 1, 20001),
                         np.array([0.0, -0.0, 1e-30, -1e-30])]).astype(np.float32)
    got = np.array([O.expf(float(v)) for v in xs], np.float32)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(np.abs(ref.astype(np.float32))).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref) / ulp
    assert err.max() <= 2.0, f"max error {err.max():.2f} ulp"
    assert O.expf(0.0) == 1.0
    assert O.expf(100.0) == float("inf") and O.expf(-110.0) == 0.0
    assert np.isnan(O.expf(float("nan")))


def test_dot_canon_exact_on_integers_and_close_in_general(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(2)
    a = rng.integers(-8, 9, 2048).astype(np.float32)
    b = rng.integers(-8, 9, 2048).astype(np.float32)
    assert O.dot_canon(a, b) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))
    a = rng.standard_normal(4096).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    ref = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    assert abs(O.dot_canon(a, b) - ref) <= 1e-5 * np.sum(np.abs(a.astype(np.float64) * b))
