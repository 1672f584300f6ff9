"""The C oracle against the committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from seeded inputs): every array bit for bit.  The fixtures are the
build's own anchors (the reference holds no test vectors); a change to the oracle's arithmetic or to
the seeded generators shows up here first."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)


@pytest.mark.parametrize("name", ["moe_cfg1_int8_m8", "gdn_b2_t5", "attn_t4", "lmhead_r8_v4096"])
def test_oracle_matches_fixture(oracle_mod, name):
    import make_golden
    want = np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)
    got = make_golden.FIXTURES[name](oracle_mod)
    assert set(want.files) == set(got)
    for k in want.files:
        assert np.array_equal(np.asarray(got[k]), want[k]), f"{name}.{k}"
