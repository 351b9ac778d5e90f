"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from
the float64 scalar loops of oracle/brute.py): the fixtures regenerate
bit-for-bit, and the vectorised oracle (oracle/pair_ops.py) reproduces them."""
import os

import numpy as np
import pytest

from oracle import pair_ops
from tests.golden import make_golden

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def params(g):
    return {k[len("param."):]: v for k, v in g.items() if k.startswith("param.")}


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_fixture_regenerates_bit_for_bit(name):
    fresh = make_golden.FIXTURES[name]()
    stored = load(name)
    assert sorted(fresh) == sorted(stored)
    for k, v in fresh.items():
        assert np.array_equal(np.asarray(v), stored[k]), k


@pytest.mark.parametrize("outgoing", [True, False])
def test_oracle_tri_mul_matches_golden(outgoing):
    g = load("tri_mul_n8.npz")
    y = pair_ops.tri_mul(g["z"], g["mask"], params(g), outgoing, dtype=np.float64)
    np.testing.assert_allclose(y, g["outgoing" if outgoing else "incoming"], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("starting", [True, False])
def test_oracle_tri_attn_matches_golden(starting):
    g = load("tri_attn_n8.npz")
    y = pair_ops.tri_attn(g["x"], g["mask"], params(g), starting, 4, dtype=np.float64)
    np.testing.assert_allclose(y, g["starting" if starting else "ending"], rtol=1e-10, atol=1e-12)


def test_oracle_raw_ops_match_golden():
    g = load("raw_ops_n8.npz")
    for outgoing in (True, False):
        x = pair_ops.contract(g["a"].astype(np.float64), g["b"].astype(np.float64), outgoing)
        np.testing.assert_allclose(x, g["contract_outgoing" if outgoing else "contract_incoming"],
                                   rtol=1e-12, atol=1e-12)
    for starting in (True, False):
        y = pair_ops.attention_core(g["q"], g["k"], g["v"], g["bias"], g["mask"], float(g["scale"]),
                                    starting, dtype=np.float64)
        np.testing.assert_allclose(y, g["attention_starting" if starting else "attention_ending"],
                                   rtol=1e-10, atol=1e-12)
    y = pair_ops.layer_norm(g["ln_x"].astype(np.float64), g["ln_w"], g["ln_b"])
    np.testing.assert_allclose(y, g["layer_norm"], rtol=1e-12, atol=1e-12)


def test_fixture_edge_cases_are_present():
    """The fixtures carry the reference tests' edge cases: a padded tail, an
    isolated masked pair and (attention) a row with no valid key."""
    g = load("tri_attn_n8.npz")
    m = g["mask"][0]
    assert m[6:].sum() == 0 and m[:, 6:].sum() == 0 and m[2, 4] == 0 and m[7].sum() == 0
    assert np.isfinite(g["starting"]).all() and np.isfinite(g["ending"]).all()
    r = load("raw_ops_n8.npz")
    # raw attention, starting: rows 6 and 7 have no valid key -> uniform weights,
    # so every query of such a row gets the mean of that row's v
    v = r["v"][0].astype(np.float64)                      # [H, N, N, D]
    want = v[:, 7].mean(axis=1).reshape(-1)               # [H*D], head-major
    got = r["attention_starting"][0, 7]                    # [N, H*D]
    assert np.allclose(got, want[None, :], atol=1e-12)
