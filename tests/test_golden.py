"""The oracle reproduces the committed fixtures (tests/golden/golden.npz)
bit-for-bit; the GPU tests compare libbq against the same fixtures."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


@pytest.fixture(scope="module")
def G():
    return dict(np.load(GOLDEN, allow_pickle=False))


def test_fixture_regenerates_exactly(O, G):
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(__file__), "golden", "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    fresh = mg.make()
    assert set(fresh) == set(G)
    for k in G:
        np.testing.assert_array_equal(np.asarray(fresh[k]), G[k], err_msg=k)


def test_fixture_internal_consistency(O, G):
    # FWHT fixtures invert (within rounding) and quant fixtures decode back
    for B in (16, 32, 64, 128, 256, 512):
        back = O.fwht_rows(G[f"fwht{B}_out"], B)
        np.testing.assert_allclose(back, G[f"fwht{B}_in"], atol=1e-5)
    np.testing.assert_array_equal(G["quant_codes"], [127, 2, 4, -2, 0, 0, 2, 64, -64, 0])
    # the MoE fixture routes are the (expert, token, k) order of its top-k table
    idx, eo = G["moe_idx"], G["moe_eo"]
    order = sorted((int(idx[t, j]), t) for t in range(idx.shape[0]) for j in range(idx.shape[1]))
    np.testing.assert_array_equal(G["moe_route_token"], [t for _, t in order])
    assert eo[-1] == idx.size
