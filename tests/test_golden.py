"""The committed golden fixtures are what the (pinned) oracle produces today."""

import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_fixture_reproduces(name):
    path = make_golden.path_of(name)
    assert os.path.exists(path), "missing fixture %s; run tests/golden/make_golden.py" % path
    stored = np.load(path, allow_pickle=False)
    fresh = make_golden.generate(name)
    assert sorted(stored.files) == sorted(fresh)
    for k, v in fresh.items():
        v = np.asarray(v)
        assert stored[k].dtype == v.dtype, k
        if v.dtype.kind == "f":
            np.testing.assert_allclose(stored[k], v, rtol=0, atol=1e-6, err_msg=k)
        else:
            np.testing.assert_array_equal(stored[k], v, err_msg=k)


def test_int4_fixtures_carry_edge_bytes():
    for name in ("int4_b2_n64_d128", "int4_b4_n3_d64"):
        f = np.load(make_golden.path_of(name), allow_pickle=False)
        np.testing.assert_array_equal(f["K"][:, 0, :5], np.tile(make_golden.EDGE_BYTES, (f["K"].shape[0], 1)))
        # byte 0x80 (position 0) decodes to elements (0, -8) of token 0
        np.testing.assert_array_equal(f["Kd"][:, 0, 1], -8 * f["Ks"][:, 0].astype(np.float32))
        np.testing.assert_array_equal(f["Kd"][:, 0, 0], 0)
