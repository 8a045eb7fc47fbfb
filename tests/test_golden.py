"""The committed golden fixtures (tests/golden/golden.npz, written by
tests/golden/gen_golden.py) reproduced by the oracle bit for bit (CPU), and
the fixture input generator checked against its definition. The same
fixtures are the GPU parity anchor in test_gpu_golden.py.
"""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT

sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import cases  # noqa: E402
import vectors as V  # noqa: E402

GOLDEN = np.load(os.path.join(ROOT, "tests", "golden", "golden.npz"))


def expected(name):
    pre = name + "/"
    return {k[len(pre):]: GOLDEN[k] for k in GOLDEN.files if k.startswith(pre)}


def test_generator_definition():
    """splitmix64 known answers (seed 0: first outputs of the published
    algorithm), uniform in (0,1), normal moments."""
    z = V.splitmix64(0, 3)
    assert [int(v) for v in z] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    u = V.uniform(5, (100000,))
    assert u.min() > 0 and u.max() < 1 and abs(u.mean() - 0.5) < 0.01
    n = V.normal(6, (200000,))
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1) < 0.01


@pytest.mark.parametrize("name", list(V.CASES))
def test_oracle_reproduces_fixture(name):
    want = expected(name)
    got = cases.oracle_outputs(name, V.CASES[name]())
    assert set(got) == set(want)
    for k, w in want.items():
        g = np.asarray(got[k])
        assert g.dtype == w.dtype and g.shape == w.shape, (name, k)
        if w.dtype.kind == "U":
            assert str(g) == str(w), (name, k)
        else:
            assert np.array_equal(np.atleast_1d(g).view(np.uint8), np.atleast_1d(w).view(np.uint8)), (name, k)


def test_oracle_model_tokens():
    import esdecode as E
    assert np.array_equal(cases.oracle_model_tokens(E), GOLDEN["model/tokens"])
