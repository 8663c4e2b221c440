"""The committed known-answer fixtures (tests/golden/) against the builders
that wrote them: every case must regenerate bit for bit, so a change to the
case recipes, the expected-value arithmetic or numpy's generator shows up
here rather than silently moving both sides of a parity test.  The oracle
and the GPU kernel are checked against the fixtures in test_oracle_kats.py
and test_decode_gpu.py (the golden_* cases)."""

import os
import sys

import numpy as np
import pytest

import golden_cases
import kat_cases

sys.path.insert(0, golden_cases.GOLDEN_DIR)
import make_golden  # noqa: E402


def test_every_case_has_a_fixture():
    names = {os.path.basename(p) for p in golden_cases.fixture_paths()}
    assert names == {f"kat_{b.__name__}.npz" for b in kat_cases.ALL}


@pytest.mark.parametrize("builder", kat_cases.ALL, ids=lambda f: f.__name__)
def test_fixture_regenerates(builder):
    path = os.path.join(golden_cases.GOLDEN_DIR, f"kat_{builder.__name__}.npz")
    z = np.load(path, allow_pickle=False)
    fresh = make_golden.case_arrays(builder())
    assert set(z.files) == set(fresh)
    for k, v in fresh.items():
        np.testing.assert_array_equal(z[k], v, err_msg=f"{builder.__name__}: {k}")
