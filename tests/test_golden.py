"""The committed golden fixtures are exactly what the oracle produces, and the reference's
known-answer values hold in them.  CPU only."""

from __future__ import annotations

import importlib.util

import numpy as np
import pytest

from conftest import GOLDEN


def _builder():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module.build()


BUILT = _builder()


@pytest.mark.parametrize("name", sorted(BUILT))
def test_fixture_matches_oracle(name):
    stored = np.load(GOLDEN / f"{name}.npz")
    assert sorted(stored.files) == sorted(BUILT[name])
    for key, value in BUILT[name].items():
        np.testing.assert_array_equal(stored[key], value, err_msg=f"{name}:{key}")


def test_reference_known_answers_in_fixtures():
    ce = np.load(GOLDEN / "cross_entropy_reference_kat.npz")
    assert abs(float(ce["oracle_loss"]) - 1.2887259920) < 1e-9
    adam = np.load(GOLDEN / "adamw_reference_kat.npz")
    assert abs(float(adam["oracle_p"]) - 0.899) < 1e-8
