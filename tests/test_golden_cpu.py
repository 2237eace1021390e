"""The oracle still reproduces the committed golden fixtures (CPU)."""

import os

import numpy as np
import pytest
import torch

from oracle import gsa_oracle as orc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
import importlib.util  # noqa: E402

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)


@pytest.mark.parametrize("name", sorted(mg.CASES))
def test_layer_fixture(name):
    z = np.load(os.path.join(HERE, f"{name}.npz"))
    got = mg.make_case(*mg.CASES[name])
    assert str(got["wdigest"]) == str(z["wdigest"])
    for key in ("x", "scores", "idx", "mask", "idx_asc", "count", "attn", "y"):
        assert np.array_equal(got[key], z[key]), key


def test_selector_fixture():
    z = np.load(os.path.join(HERE, "select_ties_T70.npz"))
    got = mg.ties_case()
    for key in z.files:
        assert np.array_equal(got[key], z[key]), key
