"""CPU: the committed golden fixtures (tests/golden/*.npz) are reproduced
bit for bit by the oracle and the generator, so neither can drift unnoticed,
and the fixtures agree with the hand-derived reference known answers."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
sys.path.insert(0, GOLDEN)

import make_golden  # noqa: E402


def load(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)


@pytest.mark.parametrize("name", sorted(make_golden.GROUPS))
def test_fixture_reproduces(name):
    fx = load(name)
    fresh = make_golden.build(name)
    assert sorted(fx.files) == sorted(fresh)
    for key in fresh:
        np.testing.assert_array_equal(fx[key], fresh[key], err_msg=f"{name}:{key}")


def test_quant_fixture_known_answers():
    fx = load("quant")
    assert fx["ref_per_tensor_sym_q"].reshape(-1).tolist() == [21, 42, 64, 85, 106, 127]
    assert fx["ref_per_channel_sym_q"].tolist() == [[42, 85, 127], [42, 85, 127]]
    assert fx["ref_asym_q"].tolist() == [-128, -78, -27, 25, 76, 126]
    assert int(fx["ref_asym_z"][0]) == -1
    assert int(fx["ref_activation_z"][0]) == -128
    assert fx["ties_q"].tolist() == [3, -3, 1, -1, 127, 2]


def test_gemm_fixture_fp64_bound():
    fx = load("gemm")
    for m, k, n in make_golden.GEMM_SHAPES:
        tag = f"{m}x{k}x{n}"
        a, b, c = (fx[f"{p}_{tag}"].astype(np.float64) for p in "abc")
        bound = (k + 1) * 2.0 ** -24 * (np.abs(a) @ np.abs(b))
        assert (np.abs(c - a @ b) <= bound).all()
