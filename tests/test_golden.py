"""The CPU oracle reproduces the committed golden fixtures (``tests/golden``)."""
import numpy as np
import pytest

from golden_io import fixture_names, load_fixture
from oracle import sparse_attn_fp64, sparse_attn_ref


def test_fixtures_present():
    assert len(fixture_names()) >= 4


@pytest.mark.parametrize("name", fixture_names())
def test_oracle_reproduces_fixture(name):
    f = load_fixture(name)
    args = (f["q"], f["kv"], f["sink"], f["idx"], f["scale"])
    np.testing.assert_allclose(sparse_attn_fp64(*args), f["expected_f64"],
                               rtol=1e-6, atol=1e-7)
    ref = sparse_attn_ref(*args).float().numpy()
    exp = f["expected_ref_bf16"].float().numpy()
    # bf16 outputs of an fp32 computation: equal up to one bf16 ulp
    assert np.all(np.abs(ref - exp) <= 2.0 ** -7 * np.abs(exp) + 1e-6)


@pytest.mark.parametrize("name", fixture_names())
def test_fixture_masking_properties(name):
    f = load_fixture(name)
    idx = f["idx"].numpy()
    exp = f["expected_f64"]
    all_masked = (idx == -1).all(axis=-1)
    assert np.all(exp[all_masked] == 0.0)
    assert np.all(np.isfinite(exp))
