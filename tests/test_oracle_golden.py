"""The CPU oracle reproduces the reference fallback's golden vectors.

Fixtures come from the reference's own ``torch_fallback`` (see
tests/golden/make_golden.py).  Both sides run torch CPU fp32 kernels in the
same order, so agreement is expected to the last few ulps.
"""

import pytest
import torch

from oracle import torch_ref
from tests.golden_io import fixture_names, load

NAMES = fixture_names()


def test_fixture_set_is_complete():
    for cov in ("spherical", "diag", "tied", "full"):
        for kind in ("basic", "chunked", "empty", "ties", "defaultvar"):
            assert f"{cov}_{kind}" in NAMES
    assert "tied_jitter" in NAMES and "full_jitter" in NAMES


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_golden(name):
    meta, a = load(name)
    cov = meta["covariance_type"]
    kw = meta["fit_kwargs"]
    labels, means, covs, w, info = torch_ref.fit(
        a["x"], a["init_means"].shape[1], cov, max_iters=kw["max_iters"], tol=0.0,
        init_means=a["init_means"], init_covs=a.get("init_variances"),
        init_weights=a.get("init_weights"), reg_covar=meta["reg_covar"],
        chunk_size_N=kw.get("chunk_size_N", 32768), chunk_size_K=kw.get("chunk_size_K", 1024))
    assert info["n_iter"] == meta["n_iter"]
    torch.testing.assert_close(means, a["means"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(covs, a["covs"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(w, a["weights"], rtol=1e-5, atol=1e-9)
    torch.testing.assert_close(torch.tensor(info["lower_bound_history"], dtype=torch.float64),
                               a["lower_bound_history"], rtol=1e-6, atol=1e-6)
    assert torch.equal(labels, a["labels"])
    ck = dict(chunk_size_N=kw.get("chunk_size_N", 32768), chunk_size_K=kw.get("chunk_size_K", 1024))
    assert torch.equal(torch_ref.assign(a["x"], a["means"], a["covs"], a["weights"], cov, **ck),
                       a["assign"])
    torch.testing.assert_close(
        torch_ref.score_samples(a["x"], a["means"], a["covs"], a["weights"], cov, **ck),
        a["score"], rtol=1e-6, atol=1e-5)
    torch.testing.assert_close(
        torch_ref.predict_proba(a["x"], a["means"], a["covs"], a["weights"], cov, **ck),
        a["proba"], rtol=1e-5, atol=1e-7)


def test_ties_pick_first_index():
    """Duplicated components produce exact ties; the first index must win."""
    for cov in ("spherical", "diag", "tied", "full"):
        _, a = load(f"{cov}_ties")
        k = a["init_means"].shape[1]
        lab = torch_ref.assign(a["x"], a["init_means"], a["init_variances"]
                               if "init_variances" in a else None,
                               torch.full((1, k), 1.0 / k), cov)
        assert int(lab.max()) < k // 2, cov


def test_record_all_lower_bounds_quirk():
    """With the quirk reproduced, non-final diag/tied/full iterations record 0.0."""
    _, a = load("diag_basic")
    _, _, _, _, info = torch_ref.fit(a["x"], 4, "diag", max_iters=3, tol=0.0,
                                     init_means=a["init_means"], init_covs=a["init_variances"],
                                     init_weights=a["init_weights"], record_all_lower_bounds=False)
    h = info["lower_bound_history"]
    assert h[0] == 0.0 and h[1] == 0.0 and h[2] != 0.0
    assert h[2] == pytest.approx(float(a["lower_bound_history"][2]), rel=1e-6)
