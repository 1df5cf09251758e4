"""The HIP engine against the reference fallback's golden vectors (GPU).

Fixtures (tests/golden/*.npz) hold the reference torch fallback's outputs for
tiny problems covering empty components, exact ties, the Cholesky jitter
ladder, chunked streaming over N and K and default variance initialisation.
Tolerances: parameters rtol 1e-4, lower bounds rtol 1e-5, labels exact except
near-ties (float64 logit gap < 1e-5·max(1, |logit|)), scores rtol 1e-5, responsibilities
atol 2e-4.
"""

import pytest
import torch

from oracle import torch_ref
from tests.golden_io import fixture_names, load

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _close(got, exp, tol):
    exp = exp.to(torch.float32)
    torch.testing.assert_close(got.cpu().to(torch.float32), exp, rtol=tol,
                               atol=tol * max(1.0, float(exp.abs().max())))


def _labels_ok(got, a, cov):
    exp = a["labels"]
    bad = (got.cpu() != exp).nonzero(as_tuple=False)
    if bad.numel() == 0:
        return
    mdl = torch_ref._Model(cov, a["means"].double(), a["covs"].double(), a["weights"].double())
    x = a["x"].double()
    xs = x.square().sum(-1) if cov == "spherical" else None
    logits = mdl.logits(x, xs, 0, a["means"].shape[1])
    for bi, ni in bad.tolist():
        gap = abs(float(logits[bi, ni, got[bi, ni]] - logits[bi, ni, exp[bi, ni]]))
        scale = max(1.0, abs(float(logits[bi, ni, exp[bi, ni]])))
        assert gap < 1e-5 * scale, f"label mismatch at ({bi},{ni}), logit gap {gap}"


@pytest.mark.parametrize("name", fixture_names())
def test_hip_fit_matches_golden(hip, name):
    print(f"[golden] {name}", flush=True)
    meta, a = load(name)
    cov = meta["covariance_type"]
    from gmmxx_amd import em
    labels, m, c, w, info = em.fit(
        a["x"].to(DEV), a["init_means"].shape[1], cov, max_iters=meta["fit_kwargs"]["max_iters"],
        tol=0.0, init_means=a["init_means"], init_covs=a.get("init_variances"),
        init_weights=a.get("init_weights"), reg_covar=meta["reg_covar"], record_all_lower_bounds=True)
    assert info["n_iter"] == meta["n_iter"]
    for got, exp in zip(info["lower_bound_history"], a["lower_bound_history"].tolist()):
        assert got == pytest.approx(exp, rel=1e-5, abs=1e-5)
    _close(m, a["means"], 1e-4)
    _close(c, a["covs"], 1e-4)
    _close(w, a["weights"], 1e-4)
    _labels_ok(labels, a, cov)


@pytest.mark.parametrize("name", fixture_names())
def test_hip_inference_matches_golden(hip, name):
    print(f"[golden-inf] {name}", flush=True)
    meta, a = load(name)
    cov = meta["covariance_type"]
    args = [t.to(DEV).contiguous() for t in (a["x"], a["means"], a["covs"], a["weights"])]
    scores, labels = hip.score(cov, *args)
    proba = hip.predict_proba(cov, *args)
    torch.testing.assert_close(scores.cpu(), a["score"], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(proba.cpu(), a["proba"], rtol=0, atol=2e-4)
    _labels_ok(labels, dict(a, labels=a["assign"]), cov)
