"""GPU tests of the ``GMMXX(backend="hip")`` estimator surface against the CPU
oracle.

The estimator draws its initial means from data rows with the device RNG
after ``torch.manual_seed(seed)`` (gmmxx/interface.py:1285-1287,
torch_fallback.py:1384-1387).  The tests redraw the same rows the same way,
hand the resulting initial parameters to the oracle, and compare.  Tolerances
as in test_hip_parity: lower bounds rtol 1e-5, parameters rtol 1e-4 (with a
cancellation floor for covariances, below), labels equal (well-separated
blobs, no near-ties at these sizes).
"""

import math

import pytest
import torch

from gmmxx_amd import GMMXX, em
from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def blobs(b, n, d, k, seed, spread=6.0):
    g = torch.Generator().manual_seed(seed)
    centers = (torch.rand((b, k, d), generator=g) * 2 - 1) * spread
    lab = torch.randint(0, k, (b, n), generator=g)
    return torch.gather(centers, 1, lab[..., None].expand(-1, -1, d)) + torch.randn((b, n, d), generator=g)


def estimator_init(x_dev, cov, k, seed, reg=1e-6):
    """The estimator's initial parameters, redrawn with the same device RNG."""
    torch.manual_seed(seed)
    torch.cuda.manual_seed_all(seed)
    means, covs, weights, _ = em.initialize(x_dev, cov, k, reg_covar=reg)
    return means.cpu(), covs.cpu(), weights.cpu()


@pytest.mark.parametrize("cov,b,n,d,k", [
    ("spherical", 1, 6000, 16, 6),
    ("diag", 2, 5000, 8, 5),
    ("tied", 1, 5000, 12, 4),
    ("full", 2, 4000, 6, 3),
    ("full", 1, 6000, 36, 3),    # D > 16: whitening kernels
])
def test_fit_matches_oracle(cov, b, n, d, k):
    x = blobs(b, n, d, k, seed=11)
    data = x if b > 1 else x[0]
    est = GMMXX(n_components=k, covariance_type=cov, max_iter=4, tol=0.0, random_state=7, backend="hip")
    est.fit(data.to(DEV))
    assert est.last_backend_used_ == "hip"
    m0, c0, w0 = estimator_init(x.to(DEV), cov, k, 7)
    # reference bookkeeping of lower_bound_history_ (0.0 before the last
    # iteration for diag/tied/full with tol = 0)
    labels, means, covs, weights, info = torch_ref.fit(
        x, k, cov, max_iters=4, tol=0.0, init_means=m0, init_covs=c0, init_weights=w0,
        record_all_lower_bounds=False)
    sq = (lambda t: t[0]) if b == 1 else (lambda t: t)
    assert est.means_.shape == sq(means).shape
    torch.testing.assert_close(est.means_.cpu(), sq(means), rtol=1e-4, atol=1e-4)
    # Covariances are E[x²] - μ² differences: besides rtol 1e-4 they get an
    # absolute floor of 3e-5·mean(x²), the size of fp32 cancellation noise in
    # that difference (summation order differs between the two sides).
    cancel = 3e-5 * float(x.square().mean())
    torch.testing.assert_close(est.covariances_.cpu(), sq(covs), rtol=1e-4, atol=cancel)
    torch.testing.assert_close(est.weights_.cpu(), sq(weights), rtol=1e-4, atol=1e-7)
    torch.testing.assert_close(torch.tensor(est.lower_bound_history_), torch.tensor(info["lower_bound_history"]),
                               rtol=1e-5, atol=0.0)
    assert est.n_iter_ == 4
    assert torch.equal(est.labels_.cpu(), sq(labels))

    # inference on fresh data with the fitted parameters
    xt = blobs(b, 3000, d, k, seed=12)
    datat = (xt if b > 1 else xt[0]).to(DEV)
    fm, fc, fw = est.means_b.cpu(), est.covariances_b.cpu(), est.weights_b.cpu()
    ref_scores = torch_ref.score_samples(xt, fm, fc, fw, cov)
    ref_labels = torch_ref.assign(xt, fm, fc, fw, cov)
    ref_proba = torch_ref.predict_proba(xt, fm, fc, fw, cov)
    torch.testing.assert_close(est.score_samples(datat).cpu(), sq(ref_scores), rtol=1e-5, atol=1e-4)
    assert torch.equal(est.predict(datat).cpu(), sq(ref_labels))
    # The oracle computes predict_proba in float64.  An fp32 computation carries an
    # error of order 2⁻²⁴·|logit| in every logit difference, which on a row far from
    # all components (log-likelihood in the hundreds: a Mahalanobis term ≈ 750 at
    # D = 36 here) exceeds 1e-4 of the responsibilities; the bar adds that floor per
    # row, 16·2⁻²⁴·|score|·p, on top of rtol 1e-4 and atol 1e-5.
    pr = sq(ref_proba)
    tol = 1e-5 + 1e-4 * pr + 16 * 2.0 ** -24 * sq(ref_scores).abs()[..., None] * pr
    err = (est.predict_proba(datat).cpu() - pr).abs()
    assert bool((err <= tol).all()), (float((err - tol).max()), int((err > tol).sum()))
    # score_samples right after predict_proba on the same tensor reuses that E-step's scores
    torch.testing.assert_close(est.score_samples(datat).cpu(), sq(ref_scores), rtol=1e-5, atol=1e-4)
    est.predict_proba(datat)
    datat.mul_(1.5)                       # an in-place change invalidates the kept scores
    torch.testing.assert_close(est.score_samples(datat).cpu(),
                               sq(torch_ref.score_samples(xt * 1.5, fm, fc, fw, cov)), rtol=1e-5, atol=1e-4)
    datat.div_(1.5)
    assert math.isclose(est.score(datat), float(ref_scores.mean()), rel_tol=1e-5)
    n_par = est._n_parameters(b)
    bic = -2.0 * float(ref_scores.double().sum()) + n_par * math.log(b * 3000)
    assert math.isclose(est.bic(datat), bic, rel_tol=1e-5)


@pytest.mark.parametrize("cov", ["spherical", "diag"])
def test_bf16_input_computes_in_fp32_by_default(cov):
    """Half-precision input without dtype= is computed in fp32, as the
    reference's estimator does (gmmxx/interface.py:426-433): the fit must match
    the oracle's fp32 fit on the same (bf16-representable) values to the fp32
    bars -- lower bounds rtol 1e-5, parameters rtol 1e-4."""
    x = blobs(1, 8192, 32, 8, seed=3)[0].to(torch.bfloat16)
    est = GMMXX(k=8, max_iter=4, tol=0.0, random_state=1, covariance_type=cov, backend="hip").fit(x.to(DEV))
    assert est.means_.dtype == torch.float32
    xf = x.float()[None]
    m0, c0, w0 = estimator_init(xf.to(DEV), cov, 8, 1)
    labels, means, covs, weights, info = torch_ref.fit(xf, 8, cov, max_iters=4, tol=0.0, init_means=m0,
                                                       init_covs=c0, init_weights=w0, record_all_lower_bounds=False)
    torch.testing.assert_close(torch.tensor(est.lower_bound_history_), torch.tensor(info["lower_bound_history"]),
                               rtol=1e-5, atol=0.0)
    torch.testing.assert_close(est.means_.cpu(), means[0], rtol=1e-4, atol=1e-4)
    cancel = 3e-5 * float(xf.square().mean())
    torch.testing.assert_close(est.covariances_.cpu(), covs[0], rtol=1e-4, atol=cancel)
    torch.testing.assert_close(est.weights_.cpu(), weights[0], rtol=1e-4, atol=1e-7)
    assert torch.equal(est.labels_.cpu(), labels[0])


def test_bf16_engine_with_explicit_dtype():
    """dtype=torch.bfloat16 selects the spherical bf16 engine (x kept in bf16,
    means in bf16 as the reference keeps them), judged against the oracle's
    bf16-means trajectory from the same initial parameters: the per-iteration
    log-likelihood within the bf16 bar 2e-3, parameters within 2e-3 relative
    plus 2e-3 of their scale (means one bf16 ulp more), labels as the parity
    tests judge them (the HIP kernel under the oracle's final parameters)."""
    from tests.test_hip_parity import assert_bf16_means, assert_labels
    from gmmxx_amd import _hip
    x = blobs(1, 8192, 32, 8, seed=3)[0].to(torch.bfloat16)
    est = GMMXX(k=8, max_iter=3, tol=0.0, random_state=1, dtype=torch.bfloat16, backend="hip").fit(x.to(DEV))
    assert est.means_.dtype == torch.float32
    assert torch.equal(est.means_, est.means_.to(torch.bfloat16).to(torch.float32))
    m0, c0, w0 = estimator_init(x[None].to(DEV), "spherical", 8, 1)
    xf = x.float()[None]
    labels, means, covs, weights, info = torch_ref.fit(xf, 8, "spherical", max_iters=3, tol=0.0, init_means=m0,
                                                       init_covs=c0, init_weights=w0, bf16_means=True)
    torch.testing.assert_close(torch.tensor(est.lower_bound_history_), torch.tensor(info["lower_bound_history"]),
                               rtol=2e-3, atol=0.0)
    assert_bf16_means(est.means_[None], means)
    for got, exp in ((est.covariances_, covs[0]), (est.weights_, weights[0])):
        torch.testing.assert_close(got.cpu(), exp, rtol=2e-3, atol=2e-3 * float(exp.abs().max()))
    xd = x[None].to(DEV)
    lab = _hip.score("spherical", xd, means.to(DEV), covs.to(DEV), weights.to(DEV), want_scores=False)[1]
    assert_labels(lab, xf, means, covs, weights, "spherical")


def test_fit_predict_and_cpu_input():
    x = blobs(1, 4000, 8, 4, seed=5)[0]
    est = GMMXX(k=4, max_iter=3, tol=0.0, covariance_type="diag")
    labels = est.fit_predict(x)          # CPU input is moved to the estimator's GPU
    assert labels.device.type == "cuda" and labels.dtype == torch.int64 and labels.shape == (4000,)
    assert torch.equal(labels, est.predict(x))


def test_tol_stops_early():
    x = blobs(1, 4000, 8, 4, seed=9)[0]
    est = GMMXX(k=4, max_iter=200, tol=1e-3, covariance_type="spherical").fit(x.to(DEV))
    assert est.n_iter_ < 200
    hist = est.lower_bound_history_
    assert len(hist) == est.n_iter_
    assert abs(hist[-1] - hist[-2]) < 1e-3


def test_batch_mismatch_raises():
    x = blobs(2, 1000, 4, 3, seed=1)
    est = GMMXX(k=3, max_iter=2, tol=0.0).fit(x.to(DEV))
    with pytest.raises(ValueError, match="batch size"):
        est.predict(x[0].to(DEV))
