"""Pins the CPU oracle with checks that do not restate its own formulas.

* logits / scores / responsibilities: float64 Gaussian log densities from
  scipy.stats (independent implementation), per covariance type;
* one EM step: scikit-learn's GaussianMixture (independent textbook EM) with
  warm-started parameters; sklearn adds ``reg_covar`` where the reference
  clamps to it, so a tiny ``reg_covar`` is used and the two agree; with
  ``bf16_means`` the means are sklearn's rounded to bf16 (half an ulp) and the
  variances and weights sklearn's;
* the Cholesky jitter ladder: a matrix whose first successful jitter is known
  in closed form, plus the batch-global retry;
* finalize: hand-computed known answers restated from the reference's tests
  (tests/test_cuda_spherical_safe.py:151-179, tests/test_cuda_diag_safe.py:153-189,
  tests/test_cuda_soft_em_non_spherical.py:95-132) under the torch-fallback
  conventions (weight floor 1e-8 and renormalisation instead of w=0);
* invariants: EM never decreases the log-likelihood, responsibilities sum to 1;
* approximate top-k statistics: a float64 brute force over sorted scipy logits,
  hard assignment at top_k = 1, exact EM at top_k = K - 1 when the dropped
  component is unreachable.
"""

import math
import warnings

import numpy as np
import pytest
import torch
from scipy.special import logsumexp
from scipy.stats import multivariate_normal

from oracle import torch_ref

COVS = ("spherical", "diag", "tied", "full")


def _problem(cov, b=2, n=60, d=4, k=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((b, n, d), generator=g) * 2.0
    means = torch.randn((b, k, d), generator=g) * 2.0
    if cov == "spherical":
        covs = torch.rand((b, k), generator=g) + 0.5
    elif cov == "diag":
        covs = torch.rand((b, k, d), generator=g) + 0.5
    else:
        shape = (b, d, d) if cov == "tied" else (b, k, d, d)
        a = torch.randn(shape, generator=g) * 0.5
        covs = a @ a.transpose(-1, -2) + 0.5 * torch.eye(d)
    w = torch.rand((b, k), generator=g) + 0.1
    w = w / w.sum(-1, keepdim=True)
    return x.float(), means.float(), covs.float(), w.float()


def _full_cov(cov, covs, bi, ki, d):
    c = covs.double().numpy()
    if cov == "spherical":
        return np.eye(d) * c[bi, ki]
    if cov == "diag":
        return np.diag(c[bi, ki])
    if cov == "tied":
        return c[bi]
    return c[bi, ki]


def _ref_logits64(cov, x, means, covs, w):
    b, n, d = x.shape
    k = means.shape[1]
    out = np.zeros((b, n, k))
    for bi in range(b):
        for ki in range(k):
            out[bi, :, ki] = math.log(float(w[bi, ki])) + multivariate_normal(
                means[bi, ki].double().numpy(), _full_cov(cov, covs, bi, ki, d)).logpdf(
                x[bi].double().numpy())
    return out


@pytest.mark.parametrize("cov", COVS)
def test_logits_scores_proba_vs_float64(cov):
    x, means, covs, w = _problem(cov)
    ref = _ref_logits64(cov, x, means, covs, w)
    mdl = torch_ref._Model(cov, means, covs, w)
    x_sq = x.square().sum(-1) if cov == "spherical" else None
    got = mdl.logits(x, x_sq, 0, means.shape[1]).double().numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-4)
    lse = logsumexp(ref, axis=-1)
    np.testing.assert_allclose(torch_ref.score_samples(x, means, covs, w, cov).double().numpy(),
                               lse, rtol=2e-5, atol=2e-4)
    np.testing.assert_allclose(torch_ref.predict_proba(x, means, covs, w, cov).double().numpy(),
                               np.exp(ref - lse[..., None]), atol=2e-4)
    np.testing.assert_array_equal(torch_ref.assign(x, means, covs, w, cov).numpy(),
                                  ref.argmax(-1))


def _precisions_init(cov, covs):
    c = covs[0].double().numpy()
    if cov in ("spherical", "diag"):
        return 1.0 / c
    if cov == "tied":
        return np.linalg.inv(c)
    return np.stack([np.linalg.inv(m) for m in c])


@pytest.mark.parametrize("cov", COVS)
def test_one_em_step_vs_sklearn(cov):
    from sklearn.exceptions import ConvergenceWarning
    from sklearn.mixture import GaussianMixture

    x, means, covs, w = _problem(cov, b=1, n=400, d=3, k=3, seed=3)
    reg = 1e-9
    _, m1, c1, w1, info = torch_ref.fit(x, 3, cov, max_iters=1, tol=0.0, init_means=means,
                                        init_covs=covs, init_weights=w, reg_covar=reg,
                                        compute_labels=False)
    gm = GaussianMixture(n_components=3, covariance_type=cov, max_iter=1, tol=0.0, reg_covar=reg,
                         means_init=means[0].double().numpy(),
                         weights_init=(w[0].double() / w[0].double().sum()).numpy(),
                         precisions_init=_precisions_init(cov, covs))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", ConvergenceWarning)
        gm.fit(x[0].double().numpy())
    np.testing.assert_allclose(m1[0].double().numpy(), gm.means_, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(w1[0].double().numpy(), gm.weights_, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(c1[0].double().numpy(), gm.covariances_, rtol=2e-4, atol=2e-5)
    assert info["lower_bound_history"][0] == pytest.approx(gm.lower_bound_, rel=1e-5)


def test_bf16_means_one_step_vs_sklearn():
    """bf16 input's means (``bf16_means``): one spherical step from bf16-valued
    means gives bf16 values within half a bf16 ulp of sklearn's float64 means,
    and sklearn's variances (about the unrounded mean) and weights."""
    from sklearn.exceptions import ConvergenceWarning
    from sklearn.mixture import GaussianMixture

    x, means, covs, w = _problem("spherical", b=1, n=400, d=3, k=3, seed=3)
    means = means.to(torch.bfloat16).to(torch.float32)
    reg = 1e-9
    _, m1, c1, w1, info = torch_ref.fit(x, 3, "spherical", max_iters=1, tol=0.0, init_means=means,
                                        init_covs=covs, init_weights=w, reg_covar=reg,
                                        compute_labels=False, bf16_means=True)
    gm = GaussianMixture(n_components=3, covariance_type="spherical", max_iter=1, tol=0.0, reg_covar=reg,
                         means_init=means[0].double().numpy(),
                         weights_init=(w[0].double() / w[0].double().sum()).numpy(),
                         precisions_init=_precisions_init("spherical", covs))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", ConvergenceWarning)
        gm.fit(x[0].double().numpy())
    assert torch.equal(m1, m1.to(torch.bfloat16).to(torch.float32))
    ref = torch.from_numpy(gm.means_)
    _, e = torch.frexp(ref)
    half_ulp = torch.ldexp(torch.ones_like(ref), e - 9)     # |v| in [2^(e-1), 2^e): ulp 2^(e-8)
    assert bool(((m1[0].double() - ref).abs() <= half_ulp * 1.001 + 1e-6).all())
    assert not torch.equal(m1[0].double(), ref)             # the rounding is visible at this size
    np.testing.assert_allclose(w1[0].double().numpy(), gm.weights_, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(c1[0].double().numpy(), gm.covariances_, rtol=2e-4, atol=2e-5)
    assert info["lower_bound_history"][0] == pytest.approx(gm.lower_bound_, rel=1e-5)


def test_precision_logdet_spd_vs_float64():
    _, _, covs, _ = _problem("full", b=2, k=3, d=5)
    p, ld = torch_ref.precision_and_logdet(covs)
    c = covs.double()
    torch.testing.assert_close(p.double(), torch.linalg.inv(c), rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(ld.double(), torch.linalg.slogdet(c)[1], rtol=1e-5, atol=1e-5)


def test_jitter_ladder_closed_form_and_batch_global():
    """diag(1, 1, -1e-3) first factorises at jitter 1e-2 (1e-6..1e-3 leave a
    non-positive pivot); the ladder is batch-global, so a healthy matrix in the
    same batch gets the same jitter."""
    bad = torch.diag(torch.tensor([1.0, 1.0, -1e-3]))
    good = torch.diag(torch.tensor([2.0, 3.0, 4.0]))
    p, ld = torch_ref.precision_and_logdet(torch.stack([bad, good]))
    exp_bad = torch.diag(torch.tensor([1.01, 1.01, 0.009], dtype=torch.float64))
    exp_good = torch.diag(torch.tensor([2.01, 3.01, 4.01], dtype=torch.float64))
    torch.testing.assert_close(p[0].double(), torch.linalg.inv(exp_bad), rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(p[1].double(), torch.linalg.inv(exp_good), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ld.double(), torch.logdet(torch.stack([exp_bad, exp_good])),
                               rtol=1e-4, atol=1e-4)


def test_finalize_spherical_known_answer():
    nk = torch.tensor([[5.0, 0.0]])
    sum_x = torch.tensor([[[10.0, 20.0], [0.0, 0.0]]])
    sum_q = torch.tensor([[150.0, 0.0]])
    old_m = torch.tensor([[[0.0, 0.0], [99.0, 99.0]]])
    old_v = torch.tensor([[1.0, 42.0]])
    m, v, w = torch_ref.finalize("spherical", nk, sum_x, sum_q, old_m, old_v, n=5)
    torch.testing.assert_close(m[0, 0], torch.tensor([2.0, 4.0]))
    assert float(v[0, 0]) == pytest.approx(5.0, abs=1e-5)       # (150 - 5*20) / (5*2)
    torch.testing.assert_close(m[0, 1], old_m[0, 1])             # inactive: keep old
    assert float(v[0, 1]) == 42.0
    assert float(w[0, 1]) == pytest.approx(1e-8, rel=1e-3)      # floor, then renormalise
    assert float(w.sum()) == pytest.approx(1.0, abs=1e-7)
    # reg clamp: raw variance 0 -> reg_covar.
    _, v2, _ = torch_ref.finalize("spherical", torch.tensor([[1.0]]), torch.tensor([[[1.0, 1.0]]]),
                                  torch.tensor([[2.0]]), torch.zeros(1, 1, 2), torch.zeros(1, 1),
                                  n=1, reg_covar=1e-3)
    assert float(v2[0, 0]) == pytest.approx(1e-3, abs=1e-9)


def test_finalize_diag_known_answer():
    nk = torch.tensor([[5.0, 0.0]])
    sum_x = torch.tensor([[[10.0, 20.0], [0.0, 0.0]]])
    sum_q = torch.tensor([[[60.0, 90.0], [0.0, 0.0]]])
    old_m = torch.tensor([[[0.0, 0.0], [99.0, 99.0]]])
    old_v = torch.tensor([[[1.0, 1.0], [42.0, 42.0]]])
    m, v, w = torch_ref.finalize("diag", nk, sum_x, sum_q, old_m, old_v, n=5)
    torch.testing.assert_close(m[0, 0], torch.tensor([2.0, 4.0]))
    torch.testing.assert_close(v[0, 0], torch.tensor([8.0, 2.0]))   # (60/5-4, 90/5-16)
    torch.testing.assert_close(v[0, 1], old_v[0, 1])
    _, v2, _ = torch_ref.finalize("diag", torch.tensor([[1.0]]), torch.tensor([[[1.0, 1.0]]]),
                                  torch.tensor([[[1.0, 1.0]]]), torch.zeros(1, 1, 2),
                                  torch.ones(1, 1, 2), n=1, reg_covar=1e-3)
    torch.testing.assert_close(v2[0, 0], torch.tensor([1e-3, 1e-3]))


def test_finalize_full_fractional_counts():
    target = torch.tensor([[[1.0, 0.0], [0.0, 1.0]]])
    nk = torch.tensor([[0.5, 1.5]])
    sum_x = nk.unsqueeze(-1) * target
    eye = torch.eye(2).view(1, 1, 2, 2)
    sum_xx = nk[:, :, None, None] * (0.25 * eye + target.unsqueeze(-1) * target.unsqueeze(-2))
    m, c, w = torch_ref.finalize("full", nk, sum_x, sum_xx, torch.full_like(target, 99.0),
                                 eye.expand(1, 2, 2, 2).clone(), n=2, reg_covar=1e-6)
    torch.testing.assert_close(m, target)
    torch.testing.assert_close(c, (0.25 + 1e-6) * eye.expand(1, 2, 2, 2), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(w, torch.tensor([[0.25, 0.75]]))


def test_finalize_tied_closed_form():
    # Two components at (±1, 0) with 2 points each at (±1, ±1): XᵀX = diag(4, 4).
    nk = torch.tensor([[2.0, 2.0]])
    sum_x = torch.tensor([[[2.0, 0.0], [-2.0, 0.0]]])
    total_xx = torch.diag(torch.tensor([4.0, 4.0])).unsqueeze(0)
    m, c, w = torch_ref.finalize("tied", nk, sum_x, None, torch.zeros(1, 2, 2),
                                 torch.eye(2).unsqueeze(0), n=4, reg_covar=0.0, total_xx=total_xx)
    torch.testing.assert_close(m, torch.tensor([[[1.0, 0.0], [-1.0, 0.0]]]))
    torch.testing.assert_close(c, torch.diag(torch.tensor([0.0, 1.0])).unsqueeze(0))
    torch.testing.assert_close(w, torch.tensor([[0.5, 0.5]]))


@pytest.mark.parametrize("cov", COVS)
def test_em_invariants(cov):
    x, means, covs, w = _problem(cov, b=2, n=300, d=3, k=4, seed=7)
    _, m, c, wt, info = torch_ref.fit(x, 4, cov, max_iters=8, tol=0.0, init_means=means,
                                      init_covs=covs, init_weights=w)
    h = info["lower_bound_history"]
    for a, b in zip(h, h[1:]):
        assert b >= a - 1e-4 * abs(a)
    torch.testing.assert_close(wt.sum(-1), torch.ones(2), atol=1e-6, rtol=0)
    p = torch_ref.predict_proba(x, m, c, wt, cov)
    torch.testing.assert_close(p.sum(-1), torch.ones(2, 300), atol=1e-5, rtol=0)


def _topk_stats64(cov, x, logits64, top_k):
    """Brute force in float64: per row, sort the logits (value descending, then
    index ascending), keep the first top_k, normalise over them and scatter."""
    b, n, d = x.shape
    k = logits64.shape[-1]
    xn = x.double().numpy()
    nk, sx = np.zeros((b, k)), np.zeros((b, k, d))
    sq = {"spherical": np.zeros((b, k)), "diag": np.zeros((b, k, d)), "full": np.zeros((b, k, d, d))}.get(cov)
    ll = 0.0
    for bi in range(b):
        for i in range(n):
            keep = sorted(range(k), key=lambda j: (-logits64[bi, i, j], j))[:top_k]
            v = logits64[bi, i, keep]
            lse = float(logsumexp(v))
            ll += lse
            row = xn[bi, i]
            for j, val in zip(keep, v):
                r = math.exp(val - lse)
                nk[bi, j] += r
                sx[bi, j] += r * row
                if cov == "spherical":
                    sq[bi, j] += r * float(row @ row)
                elif cov == "diag":
                    sq[bi, j] += r * row * row
                elif cov == "full":
                    sq[bi, j] += r * np.outer(row, row)
    return nk, sx, sq, ll


@pytest.mark.parametrize("cov", COVS)
@pytest.mark.parametrize("top_k", [1, 2, 4])
def test_topk_stats_vs_float64_brute_force(cov, top_k):
    x, means, covs, w = _problem(cov, b=2, n=50, d=3, k=5, seed=11)
    nk, sx, sq, ll = torch_ref.estep_stats_topk(x, cov, means, covs, w, top_k)
    e_nk, e_sx, e_sq, e_ll = _topk_stats64(cov, x, _ref_logits64(cov, x, means, covs, w), top_k)
    np.testing.assert_allclose(nk.double().numpy(), e_nk, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(sx.double().numpy(), e_sx, rtol=1e-4, atol=1e-4)
    if sq is not None:
        np.testing.assert_allclose(sq.double().numpy(), e_sq, rtol=1e-4, atol=1e-4)
    assert float(ll) == pytest.approx(e_ll, rel=1e-5)


@pytest.mark.parametrize("cov", COVS)
def test_topk_one_is_hard_assignment(cov):
    """top_k = 1: every row's whole mass goes to its argmax, so the statistics
    are group-by sums over the float64 labels and the log-likelihood sums the
    maximum logits."""
    x, means, covs, w = _problem(cov, b=1, n=80, d=3, k=4, seed=12)
    ref = _ref_logits64(cov, x, means, covs, w)
    lab = ref.argmax(-1)[0]
    nk, sx, sq, ll = torch_ref.estep_stats_topk(x, cov, means, covs, w, 1)
    xn = x[0].double().numpy()
    np.testing.assert_allclose(nk[0].double().numpy(), np.bincount(lab, minlength=4), rtol=0, atol=1e-6)
    for j in range(4):
        np.testing.assert_allclose(sx[0, j].double().numpy(), xn[lab == j].sum(0), rtol=1e-5, atol=1e-4)
    assert float(ll) == pytest.approx(ref.max(-1).sum(), rel=1e-5)


@pytest.mark.parametrize("cov", COVS)
def test_topk_all_but_unreachable_equals_exact(cov):
    """top_k = K - 1 with one component no row can reach: the dropped logit is
    always that component's and its responsibility underflows to zero in exact
    EM, so the approximate statistics equal the exact ones."""
    x, means, covs, w = _problem(cov, b=1, n=80, d=3, k=4, seed=13)
    means = means.clone()
    means[0, 2] = 500.0
    approx = torch_ref.estep_stats_topk(x, cov, means, covs, w, 3)
    exact = torch_ref.estep_stats(x, cov, means, covs, w)
    for a, e in zip(approx, exact):
        if e is not None:
            torch.testing.assert_close(a, e, rtol=1e-5, atol=1e-5)
    # and a fit with approx_top_k = K - 1 follows exact EM
    _, m1, c1, w1, i1 = torch_ref.fit(x, 4, cov, max_iters=3, tol=0.0, init_means=means, init_covs=covs,
                                      init_weights=w, approx_top_k=3)
    _, m2, c2, w2, i2 = torch_ref.fit(x, 4, cov, max_iters=3, tol=0.0, init_means=means, init_covs=covs,
                                      init_weights=w)
    assert i1["approximate_em_enabled"] and i1["approx_top_k"] == 3 and not i2["approximate_em_enabled"]
    torch.testing.assert_close(m1, m2, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(i1["lower_bound_history"], i2["lower_bound_history"], rtol=1e-6)
    # top_k >= K resolves to exact EM (gmmxx/torch_fallback.py:598-606)
    assert torch_ref.fit(x, 4, cov, max_iters=1, init_means=means, init_covs=covs, init_weights=w,
                         approx_top_k=4)[4]["approximate_em_enabled"] is False


@pytest.mark.parametrize("cov", COVS)
def test_random_initialize_matches_numpy_float64(cov):
    """The random-init branch (what init_params="kmeans" runs without
    flash-kmeans): means are the drawn rows, the variances numpy's float64
    population (co)variance of x (spherical: the mean of the per-feature
    variances), weights 1/K; reg_covar added on the diagonal (tied, full) or
    used as the floor (spherical, diag)."""
    g = torch.Generator().manual_seed(8)
    b, n, d, k = 2, 500, 5, 4
    x = torch.randn((b, n, d), generator=g) * 3.0 + 1.0
    idx = torch.randint(0, n, (b, k), generator=g)
    m, c, w = torch_ref.random_initialize(x, cov, k, idx, 1e-6)
    xn = x.double().numpy()
    for bi in range(b):
        np.testing.assert_array_equal(m[bi].numpy(), x[bi, idx[bi]].numpy())
        var = xn[bi].var(axis=0)                    # population variance per feature
        cov_np = np.cov(xn[bi].T, bias=True)
        if cov == "spherical":
            np.testing.assert_allclose(c[bi].double().numpy(), np.full(k, var.mean()), rtol=1e-5)
        elif cov == "diag":
            np.testing.assert_allclose(c[bi].double().numpy(), np.tile(var, (k, 1)), rtol=1e-5)
        else:
            exp = cov_np + 1e-6 * np.eye(d)
            got = c[bi].double().numpy()
            got = got if cov == "tied" else got.reshape(k, d, d)
            np.testing.assert_allclose(got, exp if cov == "tied" else np.broadcast_to(exp, (k, d, d)),
                                       rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(w.numpy(), np.full((b, k), 1.0 / k), rtol=1e-7)
