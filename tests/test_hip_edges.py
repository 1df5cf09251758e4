"""Edge cases of the HIP engine against the CPU oracle: row counts below and
around one 32-row block, a single component, components no row reaches,
very many components, misaligned and strided input, and the reference's
estimator-level approximate-EM checks (gmmxx tests/test_gmmxx.py:150-197,
tests/test_cuda_approx_topk_spherical.py:137-195) on this backend.
Tolerances as in test_hip_parity: statistics and parameters rtol 1e-4 against
the statistic's scale, log-likelihoods rtol 1e-5 (fp32)."""

import pytest
import torch

from gmmxx_amd import GMMXX, em
from oracle import torch_ref
from tests.test_hip_parity import assert_labels, make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
COVS = ("spherical", "diag", "tied", "full")


def _close(got, exp, tol=1e-4):
    torch.testing.assert_close(got.cpu(), exp, rtol=tol, atol=tol * max(1e-30, float(exp.abs().max())))


@pytest.mark.parametrize("cov", COVS)
@pytest.mark.parametrize("n", [1, 5, 31, 33, 65])
def test_few_rows(hip, cov, n):
    print(f"[edges] few rows {cov} N={n}", flush=True)
    x, means, covs, w = make_problem(cov, 2, max(n, 8), 6, 4, seed=61)
    x = x[:, :n].contiguous()
    nk, sx, sq, ll = hip.estep_stats(cov, to_dev(x), to_dev(means), to_dev(covs), to_dev(w))
    e_nk, e_sx, e_sq, e_ll = torch_ref.estep_stats(x, cov, means, covs, w)
    _close(nk, e_nk)
    _close(sx, e_sx)
    if sq is not None:
        _close(sq, e_sq)
    assert float(ll) == pytest.approx(float(e_ll), rel=1e-5, abs=1e-4)
    scores, labels = hip.score(cov, to_dev(x), to_dev(means), to_dev(covs), to_dev(w))
    _close(scores, torch_ref.score_samples(x, means, covs, w, cov), 1e-5)
    assert_labels(labels, x, means, covs, w, cov, 1e-5)


@pytest.mark.parametrize("n", [1, 31, 33, 129])
def test_few_rows_full_whitening(hip, n):
    """Full covariance at D = 20 (the whitening kernels, DP 32): a partial
    32-row block, one wave's rows past N, a four-wave workgroup's tail."""
    print(f"[edges] few rows full D=20 N={n}", flush=True)
    x, means, covs, w = make_problem("full", 2, max(n, 8), 20, 3, seed=63)
    x = x[:, :n].contiguous()
    nk, sx, sq, ll = hip.estep_stats("full", to_dev(x), to_dev(means), to_dev(covs), to_dev(w))
    e_nk, e_sx, e_sq, e_ll = torch_ref.estep_stats(x, "full", means, covs, w)
    _close(nk, e_nk)
    _close(sx, e_sx)
    _close(sq, e_sq)
    assert float(ll) == pytest.approx(float(e_ll), rel=1e-5, abs=1e-4)
    scores, labels = hip.score("full", to_dev(x), to_dev(means), to_dev(covs), to_dev(w))
    _close(scores, torch_ref.score_samples(x, means, covs, w, "full"), 1e-5)
    assert_labels(labels, x, means, covs, w, "full", 1e-5)


@pytest.mark.parametrize("cov", COVS)
def test_single_component(hip, cov):
    """K = 1: every responsibility is 1 and the M-step gives the sample moments."""
    x, means, covs, w = make_problem(cov, 2, 3000, 5, 1, seed=62)
    _, m, c, wt, info = em.fit(to_dev(x), 1, cov, max_iters=3, tol=0.0, record_all_lower_bounds=True,
                               init_means=means, init_covs=covs,
                               init_weights=w, compute_labels=False)
    _, e_m, e_c, e_w, e_info = torch_ref.fit(x, 1, cov, max_iters=3, tol=0.0, init_means=means,
                                             init_covs=covs, init_weights=w, compute_labels=False)
    for a, e in zip(info["lower_bound_history"], e_info["lower_bound_history"]):
        assert a == pytest.approx(e, rel=1e-5)
    _close(m, e_m)
    _close(c, e_c)
    torch.testing.assert_close(wt.cpu(), torch.ones(2, 1))
    _close(m, x.mean(dim=1, keepdim=True), 1e-4)


@pytest.mark.parametrize("cov", COVS)
def test_unreachable_component_keeps_its_parameters(hip, cov):
    """A component far from every row gets N_k below min_weight: it keeps its
    mean and (clamped) covariance, its weight is floored and renormalised
    (gmmxx/torch_fallback.py:2293-2305, :2654-2666, :3143-3167)."""
    x, means, covs, w = make_problem(cov, 1, 4000, 6, 5, seed=63)
    means = means.clone()
    means[0, 3] = 1e4
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    gram = hip.gram(to_dev(x), hip.Workspace(hip.problem(cov, torch.float32, 1, 4000, 6, 5), torch.device(DEV))) \
        if cov == "tied" else None
    lb = torch.zeros(1, device=DEV)
    hip.em_step(cov, to_dev(x), m_d, c_d, w_d, lb, gram_xx=gram)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, cov, means, covs, w)
    assert float(m_d[0, 3, 0].cpu()) == 1e4 and float(w_d[0, 3].cpu()) < 1e-7
    keep = [0, 1, 2, 4]
    _close(m_d[:, keep], e_m[:, keep])
    _close(m_d[:, 3], e_m[:, 3], 1e-6)
    if cov == "tied":
        _close(c_d, e_c)
    else:
        _close(c_d[:, keep], e_c[:, keep])
        _close(c_d[:, 3], e_c[:, 3], 1e-6)
    _close(w_d, e_w, 1e-5)
    assert float(lb) == pytest.approx(e_lb, rel=1e-5)


def test_many_components_spherical(hip):
    """K = 8192 (32 component tiles of 256) at D = 128."""
    x, means, covs, w = make_problem("spherical", 1, 3000, 128, 8192, seed=64)
    nk, sx, sq, ll = hip.estep_stats("spherical", to_dev(x), to_dev(means), to_dev(covs), to_dev(w))
    e_nk, e_sx, e_sq, e_ll = torch_ref.estep_stats(x, "spherical", means, covs, w)
    _close(nk, e_nk)
    _close(sx, e_sx)
    _close(sq, e_sq)
    assert float(ll) == pytest.approx(float(e_ll), rel=1e-5)


@pytest.mark.parametrize("cov", ["spherical", "diag"])
def test_misaligned_and_strided_input(hip, cov):
    """A view that starts mid-allocation (odd D) and a strided view are copied to
    aligned contiguous buffers before the launch; results as for the copy."""
    x, means, covs, w = make_problem(cov, 1, 2001, 7, 6, seed=65)
    xd = to_dev(x)
    view = xd[:, 1:, :]                                  # 28-byte offset
    assert view.data_ptr() % 16 != 0
    got = hip.estep_stats(cov, view, to_dev(means), to_dev(covs), to_dev(w))
    exp = torch_ref.estep_stats(x[:, 1:, :], cov, means, covs, w)
    for a, e in zip(got[:3], exp[:3]):
        if e is not None:
            _close(a, e)
    assert float(got[3]) == pytest.approx(float(exp[3]), rel=1e-5)
    wide = torch.zeros((1, 2000, 14), device=DEV)
    wide[:, :, ::2] = xd[:, 1:, :]
    strided = wide[:, :, ::2]
    got2 = hip.estep_stats(cov, strided, to_dev(means), to_dev(covs), to_dev(w))
    for a, b in zip(got2, got):
        if a is not None:
            torch.testing.assert_close(a, b, rtol=0, atol=0)


@pytest.mark.parametrize("cov", COVS)
def test_estimator_approx_top_k_all_covariance_shapes(hip, cov):
    """The reference's estimator check (tests/test_gmmxx.py:150-197) on this backend."""
    torch.manual_seed(11)
    centers = torch.tensor([[-3.0, -3.0, 0.0], [3.0, -3.0, 1.0], [-3.0, 3.0, -1.0], [3.0, 3.0, 0.5]])
    x = torch.cat([torch.randn(48, 3) * 0.25 + c for c in centers], dim=0)
    model = GMMXX(d=3, k=4, niter=3, tol=0.0, init_params="random", reg_covar=1e-4, covariance_type=cov,
                  compute_labels_on_fit=False, approx_top_k=2, backend="hip", device=DEV)
    model.fit(x.to(DEV))
    probs = model.predict_proba(x[:16].to(DEV))
    assert model.approximate_em_enabled_ and model.approx_top_k_ == 2
    assert model.cluster_ids_b is None
    assert probs.shape == (16, 4)
    for t in (model.means_b, model.variances_b, model.weights_b):
        assert bool(torch.isfinite(t).all())
    torch.testing.assert_close(probs.sum(-1).cpu(), torch.ones(16), atol=1e-4, rtol=0)


def test_estimator_approx_top_k_large_k(hip):
    """K = 4096, D = 128, fp16 input, top 8 (tests/test_cuda_approx_topk_spherical.py:137-170)."""
    torch.manual_seed(124)
    x = torch.randn(512, 128, device=DEV, dtype=torch.float16)
    model = GMMXX(d=128, k=4096, niter=1, tol=0.0, seed=124, init_params="random", covariance_type="spherical",
                  backend="hip", approx_top_k=8, device=DEV, compute_labels_on_fit=False)
    model.fit(x)
    assert model.last_backend_used_ == "hip" and model.approx_top_k_ == 8
    assert model.means_b.shape == (1, 4096, 128) and model.labels_ is None
    for t in (model.means_b, model.covariances_b, model.weights_b):
        assert bool(torch.isfinite(t).all())
    # equal k resolves to exact EM (tests/test_cuda_approx_topk_spherical.py:173-195)
    m2 = GMMXX(d=8, k=6, niter=2, tol=0.0, seed=7, init_params="random", covariance_type="spherical",
               backend="hip", approx_top_k=6, device=DEV, compute_labels_on_fit=False)
    m2.fit(torch.randn(192, 8, device=DEV))
    assert m2.approximate_em_enabled_ is False and m2.approx_top_k_ is None


@pytest.mark.parametrize("d", [40, 100])
def test_full_jitter_ladder_indefinite_covariance(hip, d):
    """Full covariance at D > 16 (whitening kernels): one component's covariance
    is indefinite (eigenvalues in [1e-3, 3e-3] and one of -5e-4), the others are
    well conditioned on the same scale.  The batch-global ladder takes every
    component's factorisation to jitter 1e-3 (level 4) in both implementations
    (torch_fallback.py:316-334); scores, labels and one EM step match the oracle."""
    print(f"[edges] full jitter ladder D={d}", flush=True)
    k = 3
    x, means, _, w = make_problem("full", 1, 6000, d, k, seed=68)
    x, means = 0.03 * x, 0.03 * means
    g = torch.Generator().manual_seed(69)
    covs = []
    for i in range(k):
        q, _ = torch.linalg.qr(torch.randn(d, d, generator=g, dtype=torch.float64))
        lam = 1e-3 * (1.0 + 2.0 * torch.rand(d, generator=g, dtype=torch.float64))
        if i == 1:
            lam[0] = -5e-4
        c = (q * lam) @ q.T
        covs.append(0.5 * (c + c.T))
    covs = torch.stack(covs)[None].float()
    scores, labels = hip.score("full", to_dev(x), to_dev(means), to_dev(covs), to_dev(w))
    e_sc = torch_ref.score_samples(x, means, covs, w, "full")
    torch.testing.assert_close(scores.cpu(), e_sc, rtol=1e-5, atol=1e-5 * float(e_sc.abs().mean()))
    assert_labels(labels, x, means, covs, w, "full")
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    lb = torch.zeros(1, device=DEV)
    hip.em_step("full", to_dev(x), m_d, c_d, w_d, lb)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, "full", means, covs, w)
    assert float(lb) == pytest.approx(e_lb, rel=1e-5)
    _close(m_d, e_m)
    _close(c_d, e_c)
    _close(w_d, e_w)


@pytest.mark.parametrize("d", [40, 100])
def test_tied_jitter_ladder_indefinite_covariance(hip, d):
    """An indefinite tied covariance (eigenvalues in [1e-3, 3e-3] and one of
    -5e-4): the factorisation fails at levels 0-3 and succeeds at jitter 1e-3
    (level 4) in both implementations, with a factor of 2 to spare either way
    (torch_fallback.py:316-334); the jittered matrix is well conditioned
    (κ ≈ 8), so the fp32 precisions agree closely.  Data on the same scale.  The
    per-sample log-likelihoods and the EM step from it match the oracle's.
    D = 100 runs the one-workgroup factorisation of 64 < D <= 128."""
    print(f"[edges] tied jitter ladder D={d}", flush=True)
    x, means, _, w = make_problem("tied", 1, 6000, d, 12, seed=66)
    x, means = 0.03 * x, 0.03 * means
    g = torch.Generator().manual_seed(67)
    q, _ = torch.linalg.qr(torch.randn(d, d, generator=g, dtype=torch.float64))
    lam = 1e-3 * (1.0 + 2.0 * torch.rand(d, generator=g, dtype=torch.float64))
    lam[0] = -5e-4
    covs = ((q * lam) @ q.T)[None].float()
    covs = 0.5 * (covs + covs.transpose(-1, -2))
    scores, _ = hip.score("tied", to_dev(x), to_dev(means), to_dev(covs), to_dev(w))
    e_sc = torch_ref.score_samples(x, means, covs, w, "tied")
    torch.testing.assert_close(scores.cpu(), e_sc, rtol=1e-5, atol=1e-5 * float(e_sc.abs().mean()))
    xd = to_dev(x)
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    lb = torch.zeros(1, device=DEV)
    hip.em_step("tied", xd, m_d, c_d, w_d, lb, gram_xx=hip.gram(xd))
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, "tied", means, covs, w)
    assert float(lb) == pytest.approx(e_lb, rel=1e-5)
    _close(m_d, e_m)
    _close(c_d, e_c)
    _close(w_d, e_w)
