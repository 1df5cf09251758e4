"""The single-pass cooperative kernel (spherical bf16, D = 128, 256 < K <= 1024):
short last row items, the K = 1024 (four-member group) EM trajectory, and the
timed-out-wait contract.

Tolerances as in test_hip_parity for bf16 x: mean log-likelihood rtol 2e-3,
statistics and parameters rtol 2e-3 against the statistic's scale.
"""

import math

import pytest
import torch

from gmmxx_amd import _hip, em
from oracle import torch_ref
from tests.test_hip_parity import assert_bf16_means, assert_labels, make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF = torch.bfloat16


def _close(got, exp, tol):
    torch.testing.assert_close(got.cpu(), exp, rtol=tol, atol=tol * max(1e-30, float(exp.abs().max())))


@pytest.mark.parametrize("n", [1, 20, 32, 33, 385, 1000])
@pytest.mark.parametrize("k", [520, 1000])
def test_short_items_match_oracle(hip, n, k):
    """Row items of one or two 32-row blocks (the pipeline's drain with a
    single staged block): statistics, log-likelihood and one EM step."""
    print(f"[coop-short] N={n} K={k}", flush=True)
    x, means, covs, w = make_problem("spherical", 1, max(n, 8), 128, k, seed=31, dtype=BF)
    x = x[:, :n].contiguous()
    xd = to_dev(x, BF)
    nk, sx, sq, ll = hip.estep_stats("spherical", xd, to_dev(means), to_dev(covs), to_dev(w))
    e_nk, e_sx, e_sq, e_ll = torch_ref.estep_stats(x, "spherical", means, covs, w)
    for a, e in ((nk, e_nk), (sx, e_sx), (sq, e_sq)):
        assert bool(torch.isfinite(a).all())
        _close(a, e, 2e-3)
    assert float(ll) == pytest.approx(float(e_ll), rel=2e-3)
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    lb = torch.zeros(1, device=DEV)
    hip.em_step("spherical", xd, m_d, c_d, w_d, lb)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, "spherical", means, covs, w, bf16_means=True)
    torch.cuda.synchronize()
    assert float(lb) == pytest.approx(e_lb, rel=2e-3)
    assert_bf16_means(m_d, e_m)
    _close(c_d, e_c, 2e-3)
    _close(w_d, e_w, 2e-3)


def test_k1024_trajectory_matches_oracle(hip):
    """Ten EM iterations at D = 128, K = 1024 (groups of four workgroups) with
    64 rows per component: lower-bound history, parameters and labels."""
    n, k = 65536, 1024
    print(f"[coop-traj] N={n} K={k}", flush=True)
    x, means, covs, w = make_problem("spherical", 1, n, 128, k, seed=32, dtype=BF)
    assert _hip.supported("spherical", BF, 1, n, 128, k)
    labels, m, c, wt, info = em.fit(to_dev(x, BF), k, "spherical", max_iters=10, tol=0.0, init_means=means,
                                    init_covs=covs, init_weights=w)
    e_lab, e_m, e_c, e_w, e_info = torch_ref.fit(x, k, "spherical", max_iters=10, tol=0.0, init_means=means,
                                                 init_covs=covs, init_weights=w, bf16_means=True)
    assert info["n_iter"] == e_info["n_iter"] == 10
    for got, exp in zip(info["lower_bound_history"], e_info["lower_bound_history"]):
        assert got == pytest.approx(exp, rel=2e-3)
    assert_bf16_means(m, e_m)
    _close(c, e_c, 2e-3)
    _close(wt, e_w, 2e-3)
    # bf16 parameters within their bar move logits by more than the near-tie
    # band, so the fit's own labels are not comparable with the oracle's: the
    # HIP kernel labels the rows under the oracle's final parameters and is
    # judged against the oracle's labels
    lab_o = _hip.score("spherical", to_dev(x, BF), to_dev(e_m), to_dev(e_c), to_dev(e_w), want_scores=False)[1]
    assert_labels(lab_o, x, e_m, e_c, e_w, "spherical", 1e-5)


def test_timed_out_wait_keeps_parameters_and_raises(hip, monkeypatch):
    """A negative spin limit makes every exchange give up at its first wait (all
    workgroups still run to the end).  The iteration must write a NaN lower
    bound, leave the parameters unchanged and record the failure in the
    workspace status; em.fit raises instead of returning."""
    x, means, covs, w = make_problem("spherical", 1, 4000, 128, 520, seed=33, dtype=BF)
    xd = to_dev(x, BF)
    prob = hip.problem("spherical", BF, 1, 4000, 128, 520)
    ws = hip.Workspace(prob, xd.device)
    assert int(hip.take_status(ws).item()) == 0
    monkeypatch.setenv("GMMXX_HIP_COOP_SPIN_LIMIT", "-1")
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    lb = torch.zeros(1, device=DEV)
    hip.em_step("spherical", xd, m_d, c_d, w_d, lb, ws=ws)
    torch.cuda.synchronize()
    assert math.isnan(float(lb))
    assert torch.equal(m_d.cpu(), means) and torch.equal(c_d.cpu(), covs) and torch.equal(w_d.cpu(), w)
    assert int(hip.take_status(ws).item()) != 0
    assert int(hip.take_status(ws).item()) == 0          # cleared by the read
    with pytest.raises(hip.HipRuntimeError, match="timed out"):
        em.fit(xd, 520, "spherical", max_iters=2, tol=0.0, init_means=means, init_covs=covs, init_weights=w)
    # the default limit: the same workspace works again
    monkeypatch.delenv("GMMXX_HIP_COOP_SPIN_LIMIT")
    hip.em_step("spherical", xd, m_d, c_d, w_d, lb, ws=ws)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, "spherical", means, covs, w, bf16_means=True)
    torch.cuda.synchronize()
    assert float(lb) == pytest.approx(e_lb, rel=2e-3)
    assert int(hip.take_status(ws).item()) == 0
    assert_bf16_means(m_d, e_m)
