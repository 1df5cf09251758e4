"""GPU tests of the exchange single pass (``MODE_STATS_XCH`` of the fp32 tile
kernel): fp32 spherical, diag (D <= 64) and tied EM with 2..4 component tiles
of 256 components, whose workgroups swap per-row (max, sum) partials instead of
running a separate log-normaliser pass.

* against the oracle, one iteration: lower bound rtol 1e-5, parameters
  element-wise rtol 1e-4 with the floors of test_hip_parity;
* against the two-pass kernels (GMMXX_HIP_NO_XCH=1) over three iterations: the
  two are the same fp32-accurate iteration and differ only in the order of the
  log-normaliser merge, so they agree to the same bars;
* a timed-out wait (negative spin limit, forced from the host: every wait gives
  up at once and every workgroup still runs to its end) leaves the parameters
  unchanged, writes a NaN lower bound and makes em.fit raise.
"""

import math

import pytest
import torch

from gmmxx_amd import em
from oracle import torch_ref
from tests.test_hip_parity import assert_params, make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # cov, B, N, D, K: 2, 3 and 4 component tiles, padded rows and components
    ("diag", 1, 30000, 64, 512),
    ("spherical", 2, 20000, 32, 700),
    ("tied", 1, 40000, 32, 1000),
    ("diag", 2, 9000, 20, 300),
    ("spherical", 1, 24000, 128, 300),
]


def _id(c):
    return f"{c[0]}-B{c[1]}-N{c[2]}-D{c[3]}-K{c[4]}"


def _gram(hip, cov, xd):
    if cov != "tied":
        return None
    b, n, d = xd.shape
    return hip.gram(xd, hip.Workspace(hip.problem("tied", torch.float32, b, n, d, 1), xd.device))


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_xch_iteration_matches_oracle(hip, case):
    cov, b, n, d, k = case
    print(f"[xch vs oracle] {_id(case)}", flush=True)
    x, means, covs, w = make_problem(cov, b, n, d, k, seed=61)
    xd = to_dev(x)
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    lb = torch.zeros(1, device=DEV)
    hip.em_step(cov, xd, m_d, c_d, w_d, lb, gram_xx=_gram(hip, cov, xd))
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, cov, means, covs, w)
    torch.cuda.synchronize()
    assert float(lb) == pytest.approx(e_lb, rel=1e-5)
    assert_params(m_d, e_m, "means", x, torch.float32)
    assert_params(c_d, e_c, "covs", x, torch.float32)
    assert_params(w_d, e_w, "weights", x, torch.float32)


@pytest.mark.parametrize("case", CASES[:3], ids=_id)
def test_xch_matches_two_pass(hip, monkeypatch, case):
    cov, b, n, d, k = case
    print(f"[xch vs two-pass] {_id(case)}", flush=True)
    x, means, covs, w = make_problem(cov, b, n, d, k, seed=62)
    xd = to_dev(x)
    gram = _gram(hip, cov, xd)
    out = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("GMMXX_HIP_NO_XCH", mode)
        m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
        lbs = []
        for _ in range(3):
            lb = torch.zeros(1, device=DEV)
            hip.em_step(cov, xd, m_d, c_d, w_d, lb, gram_xx=gram)
            lbs.append(float(lb))
        torch.cuda.synchronize()
        out[mode] = (m_d.cpu(), c_d.cpu(), w_d.cpu(), lbs)
    (m1, c1, w1, l1), (m2, c2, w2, l2) = out["0"], out["1"]
    for a_, e_ in zip(l1, l2):
        assert a_ == pytest.approx(e_, rel=1e-5)
    assert_params(m1, m2, "means", x, torch.float32)
    assert_params(c1, c2, "covs", x, torch.float32)
    assert_params(w1, w2, "weights", x, torch.float32)


def test_xch_timed_out_wait_keeps_parameters_and_raises(hip, monkeypatch):
    cov, b, n, d, k = CASES[0]
    x, means, covs, w = make_problem(cov, 1, 6000, d, k, seed=63)
    xd = to_dev(x)
    prob = hip.problem(cov, torch.float32, 1, 6000, d, k)
    ws = hip.Workspace(prob, xd.device)
    assert int(hip.take_status(ws).item()) == 0
    monkeypatch.setenv("GMMXX_HIP_COOP_SPIN_LIMIT", "-1")
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    lb = torch.zeros(1, device=DEV)
    hip.em_step(cov, xd, m_d, c_d, w_d, lb, ws=ws)
    torch.cuda.synchronize()
    assert math.isnan(float(lb))
    assert torch.equal(m_d.cpu(), means) and torch.equal(c_d.cpu(), covs) and torch.equal(w_d.cpu(), w)
    assert int(hip.take_status(ws).item()) != 0
    with pytest.raises(hip.HipRuntimeError, match="timed out"):
        em.fit(xd, k, cov, max_iters=2, tol=0.0, init_means=means, init_covs=covs, init_weights=w)
    monkeypatch.delenv("GMMXX_HIP_COOP_SPIN_LIMIT")
    hip.em_step(cov, xd, m_d, c_d, w_d, lb, ws=ws)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, cov, means, covs, w)
    torch.cuda.synchronize()
    assert float(lb) == pytest.approx(e_lb, rel=1e-5)
    assert int(hip.take_status(ws).item()) == 0
    assert_params(m_d, e_m, "means", x, torch.float32)


@pytest.mark.parametrize("n", [1, 20, 33, 385, 1000])
def test_xch_short_slices_match_oracle(hip, n):
    """Row slices of one or a few 32-row blocks (the pipeline's first block is
    also its last; padded rows), two and three component tiles."""
    for cov, d, k in (("diag", 20, 300), ("spherical", 32, 700)):
        print(f"[xch short] {cov} N={n} D={d} K={k}", flush=True)
        x, means, covs, w = make_problem(cov, 1, n, d, k, seed=64 + n)
        xd = to_dev(x)
        m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
        lb = torch.zeros(1, device=DEV)
        hip.em_step(cov, xd, m_d, c_d, w_d, lb)
        e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, cov, means, covs, w)
        torch.cuda.synchronize()
        assert float(lb) == pytest.approx(e_lb, rel=1e-5)
        assert_params(m_d, e_m, "means", x, torch.float32)
        assert_params(c_d, e_c, "covs", x, torch.float32)
        assert_params(w_d, e_w, "weights", x, torch.float32)
