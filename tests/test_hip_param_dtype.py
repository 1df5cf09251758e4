"""Parameters kept in a half-precision dtype (gmmxx_problem.param_dtype).

The reference computes a half-precision x's diag/tied/full logits and
statistics in fp32 (torch_fallback.py:357-465: ``x.to(torch.float32)``) and
keeps the parameters in x's dtype: its initialisers cast them
(:1661-1682, :1731-1742, :1791-1802, :1851-1862) and every M-step rounds the
new means, covariances and weights to it (:2654-2666, :3143-3167).  The oracle
given x in that dtype does the same; the engine computes the fp32 x and
rounds the parameters in its finalize.  The arithmetic of the two differs below
the parameters' own rounding (the reference's iteration prelude divides the
weights in the half dtype, the engine in fp32 before rounding), so the bar is
the half-precision one: 2e-3 relative plus 2e-3 of the parameter's scale, one
ulp of the dtype more, and the mean log-likelihood within 2e-3 relative.
"""

import pytest
import torch

from gmmxx_amd import GMMXX, em
from oracle import torch_ref
from tests.test_hip_parity import make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [("diag", torch.bfloat16, 12), ("tied", torch.bfloat16, 12), ("full", torch.bfloat16, 12),
         ("diag", torch.float16, 12), ("tied", torch.float16, 12), ("full", torch.float16, 12),
         # D > 16: the whitening kernels (the prelude's rounding in their packing kernel)
         ("full", torch.bfloat16, 40), ("full", torch.float16, 40)]


def _ulp(t: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """One ulp of dtype dt at each value of t (normal range)."""
    mant = {torch.bfloat16: 8, torch.float16: 11}[dt]
    _, e = torch.frexp(t)
    return torch.ldexp(torch.ones_like(t), e - mant)


def _close_half(got, exp, dt, what):
    got, exp = got.cpu().float(), exp.float()
    assert torch.equal(got, got.to(dt).to(torch.float32)), f"{what}: not {dt} values"
    bar = 2e-3 * exp.abs() + 2e-3 * float(exp.abs().max()) + _ulp(exp, dt)
    diff = (got - exp).abs()
    assert bool((diff <= bar).all()), f"{what}: largest |Δ| {float(diff.max()):.3e}"


@pytest.mark.parametrize("cov,dt,d", CASES, ids=[f"{c}-{str(t).split('.')[-1]}-D{d}" for c, t, d in CASES])
def test_fit_with_half_parameters_matches_oracle(hip, cov, dt, d):
    print(f"[param dtype] {cov} {dt} D={d}", flush=True)
    x, means, covs, w = make_problem(cov, 2, 6000, d, 5, seed=71, dtype=dt)
    _, e_m, e_c, e_w, e_info = torch_ref.fit(x.to(dt), 5, cov, max_iters=5, tol=0.0, init_means=means,
                                             init_covs=covs, init_weights=w, compute_labels=False)
    _, m, c, wt, info = em.fit(to_dev(x), 5, cov, max_iters=5, tol=0.0, init_means=means, init_covs=covs,
                               init_weights=w, record_all_lower_bounds=True, compute_labels=False, param_dtype=dt)
    for got, exp in zip(info["lower_bound_history"], e_info["lower_bound_history"]):
        assert got == pytest.approx(exp, rel=2e-3)
    _close_half(m, e_m, dt, "means")
    _close_half(c, e_c, dt, "covariances")
    _close_half(wt, e_w, dt, "weights")


def test_estimator_keeps_half_parameters(hip):
    """GMMXX(dtype=torch.bfloat16) on diag: the fitted parameters are bf16 values
    (fp32 tensors), as the reference's are bf16 tensors."""
    x, _, _, _ = make_problem("diag", 1, 4000, 8, 3, seed=72, dtype=torch.bfloat16)
    est = GMMXX(n_components=3, covariance_type="diag", max_iter=3, tol=0.0, random_state=5, backend="hip",
                dtype=torch.bfloat16)
    est.fit(x[0].to(DEV))
    for t in (est.means_, est.covariances_, est.weights_):
        assert torch.equal(t.cpu(), t.cpu().to(torch.bfloat16).to(torch.float32))
