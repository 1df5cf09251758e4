"""A non-finite input row through one EM iteration, against the oracle.

The reference has no finite-input check: a NaN feature makes that row's logits
NaN for every component, so its responsibilities, every N_k and the lower bound
are NaN.  The finalize's active mask (N_k > min_weight) is then false for every
component, so means and covariances keep their previous values, and the
weights (clamp_min of NaN, as torch.clamp passes NaN through) are NaN
(torch_fallback.py:2293-2305, :2654-2666, :3143-3167).

The single passes whose workgroups exchange per-row partials (the cooperative
spherical bf16 kernel, the fp32 exchange pass) must hand such a row on like
any other instead of waiting for a word that never reads as ready: the
iteration finishes, no timeout is recorded, and the results are the oracle's.
"""

import pytest
import torch

from gmmxx_amd import _hip, em
from oracle import torch_ref
from tests.test_hip_parity import make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # cov, N, D, K, dtype, kernel family
    ("diag", 8192, 64, 512, torch.float32, "exchange pass"),
    ("spherical", 8192, 32, 700, torch.float32, "exchange pass"),
    ("tied", 8192, 32, 300, torch.float32, "exchange pass"),
    ("spherical", 8192, 128, 520, torch.bfloat16, "cooperative kernel"),
    ("spherical", 8192, 128, 1024, torch.bfloat16, "cooperative kernel"),
    ("spherical", 8192, 32, 64, torch.bfloat16, "fused kernel"),
    ("diag", 8192, 16, 64, torch.float32, "one-tile pass"),
    ("full", 4096, 8, 16, torch.float32, "one-tile pass"),
    ("spherical", 8192, 64, 2048, torch.float32, "two passes"),
]


def _id(c):
    return f"{c[0]}-N{c[1]}-D{c[2]}-K{c[3]}-{'bf16' if c[4] == torch.bfloat16 else 'fp32'}"


# An infinite feature turns a row's logits into a mix of NaN and -inf (the
# expanded squared distance inf - inf): the log-normaliser is NaN either way
# for spherical and diag.  (Tied and full logits can mix +inf and -inf, whose
# NaN pattern depends on the expansion; only NaN is checked for them.)
PARAMS = [(c, v) for c in CASES for v in ("nan", "inf") if v == "nan" or c[0] in ("spherical", "diag")]


@pytest.mark.parametrize("case,value", PARAMS, ids=[f"{_id(c)}-{v}" for c, v in PARAMS])
def test_nonfinite_row_propagates_like_the_oracle(hip, case, value):
    cov, n, d, k, dt, family = case
    print(f"[non-finite row] {_id(case)} ({family}) value={value}", flush=True)
    bf = dt == torch.bfloat16
    x, means, covs, w = make_problem(cov, 1, n, d, k, seed=17, dtype=dt)
    if cov in ("tied", "full"):
        covs = 0.5 * (covs + covs.transpose(-1, -2))   # exactly symmetric: the prelude keeps it bit for bit
    value = float(value)
    x = x.clone()
    x[0, n // 3, d // 2] = value          # one feature of one row, not one of the initial means
    xd = to_dev(x, dt)
    m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
    gram = None
    if cov == "tied":
        gram = hip.gram(xd, hip.Workspace(hip.problem("tied", torch.float32, 1, n, d, 1), xd.device))
    ws = hip.Workspace(hip.problem(cov, xd.dtype, 1, n, d, k), xd.device)
    hip.take_status(ws)                   # clear the fresh workspace's status word
    lb = torch.zeros(1, device=DEV)
    hip.em_step(cov, xd, m_d, c_d, w_d, lb, gram_xx=gram, ws=ws)
    status = int(hip.take_status(ws).item())
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x.float(), cov, means, covs, w, bf16_means=bf)
    torch.cuda.synchronize()
    assert status == 0, "a non-finite row must not be reported as a timed-out exchange"
    assert torch.isnan(torch.tensor(e_lb)), "oracle: the lower bound of a NaN row is NaN"
    assert torch.isnan(lb).all()
    # weights NaN, means and covariances unchanged -- exactly the oracle's values
    torch.testing.assert_close(w_d.cpu(), e_w, equal_nan=True, rtol=0, atol=0)
    torch.testing.assert_close(m_d.cpu(), e_m, equal_nan=True, rtol=0, atol=0)
    torch.testing.assert_close(c_d.cpu(), e_c, equal_nan=True, rtol=0, atol=0)


def test_nonfinite_fit_does_not_raise_a_timeout(hip):
    """em.fit over an exchange shape with a NaN row: the NaN trajectory of the
    reference, no HipRuntimeError blaming a partner workgroup."""
    x, means, covs, w = make_problem("diag", 1, 8192, 64, 512, seed=5)
    x = x.clone()
    x[0, 77, 0] = float("nan")
    _, m, c, wt, info = em.fit(to_dev(x), 512, "diag", max_iters=3, tol=0.0, init_means=means, init_covs=covs,
                               init_weights=w, compute_labels=False, record_all_lower_bounds=True)
    assert all(v != v for v in info["lower_bound_history"])
    assert bool(torch.isnan(wt).all())
