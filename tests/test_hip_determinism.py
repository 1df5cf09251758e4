"""Run-to-run bitwise determinism of the EM iteration.

Every reduction in the engine is ordered (no atomics on floating-point data):
the per-slice statistics are summed in slice order, the cooperative kernel
merges the group's log-normaliser partials in member order, the fused kernel
combines its waves in a fixed order, and the Cholesky jitter ladder takes a
batch-global level.  So the same iteration from the same inputs must give the
same bits, launch after launch.  One case per kernel family.
"""

import pytest
import torch

from tests.test_hip_parity import make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

FAMILIES = [
    # (name, cov, B, N, D, K, dtype)
    ("coop", "spherical", 1, 20000, 128, 1000, torch.bfloat16),        # cooperative single pass, G = 4
    ("fused", "spherical", 2, 9000, 32, 64, torch.bfloat16),           # fused small-K single pass
    ("two-pass-bf16", "spherical", 1, 9000, 128, 2048, torch.bfloat16),  # LSE + STATS bf16 tile kernels
    ("one-tile", "spherical", 1, 9000, 32, 64, torch.float32),         # fp32 single tile pass
    ("two-pass-fp32", "diag", 1, 9000, 64, 512, torch.float32),        # fp32 LSE + STATS
    ("cholesky-tied", "tied", 1, 9000, 64, 128, torch.float32),        # jitter ladder + tied M-step
    ("cholesky-tied-d100", "tied", 1, 6000, 100, 40, torch.float32),   # one-workgroup factorisation, D > 64
    ("cholesky-full", "full", 4, 6000, 16, 32, torch.float32),         # per-component Cholesky
    ("whitening-full-d64", "full", 2, 6000, 64, 5, torch.float32),     # full D > 16: whitening E-step, Gram statistics
    ("whitening-full-d100", "full", 1, 5000, 100, 3, torch.float32),   # DP 128, one-workgroup Cholesky
]


@pytest.mark.parametrize("case", FAMILIES, ids=[c[0] for c in FAMILIES])
def test_em_step_bitwise_repeatable(hip, case):
    name, cov, b, n, d, k, dt = case
    print(f"[determinism] {name}", flush=True)
    x, means, covs, w = make_problem(cov, b, n, d, k, seed=41, dtype=dt)
    xd = to_dev(x, dt)
    ws = hip.Workspace(hip.problem(cov, xd.dtype, b, n, d, k), xd.device)
    gram = hip.gram(xd, ws) if cov == "tied" else None
    runs = []
    for _ in range(2):
        m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
        lbs = torch.zeros(3, device=DEV)
        for it in range(3):
            hip.em_step(cov, xd, m_d, c_d, w_d, lbs[it:it + 1], gram_xx=gram, ws=ws)
        stats = hip.estep_stats(cov, xd, m_d, c_d, w_d, ws=ws)
        scores, labels = hip.score(cov, xd, m_d, c_d, w_d, ws=ws)
        torch.cuda.synchronize()
        runs.append([t.cpu() for t in (m_d, c_d, w_d, lbs, scores, labels) + tuple(s for s in stats if s is not None)])
    for a, e in zip(*runs):
        assert torch.equal(a, e)
