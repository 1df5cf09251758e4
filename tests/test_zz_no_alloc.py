"""gmmxx_hip_em_step_noalloc (static device scratch, no workspace) against
gmmxx_hip_em_step (caller workspace) through the C ABI: two calls in a row per
case, the second on a smaller input, each bit-equal to the workspace entry
point (the same plan and kernels run; only the scratch address differs).
Also: a problem above the 64 MiB scratch limit is refused before any launch."""

import pytest
import torch

from tests.test_hip_parity import make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # cov, B, (N first call, N second call), D, K, dtype
    ("spherical", 1, (100000, 4000), 32, 64, torch.float32),     # one-tile single pass
    ("spherical", 1, (20000, 3000), 128, 520, torch.bfloat16),   # cooperative single pass
    ("spherical", 2, (9000, 2000), 32, 64, torch.bfloat16),      # fused single pass
    ("diag", 1, (12000, 5000), 64, 300, torch.float32),          # two passes
    ("tied", 1, (20000, 7000), 64, 128, torch.float32),          # Cholesky + tied M-step
    ("full", 3, (6000, 1000), 16, 32, torch.float32),            # per-component Cholesky
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-K{c[4]}-{str(c[5]).split('.')[-1]}" for c in CASES])
def test_noalloc_matches_workspace_entry(hip, case):
    cov, b, ns, d, k, dt = case
    for n in ns:
        print(f"[noalloc] {cov} B={b} N={n} D={d} K={k} {dt}", flush=True)
        x, means, covs, w = make_problem(cov, b, n, d, k, seed=51 + n % 7, dtype=dt)
        xd = to_dev(x, dt)
        gram = hip.gram(xd) if cov == "tied" else None
        out = []
        for fn in (hip.em_step, hip.em_step_noalloc):
            m_d, c_d, w_d = to_dev(means), to_dev(covs), to_dev(w)
            lb = torch.zeros(2, device=DEV)
            for it in range(2):
                fn(cov, xd, m_d, c_d, w_d, lb[it:it + 1], gram_xx=gram)
            torch.cuda.synchronize()
            out.append([t.cpu() for t in (m_d, c_d, w_d, lb)])
        for a, e in zip(out[1], out[0]):
            assert torch.equal(a, e)
        assert bool(torch.isfinite(out[1][3]).all())


def test_noalloc_refuses_problems_above_the_scratch(hip):
    """C2's shape needs ~345 MiB of workspace: refused with a clear error and
    nothing written (the parameters stay as they were)."""
    n, d, k = 4 * 1024 * 1024, 128, 1024
    prob = hip.problem("spherical", torch.bfloat16, 1, n, d, k)
    assert hip.load_library().gmmxx_hip_workspace_bytes(prob) > hip.NOALLOC_SCRATCH_BYTES
    x = torch.zeros((1, n, d), dtype=torch.bfloat16, device=DEV)
    means = torch.ones((1, k, d), device=DEV)
    covs = torch.ones((1, k), device=DEV)
    w = torch.full((1, k), 1.0 / k, device=DEV)
    lb = torch.full((1,), 7.0, device=DEV)
    with pytest.raises(hip.HipRuntimeError, match="no-allocation limit"):
        hip.em_step_noalloc("spherical", x, means, covs, w, lb)
    torch.cuda.synchronize()
    assert float(lb) == 7.0 and bool((means == 1).all())
