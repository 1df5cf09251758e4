"""The float64 EM helper (tests/f64_em.py) agrees with the fp32 oracle on
well-conditioned problems, so it can serve as the truth for drifting fp32
trajectories.  CPU only."""

import pytest
import torch

from oracle import torch_ref
from oracle import f64_em


def _problem(cov, b, n, d, k, seed):
    g = torch.Generator().manual_seed(seed)
    centers = (torch.rand((b, k, d), generator=g) * 2 - 1) * 4.0
    lab = torch.randint(0, k, (b, n), generator=g)
    x = torch.gather(centers, 1, lab[..., None].expand(-1, -1, d)) + torch.randn((b, n, d), generator=g)
    means = centers + 0.3 * torch.randn((b, k, d), generator=g)
    if cov == "spherical":
        covs = torch.rand((b, k), generator=g) + 0.5
    elif cov == "diag":
        covs = torch.rand((b, k, d), generator=g) + 0.5
    else:
        shape = (b, d, d) if cov == "tied" else (b, k, d, d)
        a = torch.randn(shape, generator=g) * 0.3
        covs = a @ a.transpose(-1, -2) + 0.7 * torch.eye(d)
    w = torch.rand((b, k), generator=g) + 0.2
    return x, means, covs, w / w.sum(-1, keepdim=True)


@pytest.mark.parametrize("cov", ["spherical", "diag", "tied", "full"])
def test_f64_step_matches_oracle(cov):
    x, means, covs, w = _problem(cov, 2, 3000, 6, 5, seed=71)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, cov, means, covs, w)
    m, c, wt, lb = f64_em.em_step(x, cov, means, covs, w)
    assert lb == pytest.approx(e_lb, rel=1e-6)
    torch.testing.assert_close(m.float(), e_m, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(c.float(), e_c, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(wt.float(), e_w, rtol=1e-5, atol=1e-7)


def test_judge_flags_a_planted_error():
    """The arbiter accepts a value outside the bar only when the float64 truth
    sides with it: an error planted in a copy of the oracle's result is flagged."""
    from oracle import judge
    x, means, covs, w = _problem("diag", 1, 2000, 4, 3, seed=72)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, "diag", means, covs, w)
    m64, c64, w64, lb64 = f64_em.em_step(x, "diag", means, covs, w)
    planted = e_m.clone()
    planted[0, 1, 2] += 1e-2
    res = judge.judge_params(planted, e_m, "means", x, False, lambda: m64)
    assert res["outside_bar"] == 1 and res["unexplained"] == 1
    # the float64 value itself passes against the oracle's (it is the truth)
    assert judge.judge_params(m64.float(), e_m, "means", x, False, lambda: m64)["unexplained"] == 0
    res = judge.judge_ll([e_lb * (1 + 1e-3)], [e_lb], 1e-5, lambda: [lb64])
    assert res["unexplained"] == 1


def test_distribution_arbiter_flags_planted_errors():
    """The distribution rule: a systematic error moves the 99th percentile, a
    gross single-element error the largest error; both are flagged, while an
    fp32 result as accurate as the oracle's passes."""
    from oracle import judge
    x, means, covs, w = _problem("diag", 1, 3000, 4, 3, seed=74)
    e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(x, "diag", means, covs, w)
    m64, c64, w64, lb64 = f64_em.em_step(x, "diag", means, covs, w)
    o = judge.error_distribution(e_c, c64, "covs", x)
    assert judge.arbiter_distribution_ok(judge.error_distribution(e_c.clone(), c64, "covs", x), o)
    systematic = e_c * (1 + 3e-4)                       # every element 3 bars off
    assert not judge.arbiter_distribution_ok(judge.error_distribution(systematic, c64, "covs", x), o)
    gross = e_c.clone()
    gross[0, 1, 2] += 0.5                               # one element far off
    assert not judge.arbiter_distribution_ok(judge.error_distribution(gross, c64, "covs", x), o)


@pytest.mark.parametrize("cov", ["spherical", "full"])
def test_label_arbiter_flags_planted_errors(cov):
    """The label check: the oracle's own labels pass; one row moved to its
    float64 runner-up component (a misordering far beyond the near-tie bar) is
    flagged, though the count rule alone would allow one such row."""
    from tests.test_hip_parity import assert_labels
    x, means, covs, w = _problem(cov, 1, 2000, 8, 6, seed=75)
    exp = torch_ref.assign(x, means, covs, w, cov)
    assert_labels(exp.clone(), x, means, covs, w, cov)
    l64 = f64_em._logits(x.double(), cov, means.double(), covs.double(), w.double())[0]
    top2 = l64.topk(2, dim=-1)
    row = int((top2.values[:, 0] - top2.values[:, 1]).argmin())
    planted = exp.clone()
    planted[0, row] = int(top2.indices[row, 1])          # the runner-up, closest of all rows to a tie
    with pytest.raises(AssertionError):
        assert_labels(planted, x, means, covs, w, cov)


def test_params_arbiter_selects_the_distribution_rule_only_when_the_oracle_is_off():
    """judge.arbiter_params_ok: the largest-error rule; the distribution rule
    only where the oracle itself is ILL_CONDITIONED bars or more from float64."""
    from oracle import judge
    well = {"p99": 0.1, "max": 0.9}          # the oracle within the bar
    assert judge.arbiter_params_ok({"p99": 0.1, "max": 1.9}, well)
    assert not judge.arbiter_params_ok({"p99": 0.1, "max": 2.5}, well)       # one element off, oracle fine
    ill = {"p99": 0.2, "max": 1.2}           # the oracle itself outside the bar
    assert judge.arbiter_params_ok({"p99": 0.27, "max": 3.9}, ill)          # noisy largest error, same bulk
    assert not judge.arbiter_params_ok({"p99": 0.9, "max": 3.9}, ill)       # bulk moved: systematic
    assert not judge.arbiter_params_ok({"p99": 0.27, "max": 40.0}, ill)     # gross single error
