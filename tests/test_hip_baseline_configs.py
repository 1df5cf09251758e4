"""The BASELINE configs' own recipes (bench.py make_data: seeded synthetic data,
the configs' initial parameters) against the CPU oracle.

C1 runs at its full size (N = 100,000, D = 32, K = 64, 20 iterations); C2-C5 at
reduced N with the recipe, K, D, B and iteration count of the config.  The same
data and initial parameters go to both sides (bf16 x: the oracle computes in
fp32 on the bf16 values and keeps the means in bf16, ``bf16_means``).  Bars and the float64 arbiter: oracle/judge.py
(log-likelihood rtol 1e-5 fp32 / 2e-3 bf16; fp32 parameters element-wise rtol
1e-4 with stated floors; a value outside the bar passes only if it is at least
as close to the float64 result from the same inputs as the oracle's is,
within a factor 4).  The recipes start from random data rows with few rows per
component at these N, where EM is ill-conditioned enough that the fp32 oracle
itself leaves the bar against float64 (measured: C3 1.3e-4, C5 9.5e-4 relative
on the lower bound after 10 iterations).

Two checks per config:
  * per iteration: from the oracle's state at iteration i, one HIP em_step
    gives the oracle's lower bound of iteration i and its parameters of
    iteration i + 1 (the reference's chained max_iters=1 protocol);
  * the whole fit: lower-bound history and final parameters (fp32; for bf16 x
    the bar is the log-likelihood), labels equal to the first-max assignment
    under the fit's own parameters except |Δlogit| < 1e-5·max(1, |l|).
"""

import pytest
import torch

import bench
from gmmxx_amd import _hip, em
from oracle import f64_em, judge, torch_ref
from tests.test_hip_parity import assert_labels

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# config, rows per problem (None: full size)
RUNS = [("c1", None), ("c2", 65536), ("c3", 65536), ("c4", 65536), ("c5", 8192)]


def _data(name, n):
    x, m0, c0, w0 = bench.make_data(name, torch.device(DEV), n=n)
    torch.cuda.synchronize()
    return x, m0, c0, w0, x.float().cpu()


def _check(res, what):
    print(f"  {what}: {res}", flush=True)
    assert res["unexplained"] == 0, f"{what}: {res}"


@pytest.mark.parametrize("name,n", RUNS, ids=[r[0] for r in RUNS])
def test_config_recipe_per_iteration(hip, name, n):
    cfg = bench.CONFIGS[name]
    print(f"[baseline-config per-iteration] {name} N={n or cfg['N']}", flush=True)
    x, m0, c0, w0, xc = _data(name, n)
    cov, k, iters, bf = cfg["cov"], cfg["K"], cfg["iters"], x.dtype == torch.bfloat16
    ll_tol = 2e-3 if bf else 1e-5
    ws = hip.Workspace(hip.problem(cov, x.dtype, *x.shape, k), x.device)
    gram = hip.gram(x, ws) if cov == "tied" else None
    lb = torch.zeros(1, device=DEV)
    means, covs, w = m0.cpu(), c0.cpu(), w0.cpu()
    worst = {}
    for it in range(iters):
        e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(xc, cov, means, covs, w, bf16_means=bf)
        m_d, c_d, w_d = (t.to(DEV).contiguous() for t in (means, covs, w))
        hip.em_step(cov, x, m_d, c_d, w_d, lb, gram_xx=gram, ws=ws)
        torch.cuda.synchronize()
        truth = []

        def t64(i, _m=means, _c=covs, _w=w):
            if not truth:
                truth.extend(f64_em.em_step(xc, cov, _m, _c, _w))
            return truth[i]

        _check(judge.judge_ll([float(lb)], [e_lb], ll_tol, lambda: [t64(3)]), f"it {it} lower bound")
        for got, exp, kind, j in ((m_d, e_m, "means", 0), (c_d, e_c, "covs", 1), (w_d, e_w, "weights", 2)):
            res = judge.judge_params(got, exp, kind, xc, bf, lambda j=j: t64(j))
            if res["outside_bar"]:
                print(f"  it {it} {kind}: {res}", flush=True)
                worst.setdefault(kind, []).append((res["hip_vs_float64"], res["oracle_vs_float64"]))
        means, covs, w = e_m, e_c, e_w
    # Per iteration, which of two fp32 implementations lands closer to float64
    # is a matter of rounding luck; over the run, the HIP engine's largest
    # error (relative to the bar) must be within 4x of the oracle's largest.
    for kind, pairs in worst.items():
        h, o = max(p[0] for p in pairs), max(p[1] for p in pairs)
        print(f"  {kind}: largest error vs float64 over the run, hip {h:.3g}, oracle {o:.3g} (x the bar)", flush=True)
        assert h <= max(judge.FACTOR * o, 1.0), (kind, h, o)


@pytest.mark.parametrize("name,n", RUNS, ids=[r[0] for r in RUNS])
def test_config_recipe_trajectory(hip, name, n):
    cfg = bench.CONFIGS[name]
    print(f"[baseline-config trajectory] {name} N={n or cfg['N']}", flush=True)
    x, m0, c0, w0, xc = _data(name, n)
    cov, k, iters, bf = cfg["cov"], cfg["K"], cfg["iters"], x.dtype == torch.bfloat16
    labels, m, c, w, info = em.fit(x, k, cov, max_iters=iters, tol=0.0, init_means=m0, init_covs=c0,
                                   init_weights=w0, record_all_lower_bounds=True)
    e_lab, e_m, e_c, e_w, e_info = torch_ref.fit(xc, k, cov, max_iters=iters, tol=0.0, init_means=m0.cpu(),
                                                 init_covs=c0.cpu(), init_weights=w0.cpu(), bf16_means=bf)
    assert info["n_iter"] == e_info["n_iter"] == iters
    truth = []

    def t64():
        if not truth:
            truth.extend(f64_em.trajectory(xc, cov, m0.cpu(), c0.cpu(), w0.cpu(), iters))
        return truth

    _check(judge.judge_ll(info["lower_bound_history"], e_info["lower_bound_history"], 2e-3 if bf else 1e-5,
                          lambda: t64()[0]), "lower bounds")
    if not bf:
        for got, exp, kind, j in ((m, e_m, "means", 1), (c, e_c, "covs", 2), (w, e_w, "weights", 3)):
            _check(judge.judge_params(got, exp, kind, xc, False, lambda j=j: t64()[j]), f"final {kind}")
    # labels: the first-max assignment under the HIP fit's own parameters
    assert_labels(labels, xc, m.cpu(), c.cpu(), w.cpu(), cov)
    if name == "c5":
        # the config's tail: predict_proba + score_samples on all points, one E-step
        proba, scores = _hip.predict_proba_score(cov, x, m, c, w)
        mc, cc, wc = m.cpu(), c.cpu(), w.cpu()
        e_proba = torch_ref.predict_proba(xc, mc, cc, wc, cov)
        e_scores = torch_ref.score_samples(xc, mc, cc, wc, cov)
        # responsibilities: absolute 2e-4; outside it, the float64 arbiter as for
        # the parameters (largest error vs float64 within 4x of the oracle's)
        t64p = []

        def truth_tail():
            if not t64p:
                t64p.extend(f64_em.proba_scores(xc, cov, mc, cc, wc))
            return t64p

        out = (proba.cpu() - e_proba).abs() > 2e-4
        if bool(out.any()):
            t_proba = truth_tail()[0]
            h = float((proba.cpu().double() - t_proba).abs().max())
            o = float((e_proba.double() - t_proba).abs().max())
            print(f"  proba: {int(out.sum())} of {out.numel()} outside 2e-4; largest error vs float64 "
                  f"hip {h:.3g}, oracle {o:.3g}", flush=True)
            assert h <= max(judge.FACTOR * o, 2e-4)
        # per-sample log-likelihoods: rtol 1e-5 with a floor of 1e-5 of the mean
        # magnitude; outside it, the same float64 arbiter (a near-singular
        # covariance makes a score as ill-conditioned as its Cholesky factor)
        band = 1e-5 * e_scores.double().abs() + 1e-5 * float(e_scores.abs().mean())
        out = (scores.cpu().double() - e_scores.double()).abs() > band
        if bool(out.any()):
            t_scores = truth_tail()[1]
            h = float(((scores.cpu().double() - t_scores).abs() / band).max())
            o = float(((e_scores.double() - t_scores).abs() / band).max())
            print(f"  scores: {int(out.sum())} of {out.numel()} outside the bar; largest error vs float64 "
                  f"(in bars) hip {h:.3g}, oracle {o:.3g}", flush=True)
            assert h <= max(judge.FACTOR * o, 1.0)
