"""The BASELINE configs' own recipes at their full sizes against the CPU oracle.

Data and initial parameters come from bench.make_data (seeded synthetic data
of each config's recipe); the same values go to both sides (bf16 x: the
oracle computes in fp32 on the bf16 values and keeps the means in bf16,
``bf16_means``).

Bars (the north star's, oracle/judge.py): mean log-likelihood rtol 1e-5 per
iteration for fp32 x and 2e-3 for bf16 x; fp32 parameters element-wise rtol
1e-4 with absolute floors 1e-5·rms(x) (means), 1e-5·mean(x²) (covariances)
and 1e-7 (weights); bf16 parameters 2e-3 of their scale, the bf16 means one
bf16 ulp more; labels equal except near-ties.

  * C1 (spherical fp32, 20 iterations) and C4 (tied fp32, 10 iterations):
    whole trajectories at the literal bars.
  * C2 (spherical bf16, N = 4,194,304): two iterations, each from the
    oracle's state (the reference's chained max_iters=1 protocol), at the
    bf16 bars; labels from the HIP kernel under the oracle's final
    parameters against the oracle's labels.
  * C3 (diag fp32, 10 iterations) and C5 (full fp32, B = 16, 10 iterations
    each from the oracle's state, then predict_proba + score_samples under
    the oracle's parameters): the log-likelihood at the literal bar.  For
    the parameters and the C5 tail the fp32 oracle itself is up to ~27 bars
    (C3 trajectory) and ~2 bars (a C5 step) away from a float64 computation
    from the same inputs, so no fp32 implementation with another summation
    order can meet the bar against it everywhere; there the float64 result
    arbitrates (oracle/judge.py): at C3, HIP's largest error against float64
    must be at most twice the oracle's own largest error, or within two bars
    of float64 (arbiter_ok); at C5, where single elements of both results
    land several bars from float64 (covariance condition numbers up to
    ~1400), the distribution rule (arbiter_distribution_ok: 99th percentile
    within 2x of the oracle's, largest error within 5x of the oracle's or one
    bar).  Each test prints the error distributions (median, 99th percentile,
    largest, in bars).

These tests run the oracle at full size on the host (about 1-2 minutes each on
16 cores), hence their own time limits.
"""

import pytest
import torch

import bench
from gmmxx_amd import _hip, em
from oracle import f64_em, judge, torch_ref
from tests.test_hip_parity import assert_labels

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _data(name):
    x, m0, c0, w0 = bench.make_data(name, torch.device(DEV))
    torch.cuda.synchronize()
    return x, m0, c0, w0, x.float().cpu()


def _dist(tag, got, ref, kind, x, bf16=False):
    d = judge.error_distribution(got, ref, kind, x, bf16)
    print(f"  {tag} {kind}: median {d['median']:.3g} p99 {d['p99']:.3g} max {d['max']:.3g} bars, "
          f"{d['outside']} of {d['elements']} outside", flush=True)
    return d


def _ll_literal(got, exp, tol, what):
    rel = [abs(g - e) / abs(e) for g, e in zip(got, exp)]
    print(f"  {what}: largest relative lower-bound difference {max(rel):.3g} (bar {tol:g})", flush=True)
    assert max(rel) <= tol, (what, rel)


def _fit_labels_report(labels, e_lab):
    differ = int((labels.cpu() != e_lab).sum())
    print(f"  labels: the HIP fit and the oracle fit differ on {differ} of {labels.numel()} rows "
          f"(their final parameters differ within the bars)", flush=True)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["c1", "c4"])
def test_config_trajectory_literal_bars(hip, name):
    """C1 and C4: the whole fit at the literal bars, no float64 arbiter."""
    cfg = bench.CONFIGS[name]
    print(f"[baseline config, full size] {name}: {cfg['desc']}", flush=True)
    x, m0, c0, w0, xc = _data(name)
    cov, k, iters = cfg["cov"], cfg["K"], cfg["iters"]
    labels, m, c, w, info = em.fit(x, k, cov, max_iters=iters, tol=0.0, init_means=m0, init_covs=c0,
                                   init_weights=w0, record_all_lower_bounds=True)
    e_lab, e_m, e_c, e_w, e_info = torch_ref.fit(xc, k, cov, max_iters=iters, tol=0.0, init_means=m0.cpu(),
                                                 init_covs=c0.cpu(), init_weights=w0.cpu())
    assert info["n_iter"] == e_info["n_iter"] == iters
    _ll_literal(info["lower_bound_history"], e_info["lower_bound_history"], 1e-5, "lower bounds")
    for got, exp, kind in ((m, e_m, "means"), (c, e_c, "covs"), (w, e_w, "weights")):
        _dist("hip vs oracle", got, exp, kind, xc)
        res = judge.judge_params(got, exp, kind, xc, False)
        assert res["outside_bar"] == 0, res
    # labels: the HIP kernel against the oracle's assignment under the same parameters
    assert_labels(labels, xc, m.cpu(), c.cpu(), w.cpu(), cov)
    _fit_labels_report(labels, e_lab)


@pytest.mark.timeout(900)
def test_c2_full_size_per_iteration(hip):
    """C2 at N = 4,194,304: two iterations, each from the oracle's state."""
    cfg = bench.CONFIGS["c2"]
    print(f"[baseline config, full size] c2: {cfg['desc']}", flush=True)
    x, m0, c0, w0, xc = _data("c2")
    k = cfg["K"]
    ws = hip.Workspace(hip.problem("spherical", x.dtype, *x.shape, k), x.device)
    lb = torch.zeros(1, device=DEV)
    means, covs, w = m0.cpu().to(torch.bfloat16).float(), c0.cpu(), w0.cpu()
    for it in range(2):
        e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(xc, "spherical", means, covs, w, bf16_means=True)
        m_d, c_d, w_d = (t.to(DEV).contiguous() for t in (means, covs, w))
        hip.em_step("spherical", x, m_d, c_d, w_d, lb, ws=ws)
        torch.cuda.synchronize()
        print(f" iteration {it}:", flush=True)
        _ll_literal([float(lb)], [e_lb], 2e-3, "lower bound")
        for got, exp, kind in ((m_d, e_m, "means"), (c_d, e_c, "covs"), (w_d, e_w, "weights")):
            _dist("hip vs oracle", got, exp, kind, xc, bf16=True)
            res = judge.judge_params(got, exp, kind, xc, True)
            assert res["outside_bar"] == 0, res
        means, covs, w = e_m, e_c, e_w
    # labels: the HIP kernel under the oracle's final parameters against the oracle's labels
    _, labels = hip.score("spherical", x, means.to(DEV), covs.to(DEV), w.to(DEV), want_scores=False, ws=ws)
    assert_labels(labels, xc, means, covs, w, "spherical")


@pytest.mark.timeout(900)
def test_c3_full_size_trajectory(hip):
    """C3: the whole fit; lower bounds at the literal bar, parameters at the
    bar or within the float64 arbiter."""
    cfg = bench.CONFIGS["c3"]
    print(f"[baseline config, full size] c3: {cfg['desc']}", flush=True)
    x, m0, c0, w0, xc = _data("c3")
    cov, k, iters = cfg["cov"], cfg["K"], cfg["iters"]
    labels, m, c, w, info = em.fit(x, k, cov, max_iters=iters, tol=0.0, init_means=m0, init_covs=c0,
                                   init_weights=w0, record_all_lower_bounds=True)
    e_lab, e_m, e_c, e_w, e_info = torch_ref.fit(xc, k, cov, max_iters=iters, tol=0.0, init_means=m0.cpu(),
                                                 init_covs=c0.cpu(), init_weights=w0.cpu())
    _ll_literal(info["lower_bound_history"], e_info["lower_bound_history"], 1e-5, "lower bounds")
    truth = f64_em.trajectory(xc, cov, m0.cpu(), c0.cpu(), w0.cpu(), iters)
    for got, exp, kind, j in ((m, e_m, "means", 1), (c, e_c, "covs", 2), (w, e_w, "weights", 3)):
        _dist("hip vs oracle", got, exp, kind, xc)
        h = _dist("hip vs float64", got, truth[j], kind, xc)["max"]
        o = _dist("oracle vs float64", exp, truth[j], kind, xc)["max"]
        if judge.judge_params(got, exp, kind, xc, False)["outside_bar"]:
            assert judge.arbiter_ok(h, o), (kind, h, o)
    assert_labels(labels, xc, m.cpu(), c.cpu(), w.cpu(), cov)
    _fit_labels_report(labels, e_lab)


@pytest.mark.timeout(900)
def test_c5_full_size_per_iteration_and_tail(hip):
    """C5 (B = 16): ten iterations, each from the oracle's state, then the
    config's tail -- predict_proba + score_samples on all points under the
    oracle's final parameters."""
    cfg = bench.CONFIGS["c5"]
    print(f"[baseline config, full size] c5: {cfg['desc']}", flush=True)
    x, m0, c0, w0, xc = _data("c5")
    cov, k, iters = cfg["cov"], cfg["K"], cfg["iters"]
    ws = hip.Workspace(hip.problem(cov, x.dtype, *x.shape, k), x.device)
    lb = torch.zeros(1, device=DEV)
    means, covs, w = m0.cpu(), c0.cpu(), w0.cpu()
    for it in range(iters):
        e_m, e_c, e_w, e_lb = torch_ref.fit_one_iteration_stats(xc, cov, means, covs, w)
        m_d, c_d, w_d = (t.to(DEV).contiguous() for t in (means, covs, w))
        hip.em_step(cov, x, m_d, c_d, w_d, lb, ws=ws)
        torch.cuda.synchronize()
        print(f" iteration {it}:", flush=True)
        _ll_literal([float(lb)], [e_lb], 1e-5, "lower bound")
        t_m, t_c, t_w, _ = f64_em.em_step(xc, cov, means, covs, w)
        for got, exp, t, kind in ((m_d, e_m, t_m, "means"), (c_d, e_c, t_c, "covs"), (w_d, e_w, t_w, "weights")):
            if judge.judge_params(got, exp, kind, xc, False)["outside_bar"]:
                _dist("hip vs oracle", got, exp, kind, xc)
                h = _dist("hip vs float64", got, t, kind, xc)
                o = _dist("oracle vs float64", exp, t, kind, xc)
                assert judge.arbiter_distribution_ok(h, o), (it, kind, h, o)
        means, covs, w = e_m, e_c, e_w
    # the tail under the oracle's final parameters
    md, cd, wd = means.to(DEV), covs.to(DEV), w.to(DEV)
    proba, scores = _hip.predict_proba_score(cov, x, md, cd, wd, ws=ws)
    e_proba = torch_ref.predict_proba(xc, means, covs, w, cov)
    e_scores = torch_ref.score_samples(xc, means, covs, w, cov)
    t_proba, t_scores = f64_em.proba_scores(xc, cov, means, covs, w)
    # responsibilities: absolute bar 2e-4
    def in_bars(err, band):
        r = (err / band).flatten()
        q = torch.quantile(r[:1 << 24].float(), torch.tensor([0.5, 0.99])).tolist()
        return {"median": q[0], "p99": q[1], "max": float(r.max())}
    out = int(((proba.cpu() - e_proba).abs() > 2e-4).sum())
    hp = in_bars((proba.cpu().double() - t_proba).abs(), 2e-4)
    op = in_bars((e_proba.double() - t_proba).abs(), 2e-4)
    print(f"  proba: {out} of {proba.numel()} outside 2e-4 of the oracle; error vs float64 (x 2e-4) "
          f"hip {hp}, oracle {op}", flush=True)
    if out:
        assert judge.arbiter_distribution_ok(hp, op), (hp, op)
    # per-sample log-likelihoods: rtol 1e-5 with a floor of 1e-5 of the mean magnitude
    band = 1e-5 * e_scores.double().abs() + 1e-5 * float(e_scores.abs().mean())
    out = int(((scores.cpu().double() - e_scores.double()).abs() > band).sum())
    hs = in_bars((scores.cpu().double() - t_scores).abs(), band)
    os_ = in_bars((e_scores.double() - t_scores).abs(), band)
    print(f"  scores: {out} of {scores.numel()} outside the bar; error vs float64 (in bars) "
          f"hip {hs}, oracle {os_}", flush=True)
    if out:
        assert judge.arbiter_distribution_ok(hs, os_), (hs, os_)
    # labels: the HIP kernel under the oracle's parameters against the oracle's
    _, labels = _hip.score(cov, x, md, cd, wd, want_scores=False, ws=ws)
    assert_labels(labels, xc, means, covs, w, cov)
