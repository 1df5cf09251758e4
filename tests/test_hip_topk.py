"""Approximate top-k EM on the GPU against the CPU oracle.

``gmmxx_hip_estep_stats_topk`` keeps, per row, the top_k largest logits (ties:
lower component index first), normalises the responsibilities over them and
scatters them into the statistics; the oracle does the same with torch.topk
(gmmxx/torch_fallback.py:667-777).  The seeded blob problems have no logit ties
at the top_k boundary, so both pick the same components.  Tolerances as for
the exact statistics: rtol 1e-4 (fp32) / 2e-3 (bf16) against the statistic's
scale; mean log-likelihood rtol 1e-5 (fp32) / 2e-3 (bf16); bf16 means, bf16
values on both sides, one bf16 ulp more than the bf16 bar.
"""

import ctypes

import pytest
import torch

from gmmxx_amd import GMMXX, em, large_n
from oracle import torch_ref
from tests.test_hip_parity import assert_bf16_means, make_problem, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # cov, B, N, D, K, dtype, top_k
    ("spherical", 2, 6000, 32, 64, torch.float32, 4),
    ("spherical", 1, 777, 5, 3, torch.float32, 2),
    ("spherical", 1, 20000, 128, 300, torch.bfloat16, 8),    # D = 128 bf16: augmented-row pass first
    ("spherical", 2, 5000, 128, 1000, torch.bfloat16, 2),
    ("spherical", 1, 9000, 128, 100, torch.bfloat16, 1),
    ("spherical", 2, 6000, 32, 64, torch.bfloat16, 3),       # shapes the fused single pass serves in exact EM
    ("spherical", 1, 5000, 20, 10, torch.bfloat16, 9),       # top_k = K - 1
    ("diag", 2, 3000, 20, 40, torch.float32, 5),
    ("diag", 1, 8000, 64, 512, torch.float32, 16),
    ("tied", 2, 1000, 7, 9, torch.float32, 8),
    ("tied", 1, 10000, 64, 256, torch.float32, 4),
    ("full", 2, 1000, 3, 5, torch.float32, 1),
    ("full", 1, 6000, 16, 32, torch.float32, 3),
    ("full", 2, 5000, 40, 6, torch.float32, 1),              # D > 16: hard assignment on the whitening kernels
    ("full", 1, 6000, 64, 5, torch.float32, 2),              # D > 16: transposed logits, top-k selection
    ("full", 2, 3000, 24, 9, torch.float32, 8),              # D > 16, top_k = K - 1
    ("full", 1, 4000, 100, 5, torch.float32, 1),             # 64 < D <= 128: two-wave statistics, hard
    ("full", 2, 3000, 128, 6, torch.float32, 3),             # D = 128: two-wave statistics, top-k
]


def _id(c):
    return f"{c[0]}-B{c[1]}-N{c[2]}-D{c[3]}-K{c[4]}-{str(c[5]).split('.')[-1]}-top{c[6]}"


def _close(got, exp, tol):
    torch.testing.assert_close(got.cpu(), exp, rtol=tol, atol=tol * float(exp.abs().max()))


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_topk_stats_match_oracle(hip, case):
    cov, b, n, d, k, dt, top_k = case
    print(f"[topk stats] {_id(case)}", flush=True)
    x, means, covs, w = make_problem(cov, b, n, d, k, seed=41, dtype=dt)
    nk, sx, sq, ll = hip.estep_stats_topk(cov, to_dev(x, dt), to_dev(means), to_dev(covs), to_dev(w), top_k)
    torch.cuda.synchronize()
    e_nk, e_sx, e_sq, e_ll = torch_ref.estep_stats_topk(x, cov, means, covs, w, top_k)
    tol = 1e-4 if dt == torch.float32 else 2e-3
    _close(nk, e_nk, tol)
    _close(sx, e_sx, tol)
    if sq is not None:
        _close(sq, e_sq, tol)
    assert float(ll) == pytest.approx(float(e_ll), rel=1e-5 if dt == torch.float32 else 2e-3)
    # every row hands out exactly one unit of responsibility
    assert float(nk.sum()) == pytest.approx(b * n, rel=1e-5)


# EM trajectories are compared only on well-conditioned problems (at least 20
# rows per component): with a few rows per component variances collapse and
# fp32 rounding differences grow chaotically in both implementations.
FIT_CASES = [c for c in CASES if c[2] >= 20 * c[4]] + [("spherical", 1, 40000, 128, 1000, torch.bfloat16, 2)]


@pytest.mark.parametrize("case", FIT_CASES, ids=_id)
def test_topk_fit_matches_oracle(hip, case):
    cov, b, n, d, k, dt, top_k = case
    print(f"[topk fit] {_id(case)}", flush=True)
    x, means, covs, w = make_problem(cov, b, n, d, k, seed=42, dtype=dt)
    iters = 4
    _, m, c, wt, info = em.fit(to_dev(x, dt), k, cov, max_iters=iters, tol=0.0, init_means=means,
                               init_covs=covs, init_weights=w, approx_top_k=top_k, compute_labels=False,
                               record_all_lower_bounds=True)
    torch.cuda.synchronize()
    _, e_m, e_c, e_w, e_info = torch_ref.fit(x, k, cov, max_iters=iters, tol=0.0, init_means=means,
                                             init_covs=covs, init_weights=w, approx_top_k=top_k,
                                             compute_labels=False, bf16_means=dt == torch.bfloat16)
    assert info["approximate_em_enabled"] and info["approx_top_k"] == top_k
    ll_tol = 1e-5 if dt == torch.float32 else 2e-3
    for a, e in zip(info["lower_bound_history"], e_info["lower_bound_history"]):
        assert a == pytest.approx(e, rel=ll_tol)
    ptol = 1e-4 if dt == torch.float32 else 2e-3
    if dt == torch.float32:
        _close(m, e_m, ptol)
    else:
        assert_bf16_means(m, e_m)
    _close(c, e_c, ptol)
    _close(wt, e_w, ptol)


@pytest.mark.parametrize("cov", ["spherical", "tied"])
def test_topk_fit_row_chunks(hip, monkeypatch, cov):
    """Several row chunks (small logit budget) give the one-chunk result."""
    x, means, covs, w = make_problem(cov, 2, 9000, 16, 24, seed=43)
    out = []
    for budget in (1 << 30, 24 * 4 * 2 * 4096):
        monkeypatch.setattr(em, "_TOPK_LOGIT_BYTES", budget)
        _, m, c, wt, info = em.fit(to_dev(x), 24, cov, max_iters=3, tol=0.0, init_means=means,
                                   init_covs=covs, init_weights=w, approx_top_k=3, compute_labels=False,
                                   record_all_lower_bounds=True)
        out.append((m.cpu(), c.cpu(), wt.cpu(), info["lower_bound_history"]))
    assert em.topk_chunk_rows(2, 9000, 24) == 4096
    (m1, c1, w1, l1), (m2, c2, w2, l2) = out
    for a, e in zip(l1, l2):
        assert a == pytest.approx(e, rel=1e-6)
    _close(m2, m1, 1e-5)
    _close(c2, c1, 1e-5)
    _close(w2, w1, 1e-5)


def test_topk_ties_go_to_lower_index(hip):
    """Components 1 and 2 identical (bit-equal logits), 0 and 3 unreachable:
    with top_k = 1 every row ties between 1 and 2 and the lower index takes the
    whole mass."""
    g = torch.Generator().manual_seed(44)
    x = torch.randn((1, 3000, 8), generator=g)
    means = torch.zeros((1, 4, 8))
    means[0, 0] += 400.0
    means[0, 3] -= 400.0
    covs = torch.ones((1, 4))
    w = torch.full((1, 4), 0.25)
    nk, sx, _, _ = hip.estep_stats_topk("spherical", to_dev(x), to_dev(means), to_dev(covs), to_dev(w), 1)
    nk = nk.cpu()
    assert float(nk[0, 1]) == pytest.approx(3000.0, rel=1e-6)
    assert float(nk[0, 0]) == 0.0 and float(nk[0, 2]) == 0.0 and float(nk[0, 3]) == 0.0
    torch.testing.assert_close(sx.cpu()[0, 1], x[0].sum(0), rtol=1e-5, atol=1e-3)


def test_topk_estimator_and_streaming(hip):
    x, _, _, _ = make_problem("diag", 1, 12000, 10, 6, seed=45)
    gm = GMMXX(n_components=6, covariance_type="diag", backend="hip", device=DEV, max_iter=5, tol=0.0,
               approx_top_k=2, seed=1)
    gm.fit(x[0].to(DEV))
    assert gm.approximate_em_enabled_ is True and gm.approx_top_k_ == 2
    gm_exact = GMMXX(n_components=6, covariance_type="diag", backend="hip", device=DEV, max_iter=2,
                     approx_top_k=6)
    gm_exact.fit(x[0].to(DEV))
    assert gm_exact.approximate_em_enabled_ is False and gm_exact.approx_top_k_ is None
    # host input longer than the stream chunk: the streamed loop with top-k sub-chunks
    means = gm.means_b.cpu()
    covs = gm.covariances_b.cpu()
    wt = gm.weights_b.cpu()
    _, m_s, c_s, w_s, info_s = large_n.fit_large_n(x, 6, "diag", device=torch.device(DEV), max_iters=3, tol=0.0,
                                                   chunk_size_N=5000, init_means=means, init_covs=covs,
                                                   init_weights=wt, approx_top_k=2)
    _, m_m, c_m, w_m, info_m = em.fit(x.to(DEV), 6, "diag", max_iters=3, tol=0.0, init_means=means,
                                      init_covs=covs, init_weights=wt, approx_top_k=2, record_all_lower_bounds=True)
    assert info_s["approximate_em_enabled"] and info_s["approx_top_k"] == 2
    for a, e in zip(info_s["lower_bound_history"], info_m["lower_bound_history"]):
        assert a == pytest.approx(e, rel=1e-5)
    _close(m_s, m_m.cpu(), 1e-4)
    _close(c_s, c_m.cpu(), 1e-4)
    _close(w_s, w_m.cpu(), 1e-4)


def test_topk_abi_rejects_bad_top_k(hip):
    """The C entry point refuses top_k outside [1, K-1] before any launch."""
    x, means, covs, w = make_problem("spherical", 1, 256, 8, 4, seed=46)
    xd, md, cd, wd = to_dev(x), to_dev(means), to_dev(covs), to_dev(w)
    prob = hip.problem("spherical", torch.float32, 1, 256, 8, 4)
    ws = hip.Workspace(prob, xd.device, top_k=2)
    out = [torch.empty(s, device=DEV) for s in ((1, 4), (1, 4, 8), (1, 4), (1,))]
    lib = hip.load_library()
    for bad in (0, 4, -1):
        rc = lib.gmmxx_hip_estep_stats_topk(ctypes.byref(prob), xd.data_ptr(), md.data_ptr(), cd.data_ptr(),
                                            wd.data_ptr(), 1e-6, 1e-8, bad, *[t.data_ptr() for t in out],
                                            ws.ptr, ws.nbytes, None)
        assert rc != 0 and b"top_k" in lib.gmmxx_hip_last_error()
    small = ws.nbytes - 256
    rc = lib.gmmxx_hip_estep_stats_topk(ctypes.byref(prob), xd.data_ptr(), md.data_ptr(), cd.data_ptr(),
                                        wd.data_ptr(), 1e-6, 1e-8, 2, *[t.data_ptr() for t in out],
                                        ws.ptr, small, None)
    assert rc != 0 and b"workspace" in lib.gmmxx_hip_last_error()
    with pytest.raises(ValueError):
        hip.estep_stats_topk("spherical", xd, md, cd, wd, 4)
