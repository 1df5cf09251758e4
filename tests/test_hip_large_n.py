"""Large-N streaming (x in host memory, row chunks through HBM) on the GPU.

The streamed fit sums the chunk statistics and applies one M-step per
iteration, so from the same initial parameters it must reproduce the
in-memory EM fit (itself checked against the CPU oracle in test_hip_parity)
and, at the end, the oracle's parameters.  Tolerances: lower bounds rtol 1e-5
(fp32) / 2e-3 (bf16), parameters rtol 1e-4 (fp32) with an absolute floor of
1e-4 of the largest entry, labels equal except float64 near-ties
(|Δlogit| < 1e-5·max(1, |logit|)).  Only the
summation order over rows differs between the paths.
"""

import pytest
import torch

from gmmxx_amd import GMMXX, _hip, em, large_n
from oracle import torch_ref
from tests.test_hip_parity import assert_bf16_means, assert_labels

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def problem(cov, n, d, k, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    centers = (torch.rand((1, k, d), generator=g) * 2 - 1) * 5.0
    lab = torch.randint(0, k, (1, n), generator=g)
    x = torch.gather(centers, 1, lab[..., None].expand(-1, -1, d)) + torch.randn((1, n, d), generator=g)
    x = x.to(dtype)
    means = centers + 0.3 * torch.randn((1, k, d), generator=g)
    if cov == "spherical":
        covs = torch.rand((1, k), generator=g) + 0.5
    elif cov == "diag":
        covs = torch.rand((1, k, d), generator=g) + 0.5
    else:
        shape = (1, d, d) if cov == "tied" else (1, k, d, d)
        a = torch.randn(shape, generator=g) * 0.3
        covs = a @ a.transpose(-1, -2) + 0.7 * torch.eye(d)
    w = torch.rand((1, k), generator=g) + 0.2
    return x, means, covs.float(), (w / w.sum(-1, keepdim=True)).float()


def close(got, exp, rtol):
    torch.testing.assert_close(got.cpu(), exp.cpu(), rtol=rtol, atol=rtol * float(exp.abs().max()))


CASES = [
    # cov, N, D, K, chunk rows, dtype
    ("spherical", 20000, 32, 16, 6000, torch.float32),     # three whole chunks and a tail
    ("spherical", 30000, 128, 300, 8192, torch.bfloat16),  # bf16 kept in bf16, single-pass kernel per chunk
    ("diag", 15000, 24, 12, 4096, torch.float32),
    ("tied", 15000, 16, 10, 5000, torch.float32),          # XᵀX streamed once
    ("full", 12000, 8, 6, 3000, torch.float32),
    ("full", 12000, 48, 4, 5000, torch.float32),          # D > 16: whitening kernels per chunk
]


def _id(c):
    return f"{c[0]}-N{c[1]}-D{c[2]}-K{c[3]}-chunk{c[4]}-{str(c[5]).split('.')[-1]}"


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_streamed_fit_matches_in_memory_fit(hip, case):
    cov, n, d, k, chunk, dt = case
    print(f"[large-n fit] {_id(case)}", flush=True)
    x, means, covs, w = problem(cov, n, d, k, seed=31, dtype=dt)
    iters = 6
    lab_s, m_s, c_s, w_s, info_s = large_n.fit_large_n(
        x, k, cov, device=torch.device(DEV), max_iters=iters, tol=0.0, chunk_size_N=chunk,
        init_means=means, init_covs=covs, init_weights=w)
    lab_m, m_m, c_m, w_m, info_m = em.fit(x.to(DEV), k, cov, max_iters=iters, tol=0.0, init_means=means,
                                          init_covs=covs, init_weights=w, record_all_lower_bounds=True)
    torch.cuda.synchronize()
    assert info_s["large_n_streaming_enabled"] and info_s["n_iter"] == iters
    ll_tol = 1e-5 if dt == torch.float32 else 2e-3
    for a, b in zip(info_s["lower_bound_history"], info_m["lower_bound_history"]):
        assert a == pytest.approx(b, rel=ll_tol)
    ptol = 1e-4 if dt == torch.float32 else 2e-3
    if dt == torch.float32:
        close(m_s, m_m, ptol)
    else:   # bf16 means: one ulp apart where the two sums straddle a rounding midpoint
        assert_bf16_means(m_s, m_m)
    close(c_s, c_m, ptol)
    close(w_s, w_m, ptol)
    assert lab_s.device.type == "cpu" and lab_s.shape == (1, n)
    # the streamed labels are the first-max assignment under the streamed
    # parameters (float64 near-ties aside)
    assert_labels(lab_s, x.float(), m_s.cpu(), c_s.cpu(), w_s.cpu(), cov)


def test_streamed_fit_matches_oracle(hip):
    """Final parameters against the CPU oracle's in-memory fit (spherical fp32)."""
    x, means, covs, w = problem("spherical", 12000, 16, 8, seed=32)
    _, m_s, c_s, w_s, info = large_n.fit_large_n(x, 8, "spherical", device=torch.device(DEV), max_iters=5,
                                                 tol=0.0, chunk_size_N=2500, init_means=means,
                                                 init_covs=covs, init_weights=w)
    _, e_m, e_c, e_w, e_info = torch_ref.fit(x, 8, "spherical", max_iters=5, tol=0.0, init_means=means,
                                             init_covs=covs, init_weights=w)
    for a, b in zip(info["lower_bound_history"], e_info["lower_bound_history"]):
        assert a == pytest.approx(b, rel=1e-5)
    close(m_s, e_m, 1e-4)
    close(c_s, e_c, 1e-4)
    close(w_s, e_w, 1e-4)


@pytest.mark.parametrize("cov", ["spherical", "diag", "full"])
def test_streamed_inference_matches_device(hip, cov):
    x, means, covs, w = problem(cov, 9000, 12, 7, seed=33)
    dev = [t.to(DEV) for t in (means, covs, w)]
    kw = dict(device=torch.device(DEV), chunk_size_N=2048)
    labels = large_n.predict_large_n(x, *dev, cov, **kw)
    scores = large_n.score_samples_large_n(x, *dev, cov, **kw)
    proba = large_n.predict_proba_large_n(x, *dev, cov, **kw)
    e_scores, e_labels = _hip.score(cov, x.to(DEV), *dev)
    e_proba = _hip.predict_proba(cov, x.to(DEV), *dev)
    assert labels.device.type == "cpu" and torch.equal(labels, e_labels.cpu())
    torch.testing.assert_close(scores, e_scores.cpu(), rtol=1e-6, atol=1e-5)
    torch.testing.assert_close(proba, e_proba.cpu(), rtol=0, atol=1e-6)


def test_estimator_streams_long_host_input(hip):
    """GMMXX routes host data longer than chunk_size_data_cpu through the
    streaming path (gmmxx/interface.py:434-439) and its inference likewise."""
    x, _, _, _ = problem("diag", 20000, 10, 5, seed=34)
    gm = GMMXX(n_components=5, covariance_type="diag", backend="hip", device=DEV, chunk_size_data_cpu=4096,
               max_iter=8, tol=0.0, seed=3)
    gm.fit(x[0])
    assert gm.large_n_streaming_enabled_ is True and gm.copy_stream_prefetch_enabled_ is True
    assert gm.fit_info_["init_source"] == "kmeans_sampled"
    labels = gm.predict(x[0])
    scores = gm.score_samples(x[0])
    proba = gm.predict_proba(x[0])
    assert labels.device.type == "cpu" and labels.shape == (20000,)
    m, c, wt = gm.means_b, gm.covariances_b, gm.weights_b
    e_scores, e_labels = _hip.score("diag", x.to(DEV), m, c, wt)
    assert torch.equal(labels, e_labels[0].cpu())
    torch.testing.assert_close(scores, e_scores[0].cpu(), rtol=1e-6, atol=1e-5)
    torch.testing.assert_close(proba.sum(-1), torch.ones(20000), rtol=0, atol=1e-5)
    assert gm.score(x[0]) == pytest.approx(float(e_scores.mean()), rel=1e-6)
    # short host input: copied to the device whole, no streaming
    gm2 = GMMXX(n_components=5, covariance_type="diag", backend="hip", device=DEV, max_iter=3, tol=0.0)
    gm2.fit(x[0, :3000])
    assert gm2.large_n_streaming_enabled_ is False
