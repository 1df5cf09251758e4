"""GPU tests of the reference-named function surface (gmmxx/__init__.py:1-34,
cuda_ops.py:11-87) against the CPU oracle: the ``*_torch_native_chunked``
inference functions, ``hip_ops`` and ``batch_gmm_*`` run the same kernels as
the ``_hip`` entry points, so the bars are those of test_hip_parity (labels
equal on well-separated blobs, log-likelihoods rtol 1e-5 with a floor of 1e-5 of
the mean magnitude, responsibilities within 2e-5 absolute, fit lower bounds
rtol 1e-5)."""

import math

import pytest
import torch

import gmmxx_amd
from gmmxx_amd import hip_ops
from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _problem(cov, b=2, n=3000, d=8, k=6, seed=11):
    g = torch.Generator().manual_seed(seed)
    centers = (torch.rand((b, k, d), generator=g) * 2 - 1) * 6.0
    lab = torch.randint(0, k, (b, n), generator=g)
    x = torch.gather(centers, 1, lab[..., None].expand(-1, -1, d)) + torch.randn((b, n, d), generator=g)
    means = centers + 0.1 * torch.randn((b, k, d), generator=g)
    w = torch.full((b, k), 1.0 / k)
    if cov == "spherical":
        covs = 0.8 + 0.4 * torch.rand((b, k), generator=g)
    elif cov == "diag":
        covs = 0.8 + 0.4 * torch.rand((b, k, d), generator=g)
    else:
        a = 0.2 * torch.randn((b, k, d, d), generator=g)
        covs = a @ a.transpose(-1, -2) + torch.eye(d)
        if cov == "tied":
            covs = covs[:, 0]
    return x, means, covs, w


@pytest.mark.parametrize("cov", ["spherical", "diag", "tied", "full"])
def test_chunked_inference_functions(cov):
    x, m, c, w = _problem(cov)
    print(f"[reference-names chunked] {cov}", flush=True)
    xd, md, cd, wd = (t.to(DEV) for t in (x, m, c, w))
    pre = {"diag": "diagonal"}.get(cov, cov)
    lab = getattr(gmmxx_amd, f"{pre}_assign_torch_native_chunked")(xd, md, cd, wd)
    sc = getattr(gmmxx_amd, f"{pre}_score_samples_torch_native_chunked")(xd, md, cd, wd)
    pr = getattr(gmmxx_amd, f"{pre}_predict_proba_torch_native_chunked")(xd, md, cd, wd)
    e_lab = torch_ref.assign(x, m, c, w, cov)
    e_sc = torch_ref.score_samples(x, m, c, w, cov)
    e_pr = torch_ref.predict_proba(x, m, c, w, cov)
    assert torch.equal(lab.cpu(), e_lab)
    torch.testing.assert_close(sc.cpu(), e_sc, rtol=1e-5, atol=1e-5 * float(e_sc.abs().mean()))
    torch.testing.assert_close(pr.cpu(), e_pr, rtol=0, atol=2e-5)
    # hip_ops: the cuda_ops names with the reference ops' arguments (log-weights;
    # the Cholesky factor for tied and full), int32 labels
    lw = wd.log()
    par = torch.linalg.cholesky(cd) if cov in ("tied", "full") else cd
    lab_o = getattr(hip_ops, f"{cov}_assign")(xd, md, par, lw)
    assert lab_o.dtype == torch.int32 and torch.equal(lab_o.cpu().long(), e_lab)
    lse_o = getattr(hip_ops, f"{cov}_logsumexp")(xd, md, par, lw)
    torch.testing.assert_close(lse_o.cpu(), e_sc, rtol=1e-5, atol=1e-5 * float(e_sc.abs().mean()))
    r_o = getattr(hip_ops, f"{cov}_resp")(xd, md, par, lw, lse_o)
    torch.testing.assert_close(r_o.cpu(), e_pr, rtol=0, atol=2e-5)
    # a log_norm shifted by c scales every responsibility by e^-c
    r_s = getattr(hip_ops, f"{cov}_resp")(xd, md, par, lw, lse_o + 0.5)
    torch.testing.assert_close(r_s.cpu(), e_pr * math.exp(-0.5), rtol=1e-5, atol=2e-5)


def test_hip_ops_fused_spherical_is_one_em_iteration():
    """fused_spherical / soft_update_spherical (_cuda.py:1056-1088, :415-682):
    the oracle's iteration from the same parameters, and the E-step's
    per-sample log-likelihood and labels under the input parameters."""
    x, m, c, w = _problem("spherical")
    print("[reference-names fused_spherical]", flush=True)
    xd, md, cd, wd = (t.to(DEV) for t in (x, m, c, w))
    mh, vh, wh, lse, lab = hip_ops.fused_spherical(xd, md, cd, wd.log(), 1e-6)
    e_m, e_c, e_w, _ = torch_ref.fit_one_iteration_stats(x, "spherical", m, c, w)
    torch.testing.assert_close(mh.cpu(), e_m, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(vh.cpu(), e_c, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(wh.cpu(), e_w, rtol=1e-4, atol=1e-7)
    e_sc = torch_ref.score_samples(x, m, c, w, "spherical")
    torch.testing.assert_close(lse.cpu(), e_sc, rtol=1e-5, atol=1e-5 * float(e_sc.abs().mean()))
    assert lab.dtype == torch.int32 and torch.equal(lab.cpu().long(), torch_ref.assign(x, m, c, w, "spherical"))
    out = hip_ops.soft_update_spherical(xd, md, cd, wd.log(), 1e-6, compute_ids=False)
    assert out[4] is None and torch.equal(out[0], mh) and torch.equal(out[3], lse)


@pytest.mark.parametrize("cov", ["spherical", "diag", "tied", "full"])
def test_batch_gmm_reference_names(cov):
    x, m, c, w = _problem(cov, n=2000)
    print(f"[reference-names batch_gmm] {cov}", flush=True)
    name = {"spherical": "Spherical", "diag": "Diagonal", "tied": "Tied", "full": "Full"}[cov]
    fn = getattr(gmmxx_amd, f"batch_gmm_{name}")
    assert fn is getattr(gmmxx_amd, f"batch_gmm_{name}_torch_native")
    labels, mh, ch, wh, info = fn(x.to(DEV), 6, max_iters=4, tol=0.0, init_means=m.to(DEV),
                                  init_variances=c.to(DEV), init_weights=w.to(DEV), chunk_size_N=4096,
                                  record_all_lower_bounds=True)
    e_lab, e_m, e_c, e_w, e_info = torch_ref.fit(x, 6, cov, max_iters=4, tol=0.0, init_means=m, init_covs=c,
                                                 init_weights=w)
    assert info["n_iter"] == e_info["n_iter"] == 4
    torch.testing.assert_close(torch.tensor(info["lower_bound_history"]),
                               torch.tensor(e_info["lower_bound_history"]), rtol=1e-5, atol=0)
    torch.testing.assert_close(mh.cpu(), e_m, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(wh.cpu(), e_w, rtol=1e-4, atol=1e-6)
