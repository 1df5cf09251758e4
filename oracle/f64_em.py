"""A float64 soft-EM iteration: the truth that fp32 trajectories are judged by.

Test infrastructure, like the rest of ``oracle/``: only ``tests/``, the smoke
check and the checker legs of ``bench.py`` use it; the product never does.

Direct float64 arithmetic (spherical/diag logits from the expanded quadratic
form, full from triangular solves of (x - μ), tied from the solves of x and μ
expanded, natural-log units), with
the reference's iteration prelude and
finalize semantics (variance clamp to reg_covar, weight floor and
renormalisation, active masks, tied/full symmetrisation plus reg·I;
gmmxx/torch_fallback.py:2061-2066, :2293-2305, :2486-2490, :2654-2666,
:2864-2868, :3143-3167).  It is independent of both the fp32 oracle and the
HIP engine, so where those two fp32 implementations drift apart over many
iterations (EM on problems with few rows per component amplifies rounding),
their distance to this float64 trajectory says which one is more accurate.
"""

import math

import torch

LOG_2PI = math.log(2.0 * math.pi)


def _chol(c):
    c = 0.5 * (c + c.transpose(-1, -2))
    L, info = torch.linalg.cholesky_ex(c)
    jitter = 1e-6
    eye = torch.eye(c.shape[-1], dtype=c.dtype)
    for _ in range(6):
        if bool((info == 0).all()):
            break
        L, info = torch.linalg.cholesky_ex(c + jitter * eye)
        jitter *= 10.0
    return L


def _logits(x, cov, means, covs, w):
    b, n, d = x.shape
    logw = torch.log(w)[:, None, :]
    if cov in ("spherical", "diag"):
        # Σ_d (x_d - μ_d)² / v_d expanded; in float64 the cancellation is harmless.
        var = covs[..., None].expand(-1, -1, d) if cov == "spherical" else covs
        p = 1.0 / var
        maha = (torch.bmm(x.square(), p.transpose(1, 2)) - 2.0 * torch.bmm(x, (means * p).transpose(1, 2))
                + (means.square() * p).sum(-1)[:, None, :])
        return -0.5 * (maha.clamp_min(0.0) + d * LOG_2PI + torch.log(var).sum(-1)[:, None, :]) + logw
    Ls = _chol(covs)
    if cov == "tied":
        # one solve for the rows and one for the means: ‖L⁻¹(x - μ)‖² expanded,
        # harmless in float64
        z = torch.linalg.solve_triangular(Ls, x.transpose(1, 2), upper=False).transpose(1, 2)
        nu = torch.linalg.solve_triangular(Ls, means.transpose(1, 2), upper=False).transpose(1, 2)
        maha = z.square().sum(-1)[:, :, None] - 2.0 * torch.bmm(z, nu.transpose(1, 2)) + nu.square().sum(-1)[:, None, :]
        logdet = 2.0 * torch.log(torch.diagonal(Ls, dim1=-2, dim2=-1)).sum(-1)
        return -0.5 * (maha.clamp_min(0.0) + d * LOG_2PI + logdet[:, None, None]) + logw
    out = torch.empty((b, n, means.shape[1]), dtype=torch.float64)
    for kk in range(means.shape[1]):
        L = Ls[:, kk]
        diff = (x - means[:, kk, None, :]).transpose(1, 2)
        z = torch.linalg.solve_triangular(L, diff, upper=False)
        logdet = 2.0 * torch.log(torch.diagonal(L, dim1=-2, dim2=-1)).sum(-1)
        out[:, :, kk] = -0.5 * (z.square().sum(1) + d * LOG_2PI + logdet[:, None])
    return out + logw


def em_step(x, cov, means, covs, w, reg_covar=1e-6, min_weight=1e-8):
    """One iteration in float64: (means, covs, weights, mean log-likelihood)."""
    x, means, covs, w = (t.double() for t in (x, means, covs, w))
    b, n, d = x.shape
    if cov in ("spherical", "diag"):
        covs = covs.clamp_min(reg_covar)
    w = w.clamp_min(min_weight)
    w = w / w.sum(-1, keepdim=True)
    out_nk, out_sx, out_sq, ll = [], [], [], 0.0
    for n0 in range(0, n, 16384):
        xc = x[:, n0:n0 + 16384]
        lg = _logits(xc, cov, means, covs, w)
        lse = torch.logsumexp(lg, -1)
        ll += float(lse.sum())
        r = torch.exp(lg - lse[..., None])
        out_nk.append(r.sum(1))
        out_sx.append(torch.bmm(r.transpose(1, 2), xc))
        if cov == "spherical":
            out_sq.append(torch.bmm(r.transpose(1, 2), xc.square().sum(-1, keepdim=True))[..., 0])
        elif cov == "diag":
            out_sq.append(torch.bmm(r.transpose(1, 2), xc.square()))
        elif cov == "full":
            out_sq.append(torch.einsum("bnk,bnd,bne->bkde", r, xc, xc))
    nk, sx = sum(out_nk), sum(out_sx)
    active = nk > min_weight
    nk_safe = nk.clamp_min(min_weight)
    mu = torch.where(active[..., None], sx / nk_safe[..., None], means)
    if cov == "spherical":
        v = ((sum(out_sq) - nk * mu.square().sum(-1)).clamp_min(0.0) / (nk_safe * d)).clamp_min(reg_covar)
        new_covs = torch.where(active, v, covs)
    elif cov == "diag":
        v = (sum(out_sq) / nk_safe[..., None] - mu.square()).clamp_min(reg_covar)
        new_covs = torch.where(active[..., None], v, covs)
    elif cov == "full":
        outer = mu[..., :, None] * mu[..., None, :]
        c = (sum(out_sq) - nk[..., None, None] * outer) / nk_safe[..., None, None]
        c = 0.5 * (c + c.transpose(-1, -2)) + reg_covar * torch.eye(d, dtype=torch.float64)
        new_covs = torch.where(active[..., None, None], c, covs)
    else:
        outer = mu[..., :, None] * mu[..., None, :]
        c = (torch.bmm(x.transpose(1, 2), x) - (nk[..., None, None] * outer).sum(1)) / n
        new_covs = 0.5 * (c + c.transpose(-1, -2)) + reg_covar * torch.eye(d, dtype=torch.float64)
    new_w = (nk / n).clamp_min(min_weight)
    new_w = new_w / new_w.sum(-1, keepdim=True)
    return mu, new_covs, new_w, ll / (b * n)


def trajectory(x, cov, means, covs, w, iters, reg_covar=1e-6):
    """Lower bounds of `iters` float64 iterations and the final parameters."""
    lbs = []
    for _ in range(iters):
        means, covs, w, lb = em_step(x, cov, means, covs, w, reg_covar)
        lbs.append(lb)
    return lbs, means, covs, w


def proba_scores(x, cov, means, covs, w):
    """float64 responsibilities (B, N, K) and per-sample log-likelihood (B, N)
    under fixed parameters (no iteration prelude)."""
    x, means, covs, w = (t.double() for t in (x, means, covs, w))
    lg = torch.cat([_logits(x[:, n0:n0 + 16384], cov, means, covs, w) for n0 in range(0, x.shape[1], 16384)], 1)
    lse = torch.logsumexp(lg, -1)
    return torch.exp(lg - lse[..., None]), lse
