"""CPU restatement of the reference GMM EM hot path (test infrastructure only).

This module restates, on the CPU with PyTorch fp32 kernels, the soft-EM loops
and inference functions of the reference's pure-PyTorch fallback
(``gmmxx/torch_fallback.py`` of OpsiClear/GMMXX).  It is the parity oracle for
the HIP engine in ``gmmxx_amd``: tests compare the HIP kernels against it on
identical seeded inputs and initial parameters.  It is never imported by the
product package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` call it.

Scope: the EM path with Triton/CUDA disabled, i.e. the branch a CPU tensor
takes through the reference, exact and with approximate top-k responsibilities
(``approx_top_k``).  Every function cites the
reference lines it follows.  The arithmetic order (chunking over N and K,
clamps, casts, the logits formulas) follows the reference op for op, because
that order is what defines parity at fp32 rounding level.

How each part is pinned (checked independently of this restatement):
  * logits / log-likelihood: float64 closed-form Gaussian log densities on
    tiny inputs, and scikit-learn's GaussianMixture E-step (tests/test_oracle_pinned.py);
  * finalize, prelude clamps, jitter retry, label tie-breaking and the
    lower-bound bookkeeping: golden vectors written by the reference's own
    torch fallback (tests/golden/make_golden.py) and closed-form known answers
    restated from the reference's tests;
  * EM trajectory: sklearn's M-step and the golden trajectories;
  * approximate top-k statistics: top_k = 1 equals hard-assignment group-by
    sums over the float64 argmax, top_k = K - 1 with one unreachable component
    equals the exact statistics, and a float64 brute force (sorted logits, then
    scatter) on tiny inputs (tests/test_oracle_pinned.py);
  * k-means initialisation: k-means++ against an independent float64 numpy
    implementation fed the same random numbers, K = S taking every row once,
    one seed per well-separated blob; Lloyd against a float64 brute force and
    the closed-form blob means; hard-label statistics against float64 loops
    (tests/test_oracle_kmeans.py).  The Lloyd stopping rule restates
    flash-kmeans (absent here) and is not pinned;
  * ``bf16_means`` (bf16 input): the rounded means are bf16 values within half
    a bf16 ulp of the pinned fp32 iteration's, whose covariances and weights
    it keeps unchanged (tests/test_oracle_pinned.py).

Difference from the reference that is deliberate: the reference records the
lower bound of non-final iterations as 0.0 for diag/tied/full when ``tol == 0``
and ``verbose`` is false (torch_fallback.py:2668-2679, :3169-3180).  Here every
iteration's lower bound is recorded (``record_all_lower_bounds=True``), which
equals what the reference records with ``verbose=True``; parameters are
unaffected.  Pass ``record_all_lower_bounds=False`` to reproduce the quirk.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

LOG_2PI = math.log(2.0 * math.pi)
DEFAULT_CHUNK_N = 32768
DEFAULT_CHUNK_K = 1024


# ---------------------------------------------------------------------------
# Matrix helpers  (torch_fallback.py:302-334)
# ---------------------------------------------------------------------------

def symmetrize(m: torch.Tensor) -> torch.Tensor:
    """0.5 (M + Mᵀ) over the last two dims (torch_fallback.py:306-307)."""
    return 0.5 * (m + m.transpose(-1, -2))


def regularize(m: torch.Tensor, reg_covar: float) -> torch.Tensor:
    """sym(M) + reg·I (torch_fallback.py:310-313)."""
    eye = torch.eye(m.shape[-1], dtype=m.dtype, device=m.device)
    return symmetrize(m) + reg_covar * eye


def precision_and_logdet(cov: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Cholesky-based precision and log-determinant (torch_fallback.py:316-334).

    A failing factorisation of ANY matrix in the batch triggers the jitter
    ladder 1e-6, 1e-5, ... (6 tries) applied to EVERY matrix of the batch; if
    all six fail the last (partial) factor is used as is.
    """
    c = symmetrize(cov.to(torch.float32))
    d = c.shape[-1]
    try:
        chol = torch.linalg.cholesky(c)
    except RuntimeError:
        eye = torch.eye(d, dtype=c.dtype, device=c.device)
        jitter = 1e-6
        chol = None
        for _ in range(6):
            chol, info = torch.linalg.cholesky_ex(c + jitter * eye)
            if bool((info == 0).all().item()):
                break
            jitter *= 10.0
    precision = torch.cholesky_inverse(chol)
    logdet = 2.0 * torch.log(torch.diagonal(chol, dim1=-2, dim2=-1)).sum(dim=-1)
    return precision, logdet


# ---------------------------------------------------------------------------
# Per-covariance logits  (torch_fallback.py:337-465)
# ---------------------------------------------------------------------------

def spherical_logits(x, x_sq, means, variances, log_weights):
    """log w_k + log N(x | μ_k, σ²_k I), in x's dtype (torch_fallback.py:337-354)."""
    d = x.shape[-1]
    means_sq = means.square().sum(dim=-1)
    dist = (x_sq.unsqueeze(-1) - 2.0 * torch.bmm(x, means.transpose(1, 2))
            + means_sq.unsqueeze(-2)).clamp_min_(0.0)
    log_norm = d * (LOG_2PI + torch.log(variances)).unsqueeze(-2)
    return log_weights.unsqueeze(-2) - 0.5 * (dist / variances.unsqueeze(-2) + log_norm)


def diag_terms(means, variances):
    """Per-component diag constants (torch_fallback.py:2491-2494)."""
    var_f = variances.to(torch.float32)
    precision = var_f.clamp_min(1e-30).reciprocal()
    logdet = torch.log(var_f.clamp_min(1e-30)).sum(dim=-1)
    weighted_means = means.to(torch.float32) * precision
    mean_precision_mean = (means.to(torch.float32) * weighted_means).sum(dim=-1)
    return precision, logdet, weighted_means, mean_precision_mean


def diag_logits(x, log_weights, precision, logdet, weighted_means, mean_precision_mean):
    """Diagonal-covariance logits in fp32 (torch_fallback.py:357-397)."""
    d = x.shape[-1]
    x_f = x.to(torch.float32)
    dist = (torch.bmm(x_f.square(), precision.transpose(1, 2))
            - 2.0 * torch.bmm(x_f, weighted_means.transpose(1, 2))
            + mean_precision_mean.unsqueeze(1)).clamp_min_(0.0)
    log_norm = d * LOG_2PI + logdet
    return log_weights.unsqueeze(1) - 0.5 * (dist + log_norm.unsqueeze(1))


def matrix_terms(means, covariances, covariance_type):
    """Precision, log-det, Pμ and μᵀPμ (torch_fallback.py:2869-2874)."""
    precision, logdet = precision_and_logdet(covariances)
    means_f = means.to(torch.float32)
    if covariance_type == "full":
        precision_means = torch.einsum("bkde,bke->bkd", precision, means_f)
    else:
        precision_means = torch.bmm(means_f, precision.transpose(1, 2))
    mean_precision_mean = (means_f * precision_means).sum(dim=-1)
    return precision, logdet, precision_means, mean_precision_mean


def full_logits(x, log_weights, precision, logdet, precision_means, mean_precision_mean):
    """Full-covariance logits in fp32 (torch_fallback.py:400-432)."""
    d = x.shape[-1]
    x_f = x.to(torch.float32)
    x_p_x = torch.einsum("bnd,bkde,bne->bnk", x_f, precision, x_f)
    cross = torch.bmm(x_f, precision_means.transpose(1, 2))
    quad = (x_p_x - 2.0 * cross + mean_precision_mean.unsqueeze(1)).clamp_min_(0.0)
    log_norm = d * LOG_2PI + logdet
    return log_weights.unsqueeze(1) - 0.5 * (quad + log_norm.unsqueeze(1))


def tied_logits(x, log_weights, precision, logdet, precision_means, mean_precision_mean):
    """Tied-covariance logits in fp32 (torch_fallback.py:435-465)."""
    d = x.shape[-1]
    x_f = x.to(torch.float32)
    x_p_x = torch.einsum("bnd,bde,bne->bn", x_f, precision, x_f)
    cross = torch.bmm(x_f, precision_means.transpose(1, 2))
    quad = (x_p_x.unsqueeze(-1) - 2.0 * cross + mean_precision_mean.unsqueeze(1)).clamp_min_(0.0)
    log_norm = d * LOG_2PI + logdet
    return log_weights.unsqueeze(1) - 0.5 * (quad + log_norm[:, None, None])


class _Model:
    """Evaluates the logits of one fitted/initial model on row chunks.

    Bundles the per-component constants the reference precomputes once per
    iteration (or once per inference call) so the chunk loops below read like
    the reference's loops.
    """

    def __init__(self, covariance_type, means, covs, weights):
        self.cov = covariance_type
        self.means = means
        self.covs = covs
        self.weights = weights
        self.k = means.shape[1]
        if covariance_type == "spherical":
            # Resp pass uses log(w.float()) (:2066); the LSE pass uses
            # log(w) in x.dtype (:481).  Identical for fp32 inputs.
            self.log_w = torch.log(weights.to(torch.float32))
            self.log_w_native = torch.log(weights)
        elif covariance_type == "diag":
            self.log_w = torch.log(weights.to(torch.float32))
            self.terms = diag_terms(means, covs)
        else:
            self.log_w = torch.log(weights.to(torch.float32))
            self.terms = matrix_terms(means, covs, covariance_type)

    def logits(self, x_chunk, x_sq_chunk, k0, k1, *, lse_pass=False):
        sl = slice(k0, k1)
        if self.cov == "spherical":
            lw = self.log_w_native if lse_pass else self.log_w
            return spherical_logits(x_chunk, x_sq_chunk, self.means[:, sl, :],
                                    self.covs[:, sl], lw[:, sl])
        if self.cov == "diag":
            p, ld, wm, mpm = self.terms
            return diag_logits(x_chunk, self.log_w[:, sl], p[:, sl, :], ld[:, sl],
                               wm[:, sl, :], mpm[:, sl])
        p, ld, pm, mpm = self.terms
        if self.cov == "full":
            return full_logits(x_chunk, self.log_w[:, sl], p[:, sl, :, :], ld[:, sl],
                               pm[:, sl, :], mpm[:, sl])
        return tied_logits(x_chunk, self.log_w[:, sl], p, ld, pm[:, sl, :], mpm[:, sl])

    def stream_lse(self, x_chunk, x_sq_chunk, chunk_k):
        """Online log-sum-exp over K tiles (torch_fallback.py:468-596)."""
        bsz, n_chunk, _ = x_chunk.shape
        dt = x_chunk.dtype if self.cov == "spherical" else torch.float32
        m = torch.full((bsz, n_chunk), -torch.inf, dtype=dt)
        s = torch.zeros((bsz, n_chunk), dtype=dt)
        for k0 in range(0, self.k, chunk_k):
            k1 = min(k0 + chunk_k, self.k)
            logits = self.logits(x_chunk, x_sq_chunk, k0, k1, lse_pass=True)
            new_m = torch.maximum(m, logits.max(dim=-1).values)
            s = s * torch.exp(m - new_m) + torch.exp(logits - new_m.unsqueeze(-1)).sum(dim=-1)
            m = new_m
        return m + torch.log(s)


def _x_sq(x):
    return x.square().sum(dim=-1)


# ---------------------------------------------------------------------------
# Inference  (torch_fallback.py:780-1345)
# ---------------------------------------------------------------------------

def assign(x, means, covs, weights, covariance_type, *, chunk_size_N=DEFAULT_CHUNK_N,
           chunk_size_K=DEFAULT_CHUNK_K):
    """argmax_k logits: first maximum inside a K tile, strict '>' across tiles
    (torch_fallback.py:780-821, :824-870, :920-980)."""
    mdl = _Model(covariance_type, means, covs, weights)
    bsz, n, _ = x.shape
    labels = torch.empty((bsz, n), dtype=torch.long)
    x_sq = _x_sq(x) if covariance_type == "spherical" else None
    best_dt = x.dtype if covariance_type == "spherical" else torch.float32
    for n0 in range(0, n, chunk_size_N):
        n1 = min(n0 + chunk_size_N, n)
        xc = x[:, n0:n1, :]
        xs = x_sq[:, n0:n1] if x_sq is not None else None
        best = torch.full((bsz, n1 - n0), -torch.inf, dtype=best_dt)
        best_lab = torch.zeros((bsz, n1 - n0), dtype=torch.long)
        for k0 in range(0, mdl.k, chunk_size_K):
            k1 = min(k0 + chunk_size_K, mdl.k)
            tile, tile_lab = mdl.logits(xc, xs, k0, k1).max(dim=-1)
            upd = tile > best
            best = torch.where(upd, tile, best)
            best_lab = torch.where(upd, tile_lab + k0, best_lab)
        labels[:, n0:n1] = best_lab
    return labels


def score_samples(x, means, covs, weights, covariance_type, *, chunk_size_N=DEFAULT_CHUNK_N,
                  chunk_size_K=DEFAULT_CHUNK_K):
    """Per-sample log-likelihood log Σ_k w_k N(x|k) (torch_fallback.py:983-1130)."""
    mdl = _Model(covariance_type, means, covs, weights)
    bsz, n, _ = x.shape
    out_dt = x.dtype if covariance_type == "spherical" else torch.float32
    scores = torch.empty((bsz, n), dtype=out_dt)
    x_sq = _x_sq(x) if covariance_type == "spherical" else None
    for n0 in range(0, n, chunk_size_N):
        n1 = min(n0 + chunk_size_N, n)
        scores[:, n0:n1] = mdl.stream_lse(x[:, n0:n1, :],
                                          x_sq[:, n0:n1] if x_sq is not None else None,
                                          chunk_size_K)
    return scores


def predict_proba(x, means, covs, weights, covariance_type, *, chunk_size_N=DEFAULT_CHUNK_N,
                  chunk_size_K=DEFAULT_CHUNK_K):
    """Responsibilities exp(l − LSE), LSE streamed first then logits recomputed
    (torch_fallback.py:1133-1345)."""
    mdl = _Model(covariance_type, means, covs, weights)
    bsz, n, _ = x.shape
    out_dt = x.dtype if covariance_type == "spherical" else torch.float32
    probs = torch.empty((bsz, n, mdl.k), dtype=out_dt)
    x_sq = _x_sq(x) if covariance_type == "spherical" else None
    for n0 in range(0, n, chunk_size_N):
        n1 = min(n0 + chunk_size_N, n)
        xc = x[:, n0:n1, :]
        xs = x_sq[:, n0:n1] if x_sq is not None else None
        lse = mdl.stream_lse(xc, xs, chunk_size_K)
        for k0 in range(0, mdl.k, chunk_size_K):
            k1 = min(k0 + chunk_size_K, mdl.k)
            probs[:, n0:n1, k0:k1] = torch.exp(mdl.logits(xc, xs, k0, k1) - lse.unsqueeze(-1))
    return probs


# ---------------------------------------------------------------------------
# Initialisation with explicit parameters  (torch_fallback.py:1348-1894)
# ---------------------------------------------------------------------------

def global_spherical_variance(x, n_components, reg_covar, x_sq=None):
    """(E‖x‖² − ‖E x‖²)/D, clamped (torch_fallback.py:1348-1363)."""
    d = x.shape[-1]
    x_f = x.to(torch.float32)
    mean = x_f.mean(dim=1)
    second = (x_f.square().sum(dim=-1) if x_sq is None else x_sq.to(torch.float32)).mean(dim=1)
    gv = (second - mean.square().sum(dim=-1)).clamp_min(0.0) / float(d)
    return gv.clamp_min(reg_covar).unsqueeze(-1).expand(-1, n_components).clone().to(x.dtype)


def global_diag_variance(x, n_components, reg_covar):
    """Per-feature variance, clamped (torch_fallback.py:1366-1369)."""
    xf = x.to(torch.float32)
    gv = (xf - xf.mean(dim=1, keepdim=True)).square().mean(dim=1).clamp_min(reg_covar)
    return gv.unsqueeze(1).expand(-1, n_components, -1).clone().to(x.dtype)


def global_tied_covariance(x, reg_covar):
    """Centered XᵀX/N + reg·I (torch_fallback.py:1372-1376)."""
    n = x.shape[1]
    xf = x.to(torch.float32)
    c = xf - xf.mean(dim=1, keepdim=True)
    return regularize(torch.bmm(c.transpose(1, 2), c) / float(n), reg_covar).to(x.dtype)


def _init_weights(init_weights, x, k):
    """Uniform or user weights, clamped at 1e-8 and renormalised
    (torch_fallback.py:1635-1643, :1672-1681)."""
    if init_weights is None:
        w = torch.full((x.shape[0], k), 1.0 / float(k), dtype=x.dtype)
    else:
        w = init_weights.clone().to(dtype=x.dtype)
    if w.shape != (x.shape[0], k):
        raise ValueError("init_weights must have shape (B, K)")
    w = w.clamp_min(1e-8)
    return w / w.sum(dim=-1, keepdim=True)


def random_initialize(x, covariance_type, n_components, indices, reg_covar):
    """The random branch of the four initialisers, which is also what
    ``init_params="kmeans"`` runs when flash-kmeans does not import
    (torch_fallback.py:1571-1582 returns None): rows ``indices`` (B, K) of x as
    the means (``_random_init_means`` :1384-1387 with its torch.randint draw
    given), the global (co)variance (:1348-1381) and weights 1/K
    (:1718-1727, :1766-1774, :1826-1834, :1886-1894)."""
    bsz, _, d = x.shape
    means = torch.gather(x, 1, indices[..., None].expand(-1, -1, d)).clone()
    if covariance_type == "spherical":
        covs = global_spherical_variance(x, n_components, reg_covar)
    elif covariance_type == "diag":
        covs = global_diag_variance(x, n_components, reg_covar)
    elif covariance_type == "tied":
        covs = global_tied_covariance(x, reg_covar)
    else:
        covs = global_tied_covariance(x, reg_covar).unsqueeze(1).expand(-1, n_components, -1, -1).clone()
    weights = torch.full((bsz, n_components), 1.0 / float(n_components), dtype=x.dtype)
    return means, covs, weights


def init_user_parameters(x, covariance_type, init_means, init_covs, init_weights, reg_covar,
                         x_sq=None):
    """Explicit-init branch of the four initialisers
    (torch_fallback.py:1661-1682, :1731-1742, :1791-1802, :1851-1862)."""
    means = init_means.clone()
    if means.ndim != 3:
        raise ValueError("init_means must have shape (B, K, D)")
    if covariance_type == "spherical":
        k = means.shape[1]
        var = (init_covs.clone() if init_covs is not None
               else global_spherical_variance(x, k, reg_covar, x_sq=x_sq))
        if var.shape != (x.shape[0], k):
            raise ValueError("init_variances must have shape (B, K)")
        return means, var.clamp_min(reg_covar), _init_weights(init_weights, x, k)
    if means.shape[0] != x.shape[0] or means.shape[2] != x.shape[2]:
        raise ValueError("init_means must have shape (B, K, D) matching x")
    means = means.to(dtype=x.dtype)
    k = means.shape[1]
    d = x.shape[2]
    if covariance_type == "diag":
        var = (init_covs.clone().to(dtype=x.dtype) if init_covs is not None
               else global_diag_variance(x, k, reg_covar))
        if var.shape != (x.shape[0], k, d):
            raise ValueError("init_variances must have shape (B, K, D) for diag covariance")
        return means, var.clamp_min(reg_covar), _init_weights(init_weights, x, k)
    if covariance_type == "full":
        cov = (init_covs.clone().to(dtype=x.dtype) if init_covs is not None
               else global_tied_covariance(x, reg_covar).unsqueeze(1).expand(-1, k, -1, -1).clone())
        if cov.shape != (x.shape[0], k, d, d):
            raise ValueError("init_variances must have shape (B, K, D, D) for full covariance")
        return means, symmetrize(cov).to(x.dtype), _init_weights(init_weights, x, k)
    cov = (init_covs.clone().to(dtype=x.dtype) if init_covs is not None
           else global_tied_covariance(x, reg_covar))
    if cov.shape != (x.shape[0], d, d):
        raise ValueError("init_variances must have shape (B, D, D) for tied covariance")
    return means, symmetrize(cov).to(x.dtype), _init_weights(init_weights, x, k)


# ---------------------------------------------------------------------------
# EM loops  (torch_fallback.py:1897-3336)
# ---------------------------------------------------------------------------

def _spherical_chunk_n(n, d, k, chunk_size_N):
    """CPU-side chunk heuristic (torch_fallback.py:116-127)."""
    if chunk_size_N == 32768 and d == 256 and k <= 64 and n >= 1048576:
        return 65536
    return chunk_size_N



def _accumulate(x, x_sq_all, mdl, covariance_type, chunk_n, chunk_size_K, collect=True):
    """E-step + M-step sufficient statistics of one iteration (the chunk loops of
    torch_fallback.py:2097-2291, :2500-2652, :2911-3141)."""
    bsz, n, d = x.shape
    k = mdl.k
    spherical = covariance_type == "spherical"
    nk = torch.zeros((bsz, k), dtype=torch.float32)
    sum_x = torch.zeros((bsz, k, d), dtype=torch.float32)
    if spherical:
        sum_q = torch.zeros((bsz, k), dtype=torch.float32)
    elif covariance_type == "diag":
        sum_q = torch.zeros((bsz, k, d), dtype=torch.float32)
    elif covariance_type == "full":
        sum_q = torch.zeros((bsz, k, d, d), dtype=torch.float32)
    else:
        sum_q = None
    total_ll = torch.zeros((), dtype=torch.float32)
    for n0 in range(0, n, chunk_n):
        n1 = min(n0 + chunk_n, n)
        xc = x[:, n0:n1, :]
        xcf = xc.to(torch.float32)
        xs = x_sq_all[:, n0:n1] if spherical else None
        if not spherical and k <= chunk_size_K:
            # Single-K-tile branch (:2602-2620, :3054-3090).
            logits = mdl.logits(xc, xs, 0, k)
            lse = torch.logsumexp(logits, dim=-1)
            if collect:
                total_ll = total_ll + lse.sum()
            resp = logits.sub(lse.unsqueeze(-1)).exp_()
            nk += resp.sum(dim=1)
            sum_x += torch.bmm(resp.transpose(1, 2), xcf)
            if covariance_type == "diag":
                sum_q += torch.bmm(resp.transpose(1, 2), xcf.square())
            elif covariance_type == "full":
                sum_q += torch.einsum("bnk,bnd,bne->bkde", resp, xcf, xcf)
            continue
        # Streaming branch (:2210-2291, :2622-2652, :3092-3141).
        lse = mdl.stream_lse(xc, xs, chunk_size_K)
        if collect:
            total_ll = total_ll + lse.sum()
        for k0 in range(0, k, chunk_size_K):
            k1 = min(k0 + chunk_size_K, k)
            resp = torch.exp(mdl.logits(xc, xs, k0, k1) - lse.unsqueeze(-1))
            nk[:, k0:k1] += resp.sum(dim=1)
            sum_x[:, k0:k1, :] += torch.bmm(resp.transpose(1, 2), xcf)
            if spherical:
                sum_q[:, k0:k1] += (resp * xs.unsqueeze(-1)).sum(dim=1)
            elif covariance_type == "diag":
                sum_q[:, k0:k1, :] += torch.bmm(resp.transpose(1, 2), xcf.square())
            elif covariance_type == "full":
                sum_q[:, k0:k1, :, :] += torch.einsum("bnk,bnd,bne->bkde", resp, xcf, xcf)
    return nk, sum_x, sum_q, total_ll


def _topk_logits(mdl, xc, xs, k, chunk_size_K, top_k):
    """Running top-k over component tiles (torch_fallback.py:667-716): the
    kept logits and their component indices, per row."""
    bsz, n_chunk = xc.shape[0], xc.shape[1]
    top_k = min(int(top_k), k)
    best = torch.full((bsz, n_chunk, top_k), -torch.inf, dtype=torch.float32)
    best_idx = torch.zeros((bsz, n_chunk, top_k), dtype=torch.long)
    for k0 in range(0, k, chunk_size_K):
        k1 = min(k0 + chunk_size_K, k)
        logits = mdl.logits(xc, xs, k0, k1).to(torch.float32)
        idx = torch.arange(k0, k1, dtype=torch.long).view(1, 1, k1 - k0).expand(bsz, n_chunk, k1 - k0)
        cand = torch.cat((best, logits), dim=-1)
        cand_idx = torch.cat((best_idx, idx), dim=-1)
        best, pos = cand.topk(top_k, dim=-1)
        best_idx = cand_idx.gather(-1, pos)
    return best, best_idx


def _accumulate_topk(x, x_sq_all, mdl, covariance_type, chunk_n, chunk_size_K, top_k):
    """Approximate top-k sufficient statistics (torch_fallback.py:719-777):
    responsibilities over each row's top-k components only, scattered into the
    statistics; the log-likelihood sums the top-k log-normalisers."""
    bsz, n, d = x.shape
    k = mdl.k
    spherical = covariance_type == "spherical"
    nk = torch.zeros((bsz, k), dtype=torch.float32)
    sum_x = torch.zeros((bsz, k, d), dtype=torch.float32)
    sum_q = {"spherical": lambda: torch.zeros((bsz, k), dtype=torch.float32),
             "diag": lambda: torch.zeros((bsz, k, d), dtype=torch.float32),
             "full": lambda: torch.zeros((bsz, k, d, d), dtype=torch.float32)}.get(covariance_type, lambda: None)()
    total_ll = torch.zeros((), dtype=torch.float32)
    for n0 in range(0, n, chunk_n):
        n1 = min(n0 + chunk_n, n)
        xc = x[:, n0:n1, :]
        xcf = xc.to(torch.float32)
        xs = x_sq_all[:, n0:n1] if spherical else None
        tl, ti = _topk_logits(mdl, xc, xs, k, chunk_size_K, top_k)
        lse = torch.logsumexp(tl, dim=-1)
        resp = torch.exp(tl - lse.unsqueeze(-1))
        total_ll = total_ll + lse.sum()
        for j in range(tl.shape[-1]):
            idx, r = ti[:, :, j], resp[:, :, j]
            nk.scatter_add_(1, idx, r)
            sum_x.scatter_add_(1, idx.unsqueeze(-1).expand(-1, -1, d), r.unsqueeze(-1) * xcf)
            if spherical:
                sum_q.scatter_add_(1, idx, r * xs)
            elif covariance_type == "diag":
                sum_q.scatter_add_(1, idx.unsqueeze(-1).expand(-1, -1, d), r.unsqueeze(-1) * xcf.square())
            elif covariance_type == "full":
                outer = xcf.unsqueeze(-1) * xcf.unsqueeze(-2)
                sum_q.scatter_add_(1, idx[:, :, None, None].expand(-1, -1, d, d), r[:, :, None, None] * outer)
    return nk, sum_x, sum_q, total_ll


@torch.no_grad()
def estep_stats_topk(x, covariance_type, means, covs, weights, top_k, *, reg_covar=1e-6, min_weight=1e-8,
                     chunk_size_N=DEFAULT_CHUNK_N, chunk_size_K=DEFAULT_CHUNK_K):
    """estep_stats with approximate top-k responsibilities (1 <= top_k < K)."""
    spherical = covariance_type == "spherical"
    if covariance_type in ("spherical", "diag"):
        covs = covs.clamp_min(reg_covar)
    weights = weights.clamp_min(min_weight)
    weights = weights / weights.sum(dim=-1, keepdim=True)
    mdl = _Model(covariance_type, means, covs, weights)
    x_sq_all = (x.to(torch.float32) ** 2).sum(dim=-1) if spherical else None
    return _accumulate_topk(x, x_sq_all, mdl, covariance_type, chunk_size_N, chunk_size_K, top_k)


@torch.no_grad()
def estep_stats(x, covariance_type, means, covs, weights, *, reg_covar=1e-6, min_weight=1e-8,
                chunk_size_N=DEFAULT_CHUNK_N, chunk_size_K=DEFAULT_CHUNK_K):
    """Sufficient statistics (nk, Σr·x, Σr·q(x), Σ lse) of one iteration from
    the given parameters, after the iteration prelude (:2061-2066, :2486-2490,
    :2866-2868)."""
    spherical = covariance_type == "spherical"
    if covariance_type in ("spherical", "diag"):
        covs = covs.clamp_min(reg_covar)
    weights = weights.clamp_min(min_weight)
    weights = weights / weights.sum(dim=-1, keepdim=True)
    mdl = _Model(covariance_type, means, covs, weights)
    x_sq_all = (x.to(torch.float32) ** 2).sum(dim=-1) if spherical else None
    n, d, k = x.shape[1], x.shape[2], means.shape[1]
    chunk_n = _spherical_chunk_n(n, d, k, chunk_size_N) if spherical else chunk_size_N
    return _accumulate(x, x_sq_all, mdl, covariance_type, chunk_n, chunk_size_K)


def finalize(covariance_type, nk, sum_x, sum_q, means, covs, *, n, reg_covar=1e-6,
             min_weight=1e-8, total_xx=None, x_dtype=torch.float32):
    """M-step parameter update from sufficient statistics.

    Spherical torch_fallback.py:2293-2305, diag :2654-2666, tied/full
    :3143-3167.  ``sum_q`` is Σr‖x‖² (spherical, (B,K)), Σr·x² (diag, (B,K,D)),
    Σr·xxᵀ (full, (B,K,D,D)) or unused (tied, which takes the fit-constant
    ``total_xx`` = XᵀX instead).
    """
    d = sum_x.shape[-1]
    active = nk > min_weight
    nk_safe = nk.clamp_min(min_weight)
    means_new = (sum_x / nk_safe.unsqueeze(-1)).to(x_dtype)
    means_new = torch.where(active.unsqueeze(-1), means_new, means)
    if covariance_type == "spherical":
        msq = means_new.square().sum(dim=-1)
        covs_new = (sum_q - nk * msq).clamp_min(0.0) / (nk_safe * float(d))
        covs_new = covs_new.clamp_min(reg_covar)
        covs_new = torch.where(active, covs_new, covs)
    elif covariance_type == "diag":
        second = sum_q / nk_safe.unsqueeze(-1)
        covs_new = (second - means_new.to(torch.float32).square()).clamp_min(reg_covar)
        covs_new = torch.where(active.unsqueeze(-1), covs_new.to(x_dtype), covs)
    else:
        eye = torch.eye(d, dtype=torch.float32)
        mf = means_new.to(torch.float32)
        outer = mf.unsqueeze(-1) * mf.unsqueeze(-2)
        if covariance_type == "full":
            scatter = sum_q - nk[..., None, None] * outer
            cn = symmetrize(scatter / nk_safe[..., None, None]) + reg_covar * eye
            covs_new = torch.where(active[..., None, None], cn.to(x_dtype), covs)
        else:
            scatter = total_xx - (nk[..., None, None] * outer).sum(dim=1)
            covs_new = (symmetrize(scatter / float(n)) + reg_covar * eye).to(x_dtype)
    weights_new = (nk / float(n)).clamp_min(min_weight)
    weights_new = weights_new / weights_new.sum(dim=-1, keepdim=True)
    if covariance_type != "spherical":
        weights_new = weights_new.to(x_dtype)
    return means_new, covs_new, weights_new


@torch.no_grad()
def fit(x: torch.Tensor, n_components: int, covariance_type: str, *, max_iters: int = 100,
        tol: float = 1e-4, init_means=None, init_covs=None, init_weights=None,
        reg_covar: float = 1e-6, min_weight: float = 1e-8,
        chunk_size_N: int = DEFAULT_CHUNK_N, chunk_size_K: int = DEFAULT_CHUNK_K,
        compute_labels: bool = True, record_all_lower_bounds: bool = True,
        approx_top_k: Optional[int] = None, bf16_means: bool = False,
        ) -> Tuple[Optional[torch.Tensor], torch.Tensor, torch.Tensor, torch.Tensor, Dict]:
    """Soft EM with explicit initial parameters, for one covariance type.

    Follows batch_gmm_Spherical_torch_native (torch_fallback.py:1897-2397),
    batch_gmm_Diagonal_torch_native (:2401-2728) and
    _batch_gmm_matrix_torch_native (:2732-3244) on their CPU branch.
    Returns (labels, means, covariances, weights, info) like the reference.

    ``bf16_means`` models bf16 input on fp32 arithmetic (pass x upcast to fp32):
    the means are rounded to bf16 on entry and after every M-step, as the
    reference's ``.to(x.dtype)`` keeps a bf16 input's means (:1451, :2295);
    covariances and weights stay fp32, and the variance is formed from the
    unrounded mean (the reference forms it from the rounded means in bf16
    arithmetic, :2297-2299).
    """
    if x.ndim != 3:
        raise ValueError("x must have shape (B, N, D)")
    if covariance_type not in ("spherical", "diag", "tied", "full"):
        raise ValueError("covariance_type must be 'spherical', 'diag', 'tied' or 'full'")
    bsz, n, d = x.shape
    if n_components <= 0:
        raise ValueError("n_components must be positive")
    if n == 0:
        raise ValueError("x must contain at least one sample")
    if max_iters <= 0:
        raise ValueError("max_iters must be positive")
    if init_means is None:
        raise ValueError("the oracle runs with explicit initial parameters only")
    k = n_components
    spherical = covariance_type == "spherical"
    x_sq_all = (x.to(torch.float32) ** 2).sum(dim=-1) if spherical else None
    means, covs, weights = init_user_parameters(x, covariance_type, init_means, init_covs,
                                                init_weights, reg_covar, x_sq=x_sq_all)
    if bf16_means:
        means = _bf16_values(means)
    chunk_n = _spherical_chunk_n(n, d, k, chunk_size_N) if spherical else chunk_size_N
    # _resolve_approx_top_k (torch_fallback.py:598-606): top_k >= K is exact EM.
    if approx_top_k is not None and int(approx_top_k) <= 0:
        raise ValueError("approx_top_k must be positive or None")
    top_k = int(approx_top_k) if approx_top_k is not None and int(approx_top_k) < k else None

    total_xx = None
    if covariance_type == "tied":                                   # :2856-2862
        total_xx = torch.zeros((bsz, d, d), dtype=torch.float32)
        for n0 in range(0, n, chunk_n):
            xf = x[:, n0:min(n0 + chunk_n, n), :].to(torch.float32)
            total_xx += torch.bmm(xf.transpose(1, 2), xf)
    history = []
    prev_lb = None
    iteration = 0
    for iteration in range(max_iters):
        last = iteration + 1 == max_iters
        collect = bool(tol > 0.0 or last or record_all_lower_bounds or spherical)
        # Iteration prelude (:2061-2066, :2485-2490, :2865-2868).
        if covariance_type in ("spherical", "diag"):
            covs = covs.clamp_min(reg_covar)
        weights = weights.clamp_min(min_weight)
        weights = weights / weights.sum(dim=-1, keepdim=True)
        mdl = _Model(covariance_type, means, covs, weights)

        if top_k is not None:
            nk, sum_x, sum_q, total_ll = _accumulate_topk(x, x_sq_all, mdl, covariance_type, chunk_n,
                                                          chunk_size_K, top_k)
        else:
            nk, sum_x, sum_q, total_ll = _accumulate(x, x_sq_all, mdl, covariance_type, chunk_n,
                                                     chunk_size_K, collect)

        means_new, covs_new, weights_new = finalize(
            covariance_type, nk, sum_x, sum_q, means, covs, n=n, reg_covar=reg_covar,
            min_weight=min_weight, total_xx=total_xx, x_dtype=x.dtype)

        lb = (total_ll / float(bsz * n)) if collect else torch.zeros((), dtype=torch.float32)
        history.append(float(lb))
        means, covs, weights = (_bf16_values(means_new) if bf16_means else means_new), covs_new, weights_new

        # Convergence (:2322-2330 spherical; :2695-2698 others).
        if spherical:
            if not last and prev_lb is not None and abs(history[-1] - prev_lb) < tol:
                break
            if not last:
                prev_lb = history[-1]
        else:
            if tol > 0.0 and prev_lb is not None and abs(history[-1] - prev_lb) < tol:
                break
            if tol > 0.0:
                prev_lb = history[-1]

    labels = None
    if compute_labels:
        labels = assign(x, means, covs, weights, covariance_type,
                        chunk_size_N=chunk_n if covariance_type == "tied" else chunk_size_N,
                        chunk_size_K=chunk_size_K)
    info = {"n_iter": iteration + 1, "lower_bound": history[-1],
            "lower_bound_history": history, "init_source": "user",
            "approximate_em_enabled": top_k is not None, "approx_top_k": top_k}
    return labels, means, covs, weights, info


def fit_one_iteration_stats(x, covariance_type, means, covs, weights, reg_covar=1e-6,
                            min_weight=1e-8, bf16_means=False):
    """Convenience: one EM iteration from explicit parameters; returns the new
    parameters and that iteration's mean log-likelihood."""
    _, m, c, w, info = fit(x, means.shape[1], covariance_type, max_iters=1, tol=0.0,
                           init_means=means, init_covs=covs, init_weights=weights,
                           reg_covar=reg_covar, min_weight=min_weight, compute_labels=False,
                           bf16_means=bf16_means)
    return m, c, w, info["lower_bound"]


def _bf16_values(t: torch.Tensor) -> torch.Tensor:
    """fp32 tensor of the bf16 round-to-nearest-even values of t."""
    return t.to(torch.bfloat16).to(torch.float32)


# ---------------------------------------------------------------------------
# k-means initialisation (init_params="kmeans", torch_fallback.py:1390-1631)
# ---------------------------------------------------------------------------

def kmeans_pp(sample, k, first_idx, draws):
    """Greedy k-means++ on a row sample (torch_fallback.py:1390-1451, its
    vectorised branch) with the random numbers given instead of drawn:
    ``first_idx`` (B,) replaces torch.randint and ``draws[:, c-1, :]`` (B, T)
    the torch.rand of step c.  Returns the centres (B, K, D) fp32."""
    bsz, s, d = sample.shape
    sf = sample.to(torch.float32)
    bidx = torch.arange(bsz)
    centers = torch.empty((bsz, k, d), dtype=torch.float32)
    centers[:, 0, :] = sf[bidx, first_idx]
    closest = (sf - centers[:, 0:1, :]).square().sum(dim=-1)
    for c in range(1, k):
        dist_sum = closest.sum(dim=1)
        cumulative = closest.cumsum(dim=1)
        targets = draws[:, c - 1, :].to(torch.float32) * dist_sum.unsqueeze(1)
        cand = torch.searchsorted(cumulative, targets).clamp_max(s - 1)
        cand = torch.where(dist_sum.unsqueeze(1) > 0, cand, torch.zeros_like(cand))
        cands = sf[bidx[:, None], cand]                                   # (B, T, D)
        new_dist = (sf.unsqueeze(2) - cands.unsqueeze(1)).square().sum(dim=-1)
        trial = torch.minimum(closest.unsqueeze(-1), new_dist)            # (B, S, T)
        best = trial.sum(dim=1).argmin(dim=1)
        centers[:, c, :] = sf[bidx, cand[bidx, best]]
        closest = trial[bidx, :, best]
    return centers


def lloyd(x, centers, max_iters, tol, chunk_n=DEFAULT_CHUNK_N):
    """Lloyd k-means from ``centers``: assign every row to its nearest centre
    (first on ties), move each centre to the mean of its rows (an empty cluster
    keeps its centre), stop after max_iters or when tol > 0 and no centre moved
    by tol or more.  This restates flash-kmeans' batch_kmeans_Euclid
    (flash-kmeans>=0.2, not in the reference tree; called at
    torch_fallback.py:1588-1622) from the textbook algorithm: the stopping rule
    is an assumption.  Returns (labels of the last assignment, centres, iterations)."""
    bsz, n, d = x.shape
    k = centers.shape[1]
    xf = x.to(torch.float32)
    means = centers.to(torch.float32).clone()
    labels = None
    it = 0
    for it in range(1, max(1, int(max_iters)) + 1):
        labels = torch.empty((bsz, n), dtype=torch.long)
        for n0 in range(0, n, chunk_n):
            xc = xf[:, n0:n0 + chunk_n]
            dist = (xc.unsqueeze(2) - means.unsqueeze(1)).square().sum(dim=-1)
            labels[:, n0:n0 + chunk_n] = dist.argmin(dim=-1)
        counts = torch.zeros((bsz, k), dtype=torch.float32)
        sums = torch.zeros((bsz, k, d), dtype=torch.float32)
        for b in range(bsz):
            counts[b].index_add_(0, labels[b], torch.ones(n))
            sums[b].index_add_(0, labels[b], xf[b])
        new = torch.where((counts > 0).unsqueeze(-1), sums / counts.clamp_min(1.0).unsqueeze(-1), means)
        shift = float((new - means).norm(dim=-1).max())
        means = new
        if tol > 0.0 and shift < tol:
            break
    return labels, means, it


def hard_label_init_stats(x, covariance_type, means, labels, reg_covar):
    """Initial (weights, covariances) from hard labels and centres, by
    _hard_label_init_stats (torch_fallback.py:1453-1477), _diag (:1480-1504),
    _tied (:1544-1566) and _full (:1507-1541): direct differences to the
    assigned centre, weights ∝ max(count, 1), the global (co)variance for empty
    clusters."""
    bsz, n, d = x.shape
    k = means.shape[1]
    xf = x.to(torch.float32)
    mf = means.to(torch.float32)
    counts = torch.zeros((bsz, k), dtype=torch.float32)
    for b in range(bsz):
        counts[b].index_add_(0, labels[b], torch.ones(n))
    weights = counts.clamp_min(1.0)
    weights = weights / weights.sum(dim=-1, keepdim=True)
    diffs = xf - torch.gather(mf, 1, labels.unsqueeze(-1).expand(-1, -1, d))
    eye = torch.eye(d, dtype=torch.float32)
    if covariance_type == "spherical":
        sq = torch.zeros((bsz, k), dtype=torch.float32)
        for b in range(bsz):
            sq[b].index_add_(0, labels[b], diffs[b].square().sum(dim=-1))
        var = sq / counts.clamp_min(1.0) / float(d)
        var = torch.where(counts > 0, var, global_spherical_variance(xf, k, reg_covar))
        return weights, var.clamp_min(reg_covar)
    if covariance_type == "diag":
        sq = torch.zeros((bsz, k, d), dtype=torch.float32)
        for b in range(bsz):
            sq[b].index_add_(0, labels[b], diffs[b].square())
        var = sq / counts.clamp_min(1.0).unsqueeze(-1)
        var = torch.where((counts > 0).unsqueeze(-1), var, global_diag_variance(xf, k, reg_covar))
        return weights, var.clamp_min(reg_covar)
    if covariance_type == "tied":
        cov = torch.bmm(diffs.transpose(1, 2), diffs) / float(n) + reg_covar * eye
        return weights, symmetrize(cov)
    cov = torch.zeros((bsz, k, d, d), dtype=torch.float32)
    for b in range(bsz):
        cov[b].index_add_(0, labels[b], diffs[b].unsqueeze(-1) * diffs[b].unsqueeze(-2))
    cov = cov / counts.clamp_min(1.0)[..., None, None] + reg_covar * eye
    glob = global_tied_covariance(xf, reg_covar).unsqueeze(1).expand(-1, k, -1, -1)
    cov = torch.where((counts > 0)[..., None, None], cov, glob)
    return weights, symmetrize(cov)


def kmeans_initialize_from(x, covariance_type, centers, *, max_iters=10, tol=1e-4, reg_covar=1e-6):
    """(means, covariances, weights) of init_params="kmeans" from given seed
    centres: Lloyd refinement, then the hard-label statistics
    (torch_fallback.py:1701-1716 and the diag/tied/full counterparts)."""
    labels, means, _ = lloyd(x, centers, max_iters, tol)
    weights, covs = hard_label_init_stats(x, covariance_type, means, labels, reg_covar)
    return means, covs, weights
