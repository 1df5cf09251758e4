"""k-means initialisation of the EM fit (``init_params="kmeans"``) on the HIP engine.

The reference's ``_kmeans_initialize`` (gmmxx/torch_fallback.py:1569-1631) seeds
centres with greedy k-means++ on a row sample (:1390-1451), refines them with
Lloyd iterations from the optional flash-kmeans package (``flash-kmeans>=0.2``,
pyproject.toml:45; ``batch_kmeans_Euclid``), and turns the final hard labels
into initial weights and covariances (``_hard_label_init_stats*``, :1453-1543).
Here:

* k-means++ runs in ``gmmxx_hip_kmeans_pp`` with the reference's constants
  (a sample of min(N, 65536, max(4096, 64·K)) rows, 2 + ⌊ln K⌋ candidates per
  step, K <= 256), the random numbers drawn on the device;
* one Lloyd iteration is one hard-assignment E-step -- the top-1 statistics of
  ``gmmxx_hip_estep_stats_topk`` under unit covariances and uniform weights,
  which puts every row's whole mass on its nearest centre (ties: lower index)
  -- followed by centre = mean of its rows (an empty cluster keeps its
  centre).  It stops after ``max_iters`` iterations, or earlier when ``tol`` > 0
  and no centre moved by ``tol`` or more (Euclidean);
* the hard-label statistics are formed from the last assignment's counts and
  sums with the final centres, by the reference's formulas.

flash-kmeans is not part of the reference tree: its Lloyd loop is the textbook
algorithm restated, and its stopping rule is this module's assumption (the CPU
oracle restates the same).  Without a centre set from k-means++ (K > 256, or K
larger than the sample) Lloyd starts from random rows, as flash-kmeans does
without ``init_centroids``.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _hip

KMEANS_PLUS_PLUS_MAX_COMPONENTS = 256      # gmmxx/torch_fallback.py:65-68
KMEANS_PLUS_PLUS_MAX_SAMPLES = 65536
KMEANS_PLUS_PLUS_MIN_SAMPLES = 4096
KMEANS_PLUS_PLUS_SAMPLES_PER_COMPONENT = 64


def kmeans_pp_sample_size(n: int, k: int) -> int:
    return min(n, KMEANS_PLUS_PLUS_MAX_SAMPLES,
               max(KMEANS_PLUS_PLUS_MIN_SAMPLES, KMEANS_PLUS_PLUS_SAMPLES_PER_COMPONENT * k))


def kmeans_pp_trials(k: int) -> int:
    return 2 + int(math.log(float(k)))


@torch.no_grad()
def kmeans_plus_plus(x: torch.Tensor, k: int, generator: Optional[torch.Generator] = None
                     ) -> Optional[torch.Tensor]:
    """Greedy k-means++ centres (B, K, D) fp32 on x's device, or None when the
    reference skips it (K > 256 or K above the sample size)."""
    bsz, n, _ = x.shape
    s = kmeans_pp_sample_size(n, k)
    if k <= 0 or k > s or k > KMEANS_PLUS_PLUS_MAX_COMPONENTS:
        return None
    dev = x.device
    if s == n:
        sample = x
    else:
        idx = torch.randperm(n, device=dev, generator=generator)[:s]
        sample = x.index_select(1, idx)
    first = torch.randint(0, s, (bsz,), device=dev, generator=generator)
    draws = torch.rand((bsz, k - 1, kmeans_pp_trials(k)), device=dev, generator=generator)
    return _hip.kmeans_pp(sample.to(torch.float32), k, first, draws)


def _unit_parameters(covariance_type: str, bsz: int, k: int, d: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Unit covariances and uniform weights: the logits are then -½‖x - μ‖² plus a
    constant, so the top-1 component of a row is its nearest centre."""
    if covariance_type == "spherical":
        covs = torch.ones((bsz, k), device=device)
    elif covariance_type == "diag":
        covs = torch.ones((bsz, k, d), device=device)
    elif covariance_type == "tied":
        covs = torch.eye(d, device=device).expand(bsz, d, d).contiguous()
    else:
        covs = torch.eye(d, device=device).expand(bsz, k, d, d).contiguous()
    return covs, torch.full((bsz, k), 1.0 / float(k), device=device)


class _HardStats:
    """Hard-assignment statistics (nk, Σx, Σq) of x against a centre set, in the
    statistics layout of ``covariance_type`` (row chunks as the top-k E-step)."""

    def __init__(self, x: torch.Tensor, covariance_type: str, k: int):
        from . import em
        self.x, self.cov, self.k = x, covariance_type, k
        bsz, _, d = x.shape
        self.covs, self.weights = _unit_parameters(covariance_type, bsz, k, d, x.device)
        self.topk = em._TopkStep(x, covariance_type, k, 1) if k > 1 else None

    def __call__(self, means: torch.Tensor):
        if self.topk is None:   # one cluster: every row belongs to it
            nk, sx, sq, _ = _hip.estep_stats(self.cov, self.x, means, self.covs, self.weights)
            return nk, sx, sq
        nk, sx, sq, _ = self.topk.stats(means, self.covs, self.weights, 1e-6, 1e-8)
        return nk, sx, sq

    def gram(self) -> torch.Tensor:
        if self.topk is not None:
            return self.topk.gram()
        bsz, n, d = self.x.shape
        return _hip.gram(self.x, _hip.Workspace(_hip.problem("tied", torch.float32, bsz, n, d, 1), self.x.device))


@torch.no_grad()
def lloyd(x: torch.Tensor, covariance_type: str, centers: torch.Tensor, max_iters: int, tol: float,
          stats: Optional[_HardStats] = None):
    """Lloyd iterations from ``centers``; returns (centres, nk, Σx, Σq, iterations),
    the statistics being those of the last assignment."""
    k = int(centers.shape[1])
    stats = stats or _HardStats(x, covariance_type, k)
    means = centers.to(torch.float32).contiguous()
    nk = sx = sq = None
    n_iter = 0
    for _ in range(max(1, int(max_iters))):
        nk, sx, sq = stats(means)
        new = torch.where((nk > 0).unsqueeze(-1), sx / nk.clamp_min(1.0).unsqueeze(-1), means).contiguous()
        shift = (new - means).norm(dim=-1).amax()
        means = new
        n_iter += 1
        if tol > 0.0 and float(shift) < tol:
            break
    return means, nk, sx, sq, n_iter


def _sym(m: torch.Tensor) -> torch.Tensor:
    return 0.5 * (m + m.transpose(-1, -2))


@torch.no_grad()
def hard_label_init_stats(x: torch.Tensor, covariance_type: str, means: torch.Tensor, nk: torch.Tensor,
                          sum_x: torch.Tensor, sum_q: Optional[torch.Tensor], reg_covar: float,
                          gram: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(weights, covariances) from hard-label statistics, by the formulas of
    _hard_label_init_stats / _diag / _tied / _full (gmmxx/torch_fallback.py:1453-1543):
    weights ∝ max(count, 1); per-cluster scatter about the given centres, the
    global (co)variance for empty clusters, reg_covar as floor (spherical,
    diag) or on the diagonal (tied, full)."""
    from . import em
    bsz, n, d = x.shape
    k = int(means.shape[1])
    counts = nk
    safe = counts.clamp_min(1.0)
    weights = (safe / safe.sum(dim=-1, keepdim=True)).contiguous()
    mu = means.to(torch.float32)
    if covariance_type == "spherical":
        sq_sums = sum_q - 2.0 * (mu * sum_x).sum(dim=-1) + counts * mu.square().sum(dim=-1)
        var = sq_sums / safe / float(d)
        var = torch.where(counts > 0, var, em.global_spherical_variance(x, k, reg_covar))
        return weights, var.clamp_min(reg_covar).contiguous()
    if covariance_type == "diag":
        sq_sums = sum_q - 2.0 * mu * sum_x + counts.unsqueeze(-1) * mu.square()
        var = sq_sums / safe.unsqueeze(-1)
        var = torch.where((counts > 0).unsqueeze(-1), var, em.global_diag_variance(x, k, reg_covar))
        return weights, var.clamp_min(reg_covar).contiguous()
    eye = torch.eye(d, device=x.device, dtype=torch.float32)
    outer = mu.unsqueeze(-1) * sum_x.unsqueeze(-2)            # μ Σxᵀ
    scatter_k = -outer - outer.transpose(-1, -2) + counts[..., None, None] * (mu.unsqueeze(-1) * mu.unsqueeze(-2))
    if covariance_type == "tied":
        cov = (gram + scatter_k.sum(dim=1)) / float(n) + reg_covar * eye
        return weights, _sym(cov).contiguous()
    cov = (sum_q + scatter_k) / safe[..., None, None] + reg_covar * eye
    glob = em.global_tied_covariance(x, reg_covar).unsqueeze(1).expand(-1, k, -1, -1)
    cov = torch.where((counts > 0)[..., None, None], cov, glob)
    return weights, _sym(cov).contiguous()


@torch.no_grad()
def kmeans_initialize(x: torch.Tensor, covariance_type: str, k: int, *, max_iters: int = 10,
                      tol: float = 1e-4, reg_covar: float = 1e-6,
                      generator: Optional[torch.Generator] = None):
    """(means, covariances, weights) from k-means++ seeding, Lloyd refinement and
    the hard-label statistics; x is an engine tensor (B, N, D) on the GPU."""
    bsz, n, d = x.shape
    centers = kmeans_plus_plus(x, k, generator)
    if centers is None:
        idx = torch.randint(0, n, (bsz, k), device=x.device, generator=generator)
        centers = torch.gather(x, 1, idx[..., None].expand(-1, -1, d)).to(torch.float32)
    stats = _HardStats(x, covariance_type, k)
    means, nk, sx, sq, _ = lloyd(x, covariance_type, centers, max_iters, tol, stats)
    gram = stats.gram() if covariance_type == "tied" else None
    weights, covs = hard_label_init_stats(x, covariance_type, means, nk, sx, sq, reg_covar, gram)
    return means, covs, weights
