"""Experimental public surface of the low-level HIP callables under the names
and argument lists of the reference's CUDA op module (gmmxx/cuda_ops.py:11-87,
gmmxx/_cuda.py).

Only the ``GMMXX`` estimator is a stable API, as in the reference.  Every name
exported here takes the reference op's arguments and returns what it returns;
the work runs in the HIP library (``gmmxx_hip_score``,
``gmmxx_hip_predict_proba_score``, ``gmmxx_hip_em_step``):

* ``<cov>_assign(x, means, var | L, log_w, out=None)`` -- first-max labels,
  int32 (B, N) (_cuda.py:328-352, :897-915, :1126-1146, :1274-1284);
* ``<cov>_logsumexp(x, means, var | L, log_w, out=None)`` -- per-sample
  log-likelihood, fp32 (B, N) (_cuda.py:355-381, :918-936, :1149-1170, :1287-1296);
* ``<cov>_resp(x, means, var | L, log_w, log_norm, out=None)`` -- responsibilities
  exp(logit - log_norm), fp32 (B, N, K), for the caller's ``log_norm`` (the
  ``<cov>_logsumexp`` output gives the normalised ones) (_cuda.py:384-412,
  :939-959, :1173-1201, :1299-1314);
* ``fused_spherical(x, means, var, log_w, reg_covar)`` and
  ``soft_update_spherical(x, means, var, log_w, reg_covar, ...)`` -- one soft-EM
  iteration: (new means, new variances, new weights, per-sample log-likelihood
  under the input parameters, int32 labels) (_cuda.py:1056-1088, :415-682).

Spherical and diagonal ops take the variances (B, K) / (B, K, D); tied and full
ops take the lower Cholesky factor L of the covariance ((B, D, D) / (B, K, D, D)),
as the reference's do; the library works from the covariance L·Lᵀ and factorises
it again.  Weights enter as log-weights; the library takes weights, so
``log_w`` is exponentiated on the way in (its logarithm is then within one
rounding of ``log_w``).  The EM-iteration ops apply the iteration prelude of the
reference's fit loops (variances clamped to ``reg_covar``, weights floored at
1e-8 and renormalised, torch_fallback.py:2061-2066), which leaves parameters
coming out of a previous iteration unchanged.

Not provided (``AttributeError`` names the replacement): the hard-assignment
accumulators ``blocked_update_*`` / ``full_blocked_update`` and the
count-based finalizers ``finalize_spherical``, ``finalize_diag``,
``tied_finalize``, ``full_finalize`` (the reference's hard-EM CUDA path; this
engine runs soft EM: ``gmmxx_amd._hip.estep_stats`` and ``finalize_stats``),
the torch-only helpers ``tied_project`` / ``tied_log_det`` (the library forms
the Cholesky factor, precision and log-determinant inside each call), and
``approx_topk_update_spherical`` (``gmmxx_amd._hip.estep_stats_topk``).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _hip

canary_add_offset = _hip.canary_add_offset


def _weights(log_w: torch.Tensor) -> torch.Tensor:
    return torch.exp(log_w.to(torch.float32))


def _cov_from_L(L: torch.Tensor) -> torch.Tensor:
    L = L.to(torch.float32)
    return (L @ L.transpose(-1, -2)).contiguous()


def _into(out: Optional[torch.Tensor], value: torch.Tensor) -> torch.Tensor:
    if out is None:
        return value
    out.copy_(value)
    return out


def _assign(cov, x, means, covs, log_w, out=None):
    lab = _hip.score(cov, x, means, covs, _weights(log_w), want_scores=False, want_labels=True)[1]
    return _into(out, lab.to(torch.int32))


def _logsumexp(cov, x, means, covs, log_w, out=None):
    return _into(out, _hip.score(cov, x, means, covs, _weights(log_w), want_scores=True, want_labels=False)[0])


def _resp(cov, x, means, covs, log_w, log_norm, out=None):
    proba, lse = _hip.predict_proba_score(cov, x, means, covs, _weights(log_w))
    # exp(l - log_norm) = r · exp(lse - log_norm): exactly r when log_norm is this lse
    shift = lse - log_norm.to(device=lse.device, dtype=torch.float32)
    r = proba if bool((shift == 0).all()) else proba * torch.exp(shift).unsqueeze(-1)
    return _into(out, r)


def spherical_assign(x, means, var, log_w, out=None):
    return _assign("spherical", x, means, var, log_w, out)


def spherical_logsumexp(x, means, var, log_w, out=None, x_sq=None, c_sq=None):
    """``x_sq`` / ``c_sq`` (the reference's cached squared norms) are accepted
    and not needed: the library forms ‖x‖² while it loads each row."""
    return _logsumexp("spherical", x, means, var, log_w, out)


def spherical_resp(x, means, var, log_w, log_norm, out=None, x_sq=None, c_sq=None):
    return _resp("spherical", x, means, var, log_w, log_norm, out)


def diag_assign(x, means, var, log_w, out=None):
    return _assign("diag", x, means, var, log_w, out)


def diag_logsumexp(x, means, var, log_w, out=None):
    return _logsumexp("diag", x, means, var, log_w, out)


def diag_resp(x, means, var, log_w, log_norm, out=None):
    return _resp("diag", x, means, var, log_w, log_norm, out)


def tied_assign(x, means, L, log_w):
    return _assign("tied", x, means, _cov_from_L(L), log_w)


def tied_logsumexp(x, means, L, log_w):
    return _logsumexp("tied", x, means, _cov_from_L(L), log_w)


def tied_resp(x, means, L, log_w, log_norm):
    return _resp("tied", x, means, _cov_from_L(L), log_w, log_norm)


def full_assign(x, means, L, log_w):
    return _assign("full", x, means, _cov_from_L(L), log_w)


def full_logsumexp(x, means, L, log_w):
    return _logsumexp("full", x, means, _cov_from_L(L), log_w)


def full_resp(x, means, L, log_w, log_norm):
    return _resp("full", x, means, _cov_from_L(L), log_w, log_norm)


def fused_spherical(x, means, var, log_w, reg_covar):
    """One soft-EM iteration: (means, var, weights) after it, and the E-step's
    per-sample log-likelihood (B, N) and int32 labels under the input
    parameters (_cuda.py:1056-1088).  Means come back in the input means' dtype."""
    w = _weights(log_w)
    lse, lab = _hip.score("spherical", x, means, var, w)
    m = means.to(torch.float32).clone()
    v = var.to(torch.float32).clone()
    w = w.clone()
    lb = torch.zeros(1, dtype=torch.float32, device=x.device)
    _hip.em_step("spherical", x, m, v, w, lb, reg_covar=float(reg_covar))
    return m.to(means.dtype), v, w, lse, lab.to(torch.int32)


def soft_update_spherical(x, means, var, log_w, reg_covar, x_f_cached=None, x_sq_cached=None,
                          x_aug_cached=None, x_estep_aug_cached=None, x_estep_aug_bf16_cached=None,
                          x_aug_bf16_cached=None, persistent_partial_buf=None, compute_ids=True,
                          compute_lse=True):
    """(means, var, weights, lse_per_sample or None, labels or None) of one
    soft-EM iteration (_cuda.py:415-682).  The cached-operand arguments are the
    reference's host-side hoisting and are accepted and not needed here."""
    m, v, w, lse, lab = fused_spherical(x, means, var, log_w, reg_covar)
    return m, v, w, (lse if compute_lse else None), (lab if compute_ids else None)


# Lifecycle / introspection helpers.
has_hip = _hip.has_hip
require_hip = _hip.require_hip
device_info = _hip.device_info
HipBackendUnavailable = _hip.HipBackendUnavailable
HipRuntimeError = _hip.HipRuntimeError
HipRuntimeFallback = _hip.HipRuntimeFallback

_NOT_PROVIDED = {
    "blocked_update_spherical": "gmmxx_amd._hip.estep_stats (soft statistics)",
    "blocked_update_spherical_sorted": "gmmxx_amd._hip.estep_stats (soft statistics)",
    "blocked_update_diag": "gmmxx_amd._hip.estep_stats (soft statistics)",
    "blocked_update_diag_sorted": "gmmxx_amd._hip.estep_stats (soft statistics)",
    "full_blocked_update": "gmmxx_amd._hip.estep_stats (soft statistics)",
    "finalize_spherical": "gmmxx_amd._hip.finalize_stats",
    "finalize_diag": "gmmxx_amd._hip.finalize_stats",
    "tied_finalize": "gmmxx_amd._hip.finalize_stats",
    "full_finalize": "gmmxx_amd._hip.finalize_stats",
    "tied_project": "none: the library factorises the covariance inside each call",
    "tied_log_det": "none: the library factorises the covariance inside each call",
    "approx_topk_update_spherical": "gmmxx_amd._hip.estep_stats_topk",
}


def __getattr__(name):
    if name in _NOT_PROVIDED:
        raise AttributeError(f"gmmxx_amd.hip_ops.{name} is not provided (the reference's hard-EM / torch-only "
                             f"op); use {_NOT_PROVIDED[name]}")
    raise AttributeError(f"module 'gmmxx_amd.hip_ops' has no attribute {name!r}")


__all__ = [
    "canary_add_offset",
    "spherical_assign", "spherical_logsumexp", "spherical_resp", "soft_update_spherical", "fused_spherical",
    "diag_assign", "diag_logsumexp", "diag_resp",
    "tied_assign", "tied_logsumexp", "tied_resp",
    "full_assign", "full_logsumexp", "full_resp",
    "has_hip", "require_hip", "device_info", "HipBackendUnavailable", "HipRuntimeError", "HipRuntimeFallback",
]
