"""Experimental public surface of the low-level HIP callables, under the names
of the reference's CUDA op module (gmmxx/cuda_ops.py:11-87).

Only the ``GMMXX`` estimator is a stable API.  Each name below binds the
covariance type of a ``gmmxx_amd._hip`` entry point, so the arguments are that
function's (device tensors ``x`` (B, N, D), ``means`` (B, K, D), ``covs``,
``weights``), not the reference CUDA ops' own argument lists:

* ``<cov>_assign``        first-max labels (B, N) int64   (gmmxx_hip_score)
* ``<cov>_logsumexp``     per-sample log-likelihood (B, N) (gmmxx_hip_score)
* ``<cov>_resp``          responsibilities (B, N, K)       (gmmxx_hip_predict_proba)
* ``<cov>_resp_logsumexp``  both from one E-step pass      (gmmxx_hip_predict_proba_score)
* ``soft_update_<cov>``   E-step sufficient statistics (nk, sum_x, sum_q, ll_sum)
                          (gmmxx_hip_estep_stats; the reference's soft/blocked updates)
* ``finalize_<cov>``      M-step from summed statistics, in place (gmmxx_hip_finalize_stats)
* ``fused_<cov>``         one in-place EM iteration (gmmxx_hip_em_step)
* ``approx_topk_update_<cov>``  top-k E-step statistics (gmmxx_hip_estep_stats_topk)

The reference's tied projection and log-determinant ops (``tied_project``,
``tied_log_det``) have no separate entry point here: the library computes the
Cholesky factor, precision and log-determinant inside each call.
"""

from __future__ import annotations

import functools

from . import _hip


def _assign(cov, x, means, covs, weights, **kw):
    return _hip.score(cov, x, means, covs, weights, want_scores=False, want_labels=True, **kw)[1]


def _logsumexp(cov, x, means, covs, weights, **kw):
    return _hip.score(cov, x, means, covs, weights, want_scores=True, want_labels=False, **kw)[0]


def _bind(fn, cov, name):
    f = functools.partial(fn, cov)
    functools.update_wrapper(f, fn)
    f.__name__ = name
    return f


canary_add_offset = _hip.canary_add_offset

_OPS = {
    "assign": _assign,
    "logsumexp": _logsumexp,
    "resp": _hip.predict_proba,
    "resp_logsumexp": _hip.predict_proba_score,
}
_UPDATES = {
    "soft_update": _hip.estep_stats,
    "finalize": _hip.finalize_stats,
    "fused": _hip.em_step,
    "approx_topk_update": _hip.estep_stats_topk,
}
_COVS = {"spherical": "spherical", "diag": "diag", "tied": "tied", "full": "full"}

__all__ = ["canary_add_offset"]
for _pre, _cov in _COVS.items():
    for _op, _fn in _OPS.items():
        _nm = f"{_pre}_{_op}"
        globals()[_nm] = _bind(_fn, _cov, _nm)
        __all__.append(_nm)
    for _op, _fn in _UPDATES.items():
        _nm = f"{_op}_{_pre}"
        globals()[_nm] = _bind(_fn, _cov, _nm)
        __all__.append(_nm)

# Lifecycle / introspection helpers.
has_hip = _hip.has_hip
require_hip = _hip.require_hip
device_info = _hip.device_info
HipBackendUnavailable = _hip.HipBackendUnavailable
HipRuntimeError = _hip.HipRuntimeError
HipRuntimeFallback = _hip.HipRuntimeFallback
__all__ += ["has_hip", "require_hip", "device_info", "HipBackendUnavailable", "HipRuntimeError",
            "HipRuntimeFallback"]
