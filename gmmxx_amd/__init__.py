"""gmmxx_amd: the GMM EM hot path of OpsiClear/GMMXX on MI355X (gfx950).

``GMMXX(backend="hip")`` is the reference estimator surface with every compute
call on hand-written HIP kernels in ``libgmmxx_hip.so`` (C ABI in
``include/gmmxx_hip.h``).  ``batch_gmm_*_hip`` are the function-level
counterparts of the reference's ``batch_gmm_*_torch_native``; ``fit_large_n``
and the ``*_large_n`` inference functions stream host-resident data through HBM
(the reference's ``large_n`` module).
"""

from ._hip import HipBackendUnavailable, HipRuntimeError, has_hip, require_hip
from ._dispatch import UnsupportedShape, resolve_backend, resolve_backend_with_env
from .em import (batch_gmm_Diagonal_hip, batch_gmm_Full_hip, batch_gmm_Spherical_hip,
                 batch_gmm_Tied_hip)
from .interface import GMMXX
from .large_n import fit_large_n, predict_large_n, predict_proba_large_n, score_samples_large_n

__all__ = [
    "GMMXX", "HipBackendUnavailable", "HipRuntimeError", "UnsupportedShape", "has_hip", "require_hip",
    "resolve_backend", "resolve_backend_with_env", "batch_gmm_Spherical_hip", "batch_gmm_Diagonal_hip",
    "batch_gmm_Tied_hip", "batch_gmm_Full_hip", "fit_large_n", "predict_large_n", "predict_proba_large_n",
    "score_samples_large_n",
]
