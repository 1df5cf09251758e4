"""gmmxx_amd: the GMM EM hot path of OpsiClear/GMMXX on MI355X (gfx950).

``GMMXX(backend="hip")`` is the reference estimator surface with every compute
call on hand-written HIP kernels in ``libgmmxx_hip.so`` (C ABI in
``include/gmmxx_hip.h``).  ``batch_gmm_*_hip`` are the function-level
counterparts of the reference's ``batch_gmm_*_torch_native``.
"""

from ._hip import HipBackendUnavailable, HipRuntimeError, has_hip, require_hip
from ._dispatch import UnsupportedShape, resolve_backend, resolve_backend_with_env
from .em import (batch_gmm_Diagonal_hip, batch_gmm_Full_hip, batch_gmm_Spherical_hip,
                 batch_gmm_Tied_hip)
from .interface import GMMXX

__all__ = [
    "GMMXX", "HipBackendUnavailable", "HipRuntimeError", "UnsupportedShape", "has_hip", "require_hip",
    "resolve_backend", "resolve_backend_with_env", "batch_gmm_Spherical_hip", "batch_gmm_Diagonal_hip",
    "batch_gmm_Tied_hip", "batch_gmm_Full_hip",
]
