"""gmmxx_amd: the GMM EM hot path of OpsiClear/GMMXX on MI355X (gfx950).

``GMMXX(backend="hip")`` is the reference estimator surface with every compute
call on hand-written HIP kernels in ``libgmmxx_hip.so`` (C ABI in
``include/gmmxx_hip.h``).  The function-level names of the reference package
(gmmxx/__init__.py:1-34: ``batch_gmm_*``, the ``*_torch_native_chunked``
inference functions and the ``large_n`` streaming functions) are exported with
the same signatures and run on the same kernels; ``batch_gmm_*_hip``,
``fit_large_n`` and the ``*_large_n`` inference functions are this package's
own spellings of them.  ``hip_ops`` mirrors the reference's experimental
``cuda_ops`` module.
"""

from ._hip import HipBackendUnavailable, HipRuntimeError, HipRuntimeFallback, has_hip, require_hip
from ._dispatch import UnsupportedShape, resolve_backend, resolve_backend_with_env
from .em import (batch_gmm_Diagonal, batch_gmm_Diagonal_hip, batch_gmm_Diagonal_torch_native, batch_gmm_diag,
                 batch_gmm_diagonal, batch_gmm_Full, batch_gmm_Full_hip, batch_gmm_Full_torch_native,
                 batch_gmm_full, batch_gmm_Spherical, batch_gmm_Spherical_hip, batch_gmm_Spherical_torch_native,
                 batch_gmm_spherical, batch_gmm_Tied, batch_gmm_Tied_hip, batch_gmm_Tied_torch_native,
                 batch_gmm_tied, diagonal_assign_torch_native_chunked,
                 diagonal_predict_proba_torch_native_chunked, diagonal_score_samples_torch_native_chunked,
                 full_assign_torch_native_chunked, full_predict_proba_torch_native_chunked,
                 full_score_samples_torch_native_chunked, spherical_assign_torch_native_chunked,
                 spherical_predict_proba_torch_native_chunked, spherical_score_samples_torch_native_chunked,
                 tied_assign_torch_native_chunked, tied_predict_proba_torch_native_chunked,
                 tied_score_samples_torch_native_chunked)
from .interface import GMMXX
from .large_n import (batch_gmm_largeN_cpu, fit_large_n, large_n_predict_cpu, large_n_predict_proba_cpu,
                      large_n_score_samples_cpu, predict_large_n, predict_proba_large_n, score_samples_large_n)
from . import hip_ops

__all__ = [
    "GMMXX", "HipBackendUnavailable", "HipRuntimeError", "HipRuntimeFallback", "UnsupportedShape", "has_hip",
    "require_hip", "resolve_backend", "resolve_backend_with_env",
    "batch_gmm_Spherical", "batch_gmm_Spherical_torch_native", "batch_gmm_Diagonal",
    "batch_gmm_Diagonal_torch_native", "batch_gmm_Full", "batch_gmm_Full_torch_native", "batch_gmm_Tied",
    "batch_gmm_Tied_torch_native", "batch_gmm_spherical", "batch_gmm_diagonal", "batch_gmm_diag",
    "batch_gmm_full", "batch_gmm_tied",
    "spherical_assign_torch_native_chunked", "spherical_predict_proba_torch_native_chunked",
    "spherical_score_samples_torch_native_chunked",
    "diagonal_assign_torch_native_chunked", "diagonal_predict_proba_torch_native_chunked",
    "diagonal_score_samples_torch_native_chunked", "full_assign_torch_native_chunked",
    "full_predict_proba_torch_native_chunked", "full_score_samples_torch_native_chunked",
    "tied_assign_torch_native_chunked", "tied_predict_proba_torch_native_chunked",
    "tied_score_samples_torch_native_chunked",
    "batch_gmm_largeN_cpu", "large_n_predict_cpu", "large_n_predict_proba_cpu", "large_n_score_samples_cpu",
    "batch_gmm_Spherical_hip", "batch_gmm_Diagonal_hip", "batch_gmm_Tied_hip", "batch_gmm_Full_hip",
    "fit_large_n", "predict_large_n", "predict_proba_large_n", "score_samples_large_n", "hip_ops",
]

__version__ = "0.1.0"
