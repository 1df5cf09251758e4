"""``GMMXX`` estimator with the HIP/gfx950 engine behind it.

The public surface is the reference's ``gmmxx.interface.GMMXX``
(gmmxx/interface.py:128-2558): the same constructor arguments and sklearn
aliases, ``fit`` / ``train`` / ``fit_predict`` / ``predict`` /
``predict_proba`` / ``score_samples`` / ``score`` / ``bic`` / ``aic``,
``get_params`` / ``set_params`` and the fitted attributes (``means_``,
``weights_``, ``covariances_``, ``labels_``, ``lower_bound_``,
``lower_bound_history_``, ``n_iter_``, ``last_backend_used_`` ...).  The
``backend=`` kwarg gains ``"hip"``; ``"auto"`` resolves to it.  Every compute
call goes to ``libgmmxx_hip.so``; there is no CPU or PyTorch fallback (see
``gmmxx_amd._dispatch``).

Input handling follows the reference: ``(N, D)`` or ``(B, N, D)`` floating
point tensors, fitted attributes squeezed when the input was unbatched
(:322-325, :401-424), half-precision inputs computed in fp32 unless ``dtype=``
says otherwise (:426-433): bf16/fp16 input runs the fp32 algorithm.  With
``dtype=torch.bfloat16`` spherical input stays bf16 in HBM and runs the bf16
engine (bf16 means as the reference keeps them, products of exact bf16 values
with fp32 accumulation, responsibilities rounded to bf16 before the M-step
product): more accurate than the reference's bf16 arithmetic, held to the bf16
bar (2e-3 on the log-likelihood), not to the fp32 one.

Attribution: the estimator contract -- the constructor signature and sklearn
aliases, the parameter validation and its messages, the ``set_params``
branches and ``_n_parameters`` / ``bic`` / ``aic`` -- follows the reference's
``gmmxx/interface.py`` (:77-121, :125-230, :1318-1360, :1605-1607,
:2537-2558), GMMXX, MIT License, Copyright (c) 2026 GMMXX contributors; a
drop-in must accept the same calls.  Everything that computes is this
package's own.
"""

from __future__ import annotations

import contextlib
import math
import warnings
import weakref
from typing import Any, Optional

import torch

from . import _dispatch, _hip, em, large_n

_VALID_COVARIANCE_TYPES = {"spherical", "diag", "tied", "full"}
_COVARIANCE_ALIASES = {"diagonal": "diag"}
_SKLEARN_PARAM_ALIASES = {"n_components": "k", "max_iter": "niter", "random_state": "seed", "n_features": "d"}
_PARAM_NAMES = (
    "d", "n_components", "max_iter", "tol", "random_state", "chunk_size_data", "chunk_size_centroids",
    "chunk_size_data_cpu", "verbose", "dtype", "device", "init_params", "reg_covar", "init_kmeans_iters",
    "init_kmeans_tol", "covariance_type", "matmul_precision", "compute_labels_on_fit", "approx_top_k", "backend",
)


def _normalize_covariance_type(covariance_type: str) -> str:
    covariance_type = _COVARIANCE_ALIASES.get(covariance_type, covariance_type)
    if covariance_type not in _VALID_COVARIANCE_TYPES:
        raise ValueError("covariance_type must be 'spherical', 'diag', 'diagonal', 'tied', or 'full'")
    return covariance_type


def _optional_positive_int(value: Optional[int], name: str) -> Optional[int]:
    if value is None:
        return None
    value = int(value)
    if value <= 0:
        raise ValueError(f"{name} must be positive")
    return value


def _positive_int(value: int, name: str) -> int:
    value = int(value)
    if value <= 0:
        raise ValueError(f"{name} must be positive")
    return value


def _resolve_alias(primary, alias, *, primary_name: str, alias_name: str):
    if primary is not None and alias is not None and int(primary) != int(alias):
        raise ValueError(f"Received conflicting {primary_name}={primary} and {alias_name}={alias}")
    return primary if primary is not None else alias


def _check_backend(backend: str) -> None:
    if backend not in _dispatch.VALID_BACKENDS:
        raise ValueError(f"backend must be one of {sorted(_dispatch.VALID_BACKENDS)}, got {backend!r}")


class GMMXX:
    """Gaussian mixture model fitted by soft EM on MI355X (gfx950).

    ``covariance_type`` is ``spherical``, ``diag``/``diagonal``, ``tied`` or
    ``full``.  Supported shapes: D <= 128; any N, K <= 65536, B <= 65535.
    Half-precision input is computed in fp32 unless ``dtype=torch.bfloat16``
    (spherical: the bf16 engine); other explicit half dtypes are computed in
    fp32 with the parameters kept in that dtype, as the reference keeps them.
    ``approx_top_k`` (1 <= k < K) opts into the reference's approximate EM:
    each row's responsibilities cover only its k largest logits; prediction
    stays exact.
    """

    def __init__(
        self,
        d: Optional[int] = None,
        k: Optional[int] = None,
        niter: Optional[int] = None,
        tol: float = 1e-4,
        use_triton: Optional[bool] = None,
        seed: Optional[int] = None,
        chunk_size_data: int = 32768,
        chunk_size_centroids: int = 1024,
        chunk_size_data_cpu: int = 1048576,
        verbose: bool = False,
        dtype: Optional[torch.dtype] = None,
        device: Optional[torch.device] = None,
        init_params: str = "kmeans",
        reg_covar: float = 1e-6,
        init_kmeans_iters: int = 10,
        init_kmeans_tol: float = 1e-4,
        covariance_type: str = "spherical",
        matmul_precision: Optional[str] = None,
        compute_labels_on_fit: bool = True,
        approx_top_k: Optional[int] = None,
        n_components: Optional[int] = None,
        max_iter: Optional[int] = None,
        random_state: Optional[int] = None,
        n_features: Optional[int] = None,
        backend: str = "auto",
    ):
        d = _resolve_alias(d, n_features, primary_name="d", alias_name="n_features")
        k = _resolve_alias(k, n_components, primary_name="k", alias_name="n_components")
        niter = _resolve_alias(niter, max_iter, primary_name="niter", alias_name="max_iter")
        seed = _resolve_alias(seed, random_state, primary_name="seed", alias_name="random_state")
        _check_backend(backend)
        if use_triton is not None:
            # Deprecated knob of the reference (gmmxx/interface.py:180-199); it
            # selects nothing here since the only engine is HIP.
            if backend != "auto":
                raise ValueError("Cannot pass both backend= and use_triton= to GMMXX. "
                                 "Drop use_triton; backend= is the canonical kwarg.")
            warnings.warn("use_triton is deprecated and has no effect with gmmxx_amd; use backend='hip'",
                          DeprecationWarning, stacklevel=2)
        self._legacy_no_triton = use_triton is False
        self.backend = backend
        if k is None:
            raise ValueError("k or n_components is required")
        self.d = _optional_positive_int(d, "d")
        self.k = _positive_int(k, "k")
        self.niter = _positive_int(100 if niter is None else niter, "niter")
        self.tol = float(tol)
        if self.tol < 0.0:
            raise ValueError("tol must be non-negative")
        self.seed = int(0 if seed is None else seed)
        self.chunk_size_data = _positive_int(chunk_size_data, "chunk_size_data")
        self.chunk_size_centroids = _positive_int(chunk_size_centroids, "chunk_size_centroids")
        self.chunk_size_data_cpu = _positive_int(chunk_size_data_cpu, "chunk_size_data_cpu")
        self.verbose = bool(verbose)
        self.dtype = dtype
        self.init_params = init_params
        self.reg_covar = float(reg_covar)
        if self.reg_covar < 0.0:
            raise ValueError("reg_covar must be non-negative")
        self.init_kmeans_iters = _positive_int(init_kmeans_iters, "init_kmeans_iters")
        self.init_kmeans_tol = float(init_kmeans_tol)
        if self.init_kmeans_tol < 0.0:
            raise ValueError("init_kmeans_tol must be non-negative")
        self.covariance_type = _normalize_covariance_type(covariance_type)
        if matmul_precision is not None and matmul_precision not in {"highest", "high", "medium"}:
            raise ValueError("matmul_precision must be None, 'highest', 'high', or 'medium'")
        self.matmul_precision = matmul_precision
        self.compute_labels_on_fit = bool(compute_labels_on_fit)
        self.approx_top_k = _optional_positive_int(approx_top_k, "approx_top_k")
        self._raw_device = device
        self.device = torch.device(device) if device is not None else torch.device(
            "cuda:0" if torch.cuda.is_available() else "cpu")
        self._reset_fit_state()

    # -- state --------------------------------------------------------------

    @property
    def use_triton(self) -> bool:
        """Always False: no Triton path exists in this package."""
        return False

    def _reset_fit_state(self) -> None:
        self.means_b = self.variances_b = self.covariances_b = self.weights_b = None
        self.cluster_ids_b = None
        self.means_ = self.weights_ = self.covariances_ = self.labels_ = None
        self.lower_bound_: Optional[float] = None
        self.lower_bound_history_: Optional[list] = None
        self.n_iter_: Optional[int] = None
        self.init_source_: Optional[str] = None
        self.fit_info_: Optional[dict] = None
        self.hip_estep_enabled_: Optional[bool] = None
        self.triton_estep_enabled_ = self.triton_fused_update_enabled_ = None
        self.triton_approx_topk_enabled_ = self.triton_streaming_update_enabled_ = None
        self.triton_labels_enabled_ = self.approximate_em_enabled_ = None
        self.approx_top_k_ = None
        self.large_n_streaming_enabled_ = self.copy_stream_prefetch_enabled_ = None
        self.cuda_estep_enabled_ = self.cuda_fused_update_enabled_ = self.cuda_approx_topk_enabled_ = None
        self.last_fallback_reason_: Optional[str] = None
        self.last_backend_used_: Optional[str] = None
        self._batch_size: Optional[int] = None
        self._scores_cache = None

    def _squeeze_if_unbatched(self, value: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        if value is None:
            return None
        return value.squeeze(0) if self._batch_size is None else value

    @contextlib.contextmanager
    def _matmul_precision_scope(self):
        """Applies ``matmul_precision`` for one call and restores it
        (gmmxx/interface.py:285-315).  The engine's own products are not
        affected; torch-side helpers (initial covariances) are."""
        prev = None
        if self.matmul_precision is not None:
            prev = torch.get_float32_matmul_precision()
            torch.set_float32_matmul_precision(self.matmul_precision)
        try:
            yield
        finally:
            if prev is not None:
                torch.set_float32_matmul_precision(prev)

    # -- input handling (gmmxx/interface.py:401-450) ------------------------

    def _normalize_input(self, data: torch.Tensor) -> tuple[torch.Tensor, Optional[int]]:
        if not torch.is_tensor(data):
            raise TypeError("data must be a torch.Tensor")
        if not data.dtype.is_floating_point:
            raise TypeError("data must be a floating point tensor")
        if data.ndim == 2:
            n, d = data.shape
            if n == 0:
                raise ValueError("data must contain at least one sample")
            batch = None
            data = data.unsqueeze(0)
        elif data.ndim == 3:
            bsz, n, d = data.shape
            if bsz == 0 or n == 0:
                raise ValueError("data must contain at least one sample")
            batch = bsz
        else:
            raise ValueError("data must have shape (N, D) or (B, N, D)")
        if self.d is None:
            self.d = int(d)
        elif d != self.d:
            raise ValueError(f"Expected d={self.d}, got d={d}")
        return data, batch

    def _compute_dtype_for_input(self, x_b: torch.Tensor) -> torch.dtype:
        if self.dtype is not None:
            return self.dtype
        return torch.float32 if x_b.dtype in (torch.float16, torch.bfloat16) else x_b.dtype

    def _engine_dtype(self, x_b: torch.Tensor) -> torch.dtype:
        compute = self._compute_dtype_for_input(x_b)
        if compute == torch.float64:
            raise TypeError("float64 data is not supported by the hip backend; pass dtype=torch.float32")
        return torch.bfloat16 if (compute == torch.bfloat16 and self.covariance_type == "spherical") else torch.float32

    def _param_dtype(self, x_b: torch.Tensor) -> Optional[torch.dtype]:
        """The dtype the parameters are kept in: an explicit half-precision
        ``dtype`` computed by the fp32 engine keeps them in that dtype between
        iterations, as the reference keeps its parameters in the compute dtype
        (the bf16 spherical engine rounds its means itself)."""
        if self.dtype in (torch.float16, torch.bfloat16) and self._engine_dtype(x_b) == torch.float32:
            return self.dtype
        return None

    def _engine_tensor(self, x_b: torch.Tensor) -> torch.Tensor:
        """x on the estimator's GPU in the dtype the engine reads: fp32 (the
        reference's compute dtype for float32 and half-precision input,
        gmmxx/interface.py:426-433), or bf16 for spherical when
        ``dtype=torch.bfloat16`` asks for it.  Other covariance types have no
        bf16 engine and compute an explicit bf16 dtype in fp32."""
        if self.device.type != "cuda":
            raise _hip.HipBackendUnavailable(
                f"the hip backend runs on a ROCm GPU; estimator device is {self.device}")
        return x_b.to(device=self.device, dtype=self._engine_dtype(x_b)).contiguous()

    def _is_large_cpu_stream_input(self, x_b: torch.Tensor) -> bool:
        """Host data longer than chunk_size_data_cpu rows streams through HBM in
        chunks instead of being copied whole (gmmxx/interface.py:434-439)."""
        return (x_b.device.type == "cpu" and self.device.type == "cuda"
                and x_b.shape[1] > self.chunk_size_data_cpu)

    def _resolve(self, x_b: torch.Tensor, k: int) -> str:
        shape = (x_b.shape[0], x_b.shape[1], x_b.shape[2], k)
        return _dispatch.resolve_backend_with_env(self.backend, self.covariance_type, shape, x_b.dtype,
                                                  legacy_no_triton=self._legacy_no_triton)

    # -- fit (gmmxx/interface.py:1277-1506) ---------------------------------

    def train(self, data: torch.Tensor):
        with self._matmul_precision_scope():
            return self._train_impl(data)

    def _train_impl(self, data: torch.Tensor):
        self._reset_fit_state()
        x_b, batch_size = self._normalize_input(data)
        torch.manual_seed(self.seed)
        if torch.cuda.is_available():
            torch.cuda.manual_seed_all(self.seed)
        streaming = self._is_large_cpu_stream_input(x_b)
        if streaming:
            # gmmxx/interface.py:452-490: host data streams through HBM (B = 1).
            self.last_backend_used_ = self._resolve(x_b, self.k)
            x_host = x_b
            labels_b, means_b, covs_b, weights_b, info = large_n.fit_large_n(
                x_host, self.k, self.covariance_type, device=self.device, max_iters=self.niter, tol=self.tol,
                verbose=self.verbose, init_params=self.init_params, reg_covar=self.reg_covar,
                chunk_size_N=self.chunk_size_data_cpu, compute_labels=self.compute_labels_on_fit,
                seed=self.seed, approx_top_k=self.approx_top_k, kmeans_init_iters=self.init_kmeans_iters,
                kmeans_init_tol=self.init_kmeans_tol, compute_dtype=self._engine_dtype(x_b),
                param_dtype=self._param_dtype(x_b))
        else:
            x_b = self._engine_tensor(x_b)
            self.last_backend_used_ = self._resolve(x_b, self.k)
            labels_b, means_b, covs_b, weights_b, info = em.fit(
                x_b, self.k, self.covariance_type, max_iters=self.niter, tol=self.tol, verbose=self.verbose,
                init_params=self.init_params, reg_covar=self.reg_covar, compute_labels=self.compute_labels_on_fit,
                approx_top_k=self.approx_top_k, kmeans_init_iters=self.init_kmeans_iters,
                kmeans_init_tol=self.init_kmeans_tol, param_dtype=self._param_dtype(x_b))
        self._scores_cache = None
        self.cluster_ids_b = labels_b
        self.means_b = means_b
        self.variances_b = covs_b
        self.covariances_b = covs_b
        self.weights_b = weights_b
        self._batch_size = batch_size
        self.means_ = self._squeeze_if_unbatched(means_b)
        self.weights_ = self._squeeze_if_unbatched(weights_b)
        self.covariances_ = self._squeeze_if_unbatched(covs_b)
        self.labels_ = self._squeeze_if_unbatched(labels_b)
        self.lower_bound_ = float(info["lower_bound"])
        self.lower_bound_history_ = list(info["lower_bound_history"])
        self.n_iter_ = int(info["n_iter"])
        self.init_source_ = str(info["init_source"])
        self.fit_info_ = dict(info)
        self.hip_estep_enabled_ = True
        self.triton_estep_enabled_ = self.triton_fused_update_enabled_ = False
        self.triton_approx_topk_enabled_ = self.triton_streaming_update_enabled_ = False
        self.triton_labels_enabled_ = False
        # gmmxx/interface.py:391-392: approximation in use and its effective k
        self.approximate_em_enabled_ = bool(info.get("approximate_em_enabled", False))
        self.approx_top_k_ = info.get("approx_top_k")
        self.large_n_streaming_enabled_ = self.copy_stream_prefetch_enabled_ = streaming
        self.cuda_estep_enabled_ = self.cuda_fused_update_enabled_ = self.cuda_approx_topk_enabled_ = False
        self.last_backend_used_ = "hip"

    def fit(self, data: torch.Tensor, y: Any = None):
        del y
        self.train(data)
        return self

    def fit_predict(self, data: torch.Tensor, y: Any = None) -> torch.Tensor:
        del y
        self.train(data)
        if self.cluster_ids_b is None:
            labels = self.predict(data)
            self.cluster_ids_b = labels.unsqueeze(0) if self._batch_size is None else labels
            self.labels_ = labels
            return labels
        return self._squeeze_if_unbatched(self.cluster_ids_b)

    # -- params (gmmxx/interface.py:1508-1603) ------------------------------

    def get_params(self, deep: bool = True) -> dict:
        del deep
        return {
            "d": self.d, "n_components": self.k, "max_iter": self.niter, "tol": self.tol,
            "random_state": self.seed, "chunk_size_data": self.chunk_size_data,
            "chunk_size_centroids": self.chunk_size_centroids, "chunk_size_data_cpu": self.chunk_size_data_cpu,
            "verbose": self.verbose, "dtype": self.dtype, "device": self.device, "init_params": self.init_params,
            "reg_covar": self.reg_covar, "init_kmeans_iters": self.init_kmeans_iters,
            "init_kmeans_tol": self.init_kmeans_tol, "covariance_type": self.covariance_type,
            "matmul_precision": self.matmul_precision, "compute_labels_on_fit": self.compute_labels_on_fit,
            "approx_top_k": self.approx_top_k, "backend": self.backend,
        }

    def set_params(self, **params: Any):
        if not params:
            return self
        valid = set(_PARAM_NAMES) | {"k", "niter", "seed", "use_triton"}
        for raw_name, value in params.items():
            if raw_name not in valid:
                raise ValueError(f"Invalid parameter {raw_name!r} for GMMXX")
            name = _SKLEARN_PARAM_ALIASES.get(raw_name, raw_name)
            if name == "d":
                value = _optional_positive_int(value, "d")
            elif name in {"k", "niter", "chunk_size_data", "chunk_size_centroids", "chunk_size_data_cpu",
                          "init_kmeans_iters"}:
                value = _positive_int(value, name)
            elif name in {"tol", "reg_covar", "init_kmeans_tol"}:
                value = float(value)
                if value < 0.0:
                    raise ValueError(f"{name} must be non-negative")
            elif name == "seed":
                value = int(value)
            elif name == "use_triton":
                if value is not None:
                    if self.backend != "auto":
                        raise ValueError("Cannot set use_triton when backend is already explicit "
                                         f"(self.backend={self.backend!r}). Drop use_triton; "
                                         "backend= is the canonical kwarg.")
                    warnings.warn("use_triton is deprecated and has no effect with gmmxx_amd; use backend='hip'",
                                  DeprecationWarning, stacklevel=2)
                    self._legacy_no_triton = not bool(value)
                continue
            elif name == "backend":
                _check_backend(value)
            elif name in {"verbose", "compute_labels_on_fit"}:
                value = bool(value)
            elif name == "covariance_type":
                value = _normalize_covariance_type(value)
            elif name == "matmul_precision" and value is not None and value not in {"highest", "high", "medium"}:
                raise ValueError("matmul_precision must be None, 'highest', 'high', or 'medium'")
            elif name == "approx_top_k":
                value = _optional_positive_int(value, "approx_top_k")
            elif name == "device":
                value = torch.device(value)
                self._raw_device = value
            setattr(self, name, value)
        self._reset_fit_state()
        return self

    # -- inference (gmmxx/interface.py:1605-2521) ---------------------------

    def _require_trained(self) -> None:
        if self.means_b is None or self.variances_b is None or self.weights_b is None:
            raise RuntimeError("Model not trained. Call train() or fit() first.")

    def _prepare_predict_input(self, data: torch.Tensor) -> tuple[torch.Tensor, Optional[int], bool]:
        """(x, batch size, streamed): host data longer than chunk_size_data_cpu rows
        stays on the host and is streamed (gmmxx/interface.py:1758-1769)."""
        self._require_trained()
        x_b, batch_size = self._normalize_input(data)
        if batch_size != self._batch_size:
            raise ValueError(f"Model was trained with batch size B={self._batch_size}, "
                             f"but received B={batch_size}.")
        self.last_backend_used_ = self._resolve(x_b, int(self.means_b.shape[1]))
        if self._is_large_cpu_stream_input(x_b):
            self._engine_dtype(x_b)   # rejects float64 as the in-memory path does
            return x_b, batch_size, True
        return self._engine_tensor(x_b), batch_size, False

    def _params(self):
        return self.means_b.contiguous(), self.variances_b.contiguous(), self.weights_b.contiguous()

    def predict(self, data: torch.Tensor) -> torch.Tensor:
        """First-max component index per sample, int64 (gmmxx/interface.py:1753-1971)."""
        with self._matmul_precision_scope():
            x_b, batch_size, streamed = self._prepare_predict_input(data)
            means, covs, weights = self._params()
            if streamed:
                labels = large_n.predict_large_n(x_b, means, covs, weights, self.covariance_type,
                    compute_dtype=self._engine_dtype(x_b),
                                                 device=self.device, chunk_size_N=self.chunk_size_data_cpu)
            else:
                _, labels = _hip.score(self.covariance_type, x_b, means, covs, weights, want_scores=False)
            return labels.squeeze(0) if batch_size is None else labels

    def _cache_scores(self, data: torch.Tensor, scores: torch.Tensor) -> None:
        """Keeps the per-sample scores that predict_proba computed on ``data``
        (the same E-step gives both), for a score_samples call on the same,
        unmodified tensor under the same fitted parameters."""
        try:
            params = self._fitted_params()
            self._scores_cache = (weakref.ref(data), data._version, tuple(weakref.ref(t) for t in params),
                                  tuple(t._version for t in params), scores)
        except TypeError:
            self._scores_cache = None

    def _fitted_params(self):
        return (self.means_b, self.variances_b, self.weights_b)

    def _cached_scores(self, data: torch.Tensor) -> Optional[torch.Tensor]:
        """The cached scores when ``data`` and the fitted parameter tensors are
        the very objects (identity through weak references, never ``id()``,
        which a new tensor can reuse after a refit) at the same versions."""
        c = self._scores_cache
        if c is None or not torch.is_tensor(data) or c[0]() is not data or c[1] != data._version:
            return None
        params = self._fitted_params()
        if (any(r() is not t for r, t in zip(c[2], params))
                or c[3] != tuple(t._version for t in params)):
            return None
        self._scores_cache = None
        return c[4]

    def predict_proba(self, data: torch.Tensor) -> torch.Tensor:
        """Responsibilities (B, N, K) fp32 (gmmxx/interface.py:1973-2268).  The
        per-sample scores come out of the same E-step
        (gmmxx_hip_predict_proba_score) and serve a following score_samples
        call on the same tensor."""
        with self._matmul_precision_scope():
            x_b, batch_size, streamed = self._prepare_predict_input(data)
            means, covs, weights = self._params()
            if streamed:
                probs = large_n.predict_proba_large_n(x_b, means, covs, weights, self.covariance_type,
                    compute_dtype=self._engine_dtype(x_b),
                                                      device=self.device, chunk_size_N=self.chunk_size_data_cpu)
            else:
                probs, scores = _hip.predict_proba_score(self.covariance_type, x_b, means, covs, weights)
                self._cache_scores(data, scores.squeeze(0) if batch_size is None else scores)
            return probs.squeeze(0) if batch_size is None else probs

    def score_samples(self, data: torch.Tensor) -> torch.Tensor:
        """Per-sample log-likelihood log Σ_k w_k N(x | μ_k, Σ_k), fp32
        (gmmxx/interface.py:2270-2521)."""
        cached = self._cached_scores(data)
        if cached is not None:
            return cached
        with self._matmul_precision_scope():
            x_b, batch_size, streamed = self._prepare_predict_input(data)
            means, covs, weights = self._params()
            if streamed:
                scores = large_n.score_samples_large_n(x_b, means, covs, weights, self.covariance_type,
                    compute_dtype=self._engine_dtype(x_b),
                                                       device=self.device, chunk_size_N=self.chunk_size_data_cpu)
            else:
                scores, _ = _hip.score(self.covariance_type, x_b, means, covs, weights, want_labels=False)
            return scores.squeeze(0) if batch_size is None else scores

    def score(self, data: torch.Tensor, y: Any = None) -> float:
        del y
        return float(self.score_samples(data).mean().item())

    # -- model selection (gmmxx/interface.py:2537-2558) ---------------------

    def _n_parameters(self, batch_size: int = 1) -> int:
        self._require_trained()
        d = int(self.means_b.shape[-1])
        k = int(self.means_b.shape[1])
        covariance_params = {"spherical": k, "diag": k * d, "tied": d * (d + 1) // 2,
                             "full": k * d * (d + 1) // 2}[self.covariance_type]
        return int(batch_size * (k * d + covariance_params + k - 1))

    def bic(self, data: torch.Tensor) -> float:
        scores = self.score_samples(data)
        n_samples = int(scores.numel())
        batch_size = int(scores.shape[0]) if scores.ndim == 2 else 1
        return float(-2.0 * scores.sum().item() + self._n_parameters(batch_size) * math.log(float(n_samples)))

    def aic(self, data: torch.Tensor) -> float:
        scores = self.score_samples(data)
        batch_size = int(scores.shape[0]) if scores.ndim == 2 else 1
        return float(-2.0 * scores.sum().item() + 2.0 * self._n_parameters(batch_size))
