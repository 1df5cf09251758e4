"""Backend resolution for the ``"hip"`` backend.

Mirrors the reference's ``gmmxx/_dispatch.py`` (:88-144): the estimator asks
``resolve_backend_with_env(requested, covariance, shape, dtype)`` which backend
runs a call, and ``GMMXX_BACKEND`` is consulted only when the request is
``"auto"``.  This package ships one compute backend, the HIP/gfx950 engine, so
the truth table is:

    requested  | engine usable and shape supported | otherwise
    -----------+-----------------------------------+-----------------------------
    "auto"     | "hip"                             | HipBackendUnavailable /
    "hip"      | "hip"                             |   UnsupportedShape (raised)
    "cuda", "triton", "torch"                      | ValueError: not provided here

There is deliberately no silent fallback: a request the engine cannot serve
raises, where the reference would have routed to its torch path
(gmmxx/_dispatch.py:124-129).  A caller who wants the torch path uses the
reference package for that call.
"""

from __future__ import annotations

import os
from typing import Any

import torch

from . import _hip

VALID_BACKENDS = {"auto", "hip", "cuda", "triton", "torch"}
PROVIDED_BACKENDS = {"auto", "hip"}
_COVARIANCES = ("spherical", "diag", "tied", "full")


class UnsupportedShape(_hip.HipRuntimeError):
    """The engine has no kernel for this covariance/shape/dtype."""


def _shape_bndk(shape: tuple) -> tuple[int, int, int, int]:
    """(B, N, D, K) from a (B, N, D, K) tuple, or (B, N, D) with K unknown (0)
    as the reference's inference paths pass it (gmmxx/_dispatch.py:36-49)."""
    if len(shape) == 4:
        return tuple(int(v) for v in shape)  # type: ignore[return-value]
    if len(shape) == 3:
        return int(shape[0]), int(shape[1]), int(shape[2]), 0
    raise ValueError(f"shape must have 3 or 4 dims, got {shape!r}")


def engine_dtype(covariance: str, dtype: Any) -> torch.dtype:
    """The dtype x is handed to the engine in: bf16 stays bf16 for spherical
    (exact bf16 products, fp32 accumulation); everything else runs in fp32."""
    if dtype == torch.bfloat16 and covariance == "spherical":
        return torch.bfloat16
    return torch.float32


def hip_supported(covariance: str, shape: tuple, dtype: Any) -> bool:
    """True iff the library has kernels for this call (role of the reference's
    cuda_*_supported gates, gmmxx/_runtime.py).  K unknown (0) checks K = 1."""
    if covariance not in _COVARIANCES:
        return False
    b, n, d, k = _shape_bndk(shape)
    return _hip.supported(covariance, engine_dtype(covariance, dtype), max(b, 1), max(n, 1), d, max(k, 1))


def resolve_backend(requested: str, covariance: str, shape: tuple, dtype: Any,
                    legacy_no_triton: bool = False) -> str:
    """Returns ``"hip"`` or raises; see the module docstring for the table.
    ``legacy_no_triton`` is accepted for signature parity and has no effect."""
    del legacy_no_triton
    if requested not in VALID_BACKENDS:
        raise ValueError(f"unknown backend {requested!r}; expected one of {sorted(VALID_BACKENDS)}")
    if requested not in PROVIDED_BACKENDS:
        raise ValueError(
            f"backend {requested!r} is provided by the reference gmmxx package; "
            "gmmxx_amd implements backend='hip' (and 'auto', which resolves to it)")
    _hip.require_hip()
    if not hip_supported(covariance, shape, dtype):
        raise UnsupportedShape(
            f"the hip backend has no kernel for covariance={covariance!r} shape={tuple(shape)!r} "
            f"dtype={dtype}: {_hip.last_error()}")
    return "hip"


def resolve_backend_with_env(requested: str, covariance: str, shape: tuple, dtype: Any,
                             legacy_no_triton: bool = False) -> str:
    """As ``resolve_backend``, but ``GMMXX_BACKEND`` overrides an ``"auto"``
    request (gmmxx/_dispatch.py:147-162).  Invalid values are ignored."""
    effective = requested
    if effective == "auto":
        env = os.environ.get("GMMXX_BACKEND")
        if env in VALID_BACKENDS:
            effective = env
    return resolve_backend(effective, covariance, shape, dtype, legacy_no_triton=legacy_no_triton)
