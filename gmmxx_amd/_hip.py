"""ctypes boundary to libgmmxx_hip.so (the HIP/gfx950 EM engine).

Role of the reference's ``gmmxx/_cuda.py`` (:1-1416) for the ``"hip"``
backend: validate tensors, pass raw device pointers and the current HIP stream
across the C ABI declared in ``include/gmmxx_hip.h``, and turn status codes
into Python exceptions.  There is no fallback path: if the library is missing
or a call fails, the caller gets an exception (``HipBackendUnavailable`` /
``HipRuntimeError``), never a silent CPU or PyTorch result.

Workspace and output tensors are allocated here through PyTorch's caching
allocator and handed to the library, which itself never allocates.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import torch

_LIB_NAME = "libgmmxx_hip.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)
ABI_VERSION = 2

COV_CODES = {"spherical": 0, "diag": 1, "tied": 2, "full": 3}
_DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1}
# parameter dtypes (gmmxx_problem.param_dtype): None / float32 keeps the parameters unrounded
_PARAM_CODES = {None: 0, torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


class HipBackendUnavailable(RuntimeError):
    """The HIP library is not built/loadable, or no GPU is visible
    (role of CudaBackendUnavailable, gmmxx/_cuda.py:35-36)."""


class HipRuntimeError(RuntimeError):
    """A library call returned a nonzero status (the message comes from
    gmmxx_hip_last_error), or a cooperative pass reported a timed-out wait."""


class HipRuntimeFallback(HipRuntimeError):
    """The reference's runtime-error contract (CudaRuntimeFallback,
    gmmxx/_cuda.py:39-54, gmmxx/_dispatch.py:189-204): a failing library call
    raises this, unless ``GMMXX_HIP_NO_FALLBACK=1``, in which case the plain
    HipRuntimeError propagates.  Nothing in this package catches it -- there is
    no CPU or PyTorch path to fall to; a dispatcher that has one (the
    reference's dispatch_kernel) catches it and re-resolves to torch."""


def no_fallback() -> bool:
    """``GMMXX_HIP_NO_FALLBACK=1``: errors surface as plain HipRuntimeError
    (role of _no_fallback, gmmxx/_cuda.py:51-54)."""
    return os.environ.get("GMMXX_HIP_NO_FALLBACK", "").lower() in {"1", "true", "yes"}


class DevInfo(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int32), ("supported", ctypes.c_int32), ("arch", ctypes.c_char * 64),
                ("compute_units", ctypes.c_int32), ("wave_size", ctypes.c_int32), ("clock_khz", ctypes.c_int32),
                ("coop_capacity", ctypes.c_int32), ("hbm_bytes", ctypes.c_int64),
                ("lds_per_workgroup", ctypes.c_int64)]


class _Problem(ctypes.Structure):
    _fields_ = [("covariance_type", ctypes.c_int32), ("x_dtype", ctypes.c_int32),
                ("B", ctypes.c_int64), ("N", ctypes.c_int64), ("D", ctypes.c_int64),
                ("K", ctypes.c_int64), ("param_dtype", ctypes.c_int32), ("reserved", ctypes.c_int32)]


_lib = None
_load_error: Optional[BaseException] = None


def _declare(lib):
    P = ctypes.POINTER(_Problem)
    vp, i64, f64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_int32
    sig = {
        "gmmxx_hip_abi_version": (ctypes.c_int, []),
        "gmmxx_hip_last_error": (ctypes.c_char_p, []),
        "gmmxx_hip_canary": (ctypes.c_int, [vp, vp, i64, i32, vp]),
        "gmmxx_hip_supported": (ctypes.c_int, [P]),
        "gmmxx_hip_device_info": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(DevInfo)]),
        "gmmxx_hip_take_status": (ctypes.c_int, [P, vp, i64, vp, vp]),
        "gmmxx_hip_workspace_bytes": (i64, [P]),
        "gmmxx_hip_em_step": (ctypes.c_int, [P, vp, vp, vp, vp, vp, f64, f64, vp, vp, i64, vp]),
        "gmmxx_hip_em_step_noalloc": (ctypes.c_int, [P, vp, vp, vp, vp, vp, f64, f64, vp, vp]),
        "gmmxx_hip_em_phase": (ctypes.c_int, [P, ctypes.c_int, vp, vp, vp, vp, vp, f64, f64, vp, vp, i64, vp]),
        "gmmxx_hip_estep_stats": (ctypes.c_int, [P, vp, vp, vp, vp, f64, f64, vp, vp, vp, vp, vp, i64, vp]),
        "gmmxx_hip_score": (ctypes.c_int, [P, vp, vp, vp, vp, vp, vp, vp, i64, vp]),
        "gmmxx_hip_predict_proba": (ctypes.c_int, [P, vp, vp, vp, vp, vp, vp, i64, vp]),
        "gmmxx_hip_predict_proba_score": (ctypes.c_int, [P, vp, vp, vp, vp, vp, vp, vp, i64, vp]),
        "gmmxx_hip_gram": (ctypes.c_int, [P, vp, vp, vp, i64, vp]),
        "gmmxx_hip_finalize_stats": (ctypes.c_int, [P, vp, vp, vp, vp, f64, f64, vp, vp, vp, vp, i64, vp]),
        "gmmxx_hip_kmeans_pp_workspace_bytes": (i64, [i64, i64, i64, i64, ctypes.c_int]),
        "gmmxx_hip_kmeans_pp": (ctypes.c_int, [vp, i64, i64, i64, i64, ctypes.c_int, vp, vp, vp, vp, i64, vp]),
        "gmmxx_hip_topk_workspace_bytes": (i64, [P, ctypes.c_int]),
        "gmmxx_hip_estep_stats_topk": (ctypes.c_int, [P, vp, vp, vp, vp, f64, f64, ctypes.c_int, vp, vp, vp,
                                                      vp, vp, i64, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def exported_symbols() -> Tuple[str, ...]:
    return ("gmmxx_hip_abi_version", "gmmxx_hip_last_error", "gmmxx_hip_canary",
            "gmmxx_hip_supported", "gmmxx_hip_device_info", "gmmxx_hip_take_status", "gmmxx_hip_workspace_bytes", "gmmxx_hip_em_step", "gmmxx_hip_em_step_noalloc",
            "gmmxx_hip_em_phase",
            "gmmxx_hip_estep_stats", "gmmxx_hip_score", "gmmxx_hip_predict_proba",
            "gmmxx_hip_predict_proba_score",
            "gmmxx_hip_gram", "gmmxx_hip_finalize_stats", "gmmxx_hip_topk_workspace_bytes",
            "gmmxx_hip_estep_stats_topk", "gmmxx_hip_kmeans_pp_workspace_bytes", "gmmxx_hip_kmeans_pp")


def load_library(path: Optional[str] = None):
    """Loads (once) and returns the ctypes handle; raises HipBackendUnavailable."""
    global _lib, _load_error
    if _lib is not None and path is None:
        return _lib
    p = path or os.environ.get("GMMXX_HIP_LIBRARY", _LIB_PATH)
    try:
        lib = _declare(ctypes.CDLL(p, mode=ctypes.RTLD_LOCAL))
    except OSError as exc:
        _load_error = exc
        raise HipBackendUnavailable(
            f"cannot load {p}: {exc}. Build it with `python -m gmmxx_amd.build`.") from exc
    ver = lib.gmmxx_hip_abi_version()
    if ver != ABI_VERSION:
        raise HipBackendUnavailable(f"{p} has ABI version {ver}, expected {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def library_loaded() -> bool:
    return _lib is not None


def has_hip() -> bool:
    """True iff the library loads and a GPU is visible (role of has_cuda, gmmxx/_cuda.py:44-46)."""
    if not torch.cuda.is_available():
        return False
    try:
        load_library()
    except HipBackendUnavailable:
        return False
    return True


def require_hip() -> None:
    """Raises HipBackendUnavailable unless the engine can run (gmmxx/_cuda.py:57-64)."""
    load_library()
    if not torch.cuda.is_available():
        raise HipBackendUnavailable("no ROCm GPU is visible to PyTorch")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def last_error() -> str:
    """The calling thread's last error message from the library."""
    return load_library().gmmxx_hip_last_error().decode(errors="replace")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        cls = HipRuntimeError if no_fallback() else HipRuntimeFallback
        raise cls(f"{what} failed (status {rc}): {last_error()}")


def problem(covariance_type: str, x_dtype: torch.dtype, B: int, N: int, D: int, K: int,
            param_dtype: Optional[torch.dtype] = None) -> _Problem:
    """The problem descriptor.  ``param_dtype`` (bfloat16 / float16) keeps the
    parameters in that dtype between iterations, as the reference does for a
    half-precision x computed in fp32 (see gmmxx_problem in include/gmmxx_hip.h)."""
    if covariance_type not in COV_CODES:
        raise ValueError(f"unknown covariance_type {covariance_type!r}")
    if x_dtype not in _DTYPE_CODES:
        raise ValueError(f"x dtype must be float32 or bfloat16, got {x_dtype}")
    if param_dtype not in _PARAM_CODES:
        raise ValueError(f"param_dtype must be None, float32, bfloat16 or float16, got {param_dtype}")
    return _Problem(COV_CODES[covariance_type], _DTYPE_CODES[x_dtype], int(B), int(N), int(D), int(K),
                    _PARAM_CODES[param_dtype], 0)


def supported(covariance_type: str, x_dtype: torch.dtype, B: int, N: int, D: int, K: int) -> bool:
    """Shape/dtype gate of the engine, answered by the library itself."""
    if x_dtype not in _DTYPE_CODES or covariance_type not in COV_CODES:
        return False
    lib = load_library()
    return bool(lib.gmmxx_hip_supported(ctypes.byref(problem(covariance_type, x_dtype, B, N, D, K))))


def _device_tensor(t: torch.Tensor, name: str, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    if not torch.is_tensor(t):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name}: must be on a GPU device, got {t.device}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name}: dtype must be {dtype}, got {t.dtype}")
    t = t.contiguous()
    # The library reads rows with 16-byte loads (and requires it for spherical bf16 at
    # D = 128): a view that starts mid-allocation is copied to an aligned buffer.
    return t if t.data_ptr() % 16 == 0 else t.clone()


class Workspace:
    """Device scratch for one problem shape, sized by the library (256-byte aligned)."""

    def __init__(self, prob: _Problem, device: torch.device, *, top_k: Optional[int] = None):
        """``top_k``: size for gmmxx_hip_estep_stats_topk with that k instead."""
        lib = load_library()
        if top_k is None:
            nbytes = int(lib.gmmxx_hip_workspace_bytes(ctypes.byref(prob)))
        else:
            nbytes = int(lib.gmmxx_hip_topk_workspace_bytes(ctypes.byref(prob), int(top_k)))
        if nbytes < 0:
            raise HipRuntimeError("problem not supported by the HIP engine: "
                                  + lib.gmmxx_hip_last_error().decode(errors="replace"))
        # Zeroed once: the asynchronous status word (gmmxx_hip_take_status) starts clear.
        self._buf = torch.zeros(nbytes + 256, dtype=torch.uint8, device=device)
        base = self._buf.data_ptr()
        self.ptr = ctypes.c_void_p(base + (-base) % 256)
        self.nbytes = nbytes
        self.prob = prob
        self.device = torch.device(device)


def take_status(ws: Workspace) -> torch.Tensor:
    """Device uint32 word: the asynchronous failures recorded on ``ws`` since the
    last call (nonzero: a single pass whose workgroups exchange row partials --
    the cooperative spherical bf16 kernel or the fp32 exchange pass -- gave up
    waiting for a partner; its iteration kept the parameters and wrote a NaN
    lower bound).  Clears it;
    stream-ordered, no synchronisation."""
    out = torch.zeros((1,), dtype=torch.int32, device=ws.device)
    _check(_lib.gmmxx_hip_take_status(ctypes.byref(ws.prob), ws.ptr, ws.nbytes, _ptr(out), _stream(ws.device)),
           "gmmxx_hip_take_status")
    return out


def raise_on_status(status: torch.Tensor, what: str) -> None:
    """Raises HipRuntimeError when a take_status word is nonzero (synchronises)."""
    if int(status.item()) != 0:
        raise HipRuntimeError(
            f"{what}: a single-pass kernel whose workgroups exchange row partials (cooperative "
            "spherical bf16 kernel or fp32 exchange pass) timed out waiting for a partner workgroup: "
            "the members of a group were not all resident (another kernel or process holding part of "
            "the GPU); the affected iterations left the parameters unchanged and recorded a NaN lower "
            "bound (GMMXX_HIP_NO_COOP=1 / GMMXX_HIP_NO_XCH=1 select the two-pass kernels)")


def device_info(device: int = 0) -> dict:
    """The library's view of a device (gmmxx_hip_device_info)."""
    info = DevInfo()
    _check(load_library().gmmxx_hip_device_info(int(device), ctypes.byref(info)), "gmmxx_hip_device_info")
    return {"device": info.device, "supported": bool(info.supported), "arch": info.arch.decode(errors="replace"),
            "compute_units": info.compute_units, "wave_size": info.wave_size, "clock_khz": info.clock_khz,
            "coop_capacity": info.coop_capacity, "hbm_bytes": info.hbm_bytes,
            "lds_per_workgroup": info.lds_per_workgroup}


def _shape(x: torch.Tensor, means: torch.Tensor) -> Tuple[int, int, int, int]:
    if x.ndim != 3:
        raise ValueError("x must have shape (B, N, D)")
    if means.ndim != 3 or means.shape[0] != x.shape[0] or means.shape[2] != x.shape[2]:
        raise ValueError("means must have shape (B, K, D) matching x")
    return int(x.shape[0]), int(x.shape[1]), int(x.shape[2]), int(means.shape[1])


def _cov_shape(cov: str, B: int, K: int, D: int) -> Tuple[int, ...]:
    return {"spherical": (B, K), "diag": (B, K, D), "tied": (B, D, D), "full": (B, K, D, D)}[cov]


def _check_params(cov, means, covs, weights, B, K, D):
    if tuple(covs.shape) != _cov_shape(cov, B, K, D):
        raise ValueError(f"{cov} covariances must have shape {_cov_shape(cov, B, K, D)}, got {tuple(covs.shape)}")
    if tuple(weights.shape) != (B, K):
        raise ValueError(f"weights must have shape {(B, K)}, got {tuple(weights.shape)}")


# ---------------------------------------------------------------------------
# Operations
# ---------------------------------------------------------------------------

def canary_add_offset(inp: torch.Tensor, offset: int) -> torch.Tensor:
    """out = inp + offset on the GPU (role of gmmxx/_cuda.py canary_add_offset)."""
    require_hip()
    inp = _device_tensor(inp, "input", torch.int32)
    out = torch.empty_like(inp)
    _check(_lib.gmmxx_hip_canary(_ptr(inp), _ptr(out), inp.numel(), int(offset), _stream(inp.device)),
           "gmmxx_hip_canary")
    return out


def gram(x: torch.Tensor, ws: Optional[Workspace] = None) -> torch.Tensor:
    """XᵀX per batch, (B, D, D) fp32."""
    require_hip()
    x = _device_tensor(x, "x", torch.float32)
    B, N, D = x.shape
    prob = problem("tied", x.dtype, B, N, D, 1)
    ws = ws or Workspace(prob, x.device)
    out = torch.empty((B, D, D), dtype=torch.float32, device=x.device)
    _check(_lib.gmmxx_hip_gram(ctypes.byref(prob), _ptr(x), _ptr(out), ws.ptr, ws.nbytes, _stream(x.device)),
           "gmmxx_hip_gram")
    return out


def em_step(covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
            weights: torch.Tensor, lower_bound_out: torch.Tensor, *, reg_covar: float = 1e-6,
            min_weight: float = 1e-8, gram_xx: Optional[torch.Tensor] = None,
            ws: Optional[Workspace] = None, param_dtype: Optional[torch.dtype] = None) -> None:
    """One in-place soft-EM iteration on (means, covs, weights); fp32 contiguous
    device tensors.  ``lower_bound_out`` (1 float, device) receives the mean
    log-likelihood under the entry parameters.  ``param_dtype``: see ``problem``."""
    require_hip()
    x = _device_tensor(x, "x")
    B, N, D, K = _shape(x, means)
    for t, nm in ((means, "means"), (covs, "covariances"), (weights, "weights"), (lower_bound_out, "lower_bound")):
        if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
            raise ValueError(f"{nm} must be a contiguous float32 GPU tensor")
    _check_params(covariance_type, means, covs, weights, B, K, D)
    prob = problem(covariance_type, x.dtype, B, N, D, K, param_dtype)
    ws = ws or Workspace(prob, x.device)
    if covariance_type == "tied" and gram_xx is None:
        raise ValueError("tied EM needs gram_xx = XᵀX")
    _check(_lib.gmmxx_hip_em_step(ctypes.byref(prob), _ptr(x), _ptr(means), _ptr(covs), _ptr(weights),
                                  _ptr(gram_xx), float(reg_covar), float(min_weight), _ptr(lower_bound_out),
                                  ws.ptr, ws.nbytes, _stream(x.device)), "gmmxx_hip_em_step")


NOALLOC_SCRATCH_BYTES = 64 << 20


def em_step_noalloc(covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
                    weights: torch.Tensor, lower_bound_out: torch.Tensor, *, reg_covar: float = 1e-6,
                    min_weight: float = 1e-8, gram_xx: Optional[torch.Tensor] = None) -> None:
    """em_step on the library's static device scratch (gmmxx_hip_em_step_noalloc):
    no workspace is allocated; problems needing more than 64 MiB of workspace
    are refused.  Calls on one device share the scratch and must not overlap."""
    require_hip()
    x = _device_tensor(x, "x")
    B, N, D, K = _shape(x, means)
    for t, nm in ((means, "means"), (covs, "covariances"), (weights, "weights"), (lower_bound_out, "lower_bound")):
        if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
            raise ValueError(f"{nm} must be a contiguous float32 GPU tensor")
    _check_params(covariance_type, means, covs, weights, B, K, D)
    if covariance_type == "tied" and gram_xx is None:
        raise ValueError("tied EM needs gram_xx = XᵀX")
    prob = problem(covariance_type, x.dtype, B, N, D, K)
    with torch.cuda.device(x.device):
        _check(_lib.gmmxx_hip_em_step_noalloc(ctypes.byref(prob), _ptr(x), _ptr(means), _ptr(covs), _ptr(weights),
                                              _ptr(gram_xx), float(reg_covar), float(min_weight),
                                              _ptr(lower_bound_out), _stream(x.device)),
               "gmmxx_hip_em_step_noalloc")


EM_PHASES = ("prepare", "lse_tile", "combine", "stats_tile", "reduce", "finalize")


def em_phase(phase: str, covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
             weights: torch.Tensor, lower_bound_out: torch.Tensor, ws: Workspace, *,
             reg_covar: float = 1e-6, min_weight: float = 1e-8,
             gram_xx: Optional[torch.Tensor] = None, param_dtype: Optional[torch.dtype] = None) -> None:
    """Runs one phase of em_step (see EM_PHASES) on the current stream; the
    workspace carries the state between phases."""
    require_hip()
    if phase not in EM_PHASES:
        raise ValueError(f"phase must be one of {EM_PHASES}")
    x = _device_tensor(x, "x")
    B, N, D, K = _shape(x, means)
    for t, nm in ((means, "means"), (covs, "covariances"), (weights, "weights"), (lower_bound_out, "lower_bound")):
        if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
            raise ValueError(f"{nm} must be a contiguous float32 GPU tensor")
    _check_params(covariance_type, means, covs, weights, B, K, D)
    prob = problem(covariance_type, x.dtype, B, N, D, K, param_dtype)
    _check(_lib.gmmxx_hip_em_phase(ctypes.byref(prob), EM_PHASES.index(phase), _ptr(x), _ptr(means), _ptr(covs),
                                   _ptr(weights), _ptr(gram_xx), float(reg_covar), float(min_weight),
                                   _ptr(lower_bound_out), ws.ptr, ws.nbytes, _stream(x.device)),
           f"gmmxx_hip_em_phase({phase})")


def estep_stats(covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
                weights: torch.Tensor, *, reg_covar: float = 1e-6, min_weight: float = 1e-8,
                ws: Optional[Workspace] = None, param_dtype: Optional[torch.dtype] = None):
    """Sufficient statistics of one E-step: (nk, sum_x, sum_q, ll_sum).
    ``param_dtype``: the prelude's weights kept in it (see ``problem``)."""
    require_hip()
    x = _device_tensor(x, "x")
    means = _device_tensor(means, "means", torch.float32)
    covs = _device_tensor(covs, "covariances", torch.float32)
    weights = _device_tensor(weights, "weights", torch.float32)
    B, N, D, K = _shape(x, means)
    _check_params(covariance_type, means, covs, weights, B, K, D)
    prob = problem(covariance_type, x.dtype, B, N, D, K, param_dtype)
    ws = ws or Workspace(prob, x.device)
    dev = x.device
    nk = torch.empty((B, K), dtype=torch.float32, device=dev)
    sum_x = torch.empty((B, K, D), dtype=torch.float32, device=dev)
    q_shape = {"spherical": (B, K), "diag": (B, K, D), "full": (B, K, D, D)}.get(covariance_type)
    sum_q = torch.empty(q_shape, dtype=torch.float32, device=dev) if q_shape else None
    ll = torch.empty((1,), dtype=torch.float32, device=dev)
    _check(_lib.gmmxx_hip_estep_stats(ctypes.byref(prob), _ptr(x), _ptr(means), _ptr(covs), _ptr(weights),
                                      float(reg_covar), float(min_weight), _ptr(nk), _ptr(sum_x), _ptr(sum_q),
                                      _ptr(ll), ws.ptr, ws.nbytes, _stream(dev)), "gmmxx_hip_estep_stats")
    return nk, sum_x, sum_q, ll


def estep_stats_topk(covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
                     weights: torch.Tensor, top_k: int, *, reg_covar: float = 1e-6, min_weight: float = 1e-8,
                     ws: Optional[Workspace] = None, param_dtype: Optional[torch.dtype] = None):
    """Approximate top-k E-step statistics (nk, sum_x, sum_q, ll_sum): each row's
    responsibility mass is spread over its ``top_k`` largest logits only (ties by
    lower component index), normalised over them; ``ll_sum`` sums the top-k
    log-normalisers.  ``1 <= top_k < K``.  For top_k > 1 the workspace holds the
    (B, N, K) logits, so callers pass row chunks (gmmxx/torch_fallback.py:667-777);
    top_k = 1 (hard assignment) stores none."""
    require_hip()
    x = _device_tensor(x, "x")
    means = _device_tensor(means, "means", torch.float32)
    covs = _device_tensor(covs, "covariances", torch.float32)
    weights = _device_tensor(weights, "weights", torch.float32)
    B, N, D, K = _shape(x, means)
    _check_params(covariance_type, means, covs, weights, B, K, D)
    if not 1 <= int(top_k) < K:
        raise ValueError(f"top_k must satisfy 1 <= top_k < K={K}, got {top_k}")
    prob = problem(covariance_type, x.dtype, B, N, D, K, param_dtype)
    ws = ws or Workspace(prob, x.device, top_k=int(top_k))
    dev = x.device
    nk = torch.empty((B, K), dtype=torch.float32, device=dev)
    sum_x = torch.empty((B, K, D), dtype=torch.float32, device=dev)
    q_shape = {"spherical": (B, K), "diag": (B, K, D), "full": (B, K, D, D)}.get(covariance_type)
    sum_q = torch.empty(q_shape, dtype=torch.float32, device=dev) if q_shape else None
    ll = torch.empty((1,), dtype=torch.float32, device=dev)
    _check(_lib.gmmxx_hip_estep_stats_topk(ctypes.byref(prob), _ptr(x), _ptr(means), _ptr(covs), _ptr(weights),
                                           float(reg_covar), float(min_weight), int(top_k), _ptr(nk),
                                           _ptr(sum_x), _ptr(sum_q), _ptr(ll), ws.ptr, ws.nbytes, _stream(dev)),
           "gmmxx_hip_estep_stats_topk")
    return nk, sum_x, sum_q, ll


def kmeans_pp(sample: torch.Tensor, n_components: int, first_idx: torch.Tensor, draws: torch.Tensor) -> torch.Tensor:
    """Greedy k-means++ centres (B, K, D) fp32 from a row sample (B, S, D), with the
    random numbers given: ``first_idx`` (B,) int64 and ``draws`` (B, K-1, T) uniform
    in [0, 1), T candidates per step (gmmxx/torch_fallback.py:1390-1451)."""
    require_hip()
    sample = _device_tensor(sample, "sample", torch.float32)
    if sample.ndim != 3:
        raise ValueError("sample must have shape (B, S, D)")
    B, S, D = (int(v) for v in sample.shape)
    K = int(n_components)
    dev = sample.device
    first_idx = first_idx.to(device=dev, dtype=torch.int64).contiguous()
    draws = draws.to(device=dev, dtype=torch.float32).contiguous()
    if tuple(first_idx.shape) != (B,):
        raise ValueError("first_idx must have shape (B,)")
    if draws.ndim != 3 or draws.shape[0] != B or draws.shape[1] != K - 1:
        raise ValueError("draws must have shape (B, K-1, trials)")
    trials = int(draws.shape[2]) if K > 1 else 1
    need = int(_lib.gmmxx_hip_kmeans_pp_workspace_bytes(B, S, D, K, trials))
    if need < 0:
        raise ValueError("k-means++ needs 1 <= K <= S <= 65536, D <= 1024 and 1 <= trials <= 16")
    buf = torch.empty(need + 256, dtype=torch.uint8, device=dev)
    base = buf.data_ptr()
    centers = torch.empty((B, K, D), dtype=torch.float32, device=dev)
    _check(_lib.gmmxx_hip_kmeans_pp(_ptr(sample), B, S, D, K, trials, _ptr(first_idx), _ptr(draws),
                                    _ptr(centers), ctypes.c_void_p(base + (-base) % 256), need, _stream(dev)),
           "gmmxx_hip_kmeans_pp")
    return centers


def finalize_stats(covariance_type: str, nk: torch.Tensor, sum_x: torch.Tensor, sum_q: Optional[torch.Tensor],
                   means: torch.Tensor, covs: torch.Tensor, weights: torch.Tensor, n_rows: int, *,
                   gram_xx: Optional[torch.Tensor] = None, reg_covar: float = 1e-6,
                   min_weight: float = 1e-8, ws: Optional[Workspace] = None,
                   x_dtype: torch.dtype = torch.float32, param_dtype: Optional[torch.dtype] = None) -> None:
    """M-step in place on (means, covs, weights) from sufficient statistics summed
    over row chunks (``estep_stats`` layout); ``n_rows`` is the total row count.
    ``x_dtype`` is the statistics' input dtype: spherical bf16 x stores the means
    rounded to bf16, as ``em_step`` does; ``param_dtype``: see ``problem``."""
    require_hip()
    for t, nm in ((means, "means"), (covs, "covariances"), (weights, "weights")):
        if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
            raise ValueError(f"{nm} must be a contiguous float32 GPU tensor")
    B, K, D = int(means.shape[0]), int(means.shape[1]), int(means.shape[2])
    _check_params(covariance_type, means, covs, weights, B, K, D)
    nk = _device_tensor(nk, "nk", torch.float32)
    sum_x = _device_tensor(sum_x, "sum_x", torch.float32)
    if sum_q is not None:
        sum_q = _device_tensor(sum_q, "sum_q", torch.float32)
    if gram_xx is not None:
        gram_xx = _device_tensor(gram_xx, "gram_xx", torch.float32)
    prob = problem(covariance_type, x_dtype, B, int(n_rows), D, K, param_dtype)
    ws = ws or Workspace(problem(covariance_type, x_dtype, B, 1, D, K), means.device)
    _check(_lib.gmmxx_hip_finalize_stats(ctypes.byref(prob), _ptr(nk), _ptr(sum_x), _ptr(sum_q), _ptr(gram_xx),
                                         float(reg_covar), float(min_weight), _ptr(means), _ptr(covs),
                                         _ptr(weights), ws.ptr, ws.nbytes, _stream(means.device)),
           "gmmxx_hip_finalize_stats")


def score(covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
          weights: torch.Tensor, *, want_scores: bool = True, want_labels: bool = True,
          ws: Optional[Workspace] = None):
    """Per-sample log-likelihood (B, N) fp32 and/or first-max labels (B, N) int64."""
    require_hip()
    x = _device_tensor(x, "x")
    means = _device_tensor(means, "means", torch.float32)
    covs = _device_tensor(covs, "covariances", torch.float32)
    weights = _device_tensor(weights, "weights", torch.float32)
    B, N, D, K = _shape(x, means)
    _check_params(covariance_type, means, covs, weights, B, K, D)
    prob = problem(covariance_type, x.dtype, B, N, D, K)
    ws = ws or Workspace(prob, x.device)
    scores = torch.empty((B, N), dtype=torch.float32, device=x.device) if want_scores else None
    labels = torch.empty((B, N), dtype=torch.int64, device=x.device) if want_labels else None
    _check(_lib.gmmxx_hip_score(ctypes.byref(prob), _ptr(x), _ptr(means), _ptr(covs), _ptr(weights),
                                _ptr(scores), _ptr(labels), ws.ptr, ws.nbytes, _stream(x.device)),
           "gmmxx_hip_score")
    return scores, labels


def predict_proba(covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
                  weights: torch.Tensor, *, ws: Optional[Workspace] = None) -> torch.Tensor:
    """Responsibilities (B, N, K) fp32."""
    require_hip()
    x = _device_tensor(x, "x")
    means = _device_tensor(means, "means", torch.float32)
    covs = _device_tensor(covs, "covariances", torch.float32)
    weights = _device_tensor(weights, "weights", torch.float32)
    B, N, D, K = _shape(x, means)
    _check_params(covariance_type, means, covs, weights, B, K, D)
    prob = problem(covariance_type, x.dtype, B, N, D, K)
    ws = ws or Workspace(prob, x.device)
    out = torch.empty((B, N, K), dtype=torch.float32, device=x.device)
    _check(_lib.gmmxx_hip_predict_proba(ctypes.byref(prob), _ptr(x), _ptr(means), _ptr(covs), _ptr(weights),
                                        _ptr(out), ws.ptr, ws.nbytes, _stream(x.device)),
           "gmmxx_hip_predict_proba")
    return out


def predict_proba_score(covariance_type: str, x: torch.Tensor, means: torch.Tensor, covs: torch.Tensor,
                        weights: torch.Tensor, *, ws: Optional[Workspace] = None):
    """(responsibilities (B, N, K), per-sample log-likelihood (B, N)) from one
    E-step (gmmxx_hip_predict_proba_score)."""
    require_hip()
    x = _device_tensor(x, "x")
    means = _device_tensor(means, "means", torch.float32)
    covs = _device_tensor(covs, "covariances", torch.float32)
    weights = _device_tensor(weights, "weights", torch.float32)
    B, N, D, K = _shape(x, means)
    _check_params(covariance_type, means, covs, weights, B, K, D)
    prob = problem(covariance_type, x.dtype, B, N, D, K)
    ws = ws or Workspace(prob, x.device)
    proba = torch.empty((B, N, K), dtype=torch.float32, device=x.device)
    scores = torch.empty((B, N), dtype=torch.float32, device=x.device)
    _check(_lib.gmmxx_hip_predict_proba_score(ctypes.byref(prob), _ptr(x), _ptr(means), _ptr(covs), _ptr(weights),
                                              _ptr(proba), _ptr(scores), ws.ptr, ws.nbytes, _stream(x.device)),
           "gmmxx_hip_predict_proba_score")
    return proba, scores
