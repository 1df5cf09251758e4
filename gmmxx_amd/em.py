"""Host-side EM loops of the HIP backend.

Function-level API mirroring the reference's ``batch_gmm_*_torch_native``
(gmmxx/torch_fallback.py:1897-3336): same positional/keyword arguments, same
return tuple ``(labels, means, covariances, weights, info)``.  Every EM
iteration is one call of ``gmmxx_hip_em_step`` on the current stream; with
``tol == 0`` and ``verbose=False`` nothing synchronises until the loop ends.

Semantics follow the reference's soft EM.  fp32 input runs the fp32 algorithm
(every product fp32-accurate).  bf16 input (spherical only) stays bf16 in HBM
and is computed by the bf16 engine.  Its means are bf16, as the reference keeps
them in x's dtype (torch_fallback.py:1451, :2295): the initial means and every
M-step's means are rounded to bf16 (stored in fp32 tensors), while variances
and weights stay fp32.  The E-step multiplies exact bf16 x by the bf16 means
with fp32 accumulation (the cooperative and fused kernels; the two-pass kernels use a
hi + lo bf16 split of the fp32 operand -2·μ/σ², about 16 significand bits), and
the responsibilities are rounded to bf16 before the M-step product -- more
accurate than the reference's bf16 arithmetic on the same input, but not the
fp32 algorithm (the bf16 bar is 2e-3 on the log-likelihood).  The estimator
upcasts half-precision input to fp32 unless ``dtype=torch.bfloat16`` is given,
as the reference does.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from . import _hip

_COVS = ("spherical", "diag", "tied", "full")


def _as_device_input(x: torch.Tensor, covariance_type: str) -> torch.Tensor:
    if not torch.is_tensor(x):
        raise TypeError("x must be a torch.Tensor")
    if x.ndim != 3:
        raise ValueError("x must have shape (B, N, D)")
    if not x.is_cuda:
        raise ValueError(f"x must be on a GPU device for the hip backend, got {x.device}")
    if x.dtype == torch.bfloat16 and covariance_type == "spherical":
        return x.contiguous()
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        raise TypeError(f"unsupported dtype {x.dtype}")
    return x.to(torch.float32).contiguous()


def _f32(t: torch.Tensor, device) -> torch.Tensor:
    return t.detach().to(device=device, dtype=torch.float32).contiguous().clone()


def _sym(m: torch.Tensor) -> torch.Tensor:
    return 0.5 * (m + m.transpose(-1, -2))


# --- default-variance initialisers (torch_fallback.py:1348-1381), on device ---

def global_spherical_variance(x: torch.Tensor, k: int, reg_covar: float) -> torch.Tensor:
    d = x.shape[-1]
    xf = x.to(torch.float32)
    mean = xf.mean(dim=1)
    second = xf.square().sum(dim=-1).mean(dim=1)
    gv = (second - mean.square().sum(dim=-1)).clamp_min(0.0) / float(d)
    return gv.clamp_min(reg_covar).unsqueeze(-1).expand(-1, k).contiguous()


def global_diag_variance(x: torch.Tensor, k: int, reg_covar: float) -> torch.Tensor:
    xf = x.to(torch.float32)
    gv = (xf - xf.mean(dim=1, keepdim=True)).square().mean(dim=1).clamp_min(reg_covar)
    return gv.unsqueeze(1).expand(-1, k, -1).contiguous()


def global_tied_covariance(x: torch.Tensor, reg_covar: float) -> torch.Tensor:
    n, d = x.shape[1], x.shape[2]
    xf = x.to(torch.float32)
    c = xf - xf.mean(dim=1, keepdim=True)
    cov = torch.bmm(c.transpose(1, 2), c) / float(n)
    return (_sym(cov) + reg_covar * torch.eye(d, device=x.device)).contiguous()


def _engine_means(means: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """bf16 x keeps its means in bf16 (torch_fallback.py:1451, :2295), stored
    here as fp32 tensors holding bf16 values."""
    return means.to(torch.bfloat16).to(torch.float32) if x.dtype == torch.bfloat16 else means


def round_params(means, covs, weights, covariance_type, param_dtype):
    """The parameters as kept in ``param_dtype`` (None: unchanged), as fp32
    tensors: the means, and for diag/tied/full the covariances and weights too,
    as the reference keeps a half-precision x's parameters in its dtype
    (torch_fallback.py:1661-1682 at entry, :2295, :2654-2666, :3143-3167 after
    every M-step; spherical variances and weights stay fp32)."""
    if param_dtype is None or param_dtype == torch.float32:
        return means, covs, weights
    r = lambda t: t.to(param_dtype).to(torch.float32).contiguous()
    if covariance_type == "spherical":
        return r(means), covs, weights
    return r(means), r(covs), r(weights)


def _init_weights(init_weights, bsz, k, device):
    w = (torch.full((bsz, k), 1.0 / float(k), device=device) if init_weights is None
         else _f32(init_weights, device))
    if tuple(w.shape) != (bsz, k):
        raise ValueError("init_weights must have shape (B, K)")
    w = w.clamp_min(1e-8)
    return (w / w.sum(dim=-1, keepdim=True)).contiguous()


def flash_kmeans_emulated() -> bool:
    """Whether ``init_params="kmeans"`` runs the k-means initialisation.

    The reference runs k-means only when the optional flash-kmeans package
    imports (``_kmeans_initialize`` returns None without it,
    torch_fallback.py:1571-1582); its default ``init_params="kmeans"`` then
    silently becomes random rows plus the global variance with
    ``init_source="random"`` (:1700-1727, and likewise :1747-1774, :1807-1834,
    :1867-1894).  This engine runs the k-means initialisation on the device by
    default, i.e. it behaves like a reference with flash-kmeans installed.
    ``GMMXX_HIP_FLASH_KMEANS=0`` reproduces a reference without it: the random
    branch, drawn from the same global RNG call (``torch.randint`` on x's
    device) as the reference's ``_random_init_means`` (:1384-1387)."""
    import os
    return os.environ.get("GMMXX_HIP_FLASH_KMEANS", "1") != "0"


def initialize(x: torch.Tensor, covariance_type: str, n_components: int, *, init_means=None,
               init_covs=None, init_weights=None, reg_covar: float = 1e-6,
               init_params: str = "kmeans", generator: Optional[torch.Generator] = None,
               kmeans_init_iters: int = 10, kmeans_init_tol: float = 1e-4,
               param_dtype: Optional[torch.dtype] = None):
    """Initial (means, covariances, weights, source), fp32 on x's device
    (holding ``param_dtype`` values when one is given, ``round_params``).

    Explicit parameters get the reference's entry clamps
    (torch_fallback.py:1661-1682, :1731-1742, :1791-1802, :1851-1862).  Without
    ``init_means``, ``init_params="kmeans"`` runs k-means++ seeding, Lloyd
    refinement and the hard-label statistics on the device (``kmeans.py``; the
    reference's branch at :1701-1716, :1747-1762, :1807-1822, :1867-1882) --
    unless ``GMMXX_HIP_FLASH_KMEANS=0`` (see ``flash_kmeans_emulated``) -- and
    ``"random"`` takes random data rows plus the global variance (:1718-1727).
    """
    bsz, n, d = x.shape
    dev = x.device
    if init_means is not None:
        means = _f32(init_means, dev)
        if means.ndim != 3 or means.shape[0] != bsz or means.shape[2] != d:
            raise ValueError("init_means must have shape (B, K, D) matching x")
        k = means.shape[1]
        source = "user"
    else:
        if init_params not in {"kmeans", "random"}:
            raise ValueError("init_params must be 'kmeans' or 'random'")
        k = int(n_components)
        if init_params == "kmeans" and flash_kmeans_emulated():
            from . import kmeans
            means, covs, weights = kmeans.kmeans_initialize(
                x, covariance_type, k, max_iters=kmeans_init_iters, tol=kmeans_init_tol, reg_covar=reg_covar,
                generator=generator)
            return (*round_params(_engine_means(means, x), covs, weights, covariance_type, param_dtype),
                    "kmeans")
        idx = torch.randint(0, n, (bsz, k), device=dev, generator=generator)
        means = torch.gather(x, 1, idx[..., None].expand(-1, -1, d)).to(torch.float32).contiguous()
        source = "random"
        init_covs, init_weights = None, None
    if covariance_type == "spherical":
        covs = _f32(init_covs, dev) if init_covs is not None else global_spherical_variance(x, k, reg_covar)
        if tuple(covs.shape) != (bsz, k):
            raise ValueError("init_variances must have shape (B, K)")
        covs = covs.clamp_min(reg_covar)
    elif covariance_type == "diag":
        covs = _f32(init_covs, dev) if init_covs is not None else global_diag_variance(x, k, reg_covar)
        if tuple(covs.shape) != (bsz, k, d):
            raise ValueError("init_variances must have shape (B, K, D) for diag covariance")
        covs = covs.clamp_min(reg_covar)
    elif covariance_type == "tied":
        covs = _f32(init_covs, dev) if init_covs is not None else global_tied_covariance(x, reg_covar)
        if tuple(covs.shape) != (bsz, d, d):
            raise ValueError("init_variances must have shape (B, D, D) for tied covariance")
        covs = _sym(covs)
    else:
        covs = (_f32(init_covs, dev) if init_covs is not None
                else global_tied_covariance(x, reg_covar).unsqueeze(1).expand(-1, k, -1, -1))
        if tuple(covs.shape) != (bsz, k, d, d):
            raise ValueError("init_variances must have shape (B, K, D, D) for full covariance")
        covs = _sym(covs)
    weights = _init_weights(init_weights, bsz, k, dev)
    means, covs, weights = round_params(_engine_means(means, x).contiguous(), covs.contiguous(), weights,
                                        covariance_type, param_dtype)
    return means, covs, weights, source


def resolve_approx_top_k(approx_top_k: Optional[int], n_components: int) -> Optional[int]:
    """None for exact EM; ``approx_top_k >= K`` is exact EM too
    (gmmxx/torch_fallback.py:598-606)."""
    if approx_top_k is None:
        return None
    top_k = int(approx_top_k)
    if top_k <= 0:
        raise ValueError("approx_top_k must be positive or None")
    return None if top_k >= n_components else top_k


# The approximate E-step keeps the (B, rows, K) fp32 logits of one row chunk in
# its workspace; chunks are sized to hold at most this many logit bytes.
_TOPK_LOGIT_BYTES = 1 << 30


def topk_chunk_rows(bsz: int, n: int, k: int) -> int:
    rows = max(4096, _TOPK_LOGIT_BYTES // (4 * bsz * k)) // 32 * 32
    return min(n, rows)


class _TopkStep:
    """One approximate-EM iteration over row chunks: per chunk the top-k
    statistics (``gmmxx_hip_estep_stats_topk``), summed, then one M-step from
    the totals (``gmmxx_hip_finalize_stats``).  Follows the approximate
    branches of the reference's EM loops (gmmxx/torch_fallback.py:2097-2145,
    :2500-2526, :2911-2936), which likewise accumulate over row chunks."""

    def __init__(self, x, covariance_type, k, top_k, param_dtype=None):
        self.x, self.cov, self.k, self.top_k = x, covariance_type, k, top_k
        self.param_dtype = param_dtype
        bsz, n, d = x.shape
        self.n = n
        # top-1 (hard assignment) keeps no logits: one chunk
        self.rows = n if top_k == 1 else topk_chunk_rows(bsz, n, k)
        self.ws: Dict[int, _hip.Workspace] = {}
        self.fin_ws = _hip.Workspace(_hip.problem(covariance_type, x.dtype, bsz, 1, d, k), x.device)

    def chunks(self):
        for n0 in range(0, self.n, self.rows):
            xc = self.x[:, n0:min(n0 + self.rows, self.n), :]
            rows = int(xc.shape[1])
            ws = self.ws.get(rows)
            if ws is None:
                ws = _hip.Workspace(_hip.problem(self.cov, xc.dtype, xc.shape[0], rows, xc.shape[2], self.k),
                                    xc.device, top_k=self.top_k)
                self.ws[rows] = ws
            yield xc, ws

    def gram(self):
        total = None
        for xc, ws in self.chunks():
            g = _hip.gram(xc, ws)
            total = g if total is None else total + g
        return total

    def stats(self, means, covs, weights, reg_covar, min_weight):
        """(nk, sum_x, sum_q, ll_sum) of the top-k E-step, summed over the chunks."""
        tot = None
        for xc, ws in self.chunks():
            part = _hip.estep_stats_topk(self.cov, xc, means, covs, weights, self.top_k, reg_covar=reg_covar,
                                         min_weight=min_weight, ws=ws, param_dtype=self.param_dtype)
            tot = list(part) if tot is None else [a if a is None else a + b for a, b in zip(tot, part)]
        return tot

    def step(self, means, covs, weights, lb_out, gram, reg_covar, min_weight):
        nk, sum_x, sum_q, ll = self.stats(means, covs, weights, reg_covar, min_weight)
        _hip.finalize_stats(self.cov, nk, sum_x, sum_q, means, covs, weights, self.n, gram_xx=gram,
                            reg_covar=reg_covar, min_weight=min_weight, ws=self.fin_ws, x_dtype=self.x.dtype,
                            param_dtype=self.param_dtype)
        torch.div(ll, float(self.x.shape[0] * self.n), out=lb_out)


@torch.no_grad()
def fit(x: torch.Tensor, n_components: int, covariance_type: str, *, max_iters: int = 100,
        tol: float = 1e-4, init_means=None, init_covs=None, init_weights=None, verbose: bool = False,
        init_params: str = "kmeans", reg_covar: float = 1e-6, min_weight: float = 1e-8,
        compute_labels: bool = True, generator: Optional[torch.Generator] = None,
        approx_top_k: Optional[int] = None, kmeans_init_iters: int = 10, kmeans_init_tol: float = 1e-4,
        record_all_lower_bounds: bool = False, param_dtype: Optional[torch.dtype] = None,
        ) -> Tuple[Optional[torch.Tensor], torch.Tensor, torch.Tensor, torch.Tensor, Dict[str, object]]:
    """Soft EM on the HIP engine; see the module docstring.  ``approx_top_k``
    (1 <= k < K) restricts each row's responsibilities to its k largest logits,
    renormalised over them, as the reference's approximate EM does.

    ``lower_bound_history`` follows the reference's bookkeeping: for diag, tied
    and full with ``tol == 0`` and ``verbose=False`` only the last iteration's
    lower bound is recorded and the others are 0.0
    (gmmxx/torch_fallback.py:2484-2485, :2668-2679, :3169-3180); spherical
    records every iteration.  ``record_all_lower_bounds=True`` records every
    iteration for every type (the engine computes them all anyway).

    ``param_dtype`` (bfloat16 / float16, fp32 x) keeps the parameters in that
    dtype between iterations, as the reference keeps a half-precision x's
    (``round_params``; the library rounds them in its M-step)."""
    if covariance_type not in _COVS:
        raise ValueError("covariance_type must be 'spherical', 'diag', 'tied' or 'full'")
    if n_components <= 0:
        raise ValueError("n_components must be positive")
    if max_iters <= 0:
        raise ValueError("max_iters must be positive")
    if min_weight <= 0.0:
        raise ValueError("min_weight must be positive")
    _hip.require_hip()
    x = _as_device_input(x, covariance_type)
    bsz, n, d = x.shape
    if n == 0:
        raise ValueError("x must contain at least one sample")
    means, covs, weights, source = initialize(
        x, covariance_type, n_components, init_means=init_means, init_covs=init_covs,
        init_weights=init_weights, reg_covar=reg_covar, init_params=init_params, generator=generator,
        kmeans_init_iters=kmeans_init_iters, kmeans_init_tol=kmeans_init_tol, param_dtype=param_dtype)
    k = means.shape[1]
    if not _hip.supported(covariance_type, x.dtype, bsz, n, d, k):
        raise _hip.HipRuntimeError(
            f"shape not supported by the hip backend: {covariance_type} B={bsz} N={n} D={d} K={k} {x.dtype}")
    top_k = resolve_approx_top_k(approx_top_k, k)
    topk_step = None
    if top_k is None:
        prob = _hip.problem(covariance_type, x.dtype, bsz, n, d, k)
        ws = _hip.Workspace(prob, x.device)
        gram = _hip.gram(x, ws) if covariance_type == "tied" else None
    else:
        ws = None
        topk_step = _TopkStep(x, covariance_type, k, top_k, param_dtype)
        gram = topk_step.gram() if covariance_type == "tied" else None
    lb = torch.zeros((max_iters,), dtype=torch.float32, device=x.device)
    spherical = covariance_type == "spherical"
    sync_each = bool(verbose or tol > 0.0)
    prev = None
    n_iter = 0
    for it in range(max_iters):
        if topk_step is None:
            _hip.em_step(covariance_type, x, means, covs, weights, lb[it:it + 1], reg_covar=reg_covar,
                         min_weight=min_weight, gram_xx=gram, ws=ws, param_dtype=param_dtype)
        else:
            topk_step.step(means, covs, weights, lb[it:it + 1], gram, reg_covar, min_weight)
        n_iter = it + 1
        if not sync_each:
            continue
        value = float(lb[it].item())
        if verbose:
            print(f"Iter {it}, lower_bound: {value:.6f}")
        # Convergence rules: spherical torch_fallback.py:2322-2330, others :2695-2698.
        last = it + 1 == max_iters
        if spherical:
            if not last and prev is not None and abs(value - prev) < tol:
                break
            if not last:
                prev = value
        else:
            if tol > 0.0 and prev is not None and abs(value - prev) < tol:
                break
            if tol > 0.0:
                prev = value
    if ws is not None:
        # A cooperative pass that gave up waiting left its iteration's parameters
        # unchanged and a NaN lower bound; the fit reports it instead of returning.
        _hip.raise_on_status(_hip.take_status(ws), "EM fit")
    history = [float(v) for v in lb[:n_iter].tolist()]
    if not (spherical or tol > 0.0 or verbose or record_all_lower_bounds):
        history = [0.0] * (n_iter - 1) + history[-1:]
    labels = None
    if compute_labels:
        _, labels = _hip.score(covariance_type, x, means, covs, weights, want_scores=False, ws=ws)
    info: Dict[str, object] = {
        "n_iter": n_iter,
        "lower_bound": history[-1],
        "lower_bound_history": history,
        "init_source": source,
        "hip_enabled": True,
        "triton_estep_enabled": False,
        "triton_fused_update_enabled": False,
        "triton_streaming_update_enabled": False,
        "triton_labels_enabled": False,
        "approximate_em_enabled": top_k is not None,
        "approx_top_k": top_k,
        "backend_breakdown": {"hip": n_iter},
    }
    return labels, means, covs, weights, info


def _api(covariance_type):
    def run(x, n_components, max_iters=100, tol=1e-4, init_means=None, init_variances=None,
            init_weights=None, verbose=False, *, init_params="kmeans", reg_covar=1e-6,
            min_weight=1e-8, compute_labels=True, generator=None, approx_top_k=None, kmeans_init_iters=10,
            kmeans_init_tol=1e-4, record_all_lower_bounds=False, **unused):
        for key in unused:
            if key not in {"chunk_size_N", "chunk_size_K", "kmeans_use_triton", "gmm_use_triton",
                           "gmm_use_triton_estep", "gmm_use_triton_streaming_update"}:
                raise TypeError(f"unexpected keyword argument {key!r}")
        x_dev, home = _to_engine_device(x)
        labels, means, covs, weights, info = fit(
            x_dev, n_components, covariance_type, max_iters=max_iters, tol=tol, init_means=init_means,
            init_covs=init_variances, init_weights=init_weights, verbose=verbose,
            init_params=init_params, reg_covar=reg_covar, min_weight=min_weight,
            compute_labels=compute_labels, generator=generator, approx_top_k=approx_top_k,
            kmeans_init_iters=kmeans_init_iters, kmeans_init_tol=kmeans_init_tol,
            record_all_lower_bounds=record_all_lower_bounds)
        return (*_to_home((labels, means, covs, weights), home), info)
    run.__name__ = f"batch_gmm_{ {'diag': 'Diagonal'}.get(covariance_type, covariance_type.capitalize()) }_hip"
    run.__doc__ = (f"{covariance_type} soft EM on the HIP engine; signature and return value of "
                   f"the reference's batch_gmm_*_torch_native (chunk/Triton knobs are accepted and ignored). "
                   f"Host (CPU) input is copied to the current GPU and the results come back to the "
                   f"input's device, so a caller of the reference's CPU function gets CPU tensors.")
    return run


def _to_engine_device(x):
    """(x on a GPU, the device the caller's tensors live on).  The reference's
    ``*_torch_native`` functions run wherever x is, CPU included; here the work
    always runs on the GPU, so host input is copied to the current device once
    and the results are copied back (the estimator does the same)."""
    if not torch.is_tensor(x):
        raise TypeError("x must be a torch.Tensor")
    if x.is_cuda:
        return x, None
    if not torch.cuda.is_available():
        raise _hip.HipBackendUnavailable("the hip backend needs a GPU; none is visible")
    return x.to(torch.device("cuda", torch.cuda.current_device())), x.device


def _to_home(tensors, home):
    if home is None:
        return tuple(tensors)
    return tuple(None if t is None else t.to(home) for t in tensors)


batch_gmm_Spherical_hip = _api("spherical")
batch_gmm_Diagonal_hip = _api("diag")
batch_gmm_Tied_hip = _api("tied")
batch_gmm_Full_hip = _api("full")


# The reference's names for the same entry points (gmmxx/torch_fallback.py:3339-3520):
# the batch_gmm_* wrappers and their *_torch_native bodies both run the HIP engine here.
batch_gmm_Spherical = batch_gmm_Spherical_torch_native = batch_gmm_spherical = batch_gmm_Spherical_hip
batch_gmm_Diagonal = batch_gmm_Diagonal_torch_native = batch_gmm_diagonal = batch_gmm_diag = batch_gmm_Diagonal_hip
batch_gmm_Tied = batch_gmm_Tied_torch_native = batch_gmm_tied = batch_gmm_Tied_hip
batch_gmm_Full = batch_gmm_Full_torch_native = batch_gmm_full = batch_gmm_Full_hip


def _chunked(covariance_type, what):
    """<cov>_<assign|score_samples|predict_proba>_torch_native_chunked
    (gmmxx/torch_fallback.py:780-1345) on the HIP kernels.  Host input is copied
    to the current GPU and the result comes back to x's device; chunk sizes are
    accepted and ignored (the library tiles rows and components itself).
    Scores and responsibilities are returned in x's dtype and labels as int64,
    as the reference returns them.  One deliberate difference: bf16/fp16 x is
    computed in fp32 here (the reference's chunked functions compute in x's
    dtype, :780-821), so the values are the fp32 algorithm's rounded to x's
    dtype rather than the result of half-precision arithmetic."""
    def run(x, means, variances, weights, *, chunk_size_N=32768, chunk_size_K=1024):
        xd, home = _to_engine_device(x)
        dev = xd.device
        xd = xd if xd.dtype == torch.float32 else xd.to(torch.float32)
        args = (covariance_type, xd, *(t.to(dev) for t in (means, variances, weights)))
        if what == "assign":
            out = _hip.score(*args, want_scores=False, want_labels=True)[1]
        elif what == "score_samples":
            out = _hip.score(*args, want_scores=True, want_labels=False)[0].to(x.dtype)
        else:
            out = _hip.predict_proba(*args).to(x.dtype)
        return out if home is None else out.to(home)
    prefix = {"diag": "diagonal"}.get(covariance_type, covariance_type)
    run.__name__ = f"{prefix}_{what}_torch_native_chunked"
    run.__doc__ = _chunked.__doc__
    return run


spherical_assign_torch_native_chunked = _chunked("spherical", "assign")
spherical_score_samples_torch_native_chunked = _chunked("spherical", "score_samples")
spherical_predict_proba_torch_native_chunked = _chunked("spherical", "predict_proba")
diagonal_assign_torch_native_chunked = _chunked("diag", "assign")
diagonal_score_samples_torch_native_chunked = _chunked("diag", "score_samples")
diagonal_predict_proba_torch_native_chunked = _chunked("diag", "predict_proba")
tied_assign_torch_native_chunked = _chunked("tied", "assign")
tied_score_samples_torch_native_chunked = _chunked("tied", "score_samples")
tied_predict_proba_torch_native_chunked = _chunked("tied", "predict_proba")
full_assign_torch_native_chunked = _chunked("full", "assign")
full_score_samples_torch_native_chunked = _chunked("full", "score_samples")
full_predict_proba_torch_native_chunked = _chunked("full", "predict_proba")
