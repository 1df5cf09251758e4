"""Large-N host-to-HBM streaming: EM fit and inference with x in host memory.

Role of the reference's ``gmmxx/large_n.py`` for the ``"hip"`` backend: the
fit ``batch_gmm_largeN_cpu`` (:866-1595) and the streamed inference
``large_n_predict_cpu`` / ``large_n_score_samples_cpu`` /
``large_n_predict_proba_cpu`` (:1907-2502).  x stays in host memory (B = 1) and
passes through HBM in row chunks:

* a copy stream (default priority) moves chunk j+1 into one of two device
  buffers while the compute stream works on chunk j in the other; pinned host
  staging buffers (or x itself when it is already pinned and in the engine's
  dtype) make the copies asynchronous, and events order buffer reuse both ways;
* each EM iteration sums the chunks' sufficient statistics
  (``gmmxx_hip_estep_stats``, which applies the iteration prelude) and applies
  ONE M-step from the totals (``gmmxx_hip_finalize_stats``), so the result is
  the soft-EM iteration over all N rows, as in the reference's streaming loop
  (:1040-1555): lower bound = Σ log-normalisers / N every iteration, stop when
  it changes by less than ``tol``;
* initial parameters come from a random row sample, as
  ``_select_init_sample`` / ``_initialize_from_sample`` (:630-735): at most
  ``max_init_samples`` rows (at least 4096 or 64 per component), then the
  in-memory initialiser (random rows + global variance) on that sample.

The engine never sees more than ``chunk_size_N`` rows at once; with 288 GB of
HBM per MI355X this path is for data that does not fit on the device, or for
callers that keep x in host memory.
"""

from __future__ import annotations

from typing import Dict, Iterator, Optional, Tuple

import torch

from . import _hip, em

_COVS = ("spherical", "diag", "tied", "full")


def _engine_dtype(x_cpu: torch.Tensor, covariance_type: str, requested: Optional[torch.dtype] = None) -> torch.dtype:
    """bf16 (the bf16 engine) for spherical when requested, or by default for bf16
    input at the function level; fp32 otherwise.  The estimator passes its compute
    dtype, which is fp32 for half-precision input unless dtype= says otherwise."""
    if requested is not None:
        return torch.bfloat16 if (requested == torch.bfloat16 and covariance_type == "spherical") else torch.float32
    if x_cpu.dtype == torch.bfloat16 and covariance_type == "spherical":
        return torch.bfloat16
    return torch.float32


def _validate(x_cpu: torch.Tensor, device: torch.device) -> None:
    """gmmxx/large_n.py:468-478."""
    if not torch.is_tensor(x_cpu):
        raise TypeError("x must be a torch.Tensor")
    if x_cpu.ndim != 3:
        raise ValueError("x must have shape (B, N, D)")
    if x_cpu.shape[0] != 1:
        raise NotImplementedError("Large-N CPU streaming currently supports only B=1")
    if x_cpu.device.type != "cpu":
        raise ValueError("Large-N streaming expects a CPU input tensor")
    if device.type != "cuda":
        raise ValueError("Large-N streaming expects a GPU target device")
    if not x_cpu.dtype.is_floating_point:
        raise TypeError("GMM input must be a floating point tensor")
    if x_cpu.shape[1] == 0:
        raise ValueError("x must contain at least one sample")


class ChunkStream:
    """Row chunks of a host tensor (1, N, D) delivered in HBM, double-buffered.

    Iterating yields ``(start, end, x_chunk)`` with ``x_chunk`` a (1, rows, D)
    device view in the engine dtype that is valid on the current stream until
    the next item is requested.
    """

    def __init__(self, x_cpu: torch.Tensor, device: torch.device, dtype: torch.dtype, chunk_rows: int):
        self.x = x_cpu
        self.n, self.d = int(x_cpu.shape[1]), int(x_cpu.shape[2])
        self.rows = max(1, min(int(chunk_rows), self.n))
        self.device = device
        self.direct = bool(x_cpu.is_pinned() and x_cpu.dtype == dtype and x_cpu.is_contiguous())
        self.host = [] if self.direct else [
            torch.empty((1, self.rows, self.d), dtype=dtype, pin_memory=True) for _ in range(2)]
        self.dev = [torch.empty((1, self.rows, self.d), dtype=dtype, device=device) for _ in range(2)]
        self.copy_stream = torch.cuda.Stream(device=device)
        self.copied = [torch.cuda.Event() for _ in range(2)]
        self.consumed = [torch.cuda.Event() for _ in range(2)]
        self.used = [False, False]

    def _issue(self, slot: int, start: int) -> Tuple[int, int]:
        end = min(start + self.rows, self.n)
        rows = end - start
        if self.direct:
            src = self.x[:, start:end]
        else:
            # The pinned buffer may still feed this slot's previous copy.
            if self.used[slot]:
                self.copied[slot].synchronize()
            src = self.host[slot][:, :rows]
            src.copy_(self.x[:, start:end])
        with torch.cuda.stream(self.copy_stream):
            if self.used[slot]:
                self.copy_stream.wait_event(self.consumed[slot])
            self.dev[slot][:, :rows].copy_(src, non_blocking=True)
            self.copied[slot].record(self.copy_stream)
        self.used[slot] = True
        return start, end

    def __iter__(self) -> Iterator[Tuple[int, int, torch.Tensor]]:
        compute = torch.cuda.current_stream(self.device)
        pending = self._issue(0, 0)
        slot = 0
        while pending is not None:
            start, end = pending
            compute.wait_event(self.copied[slot])
            nxt = end if end < self.n else None
            # Next chunk's copy goes out before this chunk's kernels are enqueued.
            pending = self._issue(1 - slot, nxt) if nxt is not None else None
            yield start, end, self.dev[slot][:, :end - start]
            self.consumed[slot].record(compute)
            slot = 1 - slot


def _sample_init(x_cpu, n_components, covariance_type, device, dtype, *, init_params, reg_covar,
                 max_init_samples, seed, kmeans_init_iters=10, kmeans_init_tol=1e-4):
    """Random-row sample of at most max_init_samples rows (gmmxx/large_n.py:630-646),
    then the in-memory initialiser on it (:649-735)."""
    n = int(x_cpu.shape[1])
    target = max(4096, n_components * 64, n_components)
    sample_n = min(n, max(n_components, min(int(max_init_samples), target)))
    if sample_n == n:
        sample_cpu = x_cpu
    else:
        g = torch.Generator().manual_seed(int(seed))
        idx = torch.randint(0, n, (sample_n,), generator=g)
        sample_cpu = x_cpu.index_select(1, idx)
    sample = sample_cpu.to(device=device, dtype=dtype).contiguous()
    dg = torch.Generator(device=device).manual_seed(int(seed))
    means, covs, weights, source = em.initialize(sample, covariance_type, n_components, reg_covar=reg_covar,
                                                 init_params=init_params, generator=dg,
                                                 kmeans_init_iters=kmeans_init_iters,
                                                 kmeans_init_tol=kmeans_init_tol)
    if sample_n < n:
        source = f"{source}_sampled"
    return means, covs, weights, source, sample_n


class _Workspaces:
    """One workspace per chunk shape (the full chunk and the last, shorter one)."""

    def __init__(self, covariance_type, dtype, d, k, device, top_k=None):
        self.cov, self.dtype, self.d, self.k, self.device = covariance_type, dtype, d, k, device
        self.top_k = top_k
        self.cache: Dict[int, _hip.Workspace] = {}

    def get(self, rows: int) -> _hip.Workspace:
        ws = self.cache.get(rows)
        if ws is None:
            if not _hip.supported(self.cov, self.dtype, 1, rows, self.d, self.k):
                raise _hip.HipRuntimeError(
                    f"shape not supported by the hip backend: {self.cov} N={rows} D={self.d} K={self.k}")
            ws = _hip.Workspace(_hip.problem(self.cov, self.dtype, 1, rows, self.d, self.k), self.device,
                                top_k=self.top_k)
            self.cache[rows] = ws
        return ws


@torch.no_grad()
def fit_large_n(x_cpu: torch.Tensor, n_components: int, covariance_type: str, *,
                device: Optional[torch.device] = None, max_iters: int = 100, tol: float = 1e-4,
                verbose: bool = False, init_params: str = "kmeans", reg_covar: float = 1e-6,
                chunk_size_N: int = 1 << 20, min_weight: float = 1e-8, compute_labels: bool = True,
                max_init_samples: int = 65536, init_means=None, init_covs=None, init_weights=None,
                seed: int = 0, approx_top_k: Optional[int] = None, kmeans_init_iters: int = 10,
                kmeans_init_tol: float = 1e-4, compute_dtype: Optional[torch.dtype] = None,
                param_dtype: Optional[torch.dtype] = None):
    """Soft EM with x (1, N, D) in host memory; returns (labels, means, covariances,
    weights, info) like gmmxx/large_n.py:866-1595 (labels on the host).
    ``approx_top_k`` selects the approximate top-k E-step per chunk, as the
    reference's streamed loop does (gmmxx/large_n.py:1325-1370).  ``compute_dtype``
    (fp32, or bf16 for the spherical bf16 engine) defaults to bf16 for bf16
    spherical input and fp32 otherwise; ``param_dtype`` as in ``em.fit``."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if covariance_type not in _COVS:
        raise ValueError("covariance_type must be 'spherical', 'diag', 'tied', or 'full'")
    if n_components <= 0:
        raise ValueError("n_components must be positive")
    if max_iters <= 0:
        raise ValueError("max_iters must be positive")
    if chunk_size_N <= 0:
        raise ValueError("chunk_size_N must be positive")
    if min_weight <= 0.0:
        raise ValueError("min_weight must be positive")
    _validate(x_cpu, device)
    _hip.require_hip()
    dtype = _engine_dtype(x_cpu, covariance_type, compute_dtype)
    n, d = int(x_cpu.shape[1]), int(x_cpu.shape[2])
    if init_means is not None:
        sample = x_cpu[:, : min(n, max(4096, int(max_init_samples)))].to(device=device, dtype=dtype)
        means, covs, weights, source = em.initialize(sample, covariance_type, n_components,
                                                     init_means=init_means, init_covs=init_covs,
                                                     init_weights=init_weights, reg_covar=reg_covar,
                                                     param_dtype=param_dtype)
        sample_n = int(sample.shape[1])
    else:
        means, covs, weights, source, sample_n = _sample_init(
            x_cpu, n_components, covariance_type, device, dtype, init_params=init_params,
            reg_covar=reg_covar, max_init_samples=max_init_samples, seed=seed,
            kmeans_init_iters=kmeans_init_iters, kmeans_init_tol=kmeans_init_tol)
    means, covs, weights = em.round_params(means, covs, weights, covariance_type, param_dtype)
    k = int(means.shape[1])
    top_k = em.resolve_approx_top_k(approx_top_k, k)
    stream = ChunkStream(x_cpu, device, dtype, chunk_size_N)
    wss = _Workspaces(covariance_type, dtype, d, k, device)
    # the top-k E-step holds a chunk's logits: sub-chunks bound that buffer
    sub_rows = (min(n, chunk_size_N) if top_k == 1 else em.topk_chunk_rows(1, min(n, chunk_size_N), k)) \
        if top_k is not None else 0
    topk_wss = _Workspaces(covariance_type, dtype, d, k, device, top_k=top_k) if top_k is not None else None
    fin_ws = _hip.Workspace(_hip.problem(covariance_type, dtype, 1, 1, d, k), device)

    gram = None
    if covariance_type == "tied":   # XᵀX once per fit, summed over the chunks
        gram = torch.zeros((1, d, d), dtype=torch.float32, device=device)
        for _, end_, xc in stream:
            gram += _hip.gram(xc, wss.get(int(xc.shape[1])))

    q_shape = {"spherical": (1, k), "diag": (1, k, d), "full": (1, k, d, d)}.get(covariance_type)
    history = []
    prev = None
    n_iter = 0
    for it in range(max_iters):
        nk = torch.zeros((1, k), dtype=torch.float32, device=device)
        sx = torch.zeros((1, k, d), dtype=torch.float32, device=device)
        sq = torch.zeros(q_shape, dtype=torch.float32, device=device) if q_shape else None
        ll = torch.zeros((), dtype=torch.float64, device=device)
        for _, _, xc in stream:
            parts = ((xc,) if top_k is None else
                     tuple(xc[:, r0:r0 + sub_rows] for r0 in range(0, int(xc.shape[1]), sub_rows)))
            for xp in parts:
                rows = int(xp.shape[1])
                if top_k is None:
                    c_nk, c_sx, c_sq, c_ll = _hip.estep_stats(covariance_type, xp, means, covs, weights,
                                                              reg_covar=reg_covar, min_weight=min_weight,
                                                              ws=wss.get(rows), param_dtype=param_dtype)
                else:
                    c_nk, c_sx, c_sq, c_ll = _hip.estep_stats_topk(covariance_type, xp, means, covs, weights,
                                                                   top_k, reg_covar=reg_covar,
                                                                   min_weight=min_weight, ws=topk_wss.get(rows),
                                                                   param_dtype=param_dtype)
                nk += c_nk
                sx += c_sx
                if sq is not None:
                    sq += c_sq
                ll += c_ll[0].double()
        if top_k is None:   # a timed-out cooperative chunk pass: raise before its statistics are used
            for ws in wss.cache.values():
                _hip.raise_on_status(_hip.take_status(ws), "streamed EM fit")
        _hip.finalize_stats(covariance_type, nk, sx, sq, means, covs, weights, n, gram_xx=gram,
                            reg_covar=reg_covar, min_weight=min_weight, ws=fin_ws, x_dtype=dtype,
                            param_dtype=param_dtype)
        value = float(ll.item()) / float(n)
        history.append(value)
        n_iter = it + 1
        if verbose:
            print(f"Iter {it}, lower_bound: {value:.6f}")
        if prev is not None and abs(value - prev) < tol:
            break
        prev = value

    labels = predict_large_n(x_cpu, means, covs, weights, covariance_type, device=device,
                             chunk_size_N=chunk_size_N) if compute_labels else None
    info: Dict[str, object] = {
        "n_iter": n_iter,
        "lower_bound": history[-1],
        "lower_bound_history": history,
        "init_source": source,
        "init_sample_size": sample_n,
        "large_n_streaming_enabled": True,
        "copy_stream_prefetch_enabled": True,
        "hip_enabled": True,
        "triton_estep_enabled": False,
        "triton_fused_update_enabled": False,
        "triton_approx_topk_enabled": False,
        "triton_streaming_update_enabled": False,
        "triton_labels_enabled": False,
        "approximate_em_enabled": top_k is not None,
        "approx_top_k": top_k,
        "fallback_reason": None,
        "backend_breakdown": {"hip": n_iter},
    }
    return labels, means, covs, weights, info


def _params(means, covs, weights, device):
    return tuple(t.detach().to(device=device, dtype=torch.float32).contiguous() for t in (means, covs, weights))


def _infer(x_cpu, means, covs, weights, covariance_type, device, chunk_size_N, what, compute_dtype=None):
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    _validate(x_cpu, device)
    _hip.require_hip()
    dtype = _engine_dtype(x_cpu, covariance_type, compute_dtype)
    means, covs, weights = _params(means, covs, weights, device)
    n, d, k = int(x_cpu.shape[1]), int(x_cpu.shape[2]), int(means.shape[1])
    stream = ChunkStream(x_cpu, device, dtype, chunk_size_N)
    wss = _Workspaces(covariance_type, dtype, d, k, device)
    shape = {"labels": (1, n), "scores": (1, n), "proba": (1, n, k)}[what]
    out = torch.empty(shape, dtype=torch.int64 if what == "labels" else torch.float32)
    for start, end, xc in stream:
        ws = wss.get(end - start)
        if what == "labels":
            _, res = _hip.score(covariance_type, xc, means, covs, weights, want_scores=False, ws=ws)
        elif what == "scores":
            res, _ = _hip.score(covariance_type, xc, means, covs, weights, want_labels=False, ws=ws)
        else:
            res = _hip.predict_proba(covariance_type, xc, means, covs, weights, ws=ws)
        out[:, start:end].copy_(res)   # to pageable host memory: waits for this chunk
    return out


def predict_large_n(x_cpu, means, covs, weights, covariance_type, *, device=None, chunk_size_N=1 << 20,
                    compute_dtype=None):
    """First-max labels (1, N) int64 on the host (gmmxx/large_n.py:1907-2076)."""
    return _infer(x_cpu, means, covs, weights, covariance_type, device, chunk_size_N, "labels", compute_dtype)


def score_samples_large_n(x_cpu, means, covs, weights, covariance_type, *, device=None, chunk_size_N=1 << 20,
                          compute_dtype=None):
    """Per-sample log-likelihood (1, N) fp32 on the host (gmmxx/large_n.py:2078-2257)."""
    return _infer(x_cpu, means, covs, weights, covariance_type, device, chunk_size_N, "scores", compute_dtype)


def predict_proba_large_n(x_cpu, means, covs, weights, covariance_type, *, device=None, chunk_size_N=1 << 20,
                          compute_dtype=None):
    """Responsibilities (1, N, K) fp32 on the host (gmmxx/large_n.py:2259-2502)."""
    return _infer(x_cpu, means, covs, weights, covariance_type, device, chunk_size_N, "proba", compute_dtype)


# ---------------------------------------------------------------------------
# The reference module's function names (gmmxx/large_n.py:866, :1907, :2078,
# :2259) over the functions above.  ``dtype`` is the compute dtype request
# (bf16 selects the spherical bf16 engine, anything else fp32; float64 raises);
# the Triton/backend knobs and chunk_size_K are accepted and ignored: every
# chunk runs on the HIP kernels.  ``chunk_size_N`` is the streamed chunk.
# ---------------------------------------------------------------------------

_IGNORED = {"chunk_size_K", "kmeans_use_triton", "gmm_use_triton", "use_triton", "backend", "legacy_no_triton"}


def _reject_unknown(kw):
    for key in kw:
        if key not in _IGNORED:
            raise TypeError(f"unexpected keyword argument {key!r}")


def batch_gmm_largeN_cpu(x_cpu, n_components, *, covariance_type, device, dtype, max_iters=100, tol=1e-4,
                         verbose=False, init_params="kmeans", reg_covar=1e-6, chunk_size_N=1 << 20,
                         kmeans_init_iters=10, kmeans_init_tol=1e-4, min_weight=1e-8, compute_labels=True,
                         max_init_samples=65536, approx_top_k=None, seed=0, **ignored):
    """fit_large_n under the reference's name and keyword set (gmmxx/large_n.py:866-890)."""
    _reject_unknown(ignored)
    return fit_large_n(x_cpu, n_components, covariance_type, device=device, max_iters=max_iters, tol=tol,
                       verbose=verbose, init_params=init_params, reg_covar=reg_covar, chunk_size_N=chunk_size_N,
                       min_weight=min_weight, compute_labels=compute_labels, max_init_samples=max_init_samples,
                       seed=seed, approx_top_k=approx_top_k, kmeans_init_iters=kmeans_init_iters,
                       kmeans_init_tol=kmeans_init_tol, compute_dtype=dtype)


def _ref_infer(fn, x_cpu, means, variances, weights, covariance_type, device, dtype, chunk_size_N,
               return_triton_used, return_backend_used, ignored):
    _reject_unknown(ignored)
    out = fn(x_cpu, means, variances, weights, covariance_type, device=device, chunk_size_N=chunk_size_N,
             compute_dtype=dtype)
    if return_backend_used:
        return out, "hip"
    if return_triton_used:
        return out, False
    return out


def large_n_predict_cpu(x_cpu, means, variances, weights, *, covariance_type, device, dtype, chunk_size_N=1 << 20,
                        return_triton_used=False, return_backend_used=False, **ignored):
    """predict_large_n under the reference's name (gmmxx/large_n.py:1907-1923)."""
    return _ref_infer(predict_large_n, x_cpu, means, variances, weights, covariance_type, device, dtype,
                      chunk_size_N, return_triton_used, return_backend_used, ignored)


def large_n_score_samples_cpu(x_cpu, means, variances, weights, *, covariance_type, device, dtype,
                              chunk_size_N=1 << 20, return_triton_used=False, return_backend_used=False, **ignored):
    """score_samples_large_n under the reference's name (gmmxx/large_n.py:2078)."""
    return _ref_infer(score_samples_large_n, x_cpu, means, variances, weights, covariance_type, device, dtype,
                      chunk_size_N, return_triton_used, return_backend_used, ignored)


def large_n_predict_proba_cpu(x_cpu, means, variances, weights, *, covariance_type, device, dtype,
                              chunk_size_N=1 << 20, return_triton_used=False, return_backend_used=False, **ignored):
    """predict_proba_large_n under the reference's name (gmmxx/large_n.py:2259)."""
    return _ref_infer(predict_proba_large_n, x_cpu, means, variances, weights, covariance_type, device, dtype,
                      chunk_size_N, return_triton_used, return_backend_used, ignored)
