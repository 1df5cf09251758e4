"""Host-side checks that need no GPU: the C-ABI library loads and exports every
entry point the header declares, the planner's gates and error reporting, the
backend truth table, and the estimator surface (parameter handling and the
model-selection formulas, the latter against scikit-learn).

No kernel is launched here: the only library calls are host-side queries and
argument validation that returns before any device work.
"""

import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

from gmmxx_amd import _dispatch, _hip
from gmmxx_amd.interface import GMMXX

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gmmxx_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gmmxx_hip_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    try:
        return _hip.load_library()
    except _hip.HipBackendUnavailable as exc:
        pytest.fail(f"libgmmxx_hip.so must be built before the tests (python -m gmmxx_amd.build): {exc}")


def test_header_declares_entry_points():
    syms = _declared_symbols()
    assert "gmmxx_hip_em_step" in syms and "gmmxx_hip_abi_version" in syms
    assert len(syms) >= 10


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in _declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"declared in include/gmmxx_hip.h but not exported: {missing}"
    assert set(_hip.exported_symbols()) == set(_declared_symbols())


def test_abi_version(lib):
    assert lib.gmmxx_hip_abi_version() == _hip.ABI_VERSION


def _prob(cov, dtype, b, n, d, k):
    return _hip.problem(cov, dtype, b, n, d, k)


@pytest.mark.parametrize("cov,dtype,d,ok", [
    ("spherical", torch.float32, 128, True),
    ("spherical", torch.bfloat16, 128, True),
    ("spherical", torch.float32, 129, False),
    ("diag", torch.float32, 64, True),
    ("diag", torch.float32, 128, True),
    ("diag", torch.bfloat16, 64, False),
    ("tied", torch.float32, 64, True),
    ("tied", torch.float32, 65, True),
    ("tied", torch.float32, 128, True),
    ("tied", torch.float32, 129, False),
    ("full", torch.float32, 16, True),
    ("full", torch.float32, 17, True),
    ("full", torch.float32, 128, True),
    ("full", torch.float32, 129, False),
])
def test_supported_gate(lib, cov, dtype, d, ok):
    assert _hip.supported(cov, dtype, 2, 1000, d, 37) == ok
    nbytes = lib.gmmxx_hip_workspace_bytes(ctypes.byref(_prob(cov, dtype, 2, 1000, d, 37)))
    if ok:
        assert nbytes > 0 and nbytes % 256 == 0
    else:
        assert nbytes == -1
        assert _hip.last_error()


@pytest.mark.parametrize("b,n,d,k", [(0, 10, 4, 2), (1, 0, 4, 2), (1, 10, 0, 2), (1, 10, 4, 0),
                                     (1, 10, 4, 65537), (65536, 10, 4, 2)])
def test_planner_rejects_bad_shapes(b, n, d, k):
    assert not _hip.supported("spherical", torch.float32, b, n, d, k)


def test_workspace_grows_with_n(lib):
    small = lib.gmmxx_hip_workspace_bytes(ctypes.byref(_prob("diag", torch.float32, 1, 10_000, 64, 512)))
    large = lib.gmmxx_hip_workspace_bytes(ctypes.byref(_prob("diag", torch.float32, 1, 1_000_000, 64, 512)))
    assert 0 < small < large


def test_entry_points_validate_before_device_work(lib):
    """Argument errors come back as status codes with a message, no exception
    crosses the ABI and nothing is launched."""
    p = _prob("spherical", torch.float32, 1, 100, 8, 4)
    need = lib.gmmxx_hip_workspace_bytes(ctypes.byref(p))
    dummy = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    rc = lib.gmmxx_hip_em_step(None, dummy, dummy, dummy, dummy, None, 1e-6, 1e-8, dummy, dummy, need, None)
    assert rc == 1 and "NULL" in _hip.last_error()
    rc = lib.gmmxx_hip_em_step(ctypes.byref(p), None, dummy, dummy, dummy, None, 1e-6, 1e-8, dummy, dummy,
                               need, None)
    assert rc == 1 and "x is NULL" in _hip.last_error()
    rc = lib.gmmxx_hip_em_step(ctypes.byref(p), dummy, dummy, dummy, dummy, None, 1e-6, 1e-8, dummy, None,
                               need, None)
    assert rc == 3 and "workspace" in _hip.last_error()
    rc = lib.gmmxx_hip_em_step(ctypes.byref(p), dummy, dummy, dummy, dummy, None, 1e-6, 1e-8, dummy, dummy,
                               need - 256, None)
    assert rc == 3 and "too small" in _hip.last_error()
    rc = lib.gmmxx_hip_em_step(ctypes.byref(p), dummy, dummy, dummy, dummy, None, 1e-6, 1e-8, dummy,
                               ctypes.c_void_p(512 + 64), need, None)
    assert rc == 3 and "aligned" in _hip.last_error()
    bad = _hip._Problem(7, 0, 1, 100, 8, 4)
    assert lib.gmmxx_hip_em_step(ctypes.byref(bad), dummy, dummy, dummy, dummy, None, 1e-6, 1e-8, dummy,
                                 dummy, need, None) == 1
    tied = _prob("tied", torch.float32, 1, 100, 8, 4)
    need_t = lib.gmmxx_hip_workspace_bytes(ctypes.byref(tied))
    rc = lib.gmmxx_hip_em_step(ctypes.byref(tied), dummy, dummy, dummy, dummy, None, 1e-6, 1e-8, dummy, dummy,
                               need_t, None)
    assert rc == 1 and "XᵀX" in _hip.last_error()
    assert lib.gmmxx_hip_canary(dummy, dummy, -1, 0, None) == 1
    assert lib.gmmxx_hip_canary(None, None, 0, 0, None) == 0


def test_param_dtype_validation(lib):
    """gmmxx_problem.param_dtype: GMMXX_F32 / BF16 / F16, not F16 with bf16 x;
    reserved must be 0 (a rejected descriptor plans no workspace)."""
    ok = _hip.problem("diag", torch.float32, 1, 100, 8, 4, torch.float16)
    assert lib.gmmxx_hip_workspace_bytes(ctypes.byref(ok)) > 0
    bad = _hip._Problem(1, 0, 1, 100, 8, 4, 3, 0)
    assert lib.gmmxx_hip_workspace_bytes(ctypes.byref(bad)) == -1
    bad = _hip._Problem(1, 0, 1, 100, 8, 4, 0, 1)
    assert lib.gmmxx_hip_workspace_bytes(ctypes.byref(bad)) == -1
    bad = _hip._Problem(0, 1, 1, 100, 128, 4, 2, 0)
    assert lib.gmmxx_hip_workspace_bytes(ctypes.byref(bad)) == -1
    with pytest.raises(ValueError):
        _hip.problem("diag", torch.float32, 1, 100, 8, 4, torch.float64)


def test_problem_rejects_unknown_dtype():
    with pytest.raises(ValueError):
        _hip.problem("spherical", torch.float16, 1, 10, 4, 2)
    with pytest.raises(ValueError):
        _hip.problem("banana", torch.float32, 1, 10, 4, 2)


# ---------------------------------------------------------------------------
# Backend resolution (gmmxx/_dispatch.py:88-162 truth table, hip edition)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("requested", ["torch", "cuda", "triton"])
def test_resolve_rejects_backends_not_provided(requested):
    with pytest.raises(ValueError, match="reference gmmxx package"):
        _dispatch.resolve_backend(requested, "spherical", (1, 100, 8, 4), torch.float32)


def test_resolve_rejects_unknown_backend():
    with pytest.raises(ValueError, match="unknown backend"):
        _dispatch.resolve_backend("metal", "spherical", (1, 100, 8, 4), torch.float32)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
@pytest.mark.parametrize("requested", ["auto", "hip"])
def test_resolve_without_gpu_raises(requested):
    with pytest.raises(_hip.HipBackendUnavailable):
        _dispatch.resolve_backend(requested, "spherical", (1, 100, 8, 4), torch.float32)


def test_env_override_only_applies_to_auto(monkeypatch):
    monkeypatch.setenv("GMMXX_BACKEND", "torch")
    with pytest.raises(ValueError, match="reference gmmxx package"):
        _dispatch.resolve_backend_with_env("auto", "spherical", (1, 100, 8, 4), torch.float32)
    monkeypatch.setenv("GMMXX_BACKEND", "not-a-backend")
    if not torch.cuda.is_available():
        with pytest.raises(_hip.HipBackendUnavailable):
            _dispatch.resolve_backend_with_env("auto", "spherical", (1, 100, 8, 4), torch.float32)


def test_engine_dtype_policy():
    assert _dispatch.engine_dtype("spherical", torch.bfloat16) == torch.bfloat16
    assert _dispatch.engine_dtype("diag", torch.bfloat16) == torch.float32
    assert _dispatch.engine_dtype("full", torch.float16) == torch.float32


def test_shape_gate_uses_library():
    assert _dispatch.hip_supported("spherical", (1, 100, 128, 1024), torch.bfloat16)
    assert _dispatch.hip_supported("full", (1, 100, 32, 4), torch.float32)
    assert not _dispatch.hip_supported("full", (1, 100, 129, 4), torch.float32)
    assert _dispatch.hip_supported("tied", (1, 100, 64), torch.float32)  # K unknown at inference


# ---------------------------------------------------------------------------
# Estimator surface (gmmxx/interface.py:141-270, :1508-1603, :2537-2558)
# ---------------------------------------------------------------------------

def test_constructor_validation():
    with pytest.raises(ValueError, match="k or n_components"):
        GMMXX()
    with pytest.raises(ValueError, match="conflicting"):
        GMMXX(k=3, n_components=4)
    with pytest.raises(ValueError, match="backend"):
        GMMXX(k=3, backend="metal")
    with pytest.raises(ValueError):
        GMMXX(k=3, covariance_type="banana")
    with pytest.raises(ValueError):
        GMMXX(k=3, tol=-1.0)
    with pytest.raises(ValueError):
        GMMXX(k=0)
    with pytest.raises(ValueError):
        GMMXX(k=3, matmul_precision="low")
    with pytest.raises(ValueError, match="both backend"):
        GMMXX(k=3, backend="hip", use_triton=True)
    with pytest.warns(DeprecationWarning):
        GMMXX(k=3, use_triton=False)
    est = GMMXX(n_components=5, max_iter=7, random_state=3, n_features=4, covariance_type="diagonal")
    assert (est.k, est.niter, est.seed, est.d, est.covariance_type) == (5, 7, 3, 4, "diag")
    assert est.niter == 7 and GMMXX(k=2).niter == 100


def test_get_set_params_round_trip():
    est = GMMXX(k=4, covariance_type="tied", backend="hip", reg_covar=1e-5)
    params = est.get_params()
    clone = GMMXX(k=1).set_params(**{k: v for k, v in params.items() if k != "device"})
    assert clone.get_params() == {**params, "device": clone.device}
    with pytest.raises(ValueError, match="Invalid parameter"):
        est.set_params(bogus=1)
    est.set_params(n_components=9, covariance_type="diagonal")
    assert est.k == 9 and est.covariance_type == "diag"
    with pytest.raises(ValueError):
        est.set_params(use_triton=True)  # backend is explicit


def test_unfitted_inference_raises():
    est = GMMXX(k=2)
    with pytest.raises(RuntimeError, match="not trained"):
        est.predict(torch.zeros(4, 2))


def test_input_normalisation():
    est = GMMXX(k=2)
    with pytest.raises(TypeError):
        est.fit(np.zeros((4, 2)))
    with pytest.raises(TypeError):
        est.fit(torch.zeros(4, 2, dtype=torch.int64))
    with pytest.raises(ValueError, match="at least one sample"):
        est.fit(torch.zeros(0, 2))
    with pytest.raises(ValueError, match="shape"):
        est.fit(torch.zeros(2, 2, 2, 2))
    est = GMMXX(k=2, d=3)
    with pytest.raises(ValueError, match="Expected d=3"):
        est.fit(torch.zeros(4, 2))


def test_fit_on_cpu_device_refuses():
    est = GMMXX(k=2, device="cpu")
    with pytest.raises(_hip.HipBackendUnavailable):
        est.fit(torch.randn(16, 3))


def test_approx_top_k_resolution():
    """gmmxx/torch_fallback.py:598-606: None and k >= K are exact EM."""
    from gmmxx_amd import em
    assert em.resolve_approx_top_k(None, 4) is None
    assert em.resolve_approx_top_k(4, 4) is None and em.resolve_approx_top_k(9, 4) is None
    assert em.resolve_approx_top_k(3, 4) == 3
    with pytest.raises(ValueError):
        em.resolve_approx_top_k(0, 4)
    assert em.topk_chunk_rows(1, 100, 8) == 100
    rows = em.topk_chunk_rows(2, 10 ** 9, 1024)
    assert rows % 32 == 0 and 2 * rows * 1024 * 4 <= 1 << 30
    with pytest.raises(ValueError):
        GMMXX(k=2, approx_top_k=0)


def _fitted(cov, b, k, d, rng):
    est = GMMXX(k=k, covariance_type=cov)
    est.means_b = torch.tensor(rng.normal(size=(b, k, d)), dtype=torch.float32)
    w = rng.random((b, k)) + 0.1
    est.weights_b = torch.tensor(w / w.sum(-1, keepdims=True), dtype=torch.float32)
    if cov == "spherical":
        cv = rng.random((b, k)) + 0.5
    elif cov == "diag":
        cv = rng.random((b, k, d)) + 0.5
    else:
        a = rng.normal(size=(b, k, d, d))
        cv = a @ np.swapaxes(a, -1, -2) / d + np.eye(d)
        if cov == "tied":
            cv = cv[:, 0]
    est.variances_b = est.covariances_b = torch.tensor(cv, dtype=torch.float32)
    est._batch_size = None if b == 1 else b
    return est


@pytest.mark.parametrize("cov", ["spherical", "diag", "tied", "full"])
def test_bic_aic_match_sklearn(cov, monkeypatch):
    """bic/aic and the free-parameter count against scikit-learn's
    GaussianMixture on the same parameters; score_samples comes from the CPU
    oracle here (the GPU path is covered by the GPU tests)."""
    from sklearn.mixture import GaussianMixture

    from oracle import torch_ref

    rng = np.random.default_rng(5)
    k, d, n = 3, 4, 200
    est = _fitted(cov, 1, k, d, rng)
    x = torch.tensor(rng.normal(size=(n, d)), dtype=torch.float32)
    monkeypatch.setattr(est, "score_samples", lambda data: torch_ref.score_samples(
        data.unsqueeze(0), est.means_b, est.covariances_b, est.weights_b, cov).squeeze(0))
    gm = GaussianMixture(n_components=k, covariance_type=cov)
    gm.weights_ = est.weights_b[0].double().numpy()
    gm.means_ = est.means_b[0].double().numpy()
    cv = est.covariances_b[0].double().numpy()
    gm.covariances_ = cv
    if cov in ("spherical", "diag"):
        gm.precisions_cholesky_ = 1.0 / np.sqrt(cv)
    elif cov == "tied":
        gm.precisions_cholesky_ = np.linalg.inv(np.linalg.cholesky(cv)).T
    else:
        gm.precisions_cholesky_ = np.stack([np.linalg.inv(np.linalg.cholesky(c)).T for c in cv])
    assert est._n_parameters() == gm._n_parameters()
    xd = x.double().numpy()
    assert math.isclose(est.bic(x), gm.bic(xd), rel_tol=1e-5)
    assert math.isclose(est.aic(x), gm.aic(xd), rel_tol=1e-5)


def test_n_parameters_batched():
    rng = np.random.default_rng(0)
    est = _fitted("diag", 3, 4, 5, rng)
    assert est._n_parameters(3) == 3 * (4 * 5 + 4 * 5 + 3)


# --- large-N streaming: input validation (gmmxx/large_n.py:468-478), no GPU needed ---

def test_large_n_rejects_bad_input():
    from gmmxx_amd import large_n
    dev = torch.device("cuda")
    with pytest.raises(NotImplementedError):
        large_n.fit_large_n(torch.zeros((2, 10, 3)), 2, "spherical", device=dev)
    with pytest.raises(ValueError):
        large_n.fit_large_n(torch.zeros((10, 3)), 2, "spherical", device=dev)
    with pytest.raises(ValueError):
        large_n.fit_large_n(torch.zeros((1, 10, 3)), 2, "spherical", device=torch.device("cpu"))
    with pytest.raises(TypeError):
        large_n.fit_large_n(torch.zeros((1, 10, 3), dtype=torch.int32), 2, "spherical", device=dev)
    with pytest.raises(ValueError):
        large_n.fit_large_n(torch.zeros((1, 10, 3)), 2, "bogus", device=dev)
    with pytest.raises(ValueError):
        large_n.fit_large_n(torch.zeros((1, 10, 3)), 2, "diag", device=dev, chunk_size_N=0)


def test_large_n_engine_dtype():
    from gmmxx_amd import large_n
    x = torch.zeros((1, 4, 3), dtype=torch.bfloat16)
    assert large_n._engine_dtype(x, "spherical") == torch.bfloat16
    assert large_n._engine_dtype(x, "diag") == torch.float32
    assert large_n._engine_dtype(x.double(), "spherical") == torch.float32


def test_estimator_routes_long_host_input_to_streaming():
    from gmmxx_amd import GMMXX
    gm = GMMXX(n_components=3, backend="hip", device="cuda", chunk_size_data_cpu=100)
    assert gm._is_large_cpu_stream_input(torch.zeros((1, 101, 2)))
    assert not gm._is_large_cpu_stream_input(torch.zeros((1, 100, 2)))


# The reference package's function-level names in this build's scope
# (gmmxx/__init__.py:1-34, cuda_ops.py:11-87): every one must exist here.
REFERENCE_NAMES = [
    "GMMXX", "batch_gmm_Spherical", "batch_gmm_Spherical_torch_native", "batch_gmm_Diagonal",
    "batch_gmm_Diagonal_torch_native", "batch_gmm_Full", "batch_gmm_Full_torch_native", "batch_gmm_Tied",
    "batch_gmm_Tied_torch_native", "batch_gmm_spherical", "batch_gmm_diagonal", "batch_gmm_diag",
    "batch_gmm_full", "batch_gmm_tied", "diagonal_assign_torch_native_chunked",
    "diagonal_predict_proba_torch_native_chunked", "diagonal_score_samples_torch_native_chunked",
    "full_assign_torch_native_chunked", "full_predict_proba_torch_native_chunked",
    "full_score_samples_torch_native_chunked", "tied_assign_torch_native_chunked",
    "tied_predict_proba_torch_native_chunked", "tied_score_samples_torch_native_chunked",
    "batch_gmm_largeN_cpu", "large_n_predict_cpu", "large_n_score_samples_cpu", "large_n_predict_proba_cpu",
]
REFERENCE_OPS = [
    "canary_add_offset", "spherical_assign", "spherical_logsumexp", "spherical_resp", "soft_update_spherical",
    "fused_spherical", "diag_assign", "diag_logsumexp", "diag_resp", "tied_assign", "tied_logsumexp",
    "tied_resp", "full_assign", "full_logsumexp", "full_resp",
]
# cuda_ops names of the reference's hard-EM and torch-only ops, which hip_ops
# does not provide: each must fail with an AttributeError naming the replacement.
REFERENCE_OPS_NOT_PROVIDED = [
    "blocked_update_spherical", "blocked_update_spherical_sorted", "finalize_spherical", "blocked_update_diag",
    "blocked_update_diag_sorted", "finalize_diag", "tied_project", "tied_log_det", "tied_finalize",
    "full_blocked_update", "full_finalize", "approx_topk_update_spherical",
]


def test_reference_function_names_exported():
    import gmmxx_amd
    missing = [n for n in REFERENCE_NAMES if not callable(getattr(gmmxx_amd, n, None))]
    assert not missing
    assert set(REFERENCE_NAMES) <= set(gmmxx_amd.__all__)
    # the aliases are the HIP engine's entry points
    assert gmmxx_amd.batch_gmm_diag is gmmxx_amd.batch_gmm_Diagonal_hip
    assert gmmxx_amd.batch_gmm_Full_torch_native is gmmxx_amd.batch_gmm_Full_hip


def test_hip_ops_mirrors_cuda_ops_names():
    import inspect
    from gmmxx_amd import hip_ops
    missing = [n for n in REFERENCE_OPS if not callable(getattr(hip_ops, n, None))]
    assert not missing
    assert set(REFERENCE_OPS) <= set(hip_ops.__all__)
    assert hip_ops.HipRuntimeFallback.__mro__[1].__name__ == "HipRuntimeError"
    # the reference ops' leading parameters (_cuda.py:328-412, :897-959, :1126-1201, :1274-1314, :1056)
    params = lambda f: list(inspect.signature(f).parameters)
    assert params(hip_ops.spherical_resp)[:6] == ["x", "means", "var", "log_w", "log_norm", "out"]
    assert params(hip_ops.diag_assign) == ["x", "means", "var", "log_w", "out"]
    assert params(hip_ops.tied_resp) == ["x", "means", "L", "log_w", "log_norm"]
    assert params(hip_ops.full_logsumexp) == ["x", "means", "L", "log_w"]
    assert params(hip_ops.fused_spherical) == ["x", "means", "var", "log_w", "reg_covar"]
    for name in REFERENCE_OPS_NOT_PROVIDED:
        with pytest.raises(AttributeError, match="not provided"):
            getattr(hip_ops, name)


def test_reference_named_wrappers_reject_unknown_keywords():
    import gmmxx_amd
    with pytest.raises(TypeError):
        gmmxx_amd.large_n_predict_cpu(torch.zeros(1, 4, 2), torch.zeros(1, 2, 2), torch.ones(1, 2),
                                      torch.ones(1, 2) / 2, covariance_type="spherical", device="cpu",
                                      dtype=torch.float32, not_a_knob=1)
