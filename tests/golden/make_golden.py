"""Writes the golden vectors in this folder from the reference's own torch fallback.

Run in the build container only (the reference tree does not exist on the GPU
box):  python tests/golden/make_golden.py [/root/reference]

It imports ``gmmxx.torch_fallback`` from the reference checkout and runs its
CPU soft-EM functions on tiny seeded problems with explicit initial
parameters, then stores inputs and outputs as small ``.npz`` files.  These pin
the parts of the oracle that closed forms cannot: the finalize sequences and
active masks, the per-iteration prelude clamps, the Cholesky jitter ladder,
first-maximum label tie-breaking, chunked streaming over N and K, and the
lower-bound history.  Lower bounds are taken with ``verbose=True`` so every
iteration is recorded (the reference stores 0.0 for non-final iterations of
diag/tied/full otherwise).
"""

from __future__ import annotations

import contextlib
import io
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _blobs(gen, b, n, d, k, spread=4.0, scale=1.0):
    centers = (torch.rand((b, k, d), generator=gen) * 2 - 1) * spread
    lab = torch.randint(0, k, (b, n), generator=gen)
    x = torch.gather(centers, 1, lab[..., None].expand(-1, -1, d))
    x = x + scale * torch.randn((b, n, d), generator=gen)
    return x.float().contiguous()


def _spd(gen, shape, d, jit=0.3):
    a = torch.randn(shape + (d, d), generator=gen) * 0.4
    return (a @ a.transpose(-1, -2) + jit * torch.eye(d)).float()


def cases():
    """(name, covariance, x, init dict, fit kwargs)."""
    g = torch.Generator().manual_seed(1234)
    out = []
    # Plain problems, B=2, default chunking.
    for cov in ("spherical", "diag", "tied", "full"):
        b, n, d, k = 2, 384, 5, 4
        x = _blobs(g, b, n, d, k)
        means = x[:, :k, :].clone()
        if cov == "spherical":
            covs = torch.rand((b, k), generator=g) + 0.5
        elif cov == "diag":
            covs = torch.rand((b, k, d), generator=g) + 0.5
        elif cov == "tied":
            covs = _spd(g, (b,), d)
        else:
            covs = _spd(g, (b, k), d)
        w = torch.rand((b, k), generator=g) + 0.2
        out.append((f"{cov}_basic", cov, x, dict(init_means=means, init_variances=covs,
                                                   init_weights=w), dict(max_iters=3)))
    # Streaming over N and K chunks (N > chunk_N, K > chunk_K).
    for cov in ("spherical", "diag", "tied", "full"):
        b, n, d, k = 1, 300, 3, 7
        x = _blobs(g, b, n, d, k, spread=3.0)
        means = x[:, 10:10 + k, :].clone()
        covs = {"spherical": torch.ones((b, k)), "diag": torch.ones((b, k, d)),
                "tied": torch.eye(d).expand(b, d, d).clone(),
                "full": torch.eye(d).expand(b, k, d, d).clone()}[cov]
        out.append((f"{cov}_chunked", cov, x, dict(init_means=means, init_variances=covs,
                                                     init_weights=None),
                    dict(max_iters=3, chunk_size_N=64, chunk_size_K=3)))
    # Empty component (active mask) + weight floor: one mean far from all data.
    for cov in ("spherical", "diag", "tied", "full"):
        b, n, d, k = 1, 200, 4, 3
        x = _blobs(g, b, n, d, 2, spread=2.0)
        means = torch.cat([x[:, :2, :], torch.full((b, 1, d), 1e3)], dim=1)
        covs = {"spherical": torch.ones((b, k)), "diag": torch.ones((b, k, d)),
                "tied": torch.eye(d).expand(b, d, d).clone(),
                "full": torch.eye(d).expand(b, k, d, d).clone()}[cov]
        out.append((f"{cov}_empty", cov, x, dict(init_means=means, init_variances=covs,
                                                   init_weights=torch.tensor([[0.5, 0.5, 1e-12]])),
                    dict(max_iters=2)))
    # Duplicate components: exact logit ties -> first index wins.
    for cov in ("spherical", "diag", "tied", "full"):
        b, n, d, k = 1, 128, 3, 4
        x = _blobs(g, b, n, d, 2, spread=3.0)
        m = x[:, :2, :].clone()
        means = torch.cat([m, m], dim=1)
        covs = {"spherical": torch.ones((b, k)), "diag": torch.ones((b, k, d)),
                "tied": torch.eye(d).expand(b, d, d).clone(),
                "full": torch.eye(d).expand(b, k, d, d).clone()}[cov]
        out.append((f"{cov}_ties", cov, x, dict(init_means=means, init_variances=covs,
                                                  init_weights=None), dict(max_iters=2)))
    # Indefinite covariance -> Cholesky jitter ladder (tied and full).  diag(1, 1, -1e-3)
    # first factorises at jitter 1e-2 and is then well conditioned; for full only
    # one component is indefinite, so the batch-global retry is exercised too.
    for cov in ("tied", "full"):
        b, n, d, k = 1, 160, 3, 2
        x = _blobs(g, b, n, d, k, spread=2.0)
        bad = torch.diag(torch.tensor([1.0, 1.0, -1e-3]))
        good = torch.diag(torch.tensor([1.5, 0.8, 1.2]))
        covs = bad.expand(b, d, d).clone() if cov == "tied" else torch.stack([bad, good]).unsqueeze(0)
        out.append((f"{cov}_jitter", cov, x, dict(init_means=x[:, :k, :].clone(),
                                                    init_variances=covs, init_weights=None),
                    dict(max_iters=2)))
    # Default variance initialisation (init_variances=None).
    for cov in ("spherical", "diag", "tied", "full"):
        b, n, d, k = 1, 256, 4, 3
        x = _blobs(g, b, n, d, k)
        out.append((f"{cov}_defaultvar", cov, x, dict(init_means=x[:, :k, :].clone(),
                                                        init_variances=None, init_weights=None),
                    dict(max_iters=2)))
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from gmmxx import torch_fallback as tf  # the reference fallback (read-only checkout)

    fns = {"spherical": tf.batch_gmm_Spherical_torch_native,
           "diag": tf.batch_gmm_Diagonal_torch_native,
           "tied": tf.batch_gmm_Tied_torch_native,
           "full": tf.batch_gmm_Full_torch_native}
    inf = {"spherical": (tf.spherical_assign_torch_native_chunked,
                         tf.spherical_score_samples_torch_native_chunked,
                         tf.spherical_predict_proba_torch_native_chunked),
           "diag": (tf.diagonal_assign_torch_native_chunked,
                    tf.diagonal_score_samples_torch_native_chunked,
                    tf.diagonal_predict_proba_torch_native_chunked),
           "tied": (tf.tied_assign_torch_native_chunked,
                    tf.tied_score_samples_torch_native_chunked,
                    tf.tied_predict_proba_torch_native_chunked),
           "full": (tf.full_assign_torch_native_chunked,
                    tf.full_score_samples_torch_native_chunked,
                    tf.full_predict_proba_torch_native_chunked)}
    manifest = []
    for name, cov, x, init, kw in cases():
        kwargs = dict(tol=0.0, verbose=True, reg_covar=1e-6, gmm_use_triton=False) \
            if cov != "spherical" else dict(tol=0.0, verbose=True, reg_covar=1e-6,
                                            gmm_use_triton_estep=False,
                                            gmm_use_triton_streaming_update=False)
        kwargs.update(kw)
        with contextlib.redirect_stdout(io.StringIO()):
            labels, means, covs, w, info = fns[cov](x, init["init_means"].shape[1], **init,
                                                     **kwargs)
        ck = dict(chunk_size_N=kw.get("chunk_size_N", 32768),
                  chunk_size_K=kw.get("chunk_size_K", 1024))
        assign_fn, score_fn, proba_fn = inf[cov]
        lab2 = assign_fn(x, means, covs, w, **ck)
        score = score_fn(x, means, covs, w, **ck)
        proba = proba_fn(x, means, covs, w, **ck)
        arrays = {"x": x.numpy(), "means": means.numpy(), "covs": covs.numpy(),
                  "weights": w.numpy(), "labels": labels.numpy(),
                  "lower_bound_history": np.asarray(info["lower_bound_history"], np.float64),
                  "assign": lab2.numpy(), "score": score.numpy(), "proba": proba.numpy()}
        for key in ("init_means", "init_variances", "init_weights"):
            if init.get(key) is not None:
                arrays[key] = init[key].numpy()
        meta = {"name": name, "covariance_type": cov, "n_iter": int(info["n_iter"]),
                "fit_kwargs": {k: v for k, v in kw.items()}, "reg_covar": 1e-6,
                "torch_version": torch.__version__,
                "source": "gmmxx/torch_fallback.py batch_gmm_*_torch_native (verbose=True)"}
        arrays["meta"] = np.asarray(json.dumps(meta))
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        manifest.append(meta)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(f"wrote {len(manifest)} fixtures")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
