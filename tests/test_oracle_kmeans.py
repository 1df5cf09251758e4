"""Pins the oracle's k-means initialisation (oracle/torch_ref.py: kmeans_pp,
lloyd, hard_label_init_stats) with checks that do not restate it:

* k-means++: an independent float64 numpy implementation fed the same random
  numbers picks the same rows; with K = S every row is picked exactly once; on
  well-separated blobs every blob gets exactly one seed;
* Lloyd: one iteration equals a float64 brute force; from one seed per blob it
  lands on the blob means (closed form) with the true partition;
* hard-label statistics: float64 loops over the rows, with an empty cluster
  (global (co)variance) in the mix.
"""

import math

import numpy as np
import pytest
import torch

from oracle import torch_ref

COVS = ("spherical", "diag", "tied", "full")


def _blobs(b, per, d, k, sep, seed):
    g = torch.Generator().manual_seed(seed)
    centers = torch.randn((b, k, d), generator=g) * sep
    lab = torch.arange(k).repeat_interleave(per).expand(b, -1).clone()
    x = torch.gather(centers, 1, lab[..., None].expand(-1, -1, d)) + torch.randn((b, k * per, d), generator=g)
    return x, lab, centers


def _kpp_numpy(sample, k, first, draws):
    s = sample.double().numpy()
    bsz, n, _ = s.shape
    out = np.zeros((bsz, k), dtype=np.int64)
    for b in range(bsz):
        chosen = [int(first[b])]
        closest = ((s[b] - s[b, chosen[0]]) ** 2).sum(-1)
        for c in range(1, k):
            total = closest.sum()
            cum = np.cumsum(closest)
            cands = []
            for u in draws[b, c - 1].double().numpy():
                i = int(np.searchsorted(cum, u * total, side="left")) if total > 0 else 0
                cands.append(min(i, n - 1))
            pots = [np.minimum(closest, ((s[b] - s[b, i]) ** 2).sum(-1)).sum() for i in cands]
            j = cands[int(np.argmin(pots))]
            chosen.append(j)
            closest = np.minimum(closest, ((s[b] - s[b, j]) ** 2).sum(-1))
        out[b] = chosen
    return out


def _rows_of(centers, sample):
    """Row index of each centre in the sample (centres are copies of rows)."""
    eq = (centers.unsqueeze(2) == sample.to(torch.float32).unsqueeze(1)).all(-1)   # (B, K, S)
    assert bool(eq.any(-1).all()), "every centre is a sample row"
    return eq.float().argmax(-1).numpy()


@pytest.mark.parametrize("b,s,d,k", [(2, 300, 4, 12), (1, 500, 7, 30), (3, 64, 2, 5)])
def test_kmeans_pp_vs_float64_numpy(b, s, d, k):
    g = torch.Generator().manual_seed(b * 100 + k)
    sample = torch.randn((b, s, d), generator=g) * 3
    first = torch.randint(0, s, (b,), generator=g)
    draws = torch.rand((b, k - 1, 2 + int(math.log(k))), generator=g)
    centers = torch_ref.kmeans_pp(sample, k, first, draws)
    np.testing.assert_array_equal(_rows_of(centers, sample), _kpp_numpy(sample, k, first, draws))


def test_kmeans_pp_k_equals_s_takes_every_row_once():
    g = torch.Generator().manual_seed(5)
    sample = torch.randn((2, 40, 3), generator=g)
    centers = torch_ref.kmeans_pp(sample, 40, torch.tensor([0, 17]), torch.rand((2, 39, 5), generator=g))
    rows = _rows_of(centers, sample)
    for b in range(2):
        assert sorted(rows[b].tolist()) == list(range(40))


def test_kmeans_pp_one_seed_per_blob():
    x, lab, _ = _blobs(2, 50, 6, 8, sep=200.0, seed=6)
    g = torch.Generator().manual_seed(7)
    centers = torch_ref.kmeans_pp(x, 8, torch.tensor([3, 120]), torch.rand((2, 7, 4), generator=g))
    rows = _rows_of(centers, x)
    for b in range(2):
        assert sorted(lab[b, rows[b]].tolist()) == list(range(8))


def test_lloyd_one_step_vs_float64():
    g = torch.Generator().manual_seed(8)
    x = torch.randn((2, 400, 5), generator=g) * 2
    seeds = torch.randn((2, 9, 5), generator=g) * 2
    seeds[1, 4] = 1e4                        # a centre no row is nearest to: keeps its place
    labels, means, it = torch_ref.lloyd(x, seeds, max_iters=1, tol=0.0)
    assert it == 1
    xn, cn = x.double().numpy(), seeds.double().numpy()
    for b in range(2):
        dist = ((xn[b][:, None, :] - cn[b][None, :, :]) ** 2).sum(-1)
        lab = dist.argmin(-1)
        np.testing.assert_array_equal(labels[b].numpy(), lab)
        for j in range(9):
            exp = xn[b][lab == j].mean(0) if (lab == j).any() else cn[b, j]
            np.testing.assert_allclose(means[b, j].double().numpy(), exp, rtol=1e-5, atol=1e-5)
    assert float(means[1, 4, 0]) == 1e4


def test_lloyd_from_one_seed_per_blob_lands_on_blob_means():
    x, lab, _ = _blobs(1, 80, 4, 6, sep=50.0, seed=9)
    seeds = torch.stack([x[0, lab[0] == j][0] for j in range(6)]).unsqueeze(0)   # a row of every blob
    labels, means, it = torch_ref.lloyd(x, seeds, max_iters=10, tol=1e-4)
    assert it <= 3
    torch.testing.assert_close(labels, lab)
    exp = torch.stack([x[0, lab[0] == j].mean(0) for j in range(6)]).unsqueeze(0)
    torch.testing.assert_close(means, exp, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("cov", COVS)
def test_hard_label_init_stats_vs_float64(cov):
    g = torch.Generator().manual_seed(10)
    b, n, d, k = 2, 120, 3, 5
    x = torch.randn((b, n, d), generator=g) * 2
    means = torch.randn((b, k, d), generator=g)
    labels = torch.randint(0, k - 1, (b, n), generator=g)     # cluster k-1 stays empty
    reg = 1e-3
    w, c = torch_ref.hard_label_init_stats(x, cov, means, labels, reg)
    xn, mn, ln = x.double().numpy(), means.double().numpy(), labels.numpy()
    for bi in range(b):
        counts = np.bincount(ln[bi], minlength=k).astype(float)
        np.testing.assert_allclose(w[bi].double().numpy(), np.maximum(counts, 1) / np.maximum(counts, 1).sum(),
                                   rtol=1e-6)
        xc = xn[bi] - xn[bi].mean(0)
        gcov = xc.T @ xc / n
        diffs = xn[bi] - mn[bi][ln[bi]]
        if cov == "tied":
            np.testing.assert_allclose(c[bi].double().numpy(), diffs.T @ diffs / n + reg * np.eye(d),
                                       rtol=1e-5, atol=1e-5)
            continue
        for j in range(k):
            dj = diffs[ln[bi] == j]
            if cov == "spherical":
                exp = max((dj ** 2).sum() / len(dj) / d, reg) if len(dj) else max(np.trace(gcov) / d, reg)
            elif cov == "diag":
                exp = np.maximum((dj ** 2).sum(0) / len(dj), reg) if len(dj) else np.maximum(np.diag(gcov), reg)
            else:
                exp = (dj.T @ dj / len(dj) if len(dj) else gcov) + reg * np.eye(d)
            np.testing.assert_allclose(c[bi, j].double().numpy(), exp, rtol=1e-5, atol=1e-5)


def _lloyd_f64(x, c, max_iters, tol):
    """float64 numpy Lloyd: assignment to the nearest centre (first on ties),
    centre = mean of its rows (empty keeps its place); stop after max_iters, or
    once tol > 0 and the largest centre move is below tol.  Returns (centres,
    iterations, per-iteration largest moves, per-iteration k-means objective)."""
    xn, cn = x.double().numpy(), c.double().numpy().copy()
    bsz, k = cn.shape[0], cn.shape[1]
    shifts, objs = [], []
    for it in range(1, max_iters + 1):
        new = cn.copy()
        obj = 0.0
        for b in range(bsz):
            dist = ((xn[b][:, None, :] - cn[b][None, :, :]) ** 2).sum(-1)
            lab = dist.argmin(-1)
            obj += float(dist[np.arange(len(lab)), lab].sum())
            for j in range(k):
                if (lab == j).any():
                    new[b, j] = xn[b][lab == j].mean(0)
        shift = float(np.sqrt(((new - cn) ** 2).sum(-1)).max())
        cn = new
        shifts.append(shift)
        objs.append(obj)
        if tol > 0.0 and shift < tol:
            return cn, it, shifts, objs
    return cn, max_iters, shifts, objs


def test_lloyd_stop_rule_mid_run_vs_float64():
    """The stop rule as implemented: on overlapping clusters Lloyd moves for
    several iterations; a tol between two consecutive float64 moves (far from
    both) must stop the oracle at the same iteration with the same centres, the
    k-means objective never increases, and tol = 0 runs every iteration.  (The
    rule itself is flash-kmeans'; that package is not in the reference tree, so
    its agreement with flash-kmeans is not pinned -- see the module docstring of
    gmmxx_amd/kmeans.py.)"""
    g = torch.Generator().manual_seed(21)
    x = torch.randn((2, 300, 3), generator=g)
    x[:, :150] += 1.5
    seeds = x[:, :5].clone()
    _, _, shifts, objs = _lloyd_f64(x, seeds, 12, 0.0)
    assert all(b <= a + 1e-9 for a, b in zip(objs, objs[1:])), "objective must not increase"
    # a stopping point in the middle of the run, tol halfway (geometric) between two moves
    cand = [i for i in range(2, len(shifts) - 1) if shifts[i] < 0.5 * shifts[i - 1] and shifts[i] > 1e-3]
    assert cand, f"no well-separated consecutive moves in {shifts}"
    i = cand[0]
    tol = math.sqrt(shifts[i] * shifts[i - 1])
    e_c, e_it, _, _ = _lloyd_f64(x, seeds, 12, tol)
    assert 1 < e_it < 12
    labels, means, it = torch_ref.lloyd(x, seeds, max_iters=12, tol=tol)
    assert it == e_it
    np.testing.assert_allclose(means.double().numpy(), e_c, rtol=1e-5, atol=1e-5)
    _, means0, it0 = torch_ref.lloyd(x, seeds, max_iters=7, tol=0.0)
    assert it0 == 7
