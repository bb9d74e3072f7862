"""Seeded random shapes through the whole Lloyd loop, beyond the hand-picked
cases of the other GPU tests: batch, point count, cluster count, feature
width and storage type drawn at random (within the documented limits), so
that plan choices meet in combinations no fixed list names (tiles per wave,
K slicing, kept scores, whole-table staging, the resident kernel, the
sort-free update with one or several labels per workgroup, ragged N, K > N).

Each case checks:
- the loop against the per-op (verbose) path, bit for bit;
- for rows the sort-free update takes (N <= 32768), that update against the
  sort path (FKC_UPDATE_SCAN=1 / 0), bit for bit;
- the final labels against the oracle's exact-distance assignment to the
  centroids they were scored against (the centroids after one iteration
  fewer), up to near-ties: all points when the oracle finishes in well under
  a second, else a random subsample.

The near-tie bar is the assign tests' 2^-16 of ||x||^2 + ||c||^2, widened in
proportion for D > 256 (the fp32 dot product's error bound grows with D).
A fixed list of edge shapes runs the same checks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import near_tie_report
from oracle import kmeans_oracle as O

pytestmark = pytest.mark.gpu


def _draw(seed, n, Ns, Ks, Ds, Bs, max_work, max_elems):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B, N = int(rng.choice(Bs)), int(rng.choice(Ns))
        K, D = int(rng.choice(Ks)), int(rng.choice(Ds))
        dt = str(rng.choice(["f16", "bf16", "f32"]))
        crowd = bool(rng.random() < 0.3)
        if B * N * max(K, 64) * D > max_work or B * N * D > max_elems:
            continue
        out.append((B, N, K, D, dt, crowd, int(rng.integers(1 << 30))))
    return out


SMALL = _draw(7, 80, [1, 7, 100, 513, 2048, 4099, 8192, 8193, 16384, 20000, 32768],
              [1, 2, 17, 64, 200, 256, 300, 1000, 2049, 4096],
              [8, 16, 24, 32, 40, 64, 96, 128, 136, 256, 300, 512],
              [1, 1, 1, 2, 3, 4], 3e10, 1 << 24)
LARGE = _draw(3, 32, [32769, 65536, 100003, 262144, 524288, 1 << 20],
              [100, 1000, 1024, 4096, 8192, 9000, 16384],
              [16, 32, 64, 100, 128, 256], [1, 1, 2, 4], 6e12, 1 << 26)


def _case_id(c):
    B, N, K, D, dt, crowd, _ = c
    return f"B{B}-N{N}-K{K}-D{D}-{dt}" + ("-crowd" if crowd else "")


def _inputs(B, N, K, D, dt, crowd, seed):
    from flash_kmeans_cuda import synth
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, N, D), dtype=np.float32) * 2
    if crowd and N > 10:   # most points on one spot: long runs of one label
        m = rng.random((B, N)) < 0.7
        x[m] = rng.standard_normal((int(m.sum()), D), dtype=np.float32) * 0.01
    xs = O.from_f32(x, dt)
    init = np.ascontiguousarray(xs[:, rng.choice(N, size=min(K, N), replace=False)])
    if init.shape[1] < K:  # more clusters than points: repeat a row
        init = np.ascontiguousarray(np.concatenate(
            [init, np.repeat(init[:, :1], K - init.shape[1], axis=1)], axis=1))
    return xs, init, synth.to_torch(xs, dt), synth.to_torch(init, dt), rng


def _check_labels(xs, xt, it, K, D, dt, labels, iters, rng):
    """Labels of an `iters`-iteration run against the oracle's assignment to
    the centroids of an (iters - 1)-iteration run."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    prev = batch_kmeans_Euclid(xt, K, max_iters=iters - 1, init_centroids=it)
    cen = synth.from_torch(prev[1], dt)
    B, N = labels.shape
    if B * N * K * D <= 2e8:
        xsub, got = xs, labels
    else:
        sub = rng.choice(N, size=min(N, 1024 if K * D <= 4e6 else 256), replace=False)
        xsub, got = np.ascontiguousarray(xs[:, sub]), labels[:, sub]
    ref = O.assign(xsub, cen, dt)
    nd, bad, worst = near_tie_report(xsub, cen, dt, got, ref,
                                     rel=2.0 ** -16 * max(1.0, D / 256))
    assert bad == 0, f"{bad} of {nd} disagreements beyond near-ties (worst {worst:.3e})"


def _same(a, b, what):
    assert a[2] == b[2], (what, "iterations", a[2], b[2])
    assert torch.equal(a[0], b[0]), (what, "labels")
    assert torch.equal(a[1], b[1]), (what, "centroids")


@pytest.mark.parametrize("case", SMALL, ids=_case_id)
def test_small_shapes(monkeypatch, case):
    from flash_kmeans_cuda import batch_kmeans_Euclid
    B, N, K, D, dt, crowd, seed = case
    print(_case_id(case), flush=True)
    xs, _, xt, it, rng = _inputs(*case)
    out = {}
    for v in ["1", "0"]:
        monkeypatch.setenv("FKC_UPDATE_SCAN", v)
        out[v] = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
    monkeypatch.delenv("FKC_UPDATE_SCAN")
    _same(out["1"], out["0"], "scan vs sort")
    per_op = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it, verbose=True)
    _same(out["1"], per_op, "loop vs per-op path")
    _check_labels(xs, xt, it, K, D, dt, out["1"][0].cpu().numpy(), 3, rng)


@pytest.mark.parametrize("case", LARGE, ids=_case_id)
def test_large_shapes(case):
    from flash_kmeans_cuda import batch_kmeans_Euclid
    B, N, K, D, dt, crowd, seed = case
    print(_case_id(case), flush=True)
    xs, _, xt, it, rng = _inputs(*case)
    a = batch_kmeans_Euclid(xt, K, max_iters=2, init_centroids=it)
    c = batch_kmeans_Euclid(xt, K, max_iters=2, init_centroids=it, verbose=True)
    _same(a, c, "loop vs per-op path")
    _check_labels(xs, xt, it, K, D, dt, a[0].cpu().numpy(), 2, rng)


EDGE = [
    (1, 1000, 100000, 16, "f16", False, 1),    # K far above N
    (64, 1000, 10, 8, "bf16", False, 2),       # many batch rows
    (1, 4096, 64, 1024, "f16", False, 3),      # D above the matrix-core route
    (1, 1 << 22, 16, 8, "f16", False, 4),      # 4M points, tiny K and D
    (3, 70000, 4097, 200, "bf16", False, 5),   # padded width, K one past a power of two
    (1, 100, 1, 4, "f32", False, 6),           # one cluster
    (2, 33000, 65535, 8, "f16", False, 7),     # K = 2^16 - 1, N just past the sort-free rows
    (1, 8192, 65536, 128, "bf16", False, 8),   # centroid slices
    (5, 3, 7, 520, "f16", False, 9),           # three points per row, D past 512
    (1, 50000, 300, 600, "f32", False, 10),    # wide fp32 rows
    (128, 256, 256, 32, "bf16", False, 11),    # 128 short batch rows
]


@pytest.mark.parametrize("case", EDGE, ids=_case_id)
def test_edge_shapes(case):
    """Shapes at the edges of what the plans choose between: K far above N,
    many rows, widths past the matrix-core route, millions of points, one
    cluster, K near 2^16 with N just past the sort-free update's 32768 rows,
    centroid slices."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    B, N, K, D, dt, crowd, seed = case
    print(_case_id(case), flush=True)
    xs, _, xt, it, rng = _inputs(*case)
    a = batch_kmeans_Euclid(xt, K, max_iters=2, init_centroids=it)
    c = batch_kmeans_Euclid(xt, K, max_iters=2, init_centroids=it, verbose=True)
    _same(a, c, "loop vs per-op path")
    _check_labels(xs, xt, it, K, D, dt, a[0].cpu().numpy(), 2, rng)
