"""The Lloyd loop's sort-free update for short rows (update_scan) against the
sort path it replaces (label_sort + update_runs + update_merge): the loop run
with FKC_UPDATE_SCAN=1 and =0 must give the same labels, centroids and
iteration counts bit for bit, and the per-op (verbose) path the same again.

Cases: the c1 / c2 shapes the plan takes it for, batches, ragged N (labels
read one by one instead of four at a time), odd and wide feature widths
(one to four column slices per lane, two columns per lane or one), several
labels per workgroup, empty clusters, one point, tol > 0, and rows whose
points crowd into a few labels: runs over many units, whole 64-unit blocks
summed as block partials, and a label with more rows than one placement
window holds; and, for one label per workgroup, runs sized on both sides
of the LDS room for unit partials.  The two switches that reshape the
update (labels per workgroup, rows per unit) are swept too.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kmeans_oracle as O

pytestmark = pytest.mark.gpu


def _T(a, dtype):
    from flash_kmeans_cuda import synth
    return synth.to_torch(a, dtype)


def _both(monkeypatch, xt, K, init, iters, tol=0.0):
    from flash_kmeans_cuda import batch_kmeans_Euclid
    out = []
    for v in ["1", "0"]:
        monkeypatch.setenv("FKC_UPDATE_SCAN", v)
        out.append(batch_kmeans_Euclid(xt, K, max_iters=iters, tol=tol,
                                       init_centroids=init))
    monkeypatch.delenv("FKC_UPDATE_SCAN")
    return out


def _same(a, b, what):
    assert a[2] == b[2], (what, "iterations", a[2], b[2])
    assert torch.equal(a[0], b[0]), (what, "labels")
    assert torch.equal(a[1], b[1]), (what, "centroids")


@pytest.mark.parametrize("B,N,K,D,dtype", [
    (1, 32768, 256, 128, "f16"),     # c2
    (1, 4096, 64, 128, "f32"),       # c1
    (3, 5000, 100, 64, "bf16"),
    (2, 4099, 37, 96, "f16"),        # N % 4 != 0
    (1, 3001, 50, 7, "f32"),         # odd D: one column per lane
    (1, 2000, 20, 512, "f16"),       # four column slices
    (2, 2500, 30, 300, "bf16"),
    (1, 20000, 1000, 32, "f16"),     # four labels per workgroup
    (16, 2048, 200, 16, "f32"),      # thirteen labels per workgroup
    (1, 1, 1, 16, "f16"),
    (2, 70, 64, 8, "bf16"),          # most clusters empty
    (1, 8192, 300, 64, "f16"),       # the largest row of two label quads per thread
    (1, 8193, 300, 64, "f16"),       # the smallest of eight
    (2, 32768, 256, 128, "bf16"),    # the largest row, batched
])
def test_scan_update_equals_sort_path(monkeypatch, B, N, K, D, dtype):
    from flash_kmeans_cuda import batch_kmeans_Euclid
    print(f"B={B} N={N} K={K} D={D} {dtype}", flush=True)
    rng = np.random.default_rng(N + K + D)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 2, dtype)
    init = np.ascontiguousarray(x[:, rng.choice(N, min(K, N), replace=False)])
    if init.shape[1] < K:  # more clusters than points: repeat rows
        init = np.ascontiguousarray(np.concatenate(
            [init, np.repeat(init[:, :1], K - init.shape[1], axis=1)], axis=1))
    xt, it = _T(x, dtype), _T(init, dtype)
    a, b = _both(monkeypatch, xt, K, it, 3)
    _same(a, b, "scan vs sort")
    c = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it, verbose=True)
    _same(a, c, "loop vs per-op path")


@pytest.mark.parametrize("B,N,K,D,dtype,share", [
    (1, 32768, 64, 64, "bf16", 0.95),   # one label with ~31000 rows: two windows
    (2, 30000, 300, 128, "f16", 0.6),
    (1, 9000, 40, 24, "f32", 0.9),
])
def test_scan_update_crowded_labels(monkeypatch, B, N, K, D, dtype, share):
    """Most points sit on one centroid: its run covers hundreds of units and
    whole 64-unit blocks, and (first case) more sorted positions than one
    placement window (16384)."""
    print(f"B={B} N={N} K={K} D={D} {dtype} share={share}", flush=True)
    rng = np.random.default_rng(K + N)
    x = rng.standard_normal((B, N, D)).astype(np.float32) * 4
    crowd = rng.random((B, N)) < share
    x[crowd] = rng.standard_normal((int(crowd.sum()), D)).astype(np.float32) * 0.01
    x = O.from_f32(x, dtype)
    init = np.ascontiguousarray(x[:, :K])
    xt, it = _T(x, dtype), _T(init, dtype)
    a, b = _both(monkeypatch, xt, K, it, 3)
    _same(a, b, "scan vs sort")
    counts = np.bincount(a[0].cpu().numpy()[0], minlength=K)
    assert counts.max() > 0.5 * share * N


def test_scan_update_with_tol(monkeypatch):
    from flash_kmeans_cuda import synth
    cfg = synth.CONFIGS["c2"]
    x, init = synth.make(cfg, N=16384)
    xt, it = _T(x, "f16"), _T(init, "f16")
    a, b = _both(monkeypatch, xt, cfg.K, it, 30, tol=1e-3)
    _same(a, b, "tol")
    assert a[2] < 30


@pytest.mark.parametrize("D,dtype", [(512, "f16"), (256, "bf16")])
def test_scan_update_lds_partial_boundary(monkeypatch, D, dtype):
    """One label per workgroup: a run over several units keeps its unit
    partials in LDS only while (units spanned) x D fits the 16384-float
    region (32 units of 32 rows at D = 512, 64 at D = 256) and no whole
    64-unit block lies inside it.  Labels sized around that capacity (and a
    few long enough for whole blocks) must give the sort path's bits either
    way.  Points are copies of well separated centroids plus small noise, so
    the label sizes are set by construction."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    print(f"D={D} {dtype}", flush=True)
    rng = np.random.default_rng(D)
    cap_rows = 16384 // D * 32
    sizes = [cap_rows - 64 + 16 * i for i in range(9)]   # both sides of the capacity
    sizes += [2100, 2600, 3100]                          # whole 64-unit blocks inside
    sizes += [37, 5, 1, 90, 300]
    K = len(sizes) + 3                                   # three empty labels
    cent = rng.standard_normal((K, D)).astype(np.float32) * 8
    rows = [cent[k] + rng.standard_normal((n, D)).astype(np.float32) * 0.01
            for k, n in enumerate(sizes)]
    x = np.concatenate(rows)[rng.permutation(sum(sizes))]
    assert x.shape[0] <= 32768
    x = O.from_f32(x[None], dtype)
    init = O.from_f32(cent[None], dtype)
    xt, it = _T(x, dtype), _T(init, dtype)
    a, b = _both(monkeypatch, xt, K, it, 3)
    _same(a, b, "scan vs sort")
    c = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it, verbose=True)
    _same(a, c, "loop vs per-op path")
    counts = np.bincount(a[0].cpu().numpy()[0], minlength=K)
    assert counts[:len(sizes)].tolist() == sizes and counts[len(sizes):].sum() == 0



@pytest.mark.parametrize("B,N,K,D,dtype", [
    (2, 20000, 300, 64, "bf16"),
    (1, 32768, 256, 128, "f16"),     # c2
])
def test_scan_update_labels_per_workgroup(monkeypatch, B, N, K, D, dtype):
    """FKC_SCAN_WGS sets how many workgroups share a row's labels (labels per
    workgroup kpw = ceil(B K / FKC_SCAN_WGS)): one label each (the one-label
    form), a few, the most the bitmap form holds (16), and one more than
    that (17: the plan then takes the sort path).  Positions, units and
    summation order do not depend on kpw, so every setting gives the sort
    path's bits."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    print(f"B={B} N={N} K={K} D={D} {dtype}", flush=True)
    rng = np.random.default_rng(B * N + K)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 2, dtype)
    init = np.ascontiguousarray(x[:, rng.choice(N, K, replace=False)])
    xt, it = _T(x, dtype), _T(init, dtype)
    monkeypatch.setenv("FKC_UPDATE_SCAN", "0")
    ref = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
    monkeypatch.setenv("FKC_UPDATE_SCAN", "1")
    BK = B * K
    for kpw in [1, 2, 3, 7, 16, 17]:
        monkeypatch.setenv("FKC_SCAN_WGS", str(-(-BK // kpw)))
        got = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
        _same(got, ref, f"kpw {kpw}")
    monkeypatch.delenv("FKC_SCAN_WGS")
    monkeypatch.delenv("FKC_UPDATE_SCAN")


@pytest.mark.parametrize("B,N,K,D,dtype", [
    (1, 20000, 200, 128, "bf16"),    # sort-free update
    (2, 40000, 300, 64, "f16"),      # sort path
])
def test_update_rows_per_unit(monkeypatch, B, N, K, D, dtype):
    """FKC_UPDATE_ROWS (32, 64 or 128 rows per unit) changes the summation
    bracketing, so centroids may differ from the automatic choice by fp32
    accumulation error (bounded here by 1e-4 absolute: ~200 rows of |x| < 10
    at 2^-23 each, far looser than typical) plus one unit in the last place
    of the storage type.  For each setting the sort-free update still equals
    the sort path and the loop equals the per-op path bit for bit; the
    one-iteration labels never change (they come from the initial
    centroids)."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    print(f"B={B} N={N} K={K} D={D} {dtype}", flush=True)
    rng = np.random.default_rng(N + K + D)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 2, dtype)
    init = np.ascontiguousarray(x[:, rng.choice(N, K, replace=False)])
    xt, it = _T(x, dtype), _T(init, dtype)
    base = batch_kmeans_Euclid(xt, K, max_iters=1, init_centroids=it)
    c0 = O.to_f64(_np_of(base[1], dtype), dtype)
    ulp = 2.0 ** (-10 if dtype == "f16" else -7)
    for ur in ["32", "64", "128"]:
        monkeypatch.setenv("FKC_UPDATE_ROWS", ur)
        a, b = _both(monkeypatch, xt, K, it, 1)
        _same(a, b, f"rows {ur}: scan vs sort")
        c = batch_kmeans_Euclid(xt, K, max_iters=1, init_centroids=it, verbose=True)
        _same(a, c, f"rows {ur}: loop vs per-op path")
        assert torch.equal(a[0], base[0]), ur
        cu = O.to_f64(_np_of(a[1], dtype), dtype)
        assert np.all(np.abs(cu - c0) <= ulp * np.abs(c0) + 1e-4), ur
    monkeypatch.delenv("FKC_UPDATE_ROWS")


def _np_of(t, dtype):
    from flash_kmeans_cuda import synth
    return synth.from_torch(t, dtype)
