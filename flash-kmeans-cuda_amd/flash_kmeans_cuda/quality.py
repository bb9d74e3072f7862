"""Clustering quality on the device: assigned inertia, empty clusters and
the inertia of a point sample.

Mirror of the evaluator in the reference's quality benchmark
(benchmarks/quality_compare.py:63-116), same names without the leading
underscore and the same argument meaning:

* `assign_with_fixed_evaluator(x, cents)` re-assigns with the final
  centroids through `euclid_assign` with explicit x_sq and c_sq (:63-66);
* `assigned_inertia(x, ids, cents, chunk_n)` sums ||x - c_id||^2 over every
  batch row with fp32 differences and squares and an fp64 total (:69-83);
* `empty_clusters(ids, K)` counts the k in [0, K) that no label of any batch
  row carries: the labels of all rows go into one K-bin histogram, as the
  reference's `bincount(ids.reshape(-1), minlength=K) == 0` does (:86-88);
* `sample_exact_inertia(x, cents, sample_points, seed, chunk_n)` sums, over a
  random sample of point indices shared by every row, the squared distance
  to the nearest centroid (:91-116).

Each runs as one pass of HIP kernels (fkc_assigned_inertia,
fkc_sampled_inertia); chunk_n is accepted for signature parity and not
needed (nothing is materialised per chunk).  The sums are bitwise
reproducible.
"""

from __future__ import annotations

from typing import Dict

import torch

from . import _lib
from .ops import _gpu_dense, euclid_assign, row_sqnorm


def _check_pair(x: torch.Tensor, cents: torch.Tensor, what: str):
    x = _gpu_dense("x", x)
    cents = _gpu_dense("centroids", cents)
    if x.dim() != 3 or cents.dim() != 3 or cents.shape[0] != x.shape[0] or \
            cents.shape[2] != x.shape[2]:
        raise RuntimeError(f"{what}: shapes must be x (B,N,D), centroids (B,K,D)")
    if cents.dtype != x.dtype:
        raise RuntimeError(f"{what}: x and centroids must share a dtype")
    return x, cents


def _run(x, ids: torch.Tensor, cents, K: int, want_inertia: bool):
    ids = _gpu_dense("ids", ids)
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    B, N = ids.shape
    dev = ids.device
    if want_inertia:
        x, cents = _check_pair(x, cents, "assigned_inertia")
        if x.shape[:2] != (B, N):
            raise RuntimeError("assigned_inertia: ids must be (B,N) like x")
        D = x.shape[2]
        dt = _lib.dtype_code(x.dtype)
    else:
        D, dt = 1, _lib.FKC_F32
    inertia = torch.empty(B, dtype=torch.float64, device=dev) if want_inertia else None
    empty = torch.empty(1, dtype=torch.int32, device=dev)
    ws = _lib.workspace(_lib.lib.fkc_quality_workspace_bytes(B, N, K), dev)
    _lib.check(_lib.lib.fkc_assigned_inertia(
        _lib.ptr(x) if want_inertia else None, _lib.ptr(cents) if want_inertia else None,
        ids.data_ptr(), B, N, K, D, dt, _lib.ptr(inertia), empty.data_ptr(),
        ws.data_ptr(), ws.numel(), _lib.stream_of(ids)), "assigned_inertia")
    return inertia, empty


def assigned_inertia(x: torch.Tensor, ids: torch.Tensor, cents: torch.Tensor,
                     chunk_n: int = 65536) -> float:
    """sum over all (b, n) of ||x[b,n] - cents[b, ids[b,n]]||^2 (fp64 total)."""
    del chunk_n
    inertia, _ = _run(x, ids, cents, cents.shape[1], True)
    return float(inertia.sum().item())


def empty_clusters(ids: torch.Tensor, K: int) -> int:
    """Number of k in [0, K) that no label of any batch row carries."""
    _, empty = _run(None, ids, None, int(K), False)
    return int(empty.item())


def sample_exact_inertia(x: torch.Tensor, cents: torch.Tensor, sample_points: int,
                         seed: int, chunk_n: int = 512) -> float:
    """Nearest-centroid inertia of `sample_points` points drawn without
    replacement (the same indices in every batch row), summed over rows;
    nan when sample_points <= 0.  The indices come from
    torch.randperm(N, generator=Generator(device).manual_seed(seed)) as in
    the reference; the distances from fkc_sampled_inertia."""
    del chunk_n
    x, cents = _check_pair(x, cents, "sample_exact_inertia")
    B, N, D = x.shape
    K = cents.shape[1]
    if sample_points <= 0:
        return float("nan")
    S = min(int(sample_points), N)
    g = torch.Generator(device=x.device).manual_seed(int(seed))
    idx = torch.randperm(N, generator=g, device=x.device)[:S].to(torch.int32)
    return sampled_inertia(x, cents, idx)


def sampled_inertia(x: torch.Tensor, cents: torch.Tensor, idx: torch.Tensor) -> float:
    """Nearest-centroid inertia of the points x[:, idx] (idx int32 on x's
    device, shared by every batch row), summed over rows (fp64)."""
    x, cents = _check_pair(x, cents, "sampled_inertia")
    B, N, D = x.shape
    K = cents.shape[1]
    idx = _gpu_dense("idx", idx)
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    S = idx.numel()
    dt = _lib.dtype_code(x.dtype)
    out = torch.empty(B, dtype=torch.float64, device=x.device)
    ws = _lib.workspace(_lib.lib.fkc_sampled_inertia_workspace_bytes(B, S, K, D, dt),
                        x.device)
    _lib.check(_lib.lib.fkc_sampled_inertia(
        x.data_ptr(), cents.data_ptr(), idx.data_ptr(), S, B, N, K, D, dt,
        out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(x)),
        "sampled_inertia")
    return float(out.sum().item())


def assign_with_fixed_evaluator(x: torch.Tensor, cents: torch.Tensor) -> torch.Tensor:
    """Labels of x against final centroids, with explicit x_sq and c_sq."""
    return euclid_assign(x, cents.contiguous(), row_sqnorm(x), c_sq=row_sqnorm(cents))


def evaluate(x: torch.Tensor, cents: torch.Tensor, *, sample_points: int = 4096,
             seed: int = 1000) -> Dict[str, object]:
    """Re-assign with `cents`, then the inertia and empty-cluster count of
    those labels and the sampled inertia (what quality_compare.py reports per
    run; its sample seed is args.seed + 1000)."""
    ids = assign_with_fixed_evaluator(x, cents)
    inertia, empty = _run(x, ids, cents, cents.shape[1], True)
    return {"ids": ids, "inertia": float(inertia.sum().item()),
            "inertia_per_batch": inertia.cpu().tolist(),
            "empty_clusters": int(empty.item()),
            "sample_exact_inertia": sample_exact_inertia(x, cents, sample_points, seed)}
