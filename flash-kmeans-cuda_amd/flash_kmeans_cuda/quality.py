"""Clustering quality on the device: assigned inertia and empty clusters.

Mirror of the evaluator in the reference's quality benchmark
(benchmarks/quality_compare.py:63-90): `assign_with_fixed_evaluator`
re-assigns with final centroids through `euclid_assign` with explicit x_sq
and c_sq (:63-66), `assigned_inertia` sums ||x - c_id||^2 with fp32
differences and squares and an fp64 total (:69-83), `empty_clusters` counts
clusters no point carries (:86-88).  One fused pass over x on the GPU
(fkc_assigned_inertia); the totals are bitwise reproducible.
"""

from __future__ import annotations

from typing import Dict

import torch

from . import _lib
from .ops import _ensure_contig, euclid_assign, row_sqnorm


def _run(x, ids: torch.Tensor, cents, K: int, want_inertia: bool):
    ids = _ensure_contig(ids, "ids")
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    B, N = ids.shape
    dev = ids.device
    if want_inertia:
        x = _ensure_contig(x, "x")
        cents = _ensure_contig(cents, "centroids")
        if x.dim() != 3 or cents.dim() != 3 or x.shape[:2] != (B, N) or \
                cents.shape[0] != B or cents.shape[2] != x.shape[2]:
            raise RuntimeError("assigned_inertia: shapes must be x (B,N,D), "
                               "ids (B,N), centroids (B,K,D)")
        if cents.dtype != x.dtype:
            raise RuntimeError("assigned_inertia: x and centroids must share a dtype")
        D = x.shape[2]
        dt = _lib.dtype_code(x.dtype)
    else:
        D, dt = 1, _lib.FKC_F32
    inertia = torch.empty(B, dtype=torch.float64, device=dev) if want_inertia else None
    empty = torch.empty(B, dtype=torch.int32, device=dev)
    ws = _lib.workspace(_lib.lib.fkc_quality_workspace_bytes(B, N, K), dev)
    _lib.check(_lib.lib.fkc_assigned_inertia(
        _lib.ptr(x) if want_inertia else None, _lib.ptr(cents) if want_inertia else None,
        ids.data_ptr(), B, N, K, D, dt, _lib.ptr(inertia), empty.data_ptr(),
        ws.data_ptr(), ws.numel(), _lib.stream_of(ids)), "assigned_inertia")
    return inertia, empty


def assigned_inertia(x: torch.Tensor, ids: torch.Tensor, cents: torch.Tensor) -> float:
    """sum over all (b, n) of ||x[b,n] - cents[b, ids[b,n]]||^2 (fp64 total)."""
    inertia, _ = _run(x, ids, cents, cents.shape[1], True)
    return float(inertia.sum().item())


def empty_clusters(ids: torch.Tensor, K: int) -> int:
    """Number of (b, k), k < K, that no point carries (summed over b)."""
    _, empty = _run(None, ids, None, int(K), False)
    return int(empty.sum().item())


def assign_with_fixed_evaluator(x: torch.Tensor, cents: torch.Tensor) -> torch.Tensor:
    """Labels of x against final centroids, with explicit x_sq and c_sq."""
    return euclid_assign(x, cents.contiguous(), row_sqnorm(x), c_sq=row_sqnorm(cents))


def evaluate(x: torch.Tensor, cents: torch.Tensor) -> Dict[str, object]:
    """Re-assign with `cents`, then inertia and empty-cluster count of those
    labels (what quality_compare.py reports per run)."""
    ids = assign_with_fixed_evaluator(x, cents)
    inertia, empty = _run(x, ids, cents, cents.shape[1], True)
    return {"ids": ids, "inertia": float(inertia.sum().item()),
            "inertia_per_batch": inertia.cpu().tolist(),
            "empty_clusters": int(empty.sum().item())}
