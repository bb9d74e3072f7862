"""Thin Python wrappers around the gfx950 kernels (mirror of the reference's
flash_kmeans_cuda/ops.py:30-130, same names, arguments and errors).

Differences, all internal: the labels are sorted by this library's stable
radix sort instead of torch.sort (ops.py:89), the centroid update always
reads x through the sorted permutation (no gathered copy of x), and c_sq is
computed by a HIP kernel.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _C, _lib


def _ensure_contig(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor (got {t.device})")
    if not t.is_contiguous():
        return t.contiguous()
    return t


def row_sqnorm(t: torch.Tensor) -> torch.Tensor:
    """(..., D) -> (...) fp32 sum of squares of the stored values."""
    t = _ensure_contig(t, "t")
    D = t.shape[-1]
    out = torch.empty(t.shape[:-1], dtype=torch.float32, device=t.device)
    rows = out.numel()
    _lib.check(_lib.lib.fkc_row_sqnorm(t.data_ptr(), out.data_ptr(), rows, D,
                                       _lib.dtype_code(t.dtype), _lib.stream_of(t)),
               "row_sqnorm")
    return out


def euclid_assign(
    x: torch.Tensor,
    centroids: torch.Tensor,
    x_sq: torch.Tensor,
    c_sq: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Assign each point to its nearest centroid (Euclidean).

    Args:
        x: (B, N, D) fp16/bf16/fp32, CUDA.
        centroids: (B, K, D) same dtype as x.
        x_sq: (B, N) fp32 ||x||^2 per point (read only by the fp32 route).
        c_sq: (B, K) fp32 ||c||^2 per centroid; computed if None.
        out: optional (B, N) int32 buffer to write into.

    Returns:
        cluster_ids: (B, N) int32.
    """
    x = _ensure_contig(x, "x")
    centroids = _ensure_contig(centroids, "centroids")
    x_sq = _ensure_contig(x_sq, "x_sq").to(torch.float32)
    if c_sq is None:
        c_sq = row_sqnorm(centroids)
    c_sq = _ensure_contig(c_sq, "c_sq").to(torch.float32)
    return _C.euclid_assign(x, centroids, x_sq, c_sq, out)


def label_sort(cluster_ids: torch.Tensor, K: int, *,
               workspace: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stable sort of (B, N) int32 labels along N -> (sorted_ids, perm) int32.

    Labels outside [0, K) sort after every valid label, in index order.
    workspace: optional caller-owned uint8 CUDA tensor of at least
    fkc_label_sort_workspace_bytes(B, N, K) bytes, 256-byte aligned; after
    the call its first int32 counts the tiles whose bounded look-back wait ran
    out and that recounted their prefix instead (a diagnostic: the output is
    valid either way).
    """
    cluster_ids = _ensure_contig(cluster_ids, "cluster_ids")
    if cluster_ids.dtype != torch.int32:
        cluster_ids = cluster_ids.to(torch.int32)
    B, N = cluster_ids.shape
    sorted_ids = torch.empty_like(cluster_ids)
    perm = torch.empty_like(cluster_ids)
    need = _lib.lib.fkc_label_sort_workspace_bytes(B, N, K)
    if workspace is None:
        ws = _lib.workspace(need, cluster_ids.device)
    else:
        if (workspace.dtype != torch.uint8 or not workspace.is_contiguous()
                or workspace.device != cluster_ids.device or workspace.numel() < need):
            raise ValueError(f"label_sort: workspace must be a contiguous uint8 tensor of "
                             f">= {need} bytes on {cluster_ids.device}")
        ws = workspace
    _lib.check(_lib.lib.fkc_label_sort(
        cluster_ids.data_ptr(), sorted_ids.data_ptr(), perm.data_ptr(), B, N, K,
        ws.data_ptr(), ws.numel(), _lib.stream_of(cluster_ids)), "label_sort")
    return sorted_ids, perm


def centroid_update_sorted(
    x: torch.Tensor,
    cluster_ids: torch.Tensor,
    K: int,
    *,
    sums_out: Optional[torch.Tensor] = None,
    counts_out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sort cluster_ids along N, then accumulate per-cluster sums/counts.

    Args:
        x: (B, N, D) compute dtype.
        cluster_ids: (B, N) int32 (any order).
        K: number of clusters.
        sums_out: optional (B, K, D) fp32 (zeroed here).
        counts_out: optional (B, K) int32 (zeroed here).

    Returns:
        (centroid_sums, centroid_counts).
    """
    x = _ensure_contig(x, "x")
    cluster_ids = _ensure_contig(cluster_ids, "cluster_ids")
    if cluster_ids.dtype != torch.int32:
        cluster_ids = cluster_ids.to(torch.int32)
    B, N, D = x.shape
    sorted_ids, perm = label_sort(cluster_ids, K)
    if sums_out is None:
        sums_out = torch.zeros((B, K, D), device=x.device, dtype=torch.float32)
    else:
        sums_out.zero_()
    if counts_out is None:
        counts_out = torch.zeros((B, K), device=x.device, dtype=torch.int32)
    else:
        counts_out.zero_()
    _C.centroid_update_sorted_indexed(x, perm, sorted_ids, sums_out, counts_out)
    return sums_out, counts_out


def centroid_finalize(
    centroid_sums: torch.Tensor,
    centroid_counts: torch.Tensor,
    old_centroids: torch.Tensor,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """new[b,k] = sums[b,k] / counts[b,k] if counts > 0 else old_centroids[b,k].

    Casts back to old_centroids.dtype.
    """
    return _C.centroid_finalize(
        centroid_sums.contiguous(),
        centroid_counts.contiguous(),
        old_centroids.contiguous(),
        out,
    )
