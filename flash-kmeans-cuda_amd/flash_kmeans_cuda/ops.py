"""Per-operation entry points of the K-Means hot path.

These keep the reference's public names, argument meaning, return values and
error classes (flash_kmeans_cuda/ops.py:30-130): `euclid_assign`,
`centroid_update_sorted` and `centroid_finalize`, plus `label_sort` and
`row_sqnorm`, which expose two steps the reference does with torch ops.
Host tensors raise ValueError; everything else is checked by the `_C` layer
and by the C ABI underneath (RuntimeError).

Internally the labels are ordered by this library's stable radix sort (the
reference calls torch.sort, ops.py:89), the update always reads x through the
sorted permutation (no gathered copy of x is made), and c_sq comes from a HIP
kernel rather than a torch expression.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _C, _lib


def _gpu_dense(name: str, t: torch.Tensor) -> torch.Tensor:
    """`t` itself when it is a dense GPU tensor, a dense copy when it is a
    strided view; host tensors are refused with ValueError (as the reference
    refuses them, ops.py:23-24)."""
    if t.device.type != "cuda":
        raise ValueError(f"{name}: expected a tensor on a GPU device, found one on {t.device}")
    return t if t.is_contiguous() else t.contiguous()


def _as_i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def row_sqnorm(t: torch.Tensor) -> torch.Tensor:
    """Squared Euclidean norm of every row of a (..., D) tensor, summed in
    fp32 over the stored element values; shape (...)."""
    t = _gpu_dense("t", t)
    out = torch.empty(t.shape[:-1], dtype=torch.float32, device=t.device)
    _lib.check(_lib.lib.fkc_row_sqnorm(t.data_ptr(), out.data_ptr(), out.numel(),
                                       t.shape[-1], _lib.dtype_code(t.dtype),
                                       _lib.stream_of(t)), "row_sqnorm")
    return out


def euclid_assign(
    x: torch.Tensor,
    centroids: torch.Tensor,
    x_sq: torch.Tensor,
    c_sq: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Label of the closest centroid for every point.

    x (B, N, D) and centroids (B, K, D) share one dtype: fp16, bf16 or fp32.
    x_sq (B, N) and c_sq (B, K) hold the fp32 squared row norms; x_sq only
    matters on the fp32 route (the matrix-core route ranks by
    c_sq - 2<x, c>), and c_sq is computed here when omitted.  The labels,
    int32 (B, N), are written to `out` when given; equal distances go to the
    lower centroid index.
    """
    x = _gpu_dense("x", x)
    centroids = _gpu_dense("centroids", centroids)
    x_sq = _gpu_dense("x_sq", x_sq).float()
    c_sq = row_sqnorm(centroids) if c_sq is None else _gpu_dense("c_sq", c_sq).float()
    return _C.euclid_assign(x, centroids, x_sq, c_sq, out)


def label_sort(cluster_ids: torch.Tensor, K: int, *,
               workspace: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stable sort of (B, N) int32 labels along N -> (sorted_ids, perm) int32.

    Labels outside [0, K) sort after every valid label, in index order.
    workspace: optional caller-owned uint8 CUDA tensor of at least
    fkc_label_sort_workspace_bytes(B, N, K) bytes, 256-byte aligned; after
    the call its first int32 counts the sort tiles whose bounded wait (on
    earlier tiles, or at the first pass's row barrier) ran out and that
    recounted from the pass's input instead (a diagnostic: the output is
    valid either way).
    """
    cluster_ids = _as_i32(_gpu_dense("cluster_ids", cluster_ids))
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
    """Per-cluster fp32 row sums (B, K, D) and int32 counts (B, K) of x under
    labels given in any order.

    The labels are sorted first; the sums are taken over each label's rows
    in that order.  Buffers passed as sums_out / counts_out are cleared and
    filled; otherwise new ones are returned.
    """
    x = _gpu_dense("x", x)
    cluster_ids = _as_i32(_gpu_dense("cluster_ids", cluster_ids))
    B, N, D = x.shape
    sorted_ids, perm = label_sort(cluster_ids, K)
    sums = (torch.zeros((B, K, D), device=x.device, dtype=torch.float32)
            if sums_out is None else sums_out.zero_())
    counts = (torch.zeros((B, K), device=x.device, dtype=torch.int32)
              if counts_out is None else counts_out.zero_())
    _C.centroid_update_sorted_indexed(x, perm, sorted_ids, sums, counts)
    return sums, counts


def centroid_finalize(
    centroid_sums: torch.Tensor,
    centroid_counts: torch.Tensor,
    old_centroids: torch.Tensor,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """New centroids in old_centroids' dtype: the mean sums / counts for
    clusters with points, the old centroid for empty ones (the mean is an
    IEEE fp32 division rounded to nearest)."""
    dense = [t if t.is_contiguous() else t.contiguous()
             for t in (centroid_sums, centroid_counts, old_centroids)]
    return _C.centroid_finalize(*dense, out)
