"""Drop-in for the reference's compiled `_C` module, over the C ABI.

Same four functions, argument names and in/out conventions as
flash_kmeans_cuda/csrc/bindings.cpp:107-127 of the reference:

  euclid_assign(x, centroids, x_sq, c_sq, out=None) -> (B,N) int32
  centroid_update_sorted(x_sorted, cluster_ids_sorted, centroid_sums, centroid_counts)
  centroid_update_sorted_indexed(x, sorted_idx, cluster_ids_sorted, centroid_sums, centroid_counts)
  centroid_finalize(centroid_sums, centroid_counts, old_centroids, out=None) -> (B,K,D)

The update functions add into the given sums/counts without zeroing them,
as the reference's _C functions do.  Argument checks raise RuntimeError, as
the reference's TORCH_CHECKs do (assign_sm80.cu:712-731,
update_sorted.cu:196-206, 253-277, update_finalize.cu:76-83).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _cuda(t: torch.Tensor, name: str) -> None:
    _require(t.is_cuda, f"{name} must be a CUDA tensor")


def _contig(*ts: torch.Tensor) -> None:
    _require(all(t.is_contiguous() for t in ts), "all tensors must be contiguous")


def euclid_assign(x: torch.Tensor, centroids: torch.Tensor, x_sq: torch.Tensor,
                  c_sq: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Compute argmin_k ||x - c_k||^2 for each point. Returns (B,N) int32."""
    _cuda(x, "x")
    _cuda(centroids, "centroids")
    _require(x.dim() == 3 and centroids.dim() == 3,
             "x and centroids must be 3D (B,N,D)/(B,K,D)")
    _require(x.dtype == centroids.dtype, "x and centroids must share dtype")
    _require((x_sq is None or x_sq.dtype == torch.float32)
             and c_sq.dtype == torch.float32, "x_sq and c_sq must be fp32")
    B, N, D = x.shape
    K = centroids.shape[1]
    _require(centroids.shape[0] == B and centroids.shape[2] == D,
             "centroids must be (B, K, D) matching x")
    _require(c_sq.numel() == B * K, "c_sq must be (B, K)")
    if out is None:
        out = torch.empty((B, N), dtype=torch.int32, device=x.device)
    _require(out.dtype == torch.int32, "out must be int32")
    _require(out.dim() == 2 and out.shape[0] == B and out.shape[1] == N,
             "out must be (B, N) int32")
    _contig(x, centroids, c_sq, out)
    xsq_ptr = None
    if x_sq is not None and x_sq.numel() == B * N:
        _contig(x_sq)
        xsq_ptr = x_sq.data_ptr()
    dt = _lib.dtype_code(x.dtype)
    need = _lib.lib.fkc_euclid_assign_workspace_bytes(B, N, K, D, dt)
    if need == 0:
        _lib.check(_lib.lib.fkc_euclid_assign(
            x.data_ptr(), centroids.data_ptr(), xsq_ptr, c_sq.data_ptr(),
            out.data_ptr(), B, N, K, D, dt, _lib.stream_of(x)),
            "euclid_assign")
    else:
        # Shapes whose point tiles alone cannot fill the GPU slice K across
        # workgroups; the partial winners live in a stream-ordered workspace.
        ws = _lib.workspace(need, x.device)
        _lib.check(_lib.lib.fkc_euclid_assign_ws(
            x.data_ptr(), centroids.data_ptr(), xsq_ptr, c_sq.data_ptr(),
            out.data_ptr(), B, N, K, D, dt, ws.data_ptr(), ws.numel(),
            _lib.stream_of(x)),
            "euclid_assign")
    return out


def _check_update(x, ids, sums, counts, what):
    _cuda(x, "x")
    _require(x.dim() == 3, "x must be (B, N, D)")
    _require(ids.dtype == torch.int32, "cluster_ids must be int32")
    _require(sums.dtype == torch.float32, "centroid_sums must be fp32")
    _require(counts.dtype == torch.int32, "centroid_counts must be int32")
    B, N, D = x.shape
    _require(ids.dim() == 2 and ids.shape[0] == B and ids.shape[1] == N,
             "cluster_ids_sorted must be (B, N)")
    _require(sums.dim() == 3 and sums.shape[0] == B and sums.shape[2] == D,
             "centroid_sums must be (B, K, D)")
    K = sums.shape[1]
    _require(counts.numel() == B * K, "centroid_counts must be (B, K)")
    _contig(x, ids, sums, counts)
    return B, N, K, D


def centroid_update_sorted(x_sorted: torch.Tensor, cluster_ids_sorted: torch.Tensor,
                           centroid_sums: torch.Tensor, centroid_counts: torch.Tensor) -> None:
    """Sorted-run centroid accumulator (in-place into sums/counts)."""
    B, N, K, D = _check_update(x_sorted, cluster_ids_sorted, centroid_sums,
                               centroid_counts, "centroid_update_sorted")
    ws = _lib.workspace(_lib.lib.fkc_update_workspace_bytes(B, N, D), x_sorted.device)
    _lib.check(_lib.lib.fkc_centroid_update_sorted(
        x_sorted.data_ptr(), cluster_ids_sorted.data_ptr(), centroid_sums.data_ptr(),
        centroid_counts.data_ptr(), B, N, K, D, _lib.dtype_code(x_sorted.dtype),
        ws.data_ptr(), ws.numel(), _lib.stream_of(x_sorted)), "centroid_update_sorted")


def centroid_update_sorted_indexed(x: torch.Tensor, sorted_idx: torch.Tensor,
                                   cluster_ids_sorted: torch.Tensor,
                                   centroid_sums: torch.Tensor,
                                   centroid_counts: torch.Tensor) -> None:
    """Sorted-run accumulator reading x rows through sorted_idx."""
    B, N, K, D = _check_update(x, cluster_ids_sorted, centroid_sums,
                               centroid_counts, "centroid_update_sorted_indexed")
    _require(sorted_idx.dtype == torch.int32, "sorted_idx must be int32")
    _require(sorted_idx.dim() == 2 and sorted_idx.shape[0] == B and sorted_idx.shape[1] == N,
             "sorted_idx must be (B, N)")
    _contig(sorted_idx)
    ws = _lib.workspace(_lib.lib.fkc_update_workspace_bytes(B, N, D), x.device)
    _lib.check(_lib.lib.fkc_centroid_update_sorted_indexed(
        x.data_ptr(), sorted_idx.data_ptr(), cluster_ids_sorted.data_ptr(),
        centroid_sums.data_ptr(), centroid_counts.data_ptr(), B, N, K, D,
        _lib.dtype_code(x.dtype), ws.data_ptr(), ws.numel(), _lib.stream_of(x)),
        "centroid_update_sorted_indexed")


def centroid_finalize(centroid_sums: torch.Tensor, centroid_counts: torch.Tensor,
                      old_centroids: torch.Tensor,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sums/counts -> new centroids; keep old for empty clusters."""
    _cuda(centroid_sums, "centroid_sums")
    _require(centroid_sums.dtype == torch.float32, "sums must be fp32")
    _require(centroid_counts.dtype == torch.int32, "counts must be int32")
    if out is None:
        out = torch.empty_like(old_centroids)
    _require(old_centroids.dtype == out.dtype, "old and new centroids must share dtype")
    _require(centroid_sums.dim() == 3, "centroid_sums must be (B, K, D)")
    B, K, D = centroid_sums.shape
    _require(tuple(old_centroids.shape) == (B, K, D) and tuple(out.shape) == (B, K, D),
             "old/new centroids must be (B, K, D) like centroid_sums")
    _require(centroid_counts.numel() == B * K, "counts must be (B, K)")
    _contig(centroid_sums, centroid_counts, old_centroids, out)
    _lib.check(_lib.lib.fkc_centroid_finalize(
        centroid_sums.data_ptr(), centroid_counts.data_ptr(), old_centroids.data_ptr(),
        out.data_ptr(), B, K, D, _lib.dtype_code(out.dtype), _lib.stream_of(out)),
        "centroid_finalize")
    return out
