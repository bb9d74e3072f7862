"""torch-CPU restatement of the reference's Euclidean Lloyd loop: the CPU
baseline that bench.py times beside the GPU path.

TEST INFRASTRUCTURE ONLY.  Only tests/ and bench.py's cpu_baseline leg may
import this module; the product path (flash_kmeans_cuda) never routes through
it.

The reference has no CPU path (flash_kmeans_cuda/ops.py:23-24 and
kmeans.py:141 refuse host tensors), so this is the same loop written with
torch's CPU operators, step for step:
  x_sq        fp32 row norms of x, once per call (kmeans.py:146-151)
  c_sq        fp32 row norms of the centroids, every iteration (kmeans.py:94)
  assign      argmin_k x_sq + c_sq - 2 <x, c> with fp32 products and sums
              (torch.matmul on fp32 copies), the first minimum winning ties
              (torch.argmin; assign_common.cuh:20-28); rows in chunks so one
              chunk's (rows x K) distance block stays near 256 MiB
  update      stable torch.sort of the labels (ops.py:89), fp32 sums of the
              rows in sorted order (index_add_) and int counts (bincount)
              (ops.py:92-111, update_sorted.cu:77-115)
  finalize    sums / counts in fp32, cast to the storage dtype, the old
              centroid kept for empty clusters (ops.py:115-130,
              update_finalize.cu:59-64)
  shift       (new.float() - old.float()).norm(dim=-1).max(), stop once
              < tol (kmeans.py:104, 190)
The labels returned are those of the last assignment, made against the
centroids before the last update (kmeans.py:179-195).
"""

from __future__ import annotations

import torch

CHUNK_BYTES = 256 << 20


def _assign(xf: torch.Tensor, x_sq: torch.Tensor, cf: torch.Tensor) -> torch.Tensor:
    """(N, D) fp32 points, (N,) fp32 norms, (K, D) fp32 centroids ->
    int64 (N,) nearest centroid (first minimum on ties)."""
    N = xf.shape[0]
    K = cf.shape[0]
    c_sq = (cf * cf).sum(-1)
    rows = max(1, min(N, CHUNK_BYTES // (4 * max(K, 1))))
    out = torch.empty(N, dtype=torch.int64)
    ct = cf.t().contiguous()
    for s in range(0, N, rows):
        # (-2 <x, c> + c_sq) + x_sq, in place on the product (the doubling is
        # exact, so this ranks as x_sq + c_sq - 2 <x, c> up to fp32 rounding
        # of the two additions)
        dist = xf[s:s + rows] @ ct
        dist.mul_(-2.0).add_(c_sq[None, :]).add_(x_sq[s:s + rows, None])
        out[s:s + rows] = torch.argmin(dist, dim=1)
    return out


def lloyd_step(x: torch.Tensor, x_sq: torch.Tensor, c: torch.Tensor):
    """One iteration for every batch row: (new centroids in c.dtype, labels
    int64 (B, N)).  x (B, N, D) and c (B, K, D) are CPU tensors of one
    storage dtype; x_sq (B, N) fp32."""
    B, N, D = x.shape
    K = c.shape[1]
    ids = torch.empty((B, N), dtype=torch.int64)
    new = torch.empty_like(c)
    for b in range(B):
        xf = x[b].float()
        cf = c[b].float()
        ids[b] = _assign(xf, x_sq[b], cf)
        sorted_ids, perm = torch.sort(ids[b], stable=True)
        sums = torch.zeros((K, D), dtype=torch.float32)
        sums.index_add_(0, sorted_ids, xf[perm])
        counts = torch.bincount(sorted_ids, minlength=K)
        mean = sums / counts.clamp(min=1).to(torch.float32)[:, None]
        new[b] = torch.where(counts[:, None] > 0, mean, cf).to(c.dtype)
    return new, ids


def kmeans(x: torch.Tensor, init: torch.Tensor, max_iters: int, tol: float = 0.0):
    """batch_kmeans_Euclid on the CPU with explicit initial centroids:
    (labels int64 (B, N), centroids (B, K, D) in x.dtype, iterations run)."""
    x = x.contiguous()
    x_sq = (x.float() ** 2).sum(-1)
    cur = init.clone()
    ids = torch.zeros(x.shape[:2], dtype=torch.int64)
    n = 0
    for it in range(max_iters):
        new, ids = lloyd_step(x, x_sq, cur)
        n = it + 1
        if tol > 0:
            shift = float((new.float() - cur.float()).norm(dim=-1).max())
            cur = new
            if shift < tol:
                break
        else:
            cur = new
    return ids, cur, n
