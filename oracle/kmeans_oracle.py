"""CPU restatement of the reference's Euclidean Lloyd path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the checker
or the CPU baseline; the product path (flash_kmeans_cuda) never routes through
it and fails loudly when its HIP library is missing.

Reference (OpsiClear/flash-kmeans-cuda) semantics restated here:
  assign      flash_kmeans_cuda/kmeans.py:94-95, ops.py:30-55,
              csrc/assign/assign_common.cuh:15-36 (strict-< running minimum:
              the lowest centroid index wins exact ties),
              csrc/assign/assign_safe.cu:55-80, assign_sm80.cu:437-441
  label_sort  flash_kmeans_cuda/ops.py:89 (torch.sort of the labels along N)
  update      ops.py:92-111, csrc/update/update_sorted.cu:77-115, 151-185
              (runs of equal sorted labels; labels outside [0,K) skipped)
  finalize    ops.py:115-130, csrc/update/update_finalize.cu:39-66
  loop        flash_kmeans_cuda/kmeans.py:73-195
  quality     benchmarks/quality_compare.py:69-116 (assigned inertia with
              fp32 differences and squares summed in fp64; empty clusters
              over the flattened labels; sampled nearest-centroid inertia)

Arithmetic choices (documented, not the reference's exact rounding):
  * assign ranks exact squared distances: x_sq + c_sq - 2<x,c> evaluated in
    float64 from the stored element values ("f64" precision, the parity
    oracle), or in float32 with BLAS ("f32", the CPU baseline, mirroring a
    torch-CPU fp32 path).  Ties go to the lowest index (numpy argmin).
  * update sums rows in float64, then rounds the sums to float32 once (the
    reference accumulates fp32 with atomics in scheduling order).
  * finalize divides the float32 sums by the count in float32 (IEEE) and
    rounds to the storage dtype with round-to-nearest-even.
Pins for every function live in tests/test_oracle_pins.py (brute force,
scipy/numpy library routines, known answers, planted-mistake checks).

Element types: "f64", "f32", "f16" (numpy float16) and "bf16" (uint16 raw
bits; numpy has no bfloat16).
"""

from __future__ import annotations

import numpy as np

DTYPES = ("f64", "f32", "f16", "bf16")


# ----------------------------------------------------------------- dtypes
def to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    """Storage array -> float32 values (exact for f32/f16/bf16)."""
    if dtype == "bf16":
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    return np.asarray(a).astype(np.float32)


def to_f64(a: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f64":
        return np.asarray(a, dtype=np.float64)
    return to_f32(a, dtype).astype(np.float64)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bits; NaN -> 0x7FC0."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, 0x7FC0, r)
    return r.astype(np.uint16)


def from_f32(f: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values -> storage array of `dtype` (round to nearest even)."""
    f = np.asarray(f, dtype=np.float32)
    if dtype == "f32":
        return f.copy()
    if dtype == "f16":
        return f.astype(np.float16)
    if dtype == "bf16":
        return f32_to_bf16_bits(f)
    if dtype == "f64":
        return f.astype(np.float64)
    raise ValueError(dtype)


def storage_dtype(dtype: str):
    return {"f64": np.float64, "f32": np.float32, "f16": np.float16,
            "bf16": np.uint16}[dtype]


# ----------------------------------------------------------------- norms
def row_sqnorm(a: np.ndarray, dtype: str) -> np.ndarray:
    """sum_d value^2 per row, float64 (kmeans.py:94, kmeans.py:151)."""
    v = to_f64(a, dtype)
    return np.einsum("...d,...d->...", v, v)


# ----------------------------------------------------------------- assign
def assign(x: np.ndarray, c: np.ndarray, dtype: str, *, precision: str = "f64",
           chunk: int = 8192) -> np.ndarray:
    """Nearest centroid per point, lowest index on exact ties.

    x: (B,N,D), c: (B,K,D) storage arrays.  Returns int64 (B,N).
    Follows assign_common.cuh:23-28 (strict < keeps the first minimum) and the
    distance of assign_common.cuh:33-36 / assign_sm80.cu:437-441 (x_sq is a
    per-row constant, so both rank identically).
    """
    x = np.asarray(x)
    c = np.asarray(c)
    B, N, D = x.shape
    K = c.shape[1]
    ft = np.float64 if precision == "f64" else np.float32
    out = np.empty((B, N), dtype=np.int64)
    for b in range(B):
        cb = to_f64(c[b], dtype).astype(ft)
        c_sq = np.einsum("kd,kd->k", cb, cb)
        for s in range(0, N, chunk):
            xb = to_f64(x[b, s:s + chunk], dtype).astype(ft)
            x_sq = np.einsum("nd,nd->n", xb, xb)
            dist = x_sq[:, None] + c_sq[None, :] - 2.0 * (xb @ cb.T)
            out[b, s:s + chunk] = np.argmin(dist, axis=1)
    return out


def distances(x: np.ndarray, c: np.ndarray, dtype: str, ids: np.ndarray) -> np.ndarray:
    """Exact float64 squared distance of each point to centroid ids[b,n]."""
    xv = to_f64(x, dtype)
    cv = to_f64(c, dtype)
    chosen = np.take_along_axis(cv, ids[..., None].astype(np.int64), axis=1)
    return ((xv - chosen) ** 2).sum(-1)


# ----------------------------------------------------------------- sort
def sort_keys(ids: np.ndarray, K: int) -> np.ndarray:
    """Labels outside [0,K) sort as K (after every valid label)."""
    ids = np.asarray(ids)
    return np.where((ids >= 0) & (ids < K), ids, K).astype(np.int64)


def label_sort(ids: np.ndarray, K: int):
    """Stable sort of each batch row of labels -> (sorted_ids, perm), int32.

    Restates the label sort of ops.py:89 with a stable order (equal labels in
    index order); numpy's stable argsort is the textbook routine used.
    """
    ids = np.asarray(ids)
    keys = sort_keys(ids, K)
    perm = np.argsort(keys, axis=-1, kind="stable")
    sorted_ids = np.take_along_axis(ids, perm, axis=-1)
    return sorted_ids.astype(np.int32), perm.astype(np.int32)


# ----------------------------------------------------------------- update
def update_sorted(x_rows: np.ndarray, ids_sorted: np.ndarray, K: int, dtype: str):
    """Run-wise sums/counts over label-sorted rows (update_sorted.cu:77-115).

    x_rows: (B,N,D) rows already in sorted order.  Returns (sums float64
    (B,K,D), counts int64 (B,K)); labels outside [0,K) are skipped.
    """
    xv = to_f64(x_rows, dtype)
    ids_sorted = np.asarray(ids_sorted).astype(np.int64)
    B, N, D = xv.shape
    sums = np.zeros((B, K, D), dtype=np.float64)
    counts = np.zeros((B, K), dtype=np.int64)
    for b in range(B):
        s = ids_sorted[b]
        if N == 0:
            continue
        starts = np.flatnonzero(np.concatenate(([True], s[1:] != s[:-1])))
        ends = np.concatenate((starts[1:], [N]))
        run_sums = np.add.reduceat(xv[b], starts, axis=0)
        for r, (st, en) in enumerate(zip(starts, ends)):
            k = s[st]
            if 0 <= k < K:
                sums[b, k] += run_sums[r]
                counts[b, k] += en - st
    return sums, counts


def update_sorted_indexed(x: np.ndarray, perm: np.ndarray, ids_sorted: np.ndarray,
                          K: int, dtype: str):
    """Same accumulation reading row perm[p] for sorted position p
    (update_sorted.cu:118-186)."""
    rows = np.take_along_axis(np.asarray(x), np.asarray(perm).astype(np.int64)[..., None], axis=1)
    return update_sorted(rows, ids_sorted, K, dtype)


# ----------------------------------------------------------------- finalize
def finalize(sums: np.ndarray, counts: np.ndarray, old: np.ndarray, dtype: str) -> np.ndarray:
    """new = count > 0 ? cast(sum / count) : old (update_finalize.cu:59-64)."""
    counts = np.asarray(counts)
    if dtype == "f64":
        mean = np.asarray(sums, dtype=np.float64) / np.maximum(counts, 1)[..., None]
        return np.where(counts[..., None] > 0, mean, old)
    s32 = np.asarray(sums, dtype=np.float32)
    c32 = np.maximum(counts, 1).astype(np.float32)
    mean = from_f32(s32 / c32[..., None], dtype)
    return np.where(counts[..., None] > 0, mean, np.asarray(old))


def shift(new: np.ndarray, old: np.ndarray, dtype: str) -> float:
    """max over every (b,k) of ||new - old||_2, in float32 as the reference
    computes it: `(new.float() - old.float()).norm(dim=-1).max()`
    (kmeans.py:104), the loop stopping once it is < tol (kmeans.py:190).
    The difference, squares, row sums and square root are float32 (numpy's
    pairwise float32 sum; the reference's reduction order differs by a few
    ulp at most)."""
    d = to_f32(new, dtype) - to_f32(old, dtype)
    if d.size == 0:
        return 0.0
    sq = np.sum(d * d, axis=-1, dtype=np.float32)
    return float(np.sqrt(sq).max())


# ----------------------------------------------------------------- loop
def lloyd_step(x, c, K, dtype, *, precision="f64"):
    """One iteration of kmeans.py:73-105: (new_centroids, ids, counts, sums)."""
    ids = assign(x, c, dtype, precision=precision)
    sorted_ids, perm = label_sort(ids, K)
    sums, counts = update_sorted_indexed(x, perm, sorted_ids, K, dtype)
    new = finalize(sums, counts, c, dtype)
    return new, ids, counts, sums


def kmeans(x: np.ndarray, K: int, max_iters: int, tol: float, init: np.ndarray,
           dtype: str, *, precision: str = "f64"):
    """batch_kmeans_Euclid (kmeans.py:108-195) with explicit initial centroids.

    Returns (ids int64 (B,N) from the last assignment, centroids storage
    (B,K,D), n_iters).  With tol <= 0 it runs exactly max_iters iterations;
    otherwise it stops after the first iteration whose shift < tol.
    """
    x = np.asarray(x)
    cur = np.array(init, copy=True)
    B, N, _ = x.shape
    ids = np.zeros((B, N), dtype=np.int64)
    n = 0
    for it in range(max_iters):
        new, ids, _, _ = lloyd_step(x, cur, K, dtype, precision=precision)
        n = it + 1
        if tol > 0 and shift(new, cur, dtype) < tol:
            cur = new
            break
        cur = new
    return ids, cur, n


def assigned_inertia(x: np.ndarray, ids: np.ndarray, c: np.ndarray, dtype: str) -> np.ndarray:
    """Per batch row: sum over points and features of (x - c[id])^2, the
    difference and the square in float32, the total in float64
    (quality_compare.py:69-83, `diff.square().sum(dtype=torch.float64)`).
    Rows labelled outside [0,K) add nothing."""
    xf = to_f32(x, dtype)
    cf = to_f32(c, dtype)
    B, N, D = xf.shape
    K = cf.shape[1]
    out = np.zeros(B, dtype=np.float64)
    for b in range(B):
        ib = np.asarray(ids[b]).astype(np.int64)
        ok = (ib >= 0) & (ib < K)
        diff = (xf[b][ok] - cf[b][ib[ok]]).astype(np.float32)
        sq = (diff * diff).astype(np.float32)
        out[b] = sq.astype(np.float64).sum()
    return out


def empty_clusters(ids: np.ndarray, K: int) -> int:
    """Number of k in [0,K) that no point of any batch row carries: the
    labels of all rows are counted into one histogram of K bins
    (quality_compare.py:86-88, `bincount(ids.reshape(-1), minlength=K) == 0`),
    so at B > 1 a k is empty only when every row leaves it empty.  Labels
    outside [0,K) are ignored (the reference's bincount rejects negative
    labels and grows extra bins past K-1)."""
    flat = np.asarray(ids).astype(np.int64).reshape(-1)
    flat = flat[(flat >= 0) & (flat < K)]
    return int((np.bincount(flat, minlength=K) == 0).sum())


def sample_exact_inertia(x: np.ndarray, c: np.ndarray, sample_idx: np.ndarray,
                         dtype: str) -> float:
    """Inertia of a point sample against the nearest centroid, over every
    batch row (quality_compare.py:91-116, `_sample_exact_inertia`): for each
    sampled index n (the same indices in every row) the distance
    x_sq + c_sq - 2<x,c> is formed in float32 from float32 products, its
    minimum over k is clamped at 0, and the minima are summed in float64.
    The reference draws sample_idx with torch.randperm on the device; here it
    is an argument."""
    xs = to_f32(np.asarray(x)[:, np.asarray(sample_idx, dtype=np.int64)], dtype)
    cf = to_f32(c, dtype)
    total = 0.0
    for b in range(xs.shape[0]):
        x_sq = np.sum(xs[b] * xs[b], axis=-1, dtype=np.float32)
        c_sq = np.sum(cf[b] * cf[b], axis=-1, dtype=np.float32)
        cross = (xs[b] @ cf[b].T).astype(np.float32)
        dist = (x_sq[:, None] + c_sq[None, :]) - np.float32(2.0) * cross
        total += float(np.maximum(dist.min(axis=-1), np.float32(0.0))
                       .astype(np.float64).sum())
    return total
