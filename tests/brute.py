"""Pure-Python brute-force restatements for tiny inputs (independent of the
oracle's numpy code paths).  Used to pin the oracle; never imported by the
product package."""

from __future__ import annotations

import math
import struct


def f32(v: float) -> float:
    """Round a Python float to the nearest float32."""
    return struct.unpack("<f", struct.pack("<f", v))[0]


def bf16_bits_rne(v: float) -> int:
    """float32 -> bfloat16 bits by the IEEE round-to-nearest-even rule,
    computed on the rational value rather than by bit tricks."""
    (u,) = struct.unpack("<I", struct.pack("<f", v))
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return 0x7FC0
    if (u & 0x7FFFFFFF) == 0x7F800000:
        return u >> 16
    sign = -1.0 if u >> 31 else 1.0
    a = abs(struct.unpack("<f", struct.pack("<I", u))[0])
    if a == 0.0:
        return u >> 16
    # candidates: truncation and next bf16 up (in magnitude)
    lo = (u & 0x7FFFFFFF) >> 16
    hi = lo + 1
    def val(bits):
        # 0x7F80 stands for 2^128, the next step past the largest finite
        # value: rounding up to it yields infinity, as IEEE overflow does.
        if (bits & 0x7FFF) >= 0x7F80:
            return 2.0 ** 128
        return struct.unpack("<f", struct.pack("<I", (bits & 0x7FFF) << 16))[0]
    vlo, vhi = val(lo), val(hi)
    dlo, dhi = a - vlo, vhi - a
    if dlo < dhi or (dlo == dhi and lo % 2 == 0):
        r = lo
    else:
        r = hi
    return r | (0x8000 if sign < 0 else 0)


def assign(x, c):
    """x: list of points (lists of floats), c: list of centroids.
    Returns the index of the first centroid with minimal squared distance."""
    out = []
    for p in x:
        best, bi = None, 0
        for k, q in enumerate(c):
            d = math.fsum((a - b) * (a - b) for a, b in zip(p, q))
            if best is None or d < best:
                best, bi = d, k
        out.append(bi)
    return out


def counting_sort(ids, K):
    """Stable counting sort: labels outside [0,K) sort as K."""
    keys = [i if 0 <= i < K else K for i in ids]
    buckets = [[] for _ in range(K + 1)]
    for n, k in enumerate(keys):
        buckets[k].append(n)
    perm = [n for b in buckets for n in b]
    return [ids[n] for n in perm], perm


def accumulate(rows, ids, K, D):
    """Per-label sums (exact rational via fsum per column) and counts."""
    cols = [[[] for _ in range(D)] for _ in range(K)]
    counts = [0] * K
    for r, k in zip(rows, ids):
        if 0 <= k < K:
            counts[k] += 1
            for d in range(D):
                cols[k][d].append(r[d])
    sums = [[math.fsum(cols[k][d]) for d in range(D)] for k in range(K)]
    return sums, counts


def lloyd(x, c, iters):
    """Plain Lloyd in Python floats: labels of the last assignment and the
    centroids after `iters` updates; empty clusters keep their centroid."""
    c = [list(q) for q in c]
    labels = []
    D = len(x[0])
    for _ in range(iters):
        labels = assign(x, c)
        sums, counts = accumulate(x, labels, len(c), D)
        c = [[s / n for s in sums[k]] if n > 0 else c[k] for k, n in enumerate(counts)]
    return labels, c


def assigned_inertia(x_rows, ids, cents, K):
    """sum over rows of sum_d f32(f32(x - c)^2), total as a Python float;
    rows labelled outside [0,K) are skipped."""
    tot = 0.0
    for row, k in zip(x_rows, ids):
        if not 0 <= k < K:
            continue
        for a, c in zip(row, cents[k]):
            d = f32(f32(a) - f32(c))
            tot += f32(d * d)
    return tot


def empty_clusters(rows_of_ids, K):
    """rows_of_ids: one list of labels per batch row.  A k in [0,K) is empty
    when no row carries it (the rows' labels share one set of K bins)."""
    seen = set(k for ids in rows_of_ids for k in ids if 0 <= k < K)
    return sum(1 for k in range(K) if k not in seen)


def nearest_sqdist(p, cents):
    """Exact minimum over centroids of the squared distance (Python floats)."""
    return min(math.fsum((a - b) * (a - b) for a, b in zip(p, q)) for q in cents)


def max_row_norm(new_rows, old_rows):
    """max over rows of the Euclidean norm of new - old (exact sum, Python
    floats)."""
    best = 0.0
    for n, o in zip(new_rows, old_rows):
        best = max(best, math.sqrt(math.fsum((a - b) * (a - b) for a, b in zip(n, o))))
    return best
