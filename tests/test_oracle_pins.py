"""Pins of the CPU oracle (oracle/kmeans_oracle.py) — CPU only.

The reference ships no golden vectors for this path (its tests draw random
CUDA tensors at run time), so every oracle function is pinned here by
something other than its own formula: pure-Python brute force on tiny inputs
(tests/brute.py), independent library routines (scipy.cluster.vq.vq and
kmeans2, numpy stable argsort / add.at, sklearn KMeans, torch's bf16 cast),
known answers taken from the reference's tests (identity centroids, K=1,
ties, tails: tests/test_persistent.py:35-48, tests/test_shapes.py:14-18),
and invariants.  Each battery is also run against planted mistakes in the
oracle (wrong tie rule, dropped term, off-by-one run, wrong rounding, ...)
and must reject every one of them.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

import brute
from oracle import kmeans_oracle as O


def _rng(seed=0):
    return np.random.default_rng(seed)


def _as_lists(a):
    return [list(map(float, r)) for r in np.asarray(a, dtype=np.float64)]


# ===================================================================== assign
def _assign_battery(assign_fn):
    """Return a list of failure descriptions for an assign implementation."""
    fails = []
    rng = _rng(1)
    # 1. brute force on tiny inputs, every storage dtype
    for dtype in ("f32", "f16", "bf16", "f64"):
        for trial in range(4):
            B, N, K, D = 2, 23, 7, 5
            xf = rng.standard_normal((B, N, D)).astype(np.float32)
            cf = rng.standard_normal((B, K, D)).astype(np.float32)
            x = O.from_f32(xf, dtype) if dtype != "f64" else xf.astype(np.float64)
            c = O.from_f32(cf, dtype) if dtype != "f64" else cf.astype(np.float64)
            got = assign_fn(x, c, dtype)
            for b in range(B):
                exp = brute.assign(_as_lists(O.to_f64(x[b], dtype)),
                                   _as_lists(O.to_f64(c[b], dtype)))
                if list(got[b]) != exp:
                    fails.append(f"brute {dtype} trial {trial} batch {b}")
    # 2. scipy vq on float64 data
    from scipy.cluster.vq import vq
    x = rng.standard_normal((1, 2000, 16))
    c = rng.standard_normal((1, 50, 16))
    if not np.array_equal(assign_fn(x, c, "f64")[0], vq(x[0], c[0])[0]):
        fails.append("scipy vq")
    # 3. known answers
    x = O.from_f32(rng.standard_normal((1, 300, 32)).astype(np.float32), "f16")
    c = x[:, :64].copy()
    if not np.array_equal(assign_fn(x, c, "f16")[0, :64], np.arange(64)):
        fails.append("identity centroids")
    if np.any(assign_fn(x, x[:, :1].copy(), "f16") != 0):
        fails.append("K=1")
    # exact ties: origin equidistant from several centroids -> lowest index
    c = np.array([[[2.0, 0.0], [1.0, 0.0], [-1.0, 0.0], [0.0, 1.0]]], dtype=np.float32)
    x = np.zeros((1, 3, 2), dtype=np.float32)
    if list(assign_fn(x, c, "f32")[0]) != [1, 1, 1]:
        fails.append("tie -> lowest index")
    # duplicate centroids: the first copy wins
    xs = rng.standard_normal((1, 200, 8)).astype(np.float32)
    cs = rng.standard_normal((1, 10, 8)).astype(np.float32)
    cs[0, 7] = cs[0, 2]
    got = assign_fn(xs, cs, "f32")
    if np.any(got == 7):
        fails.append("duplicate centroid picked second copy")
    return fails


def _mut_argmax(x, c, dtype):
    xv, cv = O.to_f64(x, dtype), O.to_f64(c, dtype)
    d = ((xv[:, :, None, :] - cv[:, None, :, :]) ** 2).sum(-1)
    return np.argmax(d, axis=-1)


def _mut_last_tie(x, c, dtype):
    xv, cv = O.to_f64(x, dtype), O.to_f64(c, dtype)
    d = ((xv[:, :, None, :] - cv[:, None, :, :]) ** 2).sum(-1)
    K = d.shape[-1]
    return K - 1 - np.argmin(d[..., ::-1], axis=-1)


def _mut_no_csq(x, c, dtype):
    xv, cv = O.to_f64(x, dtype), O.to_f64(c, dtype)
    return np.argmin(-2 * np.einsum("bnd,bkd->bnk", xv, cv), axis=-1)


def _mut_plus_cross(x, c, dtype):
    xv, cv = O.to_f64(x, dtype), O.to_f64(c, dtype)
    csq = (cv * cv).sum(-1)
    return np.argmin(csq[:, None, :] + 2 * np.einsum("bnd,bkd->bnk", xv, cv), axis=-1)


def _mut_f16_accum(x, c, dtype):
    # distances rounded to fp16 before the argmin (a precision mistake)
    xv, cv = O.to_f64(x, dtype), O.to_f64(c, dtype)
    d = ((xv[:, :, None, :] - cv[:, None, :, :]) ** 2).sum(-1).astype(np.float16)
    return np.argmin(d, axis=-1)


def test_assign_oracle_pinned():
    assert _assign_battery(lambda x, c, dt: O.assign(x, c, dt)) == []


def test_assign_oracle_chunking_is_invisible():
    rng = _rng(5)
    x = O.from_f32(rng.standard_normal((2, 1000, 24)).astype(np.float32), "bf16")
    c = O.from_f32(rng.standard_normal((2, 37, 24)).astype(np.float32), "bf16")
    a = O.assign(x, c, "bf16", chunk=64)
    b = O.assign(x, c, "bf16", chunk=100000)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("mutant", [_mut_argmax, _mut_last_tie, _mut_no_csq,
                                    _mut_plus_cross, _mut_f16_accum])
def test_assign_battery_rejects_planted_mistakes(mutant):
    assert _assign_battery(mutant) != []


# ================================================================ label sort
def _sort_battery(sort_fn):
    fails = []
    rng = _rng(2)
    for K in (1, 2, 5, 17, 256, 300):
        for N in (1, 7, 64, 333):
            ids = rng.integers(-2, K + 2, (2, N)).astype(np.int32)
            if K > 3:
                ids[:, ::5] = rng.integers(0, 3, ids[:, ::5].shape)  # many ties
            s, p = sort_fn(ids, K)
            for b in range(2):
                es, ep = brute.counting_sort(list(map(int, ids[b])), K)
                if list(map(int, s[b])) != es or list(map(int, p[b])) != ep:
                    fails.append(f"brute K={K} N={N} b={b}")
    # library routine: numpy stable argsort of the mapped keys
    ids = rng.integers(0, 1000, (3, 5000)).astype(np.int32)
    s, p = sort_fn(ids, 1000)
    ref = np.argsort(ids, axis=1, kind="stable")
    if not np.array_equal(p, ref):
        fails.append("numpy stable argsort")
    # invariants
    if not np.all(np.diff(s.astype(np.int64), axis=1) >= 0):
        fails.append("not sorted")
    if not all(np.array_equal(np.sort(p[b]), np.arange(5000)) for b in range(3)):
        fails.append("not a permutation")
    return fails


def _mut_unstable(ids, K):
    s, p = O.label_sort(ids, K)
    p = p.copy()
    for b in range(p.shape[0]):  # reverse index order inside every run
        keys = O.sort_keys(np.take_along_axis(ids, p.astype(np.int64), 1), K)[b]
        starts = np.flatnonzero(np.concatenate(([True], keys[1:] != keys[:-1])))
        ends = np.concatenate((starts[1:], [len(keys)]))
        for st, en in zip(starts, ends):
            p[b, st:en] = p[b, st:en][::-1]
    return np.take_along_axis(ids, p.astype(np.int64), 1), p


def _mut_invalid_first(ids, K):
    keys = np.where((ids >= 0) & (ids < K), ids, -1)
    p = np.argsort(keys, axis=-1, kind="stable")
    return np.take_along_axis(ids, p, 1).astype(np.int32), p.astype(np.int32)


def test_label_sort_oracle_pinned():
    assert _sort_battery(O.label_sort) == []


@pytest.mark.parametrize("mutant", [_mut_unstable, _mut_invalid_first])
def test_sort_battery_rejects_planted_mistakes(mutant):
    assert _sort_battery(mutant) != []


# ==================================================================== update
def _update_battery(update_fn):
    fails = []
    rng = _rng(3)
    for dtype in ("f32", "f16", "bf16"):
        for K in (1, 4, 9):
            N, D = 57, 6
            xf = rng.standard_normal((1, N, D)).astype(np.float32)
            x = O.from_f32(xf, dtype)
            ids = rng.integers(-1, K + 1, (1, N)).astype(np.int32)
            s_ids, perm = O.label_sort(ids, K)
            rows = np.take_along_axis(x, perm.astype(np.int64)[..., None], 1)
            sums, counts = update_fn(rows, s_ids, K, dtype)
            es, ec = brute.accumulate(_as_lists(O.to_f64(rows[0], dtype)),
                                      list(map(int, s_ids[0])), K, D)
            if list(map(int, counts[0])) != ec:
                fails.append(f"counts {dtype} K={K}")
            if not np.allclose(sums[0], np.array(es), rtol=1e-12, atol=1e-12):
                fails.append(f"sums {dtype} K={K}")
    # library routine: np.add.at / bincount on a larger case
    x = rng.standard_normal((2, 4000, 16))
    ids = rng.integers(0, 50, (2, 4000)).astype(np.int32)
    s_ids, perm = O.label_sort(ids, 50)
    rows = np.take_along_axis(x, perm.astype(np.int64)[..., None], 1)
    sums, counts = update_fn(rows, s_ids, 50, "f64")
    for b in range(2):
        ref = np.zeros((50, 16))
        np.add.at(ref, ids[b], x[b])
        if not np.allclose(sums[b], ref, rtol=1e-12, atol=1e-10):
            fails.append("np.add.at sums")
        if not np.array_equal(counts[b], np.bincount(ids[b], minlength=50)):
            fails.append("bincount counts")
    return fails


def _mut_drop_last_row(rows, ids, K, dtype):
    ids = np.asarray(ids).copy()
    ends = np.flatnonzero(np.concatenate((ids[0, 1:] != ids[0, :-1], [True])))
    ids[0, ends] = -5  # the last row of every run is lost
    return O.update_sorted(rows, ids, K, dtype)


def _mut_keep_invalid(rows, ids, K, dtype):
    return O.update_sorted(rows, np.clip(ids, 0, K - 1), K, dtype)


def _mut_count_runs(rows, ids, K, dtype):
    sums, counts = O.update_sorted(rows, ids, K, dtype)
    return sums, (counts > 0).astype(np.int64)


def test_update_oracle_pinned():
    assert _update_battery(O.update_sorted) == []


@pytest.mark.parametrize("mutant", [_mut_drop_last_row, _mut_keep_invalid, _mut_count_runs])
def test_update_battery_rejects_planted_mistakes(mutant):
    assert _update_battery(mutant) != []


def test_update_indexed_equals_materialized():
    rng = _rng(4)
    x = O.from_f32(rng.standard_normal((2, 500, 12)).astype(np.float32), "f16")
    ids = rng.integers(0, 20, (2, 500)).astype(np.int32)
    s_ids, perm = O.label_sort(ids, 20)
    rows = np.take_along_axis(x, perm.astype(np.int64)[..., None], 1)
    a = O.update_sorted(rows, s_ids, 20, "f16")
    b = O.update_sorted_indexed(x, perm, s_ids, 20, "f16")
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


# ================================================================== finalize
def _finalize_battery(fin_fn):
    fails = []
    rng = _rng(6)
    for dtype in ("f32", "f16", "bf16"):
        K, D = 40, 9
        v = O.from_f32(rng.standard_normal((1, K, D)).astype(np.float32) * 3, dtype)
        vf = O.to_f32(v, dtype).astype(np.float64)
        counts = rng.choice([0, 1, 2, 4, 8], (1, K))  # powers of two: exact
        counts[0, :5] = 0
        sums = vf * counts[..., None]
        old = O.from_f32(rng.standard_normal((1, K, D)).astype(np.float32), dtype)
        out = fin_fn(sums, counts, old, dtype)
        full = counts[0] > 0
        if not np.array_equal(np.asarray(out)[0][full].view(np.uint8),
                              np.asarray(v)[0][full].view(np.uint8)):
            fails.append(f"mean of copies {dtype}")
        if not np.array_equal(np.asarray(out)[0][~full].view(np.uint8),
                              np.asarray(old)[0][~full].view(np.uint8)):
            fails.append(f"empty keeps old {dtype}")
    # rounding of a non-exact quotient, per element, against brute force
    sums = rng.standard_normal((1, 8, 16)) * 10
    counts = np.full((1, 8), 3)
    old = np.zeros((1, 8, 16), np.float16)
    out16 = fin_fn(sums, counts, old, "f16")
    q32 = (sums.astype(np.float32) / np.float32(3)).astype(np.float32)
    if not np.array_equal(out16, q32.astype(np.float16)):
        fails.append("f16 rounding")
    outbf = fin_fn(sums, counts, np.zeros((1, 8, 16), np.uint16), "bf16")
    expbf = np.array([[[brute.bf16_bits_rne(float(v)) for v in r] for r in q32[0]]],
                     dtype=np.uint16)
    if not np.array_equal(outbf, expbf):
        fails.append("bf16 rounding")
    return fails


def _mut_trunc_bf16(sums, counts, old, dtype):
    if dtype != "bf16":
        return O.finalize(sums, counts, old, dtype)
    q = (np.asarray(sums, np.float32) / np.maximum(counts, 1)[..., None].astype(np.float32))
    t = (q.view(np.uint32) >> 16).astype(np.uint16)
    return np.where(counts[..., None] > 0, t, old)


def _mut_zero_empty(sums, counts, old, dtype):
    out = O.finalize(sums, counts, old, dtype)
    return np.where(counts[..., None] > 0, out, np.zeros_like(out))


def _mut_count_plus_one(sums, counts, old, dtype):
    return O.finalize(sums, np.asarray(counts) + (np.asarray(counts) > 0), old, dtype)


def test_finalize_oracle_pinned():
    assert _finalize_battery(O.finalize) == []


@pytest.mark.parametrize("mutant", [_mut_trunc_bf16, _mut_zero_empty, _mut_count_plus_one])
def test_finalize_battery_rejects_planted_mistakes(mutant):
    assert _finalize_battery(mutant) != []


def test_bf16_rounding_matches_torch_and_brute_force():
    import torch
    rng = _rng(7)
    vals = np.concatenate([
        rng.standard_normal(5000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 5000),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, 1e-40, -1e-41,
                  1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9], dtype=np.float32),
    ]).astype(np.float32)
    ours = O.f32_to_bf16_bits(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    assert all(brute.bf16_bits_rne(float(v)) == int(o) for v, o in zip(vals[::7], ours[::7]))


# ===================================================================== norms
def test_row_sqnorm_pinned():
    rng = _rng(8)
    a = O.from_f32(rng.standard_normal((3, 5, 7)).astype(np.float32), "bf16")
    got = O.row_sqnorm(a, "bf16")
    v = O.to_f64(a, "bf16")
    for i in range(3):
        for j in range(5):
            import math
            assert got[i, j] == pytest.approx(math.fsum(float(t) ** 2 for t in v[i, j]), rel=1e-15)


# ================================================================= distances
def _distances_battery(dist_fn):
    """dist_fn(x, c, dtype, ids) -> float64 (B, N): the exact squared distance
    of every point to its labelled centroid (the figure the frozen fixtures'
    inertia and the GPU tests' inertia checks are summed from)."""
    import math
    fails = []
    rng = _rng(9)
    # 1. brute force (exact sums of Python floats) for every storage dtype,
    # batch rows with their own tables and labels
    for dtype in ("f32", "f16", "bf16", "f64"):
        B, N, K, D = 3, 19, 5, 7
        xf = (rng.standard_normal((B, N, D)) * 3).astype(np.float32)
        cf = (rng.standard_normal((B, K, D)) * 3).astype(np.float32)
        x = O.from_f32(xf, dtype) if dtype != "f64" else xf.astype(np.float64)
        c = O.from_f32(cf, dtype) if dtype != "f64" else cf.astype(np.float64)
        ids = rng.integers(0, K, (B, N)).astype(np.int32)
        got = dist_fn(x, c, dtype, ids)
        if got.shape != (B, N):
            fails.append(f"shape {got.shape}")
            continue
        xv, cv = O.to_f64(x, dtype), O.to_f64(c, dtype)
        for b in range(B):
            for n in range(N):
                want = math.fsum((float(p) - float(q)) ** 2
                                 for p, q in zip(xv[b, n], cv[b, ids[b, n]]))
                if not math.isclose(float(got[b, n]), want, rel_tol=1e-14, abs_tol=1e-300):
                    fails.append(f"brute {dtype} ({b},{n}): {got[b, n]!r} vs {want!r}")
                    break
    # 2. library: scipy's vq returns the Euclidean distance to the nearest
    # centroid; its square at vq's labels is this function at those labels
    from scipy.cluster.vq import vq
    x = rng.standard_normal((1, 400, 12))
    c = rng.standard_normal((1, 30, 12))
    lab, dist = vq(x[0], c[0])
    got = dist_fn(x, c, "f64", lab[None].astype(np.int64))
    if not np.allclose(got[0], dist ** 2, rtol=1e-12, atol=0):
        fails.append("scipy vq distances")
    # 3. known answers: a 3-4-5 triangle and a point on its own centroid
    c = np.zeros((1, 2, 3), np.float32)
    c[0, 1] = (1.0, 1.0, 1.0)
    x = np.array([[[3.0, 4.0, 0.0], [1.0, 1.0, 1.0]]], np.float32)
    got = dist_fn(x, c, "f32", np.array([[0, 1]], np.int32))
    if list(map(float, got[0])) != [25.0, 0.0]:
        fails.append(f"known answers {got[0]}")
    return fails


def _mut_dist_not_squared(x, c, dtype, ids):
    return np.sqrt(O.distances(x, c, dtype, ids))


def _mut_dist_first_row_table(x, c, dtype, ids):
    # every batch row scored against batch row 0's centroids
    c0 = np.broadcast_to(np.asarray(c)[:1], np.asarray(c).shape).copy()
    return O.distances(x, c0, dtype, ids)


def _mut_dist_label_off_by_one(x, c, dtype, ids):
    K = np.asarray(c).shape[1]
    return O.distances(x, c, dtype, (np.asarray(ids) + 1) % K)


def _mut_dist_f16_values(x, c, dtype, ids):
    # distances computed from values rounded to fp16 (a precision mistake)
    xv = O.to_f64(x, dtype).astype(np.float16).astype(np.float64)
    cv = O.to_f64(c, dtype).astype(np.float16).astype(np.float64)
    chosen = np.take_along_axis(cv, np.asarray(ids).astype(np.int64)[..., None], axis=1)
    return ((xv - chosen) ** 2).sum(-1)


def _mut_dist_dropped_feature(x, c, dtype, ids):
    xv, cv = O.to_f64(x, dtype), O.to_f64(c, dtype)
    chosen = np.take_along_axis(cv, np.asarray(ids).astype(np.int64)[..., None], axis=1)
    return ((xv - chosen)[..., 1:] ** 2).sum(-1)


def test_distances_oracle_pinned():
    assert _distances_battery(O.distances) == []


@pytest.mark.parametrize("mutant", [_mut_dist_not_squared, _mut_dist_first_row_table,
                                    _mut_dist_label_off_by_one, _mut_dist_f16_values,
                                    _mut_dist_dropped_feature])
def test_distances_battery_rejects_planted_mistakes(mutant):
    assert _distances_battery(mutant) != []


# ====================================================================== loop
def _loop_battery(kmeans_fn):
    fails = []
    rng = _rng(9)
    from scipy.cluster.vq import kmeans2
    # 1. scipy kmeans2 ('matrix' init, missing='warn' keeps empty centroids)
    for trial, (N, K, D, iters) in enumerate([(500, 8, 4, 6), (800, 20, 3, 10)]):
        x = rng.standard_normal((1, N, D))
        init = x[:, rng.choice(N, K, replace=False)].copy()
        init[0, 0] = 50.0  # a far centroid that stays empty
        ids, cents, n = kmeans_fn(x, K, iters, 0.0, init, "f64")
        import warnings
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            sc, sl = kmeans2(x[0], init[0].copy(), iter=iters, minit="matrix", missing="warn")
        if n != iters:
            fails.append(f"n_iters {trial}")
        if not np.array_equal(ids[0], sl):
            fails.append(f"scipy labels {trial}")
        if not np.allclose(cents[0], sc, rtol=1e-12, atol=1e-12):
            fails.append(f"scipy centroids {trial}")
    # 2. brute force Lloyd in Python floats
    x = rng.standard_normal((1, 60, 3))
    init = x[:, :5].copy()
    ids, cents, _ = kmeans_fn(x, 5, 4, 0.0, init, "f64")
    bl, bc = brute.lloyd(_as_lists(x[0]), _as_lists(init[0]), 4)
    if list(ids[0]) != bl or not np.allclose(cents[0], np.array(bc), rtol=1e-12, atol=1e-12):
        fails.append("brute lloyd")
    # 3. sklearn Lloyd centres (no empty clusters)
    from sklearn.cluster import KMeans
    x = rng.standard_normal((1, 1000, 5))
    init = x[:, :6].copy()
    _, cents, _ = kmeans_fn(x, 6, 30, 0.0, init, "f64")
    km = KMeans(n_clusters=6, init=init[0], n_init=1, max_iter=30, tol=0.0,
                algorithm="lloyd").fit(x[0])
    if not np.allclose(cents[0], km.cluster_centers_, rtol=1e-10, atol=1e-10):
        fails.append("sklearn centres")
    # 4. tol semantics: stop after the first iteration with shift < tol
    x = rng.standard_normal((1, 400, 4))
    init = x[:, :4].copy()
    ids_all, c_all, n_all = kmeans_fn(x, 4, 50, 0.0, init, "f64")
    ids_t, c_t, n_t = kmeans_fn(x, 4, 50, 1e-9, init, "f64")
    if not (1 <= n_t < 50):
        fails.append("tol did not stop early")
    elif not np.allclose(c_t, c_all):
        fails.append("tol result differs from converged result")
    return fails


def _mut_labels_after_update(x, K, iters, tol, init, dtype):
    ids, cents, n = O.kmeans(x, K, iters, tol, init, dtype)
    return O.assign(x, cents, dtype), cents, n


def _mut_one_extra_iter(x, K, iters, tol, init, dtype):
    return O.kmeans(x, K, iters + 1, tol, init, dtype)


def _mut_empty_to_zero(x, K, iters, tol, init, dtype):
    cur = np.array(init, copy=True)
    ids = None
    for _ in range(iters):
        ids = O.assign(x, cur, dtype)
        s, p = O.label_sort(ids, K)
        sums, counts = O.update_sorted_indexed(x, p, s, K, dtype)
        cur = np.where(counts[..., None] > 0, sums / np.maximum(counts, 1)[..., None], 0.0)
    return ids, cur, iters


def test_loop_oracle_pinned():
    assert _loop_battery(O.kmeans) == []


@pytest.mark.parametrize("mutant", [_mut_labels_after_update, _mut_one_extra_iter,
                                    _mut_empty_to_zero])
def test_loop_battery_rejects_planted_mistakes(mutant):
    assert _loop_battery(mutant) != []


# ===================================================================== shift
def _shift_battery(shift_fn):
    """shift_fn(new, old, dtype) -> float, the convergence measure of
    kmeans.py:104: max over every batch row and centroid of ||new - old||_2."""
    fails = []
    rng = _rng(21)
    # 1. closed form.  Row deltas (3,4), (0,9) in row 0 and (6,8), (1,0) in
    # row 1: the L2 norms are 5, 9, 10, 1, so the measure is 10 (row 1).  A
    # squared norm gives 100, the mean 6.25, the L1 norm 14, the largest
    # element 9, and a max over row 0 alone 9.
    for dtype in ("f32", "f16", "bf16"):
        old = np.array([[[1, 2], [4, -3]], [[-5, 0], [2, 2]]], np.float32)
        delta = np.array([[[3, 4], [0, 9]], [[6, 8], [1, 0]]], np.float32)
        new = O.from_f32(old + delta, dtype)
        got = shift_fn(new, O.from_f32(old, dtype), dtype)
        if got != 10.0:
            fails.append(f"closed form {dtype}: {got!r}")
    # no motion
    c = O.from_f32(rng.standard_normal((2, 5, 8)).astype(np.float32), "f16")
    if shift_fn(c, c.copy(), "f16") != 0.0:
        fails.append("zero shift")
    # 2. brute force on random rows (exact sums; float32 rounding only)
    for dtype in ("f32", "f16", "bf16"):
        old = O.from_f32(rng.standard_normal((3, 11, 7)).astype(np.float32), dtype)
        new = O.from_f32(rng.standard_normal((3, 11, 7)).astype(np.float32), dtype)
        of, nf = O.to_f32(old, dtype), O.to_f32(new, dtype)
        want = max(brute.max_row_norm(_as_lists(nf[b]), _as_lists(of[b])) for b in range(3))
        got = shift_fn(new, old, dtype)
        if not np.isclose(got, want, rtol=2e-7, atol=0):
            fails.append(f"brute {dtype}: {got!r} vs {want!r}")
    return fails


def _mut_shift_squared(new, old, dtype):
    d = O.to_f64(new, dtype) - O.to_f64(old, dtype)
    return float((d * d).sum(-1).max())


def _mut_shift_mean(new, old, dtype):
    d = O.to_f64(new, dtype) - O.to_f64(old, dtype)
    return float(np.sqrt((d * d).sum(-1)).mean())


def _mut_shift_l1(new, old, dtype):
    d = O.to_f64(new, dtype) - O.to_f64(old, dtype)
    return float(np.abs(d).sum(-1).max())


def _mut_shift_linf(new, old, dtype):
    d = O.to_f64(new, dtype) - O.to_f64(old, dtype)
    return float(np.abs(d).max())


def _mut_shift_first_row(new, old, dtype):
    return O.shift(np.asarray(new)[:1], np.asarray(old)[:1], dtype)


_SHIFT_MUTANTS = [_mut_shift_squared, _mut_shift_mean, _mut_shift_l1, _mut_shift_linf,
                  _mut_shift_first_row]


def test_shift_oracle_pinned():
    assert _shift_battery(O.shift) == []


@pytest.mark.parametrize("mutant", _SHIFT_MUTANTS)
def test_shift_battery_rejects_planted_mistakes(mutant):
    assert _shift_battery(mutant) != []


def _kmeans_with_shift(shift_fn):
    """O.kmeans with its convergence measure replaced (a planted mistake)."""
    def run(x, K, iters, tol, init, dtype):
        cur = np.array(init, copy=True)
        ids, n = None, 0
        for it in range(iters):
            new, ids, _, _ = O.lloyd_step(x, cur, K, dtype)
            n = it + 1
            if tol > 0 and shift_fn(new, cur, dtype) < tol:
                cur = new
                break
            cur = new
        return ids, cur, n
    return run


def _stop_battery(kmeans_fn):
    """The iteration the tol test stops at, where the answer depends on how
    the shift is measured.  Two batch rows, the second moving more; the
    shifts of every iteration are measured independently (brute-force norms
    of the centroid trajectory), and tol is put between two consecutive
    shifts below 1, so that a squared, mean, L1, largest-element or
    first-row measure stops at another iteration."""
    fails = []
    rng = _rng(23)
    B, N, K, D = 2, 300, 6, 3
    x = rng.standard_normal((B, N, D))
    x[1] *= 3.0
    init = x[:, :K].copy()
    traj = [init]
    for it in range(1, 13):
        traj.append(O.kmeans(x, K, it, 0.0, init, "f64")[1])
    shifts = [max(brute.max_row_norm(_as_lists(traj[i][b]), _as_lists(traj[i - 1][b]))
                  for b in range(B)) for i in range(1, len(traj))]
    # first iteration i (1-based) whose shift is below 0.5 and still above the
    # next one; tol halfway (geometric) between them
    i = next(j for j in range(len(shifts) - 1)
             if shifts[j] < 0.5 and shifts[j + 1] < shifts[j] and shifts[j + 1] > 0)
    tol = float(np.sqrt(shifts[i] * shifts[i + 1]))
    want_n = next(j + 1 for j, v in enumerate(shifts) if v < tol)
    ids, cents, n = kmeans_fn(x, K, 50, tol, init, "f64")
    if n != want_n:
        fails.append(f"stopped after {n}, expected {want_n} (tol {tol:.3g})")
    elif not np.allclose(cents, traj[want_n]):
        fails.append("centroids at the stop differ from the trajectory")
    return fails


def test_tol_stop_iteration_pinned():
    assert _stop_battery(O.kmeans) == []


@pytest.mark.parametrize("mutant", _SHIFT_MUTANTS)
def test_tol_stop_rejects_planted_shift_mistakes(mutant):
    assert _stop_battery(_kmeans_with_shift(mutant)) != []


# ==================================================================== quality
def _quality_battery(inertia_fn, empty_fn):
    fails = []
    rng = _rng(11)
    # 1. brute force (float32 difference and square, float64 total)
    for dtype in ("f32", "f16", "bf16"):
        B, N, K, D = 2, 37, 6, 5
        x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 3, dtype)
        c = O.from_f32(rng.standard_normal((B, K, D)).astype(np.float32) * 3, dtype)
        ids = rng.integers(-1, K + 1, (B, N)).astype(np.int32)  # some invalid
        got = inertia_fn(x, ids, c, dtype)
        xf, cf = O.to_f32(x, dtype), O.to_f32(c, dtype)
        for b in range(B):
            want = brute.assigned_inertia(_as_lists(xf[b]), list(map(int, ids[b])),
                                          _as_lists(cf[b]), K)
            if not np.isclose(got[b], want, rtol=1e-13, atol=0):
                fails.append(f"brute {dtype} b={b}: {got[b]!r} vs {want!r}")
        if empty_fn(ids, K) != brute.empty_clusters([list(map(int, r)) for r in ids], K):
            fails.append(f"empty {dtype}")
    # 2. library: with labels from scipy's vq, inertia = sum of vq distances^2
    from scipy.cluster.vq import vq
    x = rng.standard_normal((1, 500, 16)).astype(np.float32)
    c = rng.standard_normal((1, 40, 16)).astype(np.float32)
    lab, dist = vq(x[0].astype(np.float64), c[0].astype(np.float64))
    got = inertia_fn(x, lab[None].astype(np.int32), c, "f32")
    if not np.isclose(got[0], (dist ** 2).sum(), rtol=1e-6):
        fails.append("scipy vq distances")
    # 3. known answers: labels at the centroids themselves give zero;
    # a point at distance 3 from its centroid gives 9
    c = np.zeros((1, 3, 4), np.float32)
    c[0, 1, 0] = 5.0
    x = np.zeros((1, 2, 4), np.float32)
    x[0, 0, 0] = 5.0
    x[0, 1, 2] = 3.0
    got = inertia_fn(x, np.array([[1, 0]], np.int32), c, "f32")
    if got[0] != 9.0:
        fails.append(f"known answer {got[0]}")
    if empty_fn(np.array([[1, 0, 1]], np.int32), 3) != 1:
        fails.append("known empty count")
    # 4. the reference's own formula at B > 1 (quality_compare.py:86-88): one
    # torch.bincount over the flattened labels; k is empty only when no row
    # carries it (row 0 leaves 2 and 3 empty, row 1 fills 3)
    import torch
    ids = np.array([[0, 1, 1, 4], [3, 3, 0, 4]], np.int32)
    want = int((torch.bincount(torch.from_numpy(ids).reshape(-1).long(), minlength=6) == 0)
               .sum())
    if want != 2 or empty_fn(ids, 6) != want:
        fails.append("flattened bincount at B=2")
    for trial in range(3):
        ids = rng.integers(0, 40, (4, 25)).astype(np.int32)
        want = int((torch.bincount(torch.from_numpy(ids).reshape(-1).long(), minlength=40)
                    == 0).sum())
        if empty_fn(ids, 40) != want:
            fails.append(f"torch bincount trial {trial}")
    return fails


def _mut_f64_square(x, ids, c, dtype):
    xf, cf = O.to_f64(x, dtype), O.to_f64(c, dtype)
    out = []
    for b in range(xf.shape[0]):
        ok = (ids[b] >= 0) & (ids[b] < cf.shape[1])
        out.append(((xf[b][ok] - cf[b][ids[b][ok]]) ** 2).sum())
    return np.asarray(out)


def _mut_clip_invalid(x, ids, c, dtype):
    return O.assigned_inertia(x, np.clip(ids, 0, c.shape[1] - 1), c, dtype)


def _mut_norm_not_squared(x, ids, c, dtype):
    xf, cf = O.to_f32(x, dtype), O.to_f32(c, dtype)
    out = []
    for b in range(xf.shape[0]):
        ok = (ids[b] >= 0) & (ids[b] < cf.shape[1])
        out.append(np.linalg.norm(xf[b][ok] - cf[b][ids[b][ok]], axis=1).astype(np.float64).sum())
    return np.asarray(out)


def _mut_empty_off_by_one(ids, K):
    return O.empty_clusters(ids, K) - int((np.asarray(ids) == K - 1).any())


def _mut_empty_per_row(ids, K):
    # empty (b, k) pairs summed over rows, instead of one flattened histogram
    return sum(O.empty_clusters(np.asarray(ids)[b:b + 1], K) for b in range(len(ids)))


def test_quality_oracle_pinned():
    assert _quality_battery(O.assigned_inertia, O.empty_clusters) == []


@pytest.mark.parametrize("mutant", [_mut_f64_square, _mut_clip_invalid, _mut_norm_not_squared])
def test_quality_battery_rejects_planted_inertia_mistakes(mutant):
    assert _quality_battery(mutant, O.empty_clusters) != []


@pytest.mark.parametrize("mutant", [_mut_empty_off_by_one, _mut_empty_per_row])
def test_quality_battery_rejects_planted_empty_count_mistakes(mutant):
    assert _quality_battery(O.assigned_inertia, mutant) != []


# ============================================================ sampled inertia
def _sample_battery(fn):
    """fn(x, c, sample_idx, dtype) -> float (quality_compare.py:91-116)."""
    fails = []
    rng = _rng(13)
    # 1. brute force: exact nearest squared distance of every sampled point,
    # summed over batch rows (the GEMM-form float32 distance differs from it
    # by float32 rounding only)
    for dtype in ("f32", "f16", "bf16"):
        B, N, K, D = 2, 50, 7, 6
        x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 2, dtype)
        c = O.from_f32(rng.standard_normal((B, K, D)).astype(np.float32) * 2, dtype)
        idx = rng.permutation(N)[:17]
        xf, cf = O.to_f32(x, dtype), O.to_f32(c, dtype)
        want = sum(brute.nearest_sqdist(list(map(float, xf[b, n])), _as_lists(cf[b]))
                   for b in range(B) for n in idx)
        got = fn(x, c, idx, dtype)
        if not np.isclose(got, want, rtol=1e-5, atol=1e-4):
            fails.append(f"brute {dtype}: {got!r} vs {want!r}")
    # 2. library: scipy's vq distances of the sample
    from scipy.cluster.vq import vq
    x = rng.standard_normal((1, 400, 12)).astype(np.float32)
    c = rng.standard_normal((1, 30, 12)).astype(np.float32)
    idx = rng.permutation(400)[:64]
    _, dist = vq(x[0, idx].astype(np.float64), c[0].astype(np.float64))
    if not np.isclose(fn(x, c, idx, "f32"), (dist ** 2).sum(), rtol=1e-5):
        fails.append("scipy vq")
    # 3. known answers: sampled points that are centroids give 0 (clamped);
    # a point at distance 3 from the nearest of two centroids gives 9
    c = np.array([[[0.0, 0.0], [10.0, 0.0]]], np.float32)
    x = np.array([[[10.0, 0.0], [0.0, 3.0], [0.0, 0.0], [7.0, 0.0]]], np.float32)
    if fn(x, c, np.array([0, 2]), "f32") != 0.0:
        fails.append("centroids as samples")
    if fn(x, c, np.array([1, 3]), "f32") != 18.0:
        fails.append("known distances 3 and 3")
    if fn(x, c, np.array([1]), "f32") != 9.0:
        fails.append("only the sampled points count")
    return fails


def _mut_sample_max_centroid(x, c, idx, dtype):
    xs, cf = O.to_f64(np.asarray(x)[:, idx], dtype), O.to_f64(c, dtype)
    return float(sum(((xs[b][:, None] - cf[b][None]) ** 2).sum(-1).max(-1).sum()
                     for b in range(xs.shape[0])))


def _mut_sample_first_row_only(x, c, idx, dtype):
    return O.sample_exact_inertia(np.asarray(x)[:1], np.asarray(c)[:1], idx, dtype)


def _mut_sample_no_csq(x, c, idx, dtype):
    xs, cf = O.to_f64(np.asarray(x)[:, idx], dtype), O.to_f64(c, dtype)
    tot = 0.0
    for b in range(xs.shape[0]):
        d = (xs[b] ** 2).sum(-1)[:, None] - 2.0 * xs[b] @ cf[b].T
        tot += float(np.maximum(d.min(-1), 0).sum())
    return tot


def _mut_sample_all_points(x, c, idx, dtype):
    return O.sample_exact_inertia(x, c, np.arange(np.asarray(x).shape[1]), dtype)


def test_sample_exact_inertia_oracle_pinned():
    assert _sample_battery(O.sample_exact_inertia) == []


@pytest.mark.parametrize("mutant", [_mut_sample_max_centroid, _mut_sample_first_row_only,
                                    _mut_sample_no_csq, _mut_sample_all_points])
def test_sample_battery_rejects_planted_mistakes(mutant):
    assert _sample_battery(mutant) != []
