"""GPU parity of label sort, centroid update and finalize (through the C ABI).

Bar: the sort permutation and sorted labels are bit-exact against the
oracle's stable sort; counts are bit-exact; fp32 sums agree with the
oracle's float64 sums within fp32 accumulation error; finalize is bit-exact
given identical sums and counts (IEEE division, round-to-nearest-even).
Mirrors tests/cpp/smoke.cpp:55-95 of the reference (indexed update ==
materialized update, finalize formula) plus skew, empty clusters, invalid
labels and determinism.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kmeans_oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dtype="i32"):
    from flash_kmeans_cuda import synth
    if dtype == "i32":
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()
    return synth.to_torch(a, dtype)


def _np(t, dtype=None):
    from flash_kmeans_cuda import synth
    torch.cuda.synchronize()
    return t.cpu().numpy() if dtype is None else synth.from_torch(t, dtype)


SORT_CASES = [
    (1, 1, 1), (1, 100, 1), (2, 100, 2), (1, 4096, 255), (1, 4097, 256), (3, 10000, 257),
    (1, 32768, 256), (1, 131072, 2048), (2, 65536, 1024), (1, 100000, 8192), (1, 70000, 70000),
]


def _sort_ws(B, N, K):
    """A label-sort workspace the test can inspect (word 0 = recount count)."""
    from flash_kmeans_cuda import _lib
    n = _lib.lib.fkc_label_sort_workspace_bytes(B, N, K)
    ws = torch.full((n,), 0xA5, dtype=torch.uint8, device="cuda")  # stale bytes
    return ws


def _recounts(ws):
    """Word 0 of the workspace (recounts); word 1 (tiles whose counter was
    out of step with the call sequence) must stay 0."""
    torch.cuda.synchronize()
    w = ws[:8].view(torch.int32).cpu()
    assert int(w[1]) == 0, "sort tile counter out of step"
    return int(w[0])


@pytest.mark.parametrize("B,N,K", SORT_CASES)
def test_label_sort_bit_exact(B, N, K):
    from flash_kmeans_cuda.ops import label_sort
    rng = np.random.default_rng(N + K)
    ids = rng.integers(0, K, (B, N)).astype(np.int32)
    if N > 50:
        ids[:, rng.integers(0, N, N // 50)] = rng.integers(-3, 2 * K + 3, (B, N // 50))
    ws = _sort_ws(B, N, K)
    s, p = label_sort(_t(ids), K, workspace=ws)
    es, ep = O.label_sort(ids, K)
    assert np.array_equal(_np(p), ep)
    assert np.array_equal(_np(s), es)
    assert _recounts(ws) == 0


def test_label_sort_zipf_skew():
    from flash_kmeans_cuda.ops import label_sort
    from flash_kmeans_cuda import synth
    rng = np.random.default_rng(5)
    ids = rng.choice(8192, 524288, p=synth.zipf_probs(8192, 1.1)).astype(np.int32)[None]
    s, p = label_sort(_t(ids), 8192)
    es, ep = O.label_sort(ids, 8192)
    assert np.array_equal(_np(p), ep) and np.array_equal(_np(s), es)


@pytest.mark.parametrize("tile", [256, 512, 1024, 2048, 4096, 8192])
@pytest.mark.parametrize("B,N,K,pattern", [
    (2, 100000, 8192, "random"), (1, 70001, 70000, "random"),
    (1, 300000, 4096, "same"), (3, 9000, 9000, "descending"),
])
def test_label_sort_every_tile_size(monkeypatch, tile, B, N, K, pattern):
    """Each tile size of the single-sweep passes (FKC_SORT_TILE), over
    random, all-equal and strictly descending labels (every tile then waits
    on its predecessors for every digit), bit-exact against the stable sort;
    each case is sorted twice in a row on one workspace that starts out
    filled with stale bytes (the second call finds the first call's counters
    and status words), and no wait ran out (the recount word stays 0)."""
    from flash_kmeans_cuda.ops import label_sort
    monkeypatch.setenv("FKC_SORT_TILE", str(tile))
    rng = np.random.default_rng(tile + N)
    if pattern == "random":
        ids = rng.integers(-2, K + 2, (B, N)).astype(np.int32)
    elif pattern == "same":
        ids = np.full((B, N), K - 1, np.int32)
    else:
        ids = np.broadcast_to(np.arange(N - 1, -1, -1, dtype=np.int32) % K, (B, N)).copy()
    es, ep = O.label_sort(ids, K)
    ws = _sort_ws(B, N, K)
    for _ in range(2):
        s, p = label_sort(_t(ids), K, workspace=ws)
        assert np.array_equal(_np(p), ep)
        assert np.array_equal(_np(s), es)
        assert _recounts(ws) == 0


def _update_case(B, N, K, D, dtype, seed, invalid=False, zipf=False):
    rng = np.random.default_rng(seed)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    if zipf:
        from flash_kmeans_cuda import synth
        ids = rng.choice(K, (B, N), p=synth.zipf_probs(K, 1.1)).astype(np.int32)
    else:
        ids = rng.integers(0, K, (B, N)).astype(np.int32)
    if invalid:
        ids[:, ::17] = -1
        ids[:, 5::23] = K + 4
    s_ids, perm = O.label_sort(ids, K)
    return x, ids, s_ids, perm


UPDATE_CASES = [
    (1, 512, 16, 1, "f32"), (1, 512, 16, 7, "f32"), (1, 512, 16, 257, "f32"),
    (1, 512, 64, 128, "f16"), (2, 5000, 300, 64, "bf16"), (1, 20000, 1000, 128, "f16"),
    (1, 3000, 50, 600, "f16"), (1, 1000, 5, 1100, "bf16"), (3, 777, 1, 33, "f16"),
]


@pytest.mark.parametrize("B,N,K,D,dtype", UPDATE_CASES)
def test_update_indexed_and_materialized(B, N, K, D, dtype):
    from flash_kmeans_cuda import _C
    x, ids, s_ids, perm = _update_case(B, N, K, D, dtype, seed=N + D, invalid=(D % 2 == 1))
    xt = _t(x, dtype)
    sums_i = torch.zeros((B, K, D), device="cuda")
    cnt_i = torch.zeros((B, K), device="cuda", dtype=torch.int32)
    _C.centroid_update_sorted_indexed(xt, _t(perm), _t(s_ids), sums_i, cnt_i)
    rows = np.take_along_axis(x, perm.astype(np.int64)[..., None], 1)
    sums_m = torch.zeros((B, K, D), device="cuda")
    cnt_m = torch.zeros((B, K), device="cuda", dtype=torch.int32)
    _C.centroid_update_sorted(_t(rows, dtype), _t(s_ids), sums_m, cnt_m)
    es, ec = O.update_sorted_indexed(x, perm, s_ids, K, dtype)
    si, ci, sm, cm = _np(sums_i), _np(cnt_i), _np(sums_m), _np(cnt_m)
    assert np.array_equal(ci, ec) and np.array_equal(cm, ec)
    # same rows in the same order -> bit-identical sums (smoke.cpp:81 asks 1e-4)
    assert np.array_equal(si.view(np.uint32), sm.view(np.uint32))
    tol = 1e-6 * np.maximum(ec[..., None], 1) * np.abs(O.to_f64(x, dtype)).max()
    assert np.all(np.abs(si - es) <= tol + 1e-6 * np.abs(es))


def test_update_zipf_skew_and_empty_clusters():
    from flash_kmeans_cuda import _C
    B, N, K, D = 1, 262144, 8192, 128
    x, ids, s_ids, perm = _update_case(B, N, K, D, "f16", seed=9, zipf=True)
    sums = torch.zeros((B, K, D), device="cuda")
    cnt = torch.zeros((B, K), device="cuda", dtype=torch.int32)
    _C.centroid_update_sorted_indexed(_t(x, "f16"), _t(perm), _t(s_ids), sums, cnt)
    es, ec = O.update_sorted_indexed(x, perm, s_ids, K, "f16")
    c = _np(cnt)
    assert np.array_equal(c, ec) and (ec == 0).any() and ec.max() > 30000
    s = _np(sums)
    assert np.allclose(s, es, rtol=1e-5, atol=1e-5 * np.sqrt(np.maximum(ec, 1))[..., None])
    assert np.all(s[ec == 0] == 0)


# Sorted label layouts made of long runs: a run over many 128-row units and
# 64-unit blocks exercises the two-level run merge.  (label, length) per run.
LONG_RUNS = [
    ("one_run", [[(0, 600000)]], 1, 64, "f16"),
    ("block_aligned", [[(0, 16384), (1, 70000)]], 2, 128, "bf16"),
    ("mid_block", [[(0, 1000), (1, 300000), (2, 77), (3, 50000), (5, 123456)]], 6, 40, "f32"),
    ("two_rows", [[(0, 200000), (2, 100)], [(1, 57), (2, 200043)]], 3, 16, "f16"),
    ("unit_edges", [[(0, 128 * 64 * 3 - 1), (1, 1), (2, 128 * 64 + 128)]], 3, 8, "bf16"),
]


@pytest.mark.parametrize("name,runs,K,D,dtype", LONG_RUNS, ids=[r[0] for r in LONG_RUNS])
def test_update_long_runs(name, runs, K, D, dtype):
    from flash_kmeans_cuda import _C
    B = len(runs)
    N = sum(n for _, n in runs[0])
    rng = np.random.default_rng(len(name))
    s_ids = np.stack([np.concatenate([np.full(n, k, np.int32) for k, n in row]) for row in runs])
    perm = np.stack([rng.permutation(N).astype(np.int32) for _ in range(B)])
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    es, ec = O.update_sorted_indexed(x, perm, s_ids, K, dtype)
    outs = []
    for _ in range(2):
        sums = torch.full((B, K, D), 0.25, device="cuda")
        cnt = torch.full((B, K), 2, device="cuda", dtype=torch.int32)
        _C.centroid_update_sorted_indexed(_t(x, dtype), _t(perm), _t(s_ids), sums, cnt)
        outs.append((_np(sums), _np(cnt)))
    assert np.array_equal(outs[0][1], ec + 2)
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    tol = 1e-6 * np.maximum(ec[..., None], 1) * np.abs(O.to_f64(x, dtype)).max()
    assert np.all(np.abs(outs[0][0] - 0.25 - es) <= tol + 1e-4)


def test_update_adds_into_existing_sums_and_is_deterministic():
    from flash_kmeans_cuda import _C
    x, ids, s_ids, perm = _update_case(2, 9000, 37, 64, "bf16", seed=4)
    base = torch.full((2, 37, 64), 1.5, device="cuda")
    basec = torch.full((2, 37), 3, device="cuda", dtype=torch.int32)
    outs = []
    for _ in range(2):
        s, c = base.clone(), basec.clone()
        _C.centroid_update_sorted_indexed(_t(x, "bf16"), _t(perm), _t(s_ids), s, c)
        outs.append((_np(s), _np(c)))
    es, ec = O.update_sorted_indexed(x, perm, s_ids, 37, "bf16")
    assert np.array_equal(outs[0][1], ec + 3)
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    assert np.allclose(outs[0][0], es + 1.5, rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("D", [1, 7, 64, 128, 257])
def test_finalize_bit_exact(dtype, D):
    from flash_kmeans_cuda import _C
    rng = np.random.default_rng(D)
    B, K = 2, 300
    sums = (rng.standard_normal((B, K, D)) * 50).astype(np.float32)
    counts = rng.integers(0, 9, (B, K)).astype(np.int32)
    old = O.from_f32(rng.standard_normal((B, K, D)).astype(np.float32), dtype)
    out = _C.centroid_finalize(_t(sums, "f32"), _t(counts), _t(old, dtype))
    exp = O.finalize(sums, counts, old, dtype)
    got = _np(out, dtype)
    assert np.array_equal(np.asarray(got).view(np.uint8), np.asarray(exp).view(np.uint8))


def test_finalize_in_place():
    from flash_kmeans_cuda import _C
    rng = np.random.default_rng(1)
    sums = rng.standard_normal((1, 64, 32)).astype(np.float32)
    counts = rng.integers(0, 3, (1, 64)).astype(np.int32)
    old = O.from_f32(rng.standard_normal((1, 64, 32)).astype(np.float32), "f16")
    t = _t(old, "f16")
    _C.centroid_finalize(_t(sums, "f32"), _t(counts), t, out=t)
    assert np.array_equal(_np(t, "f16"), O.finalize(sums, counts, old, "f16"))


@pytest.mark.parametrize("fuse", [True, False])
@pytest.mark.parametrize("B,N,K,tile", [(1, 100000, 8192, 4096), (2, 70001, 70000, 1024),
                                        (1, 524288, 8192, 4096), (3, 9000, 300, 256),
                                        (2, 300000, 1000, 1024), (1, 524288, 8192, 8192),
                                        (3, 300000, 2000, 8192)])
def test_label_sort_recount_path(monkeypatch, B, N, K, tile, fuse):
    """With a zero spin budget (FKC_SORT_SPIN=0) every wait gives up at
    once: each tile after the first recounts its prefix from the pass's
    input, and where the first pass counts the digits itself (every tile
    resident, at most 256; FKC_SORT_FUSE=0 sends the count to the separate
    upsweep instead) each tile also counts the whole row's digits rather than
    wait at the row barrier.  The output is still the stable sort, bit for
    bit, and the workspace's first word counts the recounts: one per such
    tile and pass, plus one per tile of a fused first pass."""
    from flash_kmeans_cuda.ops import label_sort
    monkeypatch.setenv("FKC_SORT_TILE", str(tile))
    monkeypatch.setenv("FKC_SORT_SPIN", "0")
    monkeypatch.setenv("FKC_SORT_FUSE", "1" if fuse else "0")
    rng = np.random.default_rng(N + tile)
    ids = rng.integers(-1, K + 1, (B, N)).astype(np.int32)
    ws = _sort_ws(B, N, K)
    s, p = label_sort(_t(ids), K, workspace=ws)
    es, ep = O.label_sort(ids, K)
    assert np.array_equal(_np(p), ep) and np.array_equal(_np(s), es)
    ntiles = (N + tile - 1) // tile
    bits = int(np.ceil(np.log2(K + 1)))
    passes = (bits + 7) // 8
    fused = fuse and B * ntiles <= 256
    assert _recounts(ws) == B * passes * (ntiles - 1) + (B * ntiles if fused else 0)
    monkeypatch.delenv("FKC_SORT_SPIN")
    s2, p2 = label_sort(_t(ids), K, workspace=ws)
    assert torch.equal(s2, s) and torch.equal(p2, p) and _recounts(ws) == 0


def _add_mode(x, perm, ids, K, dtype, indexed=True):
    from flash_kmeans_cuda import _C
    B, N, D = x.shape
    sums = torch.zeros((B, K, D), device="cuda")
    cnt = torch.zeros((B, K), device="cuda", dtype=torch.int32)
    if indexed:
        _C.centroid_update_sorted_indexed(_t(x, dtype), _t(perm), _t(ids), sums, cnt)
    else:
        rows = np.take_along_axis(x, perm.astype(np.int64)[..., None], 1)
        _C.centroid_update_sorted(_t(rows, dtype), _t(ids), sums, cnt)
    return _np(sums), _np(cnt)


@pytest.mark.parametrize("indexed", [True, False])
def test_update_invalid_labels_between_rows_of_one_label(indexed):
    """Invalid labels between rows of one label, placed across 128-row unit
    boundaries (..., 0, 0 | -1, 0, ...), split that label into several runs
    in different waves; each run adds its share atomically, so counts are
    exact and sums match the oracle (the reference's atomics accept any
    order, update_sorted.cu:105,109)."""
    B, N, K, D, dtype = 2, 40000, 40, 64, "f16"
    rng = np.random.default_rng(17)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    ids = np.sort(rng.integers(0, K, (B, N)).astype(np.int32), axis=1)
    for u in range(1, N // 128):
        if u % 3 == 0:
            ids[:, 128 * u] = -1
        elif u % 3 == 1:
            ids[:, 128 * u - 1] = K + 1
    perm = np.stack([rng.permutation(N).astype(np.int32) for _ in range(B)])
    es, ec = O.update_sorted_indexed(x, perm, ids, K, dtype)
    s, c = _add_mode(x, perm, ids, K, dtype, indexed)
    assert np.array_equal(c, ec)
    tol = 1e-6 * np.maximum(ec[..., None], 1) * np.abs(O.to_f64(x, dtype)).max()
    assert np.all(np.abs(s - es) <= tol + 1e-5)


@pytest.mark.parametrize("K,D,dtype", [(37, 40, "bf16"), (3, 128, "f16"), (500, 7, "f32")])
def test_update_unsorted_labels(K, D, dtype):
    """Labels in no particular order: every run adds its share atomically,
    so the totals are those of the same rows grouped by label."""
    B, N = 1, 30000
    rng = np.random.default_rng(K + D)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    ids = rng.integers(-1, K, (B, N)).astype(np.int32)
    ids[:, 1000:9000] = K // 2          # one long run over many units
    perm = np.stack([rng.permutation(N).astype(np.int32)])
    es, ec = O.update_sorted_indexed(x, perm, ids, K, dtype)
    s, c = _add_mode(x, perm, ids, K, dtype)
    assert np.array_equal(c, ec)
    tol = 1e-6 * np.maximum(ec[..., None], 1) * np.abs(O.to_f64(x, dtype)).max()
    assert np.all(np.abs(s - es) <= tol + 1e-5)
