"""GPU parity of the whole Lloyd loop (batch_kmeans_Euclid) against the oracle.

* Lockstep: every iteration the GPU kernels and the oracle start from the
  same centroids, so a near-tie flip cannot cascade: labels must agree up to
  near-ties, the sort/counts are bit-exact given the GPU labels, the sums
  agree to fp32 accumulation error and finalize is bit-exact given the GPU
  sums.
* End to end: labels < 0.1% disagreement, final inertia
  within +-0.05%, centroid drift within 1e-2 relative.
* Driver contract (kmeans.py:108-195): n_iters, tol, shapes, dtypes, init not
  modified, verbose path == fused path; reference test cases
  tests/test_shapes.py, tests/test_dtypes.py, tests/test_correctness.py.
* Full-size C5 run checked through size-independent properties.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from gpu_util import inertia, near_tie_report
from oracle import kmeans_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _T(a, dtype):
    from flash_kmeans_cuda import synth
    return synth.to_torch(a, dtype)


def _N(t, dtype):
    from flash_kmeans_cuda import synth
    torch.cuda.synchronize()
    return synth.from_torch(t, dtype)


def _lockstep(x, init, K, dtype, iters):
    from flash_kmeans_cuda import _C
    from flash_kmeans_cuda.ops import label_sort, row_sqnorm
    xt = _T(x, dtype)
    cur = init.copy()
    flips = 0
    for it in range(iters):
        ct = _T(cur, dtype)
        ids_t = _C.euclid_assign(xt, ct, row_sqnorm(xt), row_sqnorm(ct))
        ids = ids_t.cpu().numpy()
        ref = O.assign(x, cur, dtype)
        nd, bad, worst = near_tie_report(x, cur, dtype, ids, ref)
        assert bad == 0, f"iter {it}: {bad} non-near-tie flips (worst {worst:.2e})"
        flips += nd
        s_t, p_t = label_sort(ids_t, K)
        es, ep = O.label_sort(ids, K)
        assert np.array_equal(p_t.cpu().numpy(), ep) and np.array_equal(s_t.cpu().numpy(), es)
        sums = torch.zeros((x.shape[0], K, x.shape[2]), device="cuda")
        cnt = torch.zeros((x.shape[0], K), device="cuda", dtype=torch.int32)
        _C.centroid_update_sorted_indexed(xt, p_t, s_t, sums, cnt)
        osum, ocnt = O.update_sorted_indexed(x, ep, es, K, dtype)
        g_cnt = cnt.cpu().numpy()
        g_sum = sums.cpu().numpy()
        assert np.array_equal(g_cnt, ocnt), f"iter {it}: counts"
        scale = np.abs(O.to_f64(x, dtype)).max() * np.maximum(ocnt, 1)[..., None]
        assert np.all(np.abs(g_sum - osum) <= 1e-6 * scale + 1e-6), f"iter {it}: sums"
        new_t = _C.centroid_finalize(sums, cnt, ct)
        g_new = _N(new_t, dtype)
        assert np.array_equal(np.asarray(g_new).view(np.uint8),
                              np.asarray(O.finalize(g_sum, g_cnt, cur, dtype)).view(np.uint8))
        cur = g_new
    return flips


@pytest.mark.parametrize("cfg_name,N", [("c2", 32768), ("c3", 32768), ("c4", 8192), ("c1", 4096)])
def test_lockstep_iterations(cfg_name, N):
    from flash_kmeans_cuda import synth
    cfg = synth.CONFIGS[cfg_name]
    x, init = synth.make(cfg, N=N)
    flips = _lockstep(x, init, cfg.K, cfg.dtype, iters=3)
    assert flips / (x.shape[0] * N * 3) < 1e-3


def _end_to_end(cfg_name, N=None, iters=None):
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    cfg = synth.CONFIGS[cfg_name]
    x, init = synth.make(cfg, N=N)
    iters = cfg.iters if iters is None else iters
    ids_t, c_t, n = batch_kmeans_Euclid(_T(x, cfg.dtype), cfg.K, max_iters=iters,
                                        tol=cfg.tol, init_centroids=_T(init, cfg.dtype))
    ids = ids_t.cpu().numpy()
    cents = _N(c_t, cfg.dtype)
    o_ids, o_c, o_n = O.kmeans(x, cfg.K, iters, cfg.tol, init, cfg.dtype)
    return cfg, x, ids, cents, n, o_ids, o_c, o_n


@pytest.mark.parametrize("cfg_name,N", [("c2", None), ("c1", None), ("c4", 16384)])
def test_end_to_end_north_star_bar(cfg_name, N):
    cfg, x, ids, cents, n, o_ids, o_c, o_n = _end_to_end(cfg_name, N)
    assert n == o_n
    frac = float((ids != o_ids).mean())
    assert frac < 1e-3, f"label disagreement {frac:.4%}"
    gi = inertia(x, cents, cfg.dtype, O.assign(x, cents, cfg.dtype))
    oi = inertia(x, o_c, cfg.dtype, O.assign(x, o_c, cfg.dtype))
    assert abs(gi - oi) / oi < 5e-4, f"inertia {gi} vs {oi}"
    gc, oc = O.to_f64(cents, cfg.dtype), O.to_f64(o_c, cfg.dtype)
    drift = np.linalg.norm(gc - oc) / np.linalg.norm(oc)
    assert drift < 1e-2, f"centroid drift {drift:.3e}"


def test_c1_golden_fixture():
    """The fp32 plumbing config against the committed oracle output."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    z = np.load(os.path.join(GOLDEN, "c1.npz"))
    cfg = synth.CONFIGS["c1"]
    x, init = synth.make(cfg)
    ids_t, c_t, n = batch_kmeans_Euclid(_T(x, "f32"), cfg.K, max_iters=10, tol=0.0,
                                        init_centroids=_T(init, "f32"))
    assert n == int(z["n_iters"])
    ids = ids_t.cpu().numpy()[0]
    assert (ids != z["labels"]).mean() < 1e-3
    c = c_t.cpu().numpy()[0]
    assert np.linalg.norm(c - z["centroids"]) / np.linalg.norm(z["centroids"]) < 1e-2


def test_tiny_golden_fixtures_on_gpu():
    from flash_kmeans_cuda import _C
    from flash_kmeans_cuda.ops import row_sqnorm
    z = np.load(os.path.join(GOLDEN, "tiny.npz"))
    n = len([k for k in z.files if k.endswith("_dtype")])
    for i in range(n):
        dtype = str(z[f"{i}_dtype"])
        x, c, ref = z[f"{i}_x"], z[f"{i}_c"], z[f"{i}_ids"]
        xt, ct = _T(x, dtype), _T(c, dtype)
        got = _C.euclid_assign(xt, ct, row_sqnorm(xt), row_sqnorm(ct)).cpu().numpy()
        nd, bad, worst = near_tie_report(x, c, dtype, got, ref)
        assert bad == 0, (i, dtype, worst)


@pytest.mark.parametrize("B,N,K,D", [(1, 100, 8, 64), (1, 257, 16, 128), (1, 1024, 1, 64),
                                     (1, 1024, 63, 64), (1, 1024, 65, 64), (1, 1024, 32, 256),
                                     (3, 2048, 32, 64),
                                     # degenerate: K > N (duplicate initial centroids,
                                     # empty clusters), one point, K = N, narrowest width
                                     (1, 100, 500, 64), (2, 1, 4, 8), (1, 7, 1, 8), (1, 3, 3, 8)])
def test_shapes_contract(B, N, K, D):
    """tests/test_shapes.py:11-31 of the reference, plus degenerate shapes."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    x = torch.randn(B, N, D, device="cuda", dtype=torch.float16)
    ids, cents, n_iters = batch_kmeans_Euclid(x, K, max_iters=3, tol=0.0)
    assert ids.shape == (B, N) and ids.dtype == torch.int32
    assert cents.shape == (B, K, D) and cents.dtype == torch.float16
    assert n_iters == 3
    assert (ids >= 0).all() and (ids < K).all()
    assert torch.isfinite(cents.float()).all()
    # every centroid is a mean of points or an initial point: inside the data's box
    lo = x.float().amin(dim=1, keepdim=True) - 1e-2
    hi = x.float().amax(dim=1, keepdim=True) + 1e-2
    assert ((cents.float() >= lo) & (cents.float() <= hi)).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_dtypes_contract(dtype):
    """tests/test_dtypes.py:11-42 of the reference."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, euclid_assign
    x = torch.randn(2, 2048, 64, device="cuda", dtype=dtype)
    ids, cents, n = batch_kmeans_Euclid(x, 32, max_iters=5, tol=0.0)
    assert cents.dtype == dtype and n == 5
    x1 = torch.randn(1, 1024, 64, device="cuda", dtype=dtype)
    a = euclid_assign(x1, x1[:, :32].contiguous(), (x1.float() ** 2).sum(-1))
    assert a.dtype == torch.int32 and (a >= 0).all() and (a < 32).all()
    s = torch.randn(1, 64, 32, device="cuda", dtype=torch.float16)
    u = euclid_assign(s, s.clone(), (s.float() ** 2).sum(-1))
    assert u.unique().numel() > 16


def _oracle_shifts(x, init, K, dtype, iters):
    """The oracle's shift (kmeans.py:104) of every iteration of a tol = 0 run."""
    cur, out = init.copy(), []
    for _ in range(iters):
        new = O.lloyd_step(x, cur, K, dtype)[0]
        out.append(O.shift(new, cur, dtype))
        cur = new
    return out


def test_tol_stops_at_the_oracles_iteration():
    """c4's batched bf16 loop with a tolerance (kmeans.py:104,190): tol is
    put between the first nonzero oracle shift that is at least 2x below
    every earlier one and the smallest earlier one, so the GPU loop must stop
    after exactly the oracle's iteration; the result equals a tol = 0 run of
    that many iterations bit for bit, and init is not modified."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    cfg = synth.CONFIGS["c4"]
    x, init = synth.make(cfg, N=8192)
    sh = _oracle_shifts(x, init, cfg.K, "bf16", 14)
    i = next(j for j in range(1, len(sh)) if 0 < 2 * sh[j] <= min(sh[:j]))
    tol = float(np.sqrt(sh[i] * min(sh[:i])))
    o_n = i + 1
    assert o_n == O.kmeans(x, cfg.K, 50, tol, init, "bf16")[2]
    xt, it = _T(x, "bf16"), _T(init, "bf16")
    ids_a, c_a, n_a = batch_kmeans_Euclid(xt, cfg.K, max_iters=50, tol=tol, init_centroids=it)
    assert n_a == o_n, (n_a, o_n, tol, sh)
    ids_b, c_b, n_b = batch_kmeans_Euclid(xt, cfg.K, max_iters=n_a, tol=0.0, init_centroids=it)
    assert n_b == n_a
    assert torch.equal(ids_a, ids_b) and torch.equal(c_a, c_b)
    assert torch.equal(it, _T(init, "bf16")), "init_centroids was modified"


@pytest.mark.parametrize("cfg_name,N", [("c3", 65536), ("c2", 32768), ("c4", 8192),
                                        ("c5", 131072)])
def test_loop_sort_paths_agree(monkeypatch, cfg_name, N):
    """The Lloyd loop gives the same bits whichever way its sorts count
    digits (in the first pass, or in a separate upsweep: FKC_SORT_FUSE=0)
    and when every wait of every sort gives up at once (FKC_SORT_SPIN=0:
    each tile recounts from the pass's input instead of waiting).  Several
    iterations on one workspace also exercise the status words' epochs."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    cfg = synth.CONFIGS[cfg_name]
    x, init = synth.make(cfg, N=N)
    xt, it = _T(x, cfg.dtype), _T(init, cfg.dtype)
    a = batch_kmeans_Euclid(xt, cfg.K, max_iters=4, init_centroids=it)
    for fuse, spin in [("0", None), ("1", "0"), ("0", "0")]:
        monkeypatch.setenv("FKC_SORT_FUSE", fuse)
        if spin is None:
            monkeypatch.delenv("FKC_SORT_SPIN", raising=False)
        else:
            monkeypatch.setenv("FKC_SORT_SPIN", spin)
        b = batch_kmeans_Euclid(xt, cfg.K, max_iters=4, init_centroids=it)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), (fuse, spin)


@pytest.mark.parametrize("cus", ["64", "16"])
def test_loop_with_the_plans_of_a_smaller_part(monkeypatch, cus):
    """FKC_CUS plans every grid as for a part with fewer compute units
    (fewer sort tiles resident at once, so counter-ordered tiles and an
    upsweep; fewer assign workgroups to fill it, so no centroid slices): the
    loop gives the same bits as with the device's own plans (c5's shape at
    N = 262144: 64 sort tiles of 4096 keys, resident on 64 CUs, not on 16;
    c5's share of one of 8 GPUs: 3 centroid slices on 256 CUs, none on 64 or
    16; c4's shape at N = 16384)."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    for name, N in [("c5", 262144), ("c5s8", 65536), ("c4", 16384)]:
        cfg = synth.CONFIGS[name]
        x, init = synth.make(cfg, N=N)
        xt, it = _T(x, cfg.dtype), _T(init, cfg.dtype)
        monkeypatch.delenv("FKC_CUS", raising=False)
        a = batch_kmeans_Euclid(xt, cfg.K, max_iters=3, init_centroids=it)
        monkeypatch.setenv("FKC_CUS", cus)
        b = batch_kmeans_Euclid(xt, cfg.K, max_iters=3, init_centroids=it)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), (name, cus)


def test_loop_sort_recount_word_is_zero_on_an_idle_gpu(monkeypatch):
    """A c5 loop call on an otherwise idle GPU never runs out of a sort wait:
    the recount word (fkc_kmeans_sort_recounts_offset) reads 0; with
    FKC_SORT_SPIN=0 every wait gives up at once and it counts them."""
    from flash_kmeans_cuda import _lib, synth
    cfg = synth.CONFIGS["c5"]
    x, init = synth.make(cfg, N=131072)
    xt, it = _T(x, cfg.dtype), _T(init, cfg.dtype)
    L = _lib.lib
    B, N, K, D = 1, 131072, cfg.K, cfg.D

    def run():
        ws = torch.full((L.fkc_kmeans_workspace_bytes(B, N, K, D, 1, 3),), 0x5A,
                        dtype=torch.uint8, device="cuda")
        cents = torch.empty_like(it)
        ids = torch.empty((B, N), dtype=torch.int32, device="cuda")
        _lib.check(L.fkc_kmeans_lloyd_from(
            xt.data_ptr(), it.data_ptr(), cents.data_ptr(), ids.data_ptr(), B, N, K, D, 1,
            3, 0.0, ws.data_ptr(), ws.numel(), _lib.stream_of(xt), None, None), "lloyd")
        off = L.fkc_kmeans_sort_recounts_offset(B, N, K, D, 1, 3)
        torch.cuda.synchronize()
        return int(ws[off:off + 4].view(torch.int32).item()), ids, cents

    n0, ids0, c0 = run()
    assert n0 == 0
    monkeypatch.setenv("FKC_SORT_SPIN", "0")
    n1, ids1, c1 = run()
    assert n1 > 0
    assert torch.equal(ids0, ids1) and torch.equal(c0, c1)


@pytest.mark.parametrize("tile", [256, 512])
def test_loop_with_counter_ordered_sort_tiles(monkeypatch, tile):
    """Sort grids of more than 256 tiles take their tile index from a per-row
    counter that grows over the loop's iterations (each call offsets it by
    its sequence number) and count digits in a separate kernel.  c4's 8
    batch rows at N = 16384 make 512 tiles of 256 keys (that path) or 256
    tiles of 512 keys (resident: block-index tiles, digits counted in the
    first pass); either way the loop gives the same bits as with the
    default tiles, twice in a row on fresh workspaces."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    cfg = synth.CONFIGS["c4"]
    x, init = synth.make(cfg, N=16384)
    xt, it = _T(x, cfg.dtype), _T(init, cfg.dtype)
    a = batch_kmeans_Euclid(xt, cfg.K, max_iters=6, init_centroids=it)
    monkeypatch.setenv("FKC_SORT_TILE", str(tile))
    b = batch_kmeans_Euclid(xt, cfg.K, max_iters=6, init_centroids=it)
    c = batch_kmeans_Euclid(xt, cfg.K, max_iters=6, init_centroids=it)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.equal(b[0], c[0]) and torch.equal(b[1], c[1])


def test_verbose_path_equals_fused_loop(capsys):
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    cfg = synth.CONFIGS["c2"]
    x, init = synth.make(cfg, N=8192)
    xt, it = _T(x, "f16"), _T(init, "f16")
    a = batch_kmeans_Euclid(xt, cfg.K, max_iters=4, init_centroids=it)
    b = batch_kmeans_Euclid(xt, cfg.K, max_iters=4, init_centroids=it, verbose=True)
    assert "Iter 3, center shift" in capsys.readouterr().out
    assert a[2] == b[2] == 4
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1], b[1])


@pytest.mark.parametrize("B,N,K,D,dtype", [(1, 600000, 2, 16, "f16"), (2, 300000, 5, 72, "bf16")])
def test_few_clusters_many_points(B, N, K, D, dtype):
    """Clusters of 10^5 points: runs over many units and blocks in the fused
    loop's overwrite-mode update; fused loop == per-op path, and the oracle
    bar holds."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    rng = np.random.default_rng(N + K)
    centres = 3 * rng.standard_normal((K, D)).astype(np.float32)
    blob = rng.integers(0, K, (B, N))
    x = O.from_f32(centres[blob] + rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    init = np.ascontiguousarray(x[:, :K])
    xt, it = _T(x, dtype), _T(init, dtype)
    a = batch_kmeans_Euclid(xt, K, max_iters=4, init_centroids=it)
    b = batch_kmeans_Euclid(xt, K, max_iters=4, init_centroids=it, verbose=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    o_ids, o_c, o_n = O.kmeans(x, K, 4, 0.0, init, dtype)
    assert (a[0].cpu().numpy() != o_ids).mean() < 1e-3
    gc, oc = O.to_f64(_N(a[1], dtype), dtype), O.to_f64(o_c, dtype)
    assert np.linalg.norm(gc - oc) / np.linalg.norm(oc) < 1e-2


@pytest.mark.parametrize("B,N,K,D,dtype", [(3, 90000, 700, 128, "f16"), (2, 150000, 300, 64, "bf16"),
                                           (1, 40000, 4000, 8, "f32")])
def test_loop_runs_of_every_length(B, N, K, D, dtype):
    """Zipf-sized clusters (runs from a few rows to tens of thousands:
    inside one unit, over a few units, over whole 64-unit blocks): the
    loop, whose update completes every run over several units inside its
    run kernel, equals the per-op path (separate merge kernel, pinned by
    the lockstep tests) bit for bit over three iterations; one iteration
    assigns as the oracle does up to near-ties."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    rng = np.random.default_rng(K + D)
    centres = 3 * rng.standard_normal((B, K, D)).astype(np.float32)
    blob = rng.choice(K, (B, N), p=synth.zipf_probs(K, 1.1))
    x = O.from_f32(np.take_along_axis(centres, blob[..., None], 1)
                   + 0.5 * rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    init = np.ascontiguousarray(x[:, rng.choice(N, K, replace=False)])
    xt, it = _T(x, dtype), _T(init, dtype)
    a = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
    b = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it, verbose=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    one = batch_kmeans_Euclid(xt, K, max_iters=1, init_centroids=it)[0].cpu().numpy()
    nd, bad, worst = near_tie_report(x, init, dtype, one, O.assign(x, init, dtype))
    assert bad == 0 and nd / one.size < 1e-3, (nd, bad, worst)


@pytest.mark.parametrize("B,N,K,D,dtype", [(1, 200000, 2, 1100, "f16"), (2, 120000, 3, 600, "bf16")])
def test_few_clusters_wide_rows(B, N, K, D, dtype):
    """Runs over many full 64-unit blocks at widths whose update splits the
    row over several column blocks (grid z > 1): the loop sums each block
    inside its run kernel, one arrival counter per column block, and must
    equal the per-op path (separate block kernel) bit for bit."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    rng = np.random.default_rng(N + D)
    centres = 3 * rng.standard_normal((K, D)).astype(np.float32)
    blob = rng.integers(0, K, (B, N))
    x = O.from_f32(centres[blob] + rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    init = np.ascontiguousarray(x[:, :K])
    xt, it = _T(x, dtype), _T(init, dtype)
    del x
    a = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
    b = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it, verbose=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("D,dtype", [(512, "bf16"), (520, "f32"), (264, "f16"), (3, "f32")])
def test_fused_loop_equals_per_op_path_across_widths(D, dtype):
    """The loop finalizes inside the update for D <= 512 and with its own
    kernel above; both must equal the per-op path (separate update and
    finalize kernels, c_sq recomputed) bit for bit."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    rng = np.random.default_rng(D)
    x = O.from_f32(rng.standard_normal((2, 3000, D)).astype(np.float32), dtype)
    init = np.ascontiguousarray(x[:, :40])
    xt, it = _T(x, dtype), _T(init, dtype)
    a = batch_kmeans_Euclid(xt, 40, max_iters=3, init_centroids=it)
    b = batch_kmeans_Euclid(xt, 40, max_iters=3, init_centroids=it, verbose=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("B,N,K,D,dtype", [
    (1, 20000, 300, 128, "f16"),    # 2 sort passes
    (3, 10000, 256, 64, "bf16"),    # 1 sort pass (labels from the assign skip the sentinel bin)
    (2, 30000, 2000, 32, "bf16"),   # 32-feature direct stages
    (1, 80000, 70000, 16, "f16"),   # 3 sort passes
])
def test_loop_sort_digit_counts(B, N, K, D, dtype):
    """The loop's label sort alternates two state phases over iterations
    (digit counts, tile status words, tile counters) and clears them once
    per call; the per-op path runs standalone sorts.  Both must agree bit
    for bit over 3 iterations, for 1, 2 and 3 sort passes."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    rng = np.random.default_rng(K + D)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    init = np.ascontiguousarray(x[:, :K])
    xt, it = _T(x, dtype), _T(init, dtype)
    a = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
    b = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it, verbose=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("B,N,K,dtype", [(1, 6000, 4500, "f16"), (2, 6000, 5000, "bf16")])
def test_loop_with_sliced_assign(monkeypatch, B, N, K, dtype):
    """Shapes with few points and many centroids slice K inside the loop's
    assign (partial winners in the loop workspace): the loop, the per-op
    path and the loop with slicing switched off (FKC_KSPLIT=1) agree bit for
    bit over 3 iterations."""
    from flash_kmeans_cuda import _lib, batch_kmeans_Euclid
    monkeypatch.delenv("FKC_KSPLIT", raising=False)
    dt = {"f16": 1, "bf16": 2}[dtype]
    assert _lib.lib.fkc_euclid_assign_workspace_bytes(B, N, K, 128, dt) > 0
    rng = np.random.default_rng(K)
    x = O.from_f32(rng.standard_normal((B, N, 128)).astype(np.float32), dtype)
    init = np.ascontiguousarray(x[:, :K])
    xt, it = _T(x, dtype), _T(init, dtype)
    a = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
    b = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it, verbose=True)
    monkeypatch.setenv("FKC_KSPLIT", "1")
    c = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=it)
    for r in (b, c):
        assert torch.equal(a[0], r[0]) and torch.equal(a[1], r[1])


@pytest.mark.parametrize("B,N,K,D,dtype,ksplit,save,tol", [
    (1, 16384, 8192, 128, "f16", None, None, 0.0),  # the plan's own slices (kept scores)
    (1, 12000, 6000, 128, "bf16", "3", "0", 0.0),   # re-score epilogue, three slices
    (2, 5000, 4500, 128, "f16", "2", "1", 0.0),     # batches, kept scores
    (1, 9000, 5000, 64, "bf16", "4", None, 0.0),    # D = 64, four slices
    (1, 7000, 4097, 128, "f16", "3", None, 1e-3),   # tol stop: later launches exit at once
])
def test_loop_with_sliced_assign_variants(monkeypatch, B, N, K, D, dtype,
                                          ksplit, save, tol):
    """Sliced assigns inside the Lloyd loop (its workspace holding the
    partial winners) across slice counts, both epilogues (kept scores and
    re-score), batches, D = 64 and a tol stop: the loop and the per-op path
    give the same labels, centroids and iteration count."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    for k, v in (("FKC_KSPLIT", ksplit), ("FKC_SAVE", save)):
        if v is None:
            monkeypatch.delenv(k, raising=False)
        else:
            monkeypatch.setenv(k, v)
    print(f"B={B} N={N} K={K} D={D} {dtype} ksplit={ksplit} save={save} tol={tol}", flush=True)
    rng = np.random.default_rng(N + K)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    init = np.ascontiguousarray(x[:, :K])
    xt, it = _T(x, dtype), _T(init, dtype)
    a = batch_kmeans_Euclid(xt, K, max_iters=6, tol=tol, init_centroids=it)
    b = batch_kmeans_Euclid(xt, K, max_iters=6, tol=tol, init_centroids=it, verbose=True)
    assert a[2] == b[2]
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("B,N,K,D,dtype,tol", [
    (8, 65536, 1024, 64, "bf16", 0.0),    # c4's shape: resident by default
    (2, 40000, 700, 64, "bf16", 1e-4),    # forced resident, tol stop
    (1, 30000, 2000, 32, "f16", 0.0),     # D = 32, eight tiles per wave
])
def test_loop_with_resident_assign(monkeypatch, B, N, K, D, dtype, tol):
    """The Lloyd loop with the centroid-resident assign forced on and off:
    labels, centroids and iteration count equal bit for bit (clustered data,
    so the loop moves the centroids and reassigns points)."""
    from flash_kmeans_cuda import batch_kmeans_Euclid
    rng = np.random.default_rng(N + K)
    centers = rng.standard_normal((B, 64, D)).astype(np.float32) * 3.0
    pick = rng.integers(0, 64, (B, N))
    pts = np.take_along_axis(centers, pick[..., None], axis=1)
    pts = pts + rng.standard_normal((B, N, D)).astype(np.float32)
    x = O.from_f32(pts, dtype)
    init = np.ascontiguousarray(x[:, :K])
    xt, it = _T(x, dtype), _T(init, dtype)
    runs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("FKC_RESIDENT", flag)
        runs.append(batch_kmeans_Euclid(xt, K, max_iters=6, tol=tol, init_centroids=it))
    (ia, ca, na), (ib, cb, nb) = runs
    assert na == nb
    assert torch.equal(ia, ib) and torch.equal(ca, cb)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_init_kept_and_entry_points_agree(dtype):
    """batch_kmeans_Euclid never writes init_centroids (the copy is fused
    into the loop's first launch); fkc_kmeans_lloyd (in place) and
    fkc_kmeans_lloyd_from (init -> separate output) give the same bits; with
    max_iters = 0 the returned centroids are the initial ones."""
    from flash_kmeans_cuda import _lib, batch_kmeans_Euclid
    B, N, K, D = 2, 5000, 300, 64
    rng = np.random.default_rng(7)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype)
    xt = _T(x, dtype)
    init = xt[:, :K].clone()
    keep = init.clone()
    ids, cents, n = batch_kmeans_Euclid(xt, K, max_iters=3, init_centroids=init)
    assert torch.equal(init, keep) and n == 3
    dt = _lib.dtype_code(xt.dtype)
    ws = _lib.workspace(_lib.lib.fkc_kmeans_workspace_bytes(B, N, K, D, dt, 3), xt.device)
    inplace = init.clone()
    ids2 = torch.empty_like(ids)
    _lib.check(_lib.lib.fkc_kmeans_lloyd(
        xt.data_ptr(), inplace.data_ptr(), ids2.data_ptr(), B, N, K, D, dt, 3, 0.0,
        ws.data_ptr(), ws.numel(), _lib.stream_of(xt), None, None), "lloyd")
    torch.cuda.synchronize()
    assert torch.equal(inplace, cents) and torch.equal(ids2, ids)
    ids0, c0, n0 = batch_kmeans_Euclid(xt, K, max_iters=0, init_centroids=init)
    assert n0 == 0 and torch.equal(c0, keep) and c0.data_ptr() != init.data_ptr()


def test_large_k_three_sort_passes():
    """1M points, K = 65536 (17-bit labels: three sort passes, 8-tile assign
    on 2048 workgroups): invariants at a scale the oracle cannot run whole —
    labels in range, every point counted once, the sort equal to torch's
    stable sort, finite centroids — and a sampled label check against the
    oracle with the returned centroids."""
    from flash_kmeans_cuda import _C, batch_kmeans_Euclid
    from flash_kmeans_cuda.ops import label_sort, row_sqnorm
    B, N, K, D = 1, 1048576, 65536, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(B, N, D, device="cuda", generator=g).to(torch.float16)
    ids, c, n = batch_kmeans_Euclid(x, K, max_iters=2, init_centroids=x[:, :K].clone())
    assert n == 2 and int(ids.min()) >= 0 and int(ids.max()) < K
    assert torch.isfinite(c.float()).all()
    ids2 = _C.euclid_assign(x, c, row_sqnorm(x), row_sqnorm(c))
    s, p = label_sort(ids2, K)
    assert torch.equal(s[0].long(), torch.sort(ids2[0].long(), stable=True).values)
    assert torch.equal(p[0].long(), torch.sort(ids2[0].long(), stable=True).indices)
    assert int(torch.bincount(ids2[0].long(), minlength=K).sum()) == N
    sub = np.random.default_rng(0).choice(N, 1024, replace=False)
    xs = x[:, sub].cpu().numpy()
    cs = c.cpu().numpy()
    got = ids2[:, sub].cpu().numpy()
    ref = O.assign(xs, cs, "f16")
    nd, bad, worst = near_tie_report(xs, cs, "f16", got, ref)
    assert bad == 0, f"{bad} non-near-tie disagreements (worst {worst:.3e})"


def test_deterministic_loop():
    from flash_kmeans_cuda import batch_kmeans_Euclid, synth
    cfg = synth.CONFIGS["c3"]
    x, init = synth.make(cfg, N=65536)
    xt, it = _T(x, "f16"), _T(init, "f16")
    a = batch_kmeans_Euclid(xt, cfg.K, max_iters=3, init_centroids=it)
    b = batch_kmeans_Euclid(xt, cfg.K, max_iters=3, init_centroids=it)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_c5_full_size_properties():
    """Full mega config: invariants that do not need the oracle at full size."""
    from flash_kmeans_cuda import _C, batch_kmeans_Euclid, synth
    from flash_kmeans_cuda.ops import label_sort, row_sqnorm
    cfg = synth.CONFIGS["c5"]
    x, init = synth.make(cfg)
    xt, it = _T(x, "f16"), _T(init, "f16")
    ids, cents, n = batch_kmeans_Euclid(xt, cfg.K, max_iters=2, init_centroids=it)
    assert n == 2 and ids.min() >= 0 and ids.max() < cfg.K
    s, p = label_sort(ids, cfg.K)
    assert torch.equal(torch.sort(p.long(), dim=1).values[0],
                       torch.arange(cfg.N, device="cuda"))
    assert bool((s[:, 1:] >= s[:, :-1]).all())
    assert torch.equal(s.long(), torch.gather(ids.long(), 1, p.long()))
    sums = torch.zeros((1, cfg.K, cfg.D), device="cuda")
    cnt = torch.zeros((1, cfg.K), device="cuda", dtype=torch.int32)
    _C.centroid_update_sorted_indexed(xt, p, s, sums, cnt)
    assert int(cnt.sum()) == cfg.N
    assert torch.equal(cnt[0].long(), torch.bincount(ids[0].long(), minlength=cfg.K))
    tot = xt.float().sum(1)
    assert torch.allclose(sums.sum(1), tot, rtol=1e-4, atol=1e-1)
    # labels of a sampled subset against the oracle, with the GPU's centroids
    rng = np.random.default_rng(0)
    sub = rng.choice(cfg.N, 4096, replace=False)
    c_np = _N(cents, "f16")
    ids2 = _C.euclid_assign(xt, cents, row_sqnorm(xt), row_sqnorm(cents)).cpu().numpy()
    ref = O.assign(x[:, sub], c_np, "f16")
    nd, bad, worst = near_tie_report(x[:, sub], c_np, "f16", ids2[:, sub], ref)
    assert bad == 0 and nd / sub.size < 2e-3


def test_lloyd_iteration_captures_into_a_graph():
    """fkc_kmeans_lloyd with tol <= 0 and no host count is capture-safe (no
    allocation, no synchronisation, no memset nodes).  One captured
    iteration is replayed several times, with eager work and
    synchronisations between replays, and every replay must equal the eager
    iteration from the same starting centroids bit for bit."""
    from flash_kmeans_cuda import _lib, synth
    L = _lib.lib
    cfg = synth.CONFIGS["c2"]
    x_np, init_np = synth.make(cfg, N=16384)
    x = synth.to_torch(x_np, "f16")
    B, N, K, D = 1, 16384, cfg.K, cfg.D
    dt = _lib.dtype_code(x.dtype)
    ws = _lib.workspace(L.fkc_kmeans_workspace_bytes(B, N, K, D, dt, 1), x.device)
    cents = synth.to_torch(init_np, "f16").clone()
    ids = torch.empty((B, N), dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()

    def one():
        _lib.check(L.fkc_kmeans_lloyd(x.data_ptr(), cents.data_ptr(), ids.data_ptr(), B, N, K,
                                      D, dt, 1, 0.0, ws.data_ptr(), ws.numel(),
                                      s.cuda_stream, None, None), "kmeans_lloyd")

    g = torch.cuda.CUDAGraph()
    start = cents.clone()
    with torch.cuda.graph(g, stream=s):
        one()
    torch.cuda.synchronize()
    state = start.clone()
    for rep in range(4):
        cents.copy_(state)
        with torch.cuda.stream(s):
            one()                      # eager reference from `state`
        torch.cuda.synchronize()
        e_c, e_i = cents.clone(), ids.clone()
        cents.copy_(state)
        ids.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(cents, e_c), f"replay {rep}: centroids"
        assert torch.equal(ids, e_i), f"replay {rep}: labels"
        state = e_c


_FIRST_CALL_CAPTURED = r'''
import sys, torch
sys.path.insert(0, sys.argv[1])
from flash_kmeans_cuda import _lib
L = _lib.lib
B, N, K, D = 2, 8192, 700, 64
g = torch.Generator(device="cuda").manual_seed(0)
x = torch.randn(B, N, D, device="cuda", generator=g).to(torch.bfloat16)
cents = x[:, :K].contiguous().clone()
ids = torch.empty((B, N), dtype=torch.int32, device="cuda")
dt = _lib.dtype_code(x.dtype)
ws = _lib.workspace(L.fkc_kmeans_workspace_bytes(B, N, K, D, dt, 1), x.device)
s = torch.cuda.Stream()


def one():
    _lib.check(L.fkc_kmeans_lloyd(x.data_ptr(), cents.data_ptr(), ids.data_ptr(), B, N, K,
                                  D, dt, 1, 0.0, ws.data_ptr(), ws.numel(), s.cuda_stream,
                                  None, None), "kmeans_lloyd")


start = cents.clone()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):
    one()
torch.cuda.synchronize()
for rep in range(3):
    cents.copy_(start)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        one()
    torch.cuda.synchronize()
    e_c, e_i = cents.clone(), ids.clone()
    cents.copy_(start)
    ids.fill_(-1)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(cents, e_c) and torch.equal(ids, e_i), f"replay {rep}"
print("graph-ok", flush=True)
'''


def test_resident_assign_first_launched_inside_graph_capture():
    """A process whose first centroid-resident launch is inside HIP graph
    capture (the launcher raises the kernel's LDS attribute on a device's
    first use): every replay of the captured Lloyd iteration equals the
    eager one.  A fresh interpreter, so no earlier call raised it."""
    import subprocess
    import sys
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "flash-kmeans-cuda_amd")
    env = dict(os.environ, FKC_RESIDENT="1")
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, pkg], env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "graph-ok" in r.stdout, (r.stdout[-2000:], r.stderr[-2000:])


def test_two_threads_on_two_streams_with_profiling():
    """The entry points keep no state across calls beyond the profiling
    hook: two host threads run the Lloyd loop at once, each on its own
    stream with its own workspace, while a third drains the profiling
    events.  Each result equals the same call run alone, bit for bit, and the
    hook counts every iteration's assign exactly once."""
    import threading
    import time
    from flash_kmeans_cuda import _lib, batch_kmeans_Euclid
    L = _lib.lib
    rng = np.random.default_rng(11)
    jobs = []
    for (B, N, K, D, dtype) in [(1, 20000, 1100, 128, "f16"), (2, 8000, 300, 64, "bf16")]:
        x = _T(O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32), dtype), dtype)
        jobs.append((x, x[:, :K].clone(), K))
    iters = 4
    alone = [batch_kmeans_Euclid(x, K, max_iters=iters, init_centroids=c)
             for (x, c, K) in jobs]
    torch.cuda.synchronize()

    L.fkc_profile_enable(1)
    try:
        out, errs = [None] * len(jobs), []

        def run(i):
            try:
                x, c, K = jobs[i]
                s = torch.cuda.Stream()
                s.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(s):
                    r = batch_kmeans_Euclid(x, K, max_iters=iters, init_centroids=c)
                s.synchronize()
                out[i] = r
            except Exception as e:  # surfaced below
                errs.append(e)

        threads = [threading.Thread(target=run, args=(i,)) for i in range(len(jobs))]
        for t in threads:
            t.start()
        tot = _lib.ctypes.c_double(0.0)
        launches = _lib.ctypes.c_int64(0)
        while any(t.is_alive() for t in threads):
            _lib.check(L.fkc_profile_assign_ms(_lib.ctypes.byref(tot),
                                               _lib.ctypes.byref(launches)), "profile")
            time.sleep(0.001)
        for t in threads:
            t.join()
        assert not errs, errs
        _lib.check(L.fkc_profile_assign_ms(_lib.ctypes.byref(tot),
                                           _lib.ctypes.byref(launches)), "profile")
    finally:
        L.fkc_profile_enable(0)
    assert launches.value == iters * len(jobs) and tot.value > 0.0
    for a, b in zip(alone, out):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and a[2] == b[2]


@pytest.mark.parametrize("period,iters,want", [(5, 12, 2), (5, 2, 0), (5, 3, 1), (4, 9, 2), (1, 3, 3)])
def test_profile_hook_times_stratum_midpoints(period, iters, want):
    """fkc_profile_enable(k) times the middle iteration of every run of k
    (iterations k/2, k/2 + k, ...): the launch count follows, and a loop
    shorter than k/2 + 1 iterations times none."""
    from flash_kmeans_cuda import _lib, batch_kmeans_Euclid, synth
    L = _lib.lib
    cfg = synth.CONFIGS["c2"]
    x, init = synth.make(cfg, N=4096)
    xt, it = _T(x, "f16"), _T(init, "f16")
    tot = _lib.ctypes.c_double(0.0)
    launches = _lib.ctypes.c_int64(0)
    L.fkc_profile_enable(period)
    try:
        batch_kmeans_Euclid(xt, cfg.K, max_iters=iters, init_centroids=it)
        _lib.check(L.fkc_profile_assign_ms(_lib.ctypes.byref(tot),
                                           _lib.ctypes.byref(launches)), "profile")
    finally:
        L.fkc_profile_enable(0)
    assert launches.value == want
    assert (tot.value > 0.0) == (want > 0)
