"""GPU parity of the device quality evaluator (fkc_assigned_inertia,
fkc_sampled_inertia and flash_kmeans_cuda.quality) against the oracle, which
restates the reference's benchmarks/quality_compare.py:63-116.

Bar: per-element differences and squares are fp32 on both sides and the
totals fp64, so only the fp64 summation order differs: relative error
<= 1e-10 at these sizes.  Empty-cluster counts are exact (one K-bin
histogram over every batch row's labels, as the reference's flattened
bincount).  The sampled inertia is the nearest-centroid distance of each
sampled point; the reference's fp32 form x_sq + c_sq - 2<x,c> agrees with it
to fp32 rounding: relative error <= 1e-5.  The device result is bitwise
reproducible.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kmeans_oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dtype=None):
    from flash_kmeans_cuda import synth
    if dtype is None:
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return synth.to_torch(a, dtype)


def _device(x, ids, c, dtype):
    """(inertia per batch row, empty-cluster count) through the C ABI."""
    from flash_kmeans_cuda import _lib
    xt, ct = _t(x, dtype), _t(c, dtype)
    it = _t(ids.astype(np.int32))
    B, N, D = x.shape
    K = c.shape[1]
    inertia = torch.empty(B, dtype=torch.float64, device="cuda")
    empty = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    ws = _lib.workspace(_lib.lib.fkc_quality_workspace_bytes(B, N, K), torch.device("cuda"))
    _lib.check(_lib.lib.fkc_assigned_inertia(
        xt.data_ptr(), ct.data_ptr(), it.data_ptr(), B, N, K, D, _lib.dtype_code(xt.dtype),
        inertia.data_ptr(), empty.data_ptr(), ws.data_ptr(), ws.numel(),
        _lib.stream_of(xt)), "assigned_inertia")
    torch.cuda.synchronize()
    return inertia.cpu().numpy(), int(empty.item())


CASES = [(1, 4096, 64, 128, "f16"), (3, 1000, 37, 40, "bf16"), (2, 777, 5, 7, "f32"),
         (1, 65, 300, 256, "f16"), (1, 200000, 1024, 64, "bf16"), (2, 1, 3, 520, "f32")]


@pytest.mark.parametrize("B,N,K,D,dtype", CASES)
def test_inertia_and_empty_match_oracle(B, N, K, D, dtype):
    rng = np.random.default_rng(B * N + K + D)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 2, dtype)
    c = O.from_f32(rng.standard_normal((B, K, D)).astype(np.float32) * 2, dtype)
    ids = rng.integers(0, K, (B, N)).astype(np.int32)
    ids[:, ::13] = -1           # invalid labels add nothing
    ids[:, 5::29] = K + 2
    got_i, got_e = _device(x, ids, c, dtype)
    want_i = O.assigned_inertia(x, ids, c, dtype)
    want_e = O.empty_clusters(ids, K)
    assert np.allclose(got_i, want_i, rtol=1e-10, atol=0), (got_i, want_i)
    assert got_e == want_e


def test_bitwise_reproducible():
    rng = np.random.default_rng(3)
    x = O.from_f32(rng.standard_normal((1, 300000, 128)).astype(np.float32), "f16")
    c = O.from_f32(rng.standard_normal((1, 2048, 128)).astype(np.float32), "f16")
    ids = rng.integers(0, 2048, (1, 300000)).astype(np.int32)
    a = _device(x, ids, c, "f16")
    b = _device(x, ids, c, "f16")
    assert a[0].tobytes() == b[0].tobytes() and a[1] == b[1]


def test_python_quality_module():
    from flash_kmeans_cuda import euclid_assign, quality, synth
    from flash_kmeans_cuda.ops import row_sqnorm
    cfg = synth.CONFIGS["c3"]
    x, init = synth.make(cfg, N=32768)
    xt, ct = _t(x, "f16"), _t(init, "f16")
    ev = quality.evaluate(xt, ct)
    ids = euclid_assign(xt, ct, row_sqnorm(xt), row_sqnorm(ct))
    assert torch.equal(ev["ids"], ids)
    ids_np = ids.cpu().numpy()
    want = O.assigned_inertia(x, ids_np, init, "f16").sum()
    assert abs(ev["inertia"] - want) <= 1e-10 * want
    assert ev["empty_clusters"] == O.empty_clusters(ids_np, cfg.K)
    assert quality.assigned_inertia(xt, ids, ct) == ev["inertia"]
    assert quality.empty_clusters(ids, cfg.K) == ev["empty_clusters"]
    # empty count alone (no x): every label present except one
    lab = torch.arange(10, dtype=torch.int32, device="cuda").repeat(1, 3)
    lab[lab == 7] = 3
    assert quality.empty_clusters(lab, 10) == 1


def test_c5_full_size_inertia_against_host_fp64():
    """Full mega size: two Lloyd iterations, then the device evaluator's
    inertia of the returned labels against numpy's (O(N*D), cheap at full
    size), and the re-assigned inertia is not above it (Lloyd's monotone
    assignment step)."""
    from flash_kmeans_cuda import batch_kmeans_Euclid, quality, synth
    cfg = synth.CONFIGS["c5"]
    x, init = synth.make(cfg)
    xt = _t(x, "f16")
    ids, cents, n = batch_kmeans_Euclid(xt, cfg.K, max_iters=2, tol=0.0,
                                        init_centroids=_t(init, "f16"))
    got = quality.assigned_inertia(xt, ids, cents)
    from flash_kmeans_cuda import synth as S
    want = O.assigned_inertia(x, ids.cpu().numpy(), S.from_torch(cents, "f16"), "f16").sum()
    assert abs(got - want) <= 1e-10 * want
    ev = quality.evaluate(xt, cents)
    assert ev["inertia"] <= got * (1 + 1e-6)
    assert 0 <= ev["empty_clusters"] < cfg.K


def test_empty_clusters_flattened_over_batch_rows():
    """At B > 1 a k is empty only when no row carries it (the reference's
    bincount over ids.reshape(-1), quality_compare.py:86-88), checked against
    torch.bincount on the host."""
    from flash_kmeans_cuda import quality
    rng = np.random.default_rng(5)
    for B, N, K in [(2, 4, 6), (8, 500, 1024), (3, 2000, 50)]:
        ids = rng.integers(0, K, (B, N)).astype(np.int32)
        if B == 2:
            ids = np.array([[0, 1, 1, 4], [3, 3, 0, 4]], np.int32)
        want = int((torch.bincount(torch.from_numpy(ids).reshape(-1).long(),
                                   minlength=K) == 0).sum())
        assert quality.empty_clusters(_t(ids), K) == want == O.empty_clusters(ids, K)
        # per-row counts differ wherever some row leaves a bin empty
        per_row = sum(O.empty_clusters(ids[b:b + 1], K) for b in range(B))
        assert per_row != want or per_row == 0


SAMPLE_CASES = [(1, 4096, 64, 128, "f16", 512), (3, 1000, 37, 40, "bf16", 999),
                (2, 777, 5, 7, "f32", 100), (8, 65536, 1024, 64, "bf16", 4096),
                (1, 524288, 8192, 128, "f16", 4096)]


@pytest.mark.parametrize("B,N,K,D,dtype,S", SAMPLE_CASES)
def test_sampled_inertia_matches_oracle(B, N, K, D, dtype, S):
    """fkc_sampled_inertia against the oracle's restatement of
    _sample_exact_inertia (quality_compare.py:91-116) on the same indices."""
    from flash_kmeans_cuda import quality
    rng = np.random.default_rng(B + N + K + D + S)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 2, dtype)
    c = O.from_f32(rng.standard_normal((B, K, D)).astype(np.float32) * 2, dtype)
    idx = rng.permutation(N)[:S].astype(np.int32)
    got = quality.sampled_inertia(_t(x, dtype), _t(c, dtype), _t(idx))
    want = O.sample_exact_inertia(x, c, idx, dtype)
    assert abs(got - want) <= 1e-5 * want, (got, want)


def test_sample_exact_inertia_api():
    """Signature and sampling of quality_compare.py:91-116: the same seeded
    torch.randperm indices as the function itself draws, nan for no sample,
    out-of-range indices add nothing, and the value is reproducible."""
    from flash_kmeans_cuda import quality, synth
    cfg = synth.CONFIGS["c2"]
    x, init = synth.make(cfg, N=8192)
    xt, ct = _t(x, "f16"), _t(init, "f16")
    a = quality.sample_exact_inertia(xt, ct, 1000, seed=1000)
    g = torch.Generator(device="cuda").manual_seed(1000)
    idx = torch.randperm(8192, generator=g, device="cuda")[:1000]
    want = O.sample_exact_inertia(x, init, idx.cpu().numpy(), "f16")
    assert abs(a - want) <= 1e-5 * want
    assert quality.sample_exact_inertia(xt, ct, 1000, seed=1000) == a
    assert np.isnan(quality.sample_exact_inertia(xt, ct, 0, seed=1))
    # more samples than points: all points (the reference's min(S, N))
    full = quality.sample_exact_inertia(xt, ct, 10 ** 6, seed=3)
    allp = O.sample_exact_inertia(x, init, np.arange(8192), "f16")
    assert abs(full - allp) <= 1e-5 * allp
    bad = torch.tensor([0, 1, -5, 8192, 3], dtype=torch.int32, device="cuda")
    got = quality.sampled_inertia(xt, ct, bad)
    want = O.sample_exact_inertia(x, init, np.array([0, 1, 3]), "f16")
    assert abs(got - want) <= 1e-5 * want
