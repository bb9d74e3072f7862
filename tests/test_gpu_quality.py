"""GPU parity of the device quality evaluator (fkc_assigned_inertia and
flash_kmeans_cuda.quality) against the oracle, which restates the
reference's benchmarks/quality_compare.py:63-90.

Bar: per-element differences and squares are fp32 on both sides and the
totals fp64, so only the fp64 summation order differs: relative error
<= 1e-10 at these sizes.  Empty-cluster counts are exact.  The device
result is bitwise reproducible.
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
    """(inertia per batch row, empty per batch row) through the C ABI."""
    from flash_kmeans_cuda import _lib
    xt, ct = _t(x, dtype), _t(c, dtype)
    it = _t(ids.astype(np.int32))
    B, N, D = x.shape
    K = c.shape[1]
    inertia = torch.empty(B, dtype=torch.float64, device="cuda")
    empty = torch.empty(B, dtype=torch.int32, device="cuda")
    ws = _lib.workspace(_lib.lib.fkc_quality_workspace_bytes(B, N, K), torch.device("cuda"))
    _lib.check(_lib.lib.fkc_assigned_inertia(
        xt.data_ptr(), ct.data_ptr(), it.data_ptr(), B, N, K, D, _lib.dtype_code(xt.dtype),
        inertia.data_ptr(), empty.data_ptr(), ws.data_ptr(), ws.numel(),
        _lib.stream_of(xt)), "assigned_inertia")
    torch.cuda.synchronize()
    return inertia.cpu().numpy(), empty.cpu().numpy()


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
    assert np.array_equal(got_e, want_e)


def test_bitwise_reproducible():
    rng = np.random.default_rng(3)
    x = O.from_f32(rng.standard_normal((1, 300000, 128)).astype(np.float32), "f16")
    c = O.from_f32(rng.standard_normal((1, 2048, 128)).astype(np.float32), "f16")
    ids = rng.integers(0, 2048, (1, 300000)).astype(np.int32)
    a = _device(x, ids, c, "f16")
    b = _device(x, ids, c, "f16")
    assert a[0].tobytes() == b[0].tobytes() and np.array_equal(a[1], b[1])


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
    assert ev["empty_clusters"] == int(O.empty_clusters(ids_np, cfg.K).sum())
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
