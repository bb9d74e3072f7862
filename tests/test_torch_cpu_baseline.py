"""The torch-CPU restatement that bench.py times as the CPU baseline
(oracle/torch_cpu.py) is pinned to the pinned numpy oracle (CPU only).

One Lloyd step on the same centroids gives the oracle's labels except on
near-ties (fp32 ranking against the oracle's exact float64 ranking), and,
on the same labels, its new centroids within one unit in the last place of
the storage dtype; on well-separated mixtures the whole loop (tol stop
included) lands on the oracle's labels, centroids and iteration count.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kmeans_oracle as O
from oracle import torch_cpu as T

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _t(a, dtype):
    if dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(a).astype(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a))


def _np(t, dtype):
    if dtype == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _mixture(B, N, K, D, dtype, sep, seed):
    rng = np.random.default_rng(seed)
    centres = (sep * rng.standard_normal((B, K, D))).astype(np.float32)
    blob = rng.integers(0, K, (B, N))
    xf = np.take_along_axis(centres, blob[..., None], 1) + 0.5 * rng.standard_normal(
        (B, N, D)).astype(np.float32)
    x = O.from_f32(xf.astype(np.float32), dtype)
    init = np.stack([x[b, rng.choice(N, K, replace=False)] for b in range(B)])
    return x, init


def _close(a, b, dtype):
    """fp16 / bf16 storage: within one unit in the last place (the fp32 mean
    of differently ordered fp32 sums rounds the same or to a neighbour);
    fp32 storage: within fp32 accumulation error of a few hundred rows."""
    if dtype == "f32":
        return bool(np.allclose(a, b, rtol=1e-5, atol=1e-5))
    ia, ib = a.view(np.int16).astype(np.int64), b.view(np.int16).astype(np.int64)
    return int(np.abs(ia - ib).max()) <= 1


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_one_step_matches_oracle(dtype):
    B, N, K, D = 2, 3000, 40, 24
    x, init = _mixture(B, N, K, D, dtype, sep=1.0, seed=3)
    xt, ct = _t(x, dtype), _t(init, dtype)
    x_sq = (xt.float() ** 2).sum(-1)
    new_t, ids_t = T.lloyd_step(xt, x_sq, ct)
    ids = ids_t.numpy()
    ref = O.assign(x, init, dtype)
    diff = ids != ref
    if diff.any():
        # every disagreement is a near-tie of the exact distances
        d = O.distances(x, init, dtype, ids) - O.distances(x, init, dtype, ref)
        scale = O.row_sqnorm(x, dtype) + np.take_along_axis(
            O.row_sqnorm(init, dtype), ids, 1)
        assert np.all(d[diff] <= 2.0 ** -16 * scale[diff])
    assert diff.mean() < 1e-3
    s_ids, perm = O.label_sort(ids, K)
    sums, counts = O.update_sorted_indexed(x, perm, s_ids, K, dtype)
    want = O.finalize(sums, counts, init, dtype)
    assert _close(_np(new_t, dtype), np.asarray(want), dtype)


@pytest.mark.parametrize("dtype,tol", [("f32", 0.0), ("f16", 1e-4), ("bf16", 1e-3)])
def test_loop_matches_oracle_on_separated_mixture(dtype, tol):
    B, N, K, D = 2, 2000, 16, 32
    x, init = _mixture(B, N, K, D, dtype, sep=4.0, seed=7)
    ids_t, c_t, n = T.kmeans(_t(x, dtype), _t(init, dtype), 12, tol)
    ids, c, on = O.kmeans(x, K, 12, tol, init, dtype)
    assert n == on
    assert np.array_equal(ids_t.numpy(), ids)
    assert _close(_np(c_t, dtype), np.asarray(c), dtype)


def test_labels_come_from_last_assignment():
    # one iteration: labels are the assignment against the initial centroids
    x, init = _mixture(1, 500, 8, 16, "f32", sep=3.0, seed=11)
    ids_t, c_t, n = T.kmeans(_t(x, "f32"), _t(init, "f32"), 1)
    assert n == 1
    assert np.array_equal(ids_t.numpy(), O.assign(x, init, "f32"))
    assert not np.array_equal(c_t.numpy(), init)


def test_chunking_is_invisible(monkeypatch):
    x, init = _mixture(1, 1500, 30, 16, "f16", sep=1.0, seed=5)
    a = T.kmeans(_t(x, "f16"), _t(init, "f16"), 3)
    monkeypatch.setattr(T, "CHUNK_BYTES", 4 * 30 * 7)  # 7 rows per chunk
    b = T.kmeans(_t(x, "f16"), _t(init, "f16"), 3)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and a[2] == b[2]
