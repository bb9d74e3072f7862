"""GPU parity of the assignment kernels against the oracle (through the C ABI).

Bar: labels identical to the exact-distance oracle except on near-ties
(exact distance gap <= 2^-16 of ||x||^2 + ||c||^2, what an fp32-accumulated
score can misjudge), and near-ties under 0.1% of points at sizes where that
fraction is meaningful.  Integer outcomes that do not depend on rounding
(identity centroids, duplicate centroids, determinism, tile-count
invariance) must be bit-exact.  Cases mirror the reference's tests:
tests/test_mma_optin.py:35-68, tests/test_shapes.py:11-53,
tests/test_persistent.py:97-165, tests/cpp/smoke.cpp:31-53.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import near_tie_report
from oracle import kmeans_oracle as O

pytestmark = pytest.mark.gpu


def _data(B, N, K, D, dtype, seed=0, scale=1.0):
    rng = np.random.default_rng(seed)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * scale, dtype)
    c = O.from_f32(rng.standard_normal((B, K, D)).astype(np.float32) * scale, dtype)
    return x, c


def _gpu_assign(x, c, dtype, with_xsq=True):
    from flash_kmeans_cuda import _C, synth
    from flash_kmeans_cuda.ops import row_sqnorm
    xt = synth.to_torch(x, dtype)
    ct = synth.to_torch(c, dtype)
    x_sq = row_sqnorm(xt) if with_xsq else torch.empty(0, device="cuda")
    ids = _C.euclid_assign(xt, ct, x_sq, row_sqnorm(ct))
    torch.cuda.synchronize()
    return ids.cpu().numpy()


def _check(x, c, dtype, got, max_frac=None):
    ref = O.assign(x, c, dtype)
    nd, bad, worst = near_tie_report(x, c, dtype, got, ref)
    assert bad == 0, f"{bad} non-near-tie disagreements (worst rel gap {worst:.3e})"
    if max_frac is not None:
        assert nd / got.size < max_frac, f"{nd}/{got.size} near-tie flips"
    return nd


MFMA_CASES = [
    (1, 1024, 64, 64), (1, 4096, 128, 128), (2, 8192, 256, 128),   # test_mma_optin
    (1, 100, 8, 64), (1, 257, 16, 128), (1, 1024, 1, 64), (1, 1024, 63, 64),
    (1, 1024, 65, 64), (1, 1024, 32, 256), (3, 2048, 32, 64),       # test_shapes
    (1, 256, 2048, 128), (1, 777, 129, 128),
    (1, 3000, 1000, 32), (2, 2000, 700, 64), (1, 1500, 5000, 32),  # re-score, partial last stage
]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,N,K,D", MFMA_CASES)
def test_mfma_assign_matches_oracle(dtype, B, N, K, D):
    x, c = _data(B, N, K, D, dtype, seed=B * N + K + D)
    got = _gpu_assign(x, c, dtype)
    _check(x, c, dtype, got, max_frac=1e-3 if B * N >= 4096 else None)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("D", [16 * s for s in range(1, 17)] + [8, 24, 40, 72, 264, 384, 448, 512])
def test_mfma_every_feature_width(dtype, D):
    """Every 32-feature step count (D <= 512, D % 8 == 0; widths that are not
    a multiple of 32 are zero-padded inside the kernel)."""
    x, c = _data(1, 300, 97, D, dtype, seed=D)
    _check(x, c, dtype, _gpu_assign(x, c, dtype))


@pytest.mark.parametrize("ntiles", ["1", "2", "4", "8"])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_identity_centroids_and_tail(monkeypatch, ntiles, dtype):
    """First K rows as centroids map to themselves (test_persistent.py:35-64).
    Eight tiles exist only for unpadded D = 128 above the exact-index K; on
    the other shapes the override falls back to the automatic choice."""
    monkeypatch.setenv("FKC_NTILES", ntiles)
    for (N, K, D) in [(4096, 64, 128), (257, 16, 128), (8192, 128, 64),
                      (3000, 600, 128)]:
        x, _ = _data(1, N, 1, D, dtype, seed=N)
        c = x[:, :K].copy()
        got = _gpu_assign(x, c, dtype)
        assert np.array_equal(got[0, :K], np.arange(K))
        assert got.min() >= 0 and got.max() < K


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
def test_duplicate_centroids_take_lowest_index(dtype):
    x, c = _data(2, 3000, 96, 128, dtype, seed=11)
    c[:, 70] = c[:, 5]
    c[:, 95] = c[:, 5]
    c[:, 40] = c[:, 39]
    got = _gpu_assign(x, c, dtype)
    assert not np.isin(got, [70, 95, 40]).any()
    _check(x, c, dtype, got)


def test_exact_ties_take_lowest_index():
    # Every point is the origin; centroids at equal distance -> index 1.
    x = np.zeros((1, 500, 64), dtype=np.float16)
    c = np.zeros((1, 40, 64), dtype=np.float32)
    c[0, 0, 0] = 2.0
    c[0, 1:, :] = 0.0
    for k in range(1, 40):
        c[0, k, k % 64] = 1.0 if k % 2 else -1.0
    c = c.astype(np.float16)
    for dtype, xs, cs in [("f16", x, c), ("f32", x.astype(np.float32), c.astype(np.float32))]:
        got = _gpu_assign(xs, cs, dtype)
        assert np.all(got == 1), np.unique(got)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_determinism_and_ntiles_invariance(monkeypatch, dtype):
    """Repeated launches and every tile count give bit-identical labels
    (test_persistent.py:97-165 asks determinism and <1% drift; the scores here
    do not depend on the tiling, so equality is required)."""
    x, c = _data(1, 32768, 256, 128, dtype, seed=3)
    outs = []
    for nt in ["1", "2", "4", "1"]:
        monkeypatch.setenv("FKC_NTILES", nt)
        outs.append(_gpu_assign(x, c, dtype))
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,N,K", [(1, 5000, 520), (2, 3001, 1000), (1, 700, 4097)])
def test_eight_tiles_match_oracle_and_four(monkeypatch, dtype, B, N, K):
    """The eight-tile variant (128 points per wave, 128-row stages; D = 128,
    K above the exact-index cutoff) against the oracle and, bit for bit,
    against four tiles: ragged N (partial workgroups), K not a multiple of
    the 128-row stage (the last stage re-scores rows), batches."""
    x, c = _data(B, N, K, 128, dtype, seed=N + K)
    monkeypatch.setenv("FKC_NTILES", "8")
    got8 = _gpu_assign(x, c, dtype)
    monkeypatch.setenv("FKC_NTILES", "4")
    got4 = _gpu_assign(x, c, dtype)
    assert np.array_equal(got8, got4)
    _check(x, c, dtype, got8, max_frac=1e-3)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,N,K,D", [
    (1, 5000, 1030, 128), (2, 3001, 2100, 128), (1, 9000, 4097, 128),
    (1, 4000, 1500, 64), (3, 2000, 1300, 64),
    (1, 262144, 4096, 128), (1, 229376, 3072, 128), (1, 163840, 1024, 128),
])
def test_saved_scores_match_rescore(monkeypatch, dtype, B, N, K, D):
    """The four-tile kernel's two ways of naming the winner -- the scores
    of each lane's best 16-centroid block kept in registers, or the four
    candidate rows of that block re-scored after the loop -- give identical
    labels (same MFMA chain per score, first maximum either way): ragged N,
    K off the 64-row stage, batches, a K split into slices (4097 rows), and
    the grids whose plan takes the kept scores for whole rounds (1024 and
    896 workgroups).  Against the oracle where it finishes in seconds."""
    x, c = _data(B, N, K, D, dtype, seed=N + K + D)
    monkeypatch.setenv("FKC_NTILES", "4")
    outs = []
    for s in ["0", "1"]:
        monkeypatch.setenv("FKC_SAVE", s)
        outs.append(_gpu_assign(x, c, dtype))
    monkeypatch.delenv("FKC_SAVE")
    monkeypatch.delenv("FKC_NTILES")
    outs.append(_gpu_assign(x, c, dtype))  # the plan's own choice
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0], outs[2])
    if B * N * K <= 2e7:
        _check(x, c, dtype, outs[0], max_frac=1e-3)


RESIDENT_CASES = [
    # (B, N, K, D): one centroid, K below and not a multiple of 16, ragged N,
    # batches, c4's shape at reduced N, and the largest tables that fit one
    # workgroup's LDS (K = 1216 at D = 64, 2400 at D = 32).
    (1, 1000, 1, 64), (1, 777, 13, 64), (2, 3001, 100, 32), (3, 999, 517, 64),
    (8, 4096, 1024, 64), (1, 5000, 1216, 64), (1, 3000, 2400, 32),
    (1, 70000, 600, 32),
    # one point, and fewer points than one wave's tile, per batch row
    (1, 1, 100, 64), (3, 5, 1216, 64), (2, 70, 2400, 32),
]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,N,K,D", RESIDENT_CASES)
def test_resident_table_matches_staged_and_oracle(monkeypatch, dtype, B, N, K, D):
    """The centroid-resident kernel (whole table in LDS, waves walking their
    point tiles without barriers) against the oracle and, bit for bit,
    against the staged kernel on the same shape."""
    x, c = _data(B, N, K, D, dtype, seed=7 * N + K + D)
    monkeypatch.setenv("FKC_RESIDENT", "1")
    got_r = _gpu_assign(x, c, dtype)
    monkeypatch.setenv("FKC_RESIDENT", "0")
    got_s = _gpu_assign(x, c, dtype)
    assert np.array_equal(got_r, got_s)
    _check(x, c, dtype, got_r, max_frac=1e-3 if B * N >= 4096 else None)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_resident_table_ties_and_identity(monkeypatch, dtype):
    """Duplicate centroids take the lowest index and the first K points as
    centroids map to themselves on the resident kernel, including across
    the 16-row blocks and the last partial block."""
    monkeypatch.setenv("FKC_RESIDENT", "1")
    x, c = _data(2, 4000, 300, 64, dtype, seed=19)
    c[:, 299] = c[:, 3]
    c[:, 17] = c[:, 16]
    c[:, 200] = c[:, 31]
    got = _gpu_assign(x, c, dtype)
    assert not np.isin(got, [299, 17, 200]).any()
    _check(x, c, dtype, got)
    x, _ = _data(1, 5000, 1, 32, dtype, seed=23)
    c = x[:, :1100].copy()
    got = _gpu_assign(x, c, dtype)
    assert np.array_equal(got[0, :1100], np.arange(1100))


SLICE_CASES = [
    # (B, N, K, D, dtype, FKC_KSPLIT or None for the automatic plan)
    (1, 5000, 4096, 128, "f16", None),     # 2 slices of 2048 rows
    (2, 3001, 4500, 128, "bf16", None),    # 2 slices, ragged N, batches
    (1, 700, 9000, 128, "f16", None),      # 4 slices, last one 2088 rows
    (1, 3000, 1030, 128, "bf16", "8"),     # 5 slices, last one 6 rows
    (1, 2000, 700, 128, "f16", "3"),       # 3 slices of 256 / 256 / 188
    (2, 4000, 5000, 32, "bf16", None),     # 4 point tiles, 2 slices
    (1, 3000, 1500, 72, "f16", "2"),       # padded width (register stages)
]


@pytest.mark.parametrize("B,N,K,D,dtype,ksplit", SLICE_CASES)
def test_sliced_assign_matches_unsliced(monkeypatch, B, N, K, D, dtype, ksplit):
    """K cut into slices scored by separate workgroups and merged: labels
    bit-identical to the unsliced launch (same MFMA chain per score, first
    maximum in slice order) and within the oracle's near-tie bar."""
    from flash_kmeans_cuda import _lib
    x, c = _data(B, N, K, D, dtype, seed=N + K + D)
    if ksplit is None:
        monkeypatch.delenv("FKC_KSPLIT", raising=False)
    else:
        monkeypatch.setenv("FKC_KSPLIT", ksplit)
    dt = {"f16": 1, "bf16": 2}[dtype]
    assert _lib.lib.fkc_euclid_assign_workspace_bytes(B, N, K, D, dt) > 0
    got = _gpu_assign(x, c, dtype)
    monkeypatch.setenv("FKC_KSPLIT", "1")
    assert _lib.lib.fkc_euclid_assign_workspace_bytes(B, N, K, D, dt) == 0
    ref = _gpu_assign(x, c, dtype)
    assert np.array_equal(got, ref)
    _check(x, c, dtype, got, max_frac=1e-3)


def test_sliced_assign_workspace_errors(monkeypatch):
    """fkc_euclid_assign_ws rejects a short or misaligned workspace with
    FKC_ERR_WORKSPACE before launching anything, and needs none when the
    shape is not sliced."""
    from flash_kmeans_cuda import _lib
    monkeypatch.delenv("FKC_KSPLIT", raising=False)
    B, N, K, D = 1, 5000, 4096, 128
    x = torch.zeros((B, N, D), dtype=torch.float16, device="cuda")
    c = torch.zeros((B, K, D), dtype=torch.float16, device="cuda")
    csq = torch.zeros((B, K), dtype=torch.float32, device="cuda")
    ids = torch.empty((B, N), dtype=torch.int32, device="cuda")
    need = _lib.lib.fkc_euclid_assign_workspace_bytes(B, N, K, D, 1)
    assert need >= 8 * B * N * 2
    ws = torch.empty(need + 256, dtype=torch.uint8, device="cuda")
    args = (x.data_ptr(), c.data_ptr(), None, csq.data_ptr(), ids.data_ptr(), B, N, K, D, 1)
    stream = _lib.stream_of(x)
    assert _lib.lib.fkc_euclid_assign_ws(*args, ws.data_ptr(), need - 1, stream) == 2
    assert b"workspace" in _lib.lib.fkc_last_error()
    assert _lib.lib.fkc_euclid_assign_ws(*args, None, 0, stream) == 2
    assert _lib.lib.fkc_euclid_assign_ws(*args, ws.data_ptr() + 8, need, stream) == 2
    assert _lib.lib.fkc_euclid_assign_ws(*args, ws.data_ptr(), need, stream) == 0
    torch.cuda.synchronize()
    assert (ids.cpu() == 0).all()  # all-zero data: every score ties, row 0 wins
    assert _lib.lib.fkc_euclid_assign_workspace_bytes(1, 524288, 8192, 128, 1) == 0
    assert _lib.lib.fkc_euclid_assign_workspace_bytes(1, 5000, 300, 128, 1) == 0


@pytest.mark.parametrize("B,N,K,D,dtype", [(1, 140000, 40, 24, "f32"), (1, 140000, 33, 37, "f16")])
def test_vector_route_one_lane_per_point(B, N, K, D, dtype):
    """The VALU route with one lane per point (grids of >= 512 workgroups:
    N >= 131072) against the oracle, fp32 and an odd fp16 width."""
    x, c = _data(B, N, K, D, dtype, seed=N + D)
    got = _gpu_assign(x, c, dtype)
    _check(x, c, dtype, got, max_frac=1e-3)


@pytest.mark.parametrize("B,N,K,D", [(1, 4096, 64, 128), (2, 1000, 33, 37), (1, 513, 300, 16)])
def test_fp32_route_matches_oracle(B, N, K, D):
    x, c = _data(B, N, K, D, "f32", seed=N + D)
    got = _gpu_assign(x, c, "f32")
    _check(x, c, "f32", got, max_frac=1e-3 if B * N >= 4096 else None)


@pytest.mark.parametrize("D", [1, 7, 31, 48, 257, 300, 520])
def test_fp16_odd_widths_use_fp32_route(D):
    """D % 8 != 0 or D > 512 take the fp32 kernel (widths from smoke.cpp:104)."""
    x, c = _data(1, 512, 64, D, "f16", seed=D)
    got = _gpu_assign(x, c, "f16")
    _check(x, c, "f16", got)
    got2 = _gpu_assign(x, c, "f16", with_xsq=False)  # x_sq computed in-kernel
    assert np.array_equal(got, got2)


@pytest.mark.parametrize("B,N,K,D,dtype", [
    (1, 4096, 64, 128, "f32"),    # c1: sixteen lanes per point
    (2, 1000, 100, 36, "f32"),    # D not a multiple of the 32-feature chunk
    (1, 513, 1, 16, "f32"),       # one centroid
    (3, 70, 10, 4, "f32"),        # fewer points than a workgroup holds
    (1, 3000, 60, 44, "f16"),     # odd-width 16-bit rows on the fp32 route
    (2, 777, 90, 52, "bf16"),
])
def test_valu_resident_table_matches_tiled(monkeypatch, B, N, K, D, dtype):
    """The vector route's table-resident kernel (table and points loaded
    into LDS once, no barrier after) against the tiled kernel bit for bit,
    with x_sq passed and computed in the kernel, and against the oracle."""
    x, c = _data(B, N, K, D, dtype, seed=N * 3 + K + D)
    monkeypatch.setenv("FKC_RESIDENT", "1")
    got_r = _gpu_assign(x, c, dtype)
    got_r2 = _gpu_assign(x, c, dtype, with_xsq=False)
    monkeypatch.setenv("FKC_RESIDENT", "0")
    got_t = _gpu_assign(x, c, dtype)
    assert np.array_equal(got_r, got_t)
    assert np.array_equal(got_r2, got_t)
    _check(x, c, dtype, got_r, max_frac=1e-3 if B * N >= 4096 else None)


def test_force_safe_env_routes_to_fp32_kernel(monkeypatch):
    x, c = _data(1, 2048, 128, 128, "f16", seed=21)
    monkeypatch.setenv("FKC_ASSIGN_FORCE_SAFE", "1")
    got = _gpu_assign(x, c, "f16")
    _check(x, c, "f16", got)


def test_clustered_data_large_k():
    """Gaussian-mixture data at K=8192 (the mega route), N scaled down."""
    from flash_kmeans_cuda import synth
    cfg = synth.CONFIGS["c5"]
    x, init = synth.make(cfg, N=16384)
    rng = np.random.default_rng(0)
    c = x[:, rng.choice(16384, 8192, replace=False)].copy()
    got = _gpu_assign(x, c, "f16")
    _check(x, c, "f16", got, max_frac=1e-3)
