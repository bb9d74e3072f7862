"""Full-size oracle runs of configurations c3, c4 and c5, frozen as fixtures
for the GPU tests of the north-star bar (tests/test_gpu_north_star.py).

    python tests/golden/make_large.py [c3] [c4] [c5]      (all three by default)

Each configuration's inputs are regenerated from synth's seeds; the oracle
(exact float64 distances, stable sort, float64 run sums rounded to float32,
IEEE finalize, centroids kept in the storage dtype between iterations) runs
the configuration's own max_iters and tol.  <config>_full.npz holds:

  x_sha256    sha256 of x's storage bytes (the test checks it regenerated
              the same inputs)
  n_iters     iterations run (c4 stops after the first shift below tol)
  shifts      float32 [iters]: the shift of every iteration (kmeans.py:104)
  labels      uint16 (B, N): labels of the last assignment (kmeans.py:179-195)
  assigned_against
              (B, K, D) raw storage bits of the centroids that last
              assignment ranked (the state after n_iters - 1 iterations, or
              the initial centroids when n_iters = 1), so a test can assign
              every point against exactly them
  centroids   (B, K, D) final centroids, raw storage bits (uint16)
  inertia     float64: sum over every point of the exact squared distance to
              its nearest final centroid (the objective the bar compares)
  prev_*      for tol > 0: the same three items after n_iters - 1 and
  next_*      n_iters + 1 iterations (when those exist), so a GPU run that
              stops one iteration off can be compared at its own count;
              when the last shift is exactly 0 the loop has reached a fixed
              point, the next iteration repeats it, and next_* is left out
              (fixed_point = 1)
  f32_label_diff, f32_drift
              how far the same loop lands from it when its distances are
              ranked in float32 (the oracle's fp32 BLAS form) instead of
              float64: fraction of returned labels that differ and relative
              Frobenius distance of the final centroids.  A loop that has not
              converged within max_iters (c5) is sensitive to rounding, and
              this is the floor any fp32 implementation is measured against.

The oracle itself is pinned in tests/test_oracle_pins.py.  c5 takes a few
minutes on 8 cores (1.1 TFLOP of float64 distances per iteration).
"""

from __future__ import annotations

import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "flash-kmeans-cuda_amd"))

from oracle import kmeans_oracle as O  # noqa: E402
from flash_kmeans_cuda import synth  # noqa: E402  (pure numpy module)


def _bits(c: np.ndarray) -> np.ndarray:
    return c.view(np.uint16) if c.dtype == np.float16 else c.astype(np.uint16)


def _nearest_inertia(x, c, dtype):
    ids = O.assign(x, c, dtype)
    return float(O.distances(x, c, dtype, ids).sum())


def make(name: str) -> str:
    cfg = synth.CONFIGS[name]
    t0 = time.time()
    x, init = synth.make(cfg)
    assert cfg.K <= 65536
    cur = init.copy()
    traj_ids, traj_c, shifts = [], [], []
    n = 0
    # the loop of O.kmeans, keeping every iteration for the +-1 items
    for it in range(cfg.iters):
        new, ids, _, _ = O.lloyd_step(x, cur, cfg.K, cfg.dtype)
        s = O.shift(new, cur, cfg.dtype)
        shifts.append(s)
        traj_ids.append(ids)
        traj_c.append(new)
        cur = new
        n = it + 1
        print(f"{name}: iteration {n} shift {s:.6g} ({time.time() - t0:.0f} s)", flush=True)
        if cfg.tol > 0 and s < cfg.tol:
            break
    # with tol > 0 also the next iteration, when max_iters allows it
    if cfg.tol > 0 and n < cfg.iters:
        new, ids, _, _ = O.lloyd_step(x, cur, cfg.K, cfg.dtype)
        traj_ids.append(ids)
        traj_c.append(new)
    out = dict(
        x_sha256=np.array(hashlib.sha256(x.tobytes()).hexdigest()),
        n_iters=np.array(n),
        shifts=np.array(shifts, dtype=np.float32),
        labels=traj_ids[n - 1].astype(np.uint16),
        assigned_against=_bits(traj_c[n - 2] if n >= 2 else init),
        centroids=_bits(traj_c[n - 1]),
        inertia=np.array(_nearest_inertia(x, traj_c[n - 1], cfg.dtype)),
    )
    out["fixed_point"] = np.array(int(shifts[-1] == 0.0))
    if cfg.tol > 0:
        for key, i in (("prev", n - 2), ("next", n)):
            if key == "next" and shifts[-1] == 0.0:
                continue
            if 0 <= i < len(traj_c):
                out[f"{key}_labels"] = traj_ids[i].astype(np.uint16)
                out[f"{key}_centroids"] = _bits(traj_c[i])
                out[f"{key}_inertia"] = np.array(_nearest_inertia(x, traj_c[i], cfg.dtype))
    # the same loop with float32 distance ranking (same stop rule)
    f_ids, f_c, f_n = O.kmeans(x, cfg.K, cfg.iters, cfg.tol, init, cfg.dtype, precision="f32")
    ref_c = O.to_f64(traj_c[n - 1], cfg.dtype)
    out["f32_n_iters"] = np.array(f_n)
    out["f32_label_diff"] = np.array(float((f_ids != traj_ids[n - 1]).mean()))
    out["f32_drift"] = np.array(float(np.linalg.norm(O.to_f64(f_c, cfg.dtype) - ref_c)
                                      / np.linalg.norm(ref_c)))
    print(f"{name}: float32 ranking: n_iters {f_n}, labels {float(out['f32_label_diff']):.4%}, "
          f"drift {float(out['f32_drift']):.3e}", flush=True)
    path = os.path.join(HERE, f"{name}_full.npz")
    np.savez_compressed(path, **out)
    print(f"{name}: n_iters {n}, inertia {float(out['inertia']):.9g}, wrote {path} "
          f"({os.path.getsize(path) / 2**20:.2f} MiB, {time.time() - t0:.0f} s)", flush=True)
    return path


if __name__ == "__main__":
    for nm in (sys.argv[1:] or ["c3", "c4", "c5"]):
        make(nm)
