"""Regenerate the committed golden fixtures from the CPU oracle.

    python tests/golden/make_golden.py

c1.npz  — the CPU plumbing configuration: x ~ N(0,1) fp32 (1, 4096, 128)
          from seed 0, K=64 initial centroids sampled without replacement
          (seed 1), 10 Lloyd iterations, tol=0.  Stores the sha256 of x's
          bytes (x itself is regenerated from the seed), the init indices,
          labels int64[4096], centroids fp32[64,128], n_iters.
tiny.npz — small hand-shaped assignment cases (ties, duplicate centroids,
          K=1, tails, odd D) with their oracle labels, for every dtype.

The oracle is pinned independently in tests/test_oracle_pins.py; these files
freeze its outputs so a later change to it is caught.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "flash-kmeans-cuda_amd"))

from oracle import kmeans_oracle as O  # noqa: E402
from flash_kmeans_cuda import synth  # noqa: E402  (pure numpy module)


def c1_inputs():
    cfg = synth.CONFIGS["c1"]
    x, init = synth.make(cfg)
    idx = np.random.default_rng(cfg.init_seed).choice(cfg.N, cfg.K, replace=False)
    return cfg, x, init, idx


def make_c1(path):
    cfg, x, init, idx = c1_inputs()
    ids, cents, n = O.kmeans(x, cfg.K, cfg.iters, cfg.tol, init, "f32")
    np.savez_compressed(
        path,
        x_sha256=np.array(hashlib.sha256(x.tobytes()).hexdigest()),
        init_idx=idx.astype(np.int64),
        labels=ids[0].astype(np.int64),
        centroids=cents[0].astype(np.float32),
        n_iters=np.array(n),
    )


def tiny_cases():
    rng = np.random.default_rng(42)
    cases = []
    for dtype in ("f32", "f16", "bf16"):
        for (N, K, D) in [(1, 1, 1), (7, 3, 5), (33, 9, 16), (60, 8, 48), (257, 16, 32), (65, 65, 7)]:
            xf = rng.standard_normal((1, N, D)).astype(np.float32)
            cf = rng.standard_normal((1, K, D)).astype(np.float32)
            if K >= 3:
                cf[0, K - 1] = cf[0, 0]           # duplicate of centroid 0
            if N >= 2 and K >= 2:
                xf[0, 1] = 0.5 * (cf[0, 0] + cf[0, 1])  # near-equidistant point
            x = O.from_f32(xf, dtype)
            c = O.from_f32(cf, dtype)
            cases.append((dtype, x, c, O.assign(x, c, dtype)))
    return cases


def make_tiny(path):
    out = {}
    for i, (dtype, x, c, ids) in enumerate(tiny_cases()):
        out[f"{i}_dtype"] = np.array(dtype)
        out[f"{i}_x"] = x
        out[f"{i}_c"] = c
        out[f"{i}_ids"] = ids
    np.savez_compressed(path, **out)


if __name__ == "__main__":
    make_c1(os.path.join(HERE, "c1.npz"))
    make_tiny(os.path.join(HERE, "tiny.npz"))
    print("wrote", os.listdir(HERE))
