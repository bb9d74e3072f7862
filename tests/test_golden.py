"""The oracle reproduces the committed golden fixtures (CPU only).

tests/golden/c1.npz freezes the CPU plumbing configuration (x ~ N(0,1)
fp32 (1,4096,128), K=64, 10 iterations, tol=0); tests/golden/tiny.npz freezes
small assignment cases with ties, duplicate centroids and odd widths.
"""

from __future__ import annotations

import hashlib
import os

import numpy as np

from oracle import kmeans_oracle as O
from flash_kmeans_cuda import synth

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_c1_inputs_regenerate_bit_exact():
    z = np.load(os.path.join(HERE, "c1.npz"))
    x, init = synth.make(synth.CONFIGS["c1"])
    assert hashlib.sha256(x.tobytes()).hexdigest() == str(z["x_sha256"])
    assert np.array_equal(init[0], x[0, z["init_idx"]])


def test_oracle_reproduces_c1_fixture():
    z = np.load(os.path.join(HERE, "c1.npz"))
    cfg = synth.CONFIGS["c1"]
    x, init = synth.make(cfg)
    ids, cents, n = O.kmeans(x, cfg.K, cfg.iters, cfg.tol, init, "f32")
    assert n == int(z["n_iters"]) == 10
    assert np.array_equal(ids[0], z["labels"])
    assert np.array_equal(cents[0].view(np.uint32), z["centroids"].view(np.uint32))


def test_oracle_reproduces_tiny_fixtures():
    z = np.load(os.path.join(HERE, "tiny.npz"))
    n = len([k for k in z.files if k.endswith("_dtype")])
    assert n == 18
    for i in range(n):
        dtype = str(z[f"{i}_dtype"])
        got = O.assign(z[f"{i}_x"], z[f"{i}_c"], dtype)
        assert np.array_equal(got, z[f"{i}_ids"]), (i, dtype)
