"""Helpers shared by the GPU parity tests (no product code here)."""

from __future__ import annotations

import numpy as np

from oracle import kmeans_oracle as O

# Largest exact-distance gap (relative to x_sq + c_sq of the point and the
# chosen centroid) that an fp32-accumulated score may misjudge: 2^-16 covers
# a worst-case fp32 dot product over D <= 256 terms plus the fp32 c_sq.
NEAR_TIE_REL = 2.0 ** -16


def near_tie_report(x, c, dtype, got, ref, rel=NEAR_TIE_REL):
    """Compare GPU labels `got` with oracle labels `ref` (both (B,N)).

    Returns (n_disagree, n_bad, worst_rel_gap): a disagreement is bad when the
    exact squared-distance gap between the two choices exceeds
    rel * (||x||^2 + ||c_got||^2)."""
    got = np.asarray(got).astype(np.int64)
    ref = np.asarray(ref).astype(np.int64)
    mask = got != ref
    nd = int(mask.sum())
    if nd == 0:
        return 0, 0, 0.0
    xv = O.to_f64(x, dtype)
    cv = O.to_f64(c, dtype)
    b_idx, n_idx = np.nonzero(mask)
    xp = xv[b_idx, n_idx]
    cg = cv[b_idx, got[mask]]
    cr = cv[b_idx, ref[mask]]
    dg = ((xp - cg) ** 2).sum(-1)
    dr = ((xp - cr) ** 2).sum(-1)
    scale = (xp * xp).sum(-1) + (cg * cg).sum(-1)
    gap = (dg - dr) / np.maximum(scale, 1e-30)
    bad = int((gap > rel).sum())
    return nd, bad, float(gap.max())


def inertia(x, c, dtype, ids):
    return float(O.distances(x, c, dtype, np.asarray(ids)).sum())
