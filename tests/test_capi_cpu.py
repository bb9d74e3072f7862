"""C ABI checks that need no GPU: the library loads, exports every entry point
declared in include/fkc.h, and rejects bad arguments with a status code and a
message before touching the device.  Also the host-side Python wrappers'
argument checks (ValueError / RuntimeError / AssertionError as in the
reference: ops.py:23-24, kmeans.py:141-142, TORCH_CHECK -> RuntimeError)."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fkc.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"FKC_CAPI\s+[\w\s\*]+?\b(fkc_\w+)\s*\(", text)))


def test_header_declares_the_expected_surface():
    names = _declared()
    for n in ["fkc_euclid_assign", "fkc_row_sqnorm", "fkc_label_sort",
              "fkc_label_sort_workspace_bytes", "fkc_centroid_update_sorted",
              "fkc_centroid_update_sorted_indexed", "fkc_update_workspace_bytes",
              "fkc_centroid_finalize", "fkc_kmeans_lloyd", "fkc_kmeans_workspace_bytes",
              "fkc_assigned_inertia", "fkc_quality_workspace_bytes",
              "fkc_last_error", "fkc_version"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    from flash_kmeans_cuda import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert missing == []
    assert set(_declared()) <= set(_lib.SIGNATURES)


def test_version_matches_package():
    import flash_kmeans_cuda
    from flash_kmeans_cuda import _lib
    assert _lib.lib.fkc_version().decode() == flash_kmeans_cuda.__version__


def _err(rc):
    from flash_kmeans_cuda import _lib
    return rc, _lib.last_error()


def test_invalid_arguments_are_rejected_without_a_device():
    from flash_kmeans_cuda import _lib
    L = _lib.lib
    fake = 0x1000  # never dereferenced: validation fails first
    rc, msg = _err(L.fkc_euclid_assign(fake, fake, None, fake, fake, 1, 10, 0, 16, 1, None))
    assert rc == 1 and "K>=1" in msg
    rc, msg = _err(L.fkc_euclid_assign(fake, fake, None, fake, fake, 1, 10, 4, 16, 7, None))
    assert rc == 1 and "dtype" in msg
    rc, msg = _err(L.fkc_euclid_assign(None, fake, None, fake, fake, 1, 10, 4, 16, 1, None))
    assert rc == 1 and "null" in msg
    rc, msg = _err(L.fkc_label_sort(fake, fake, fake, 1, 1000, 10, None, 0, None))
    assert rc == 2 and "workspace" in msg
    rc, msg = _err(L.fkc_centroid_update_sorted_indexed(fake, None, fake, fake, fake,
                                                        1, 10, 4, 8, 1, None, 0, None))
    assert rc == 1 and "sorted_idx" in msg
    rc, msg = _err(L.fkc_centroid_update_sorted(fake, fake, fake, fake, 1, 10, 4, 8, 1,
                                                None, 0, None))
    assert rc == 2
    rc, msg = _err(L.fkc_kmeans_lloyd(fake, fake, fake, 1, 100, 4, 8, 1, 3, 0.0, None, 0,
                                      None, None, None))
    assert rc == 2 and "workspace" in msg
    rc, msg = _err(L.fkc_kmeans_lloyd(fake, fake, fake, 1, 100, 4, 8, 1, -1, 0.0, None, 0,
                                      None, None, None))
    assert rc == 1
    rc, msg = _err(L.fkc_kmeans_lloyd_from(fake, None, fake, fake, 1, 100, 4, 8, 1, 3, 0.0,
                                           fake, 1 << 24, None, None, None))
    assert rc == 1 and "null" in msg
    rc, msg = _err(L.fkc_kmeans_lloyd_from(fake, fake, fake, fake, 1, 100, 4, 8, 1, 3, 0.0,
                                           None, 0, None, None, None))
    assert rc == 2 and "workspace" in msg
    rc, msg = _err(L.fkc_centroid_finalize(None, fake, fake, fake, 1, 4, 8, 1, None))
    assert rc == 1
    assert L.fkc_euclid_assign(fake, fake, None, fake, fake, 1 << 20, 10, 4, 16, 1, None) == 4
    # a workspace that is large enough but not 256-byte aligned is refused
    # before anything is launched
    odd = 0x1010
    rc, msg = _err(L.fkc_label_sort(fake, fake, fake, 1, 1000, 10, odd, 1 << 20, None))
    assert rc == 2 and "aligned" in msg
    rc, msg = _err(L.fkc_centroid_update_sorted(fake, fake, fake, fake, 1, 10, 4, 8, 1,
                                                odd, 1 << 20, None))
    assert rc == 2 and "aligned" in msg
    rc, msg = _err(L.fkc_kmeans_lloyd(fake, fake, fake, 1, 100, 4, 8, 1, 3, 0.0, odd,
                                      1 << 24, None, None, None))
    assert rc == 2 and "aligned" in msg
    # quality evaluator: null labels, missing x for inertia, bad dtype,
    # small or misaligned workspace, all refused before any launch
    rc, msg = _err(L.fkc_assigned_inertia(fake, fake, None, 1, 10, 4, 8, 1, fake, fake,
                                          fake, 1 << 20, None))
    assert rc == 1 and "cluster_ids" in msg
    rc, msg = _err(L.fkc_assigned_inertia(None, fake, fake, 1, 10, 4, 8, 1, fake, None,
                                          fake, 1 << 20, None))
    assert rc == 1 and "inertia" in msg
    rc, msg = _err(L.fkc_assigned_inertia(fake, fake, fake, 1, 10, 4, 8, 9, fake, fake,
                                          fake, 1 << 20, None))
    assert rc == 1 and "dtype" in msg
    rc, msg = _err(L.fkc_assigned_inertia(fake, fake, fake, 1, 10, 4, 8, 1, fake, fake,
                                          fake, 8, None))
    assert rc == 2 and "workspace" in msg
    rc, msg = _err(L.fkc_assigned_inertia(fake, fake, fake, 1, 10, 4, 8, 1, fake, fake,
                                          odd, 1 << 20, None))
    assert rc == 2 and "aligned" in msg
    assert L.fkc_assigned_inertia(fake, fake, fake, 1, 10, 4, 8, 1, None, None,
                                  None, 0, None) == 0  # nothing asked
    # sliced assign: a shape that slices K (N = 5000, K = 4096, D = 128 fp16)
    # needs its workspace; short, missing and misaligned ones are refused
    need = L.fkc_euclid_assign_workspace_bytes(1, 5000, 4096, 128, 1)
    assert need > 0
    rc, msg = _err(L.fkc_euclid_assign_ws(fake, fake, None, fake, fake, 1, 5000, 4096, 128, 1,
                                          fake, need - 1, None))
    assert rc == 2 and "workspace" in msg
    rc, msg = _err(L.fkc_euclid_assign_ws(fake, fake, None, fake, fake, 1, 5000, 4096, 128, 1,
                                          None, 0, None))
    assert rc == 2 and "workspace" in msg
    rc, msg = _err(L.fkc_euclid_assign_ws(fake, fake, None, fake, fake, 1, 5000, 4096, 128, 1,
                                          odd, need, None))
    assert rc == 2 and "aligned" in msg
    rc, msg = _err(L.fkc_euclid_assign_ws(None, fake, None, fake, fake, 1, 5000, 4096, 128, 1,
                                          fake, need, None))
    assert rc == 1 and "null" in msg
    rc, msg = _err(L.fkc_euclid_assign_ws(fake, fake, None, fake, fake, 1, 10, 4, 16, 7,
                                          None, 0, None))
    assert rc == 1 and "dtype" in msg


def test_empty_inputs_are_no_ops():
    from flash_kmeans_cuda import _lib
    L = _lib.lib
    assert L.fkc_euclid_assign(None, None, None, None, None, 0, 0, 4, 16, 1, None) == 0
    assert L.fkc_euclid_assign_ws(None, None, None, None, None, 0, 0, 4, 16, 1, None, 0,
                                  None) == 0
    assert L.fkc_label_sort(None, None, None, 1, 0, 4, None, 0, None) == 0
    n = ctypes.c_int32(-1)
    assert L.fkc_kmeans_lloyd(None, None, None, 1, 100, 4, 8, 1, 0, 0.0, None, 0, None,
                              None, ctypes.byref(n)) == 0
    assert n.value == 0


def test_assign_slice_plan(monkeypatch):
    """Which shapes slice K and how large the partial-winner workspace is
    (8 bytes per point and slice, each half 256-byte aligned).  At D = 128
    the four-tile workgroups of all slices fill one round of 768 (3 per CU)
    with slices of >= 2048 rows: none for the benchmark shape (c5, 1024
    eight-tile workgroups) or c3 (512 four-tile workgroups, slices would be
    1024 rows); where slices of <= 4096 rows fill one round of 512 (the
    kept-score variant, 2 per CU) as fully, those: 2 for c5's one-GPU share
    of eight (256 workgroups), 4 for (32768, 16384).  Other
    widths slice only when no unsliced grid fills the chip: none for c4
    (2048 workgroups).  None for K <= 512 (exact in-loop index), the fp32
    route, or slices shorter than 2048 rows.  FKC_KSPLIT forces a count."""
    from flash_kmeans_cuda import _lib
    monkeypatch.delenv("FKC_KSPLIT", raising=False)
    monkeypatch.delenv("FKC_NTILES", raising=False)
    f = _lib.lib.fkc_euclid_assign_workspace_bytes
    half = lambda n: (n * 4 + 255) // 256 * 256
    assert f(1, 524288, 8192, 128, 1) == 0
    assert f(1, 131072, 2048, 128, 1) == 0
    assert f(1, 65536, 8192, 128, 2) == 2 * half(2 * 65536)   # 4096-row slices
    assert f(1, 32768, 16384, 128, 1) == 2 * half(4 * 32768)
    assert f(1, 49152, 8192, 128, 1) == 2 * half(4 * 49152)   # three-quarter round: re-score
    assert f(1, 32768, 256, 128, 1) == 0
    assert f(8, 65536, 1024, 64, 2) == 0
    assert f(1, 131072, 2048, 128, 0) == 0
    assert f(2, 30000, 2000, 32, 2) == 0                   # slices would be < 2048 rows
    assert f(1, 80000, 70000, 16, 1) == 2 * half(4 * 80000)
    assert f(1, 700, 4097, 128, 1) == 2 * half(2 * 700)    # 2176-row slices
    assert f(1, 700, 9000, 128, 1) == 2 * half(4 * 700)    # 2304-row slices
    assert f(1, 10, 4, 16, 7) == 0                         # invalid dtype
    monkeypatch.setenv("FKC_KSPLIT", "8")
    assert f(1, 3000, 1030, 128, 2) == 2 * half(5 * 3000)  # 256-row slices
    monkeypatch.setenv("FKC_KSPLIT", "1")
    assert f(1, 80000, 70000, 16, 1) == 0


def test_workspace_sizes():
    from flash_kmeans_cuda import _lib
    L = _lib.lib
    # mega config: sort needs a 256-bin table per 4096-key tile plus one
    # key/payload ping buffer (two 13/14-bit passes)
    s = L.fkc_label_sort_workspace_bytes(1, 524288, 8192)
    assert 2 * 524288 * 4 <= s < 3 * 524288 * 4
    assert L.fkc_label_sort_workspace_bytes(1, 4096, 255) < 4 * 4096 * 4
    u = L.fkc_update_workspace_bytes(1, 524288, 128)
    assert u >= 4096 * 2 * 128 * 4
    k = L.fkc_kmeans_workspace_bytes(1, 524288, 8192, 128, 1, 10)
    assert k > s + u + 8192 * 128 * 4
    # the fp32 route needs x_sq as well
    assert (L.fkc_kmeans_workspace_bytes(1, 4096, 64, 128, 0, 10)
            - L.fkc_kmeans_workspace_bytes(1, 4096, 64, 128, 1, 10)) >= 4096 * 4


def test_python_wrappers_reject_bad_arguments():
    from flash_kmeans_cuda import _C, batch_kmeans_Euclid, euclid_assign
    x = torch.randn(1, 10, 16)
    with pytest.raises(ValueError):
        euclid_assign(x, x[:, :2], (x ** 2).sum(-1))
    with pytest.raises(AssertionError):
        batch_kmeans_Euclid(x, 2, max_iters=1)
    with pytest.raises(RuntimeError):
        _C.euclid_assign(x, x[:, :2], (x ** 2).sum(-1), (x[:, :2] ** 2).sum(-1))


def test_synth_generators_are_deterministic():
    from flash_kmeans_cuda import synth
    cfg = synth.CONFIGS["c4"]
    a, ia = synth.make(cfg, N=2048)
    b, ib = synth.make(cfg, N=2048)
    assert a.dtype == np.uint16 and a.shape == (8, 2048, 64) and ia.shape == (8, 1024, 64)
    assert np.array_equal(a, b) and np.array_equal(ia, ib)
    assert not np.array_equal(a[0], a[1])  # per-batch seeds
    p = synth.zipf_probs(8192, 1.1)
    assert abs(p.sum() - 1) < 1e-12 and 0.14 < p[0] < 0.16


def test_sampled_inertia_validation_without_a_device():
    """fkc_sampled_inertia (quality_compare.py:91-116 counterpart): argument
    checks come before any device work."""
    from flash_kmeans_cuda import _lib
    L = _lib.lib
    assert "fkc_sampled_inertia" in _declared()
    fake = 0x1000
    rc, msg = _err(L.fkc_sampled_inertia(fake, fake, fake, 4, 1, 10, 0, 16, 1, fake,
                                         fake, 1 << 20, None))
    assert rc == 1 and "K>=1" in msg
    rc, msg = _err(L.fkc_sampled_inertia(fake, fake, fake, -1, 1, 10, 4, 16, 1, fake,
                                         fake, 1 << 20, None))
    assert rc == 1 and "sample count" in msg
    rc, msg = _err(L.fkc_sampled_inertia(fake, fake, None, 4, 1, 10, 4, 16, 1, fake,
                                         fake, 1 << 20, None))
    assert rc == 1 and "null" in msg
    rc, msg = _err(L.fkc_sampled_inertia(fake, fake, fake, 4, 1, 10, 4, 16, 1, None,
                                         fake, 1 << 20, None))
    assert rc == 1 and "null inertia" in msg
    need = L.fkc_sampled_inertia_workspace_bytes(2, 100, 7, 40, 2)
    # sampled rows (bf16), their norms, c_sq, labels and the evaluator's partials
    assert need >= 2 * 100 * 40 * 2 + 2 * 100 * 4 + 2 * 7 * 4 + 2 * 100 * 4 + 7 * 4
    assert L.fkc_sampled_inertia_workspace_bytes(0, 100, 7, 40, 2) == 0
    assert L.fkc_sampled_inertia(None, None, None, 0, 0, 0, 4, 8, 1, None, None, 0, None) == 0


_PLAN_PROBE = r"""
import json, sys
sys.path.insert(0, sys.argv[1])
from flash_kmeans_cuda import _lib
L = _lib.lib
print(json.dumps({
    "sort_c4": L.fkc_label_sort_workspace_bytes(8, 65536, 1024),
    "sort_c5": L.fkc_label_sort_workspace_bytes(1, 524288, 8192),
    "assign_c5s8": L.fkc_euclid_assign_workspace_bytes(1, 65536, 8192, 128, 1),
    "loop_c4": L.fkc_kmeans_workspace_bytes(8, 65536, 1024, 64, 2, 15),
}))
"""


def _plan_sizes(cus=None):
    """Workspace sizes the library plans for, in a fresh process (FKC_CUS:
    plan as if the device had that many compute units)."""
    import json
    import subprocess
    import sys
    env = dict(os.environ)
    env.pop("FKC_CUS", None)
    if cus is not None:
        env["FKC_CUS"] = str(cus)
    r = subprocess.run([sys.executable, "-c", _PLAN_PROBE,
                        os.path.join(REPO, "flash-kmeans-cuda_amd")],
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_plans_follow_the_device_cu_count():
    """The grid plans read the device's CU count (MI355X's 256 without a
    device): 256 CUs keep the MI355X plans; a 64-CU part leaves c4's 256
    sort tiles of 2048 keys non-resident, so 4096-key tiles (half the status
    words) are taken, and c5's one-GPU share slices K into fewer centroid
    slices (3 per CU of 64 CUs over 256 point tiles: none), so its assign
    needs no slice workspace."""
    base = _plan_sizes()
    assert _plan_sizes(256) == base
    assert base["assign_c5s8"] > 0
    small = _plan_sizes(64)
    assert small["sort_c4"] < base["sort_c4"]
    assert small["assign_c5s8"] == 0
    assert small["sort_c5"] == base["sort_c5"]  # 128 tiles of 4096 either way
    assert small["loop_c4"] < base["loop_c4"]


def test_sort_recounts_offset_lies_inside_the_loop_workspace():
    from flash_kmeans_cuda import _lib
    L = _lib.lib
    for (B, N, K, D, dt, it) in [(1, 524288, 8192, 128, 1, 10), (8, 65536, 1024, 64, 2, 15),
                                 (1, 4096, 64, 128, 0, 10), (2, 100, 1, 8, 1, 3)]:
        off = L.fkc_kmeans_sort_recounts_offset(B, N, K, D, dt, it)
        total = L.fkc_kmeans_workspace_bytes(B, N, K, D, dt, it)
        assert 0 < off and off % 256 == 0 and off + 4 <= total
    assert L.fkc_kmeans_sort_recounts_offset(0, 10, 4, 8, 1, 3) == 0
