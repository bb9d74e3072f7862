"""The allocation-free Lloyd entry point (fkc_kmeans_lloyd_noalloc), called
through the C ABI, against fkc_kmeans_lloyd_from on the same inputs: the
same kernels run on a static device scratch array instead of a caller
workspace, so labels, centroids and iteration counts must be identical bit
for bit.  Two calls in a row on the shared array, the second with a smaller
input (stale contents of the first must not leak into it); a shape whose
workspace exceeds the array is refused."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import kmeans_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(B, N, K, D, dtype, seed):
    from flash_kmeans_cuda import synth
    rng = np.random.default_rng(seed)
    x = O.from_f32(rng.standard_normal((B, N, D)).astype(np.float32) * 2, dtype)
    init = np.ascontiguousarray(x[:, rng.choice(N, K, replace=False)])
    return synth.to_torch(x, dtype), synth.to_torch(init, dtype)


def _with_workspace(x, init, K, iters, tol):
    from flash_kmeans_cuda import _lib
    B, N, D = x.shape
    dt = _lib.dtype_code(x.dtype)
    ws = _lib.workspace(_lib.lib.fkc_kmeans_workspace_bytes(B, N, K, D, dt, iters), x.device)
    cents = torch.empty_like(init)
    ids = torch.empty((B, N), dtype=torch.int32, device=x.device)
    n = ctypes.c_int32(-1)
    _lib.check(_lib.lib.fkc_kmeans_lloyd_from(
        x.data_ptr(), init.data_ptr(), cents.data_ptr(), ids.data_ptr(), B, N, K, D, dt,
        iters, tol, ws.data_ptr(), ws.numel(), _lib.stream_of(x), None, ctypes.byref(n)),
        "kmeans_lloyd_from")
    return ids, cents, n.value


def _no_alloc(x, init, K, iters, tol):
    from flash_kmeans_cuda import _lib
    B, N, D = x.shape
    dt = _lib.dtype_code(x.dtype)
    cents = torch.full_like(init, 3.0)
    ids = torch.full((B, N), -1, dtype=torch.int32, device=x.device)
    n_dev = torch.full((1,), -1, dtype=torch.int32, device=x.device)
    n = ctypes.c_int32(-1)
    _lib.check(_lib.lib.fkc_kmeans_lloyd_noalloc(
        x.data_ptr(), init.data_ptr(), cents.data_ptr(), ids.data_ptr(), B, N, K, D, dt,
        iters, tol, _lib.stream_of(x), n_dev.data_ptr(), ctypes.byref(n)),
        "kmeans_lloyd_noalloc")
    torch.cuda.synchronize()
    assert int(n_dev.item()) == n.value
    return ids, cents, n.value


@pytest.mark.parametrize("first,second", [
    # (B, N, K, D, dtype, iters, tol): a large call, then a smaller one
    ((1, 131072, 2048, 128, "f16", 4, 0.0), (1, 20000, 300, 128, "f16", 3, 0.0)),
    ((8, 65536, 1024, 64, "bf16", 6, 1e-4), (2, 5000, 64, 64, "bf16", 5, 1e-4)),
    ((1, 524288, 8192, 128, "f16", 2, 0.0), (3, 3000, 40, 7, "f32", 3, 0.0)),
])
def test_no_alloc_equals_workspace_entry_point(first, second):
    from flash_kmeans_cuda import _lib
    assert _lib.lib.fkc_kmeans_noalloc_max_bytes() == 64 << 20
    for i, (B, N, K, D, dtype, iters, tol) in enumerate((first, second)):
        print(f"case {i}: B={B} N={N} K={K} D={D} {dtype} iters={iters} tol={tol}", flush=True)
        x, init = _inputs(B, N, K, D, dtype, seed=N + K + i)
        keep = init.clone()
        a = _with_workspace(x, init, K, iters, tol)
        b = _no_alloc(x, init, K, iters, tol)
        assert a[2] == b[2] and (tol > 0 or b[2] == iters)
        assert torch.equal(a[0], b[0]), "labels differ"
        assert torch.equal(a[1], b[1]), "centroids differ"
        assert torch.equal(init, keep), "initial centroids were written"


def test_no_alloc_refuses_shapes_beyond_the_scratch():
    from flash_kmeans_cuda import _lib
    B, N, K, D, dt = 1, 4 << 20, 8192, 128, 1
    need = _lib.lib.fkc_kmeans_workspace_bytes(B, N, K, D, dt, 10)
    assert need > _lib.lib.fkc_kmeans_noalloc_max_bytes()
    fake = 0x1000  # refused before any pointer is used
    rc = _lib.lib.fkc_kmeans_lloyd_noalloc(fake, fake, fake, fake, B, N, K, D, dt, 10, 0.0,
                                          None, None, None)
    assert rc == 2 and "static scratch" in _lib.last_error()


_CAPTURED_NO_ALLOC = r'''
import sys, torch
sys.path.insert(0, sys.argv[1])
from flash_kmeans_cuda import _lib
L = _lib.lib
for (B, N, K, D, dtype) in [(1, 16384, 256, 128, torch.float16), (2, 8192, 700, 64, torch.bfloat16)]:
    g = torch.Generator(device="cuda").manual_seed(N + K)
    x = torch.randn(B, N, D, device="cuda", generator=g).to(dtype)
    init = x[:, :K].contiguous().clone()
    keep = init.clone()
    cents = torch.empty_like(init)
    ids = torch.empty((B, N), dtype=torch.int32, device="cuda")
    dt = _lib.dtype_code(dtype)
    s = torch.cuda.Stream()

    def call():
        _lib.check(L.fkc_kmeans_lloyd_noalloc(
            x.data_ptr(), init.data_ptr(), cents.data_ptr(), ids.data_ptr(), B, N, K, D, dt,
            2, 0.0, s.cuda_stream, None, None), "kmeans_lloyd_noalloc")

    with torch.cuda.stream(s):
        call()                       # set-up: the scratch array's address
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    with torch.cuda.stream(s):
        call()                       # a warm call allocates nothing
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free0 == free1, ("device memory changed", free0, free1)
    e_c, e_i = cents.clone(), ids.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        call()
    torch.cuda.synchronize()
    for rep in range(3):
        cents.fill_(7.0)
        ids.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cents, e_c) and torch.equal(ids, e_i), ("replay", rep)
        with torch.cuda.stream(s):
            call()                   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(cents, e_c) and torch.equal(ids, e_i), ("eager", rep)
    assert torch.equal(init, keep)
print("noalloc-graph-ok", flush=True)
'''


def test_no_alloc_allocates_nothing_and_replays_under_graph_capture():
    """The entry point's promise, in a fresh process: once set up (first
    call on the device), a call changes no device memory (hipMemGetInfo's
    free bytes are the same around it), and with tol <= 0, n_iters_dev and
    n_iters_host NULL it can be captured into a HIP graph whose replays,
    with eager calls and synchronisations between them, equal the eager
    call bit for bit (a c2-like fp16 shape and the bf16 centroid-resident
    route)."""
    import os
    import subprocess
    import sys
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "flash-kmeans-cuda_amd")
    r = subprocess.run([sys.executable, "-c", _CAPTURED_NO_ALLOC, pkg],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "noalloc-graph-ok" in r.stdout, (r.stdout[-2000:],
                                                                    r.stderr[-2000:])
