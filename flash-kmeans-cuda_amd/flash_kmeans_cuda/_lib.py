"""ctypes binding of the gfx950 kernel library (libfkc.so, include/fkc.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.  The
library is loaded after torch so that both share torch's HIP runtime
(libamdhip64.so.7 is already resident when libfkc.so resolves it).
"""

from __future__ import annotations

import contextlib
import ctypes
import os

import torch  # noqa: F401  (loads torch's HIP runtime first)

_HERE = os.path.dirname(os.path.abspath(__file__))
# FKC_LIBRARY: path of another build of libfkc.so (same-box A/B runs of two
# builds); unset, the in-tree library next to this package is loaded.
LIB_PATH = os.environ.get("FKC_LIBRARY", os.path.join(_HERE, "libfkc.so"))

FKC_OK = 0
FKC_F32, FKC_F16, FKC_BF16 = 0, 1, 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every entry point of include/fkc.h.
SIGNATURES = {
    "fkc_last_error": (ctypes.c_char_p, []),
    "fkc_version": (ctypes.c_char_p, []),
    "fkc_euclid_assign": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp]),
    "fkc_euclid_assign_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _int]),
    "fkc_euclid_assign_ws": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _sz, _vp]),
    "fkc_row_sqnorm": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fkc_label_sort_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "fkc_label_sort": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "fkc_update_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "fkc_centroid_update_sorted": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _sz, _vp]),
    "fkc_centroid_update_sorted_indexed": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _sz, _vp]),
    "fkc_centroid_finalize": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "fkc_kmeans_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _int, _int]),
    "fkc_kmeans_lloyd": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, ctypes.c_float, _vp, _sz, _vp, _vp, _vp]),
    "fkc_kmeans_lloyd_from": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, ctypes.c_float, _vp, _sz, _vp, _vp, _vp]),
    "fkc_quality_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "fkc_assigned_inertia": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _vp, _vp, _sz, _vp]),
    "fkc_sampled_inertia_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _int]),
    "fkc_sampled_inertia": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _vp, _vp, _sz, _vp]),
    "fkc_kmeans_noalloc_max_bytes": (_sz, []),
    "fkc_kmeans_lloyd_noalloc": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, ctypes.c_float, _vp, _vp, _vp]),
    "fkc_profile_enable": (None, [_int]),
    "fkc_profile_assign_ms": (_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]),
    "fkc_kmeans_sort_recounts_offset": (_sz, [_i64, _i64, _i64, _i64, _int, _int]),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"flash_kmeans_cuda: HIP kernel library not found at {LIB_PATH}. "
            "Build it with `python flash-kmeans-cuda_amd/build.py` "
            "(or __graft_entry__.build()).")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    msg = lib.fkc_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Raise RuntimeError (the class TORCH_CHECK failures surface as)."""
    if rc != FKC_OK:
        raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")


_DTYPES = {torch.float32: FKC_F32, torch.float16: FKC_F16, torch.bfloat16: FKC_BF16}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dt}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device (the raw query
    costs ~0.1 us against ~2 us for building the Stream object)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def on_device(t: torch.Tensor):
    """Context making t's device current; a no-op context when it already
    is (entering torch.cuda.device costs ~1.4 us per call)."""
    if t.device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(t.device)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned scratch for the kernels, from torch's caching allocator."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
