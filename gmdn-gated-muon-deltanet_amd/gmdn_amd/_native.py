"""ctypes binding of ``libgmdn_scan.so`` (the C ABI declared in include/gmdn_scan.h,
include/gmdn_front.h, include/gmdn_tail.h and include/gmdn_msign.h).

The library is built in-tree by ``gmdn_amd.build`` and loaded after torch, so
its HIP runtime dependency (soname ``libamdhip64.so.7``) binds to the runtime
torch already loaded.  There is no fallback: if the library is missing or a
call returns an error code, a ``RuntimeError`` is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgmdn_scan.so")

GMDN_OK = 0
PREC_TF32 = 0
PREC_IEEE = 1
DTYPE_BF16 = 0
DTYPE_F32 = 1

_lock = threading.Lock()
_lib = None

c_f32p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_size = ctypes.c_size_t
c_vp = ctypes.c_void_p


class ChunkDesc(ctypes.Structure):
    """Mirror of ``gmdn_chunk_desc``."""

    _fields_ = [
        ("B", c_i64), ("H", c_i64), ("T", c_i64),
        ("d", c_i32), ("C", c_i32), ("rule", c_i32), ("ns", c_i32),
        ("dtype", c_i32), ("precision", c_i32), ("eps", ctypes.c_float),
        ("sq", c_i64 * 3), ("sk", c_i64 * 3), ("sv", c_i64 * 3), ("so", c_i64 * 3),
    ]


# name -> (restype, argtypes); every symbol include/gmdn_scan.h declares
SIGNATURES = {
    "gmdn_error_string": (ctypes.c_char_p, [c_i32]),
    "gmdn_scan_supported": (c_i32, [c_i32]),
    "gmdn_scan_fwd": (c_i32, [c_f32p] * 9 + [c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "gmdn_scan_bwd_workspace_bytes": (c_size, [c_i64, c_i64, c_i32, c_i32, c_i32]),
    "gmdn_scan_bwd": (c_i32, [c_f32p] * 16 + [c_vp, c_size, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "gmdn_scan_bwd_noalloc": (c_i32, [c_f32p] * 16 + [c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "gmdn_chunk_states_bytes": (c_size, [ctypes.POINTER(ChunkDesc)]),
    "gmdn_chunk_fwd": (c_i32, [ctypes.POINTER(ChunkDesc)] + [c_vp] * 10),
    "gmdn_chunk_bwd_workspace_bytes": (c_size, [ctypes.POINTER(ChunkDesc)]),
    "gmdn_wy_fwd_workspace_bytes": (c_size, [ctypes.POINTER(ChunkDesc)]),
    "gmdn_wy_fwd": (c_i32, [ctypes.POINTER(ChunkDesc)] + [c_vp] * 7 + [c_size, c_vp]),
    "gmdn_wy_bwd_workspace_bytes": (c_size, [ctypes.POINTER(ChunkDesc)]),
    "gmdn_wy_bwd": (c_i32, [ctypes.POINTER(ChunkDesc)] + [c_vp] * 13 + [c_size, c_vp]),
    "gmdn_chunk_bwd": (c_i32, [ctypes.POINTER(ChunkDesc)] + [c_vp] * 17 + [c_size, c_vp]),
    # include/gmdn_front.h
    "gmdn_front_fwd": (c_i32, [c_vp] * 6 + [c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "gmdn_front_bwd_workspace_floats": (c_size, [c_i64, c_i64, c_i32, c_i32]),
    "gmdn_front_bwd": (c_i32, [c_vp] * 8 + [c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp]),
    # include/gmdn_tail.h
    "gmdn_gates_fwd": (c_i32, [c_vp, c_vp, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp]),
    "gmdn_gates_bwd": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp]),
    "gmdn_head_norm_fwd": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, ctypes.c_float, c_i32, c_vp]),
    "gmdn_head_norm_bwd_workspace_floats": (c_size, [c_i64, c_i32]),
    "gmdn_head_norm_bwd": (c_i32, [c_vp] * 7 + [c_size, c_i64, c_i32, c_i32, c_vp]),
    # include/gmdn_msign.h
    "gmdn_msign_workspace_bytes": (c_size, [c_i64, c_i64, c_i64]),
    "gmdn_msign": (c_i32, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i32, ctypes.c_float, c_i32, c_vp, c_size, c_vp]),
}


def load():
    """Load (once) and return the native library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"gmdn native library not found at {LIB_PATH}; build it with "
                "`python -m gmdn_amd.build` (or __graft_entry__.build())")
        import torch  # noqa: F401  -- make torch's HIP runtime the one we bind to
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def check(rc: int, what: str) -> None:
    if rc != GMDN_OK:
        msg = load().gmdn_error_string(rc).decode()
        raise RuntimeError(f"{what} failed with code {rc}: {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream
