"""ctypes binding of the gfx950 kernel library (``include/vlc_capi.h``).

The library is loaded lazily, after torch, so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch has already loaded (one runtime per
process; torch streams are valid handles for the library).  A missing library
is an error: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH

_lock = threading.Lock()
_lib = None

c_i32p = ctypes.POINTER(ctypes.c_int32)
c_i64p = ctypes.POINTER(ctypes.c_int64)
vp = ctypes.c_void_p
i32 = ctypes.c_int
i64 = ctypes.c_int64
f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/vlc_capi.h.
SIGNATURES = {
    "vlc_abi_version": (i32, []),
    "vlc_status_string": (ctypes.c_char_p, [i32]),
    "vlc_store_kvcache": (i32, [vp, i64, vp, i64, vp, vp, i64, vp, i64, i64, i32, vp]),
    "vlc_rope_store_kvcache": (
        i32,
        [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, vp, i32, i64, c_i32p, vp, i64,
         i64, vp, vp, i64, vp, i64, vp],
    ),
    "vlc_rerotate_copy_kv": (
        i32,
        [vp, i64, i64, i32, vp, vp, i64, i64, i32, i32, vp, vp, i32, i32, vp],
    ),
    "vlc_decode_attn_plan": (i32, [i32, i32, i32, i32, i32, i32, i32, i32, i32, c_i32p, c_i32p, c_i32p, c_i64p]),
    "vlc_decode_attn": (
        i32,
        [vp, i64, vp, vp, i64, i32, i64, vp, i64, i32, vp, i32, i32, i32, i32, f32, i32, i32, i32, vp, i64,
         vp, i64, vp],
    ),
    "vlc_decode_attn_noalloc": (
        i32,
        [vp, i64, vp, vp, i64, i32, i64, vp, i64, i32, vp, i32, i32, i32, i32, f32, i32, i32, i32, vp, i64, vp],
    ),
    "vlc_vision_rope_pad": (i32, [vp, i64, vp, vp, vp, i64, i64, i32, i32, i32, vp, i64, vp]),
    "vlc_rms_norm": (i32, [vp, i64, vp, i64, vp, i64, vp, f32, i64, i64, vp, i64, vp]),
    "vlc_silu_mul": (i32, [vp, i64, i64, i64, vp, i64, vp]),
    "vlc_linear_skinny": (i32, [vp, i64, i64, i64, vp, i64, i64, vp, vp, i64, vp]),
    "vlc_attn_plan": (
        i32,
        [c_i32p, c_i32p, i32, i32, i32, i32, i32, i32, c_i32p, i64, c_i64p, c_i64p],
    ),
    "vlc_varlen_attn_fwd": (
        i32,
        [vp, i64, vp, i64, vp, i64, vp, i64, i32, i64, vp, vp, i32, i32, i32, i32, f32, i32,
         c_i32p, vp, i64, vp, i64, vp, i64, vp],
    ),
}

ABI_VERSION = 1

VLC_OK = 0
VLC_ERR_INVALID = -1
VLC_ERR_UNSUPPORTED = -2
VLC_ERR_WORKSPACE = -3
VLC_ERR_CAPACITY = -4
VLC_ERR_PLAN = -5
VLC_ERR_SCRATCH = -6
DECODE_NOALLOC_MAX_BYTES = 16 << 20  # VLC_DECODE_NOALLOC_MAX_BYTES


class VLCError(RuntimeError):
    """A non-zero status returned by the kernel library."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the kernel library; raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        lib_path = path or LIB_PATH
        if not os.path.exists(lib_path):
            raise RuntimeError(
                f"gfx950 kernel library not found at {lib_path}; build it with "
                "`python -m vlcache_amd.build`"
            )
        import torch  # noqa: F401  (load torch's HIP runtime first)

        lib = ctypes.CDLL(lib_path, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.vlc_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"kernel library ABI {ver} != expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(fn: str, status: int) -> None:
    if status != 0:
        msg = load().vlc_status_string(status).decode()
        raise VLCError(fn, status, msg)
