"""ctypes binding of ``libsk_attn.so`` (C ABI: ``include/sk_attn.h``).

The library is loaded once, after torch (so that the HIP runtime torch
already mapped is the one the library binds to: both carry the SONAME
``libamdhip64.so.7`` and the library is linked against torch's copy).  If
the library is missing the first kernel call raises ``RuntimeError``: there
is no silent fallback to another implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading

SK_F32, SK_F16, SK_BF16 = 0, 1, 2
SK_OK, SK_EINVAL, SK_EUNSUPPORTED, SK_EWORKSPACE = 0, -1, -2, -3
ABI_VERSION = 7

_LIB_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))), "csrc")
LIB_PATH = os.environ.get("SK_ATTN_LIB", os.path.join(_LIB_DIR, "libsk_attn.so"))

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_c_int = ctypes.c_int
_c_float = ctypes.c_float
_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)
_sizep = ctypes.POINTER(ctypes.c_size_t)
_intp = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); mirrors include/sk_attn.h.
# RoPE arguments: cos, sin, table dtype, rows, row stride, positions, start.
_ROPE = (_vp, _vp, _c_int, _c_int, ctypes.c_int64, _vp, _c_int)

SIGNATURES: dict[str, tuple] = {
    "sk_abi_version": (_c_int, []),
    "sk_last_error": (ctypes.c_char_p, []),
    "sk_attn_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp,
                             _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                             _i64p, _i64p, _i64p, _i64p, _c_int, _c_float, _vp]),
    "sk_attn_bwd_workspace": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _sizep]),
    "sk_attn_bwd_workspace_min": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                           _c_int, _c_int, _sizep]),
    "sk_attn_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                             ctypes.c_size_t, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                             _c_int, _c_float, _vp]),
    "sk_decode_plan": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _intp, _sizep]),
    "sk_decode_plan_varlen": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _intp,
                                       _sizep]),
    "sk_decode_workspace": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                     _sizep]),
    "sk_decode": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _c_int,
                           _c_int, _c_int, _c_int, _c_int, _c_int,
                           _i64p, _i64p, _i64p, _i64p, _c_float, _vp]),
    "sk_decode_noalloc": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _c_int,
                                   _c_int, _c_int, _c_int, _c_int, _c_int,
                                   _i64p, _i64p, _i64p, _i64p, _c_float, _vp]),
    "sk_decode_varlen": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _c_int,
                                  _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _i64p, _i64p, _i64p, _i64p, _vp, _c_float, _vp]),
    "sk_kv_cache_update": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp,
                                    _c_int, _c_int, _c_int, _c_int, _c_int,
                                    _i64p, _i64p, _i64p, _i64p, _vp]),
    "sk_decode_paged": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _c_int,
                                 _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                 _i64p, _i64p, _i64p, _i64p, _vp, _vp, _c_float, _vp]),
    "sk_kv_cache_update_paged": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp,
                                          _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                          _i64p, _i64p, _i64p, _i64p, _vp]),
    "sk_rope_rotate": (_c_int, [_c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _i64p, _i64p,
                                *_ROPE, _c_int, _vp]),
    # *_rope: the call they extend with (cos, sin, table dtype, rows, row
    # stride, per-row positions, start) inserted before sm_scale / stream.
    "sk_attn_fwd_rope": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp,
                                  _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _i64p, _i64p, _i64p, _i64p, _c_int, *_ROPE, _c_float, _vp]),
    "sk_decode_rope": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _c_int,
                                _c_int, _c_int, _c_int, _c_int, _c_int,
                                _i64p, _i64p, _i64p, _i64p, _vp, *_ROPE, _c_float, _vp]),
    "sk_decode_paged_rope": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _c_int,
                                      _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _i64p, _i64p, _i64p, _i64p, _vp, _vp, *_ROPE, _c_float,
                                      _vp]),
    "sk_kv_cache_update_rope": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp,
                                         _c_int, _c_int, _c_int, _c_int, _c_int,
                                         _i64p, _i64p, _i64p, _i64p, *_ROPE, _vp]),
    "sk_kv_cache_update_paged_rope": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp,
                                               _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                               _i64p, _i64p, _i64p, _i64p, *_ROPE, _vp]),
    "sk_kernel_config": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _c_int, _c_int, _c_int, _c_int, _i64p, ctypes.c_char_p,
                                  ctypes.c_size_t]),
}


def load() -> ctypes.CDLL:
    """Load and type the library; raise RuntimeError if it is absent or stale."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  -- map torch's HIP runtime first

        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libsk_attn.so not found at {LIB_PATH}; build it with "
                "`python -m stackkernels_amd.csrc.build` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.sk_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"libsk_attn.so ABI {lib.sk_abi_version()} != expected {ABI_VERSION}; rebuild it"
            )
        _lib = lib
        return lib


def last_error() -> str:
    return load().sk_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    """Map a library return code to the Python exception the reference raises."""
    if rc == SK_OK:
        return
    msg = last_error()
    if rc in (SK_EINVAL,):
        raise ValueError(f"{what}: {msg}")
    if rc == SK_EUNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def strides3(t) -> ctypes.Array:
    """(b, h, s) element strides of a BHSD tensor as an int64[3]."""
    st = t.stride()
    return (ctypes.c_int64 * 3)(st[0], st[1], st[2])


def dtype_code(dtype) -> int:
    import torch

    if dtype == torch.bfloat16:
        return SK_BF16
    if dtype == torch.float16:
        return SK_F16
    if dtype == torch.float32:
        return SK_F32
    raise NotImplementedError(f"dtype {dtype} has no HIP kernel (supported: float32, float16, bfloat16)")


def stream_ptr(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def loaded_hip_runtimes() -> list[str]:
    """Paths of every libamdhip64 mapped into this process (should be exactly one)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in parts[-1]:
                paths.add(os.path.realpath(parts[-1]))
    return sorted(paths)
