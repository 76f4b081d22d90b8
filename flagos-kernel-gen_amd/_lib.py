"""ctypes binding of libmw4a8.so (the C ABI declared in include/mw4a8.h)."""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# MW4A8_LIB may point at another build of the same C ABI (e.g. an experimental one)
LIB_PATH = os.environ.get("MW4A8_LIB") or os.path.join(HERE, "libmw4a8.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

# name -> (restype, argtypes); one line per declaration in include/mw4a8.h
SIGNATURES = {
    "mw4a8_last_error": (ctypes.c_char_p, []),
    "mw4a8_abi_version": (_i, []),
    "mw4a8_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "mw4a8_grouped_gemm": (_i, [_p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "mw4a8_grouped_gemm_noalloc": (_i, [_p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i, _i, _i, _i, _i, _p]),
    "mw4a8_align_sizes": (_i, [_i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "mw4a8_select_block_m": (_i, [_i, _i, _i, _i, _i]),
    "mw4a8_moe_align": (_i, [_p, _i, _i, _i, _p, _p, _p, _p, _p]),
    "mw4a8_fused_moe": (_i, [_p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _i64,
                             _i, _i, _i, _i, _i, _i, _p]),
    "mw4a8_debug_partials": (_i, [_p, _i64, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "mw4a8_debug_partials_routed": (_i, [_p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _i64, _p,
                                         _i, _i, _i, _i, _i, _i, _i, _p]),
    "mw4a8_fused_moe_repacked": (_i, [_p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _i64,
                                      _i, _i, _i, _i, _i, _i, _p]),
    "mw4a8_repack_weights": (_i, [_p, _p, _i64, _i, _i, _i, _p]),
    "mw4a8_quant_rows": (_i, [_p, _i64, _i, _i, _p, _i64, _p, _p]),
    "mw4a8_router_topk": (_i, [_p, _i64, _i, _i, _i, _i, _p, _p, _p]),
    "mw4a8_silu_mul_quant": (_i, [_p, _i64, _i, _i, _p, _i64, _p, _p]),
    "mw4a8_combine_topk": (_i, [_p, _i64, _i, _i, _i, _p, _p, _i64, _p]),
    "mw4a8_stream_read": (_i, [_p, _i64, _p, _sz, _i, _p]),
    "mw4a8_host_selftest": (_i, []),
}

_LIB = None


class LibraryNotBuilt(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the HIP library once. Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryNotBuilt(
                f"{LIB_PATH} is missing; build it with `python flagos-kernel-gen_amd/build.py` "
                "(there is no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def last_error() -> str:
    msg = lib().mw4a8_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (code {rc}): {last_error()}")
