"""ctypes binding of libsparda.so (the C ABI declared in include/sparda.h).

The library must have been built (``sparda.build.build()``); loading fails
loudly otherwise — there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading

# SPARDA_LIBRARY overrides the path (an alternative build of the same ABI)
LIB_PATH = os.environ.get("SPARDA_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                            "libsparda.so")

F32 = 0
BF16 = 1

ROUTE_REFERENCE = 0
ROUTE_ABSOLUTE = 1

SEL_DENSE = 0
SEL_WINDOW_DECODE = 1
SEL_WINDOW_PREFILL = 2

FETCH_KERNEL = 0
FETCH_DMA = 1

TOPK_AUTO = 0
TOPK_ROWS = 1
TOPK_WAVE = 2

ERR_NAMES = {
    -1: "null pointer", -2: "shape", -3: "dtype", -4: "workspace", -5: "stride",
    -6: "mode", -7: "handle", -8: "capacity",
}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_p = ctypes.c_void_p
_size = ctypes.c_size_t


class PrefetchArgs(ctypes.Structure):
    """sparda_prefetch_args: the next layer's prefetch carried by
    sparda_decode_at_prefetch (field order and types as in the header)."""
    _fields_ = [("arena", _p), ("forecast", _p), ("f_dtype", _int), ("f_sb", _i64), ("f_sh", _i64),
                ("block_sums", _p), ("nb_stride", _i64), ("top_k", _i64), ("routing", _int), ("scale", _f32),
                ("sel", _p), ("n_sel", _p), ("sel_cap", _i64), ("k_dst", _p), ("v_dst", _p), ("stage", _int),
                ("parts", _int), ("part", _int)]

# name -> (restype, argtypes); mirrors include/sparda.h
SIGNATURES = {
    "sparda_version": (_int, []),
    "sparda_last_error": (ctypes.c_char_p, []),
    "sparda_status": (_int, [_p, _int, _p]),
    "sparda_compress": (_int, [_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p]),
    "sparda_route": (_int, [_p, _int, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _int, _i64, _i64, _f32, _p, _p, _p, _p, _i64, _p]),
    "sparda_topk_scores": (_int, [_p, _i64, _i64, _i64, _int, _p, _p]),
    "sparda_select_chunked": (_int, [_p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p]),
    "sparda_select_fixed": (_int, [_int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p]),
    "sparda_gather_blocks": (_int, [_p, _p, _int, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64,
                                    _i64, _p, _p, _p]),
    "sparda_prefill": (_int, [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _p, _p, _i64, _i64,
                              _i64, _i64, _i64, _i64, _i64, _int, _f32, _p, _i64, _i64, _p]),
    "sparda_prefill_routed": (_int, [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _p, _int, _i64, _i64,
                                     _i64, _p, _i64, _i64, _f32, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _int, _f32, _p, _i64, _i64, _p]),
    "sparda_prefill_chunked": (_int, [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _p, _i64, _i64, _p, _p,
                                      _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _p, _i64, _i64, _p]),
    "sparda_prefill_masked": (_int, [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _p, _p, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _i64, _int, _f32, _p, _int, _i64, _i64, _i64, _i64, _p, _i64,
                                     _i64, _p, _i64, _i64, _i64, _p]),
    "sparda_decode_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "sparda_decode": (_int, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _p, _int, _i64, _i64, _i64,
                             _i64, _i64, _i64, _i64, _i64, _i64, _int, _f32, _p, _p, _p, _p, _p, _i64,
                             _p, _size, _p]),
    "sparda_decode_noalloc": (_int, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _p, _int, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _i64, _i64, _i64, _int, _f32, _p, _p, _p, _p, _p, _i64,
                                     _p]),
    "sparda_decode_selected": (_int, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _int, _p, _p, _i64, _p, _p,
                                      _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _p, _i64, _p, _size,
                                      _p]),
    "sparda_decode_dense_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "sparda_select_decode": (_int, [_p, _int, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                    _int, _f32, _p, _p, _i64, _p]),
    "sparda_offload_create": (_int, [_i64, _i64, _i64, _i64, _int, ctypes.POINTER(_p)]),
    "sparda_offload_destroy": (_int, [_p]),
    "sparda_offload_host": (_int, [_p, ctypes.POINTER(_p), ctypes.POINTER(_p)]),
    "sparda_teacher_mass": (_int, [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _int, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _int, _f32, _p, _p]),
    "sparda_produce": (_int, [_p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32, _p, _p, _i64, _i64, _i64,
                              _p, _p, _p, _p, _int, _p]),
    "sparda_block_sums": (_int, [_p, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _p, _p]),
    "sparda_produce_at": (_int, [_p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32, _p, _p, _i64, _i64, _p,
                                 _p, _p, _p, _p, _int, _p]),
    "sparda_produce_cache_at": (_int, [_p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32, _p, _p, _i64, _i64, _p,
                                       _p, _p, _p, _p, _int, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "sparda_append_at": (_int, [_p, _p, _int, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p,
                                _i64, _i64, _p, _p]),
    "sparda_select_decode_at": (_int, [_p, _int, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64,
                                       _int, _f32, _p, _p, _i64, _int, _p]),
    "sparda_decode_at": (_int, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _int, _p, _p, _i64, _i64, _p, _p,
                                _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _f32, _p, _i64, _p, _size, _p]),
    "sparda_decode_at_prefetch": (_int, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _int, _p, _p, _i64, _i64,
                                         _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _f32, _p, _i64,
                                         ctypes.POINTER(PrefetchArgs), _p, _size, _p]),
    "sparda_decode_sums": (_int, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _int, _p, _int, _i64, _i64, _p, _i64,
                                  _int, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _int, _f32, _f32, _p, _p, _p,
                                  _i64, _p]),
    "sparda_ffn_decode": (_int, [_p, _i64, _p, _p, _i64, _i64, _i64, _f32, _p, _p, _i64, _p]),
    "sparda_ffn_decode_prefetch": (_int, [_p, _i64, _p, _p, _i64, _i64, _i64, _f32, _p, _p, _i64,
                                          ctypes.POINTER(PrefetchArgs), ctypes.POINTER(PrefetchArgs), _p, _i64,
                                          _p]),
    "sparda_rows_residual": (_int, [_p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p, _i64, _p]),
    "sparda_norm_gemv": (_int, [_p, _i64, _p, _i64, _i64, _i64, _f32, _p, _i64, _p]),
    "sparda_offload_fetch_at": (_int, [_p, _p, _p, _i64, _i64, _p, _p, _p, _p]),
    "sparda_offload_append_at": (_int, [_p, _p, _p, _i64, _i64, _p, _i64, _p, _p]),
    "sparda_offload_append_at_prefetch": (_int, [_p, _p, _p, _i64, _i64, _p, _i64, _p, _i64,
                                                 ctypes.POINTER(PrefetchArgs), _p]),
    "sparda_offload_append": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p]),
    "sparda_offload_rebuild_sums": (_int, [_p, _i64, _i64, _p, _p]),
    "sparda_offload_fetch": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _p, _p, _p]),
}

_lock = threading.Lock()
_lib = None


class SpardaError(RuntimeError):
    """A non-zero status from libsparda."""

    def __init__(self, func: str, code: int, message: str):
        kind = ERR_NAMES.get(code, "hip error" if code > 0 else "error")
        super().__init__(f"{func} failed ({kind}, status {code}): {message}")
        self.code = code


class SpardaArgumentError(SpardaError, ValueError):
    """Argument rejected by the library before any HIP call."""


def load() -> ctypes.CDLL:
    """Load libsparda.so once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"libsparda.so not found at {LIB_PATH}: build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and turn a non-zero status into an exception."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = (lib.sparda_last_error() or b"").decode(errors="replace")
        cls = SpardaArgumentError if rc < 0 else SpardaError
        raise cls(name, rc, msg)
