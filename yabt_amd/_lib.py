"""ctypes binding of libyabt_hip.so (C ABI declared in include/yabt_hip.h).

Mirrors the reference's loader contract (yabt/grow_c.py:203-247): ``load()``
returns the configured library or raises RuntimeError, and the failure is
cached; ``is_available()`` never raises.  Unlike the reference there is no
compile-on-first-use: the library is built ahead of time by
``yabt_amd._build.build()`` (``__graft_entry__.build()``), and a missing
library is an error, never a silent fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading

from ._build import LIB as LIB_PATH

def row_stride(F: int) -> int:
    """Bytes per row of the row-major bin layout for F features: 16, 32 or
    64 for up to 64 features, else a multiple of 128, so that no row straddles
    a 128-byte cache line and a gathered row costs one line per 128 bytes."""
    for w in (16, 32, 64):
        if F <= w:
            return w
    return (F + 127) // 128 * 128


_LOCK = threading.Lock()
_LIB = None  # ctypes handle, or False once loading failed

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float
_dbl = ctypes.c_double
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every symbol of include/yabt_hip.h
SIGNATURES = {
    "yabt_last_error": (ctypes.c_char_p, []),
    "yabt_grow_workspace_bytes": (_sz, [_i64, _int, _int]),
    "yabt_grow": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _flt, _int, _vp, _vp, _vp, _i64, _int,
                         _flt, _flt, _flt, _int, _flt, _int, _int, _vp, _sz,
                         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "yabt_grow_leaf_ids": (_int, [_vp, _i64, _int, _int, _vp, _vp, _vp, _vp, _vp]),
    "yabt_transpose_bins": (_int, [_vp, _i64, _i64, _int, _vp, _i64, _vp]),
    "yabt_apply": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _int, _vp, _vp]),
    "yabt_hist_workspace_bytes": (_sz, []),
    "yabt_hist": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _int, _vp, _i64, _vp, _vp, _vp, _vp]),
    "yabt_hist_accumulate": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _int, _vp, _i64, _int, _int,
                                    _int, _vp, _vp, _vp]),
    "yabt_bin_counts_words": (_sz, [_i64, _int]),
    "yabt_bin_counts": (_int, [_vp, _i64, _i64, _int, _vp, _vp]),
    "yabt_hist_root": (_int, [_vp, _i64, _vp, _vp, _i64, _int, _vp, _int, _int, _int, _vp, _vp]),
    "yabt_hist_noalloc": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _int, _vp, _i64, _vp, _vp, _vp]),
    "yabt_best_split_workspace_bytes": (_sz, [_int]),
    "yabt_best_split": (_int, [_vp, _int, _vp, _vp, _vp, _int, _int, _dbl, _dbl, _dbl, _int, _vp,
                               _vp, _vp, _vp]),
    "yabt_partition_workspace_bytes": (_sz, []),
    "yabt_partition": (_int, [_vp, _i64, _i64, _int, _int, _vp, _i64, _vp, _vp, _vp, _vp]),
    "yabt_hist_slots_workspace_bytes": (_sz, [_i64, _int, _int]),
    "yabt_hist_slots": (_int, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _int, _int, _vp, _sz, _vp, _vp, _vp]),
    "yabt_leaf_fit_workspace_bytes": (_sz, [_i64, _int, _int]),
    "yabt_leaf_moments_workspace_bytes": (_sz, [_i64]),
    "yabt_leaf_moments": (_int, [_int, _vp, _i64, _i64, _vp, _int, _vp, _sz, _vp, _vp, _vp]),
    "yabt_leaf_fit": (_int, [_int, _vp, _i64, _i64, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _int, _int,
                             _dbl, _int, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "yabt_leaf_fold": (_int, [_int, _int, _vp, _vp, _vp, _vp, _flt, _vp, _vp, _vp, _vp]),
    "yabt_leaf_rank_features": (_int, [_vp, _int, _int, _int, _vp, _vp, _vp, _vp]),
    "yabt_leaf_step": (_int, [_int, _vp, _i64, _i64, _int, _int, _vp, _vp, _vp, _vp, _vp, _int, _int, _dbl,
                              _flt, _int, _vp, _sz, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                              _vp, _vp, _vp, _vp]),
    "yabt_grow_batched_workspace_bytes": (_sz, [_i64, _int, _int]),
    "yabt_grow_batched": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _flt, _int, _vp, _vp, _vp, _i64,
                                 _int,
                                 _flt, _flt, _flt, _int, _flt, _int, _int, _vp, _sz,
                                 _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "yabt_grow_levelwise_workspace_bytes": (_sz, [_i64, _int, _int, _int]),
    "yabt_grow_levelwise": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _flt, _int, _vp, _vp, _i64, _int,
                                   _flt, _flt, _flt, _int, _flt, _int, _int, _vp, _sz,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "yabt_grow_ref_workspace_bytes": (_sz, [_i64, _int, _int, _int]),
    "yabt_grow_ref_workspace_min_bytes": (_sz, [_i64, _int, _int, _int]),
    "yabt_grow_ref": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _flt, _int, _vp, _vp, _i64, _int,
                             _flt, _flt, _flt, _int, _flt, _int, _int, _vp, _sz, _vp,
                             _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "yabt_ref_root_order_bytes": (_sz, [_i64, _int]),
    "yabt_ref_root_order": (_int, [_vp, _i64, _i64, _int, _vp, _sz, _vp]),
    "yabt_ref_root_hist": (_int, [_vp, _i64, _vp, _vp, _i64, _int, _vp, _sz, _vp, _vp]),
    "yabt_bin_fit_workspace_bytes": (_sz, [_i64, _int]),
    "yabt_bin_fit": (_int, [_vp, _i64, _i64, _int, _vp, _i64, _int, _vp, _sz, _vp, _i64, _vp, _vp, _vp, _vp]),
    "yabt_bin_transform": (_int, [_vp, _i64, _i64, _int, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _i64,
                                  _vp]),
    "yabt_grad_hess": (_int, [_int, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp]),
    "yabt_margin_update": (_int, [_vp, _i64, _vp, _vp, _i64, _int, _vp, _vp, _vp, _vp, _int, _vp, _i64, _vp]),
    "yabt_predict": (_int, [_vp, _i64, _i64, _int, _int, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _int, _vp, _vp,
                            _vp, _vp, _vp, _flt, _int, _vp, _vp]),
}


def _configure(lib) -> None:
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load():
    """The configured library; raises RuntimeError if it is not built/loadable."""
    global _LIB
    if _LIB is not None:
        if _LIB is False:
            raise RuntimeError(f"yabt HIP library unavailable ({LIB_PATH})")
        return _LIB
    with _LOCK:
        if _LIB is None:
            try:
                if not os.path.exists(LIB_PATH):
                    raise FileNotFoundError(
                        f"{LIB_PATH} is not built; run yabt_amd._build.build()")
                lib = ctypes.CDLL(LIB_PATH)
                _configure(lib)
                _LIB = lib
            except Exception:
                _LIB = False
                raise
    if _LIB is False:
        raise RuntimeError(f"yabt HIP library unavailable ({LIB_PATH})")
    return _LIB


def is_available() -> bool:
    """True if the library loads and a HIP device is present (grow_c.py:241-247)."""
    try:
        load()
    except Exception:
        return False
    import torch
    return torch.cuda.is_available()


def last_error() -> str:
    msg = load().yabt_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")
