"""ctypes binding of ``libifkfac_hip.so`` (the C ABI in include/ifkfac_hip.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch has already loaded (both link ``libamdhip64.so.7`` by soname).
There is no fallback: if the library is missing or cannot be loaded, every
product entry point raises :class:`IFKFACBackendError`.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the library load, see module doc)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libifkfac_hip.so")

IFK_OK = 0
IFK_F32 = 0
IFK_BF16 = 1
IFK_MATH_F32 = 0
IFK_MATH_BF16 = 1

ABI_VERSION = 2


class IFKFACBackendError(RuntimeError):
    """The HIP library is unavailable or one of its calls failed."""


_c_i64 = ctypes.c_int64
_c_sz = ctypes.c_size_t
_c_vp = ctypes.c_void_p
_c_int = ctypes.c_int
_c_f = ctypes.c_float
_c_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/ifkfac_hip.h exactly.
SIGNATURES = {
    "ifk_abi_version": (_c_int, []),
    "ifk_status_to_host": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64]),
    "ifk_last_error": (ctypes.c_char_p, []),
    "ifk_release_stream_state": (_c_int, [_c_vp]),
    "ifk_tsqr_fold_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_tsqr_fold": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64,
                               _c_i64, _c_int, _c_vp, _c_sz, _c_i64p]),
    "ifk_finalize_workspace_size": (_c_sz, [_c_i64]),
    "ifk_finalize": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_f, _c_f, _c_vp, _c_int, _c_i64,
                              _c_int, _c_vp, _c_vp, _c_sz]),
    "ifk_fold_finalize_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "ifk_fold_finalize": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64,
                                   _c_i64, _c_f, _c_f, _c_vp, _c_int, _c_i64, _c_int, _c_vp,
                                   _c_vp, _c_sz]),
    "ifk_fold_finalize_cqr_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "ifk_fold_finalize_cqr": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp,
                                       _c_i64, _c_i64, _c_f, _c_f, _c_vp, _c_int, _c_i64, _c_int,
                                       _c_vp, _c_vp, _c_sz]),
    "ifk_fold_finalize_gram_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "ifk_fold_finalize_gram": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp,
                                        _c_i64, _c_i64, _c_f, _c_f, _c_vp, _c_int, _c_i64, _c_int,
                                        _c_vp, _c_vp, _c_vp, _c_sz]),
    "ifk_fold_finalize_gram_batched_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "ifk_fold_finalize_gram_batched": (_c_int, [_c_vp, _c_i64, _c_vp, _c_int, _c_i64, _c_i64,
                                                _c_i64, _c_vp, _c_i64, _c_i64, _c_f, _c_f, _c_vp,
                                                _c_int, _c_i64, _c_i64, _c_int, _c_f, _c_vp,
                                                _c_vp, _c_vp, _c_sz]),
    "ifk_inverse_split_copies": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp,
                                          _c_i64]),
    "ifk_precondition_apply_x3_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_precondition_apply_x3": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp,
                                           _c_vp, _c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp,
                                           _c_i64, _c_vp, _c_i64, _c_vp, _c_sz]),
    "ifk_tsqr_fold_gram_batched_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "ifk_tsqr_fold_gram_batched": (_c_int, [_c_vp, _c_i64, _c_vp, _c_int, _c_i64, _c_i64, _c_i64,
                                            _c_vp, _c_i64, _c_i64, _c_f, _c_vp, _c_vp, _c_sz]),
    "ifk_precondition_apply_bf16_batched_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "ifk_precondition_apply_bf16_batched": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64,
                                                     _c_i64, _c_vp, _c_vp, _c_i64, _c_i64,
                                                     _c_vp, _c_vp, _c_i64, _c_i64, _c_vp,
                                                     _c_i64, _c_i64, _c_vp, _c_sz]),
    "ifk_precondition_apply_x3_batched_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "ifk_precondition_apply_x3_batched": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64,
                                                   _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                                   _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                                   _c_vp, _c_i64, _c_i64, _c_vp, _c_sz]),
    "ifk_tri_inverse_workspace_size": (_c_sz, [_c_i64]),
    "ifk_tri_inverse": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_int,
                                 _c_vp, _c_sz]),
    "ifk_tri_inverse_x3_workspace_size": (_c_sz, [_c_i64, _c_int]),
    "ifk_tri_inverse_x3": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp,
                                    _c_sz]),
    "ifk_tri_inverse_bf16_workspace_size": (_c_sz, [_c_i64]),
    "ifk_tri_inverse_bf16": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp,
                                      _c_vp, _c_i64, _c_vp, _c_sz]),
    "ifk_cond_estimate_workspace_size": (_c_sz, [_c_i64]),
    "ifk_cond_estimate": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp,
                                   _c_vp, _c_sz]),
    "ifk_precondition_apply_bf16_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_precondition_apply_bf16": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp,
                                             _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp,
                                             _c_sz]),
    "ifk_precondition_apply_bf16_noalloc": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp,
                                                     _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp,
                                                     _c_i64]),
    "ifk_precondition_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_int]),
    "ifk_precondition": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp,
                                  _c_i64, _c_int, _c_vp, _c_i64, _c_int, _c_vp, _c_sz]),
    "ifk_precondition_apply_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_int]),
    "ifk_precondition_apply": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64,
                                        _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_vp, _c_sz]),
    "ifk_precondition_bias_workspace_size": (_c_sz, [_c_i64]),
    "ifk_precondition_bias": (_c_int, [_c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_sz]),
    "ifk_momentum_update": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_f, _c_f, _c_f,
                                     _c_int]),
    "ifk_geqrf_r_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_geqrf_r": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_int, _c_i64,
                             _c_int, _c_vp, _c_sz]),
    "ifk_trsm_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_trsm": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_int, _c_vp, _c_int, _c_i64,
                          _c_i64, _c_vp, _c_int, _c_i64, _c_int, _c_vp, _c_sz]),
    "ifk_potrf_workspace_size": (_c_sz, [_c_i64]),
    "ifk_potrf": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_int, _c_i64, _c_int,
                           _c_vp, _c_sz]),
    "ifk_gram_accumulate_workspace_size": (_c_sz, [_c_i64]),
    "ifk_gram_accumulate": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64,
                                     _c_f, _c_vp, _c_sz]),
    "ifk_axpby": (_c_int, [_c_vp, _c_f, _c_vp, _c_i64, _c_f, _c_vp, _c_i64, _c_i64, _c_i64]),
    "ifk_inv_spd_damped_workspace_size": (_c_sz, [_c_i64]),
    "ifk_inv_spd_damped": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_f, _c_vp, _c_i64,
                                    _c_vp, _c_sz]),
    "ifk_classic_precondition_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_classic_precondition": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64,
                                          _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_sz]),
    "ifk_factor_evd_workspace_size": (_c_sz, [_c_i64]),
    "ifk_factor_evd": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp,
                                _c_vp, _c_sz]),
    "ifk_laplace_scales": (_c_int, [_c_vp, _c_vp, _c_i64, _c_f, _c_f, _c_vp]),
    "ifk_laplace_sample_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_laplace_sample": (_c_int, [_c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp,
                                    _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp,
                                    _c_sz]),
    "ifk_fold_finalize_gram_inverse_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "ifk_fold_finalize_gram_inverse": (_c_int, [_c_vp, _c_i64, _c_vp, _c_int, _c_i64, _c_i64,
                                                _c_i64, _c_vp, _c_i64, _c_i64, _c_f, _c_f, _c_vp,
                                                _c_int, _c_i64, _c_i64, _c_f, _c_vp, _c_vp, _c_vp,
                                                _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64,
                                                _c_vp, _c_sz]),
    "ifk_tsqr_fold_gram_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64]),
    "ifk_tsqr_fold_gram": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64,
                                    _c_i64, _c_f, _c_vp, _c_vp, _c_sz]),
    "ifk_inv_spd_workspace_size": (_c_sz, [_c_i64]),
    "ifk_inv_spd": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_int, _c_i64, _c_int,
                             _c_vp, _c_sz]),
    "ifk_gemm_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "ifk_gemm": (_c_int, [_c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_f, _c_vp, _c_int, _c_i64,
                          _c_int, _c_vp, _c_int, _c_i64, _c_int, _c_f, _c_vp, _c_i64, _c_vp,
                          _c_sz]),
    "ifk_profile_begin": (_c_int, [_c_int]),
    "ifk_profile_end": (_c_int, [_c_i64p]),
    "ifk_profile_get": (_c_int, [_c_i64, ctypes.POINTER(_c_int), ctypes.POINTER(_c_f),
                                 ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                 _c_i64p, _c_i64p, _c_i64p]),
}

_lock = threading.Lock()
_lib = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with every signature declared."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise IFKFACBackendError(
                f"{p} not found: build it with `python -m ifkfac_amd.build` "
                "(the IFKFAC curvature path has no non-HIP implementation)")
        try:
            lib = ctypes.CDLL(p)
        except OSError as e:
            raise IFKFACBackendError(f"cannot load {p}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.ifk_abi_version()
        if ver != ABI_VERSION:
            raise IFKFACBackendError(f"{p}: ABI version {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != IFK_OK:
        msg = _lib.ifk_last_error().decode(errors="replace") if _lib is not None else ""
        raise IFKFACBackendError(f"{what} failed (status {rc}): {msg}")
