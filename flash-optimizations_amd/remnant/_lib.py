"""Loader for the C-ABI library ``libremnant_mi355x.so`` (include/remnant_mi355x.h).

The library is built in-tree by ``flash-optimizations_amd/csrc/Makefile``
(``__graft_entry__.build()``). There is no fallback: when the library is
missing, every operator raises instead of computing anything on the CPU.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libremnant_mi355x.so")

STATUS = {
    0: "ok",
    -1: "required pointer missing",
    -2: "size or stride out of range",
    -3: "pointer not aligned",
    -4: "unsupported dtype",
    -5: "workspace too small",
    -6: "HIP launch failed",
}

# (name, restype, argtypes) for every symbol declared in include/remnant_mi355x.h
_i64, _i32, _f32, _vp, _sz = (ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p,
                              ctypes.c_size_t)
SIGNATURES = {
    "rm_version": (_i32, []),
    "rm_pack_rows": (_i32, [_vp, _i32, _i64, _vp, _f32, _vp, _i64, _vp, _i64, _vp]),
    "rm_pack_rows_k": (_i32, [_vp, _i32, _i64, _vp, _f32, _vp, _i64, _vp, _i64, _i32, _vp]),
    "rm_pack_rows_planes": (_i32, [_vp, _i32, _i64, _vp, _f32, _vp, _i64, _vp, _vp, _vp, _i64,
                                   _i32, _vp]),
    "rm_native_store_rows": (_i32, [_vp, _i32, _i64, _vp, _f32, _vp, _vp, _vp, _i64, _i64, _vp,
                                    _i64, _vp]),
    "rm_unpack_gather_bf16_planes": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _i64, _i64, _vp,
                                            _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp,
                                            _vp]),
    "rm_packed_to_native_planes": (_i32, [_vp, _vp, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                                          _vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "rm_remnant_sparse_decode_planes_fwd": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64,
                                                   _vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp,
                                                   _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp,
                                                   _f32, _vp, _vp, _vp, _sz, _vp]),
    "rm_unpack_gather_bf16": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                     _i64, _i64, _vp, _i64, _vp, _vp]),
    "rm_unpack_gather_bf16_k": (_i32, [_vp, _i64, _i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp,
                                       _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "rm_packed_to_native": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                   _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "rm_copy_records": (_i32, [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i32,
                               _i32, _vp]),
    "rm_sparse_decode_workspace": (_i32, [_i64, _i64, _i64, ctypes.POINTER(ctypes.c_int32),
                                          ctypes.POINTER(ctypes.c_size_t)]),
    "rm_remnant_sparse_decode_fwd": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i64,
                                            _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _f32, _vp,
                                            _vp, _vp, _sz, _vp]),
    "rm_native_sparse_decode_fwd": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i64,
                                           _vp, _vp, _i64, _vp, _vp, _f32, _vp, _vp, _vp, _sz,
                                           _vp]),
    "rm_sparse_decode_workspace_swa": (_i32, [_i64, _i64, _i64, _i64,
                                              ctypes.POINTER(ctypes.c_int32),
                                              ctypes.POINTER(ctypes.c_size_t)]),
    "rm_remnant_sparse_decode_swa_fwd": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64,
                                                _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64,
                                                _vp, _vp, _vp, _i64, _vp, _f32, _vp, _vp, _vp,
                                                _sz, _vp]),
    "rm_remnant_sparse_decode_swa_noalloc_fwd": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp,
                                                        _i64, _i64, _vp, _vp, _i64, _vp, _vp,
                                                        _i64, _vp, _i64, _vp, _vp, _vp, _i64,
                                                        _vp, _f32, _vp, _vp, _vp]),
    "rm_native_sparse_decode_swa_fwd": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64,
                                               _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64,
                                               _vp, _vp, _f32, _vp, _vp, _vp, _sz, _vp]),
}

_lib = None


class RemnantLibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RemnantLibraryMissing(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(or make -C flash-optimizations_amd/csrc)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what}: {STATUS.get(status, 'error')} (status {status})")
