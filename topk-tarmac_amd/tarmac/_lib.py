"""Loader for ``libtarmac.so`` -- the C ABI declared in ``include/tarmac.h``.

The library is the only compute path of this package: there is no fallback.
If it has not been built, importing :mod:`tarmac` raises with instructions.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("TARMAC_LIB", _HERE / "libtarmac.so"))

TARMAC_OK = 0
TARMAC_ERR_INVALID = 1
TARMAC_ERR_UNSUPPORTED = 2
TARMAC_ERR_HIP = 3

DTYPE_F32 = 0
DTYPE_BF16 = 1
IDX_I32 = 0
IDX_I64 = 1

VARIANT_MASKED = 1
VARIANT_SORT = 2

_P = ctypes.c_void_p
_I = ctypes.c_int

#: Every entry point of include/tarmac.h with its ctypes signature.
SIGNATURES: dict[str, tuple[list, object]] = {
    "tarmac_abi_version": ([], _I),
    "tarmac_last_error": ([], ctypes.c_char_p),
    "tarmac_dense_fwd": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _P], _I),
    "tarmac_topk_fused_fwd": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P], _I),
    "tarmac_topk_stream_fwd": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "tarmac_topk_variant_fwd": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tarmac_fixedset_fwd": ([_P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _I, _P], _I),
    "tarmac_morton_window": ([_P, _P, _I, _P, _I, _I, _I, _I, _P], _I),
    "tarmac_zorder_fwd": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "tarmac_fixedset_bwd": ([_P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _I, _I, _I, _P], _I),
    "tarmac_dense_fwd_stats": ([_P, _P, _P, _P, _P, _I, _I, _I, _P], _I),
    "tarmac_dense_bwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P], _I),
    "tarmac_dense_bwd_noalloc": ([_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P], _I),
    "tarmac_knn_radius": ([_P, _P, _I, _I, _I, _I, _P], _I),
    "tarmac_knn_grid": ([_P, _P, _I, _I, _I, _I, _P], _I),
    "tarmac_grid_knn_shape": ([_I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)], _I),
    "tarmac_set_topk_filter": ([_I], _I),
    "tarmac_set_query_tiles": ([_I], _I),
    "tarmac_noop": ([_P, _P], _I),
    "tarmac_mfma_bf16_probe": ([_P, _P, _P, _I, _I, _I, _P], _I),
}


class TarmacError(RuntimeError):
    """A HIP launch failure reported by libtarmac."""


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"libtarmac.so not found at {LIB_PATH}: build it with "
            "`python topk-tarmac_amd/build.py` (or __graft_entry__.build()). "
            "The tarmac package has no non-HIP fallback.")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


LIB = _load()


def last_error() -> str:
    msg = LIB.tarmac_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    """Raise the Python exception matching a libtarmac return code."""
    if rc == TARMAC_OK:
        return
    msg = last_error()
    if rc == TARMAC_ERR_INVALID:
        raise ValueError(msg)
    if rc == TARMAC_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise TarmacError(msg)


def abi_version() -> int:
    return int(LIB.tarmac_abi_version())
