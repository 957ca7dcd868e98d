"""The C ABI library (CPU only: no kernel is launched here).

Checks that libtarmac.so loads, exports every function include/tarmac.h
declares with the signatures the Python side binds, and rejects invalid
arguments with the documented codes before any HIP call is made.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tarmac.h"


def _declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"\b(tarmac_\w+)\s*\(", text)


def test_header_declares_the_boundary():
    names = _declared()
    assert len(names) == len(set(names))
    for want in ("tarmac_dense_fwd", "tarmac_topk_fused_fwd", "tarmac_topk_stream_fwd",
                 "tarmac_fixedset_fwd", "tarmac_morton_window", "tarmac_zorder_fwd",
                 "tarmac_noop", "tarmac_last_error", "tarmac_abi_version"):
        assert want in names


def test_library_exports_every_declared_symbol():
    from tarmac import _lib
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(_lib.SIGNATURES)


def test_abi_version():
    import tarmac
    assert tarmac.abi_version() == 1


P = ctypes.c_void_p


def _fake(addr=256):
    # Never dereferenced: validation fails before any launch.
    return P(addr)


@pytest.mark.parametrize("args,code,msg", [
    # (B, N, d, topk, dtype)
    ((0, 8, 16, 1, 0), 1, "B >= 1"),
    ((1, 1, 16, 1, 0), 1, "N >= 2"),
    ((1, 8, 12, 1, 0), 2, "head dim"),
    ((1, 8, 8, 1, 1), 2, "bf16 head dim"),
    ((1, 8, 96, 1, 0), 2, "head dim"),
    ((1, 8, 256, 1, 1), 2, "bf16 head dim"),
    ((1, 8, 16, 1, 7), 1, "dtype"),
    ((1, 8, 16, 0, 0), 1, "topk"),
    ((1, 8, 16, 8, 0), 1, "topk"),
])
def test_topk_validation(args, code, msg):
    from tarmac import _lib
    B, N, d, topk, dt = args
    rc = _lib.LIB.tarmac_topk_fused_fwd(_fake(), _fake(), _fake(), _fake(), None,
                                        B, N, d, topk, dt, None)
    assert rc == code
    assert msg in _lib.last_error()


def test_alignment_and_null_checks():
    from tarmac import _lib
    rc = _lib.LIB.tarmac_dense_fwd(None, _fake(), _fake(), _fake(), 1, 8, 16, 0, 0, None)
    assert rc == 1 and "null" in _lib.last_error()
    rc = _lib.LIB.tarmac_dense_fwd(_fake(260), _fake(), _fake(), _fake(), 1, 8, 16, 0, 0, None)
    assert rc == 1 and "aligned" in _lib.last_error()
    rc = _lib.LIB.tarmac_dense_fwd(_fake(), _fake(), _fake(), _fake(), 1, 8, 16, 0, 24, None)
    assert rc == 1 and "multiple of 16" in _lib.last_error()
    rc = _lib.LIB.tarmac_fixedset_fwd(_fake(), _fake(), _fake(), _fake(), 5, 2, _fake(),
                                      1, 8, 16, 0, None)
    assert rc == 1 and "idx dtype" in _lib.last_error()
    rc = _lib.LIB.tarmac_morton_window(_fake(), _fake(), 1, None, 1, 8, 2, 17, None)
    assert rc == 1 and "bits" in _lib.last_error()
    rc = _lib.LIB.tarmac_morton_window(_fake(), _fake(), 1, None, 1, 8, 8, 10, None)
    assert rc == 1 and "k <= N-1" in _lib.last_error()
    rc = _lib.LIB.tarmac_zorder_fwd(_fake(), _fake(), _fake(), _fake(), _fake(), None,
                                    1, 100000, 16, 2, 16, 0, None)
    assert rc == 2 and "capacity" in _lib.last_error()
    rc = _lib.LIB.tarmac_topk_stream_fwd(_fake(), _fake(), _fake(), _fake(), None,
                                         2, 64, 16, 2, 0, 40, None)
    assert rc == 1 and "multiple of 16" in _lib.last_error()


def test_python_wrappers_refuse_cpu_tensors():
    """No CPU path exists: the kernels need device tensors."""
    from tarmac.kernels import fused_dense_attention, streaming_topk_attention
    q = torch.randn(2, 8, 16)
    with pytest.raises(RuntimeError, match="GPU only"):
        fused_dense_attention(q, q, q)
    with pytest.raises(RuntimeError, match="GPU only"):
        streaming_topk_attention(q, q, q, 2)


def test_python_wrappers_mirror_reference_asserts():
    from tarmac.kernels import (fused_topk_attention, fused_topk_attention_tiled,
                                streaming_topk_attention)
    q = torch.randn(1, 1025, 16)
    with pytest.raises(AssertionError):
        fused_topk_attention(q, q, q, 2)       # fused_topk_attention.py:341
    with pytest.raises(AssertionError):
        fused_topk_attention_tiled(q, q, q, 2)  # fused_topk_attention.py:309
    q = torch.randn(1, 32, 16)
    with pytest.raises(AssertionError):
        streaming_topk_attention(q, q, q, 9)   # streaming_topk_attention.py:226
    with pytest.raises(AssertionError):
        fused_topk_attention(q, q[:, :16], q, 2)


def test_filter_mode_switch():
    """tarmac_set_topk_filter: modes 0 to 5 return the previous mode; anything
    else is refused with -1 and a message, leaving the mode unchanged."""
    from tarmac import _lib
    lib = _lib.LIB
    prev = lib.tarmac_set_topk_filter(1)
    try:
        assert lib.tarmac_set_topk_filter(2) == 1
        assert lib.tarmac_set_topk_filter(3) == 2
        assert lib.tarmac_set_topk_filter(4) == 3
        assert lib.tarmac_set_topk_filter(5) == 4
        assert lib.tarmac_set_topk_filter(0) == 5
        assert lib.tarmac_set_topk_filter(7) == -1
        assert "mode must be 0 to 5" in _lib.last_error()
        assert lib.tarmac_set_topk_filter(-1) == -1
        assert lib.tarmac_set_topk_filter(1) == 0
    finally:
        lib.tarmac_set_topk_filter(prev)


def test_query_tiles_switch():
    """tarmac_set_query_tiles: modes 0 to 2 return the previous mode; anything
    else is refused with -1 and a message, leaving the mode unchanged."""
    from tarmac import _lib
    lib = _lib.LIB
    prev = lib.tarmac_set_query_tiles(0)
    try:
        assert lib.tarmac_set_query_tiles(1) == 0
        assert lib.tarmac_set_query_tiles(2) == 1
        assert lib.tarmac_set_query_tiles(3) == -1
        assert "mode must be 0 to 2" in _lib.last_error()
        assert lib.tarmac_set_query_tiles(-1) == -1
        assert lib.tarmac_set_query_tiles(0) == 2
    finally:
        lib.tarmac_set_query_tiles(prev)


def test_grid_knn_shape_matches_the_reference_formula():
    """tarmac_grid_knn_shape (host only) against the oracle's restatement of
    grid_knn_shape (pinned to the reference's values) over a wide range."""
    import tarmac_oracle as O
    from tarmac.kernels import grid_knn_shape
    for N in list(range(2, 600)) + [1000, 1023, 1024, 2047, 2048, 4095, 4096, 8192]:
        for kk in (1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 64):
            if kk < N:
                assert grid_knn_shape(N, kk) == O.grid_knn_shape(N, kk), (N, kk)


def test_knn_validation():
    from tarmac import _lib
    L = _lib.LIB
    assert L.tarmac_knn_radius(None, _fake(), 1, 1, 8, 2, None) == 1
    assert "null" in _lib.last_error()
    assert L.tarmac_knn_radius(_fake(260), _fake(), 1, 1, 8, 2, None) == 1
    assert "aligned" in _lib.last_error()
    assert L.tarmac_knn_grid(_fake(), _fake(), 1, 1, 8, 8, None) == 1
    assert "k <= N-1" in _lib.last_error()
    assert L.tarmac_knn_grid(_fake(), _fake(), 3, 1, 8, 2, None) == 1
    assert "idx dtype" in _lib.last_error()
    assert L.tarmac_knn_radius(_fake(), _fake(), 1, 1, 9000, 2, None) == 2
    assert "capacity" in _lib.last_error()
    assert L.tarmac_knn_grid(_fake(), _fake(), 1, 1, 5000, 2, None) == 2
    assert "capacity" in _lib.last_error()
    G, M = ctypes.c_int(), ctypes.c_int()
    assert L.tarmac_grid_knn_shape(0, 2, ctypes.byref(G), ctypes.byref(M)) == 1
