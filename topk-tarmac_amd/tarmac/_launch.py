"""Tensor plumbing between PyTorch and the C ABI: device/dtype checks,
contiguity and alignment, stream handles. No compute happens here."""

from __future__ import annotations

import ctypes
import functools

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"tarmac kernels take float32 or bfloat16 tensors (float16 through "
                        f"the Python wrappers), got {t.dtype}") from None


def on_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError(
                "tarmac kernels run on the GPU only (HIP); got a tensor on "
                f"{t.device}. There is no CPU path.")


def ready(t: torch.Tensor, align: int = 16) -> torch.Tensor:
    """Contiguous and ``align``-byte aligned (a copy only when needed)."""
    t = t.contiguous()
    if t.data_ptr() % align:
        t = t.clone()
    return t


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(None if t is None else t.data_ptr())


def stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """Validate and normalise a (q, k, v) triple: same shape, 3-D, same dtype,
    on the GPU. Returns the prepared tensors."""
    assert k.shape == v.shape == q.shape, "q, k and v must share shape [B, N, d]"
    if q.dim() != 3:
        raise ValueError(f"expected [B, N, d] tensors, got shape {tuple(q.shape)}")
    on_gpu(q, k, v)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k and v must share a dtype")
    dtype_code(q)
    return ready(q), ready(k), ready(v)


def half_on_f32(fn):
    """Let a forward wrapper ``fn(q, k, v, ...)`` take float16 heads: they run
    the fp32 kernels on fp32 copies. Every float16 value is an fp32 value, so
    the scores and retained sets are those of the inputs themselves (the
    exact top k of their canonical fp32 scores); the output comes back as
    float16 (rounded once), indices unchanged."""

    @functools.wraps(fn)
    def wrapper(q, k, v, *args, **kwargs):
        if q.dtype != torch.float16:
            return fn(q, k, v, *args, **kwargs)
        if not (k.dtype == v.dtype == torch.float16):
            raise TypeError("q, k and v must share a dtype")
        res = fn(q.float(), k.float(), v.float(), *args, **kwargs)
        if isinstance(res, tuple):
            return (res[0].to(torch.float16),) + tuple(res[1:])
        return res.to(torch.float16)

    return wrapper
