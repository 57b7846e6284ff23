"""ctypes binding of librmsnorm_fuse.so (RMSNorm, fused residual-add + RMSNorm).

Drop-in API (call contract of the reference runtime/rmsnorm_fuse_binding.py:78-170):

    rmsnorm_fuse_fwd(x, weight, eps=1e-6, out=None) -> y
    rmsnorm_fuse_residual_add(x, residual, weight, eps=1e-6,
                              out_norm=None, out_new_residual=None) -> (y, new_residual)

x / residual / outputs: bf16 [..., H] on the GPU; weight: bf16 [H]. Launches
on torch's current stream.

Errors: TypeError for dtype/device, ValueError for shape/contiguity, and
RuntimeError for a non-zero return code. The library path is
$RMSNORM_FUSE_LIB or kernel/rmsnorm-fuse/librmsnorm_fuse.so.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

_LIB: Optional[ctypes.CDLL] = None


def lib_path() -> str:
    return _lib.lib_path("RMSNORM_FUSE_LIB", "rmsnorm-fuse", "librmsnorm_fuse.so")


def _load_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        lib = _lib.load(lib_path())
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        lib.rmsnorm_fuse_fwd.argtypes = [P, P, P, I, I, F, P]
        lib.rmsnorm_fuse_fwd.restype = I
        lib.rmsnorm_fuse_residual_add.argtypes = [P, P, P, P, P, I, I, F, P]
        lib.rmsnorm_fuse_residual_add.restype = I
        _LIB = lib
    return _LIB


def _check(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name}: expected bfloat16, got {t.dtype}")
    if not t.is_cuda:
        raise TypeError(f"{name}: expected a GPU tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


def _out(name: str, t: Optional[torch.Tensor], like: torch.Tensor) -> torch.Tensor:
    if t is None:
        return torch.empty_like(like)
    _check(name, t)
    if t.numel() != like.numel():
        raise ValueError(f"{name} shape {tuple(t.shape)} != {tuple(like.shape)}")
    return t.view(like.shape)


def rmsnorm_fuse_fwd(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = weight * x * rsqrt(mean(x^2) + eps), per row of the last dimension."""
    _check("x", x)
    _check("weight", weight)
    hidden = x.shape[-1]
    if weight.numel() != hidden:
        raise ValueError(f"weight numel {weight.numel()} != hidden {hidden}")
    x2 = x.view(-1, hidden)
    y = _out("out", out, x2)
    rc = _load_lib().rmsnorm_fuse_fwd(_lib.vp(x2), _lib.vp(weight), _lib.vp(y), x2.shape[0],
                                      hidden, float(eps), ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"rmsnorm_fuse_fwd kernel rc={rc}")
    return y.view(x.shape)


def rmsnorm_fuse_residual_add(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    out_norm: Optional[torch.Tensor] = None,
    out_new_residual: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """t = x + residual; returns (weight * t * rsqrt(mean(t^2) + eps), t) in bf16."""
    _check("x", x)
    _check("residual", residual)
    _check("weight", weight)
    if x.shape != residual.shape:
        raise ValueError(f"x {tuple(x.shape)} != residual {tuple(residual.shape)}")
    hidden = x.shape[-1]
    if weight.numel() != hidden:
        raise ValueError(f"weight numel {weight.numel()} != hidden {hidden}")
    x2 = x.view(-1, hidden)
    r2 = residual.view(-1, hidden)
    y = _out("out_norm", out_norm, x2)
    nr = _out("out_new_residual", out_new_residual, x2)
    rc = _load_lib().rmsnorm_fuse_residual_add(
        _lib.vp(x2), _lib.vp(r2), _lib.vp(weight), _lib.vp(y), _lib.vp(nr), x2.shape[0], hidden,
        float(eps), ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"rmsnorm_fuse_residual_add kernel rc={rc}")
    return y.view(x.shape), nr.view(x.shape)


__all__ = ["rmsnorm_fuse_fwd", "rmsnorm_fuse_residual_add"]
