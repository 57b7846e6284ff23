"""ctypes binding of libmxfp4_gemv.so (dense MXFP4 GEMV, M = 1).

Drop-in API (call contract of the reference runtime/mxfp4_gemv_binding.py:67-154):

    mxfp4_gemv(W_packed [N, K/2] u8, W_scale [N, K/32] u8, x [K] bf16,
               out=None, stream=None) -> y [N] bf16       (y = x @ dequant(W).T)

Extension (debug): mxfp4_dequant(W_packed, W_scale) -> [N, K] bf16, the kernels'
own decode, for the bit-exact dequant check.

Errors: RuntimeError for device/dtype/shape problems and for a non-zero return
code. The library path is $MXFP4_GEMV_LIB or kernel/mxfp4-dense/libmxfp4_gemv.so.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

_LIB: Optional[ctypes.CDLL] = None


def lib_path() -> str:
    return _lib.lib_path("MXFP4_GEMV_LIB", "mxfp4-dense", "libmxfp4_gemv.so")


def _load_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        lib = _lib.load(lib_path())
        sig = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p] * 2
        lib.mxfp4_gemv_m1.argtypes = sig
        lib.mxfp4_gemv_m1.restype = ctypes.c_int
        lib.mxfp4_dequant_bf16.argtypes = ([ctypes.c_void_p] * 2 + [ctypes.c_int] * 2 +
                                           [ctypes.c_int64] * 2 + [ctypes.c_void_p] * 2)
        lib.mxfp4_dequant_bf16.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def _check_w(W_packed: torch.Tensor, W_scale: torch.Tensor) -> None:
    if not (W_packed.is_cuda and W_scale.is_cuda):
        raise RuntimeError("all tensors must be on a GPU device")
    if W_packed.dtype != torch.uint8:
        raise RuntimeError(f"W_packed must be uint8, got {W_packed.dtype}")
    if W_scale.dtype != torch.uint8:
        raise RuntimeError(f"W_scale must be uint8, got {W_scale.dtype}")
    if W_packed.dim() != 2:
        raise RuntimeError(f"W_packed must be 2-D [N, K/2], got shape {tuple(W_packed.shape)}")
    if W_scale.dim() != 2:
        raise RuntimeError(f"W_scale must be 2-D [N, K/32], got shape {tuple(W_scale.shape)}")
    if W_packed.stride(1) != 1 or W_scale.stride(1) != 1:
        raise RuntimeError("W_packed / W_scale rows must be contiguous (row stride is free)")


def mxfp4_gemv(
    W_packed: torch.Tensor,
    W_scale: torch.Tensor,
    x: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> torch.Tensor:
    """y[n] = sum_k W[n,k] * x[k] with MXFP4 W; fp32 accumulate, bf16 out."""
    _check_w(W_packed, W_scale)
    if not x.is_cuda:
        raise RuntimeError("all tensors must be on a GPU device")
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"x must be bfloat16, got {x.dtype}")
    if x.dim() != 1:
        raise RuntimeError(f"x must be 1-D [K], got shape {tuple(x.shape)}")
    K = x.shape[0]
    N = W_packed.shape[0]
    if K % 32 != 0:
        raise RuntimeError(f"K={K} must be a multiple of 32")
    if W_packed.shape[1] != K // 2:
        raise RuntimeError(f"W_packed shape {tuple(W_packed.shape)} inconsistent with K={K}")
    if tuple(W_scale.shape) != (N, K // 32):
        raise RuntimeError(f"W_scale shape {tuple(W_scale.shape)} != ({N}, {K // 32})")
    x = x.contiguous()
    if out is None:
        out = torch.empty(N, dtype=torch.bfloat16, device=x.device)
    elif tuple(out.shape) != (N,) or out.dtype != torch.bfloat16 or not out.is_cuda \
            or not out.is_contiguous():
        raise RuntimeError(f"out must be a contiguous GPU bfloat16 [{N}] tensor")
    rc = _load_lib().mxfp4_gemv_m1(
        _lib.vp(x), _lib.vp(W_packed), _lib.vp(W_scale), K, N,
        W_packed.stride(0), W_scale.stride(0), _lib.vp(out),
        ctypes.c_void_p(_lib.stream_ptr(x.device, stream)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_gemv_m1 returned {rc}")
    return out


def mxfp4_dequant(W_packed: torch.Tensor, W_scale: torch.Tensor,
                  stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """[N, K] bf16 = e2m1(W) * 2^(S-127), decoded on the GPU."""
    _check_w(W_packed, W_scale)
    N, K = W_packed.shape[0], W_packed.shape[1] * 2
    if tuple(W_scale.shape) != (N, K // 32):
        raise RuntimeError(f"W_scale shape {tuple(W_scale.shape)} != ({N}, {K // 32})")
    out = torch.empty(N, K, dtype=torch.bfloat16, device=W_packed.device)
    rc = _load_lib().mxfp4_dequant_bf16(
        _lib.vp(W_packed), _lib.vp(W_scale), K, N, W_packed.stride(0), W_scale.stride(0),
        _lib.vp(out), ctypes.c_void_p(_lib.stream_ptr(W_packed.device, stream)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_dequant_bf16 returned {rc}")
    return out


__all__ = ["mxfp4_gemv", "mxfp4_dequant"]
