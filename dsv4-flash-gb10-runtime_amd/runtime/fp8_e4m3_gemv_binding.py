"""ctypes binding of libfp8_e4m3_gemv.so (FP8 E4M3FN GEMV, 128x128 E8M0 tiles).

Drop-in API (call contract of the reference runtime/fp8_e4m3_gemv_binding.py:77-168):

    fp8_e4m3_gemv(W_fp8 [N, K] u8, W_scale [ceil(N/128), K/128] u8, x [K] bf16,
                  out=None, stream=None) -> y [N] bf16

Differences, both extensions: N need not be a multiple of 128 (the reference
raises for it), and x may be [T, K] with T <= 16, in which case one launch
streams W once for all T tokens and y is [T, N].

Extension: fp8_e4m3_gemv_multi([(W, S), ...], x) -> [y, ...]: several GEMVs
on one activation in one launch.

Extension (debug): fp8_e4m3_dequant(W_fp8, W_scale) -> [N, K] bf16.

Errors: RuntimeError for device/dtype/shape problems and for a non-zero
return code. The library path is $FP8_E4M3_GEMV_LIB or
kernel/fp8-dense/libfp8_e4m3_gemv.so.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

FP8_BLOCK_TILE = 128
MAX_TOKENS = 16

_LIB: Optional[ctypes.CDLL] = None


def lib_path() -> str:
    return _lib.lib_path("FP8_E4M3_GEMV_LIB", "fp8-dense", "libfp8_e4m3_gemv.so")


def _load_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        lib = _lib.load(lib_path())
        P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        lib.fp8_e4m3_gemv_m1.argtypes = [P, P, P, I, I, L, L, P, P]
        lib.fp8_e4m3_gemv_m1.restype = I
        lib.fp8_e4m3_gemv.argtypes = [P, L, P, P, I, I, I, L, L, P, L, P]
        lib.fp8_e4m3_gemv.restype = I
        lib.fp8_e4m3_dequant_bf16.argtypes = [P, P, I, I, L, L, P, P]
        lib.fp8_e4m3_dequant_bf16.restype = I
        lib.fp8_e4m3_gemv_grouped.argtypes = [P, L, L, P, P, I, I, I, I, L, L, P, L, L, P]
        lib.fp8_e4m3_gemv_grouped.restype = I
        lib.fp8_e4m3_swiglu_gemv.argtypes = [P, L, P, P, P, P, I, I, I, L, L, ctypes.c_float, I, P, L, P]
        lib.fp8_e4m3_swiglu_gemv.restype = I
        lib.fp8_e4m3_rmsnorm_gemv.argtypes = [P, P, P, ctypes.c_float, P, P, I, I, I, L, L, P, P, P, P]
        lib.fp8_e4m3_rmsnorm_gemv.restype = I
        lib.fp8_e4m3_gemv_multi.argtypes = [P, L, I, I, I] + [P] * 7 + [P]
        lib.fp8_e4m3_gemv_multi.restype = I
        lib.fp8_e4m3_gemv_f32s.argtypes = [P, L, P, P, I, I, I, L, L, P, L, P]
        lib.fp8_e4m3_gemv_f32s.restype = I
        _LIB = lib
    return _LIB


def _check_w(W_fp8: torch.Tensor, W_scale: torch.Tensor) -> None:
    if not (W_fp8.is_cuda and W_scale.is_cuda):
        raise RuntimeError("all tensors must be on a GPU device")
    if W_fp8.dtype != torch.uint8:
        raise RuntimeError(f"W_fp8 must be uint8 (raw E4M3), got {W_fp8.dtype}")
    if W_scale.dtype != torch.uint8:
        raise RuntimeError(f"W_scale must be uint8 (raw E8M0), got {W_scale.dtype}")
    if W_fp8.dim() != 2:
        raise RuntimeError(f"W_fp8 must be 2-D [N, K], got shape {tuple(W_fp8.shape)}")
    if W_scale.dim() != 2:
        raise RuntimeError(f"W_scale must be 2-D [ceil(N/128), K/128], got {tuple(W_scale.shape)}")
    if W_fp8.stride(1) != 1 or W_scale.stride(1) != 1:
        raise RuntimeError("W_fp8 / W_scale rows must be contiguous (row stride is free)")
    N, K = W_fp8.shape
    if K % FP8_BLOCK_TILE != 0:
        raise RuntimeError(f"K={K} must be a multiple of {FP8_BLOCK_TILE}")
    want = ((N + FP8_BLOCK_TILE - 1) // FP8_BLOCK_TILE, K // FP8_BLOCK_TILE)
    if tuple(W_scale.shape) != want:
        raise RuntimeError(f"W_scale shape {tuple(W_scale.shape)} != {want} "
                           f"(one E8M0 byte per 128x128 tile)")


def fp8_e4m3_gemv(
    W_fp8: torch.Tensor,
    W_scale: torch.Tensor,
    x: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> torch.Tensor:
    """y = x @ dequant(W).T for x [K] (y [N]) or x [T, K] (y [T, N]); fp32 accumulate."""
    _check_w(W_fp8, W_scale)
    if not x.is_cuda:
        raise RuntimeError("all tensors must be on a GPU device")
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"x must be bfloat16, got {x.dtype}")
    if x.dim() not in (1, 2):
        raise RuntimeError(f"x must be [K] or [T, K], got shape {tuple(x.shape)}")
    N, K = W_fp8.shape
    if x.shape[-1] != K:
        raise RuntimeError(f"x last dim {x.shape[-1]} != K={K}")
    T = 1 if x.dim() == 1 else x.shape[0]
    if T > MAX_TOKENS:
        raise RuntimeError(f"T={T} > {MAX_TOKENS}")
    x = x.contiguous()
    oshape = (N,) if x.dim() == 1 else (T, N)
    if out is None:
        out = torch.empty(oshape, dtype=torch.bfloat16, device=x.device)
    elif tuple(out.shape) != oshape or out.dtype != torch.bfloat16 or not out.is_cuda \
            or not out.is_contiguous():
        raise RuntimeError(f"out must be a contiguous GPU bfloat16 {oshape} tensor")
    s = ctypes.c_void_p(_lib.stream_ptr(x.device, stream))
    lib = _load_lib()
    if x.dim() == 1:
        rc = lib.fp8_e4m3_gemv_m1(_lib.vp(x), _lib.vp(W_fp8), _lib.vp(W_scale), K, N,
                                  W_fp8.stride(0), W_scale.stride(0), _lib.vp(out), s)
        name = "fp8_e4m3_gemv_m1"
    else:
        rc = lib.fp8_e4m3_gemv(_lib.vp(x), K, _lib.vp(W_fp8), _lib.vp(W_scale), K, N, T,
                               W_fp8.stride(0), W_scale.stride(0), _lib.vp(out), N, s)
        name = "fp8_e4m3_gemv"
    if rc != 0:
        raise RuntimeError(f"{name} returned {rc}")
    return out


def fp8_e4m3_gemv_f32s(
    W_fp8: torch.Tensor,
    W_scale: torch.Tensor,
    x: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> torch.Tensor:
    """fp8_e4m3_gemv with one fp32 scale per 128x128 tile (W_scale float32
    [ceil(N/128), K/128], rows contiguous) instead of E8M0 bytes: y = x @
    (e4m3(W) * S).T for x [K] (y [N]) or x [T, K] (y [T, N]); fp32 accumulate."""
    if not (W_fp8.is_cuda and W_scale.is_cuda and x.is_cuda):
        raise RuntimeError("all tensors must be on a GPU device")
    if W_fp8.dtype != torch.uint8:
        raise RuntimeError(f"W_fp8 must be uint8 (E4M3FN bits), got {W_fp8.dtype}")
    if W_scale.dtype != torch.float32:
        raise RuntimeError(f"W_scale must be float32, got {W_scale.dtype}")
    if W_fp8.dim() != 2 or W_scale.dim() != 2 or W_fp8.stride(1) != 1 or W_scale.stride(1) != 1:
        raise RuntimeError("W_fp8 and W_scale must be 2-D with contiguous rows")
    N, K = W_fp8.shape
    if tuple(W_scale.shape) != ((N + 127) // 128, K // 128):
        raise RuntimeError(f"W_scale must be [{(N + 127) // 128}, {K // 128}], got {tuple(W_scale.shape)}")
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"x must be bfloat16, got {x.dtype}")
    if x.dim() not in (1, 2) or x.shape[-1] != K:
        raise RuntimeError(f"x must be [K] or [T, K] with K={K}, got shape {tuple(x.shape)}")
    T = 1 if x.dim() == 1 else x.shape[0]
    if T > MAX_TOKENS:
        raise RuntimeError(f"T={T} > {MAX_TOKENS}")
    x = x.contiguous()
    oshape = (N,) if x.dim() == 1 else (T, N)
    if out is None:
        out = torch.empty(oshape, dtype=torch.bfloat16, device=x.device)
    elif tuple(out.shape) != oshape or out.dtype != torch.bfloat16 or not out.is_cuda \
            or not out.is_contiguous():
        raise RuntimeError(f"out must be a contiguous GPU bfloat16 {oshape} tensor")
    s = ctypes.c_void_p(_lib.stream_ptr(x.device, stream))
    rc = _load_lib().fp8_e4m3_gemv_f32s(_lib.vp(x), K, _lib.vp(W_fp8), _lib.vp(W_scale), K, N, T,
                                        W_fp8.stride(0), W_scale.stride(0), _lib.vp(out), N, s)
    if rc != 0:
        raise RuntimeError(f"fp8_e4m3_gemv_f32s returned {rc}")
    return out


def fp8_e4m3_gemv_grouped(
    W_fp8: torch.Tensor,
    W_scale: torch.Tensor,
    x: torch.Tensor,
    groups: int,
    out: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> torch.Tensor:
    """G GEMVs in one launch: W [G*N, K] holds the groups' weights stacked by
    rows; x [G, K] or [T, G, K]; y[..., g, :] = x[..., g, :] @ dequant(W[g*N:(g+1)*N]).T
    ([G, N] or [T, G, N]). The grouped output projection wo_a (G=8, N=1024,
    K=4096) of kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:484-499."""
    _check_w(W_fp8, W_scale)
    if not x.is_cuda or x.dtype != torch.bfloat16:
        raise RuntimeError("x must be a GPU bfloat16 tensor")
    if x.dim() not in (2, 3):
        raise RuntimeError(f"x must be [G, K] or [T, G, K], got shape {tuple(x.shape)}")
    GN, K = W_fp8.shape
    G = groups
    if G < 1 or GN % G != 0:
        raise RuntimeError(f"W rows {GN} are not a multiple of groups={G}")
    N = GN // G
    if x.shape[-2:] != (G, K):
        raise RuntimeError(f"x trailing shape {tuple(x.shape[-2:])} != ({G}, {K})")
    T = 1 if x.dim() == 2 else x.shape[0]
    if T > MAX_TOKENS:
        raise RuntimeError(f"T={T} > {MAX_TOKENS}")
    x = x.contiguous()
    oshape = (G, N) if x.dim() == 2 else (T, G, N)
    if out is None:
        out = torch.empty(oshape, dtype=torch.bfloat16, device=x.device)
    elif tuple(out.shape) != oshape or out.dtype != torch.bfloat16 or not out.is_cuda \
            or not out.is_contiguous():
        raise RuntimeError(f"out must be a contiguous GPU bfloat16 {oshape} tensor")
    rc = _load_lib().fp8_e4m3_gemv_grouped(
        _lib.vp(x), G * K, K, _lib.vp(W_fp8), _lib.vp(W_scale), G, K, N, T, W_fp8.stride(0),
        W_scale.stride(0), _lib.vp(out), G * N, N, ctypes.c_void_p(_lib.stream_ptr(x.device, stream)))
    if rc != 0:
        raise RuntimeError(f"fp8_e4m3_gemv_grouped returned {rc}")
    return out


def fp8_e4m3_gemv_multi(
    mats,
    x: torch.Tensor,
    outs=None,
    stream: Optional[torch.cuda.Stream] = None,
):
    """Several GEMVs on one activation in one launch: mats is a list of
    (W_fp8 [N_m, K], W_scale [ceil(N_m/128), K/128]) pairs (at most 8); x is
    [K] or [T, K]; returns the list of y_m ([N_m] or [T, N_m]). wq_a and wkv on
    the normalised row, kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:395-418."""
    mats = list(mats)
    if not 1 <= len(mats) <= 8:
        raise RuntimeError(f"{len(mats)} matrices: between 1 and 8 are allowed")
    if not x.is_cuda or x.dtype != torch.bfloat16:
        raise RuntimeError("x must be a GPU bfloat16 tensor")
    K = x.shape[-1]
    T = 1 if x.dim() == 1 else x.shape[0]
    if T > MAX_TOKENS:
        raise RuntimeError(f"T={T} > {MAX_TOKENS}")
    x = x.contiguous()
    n = len(mats)
    ws, ss, Ns, wst, sst, ys, yst = [], [], [], [], [], [], []
    if outs is None:
        outs = [None] * n
    res = []
    for (W, S), o in zip(mats, outs):
        _check_w(W, S)
        if W.shape[1] != K:
            raise RuntimeError(f"W has K={W.shape[1]}, x has K={K}")
        Nm = W.shape[0]
        oshape = (Nm,) if x.dim() == 1 else (T, Nm)
        if o is None:
            o = torch.empty(oshape, dtype=torch.bfloat16, device=x.device)
        elif tuple(o.shape) != oshape or o.dtype != torch.bfloat16 or not o.is_cuda or not o.is_contiguous():
            raise RuntimeError(f"out must be a contiguous GPU bfloat16 {oshape} tensor")
        ws.append(W.data_ptr())
        ss.append(S.data_ptr())
        Ns.append(Nm)
        wst.append(W.stride(0))
        sst.append(S.stride(0))
        ys.append(o.data_ptr())
        yst.append(Nm)
        res.append(o)
    PA = ctypes.c_void_p * n
    IA = ctypes.c_int * n
    LA = ctypes.c_int64 * n
    rc = _load_lib().fp8_e4m3_gemv_multi(
        _lib.vp(x), K, K, T, n, PA(*ws), PA(*ss), IA(*Ns), LA(*wst), LA(*sst), PA(*ys), LA(*yst),
        ctypes.c_void_p(_lib.stream_ptr(x.device, stream)))
    if rc != 0:
        raise RuntimeError(f"fp8_e4m3_gemv_multi returned {rc}")
    return res


def fp8_e4m3_swiglu_gemv(
    W1_fp8: torch.Tensor,
    W1_scale: torch.Tensor,
    W3_fp8: torch.Tensor,
    W3_scale: torch.Tensor,
    x: torch.Tensor,
    limit: float = 10.0,
    clamp_up: bool = True,
    out: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> torch.Tensor:
    """act = bf16( silu(clamp(bf16(W1 x))) * clamp?(bf16(W3 x)) ) in one launch:
    the shared expert's gate, up and SwiGLU (runtime/dsv4_engine_mxfp4.py:399-410,
    which clamps both, clamp_up=True; kernel/cpp-engine-mxfp4/
    dsv4_engine_mxfp4_wire.cu:510-548 clamps the gate only, clamp_up=False).
    x [K] or [T, K]; K must be 2048 or 4096."""
    _check_w(W1_fp8, W1_scale)
    _check_w(W3_fp8, W3_scale)
    if W1_fp8.shape != W3_fp8.shape or W1_fp8.stride() != W3_fp8.stride() \
            or W1_scale.stride() != W3_scale.stride():
        raise RuntimeError("W1 and W3 must have the same shape and strides")
    if not x.is_cuda or x.dtype != torch.bfloat16 or x.dim() not in (1, 2):
        raise RuntimeError("x must be a GPU bfloat16 [K] or [T, K] tensor")
    N, K = W1_fp8.shape
    if x.shape[-1] != K:
        raise RuntimeError(f"x last dim {x.shape[-1]} != K={K}")
    T = 1 if x.dim() == 1 else x.shape[0]
    if T > MAX_TOKENS:
        raise RuntimeError(f"T={T} > {MAX_TOKENS}")
    x = x.contiguous()
    oshape = (N,) if x.dim() == 1 else (T, N)
    if out is None:
        out = torch.empty(oshape, dtype=torch.bfloat16, device=x.device)
    elif tuple(out.shape) != oshape or out.dtype != torch.bfloat16 or not out.is_cuda \
            or not out.is_contiguous():
        raise RuntimeError(f"out must be a contiguous GPU bfloat16 {oshape} tensor")
    rc = _load_lib().fp8_e4m3_swiglu_gemv(
        _lib.vp(x), K, _lib.vp(W1_fp8), _lib.vp(W1_scale), _lib.vp(W3_fp8), _lib.vp(W3_scale), K, N, T,
        W1_fp8.stride(0), W1_scale.stride(0), float(limit), int(bool(clamp_up)), _lib.vp(out), N,
        ctypes.c_void_p(_lib.stream_ptr(x.device, stream)))
    if rc != 0:
        raise RuntimeError(f"fp8_e4m3_swiglu_gemv returned {rc}")
    return out


def fp8_e4m3_rmsnorm_gemv(
    W_fp8: torch.Tensor,
    W_scale: torch.Tensor,
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    residual: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
    stream: Optional[torch.cuda.Stream] = None,
):
    """RMSNorm (with the residual add when `residual` is given) and the FP8
    GEMV that consumes it, in one launch. x, residual [K] or [T, K] (T <= 4),
    K in {2048, 4096}. Returns (y, x_norm, new_residual or None), with the bits
    of rmsnorm_fuse_residual_add / rmsnorm_fuse_fwd and fp8_e4m3_gemv."""
    _check_w(W_fp8, W_scale)
    N, K = W_fp8.shape
    for name, t in (("x", x), ("norm_weight", norm_weight)) + ((("residual", residual),) if residual is not None else ()):
        if not t.is_cuda or t.dtype != torch.bfloat16:
            raise RuntimeError(f"{name} must be a GPU bfloat16 tensor")
    if x.dim() not in (1, 2) or x.shape[-1] != K or norm_weight.shape != (K,):
        raise RuntimeError(f"x must be [K] or [T, K] and norm_weight [K], K={K}")
    if residual is not None and residual.shape != x.shape:
        raise RuntimeError("residual must have the shape of x")
    T = 1 if x.dim() == 1 else x.shape[0]
    x = x.contiguous()
    norm_weight = norm_weight.contiguous()
    y = torch.empty((N,) if x.dim() == 1 else (T, N), dtype=torch.bfloat16, device=x.device)
    x_norm = torch.empty_like(x)
    new_res = None
    if residual is not None:
        residual = residual.contiguous()
        new_res = torch.empty_like(x)
    rc = _load_lib().fp8_e4m3_rmsnorm_gemv(
        _lib.vp(x), _lib.vp(residual) if residual is not None else None, _lib.vp(norm_weight), float(eps),
        _lib.vp(W_fp8), _lib.vp(W_scale), K, N, T, W_fp8.stride(0), W_scale.stride(0), _lib.vp(y),
        _lib.vp(x_norm), _lib.vp(new_res) if new_res is not None else None,
        ctypes.c_void_p(_lib.stream_ptr(x.device, stream)))
    if rc != 0:
        raise RuntimeError(f"fp8_e4m3_rmsnorm_gemv returned {rc}")
    return y, x_norm, new_res


def fp8_e4m3_dequant(W_fp8: torch.Tensor, W_scale: torch.Tensor,
                     stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """[N, K] bf16 = e4m3(W) * 2^(S[n/128, k/128] - 127), decoded on the GPU."""
    _check_w(W_fp8, W_scale)
    N, K = W_fp8.shape
    out = torch.empty(N, K, dtype=torch.bfloat16, device=W_fp8.device)
    rc = _load_lib().fp8_e4m3_dequant_bf16(
        _lib.vp(W_fp8), _lib.vp(W_scale), K, N, W_fp8.stride(0), W_scale.stride(0), _lib.vp(out),
        ctypes.c_void_p(_lib.stream_ptr(W_fp8.device, stream)))
    if rc != 0:
        raise RuntimeError(f"fp8_e4m3_dequant_bf16 returned {rc}")
    return out


__all__ = ["fp8_e4m3_gemv", "fp8_e4m3_dequant", "FP8_BLOCK_TILE"]
