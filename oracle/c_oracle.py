"""ctypes access to the scalar C oracle (oracle/libmx_oracle.so). TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmx_oracle.so")
_LIB = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.mxo_bf16_rne.argtypes = [F]
        L.mxo_bf16_rne.restype = ctypes.c_uint16
        L.mxo_e2m1.argtypes = [I]
        L.mxo_e2m1.restype = ctypes.c_double
        L.mxo_e8m0.argtypes = [ctypes.c_uint8]
        L.mxo_e8m0.restype = F
        L.mxo_e4m3fn.argtypes = [ctypes.c_uint8]
        L.mxo_e4m3fn.restype = F
        L.mxo_mxfp4_dequant.argtypes = [P, P, I, I, P]
        L.mxo_fp8_dequant.argtypes = [P, P, I, I, P]
        L.mxo_mxfp4_gemv.argtypes = [P, I, P, P, I, I, P]
        L.mxo_fp8_gemv.argtypes = [P, I, P, P, I, I, P]
        L.mxo_grouped_gemv.argtypes = [P] * 8 + [I] * 4 + [P]
        L.mxo_rmsnorm_residual.argtypes = [P, P, P, I, I, F, P, P]
        L.mxo_rmsnorm.argtypes = [P, P, I, I, F, P]
        L.mxo_router_logits.argtypes = [P, I, P, I, I, P]
        L.mxo_route_sqrt_softplus.argtypes = [P, I, I, F, P, P]
        L.mxo_route_sqrt_softplus.restype = I
        _LIB = L
    return _LIB


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def mxfp4_dequant(packed, scale) -> np.ndarray:
    packed, scale = _c(packed, np.uint8), _c(scale, np.uint8)
    N, K = packed.shape[0], packed.shape[1] * 2
    out = np.empty((N, K), dtype=np.uint16)
    lib().mxo_mxfp4_dequant(_p(packed), _p(scale), N, K, _p(out))
    return out


def fp8_dequant(w, s) -> np.ndarray:
    w, s = _c(w, np.uint8), _c(s, np.uint8)
    N, K = w.shape
    out = np.empty((N, K), dtype=np.uint16)
    lib().mxo_fp8_dequant(_p(w), _p(s), N, K, _p(out))
    return out


def mxfp4_gemv(x, packed, scale) -> np.ndarray:
    x2 = _c(np.atleast_2d(x), np.uint16)
    packed, scale = _c(packed, np.uint8), _c(scale, np.uint8)
    T, K = x2.shape
    N = packed.shape[0]
    y = np.empty((T, N), dtype=np.uint16)
    lib().mxo_mxfp4_gemv(_p(x2), T, _p(packed), _p(scale), N, K, _p(y))
    return y.reshape((N,) if np.ndim(x) == 1 else (T, N))


def fp8_gemv(x, w, s) -> np.ndarray:
    x2 = _c(np.atleast_2d(x), np.uint16)
    w, s = _c(w, np.uint8), _c(s, np.uint8)
    T, K = x2.shape
    N = w.shape[0]
    y = np.empty((T, N), dtype=np.uint16)
    lib().mxo_fp8_gemv(_p(x2), T, _p(w), _p(s), N, K, _p(y))
    return y.reshape((N,) if np.ndim(x) == 1 else (T, N))


def grouped_gemv(x, W1p, W3p, W2p, W1s, W3s, W2s, r) -> np.ndarray:
    x = _c(x, np.uint16)
    arrs = [_c(a, np.uint8) for a in (W1p, W3p, W2p, W1s, W3s, W2s)]
    r = _c(r, np.float32)
    n_exp, H, K = arrs[0].shape[0], arrs[0].shape[1], arrs[0].shape[2] * 2
    O = arrs[2].shape[1]
    out = np.empty(O, dtype=np.uint16)
    lib().mxo_grouped_gemv(_p(x), *[_p(a) for a in arrs], _p(r), K, H, O, n_exp, _p(out))
    return out


def rmsnorm_residual(x, r, w, eps: float = 1e-6):
    x2, r2 = _c(np.atleast_2d(x), np.uint16), _c(np.atleast_2d(r), np.uint16)
    w = _c(w, np.uint16)
    rows, H = x2.shape
    y = np.empty_like(x2)
    nr = np.empty_like(x2)
    lib().mxo_rmsnorm_residual(_p(x2), _p(r2), _p(w), rows, H, eps, _p(y), _p(nr))
    return y, nr


def rmsnorm(x, w, eps: float = 1e-6) -> np.ndarray:
    x2 = _c(np.atleast_2d(x), np.uint16)
    w = _c(w, np.uint16)
    rows, H = x2.shape
    y = np.empty_like(x2)
    lib().mxo_rmsnorm(_p(x2), _p(w), rows, H, eps, _p(y))
    return y


def router_logits(x, w_gate) -> np.ndarray:
    x = _c(np.atleast_2d(x), np.uint16)
    w = _c(w_gate, np.uint16)
    T, K = x.shape
    N = w.shape[0]
    out = np.empty((T, N), dtype=np.float32)
    lib().mxo_router_logits(_p(x), T, _p(w), N, K, _p(out))
    return out


def route_sqrt_softplus(logits, topk: int, routed_scale: float = 1.5):
    """Per row: (ids, weights, number of picks that were numbers)."""
    l = _c(np.atleast_2d(logits), np.float32)
    T, n = l.shape
    ids = np.empty((T, topk), dtype=np.int32)
    w = np.empty((T, topk), dtype=np.float32)
    found = np.empty(T, dtype=np.int32)
    for t in range(T):
        row = _c(l[t], np.float32)
        it = np.empty(topk, dtype=np.int32)
        wt = np.empty(topk, dtype=np.float32)
        found[t] = lib().mxo_route_sqrt_softplus(_p(row), n, topk, ctypes.c_float(routed_scale), _p(it), _p(wt))
        ids[t], w[t] = it, wt
    return ids, w, found
