"""Device-side seeded filling of large synthetic weight tensors (libdsv4_fill.so).

``fill_uniform_u8(t, seed, offset, lo, hi)`` writes the same bytes as
``synth.uniform_u8(seed, offset, t.numel(), lo, hi)`` directly into a GPU
uint8 tensor, so 100+ GB of resident experts need no host generation or
host-to-device copy.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

_LIB: Optional[ctypes.CDLL] = None


def _load_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        lib = _lib.load(_lib.lib_path("DSV4_FILL_LIB", "fill", "libdsv4_fill.so"))
        lib.dsv4_fill_uniform_u8.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64,
                                             ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_void_p]
        lib.dsv4_fill_uniform_u8.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def fill_uniform_u8(t: torch.Tensor, seed: int, offset: int = 0, lo: int = 0, hi: int = 255) -> torch.Tensor:
    if not t.is_cuda or t.dtype != torch.uint8 or not t.is_contiguous():
        raise ValueError("fill_uniform_u8 needs a contiguous GPU uint8 tensor")
    rc = _load_lib().dsv4_fill_uniform_u8(_lib.vp(t), t.numel(), seed & 0xFFFFFFFFFFFFFFFF,
                                          offset, lo, hi, ctypes.c_void_p(_lib.stream_ptr(t.device)))
    if rc != 0:
        raise RuntimeError(f"dsv4_fill_uniform_u8 returned {rc}")
    return t
