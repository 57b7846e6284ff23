"""Device-side seeded filling of large synthetic weight tensors (libdsv4_fill.so).

``fill_uniform_u8(t, seed, offset, lo, hi)`` writes the same bytes as
``synth.uniform_u8(seed, offset, t.numel(), lo, hi)`` directly into a GPU
uint8 tensor, so 100+ GB of resident experts need no host generation or
host-to-device copy. ``read_floor`` streams a byte range once with a
read-only kernel: the benchmark's measure of the HBM read floor.
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
        lib.dsv4_read_floor.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        lib.dsv4_read_floor.restype = ctypes.c_int
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


def read_floor(src: torch.Tensor, nbytes: int, workgroups: int, sink: torch.Tensor,
               rotate: int = 1, launches: int = 1, threads: int = 512) -> None:
    """`launches` back-to-back launches of the read-only kernel, launch i
    streaming the `nbytes` at byte (i % rotate) * nbytes of the GPU tensor
    `src` once with `workgroups` workgroups of `threads` (256 or 512) threads
    (the HBM read floor for that many bytes); sink is an int32 GPU tensor of
    at least workgroups * threads elements."""
    if not src.is_cuda or not src.is_contiguous() or rotate * nbytes > src.numel() * src.element_size():
        raise ValueError("read_floor needs a contiguous GPU tensor holding rotate * nbytes bytes")
    if not sink.is_cuda or sink.dtype != torch.int32 or sink.numel() < workgroups * threads:
        raise ValueError("read_floor needs an int32 GPU sink of workgroups * threads elements")
    rc = _load_lib().dsv4_read_floor(_lib.vp(src), nbytes, rotate, launches, workgroups, threads, _lib.vp(sink),
                                     ctypes.c_void_p(_lib.stream_ptr(src.device)))
    if rc != 0:
        raise RuntimeError(f"dsv4_read_floor returned {rc}")
