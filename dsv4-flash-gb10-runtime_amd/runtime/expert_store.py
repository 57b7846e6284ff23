"""Safetensors checkpoint -> HBM-resident routed experts (libdsv4_expert_store.so).

The reference serves routed experts from a 64-per-layer LRU hot set that a
Python loader fills from memory-mapped shards on demand
(kernel/cpp-engine-mxfp4/hotset.cu:211-520, runtime/mxfp4_loader.py). On one
MI355X all 43 x 256 experts (147 GB) fit in HBM, so a layer is loaded once,
into the expert-major tensors the routed kernels read in place:

    store = ExpertStore("/path/to/snapshot")
    weights = store.load_layer(0, device)          # runtime.moe.MoEWeights
    layer = moe.RoutedMoELayer(weights)

Reading and parsing are native (C++): shard headers are parsed once at open,
tensor bytes are read with pread() and copied to the device through two pinned
buffers, so the next expert's read overlaps the previous copy.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _lib
from .moe import MoEWeights

_LIB: Optional[ctypes.CDLL] = None

_NP_DTYPES = {"I8": np.int8, "U8": np.uint8, "BOOL": np.uint8, "F8_E4M3": np.uint8, "F8_E5M2": np.uint8,
              "F8_E8M0": np.uint8, "I16": np.int16, "U16": np.uint16, "F16": np.float16, "BF16": np.uint16,
              "I32": np.int32, "U32": np.uint32, "F32": np.float32, "I64": np.int64, "U64": np.uint64,
              "F64": np.float64}


def lib_path() -> str:
    return _lib.lib_path("DSV4_EXPERT_STORE_LIB", "expert-store", "libdsv4_expert_store.so")


def _load_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        lib = _lib.load(lib_path())
        P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        lib.dsv4_store_open.argtypes = [ctypes.c_char_p]
        lib.dsv4_store_open.restype = P
        lib.dsv4_store_close.argtypes = [P]
        lib.dsv4_store_close.restype = I
        lib.dsv4_store_count.argtypes = [P]
        lib.dsv4_store_count.restype = I
        lib.dsv4_store_tensor_info.argtypes = [P, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(L),
                                               ctypes.POINTER(I), ctypes.POINTER(L)]
        lib.dsv4_store_tensor_info.restype = I
        lib.dsv4_store_read.argtypes = [P, ctypes.c_char_p, P, L]
        lib.dsv4_store_read.restype = I
        lib.dsv4_store_load_tensor.argtypes = [P, ctypes.c_char_p, P, L, P]
        lib.dsv4_store_load_tensor.restype = I
        lib.dsv4_store_load_experts.argtypes = [P, I, ctypes.c_char_p, I, P, L, P, L, ctypes.POINTER(L),
                                                ctypes.POINTER(L), P]
        lib.dsv4_store_load_experts.restype = I
        _LIB = lib
    return _LIB


class ExpertStore:
    """A safetensors snapshot (index + shards, one model.safetensors, or one file)."""

    def __init__(self, path: str):
        self._lib = _load_lib()
        self._h = self._lib.dsv4_store_open(str(path).encode())
        if not self._h:
            raise RuntimeError(f"dsv4_store_open failed for {path}")

    def close(self) -> None:
        if self._h:
            self._lib.dsv4_store_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return int(self._lib.dsv4_store_count(self._h))

    def info(self, name: str) -> Tuple[str, Tuple[int, ...], int]:
        """(dtype string, shape, byte size) of a tensor; KeyError if absent."""
        dt = ctypes.create_string_buffer(16)
        shape = (ctypes.c_int64 * 8)()
        nd, nb = ctypes.c_int(), ctypes.c_int64()
        rc = self._lib.dsv4_store_tensor_info(self._h, name.encode(), dt, shape, ctypes.byref(nd),
                                              ctypes.byref(nb))
        if rc == -1:
            raise KeyError(name)
        if rc != 0:
            raise RuntimeError(f"dsv4_store_tensor_info returned {rc}")
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value)), nb.value

    def read(self, name: str) -> np.ndarray:
        """The tensor's bytes on the host, as a numpy array of its shape (1-byte
        float formats and BF16 come back as raw unsigned integers)."""
        dtype, shape, nbytes = self.info(name)
        out = np.empty(nbytes, dtype=np.uint8)
        rc = self._lib.dsv4_store_read(self._h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), nbytes)
        if rc != 0:
            raise RuntimeError(f"dsv4_store_read({name}) returned {rc}")
        return out.view(_NP_DTYPES.get(dtype, np.uint8)).reshape(shape)

    def load_tensor(self, name: str, device, dtype: torch.dtype = torch.uint8) -> torch.Tensor:
        """The tensor's bytes in a new device tensor (raw bytes viewed as `dtype`)."""
        _, shape, nbytes = self.info(name)
        out = torch.empty(nbytes, dtype=torch.uint8, device=device)
        rc = self._lib.dsv4_store_load_tensor(self._h, name.encode(), _lib.vp(out), nbytes,
                                              ctypes.c_void_p(_lib.stream_ptr(out.device)))
        if rc != 0:
            raise RuntimeError(f"dsv4_store_load_tensor({name}) returned {rc}")
        return out.view(dtype).view(shape) if dtype != torch.uint8 else out.view(shape)

    def load_experts(self, layer: int, proj: str, n_experts: int, device) -> Dict[str, torch.Tensor]:
        """{"packed": [E, rows, cols/2], "scale": [E, rows, cols/32]} uint8 device
        tensors of layers.{layer}.ffn.experts.{e}.{proj}, e < n_experts."""
        _, wshape, _ = self.info(f"layers.{layer}.ffn.experts.0.{proj}.weight")
        _, sshape, _ = self.info(f"layers.{layer}.ffn.experts.0.{proj}.scale")
        if len(wshape) != 2 or len(sshape) != 2:
            raise RuntimeError(f"layer {layer} {proj}: expected 2-D weight and scale")
        packed = torch.empty((n_experts,) + wshape, dtype=torch.uint8, device=device)
        scale = torch.empty((n_experts,) + sshape, dtype=torch.uint8, device=device)
        rows, cols = ctypes.c_int64(), ctypes.c_int64()
        rc = self._lib.dsv4_store_load_experts(
            self._h, layer, proj.encode(), n_experts, _lib.vp(packed), packed[0].numel(), _lib.vp(scale),
            scale[0].numel(), ctypes.byref(rows), ctypes.byref(cols), ctypes.c_void_p(_lib.stream_ptr(packed.device)))
        if rc != 0:
            raise RuntimeError(f"dsv4_store_load_experts(layer {layer}, {proj}) returned {rc}")
        return {"packed": packed, "scale": scale}

    def load_layer(self, layer: int, device, n_experts: int = 256) -> MoEWeights:
        """One layer's routed experts (w1, w3, w2) as runtime.moe.MoEWeights."""
        return MoEWeights(W1=self.load_experts(layer, "w1", n_experts, device),
                          W3=self.load_experts(layer, "w3", n_experts, device),
                          W2=self.load_experts(layer, "w2", n_experts, device))


__all__ = ["ExpertStore", "lib_path"]
