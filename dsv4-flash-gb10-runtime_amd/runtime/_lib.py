"""Library loading and stream helpers shared by the ctypes bindings."""
from __future__ import annotations

import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNEL_DIR = os.path.join(PKG_ROOT, "kernel")


def lib_path(env_var: str, subdir: str, name: str) -> str:
    """Path of a kernel library: $env_var if set, else kernel/<subdir>/<name>."""
    p = os.environ.get(env_var)
    if p:
        return os.path.abspath(p)
    return os.path.join(KERNEL_DIR, subdir, name)


def load(path: str, build_hint: str = "make -C dsv4-flash-gb10-runtime_amd/csrc") -> ctypes.CDLL:
    if not os.path.exists(path):
        raise FileNotFoundError(f"{os.path.basename(path)} not found at {path}; build with `{build_hint}`")
    return ctypes.CDLL(path)


def stream_ptr(device, stream=None) -> int:
    """hipStream_t of `stream` or of torch's current stream on `device`."""
    import torch

    if stream is not None:
        return int(stream.cuda_stream)
    return int(torch.cuda.current_stream(device).cuda_stream)


def vp(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())
