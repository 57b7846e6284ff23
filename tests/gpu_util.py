"""Helpers shared by the GPU tests: numpy bf16 bits <-> device tensors, checks."""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import mx


def announce(msg: str) -> None:
    """Name the case (shape, seed, entry point) before a GPU step, flushed."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev_bf16(bits: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)


def dev_u8(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device)


def dev_f32(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def host_bits(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def assert_close(got_bits, ref_bits, what: str, rel_tol=mx.REL_TOL, cos_tol=mx.COS_TOL):
    """Tolerance of the parity contract: max|got-ref|/max|ref| <= 1e-2 and cosine >= 0.9999."""
    assert got_bits.shape == ref_bits.shape, f"{what}: shape {got_bits.shape} != {ref_bits.shape}"
    g = mx.bf16_to_f32(got_bits)
    assert np.all(np.isfinite(g)), f"{what}: non-finite output"
    rel, cos = mx.compare(got_bits, ref_bits)
    print(f"  {what}: max rel err {rel:.3e}, cosine {cos:.7f}", flush=True)
    assert rel <= rel_tol and cos >= cos_tol, f"{what}: rel {rel:.3e} cos {cos:.7f}"
