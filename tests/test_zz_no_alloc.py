"""GPU test of mxfp4_moe_grouped_gemv_noalloc, called through the C ABI: the
no-allocation variant of mxfp4_moe_grouped_gemv (its routing tables and
SwiGLU intermediate live in the library's device array instead of a
workspace). Two calls in a row, the second with fewer tokens, must each give
the bits of the workspace entry on the same inputs."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from runtime import _lib, moe, synth
from runtime import mxfp4_grouped_gemv_binding as gb
from tests.gpu_util import announce, dev_bf16, dev_f32, host_bits

pytestmark = pytest.mark.gpu


def _noalloc(x, w, ids, wt, out):
    lib = gb._load_lib()
    T, K = x.shape
    topk = ids.shape[1]
    rc = lib.mxfp4_moe_grouped_gemv_noalloc(
        _lib.vp(x), _lib.vp(w.W1["packed"]), _lib.vp(w.W3["packed"]), _lib.vp(w.W2["packed"]),
        _lib.vp(w.W1["scale"]), _lib.vp(w.W3["scale"]), _lib.vp(w.W2["scale"]), _lib.vp(ids), _lib.vp(wt),
        T, topk, w.n_experts, K, w.hidden, w.out_dim, _lib.vp(out),
        ctypes.c_void_p(_lib.stream_ptr(x.device)))
    return rc


def test_noalloc_matches_workspace_entry_two_calls(device):
    E, K, H, O, topk = 32, 4096, 2048, 4096, 8
    w = moe.make_moe_weights(14000, E, K, H, O, device)
    for step, T in enumerate((4, 1)):
        announce(f"mxfp4_moe_grouped_gemv_noalloc call {step + 1}: T={T} E={E} K={K} H={H} O={O}")
        x = dev_bf16(synth.normal_bf16(14100 + T, (T, K)), device)
        ids, wt = synth.zipf_routing(14200 + T, T, E, topk, 1.1)
        idd, wd = torch.from_numpy(ids).to(device), dev_f32(wt, device)
        out = torch.empty(T, O, dtype=torch.bfloat16, device=device)
        assert _noalloc(x, w, idd, wd, out) == 0
        got = host_bits(out)
        ref = host_bits(gb.mxfp4_moe_grouped_gemv(x, w.W1, w.W3, w.W2, idd, wd))
        assert np.array_equal(got, ref), f"call {step + 1} (T={T}) differs from the workspace entry"
        assert np.all(np.isfinite(synth.bf16_bits_to_f32(got)))
    # too large for the device array: rejected before any launch
    x = dev_bf16(synth.normal_bf16(14300, (64, K)), device)
    ids = torch.zeros(64, 16, dtype=torch.int32, device=device)
    wt = torch.zeros(64, 16, dtype=torch.float32, device=device)
    out = torch.empty(64, O, dtype=torch.bfloat16, device=device)
    assert _noalloc(x, w, ids, wt, out) == -8
    del w
    torch.cuda.empty_cache()


def test_noalloc_captured_in_a_graph_replays_match_eager(device):
    """The entry's use under HIP graph capture: after one eager call on the
    device (which looks up the array's address), a captured call replays to
    the eager bits, with eager calls of both entries on other inputs between
    the replays (they share the array; one stream orders them)."""
    E, K, H, O, topk, T = 32, 4096, 2048, 4096, 8, 1
    w = moe.make_moe_weights(14400, E, K, H, O, device)
    announce(f"mxfp4_moe_grouped_gemv_noalloc under graph capture: T={T} E={E} K={K}")
    x = dev_bf16(synth.normal_bf16(14500, (T, K)), device)
    ids, wt = synth.zipf_routing(14600, 2, E, topk, 1.1)
    idd, wd = torch.from_numpy(ids).to(device), dev_f32(wt, device)
    out = torch.empty(T, O, dtype=torch.bfloat16, device=device)
    assert _noalloc(x, w, idd[:1], wd[:1], out) == 0
    eager = host_bits(out).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert _noalloc(x, w, idd[:1], wd[:1], out) == 0
    x2 = dev_bf16(synth.normal_bf16(14501, (4, K)), device)
    ids2, wt2 = synth.zipf_routing(14601, 4, E, topk, 1.1)
    id2, wd2 = torch.from_numpy(ids2).to(device), dev_f32(wt2, device)
    out2 = torch.empty(4, O, dtype=torch.bfloat16, device=device)
    for rep in range(3):
        out.zero_()
        g.replay()
        assert np.array_equal(host_bits(out), eager), f"replay {rep} differs from the eager call"
        assert _noalloc(x2, w, id2, wd2, out2) == 0
        gb.mxfp4_moe_grouped_gemv(x, w.W1, w.W3, w.W2, idd[1:], wd[1:])
        torch.cuda.synchronize()
    assert np.array_equal(host_bits(out2), host_bits(gb.mxfp4_moe_grouped_gemv(x2, w.W1, w.W3, w.W2, id2, wd2)))
    del g, w
    torch.cuda.empty_cache()
