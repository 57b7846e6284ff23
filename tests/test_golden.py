"""Committed fixtures (tests/golden/cases.npz): the oracle must still reproduce
them bit for bit (CPU), and the HIP kernels must match them within the parity
tolerance (GPU; dequantised weights and residual sums bit-exact)."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import mx

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def cases():
    with np.load(os.path.join(HERE, "golden", "cases.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_fixtures(cases):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    fresh = mg.build()
    assert sorted(fresh) == sorted(cases)
    for k in cases:
        assert np.array_equal(fresh[k], cases[k]), k


@pytest.mark.gpu
def test_kernels_match_fixtures(cases, device):
    from runtime import fp8_e4m3_gemv_binding as fp8b
    from runtime import mxfp4_gemv_binding as mxb
    from runtime import mxfp4_grouped_gemv_binding as gb
    from runtime import rmsnorm_fuse_binding as rb
    from tests.gpu_util import announce, assert_close, dev_bf16, dev_f32, dev_u8, host_bits

    c = cases
    d = device
    announce("golden: mxfp4 dequant + gemv")
    assert np.array_equal(host_bits(mxb.mxfp4_dequant(dev_u8(c["mxfp4_p"], d), dev_u8(c["mxfp4_s"], d))),
                          c["mxfp4_deq"])
    y = mxb.mxfp4_gemv(dev_u8(c["mxfp4_p"], d), dev_u8(c["mxfp4_s"], d), dev_bf16(c["mxfp4_x"], d))
    assert_close(host_bits(y), c["mxfp4_y"], "golden mxfp4")
    announce("golden: fp8 dequant + gemv")
    assert np.array_equal(host_bits(fp8b.fp8_e4m3_dequant(dev_u8(c["fp8_w"], d), dev_u8(c["fp8_s"], d))),
                          c["fp8_deq"])
    y = fp8b.fp8_e4m3_gemv(dev_u8(c["fp8_w"], d), dev_u8(c["fp8_s"], d), dev_bf16(c["fp8_x"], d))
    assert_close(host_bits(y), c["fp8_y"], "golden fp8")
    announce("golden: grouped gemv")
    W = [{"packed": dev_u8(c[f"g_{m}p"], d), "scale": dev_u8(c[f"g_{m}s"], d)} for m in ("W1", "W3", "W2")]
    out = gb.mxfp4_grouped_gemv(W[0], W[1], W[2], None, dev_bf16(c["g_x"], d), dev_f32(c["g_r"], d))
    assert_close(host_bits(out), c["g_out"], "golden grouped")
    announce("golden: routing + expert-indexed moe")
    ids, w = gb.route_sigmoid_topk(dev_f32(c["m_logits"], d), c["m_ids"].shape[1])
    assert np.array_equal(ids.cpu().numpy(), c["m_ids"])
    assert np.allclose(w.cpu().numpy(), c["m_w"], rtol=1e-5, atol=1e-6)
    M = [{"packed": dev_u8(c[f"m_{m}p"], d), "scale": dev_u8(c[f"m_{m}s"], d)} for m in ("W1", "W3", "W2")]
    out = gb.mxfp4_moe_grouped_gemv(dev_bf16(c["m_x"], d), M[0], M[1], M[2],
                                    torch.from_numpy(c["m_ids"]).to(d), dev_f32(c["m_w"], d))
    assert_close(host_bits(out), c["m_out"], "golden moe")
    announce("golden: rmsnorm")
    yn, nr = rb.rmsnorm_fuse_residual_add(dev_bf16(c["r_h"], d), dev_bf16(c["r_r"], d), dev_bf16(c["r_g"], d))
    assert np.array_equal(host_bits(nr), c["r_newres"])
    assert_close(host_bits(yn), c["r_y"], "golden rmsnorm residual")
    assert_close(host_bits(rb.rmsnorm_fuse_fwd(dev_bf16(c["r_h"], d), dev_bf16(c["r_g"], d))), c["r_fwd"],
                 "golden rmsnorm fwd")
