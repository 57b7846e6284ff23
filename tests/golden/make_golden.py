"""Writes tests/golden/cases.npz: small seeded inputs with the oracle's outputs.

The reference ships no golden vectors, known-answer tests or fixtures for this
path (its kernels' claimed "bit-exact reference" tests are not in the tree), so
these fixtures are regression vectors of this repository's oracle, whose own
correctness is pinned by tests/test_formats.py and tests/test_oracle_math.py.
GPU tests compare the kernels against them, and tests/test_golden.py checks
the oracle still reproduces them. Re-run after an intended oracle change:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.join(REPO, "dsv4-flash-gb10-runtime_amd")]

from oracle import mx  # noqa: E402
from runtime import synth  # noqa: E402


def build() -> dict:
    c = {}
    # dense MXFP4 GEMV
    p, s = synth.mxfp4_weight(101, 48, 256)
    x = synth.normal_bf16(102, (256,))
    c.update(mxfp4_x=x, mxfp4_p=p[0], mxfp4_s=s[0], mxfp4_y=mx.mxfp4_gemv(x, p[0], s[0]),
             mxfp4_deq=mx.mxfp4_dequant_bf16(p[0], s[0]))
    # FP8 GEMV, ragged N, two tokens
    w, ws = synth.fp8_weight(103, 130, 256)
    xf = synth.normal_bf16(104, (2, 256))
    c.update(fp8_x=xf, fp8_w=w, fp8_s=ws, fp8_y=mx.fp8_gemv(xf, w, ws),
             fp8_deq=mx.fp8_dequant_bf16(w, ws))
    # grouped (drop-in shape) and expert-indexed MoE
    K, H, O, n = 128, 64, 96, 3
    W1p, W1s = synth.mxfp4_weight(105, H, K, n)
    W3p, W3s = synth.mxfp4_weight(109, H, K, n)
    W2p, W2s = synth.mxfp4_weight(113, O, H, n)
    xg = synth.normal_bf16(117, (K,))
    r = np.array([0.5, 0.3, 0.2], np.float32)
    c.update(g_x=xg, g_W1p=W1p, g_W1s=W1s, g_W3p=W3p, g_W3s=W3s, g_W2p=W2p, g_W2s=W2s, g_r=r,
             g_out=mx.grouped_gemv_topk(xg, W1p, W3p, W2p, W1s, W3s, W2s, r))
    E, T, topk = 16, 4, 4
    M1p, M1s = synth.mxfp4_weight(120, H, K, E)
    M3p, M3s = synth.mxfp4_weight(124, H, K, E)
    M2p, M2s = synth.mxfp4_weight(128, O, H, E)
    xm = synth.normal_bf16(132, (T, K))
    logits = synth.gating_logits(133, T, E)
    ids, wts = mx.route_sigmoid_topk(logits, topk)
    out = mx.moe_layer(xm, lambda e: ((M1p[e], M1s[e]), (M3p[e], M3s[e]), (M2p[e], M2s[e])),
                       ids, wts, O)
    c.update(m_x=xm, m_W1p=M1p, m_W1s=M1s, m_W3p=M3p, m_W3s=M3s, m_W2p=M2p, m_W2s=M2s,
             m_logits=logits, m_ids=ids, m_w=wts, m_out=out)
    # RMSNorm
    h = synth.normal_bf16(134, (3, 256))
    rr = synth.normal_bf16(135, (3, 256), 0.0, 0.5)
    g = synth.normal_bf16(136, (256,), 1.0, 0.1)
    y, nr = mx.rmsnorm_residual(h, rr, g)
    c.update(r_h=h, r_r=rr, r_g=g, r_y=y, r_newres=nr, r_fwd=mx.rmsnorm(h, g))
    return c


if __name__ == "__main__":
    path = os.path.join(HERE, "cases.npz")
    np.savez_compressed(path, **build())
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")
