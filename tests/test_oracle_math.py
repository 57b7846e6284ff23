"""CPU pins of the oracle's GEMV / MoE / RMSNorm / routing math.

The oracle (oracle/mx.py) is checked against: brute-force fp64 loops written
from the definitions, the independent scalar C oracle, closed forms (one-hot
activations select a dequantised column; a scale byte +1 doubles a block's
contribution exactly), structural invariants (linearity, expert permutation,
zero routing weights, single-expert reduction to dense GEMVs) and torch's
topk / sigmoid.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import c_oracle as co
from oracle import mx
from runtime import synth


def _brute_mxfp4_gemv(x_bits, packed, scale):
    """y[n] = sum_k code * 2^(s-127) * x, straight from the packing rule, fp64."""
    N, K = packed.shape[0], packed.shape[1] * 2
    xf = mx.bf16_to_f32(x_bits).astype(np.float64)
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    y = np.zeros(N)
    for n in range(N):
        for k in range(K):
            byte = int(packed[n, k // 2])
            code = (byte >> 4) if k % 2 else (byte & 15)
            v = table[code & 7] * (-1.0 if code & 8 else 1.0)
            y[n] += v * 2.0 ** (int(scale[n, k // 32]) - 127) * xf[k]
    return y


def test_mxfp4_gemv_brute_force_tiny():
    p, s = synth.mxfp4_weight(21, 6, 64)
    x = synth.normal_bf16(22, (64,))
    got = mx.bf16_to_f32(mx.mxfp4_gemv(x, p[0], s[0])).astype(np.float64)
    ref = _brute_mxfp4_gemv(x, p[0], s[0])
    assert np.allclose(got, ref, rtol=1e-2, atol=1e-3 * np.abs(ref).max())
    assert np.array_equal(co.mxfp4_gemv(x, p[0], s[0]), mx.mxfp4_gemv(x, p[0], s[0])) or \
        mx.compare(co.mxfp4_gemv(x, p[0], s[0]), mx.mxfp4_gemv(x, p[0], s[0]))[1] > 0.99999


def test_one_hot_activation_selects_dequant_column():
    p, s = synth.mxfp4_weight(23, 16, 128)
    deq = mx.mxfp4_dequant_bf16(p[0], s[0])
    for k in (0, 1, 31, 32, 127):
        x = np.zeros(128, np.uint16)
        x[k] = 0x3F80  # 1.0
        col = mx.bf16_to_f32(deq[:, k])  # compared as values: a sum gives +0 for a -0 weight
        assert np.array_equal(mx.bf16_to_f32(mx.mxfp4_gemv(x, p[0], s[0])), col)
        assert np.array_equal(mx.bf16_to_f32(co.mxfp4_gemv(x, p[0], s[0])), col)


def test_scale_plus_one_doubles_block_exactly():
    p, s = synth.mxfp4_weight(24, 8, 64)
    p, s = p[0], s[0].copy()
    x = synth.normal_bf16(25, (64,))
    x[32:] = 0  # only block 0 contributes
    y0 = mx.bf16_to_f32(mx.mxfp4_gemv(x, p, s))
    s[:, 0] += 1
    y1 = mx.bf16_to_f32(mx.mxfp4_gemv(x, p, s))
    assert np.array_equal(y1, 2 * y0)


def test_gemv_linear_in_x():
    p, s = synth.mxfp4_weight(26, 32, 256)
    x = synth.normal_bf16(27, (256,))
    x2 = mx.bf16_round(2 * mx.bf16_to_f32(x))  # exact doubling
    assert np.array_equal(mx.bf16_to_f32(mx.mxfp4_gemv(x2, p[0], s[0])),
                          2 * mx.bf16_to_f32(mx.mxfp4_gemv(x, p[0], s[0])))


def test_fp8_gemv_brute_force_and_c_oracle():
    w, s = synth.fp8_weight(28, 130, 256)  # N not a multiple of 128: ceil(N/128) scale rows
    x = synth.normal_bf16(29, (2, 256))
    y = mx.fp8_gemv(x, w, s)
    vals = mx.e4m3fn_decode(w).astype(np.float64)
    sc = np.array([[2.0 ** (int(s[n // 128, k // 128]) - 127) for k in range(256)] for n in range(130)])
    ref = mx.bf16_to_f32(x).astype(np.float64) @ (vals * sc).T
    rel, cos = mx.compare(y, mx.bf16_round(ref.astype(np.float32)))
    assert rel < 1e-2 and cos > 0.99999
    rel, cos = mx.compare(co.fp8_gemv(x, w, s), y)
    assert rel < 1e-2 and cos > 0.99999


def test_fp8_gemv_grouped_slices_and_scale_rows():
    # 128-row groups: each group is an independent GEMV on its own slice
    w, s = synth.fp8_weight(60, 3 * 128, 256)
    x = synth.normal_bf16(61, (3, 256))
    y = mx.fp8_gemv_grouped(x, w, s, 3)
    for g in range(3):
        ref = mx.fp8_gemv(x[g], w[128 * g:128 * (g + 1)], s[g:g + 1])
        assert np.array_equal(y[g], ref)
    # 64-row groups share scale rows: the scale row follows the global row
    w, s = synth.fp8_weight(62, 4 * 64, 256)
    x = synth.normal_bf16(63, (2, 4, 256))
    y = mx.fp8_gemv_grouped(x, w, s, 4)
    vals = mx.e4m3fn_decode(w).astype(np.float64)
    sc = np.array([[2.0 ** (int(s[n // 128, k // 128]) - 127) for k in range(256)] for n in range(256)])
    Wf = vals * sc
    for t in range(2):
        for g in range(4):
            ref = mx.bf16_to_f32(x[t, g]).astype(np.float64) @ Wf[64 * g:64 * (g + 1)].T
            rel, cos = mx.compare(y[t, g], mx.bf16_round(ref.astype(np.float32)))
            assert rel < 1e-2 and cos > 0.99999
    # one group is the plain GEMV
    assert np.array_equal(mx.fp8_gemv_grouped(x[:, :1], w[:64], s[:1], 1)[:, 0], mx.fp8_gemv(x[:, 0], w[:64], s[:1]))


def test_swiglu_clamped_closed_forms():
    def b(v):
        return mx.bf16_round(np.asarray(v, np.float32))

    def val(bits):
        return float(np.asarray(mx.bf16_to_f32(bits)).reshape(-1)[0])

    def silu(v):
        return v / (1.0 + np.exp(-v))

    # gate 0 gives 0; no clamp inside the limit
    assert val(mx.swiglu_clamped(b(0.0), b(3.0), 10.0, True)) == 0.0
    assert np.isclose(val(mx.swiglu_clamped(b(2.0), b(3.0), 10.0, True)), silu(2.0) * 3.0, rtol=4e-3)
    # the gate is clamped to +-limit
    assert np.isclose(val(mx.swiglu_clamped(b(100.0), b(1.0), 10.0, False)), silu(10.0), rtol=4e-3)
    assert np.isclose(val(mx.swiglu_clamped(b(-100.0), b(1.0), 10.0, False)), silu(-10.0), rtol=4e-3)
    # up is clamped only with clamp_up
    assert np.isclose(val(mx.swiglu_clamped(b(1.0), b(-50.0), 10.0, True)), silu(1.0) * -10.0, rtol=4e-3)
    assert np.isclose(val(mx.swiglu_clamped(b(1.0), b(-50.0), 10.0, False)), silu(1.0) * -50.0, rtol=4e-3)
    # limit <= 0: no clamp at all
    assert np.isclose(val(mx.swiglu_clamped(b(100.0), b(-50.0), 0.0, True)), 100.0 * -50.0, rtol=4e-3)
    # a random batch against fp64 with one final rounding
    rng = np.random.default_rng(64)
    g = b(rng.normal(0, 8, 4096))
    u = b(rng.normal(0, 8, 4096))
    gf = np.clip(mx.bf16_to_f32(g).astype(np.float64), -10, 10)
    uf = np.clip(mx.bf16_to_f32(u).astype(np.float64), -10, 10)
    rel, cos = mx.compare(mx.swiglu_clamped(g, u, 10.0, True), mx.bf16_round((silu(gf) * uf).astype(np.float32)))
    assert rel < 1e-2 and cos > 0.99999


def test_fp8_swiglu_brute_force():
    w1, s1 = synth.fp8_weight(65, 130, 256)
    w3, s3 = synth.fp8_weight(66, 130, 256)
    x = mx.bf16_round(24 * mx.bf16_to_f32(synth.normal_bf16(67, (2, 256))))  # some gates past the limit
    act = mx.fp8_swiglu(x, w1, s1, w3, s3, 10.0, False)

    def dense(w, s):
        vals = mx.e4m3fn_decode(w).astype(np.float64)
        sc = np.array([[2.0 ** (int(s[n // 128, k // 128]) - 127) for k in range(256)] for n in range(130)])
        return vals * sc

    xf = mx.bf16_to_f32(x).astype(np.float64)
    g = np.clip(xf @ dense(w1, s1).T, -10, 10)
    u = xf @ dense(w3, s3).T
    assert np.abs(xf @ dense(w1, s1).T).max() > 10  # the clamp is exercised
    ref = mx.bf16_round((g / (1 + np.exp(-g)) * u).astype(np.float32))
    rel, cos = mx.compare(act, ref)
    assert rel < 2e-2 and cos > 0.9999


def _experts(seed, n, K, H, O):
    W1p, W1s = synth.mxfp4_weight(seed, H, K, n)
    W3p, W3s = synth.mxfp4_weight(seed + 4, H, K, n)
    W2p, W2s = synth.mxfp4_weight(seed + 8, O, H, n)
    return W1p, W3p, W2p, W1s, W3s, W2s


def test_grouped_matches_c_oracle_and_brute_force():
    K, H, O, n = 128, 64, 96, 3
    W1p, W3p, W2p, W1s, W3s, W2s = _experts(30, n, K, H, O)
    x = synth.normal_bf16(31, (K,))
    r = np.array([0.5, 0.3, 0.2], np.float32)
    got = mx.grouped_gemv_topk(x, W1p, W3p, W2p, W1s, W3s, W2s, r)
    rel, cos = mx.compare(co.grouped_gemv(x, W1p, W3p, W2p, W1s, W3s, W2s, r), got)
    assert rel < 1e-2 and cos > 0.9999
    # brute force from the definition (fp64, M rounded to bf16 like the reference)
    acc = np.zeros(O)
    for e in range(n):
        g = _brute_mxfp4_gemv(x, W1p[e], W1s[e])
        u = _brute_mxfp4_gemv(x, W3p[e], W3s[e])
        m = mx.bf16_round((g / (1 + np.exp(-g)) * u).astype(np.float32))
        acc += r[e] * _brute_mxfp4_gemv(m, W2p[e], W2s[e])
    rel, cos = mx.compare(got, mx.bf16_round(acc.astype(np.float32)))
    assert rel < 1e-2 and cos > 0.9999


def test_grouped_invariants():
    K, H, O, n = 128, 64, 64, 4
    W1p, W3p, W2p, W1s, W3s, W2s = _experts(32, n, K, H, O)
    x = synth.normal_bf16(33, (K,))
    r = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    base = mx.grouped_gemv_topk(x, W1p, W3p, W2p, W1s, W3s, W2s, r)
    perm = np.array([2, 0, 3, 1])
    permuted = mx.grouped_gemv_topk(x, W1p[perm], W3p[perm], W2p[perm], W1s[perm], W3s[perm],
                                    W2s[perm], r[perm])
    rel, cos = mx.compare(permuted, base)
    assert rel < 1e-3 and cos > 0.99999
    zero = mx.grouped_gemv_topk(x, W1p, W3p, W2p, W1s, W3s, W2s, np.zeros(n, np.float32))
    assert np.all(mx.bf16_to_f32(zero) == 0)
    # one expert with weight 1 == W2 . bf16(silu(W1 x) * W3 x) from dense GEMVs
    one = mx.grouped_gemv_topk(x, W1p[:1], W3p[:1], W2p[:1], W1s[:1], W3s[:1], W2s[:1],
                               np.ones(1, np.float32))
    g = mx.bf16_to_f32(mx.mxfp4_gemv(x, W1p[0], W1s[0]))
    u = mx.bf16_to_f32(mx.mxfp4_gemv(x, W3p[0], W3s[0]))
    m = mx.bf16_round(mx.silu_f32(g) * u)
    rel, cos = mx.compare(one, mx.mxfp4_gemv(m, W2p[0], W2s[0]))
    assert rel < 2e-2 and cos > 0.9999


def test_moe_layer_equals_per_token_grouped():
    K, H, O, E, T, topk = 128, 64, 64, 12, 3, 4
    W1p, W3p, W2p, W1s, W3s, W2s = _experts(34, E, K, H, O)
    x = synth.normal_bf16(35, (T, K))
    logits = synth.gating_logits(36, T, E)
    ids, w = mx.route_sigmoid_topk(logits, topk)

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    out = mx.moe_layer(x, fn, ids, w, O)
    for t in range(T):
        i = ids[t]
        ref = mx.grouped_gemv_topk(x[t], W1p[i], W3p[i], W2p[i], W1s[i], W3s[i], W2s[i], w[t])
        rel, cos = mx.compare(out[t], ref)
        assert rel < 1e-3 and cos > 0.99999


def test_moe_layer_dequantised_is_bit_identical():
    K, H, O, E, T, topk = 128, 64, 64, 12, 3, 4
    W1p, W3p, W2p, W1s, W3s, W2s = _experts(39, E, K, H, O)
    x = synth.normal_bf16(40, (T, K))
    ids, w = mx.route_sigmoid_topk(synth.gating_logits(41, T, E), topk)

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    out = mx.moe_layer(x, fn, ids, w, O)
    pre = {e: mx.dequant_expert_f32(fn(e)) for e in range(E)}
    assert np.array_equal(mx.moe_layer_dequantised(x, pre.__getitem__, ids, w, O), out)
    # the dequantised W1 of expert 0 against the dense GEMV oracle
    y = mx.bf16_round(mx.bf16_to_f32(x) @ pre[0][0].T)
    assert np.array_equal(y, mx.mxfp4_gemv(x, W1p[0], W1s[0]))


def test_route_matches_torch():
    logits = synth.gating_logits(37, 16, 256)
    ids, w = mx.route_sigmoid_topk(logits, 8)
    tl = torch.from_numpy(logits)
    tv, ti = torch.topk(tl, 8, dim=-1)
    assert np.array_equal(ids, ti.numpy().astype(np.int32))
    tw = torch.sigmoid(tv.double())
    tw = (tw / tw.sum(-1, keepdim=True)).float().numpy()
    assert np.allclose(w, tw, rtol=1e-6, atol=1e-7)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)
    # ties go to the lower index
    tie = np.zeros((1, 16), np.float32)
    assert mx.route_sigmoid_topk(tie, 3)[0].tolist() == [[0, 1, 2]]


def test_rmsnorm_closed_forms_and_c_oracle():
    H = 256
    c = 0.75
    x = np.full((2, H), mx.bf16_round(np.float32(c)), np.uint16)
    g = synth.normal_bf16(38, (H,), 1.0, 0.1)
    y = mx.rmsnorm(x, g)
    ref = mx.bf16_round((mx.bf16_to_f32(g).astype(np.float64) * c / np.sqrt(c * c + 1e-6)).astype(np.float32))
    assert np.array_equal(y[0], ref)
    h = synth.normal_bf16(39, (4, H))
    r = synth.normal_bf16(40, (4, H), 0.0, 0.5)
    y2, nr = mx.rmsnorm_residual(h, r, g)
    tnr = (torch.from_numpy(mx.bf16_to_f32(h)) + torch.from_numpy(mx.bf16_to_f32(r))).to(torch.bfloat16)
    assert np.array_equal(nr, tnr.view(torch.uint16).numpy())
    cy, cnr = co.rmsnorm_residual(h, r, g)
    assert np.array_equal(cnr, nr)
    rel, cos = mx.compare(cy, y2)
    assert rel < 1e-2 and cos > 0.99999
    # torch formulation of the reference (runtime/dsv4_engine_mxfp4.py:136-141)
    f = tnr.float()
    ty = (f * torch.rsqrt((f * f).mean(-1, keepdim=True) + 1e-6) *
          torch.from_numpy(mx.bf16_to_f32(g))).to(torch.bfloat16).view(torch.uint16).numpy()
    rel, cos = mx.compare(y2, ty)
    assert rel < 1e-2 and cos > 0.9999


def test_mutation_transposed_weight_is_caught():
    """A transposed operand in the GEMV would break the one-hot column pin."""
    p, s = synth.mxfp4_weight(41, 64, 64)
    deq = mx.mxfp4_dequant_bf16(p[0], s[0])
    x = np.zeros(64, np.uint16)
    x[5] = 0x3F80
    wrong = mx.bf16_to_f32(x) @ mx.bf16_to_f32(deq)  # W^T x: row 5, not column 5
    right = mx.bf16_to_f32(x) @ mx.bf16_to_f32(deq).T
    assert np.array_equal(right, mx.bf16_to_f32(deq[:, 5]))
    assert not np.array_equal(wrong, mx.bf16_to_f32(deq[:, 5]))
