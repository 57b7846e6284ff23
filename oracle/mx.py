"""numpy restatement of the reference's CPU math for the decode hot path.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Every function names the
reference file:line it restates and how it is pinned (checked against
something independent of this file). bf16 values travel as uint16 bit
patterns; float32 is the working precision of the reference path
("dequant -> bf16 -> fp32 matmul -> bf16").
"""
from __future__ import annotations

import numpy as np

# ------------------------------------------------------------------ bf16 ----


def bf16_round(a) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (torch's .to(torch.bfloat16)).

    Pinned: tests compare with torch.Tensor.to(torch.bfloat16) on random, tie,
    subnormal, inf and NaN inputs."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    is_nan = (u & 0x7FFFFFFF) > 0x7F800000
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) & 0xFFFF
    r = np.where(is_nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------- number formats --


def e2m1_value(code) -> np.ndarray:
    """e2m1 code (0..15) -> value: sign bit 3, exponent bits 2..1, mantissa bit 0;
    exponent 0 is subnormal (m * 0.5), otherwise 2^(e-1) * (1 + m/2).
    Restates the codebook of runtime/mxfp4_unpack.py:36-39 (OCP MX v1.0).

    Pinned: tests compare all 16 codes with the OCP MX v1.0 FP4 table and with
    torch.float4_e2m1fn_x2 where that dtype converts."""
    c = np.asarray(code, dtype=np.int64)
    s = (c >> 3) & 1
    e = (c >> 1) & 3
    m = c & 1
    mag = np.where(e == 0, 0.5 * m, np.ldexp(1.0 + 0.5 * m, (e - 1).astype(np.int32)))
    return np.where(s == 1, -mag, mag).astype(np.float32)


E2M1_TABLE = e2m1_value(np.arange(16))


def e8m0_decode(b, kernel_convention: bool = True) -> np.ndarray:
    """E8M0 byte -> fp32 scale 2^(b-127) (runtime/e8m0_decode.py:32-64).
    Byte 0xFF is NaN in the Python reference and 0.0 in the reference kernels
    (kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:74-78,
    kernel/mxfp4-dense/mxfp4_gemv.cu:65-69); `kernel_convention` picks which.
    Byte 0 gives the fp32 subnormal 2^-127.

    Pinned: tests compare all 256 bytes with torch.float8_e8m0fnu and math.ldexp."""
    b = np.asarray(b, dtype=np.uint8)
    e = b.astype(np.int32) - 127
    v = np.ldexp(np.float64(1.0), np.where(b == 0xFF, 0, e)).astype(np.float32)
    return np.where(b == 0xFF, np.float32(0.0 if kernel_convention else np.nan), v)


def e4m3fn_decode(b) -> np.ndarray:
    """E4M3FN byte -> fp32: sign.eeee.mmm, bias 7, exponent 0 subnormal
    (m * 2^-9), 0x7F / 0xFF NaN, no infinities (torch.float8_e4m3fn, as used by
    runtime/dsv4_engine_mxfp4.py:539-540).

    Pinned: tests compare all 256 bytes with torch.float8_e4m3fn."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = (b >> 7) & 1
    e = (b >> 3) & 15
    m = b & 7
    mag = np.where(e == 0, np.ldexp(m.astype(np.float64), -9),
                   np.ldexp(1.0 + m / 8.0, (e - 7).astype(np.int32)))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(s == 1, -mag, mag).astype(np.float32)


# ------------------------------------------------------------- MXFP4 pack ---


def mxfp4_unpack(packed, shape, dtype=np.float32) -> np.ndarray:
    """Flat packed bytes -> codebook values in `shape`; low nibble = element 2i,
    high nibble = element 2i+1 (runtime/mxfp4_unpack.py:93-118).

    Pinned: known-answer bytes written from the packing rule and an exhaustive
    pack/unpack round trip in the tests."""
    flat = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8)).reshape(-1)
    if flat.size * 2 != int(np.prod(shape)):
        raise ValueError(f"{flat.size} bytes -> {flat.size * 2} nibbles != prod{tuple(shape)}")
    codes = np.empty(flat.size * 2, dtype=np.uint8)
    codes[0::2] = flat & 0x0F
    codes[1::2] = flat >> 4
    return E2M1_TABLE[codes].astype(dtype).reshape(shape)


def mxfp4_pack(values) -> np.ndarray:
    """Inverse of mxfp4_unpack for values exactly in the codebook; -0.0 packs to
    code 8 and +0.0 to code 0 (runtime/mxfp4_unpack.py:121-168)."""
    v = np.asarray(values, dtype=np.float64).reshape(-1)
    if v.size % 2:
        raise ValueError("element count must be even")
    mag = np.abs(v)
    mags = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    idx = np.searchsorted(mags, mag)
    idx = idx.clip(0, 7)
    if not np.all(mags[idx] == mag):
        bad = np.nonzero(mags[idx] != mag)[0][0]
        raise ValueError(f"value {v[bad]} at index {bad} not in the e2m1 codebook")
    codes = (idx | (np.signbit(v).astype(np.int64) << 3)).astype(np.uint8)
    return ((codes[1::2] << 4) | codes[0::2]).astype(np.uint8)


def mxfp4_dequant_bf16(packed, scale, kernel_convention: bool = True) -> np.ndarray:
    """[N, K/2] packed + [N, K/32] E8M0 -> [N, K] bf16 bits:
    bf16(code_f32 * 2^(s-127)) per 32-element block
    (runtime/mxfp4_loader.py:272-309: unpack fp32, view [N, K/32, 32] times the
    decoded scale, .to(bfloat16)). Every product is exact in fp32, so the only
    rounding is the final bf16 cast.

    Pinned: tests compare with products of torch.float8_e8m0fnu scales and the
    OCP code table converted by torch, and against the scalar C oracle."""
    packed = np.asarray(packed, dtype=np.uint8)
    scale = np.asarray(scale, dtype=np.uint8)
    N, kh = packed.shape
    K = kh * 2
    if scale.shape != (N, K // 32):
        raise ValueError(f"scale shape {scale.shape} != {(N, K // 32)}")
    vals = mxfp4_unpack(packed, (N, K // 32, 32))
    s = e8m0_decode(scale, kernel_convention)[:, :, None]
    with np.errstate(over="ignore"):  # code 6 x 2^127 overflows to inf, as in torch
        return bf16_round((vals * s).reshape(N, K))


def fp8_dequant_bf16(w, s, kernel_convention: bool = True) -> np.ndarray:
    """[N, K] E4M3FN + [ceil(N/128), K/128] E8M0 -> [N, K] bf16 bits:
    bf16(e4m3(w) * 2^(S[n/128, k/128]-127)) (runtime/dsv4_engine_mxfp4.py:531-553;
    the repeat_interleave + crop there equals indexing the tile by n//128, k//128).

    Pinned: tests compare with torch's float8_e4m3fn / float8_e8m0fnu views and
    against the scalar C oracle."""
    w = np.asarray(w, dtype=np.uint8)
    s = np.asarray(s, dtype=np.uint8)
    N, K = w.shape
    sf = e8m0_decode(s, kernel_convention)
    full = np.repeat(np.repeat(sf, 128, axis=0), 128, axis=1)[:N, :K]
    with np.errstate(over="ignore", invalid="ignore"):
        return bf16_round(e4m3fn_decode(w) * full)


def fp8_dequant_bf16_f32s(w, s_f32) -> np.ndarray:
    """[N, K] E4M3FN + [ceil(N/128), K/128] fp32 tile scales -> [N, K] bf16
    bits: bf16(fp32(e4m3(w) * S[n/128, k/128])), the product rounded to fp32
    and then to bf16, as runtime/dsv4_engine_mxfp4.py:539-548 does with a
    float scale (the benchmark's FP8 configuration).

    Pinned: tests compare with torch's float8_e4m3fn view times a float32
    scale, cast to bfloat16."""
    w = np.asarray(w, dtype=np.uint8)
    s_f32 = np.asarray(s_f32, dtype=np.float32)
    N, K = w.shape
    full = np.repeat(np.repeat(s_f32, 128, axis=0), 128, axis=1)[:N, :K]
    with np.errstate(over="ignore", invalid="ignore"):
        return bf16_round((e4m3fn_decode(w).astype(np.float32) * full).astype(np.float32))


# ------------------------------------------------------------------ GEMVs ---


def _matvec_f32(W_bf16, x_bf16) -> np.ndarray:
    """fp32 product of bf16 operands: y[..., n] = sum_k W[n,k] x[..., k]."""
    return (bf16_to_f32(x_bf16) @ bf16_to_f32(W_bf16).T).astype(np.float32)


def mxfp4_gemv(x, packed, scale) -> np.ndarray:
    """y = bf16( dequant(W) @ x ) with fp32 accumulation
    (kernel/mxfp4-dense/mxfp4_gemv.cu:72-128 via its bit-exact reference
    mxfp4_unpack + e8m0_decode + torch matmul, mxfp4_gemv.cu:33).
    x: bf16 bits [K] or [T, K]."""
    return bf16_round(_matvec_f32(mxfp4_dequant_bf16(packed, scale), x))


def fp8_gemv(x, w, s) -> np.ndarray:
    """y = bf16( x @ dequant(W).T ) with fp32 accumulation
    (runtime/fp8_e4m3_gemv_binding.py:84 contract, dequant of
    runtime/dsv4_engine_mxfp4.py:531-553). x: bf16 bits [K] or [T, K]."""
    return bf16_round(_matvec_f32(fp8_dequant_bf16(w, s), x))


def fp8_gemv_f32s(x, w, s_f32) -> np.ndarray:
    """y = bf16( x @ dequant(W).T ) with fp32 tile scales (fp8_dequant_bf16_f32s)."""
    return bf16_round(_matvec_f32(fp8_dequant_bf16_f32s(w, s_f32), x))


def fp8_gemv_grouped(x, w, s, groups: int) -> np.ndarray:
    """G GEMVs over row groups of one FP8 matrix: w [G*N, K], x [G, K] or
    [T, G, K] bf16 bits -> y[..., g, n] = bf16( x[..., g, :] . dequant(w)[g*N + n] ),
    the scale row following the global row (g*N + n) / 128
    (kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:484-499: the wo_a
    slices W_g = wo_a + g*1024 rows, S_g = + g*8 scale rows)."""
    W = bf16_to_f32(fp8_dequant_bf16(w, s))
    GN, K = W.shape
    N = GN // groups
    xf = bf16_to_f32(np.asarray(x, dtype=np.uint16))
    Wg = W.reshape(groups, N, K)
    y = np.einsum("...gk,gnk->...gn", xf.astype(np.float64), Wg.astype(np.float64))
    return bf16_round(y.astype(np.float32))


def swiglu_clamped(gate_bits, up_bits, limit: float, clamp_up: bool) -> np.ndarray:
    """act = bf16( silu(c(g)) * c_up(u) ) on bf16 gate/up, fp32 math, one
    rounding: the shared expert's SwiGLU (kernel/cpp-engine-mxfp4/
    dsv4_engine_mxfp4_wire.cu:510-521 clamps the gate only, clamp_up=False;
    runtime/dsv4_engine_mxfp4.py:405-408 clamps both, clamp_up=True, and rounds
    silu and the product to bf16 separately, a difference within tolerance).
    c clamps to [-limit, limit]; limit <= 0 disables both clamps."""
    g = bf16_to_f32(gate_bits).astype(np.float32)
    u = bf16_to_f32(up_bits).astype(np.float32)
    if limit > 0:
        g = np.clip(g, -limit, limit).astype(np.float32)
        if clamp_up:
            u = np.clip(u, -limit, limit).astype(np.float32)
    with np.errstate(over="ignore"):
        sil = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return bf16_round((sil * u).astype(np.float32))


def fp8_swiglu(x, w1, s1, w3, s3, limit: float, clamp_up: bool) -> np.ndarray:
    """The shared expert's gate, up and SwiGLU: swiglu_clamped(fp8_gemv(W1),
    fp8_gemv(W3)) (dsv4_engine_mxfp4_wire.cu:528-548)."""
    return swiglu_clamped(fp8_gemv(x, w1, s1), fp8_gemv(x, w3, s3), limit, clamp_up)


def silu_f32(v) -> np.ndarray:
    """x / (1 + exp(-x)) in fp32 (kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:122-124)."""
    v = np.asarray(v, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (v / (np.float32(1.0) + np.exp(-v))).astype(np.float32)


def expert_swiglu_m(x, W1p, W1s, W3p, W3s) -> np.ndarray:
    """M = bf16( silu(W1 x) * (W3 x) ) for one expert, fp32 math
    (kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:186-208, the bf16 rounding at :208).
    x: bf16 bits [K] or [T, K]."""
    g = _matvec_f32(mxfp4_dequant_bf16(W1p, W1s), x)
    u = _matvec_f32(mxfp4_dequant_bf16(W3p, W3s), x)
    return bf16_round(silu_f32(g) * u)


def grouped_gemv_topk(x, W1p, W3p, W2p, W1s, W3s, W2s, r) -> np.ndarray:
    """Routed SwiGLU for one token over n_exp packed experts:
    out = bf16( sum_e r[e] * (W2_e @ M_e) ), fp32 accumulation in expert order
    (kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:143-289; the reference adds the
    experts with fp32 atomics in arbitrary order).
    Shapes: x [K]; W1p/W3p [n, H, K/2]; W2p [n, O, H/2]; scales [.., /32]; r [n]."""
    r = np.asarray(r, dtype=np.float32)
    acc = np.zeros(W2p.shape[1], dtype=np.float32)
    for e in range(W1p.shape[0]):
        M = expert_swiglu_m(x, W1p[e], W1s[e], W3p[e], W3s[e])
        y = _matvec_f32(mxfp4_dequant_bf16(W2p[e], W2s[e]), M)
        acc = (acc + r[e] * y).astype(np.float32)
    return bf16_round(acc)


def moe_layer(x, expert_fn, ids, weights, out_dim: int, n_experts=None) -> np.ndarray:
    """out[t] = bf16( sum_k w[t,k] * W2_e . bf16(silu(W1_e x_t) * (W3_e x_t)) ),
    e = ids[t,k] (runtime/dsv4_engine_mxfp4.py:372-423 with the grouped kernel
    per token). expert_fn(e) -> ((W1p, W1s), (W3p, W3s), (W2p, W2s)).
    Each unique expert is dequantised once. With n_experts given, ids outside
    [0, n_experts) contribute nothing (the device entry skips them)."""
    x = np.atleast_2d(np.asarray(x, dtype=np.uint16))
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=np.float32)
    T = x.shape[0]
    acc = np.zeros((T, out_dim), dtype=np.float32)
    for e in np.unique(ids):
        if n_experts is not None and not 0 <= e < n_experts:
            continue
        tok, kk = np.nonzero(ids == e)
        (W1p, W1s), (W3p, W3s), (W2p, W2s) = expert_fn(int(e))
        M = expert_swiglu_m(x[tok], W1p, W1s, W3p, W3s)
        y = _matvec_f32(mxfp4_dequant_bf16(W2p, W2s), M)
        for i, t in enumerate(tok):
            acc[t] = (acc[t] + weights[t, kk[i]] * y[i]).astype(np.float32)
    return bf16_round(acc)


def dequant_expert_f32(expert):
    """((W1p, W1s), (W3p, W3s), (W2p, W2s)) -> (W1, W3, W2) as fp32 arrays of the
    bf16 dequantised weights, the form moe_layer_dequantised takes."""
    return tuple(bf16_to_f32(mxfp4_dequant_bf16(p, s)) for p, s in expert)


def moe_layer_dequantised(x, dq_fn, ids, weights, out_dim: int) -> np.ndarray:
    """moe_layer with the dequantisation hoisted out of the call: dq_fn(e) returns
    the expert's (W1, W3, W2) already dequantised (dequant_expert_f32). Same
    arithmetic and order as moe_layer, so the results are bit-identical; it
    times the matmuls alone, the "weights dequantised ahead of time" host path
    (runtime/mxfp4_loader.py:272-309 dequantises once at load time)."""
    x = np.atleast_2d(np.asarray(x, dtype=np.uint16))
    xf = bf16_to_f32(x)
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=np.float32)
    acc = np.zeros((x.shape[0], out_dim), dtype=np.float32)
    for e in np.unique(ids):
        tok, kk = np.nonzero(ids == e)
        W1, W3, W2 = dq_fn(int(e))
        g = (xf[tok] @ W1.T).astype(np.float32)
        u = (xf[tok] @ W3.T).astype(np.float32)
        M = bf16_round(silu_f32(g) * u)
        y = (bf16_to_f32(M) @ W2.T).astype(np.float32)
        for i, t in enumerate(tok):
            acc[t] = (acc[t] + weights[t, kk[i]] * y[i]).astype(np.float32)
    return bf16_round(acc)


def route_sigmoid_topk(logits, topk: int):
    """Config gating: top-k logits per token (descending, ties to the lower
    index), weights sigmoid(l) / sum sigmoid over the top-k. The reference's own
    gating (sqrt-softplus x 1.5, runtime/dsv4_engine_mxfp4.py:363-370) differs;
    the benchmark configuration prescribes this one.

    Pinned: tests compare with torch.topk and torch.sigmoid."""
    l = np.asarray(logits, dtype=np.float32)
    ids = np.argsort(-l.astype(np.float64), axis=1, kind="stable")[:, :topk].astype(np.int32)
    sel = np.take_along_axis(l, ids, axis=1).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        s = 1.0 / (1.0 + np.exp(-sel))
        # a token whose selected logits are all -inf gets 0/0 = NaN weights
        return ids, (s / s.sum(axis=1, keepdims=True)).astype(np.float32)


def sqrt_softplus(logits) -> np.ndarray:
    """The reference router's score s = sqrt(softplus(l)) in fp32, with
    softplus(l) = max(l, 0) + log1p(exp(-|l|))
    (kernel/cpp-engine-mxfp4/routed.cu:156-164; runtime/dsv4_engine_mxfp4.py:366
    takes torch.sqrt(F.softplus(gate))).

    Pinned: tests compare with torch.nn.functional.softplus + torch.sqrt in
    fp32 (within 2 ulp) and with fp64 closed forms: s(0) = sqrt(ln 2),
    s(l) = sqrt(l) for large l, s(-inf) = 0, s(+inf) = inf, s(NaN) = NaN."""
    l = np.asarray(logits, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        sp = (np.maximum(l, np.float32(0)) + np.log1p(np.exp(-np.abs(l)))).astype(np.float32)
        return np.sqrt(sp).astype(np.float32)


def route_sqrt_softplus_topk(logits, topk: int, routed_scale: float = 1.5):
    """The reference router's selection and weights for each row of logits
    (kernel/cpp-engine-mxfp4/routed.cu:169-208, runtime/dsv4_engine_mxfp4.py:
    363-370): the top-k scores s = sqrt_softplus(l), descending, the first
    maximum winning ties (the lower expert index); a NaN score is never above
    a number. Weights (s_k / (sum_k' s_k' + 1e-20f)) * scale evaluated in
    double with the sum in pick order, rounded to float32 (routed.cu:201-206;
    the Python engine rounds them further to bf16).

    Pinned: ids against torch.topk on distinct scores and against brute-force
    first-maximum selection on ties; weights against closed forms (their sum
    is scale * S / (S + 1e-20), their ratios are the score ratios)."""
    s = sqrt_softplus(np.atleast_2d(logits))
    key = np.where(np.isnan(s), -np.inf, s.astype(np.float64))
    ids = np.argsort(-key, axis=1, kind="stable")[:, :topk].astype(np.int32)
    sel = np.take_along_axis(s, ids, axis=1)
    scale = float(np.float32(routed_scale))
    eps = float(np.float32(1e-20))
    w = np.empty(sel.shape, dtype=np.float32)
    for t in range(sel.shape[0]):
        total = 0.0
        for k in range(topk):
            total += float(sel[t, k])
        denom = total + eps
        for k in range(topk):
            w[t, k] = np.float32((float(sel[t, k]) / denom) * scale)
    return ids, w


def router_logits(x, w_gate) -> np.ndarray:
    """logits[t, n] = sum_k W_gate[n, k] * x[t, k] over bf16 operands
    (kernel/cpp-engine-mxfp4/routed.cu:124-153), summed in fp64 and rounded
    once to fp32. The reference and the device sum in fp32 in their own
    orders, so they differ from this by a few ulps of sum_k |W x|.

    Pinned: tests check it against the fp64 scalar C oracle on small shapes
    and a one-hot x selecting a column of W_gate exactly."""
    xf = bf16_to_f32(np.atleast_2d(x)).astype(np.float64)
    wf = bf16_to_f32(w_gate).astype(np.float64)
    return (xf @ wf.T).astype(np.float32)


# ---------------------------------------------------------------- RMSNorm ---


def rmsnorm(x, w, eps: float = 1e-6) -> np.ndarray:
    """y = bf16( (w * x) * rsqrt(sum(x^2)/H + eps) ) per row
    (kernel/rmsnorm-fuse/rmsnorm_fuse.cu:86-103; runtime/dsv4_engine_mxfp4.py:136-141
    computes the same up to product order). Sum of squares in fp64."""
    xf = bf16_to_f32(np.atleast_2d(x)).astype(np.float64)
    H = xf.shape[-1]
    rms = 1.0 / np.sqrt((xf * xf).sum(axis=-1, keepdims=True) / H + eps)
    wf = bf16_to_f32(w).astype(np.float64)
    return bf16_round((wf * xf) * rms)


def rmsnorm_residual(x, r, w, eps: float = 1e-6):
    """t = x + r (fp32, exact for bf16 inputs of similar magnitude);
    new_residual = bf16(t); y = bf16( (w * bf16(t)) * rsqrt(sum(t^2)/H + eps) )
    with the sum over the unrounded t (kernel/rmsnorm-fuse/rmsnorm_fuse.cu:135-156).
    Returns (y, new_residual) as bf16 bits. Sum of squares in fp64."""
    t = (bf16_to_f32(np.atleast_2d(x)) + bf16_to_f32(np.atleast_2d(r))).astype(np.float32)
    new_res = bf16_round(t)
    td = t.astype(np.float64)
    H = td.shape[-1]
    rms = 1.0 / np.sqrt((td * td).sum(axis=-1, keepdims=True) / H + eps)
    wf = bf16_to_f32(w).astype(np.float64)
    y = bf16_round((wf * bf16_to_f32(new_res).astype(np.float64)) * rms)
    return y, new_res


# --------------------------------------------------------------- metrics ----


def compare(got_bits, ref_bits):
    """(max relative error, cosine) of two bf16 tensors, in fp64:
    rel = max|got - ref| / max|ref| and cosine over the flattened values."""
    g = bf16_to_f32(got_bits).astype(np.float64).reshape(-1)
    r = bf16_to_f32(ref_bits).astype(np.float64).reshape(-1)
    denom = np.abs(r).max()
    rel = np.abs(g - r).max() / denom if denom > 0 else np.abs(g - r).max()
    ng, nr = np.linalg.norm(g), np.linalg.norm(r)
    cos = float(g @ r / (ng * nr)) if ng > 0 and nr > 0 else (1.0 if ng == nr else 0.0)
    return float(rel), cos


REL_TOL = 1e-2
COS_TOL = 0.9999
