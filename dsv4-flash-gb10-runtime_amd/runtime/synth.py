"""Seeded synthetic inputs for the decode hot path (numpy side of the generator).

Integer draws come from counter-based SplitMix64 (Steele, Lea & Flood,
OOPSLA 2014): element ``i`` of stream ``seed`` is
``mix64(seed + (i + 1) * 0x9E3779B97F4A7C15)``. The device filler
(``csrc/dsv4_fill.hip``) computes the same function, so packed MXFP4 weights
and E8M0 scales filled on the GPU equal, byte for byte, what this module
returns for the same ``(seed, offset)``. Real-valued inputs (activations,
FP8 weights, RMSNorm tensors, gating logits) are drawn here with Box-Muller
on two 53-bit uniforms and uploaded, so the GPU and the CPU oracle always see
the same bytes.

Distributions follow the benchmark configurations:
  * MXFP4 weights: packed bytes uniform over 0..255 (both nibbles uniform over
    the 16 e2m1 codes); scale bytes uniform over 119..125 (2^-8 .. 2^-2).
  * activations: bf16 of N(0, 1).
  * FP8 weights: N(0, 0.02), one power-of-two scale per 128x128 tile
    (2^ceil(log2(amax/448)), stored as E8M0), codes = RNE E4M3FN of W/scale.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

SCALE_LO = 119
SCALE_HI = 125


def splitmix64(seed: int, offset: int, n: int) -> np.ndarray:
    """Elements offset .. offset+n-1 of SplitMix64 stream ``seed`` (uint64)."""
    idx = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (idx + np.uint64(1)) * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform_u8(seed: int, offset: int, n: int, lo: int = 0, hi: int = 255) -> np.ndarray:
    """Bytes uniform over [lo, hi]: lo + ((draw >> 32) * (hi - lo + 1)) >> 32."""
    if not (0 <= lo <= hi <= 255):
        raise ValueError(f"bad byte range [{lo}, {hi}]")
    z = splitmix64(seed, offset, n)
    span = np.uint64(hi - lo + 1)
    with np.errstate(over="ignore"):
        v = ((z >> np.uint64(32)) * span) >> np.uint64(32)
    return (v + np.uint64(lo)).astype(np.uint8)


def normal_f64(seed: int, offset: int, n: int) -> np.ndarray:
    """n standard normals (float64) from draws offset .. offset+2n-1 of the stream."""
    z = splitmix64(seed, 2 * offset, 2 * n)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even, NaN -> 0x7FC0|sign."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    r = np.where(nan, (u >> np.uint64(16)) | np.uint64(0x40), r)
    return (r & np.uint64(0xFFFF)).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(seed: int, shape, mean: float = 0.0, std: float = 1.0, offset: int = 0) -> np.ndarray:
    """bf16 bits of mean + std * N(0,1), rounded float64 -> float32 -> bf16 (RNE)."""
    n = int(np.prod(shape))
    v = (mean + std * normal_f64(seed, offset, n)).astype(np.float32)
    return f32_to_bf16_bits(v).reshape(shape)


# ----------------------------------------------------------------- MXFP4 ----

def mxfp4_weight(seed: int, rows: int, cols: int, n_mats: int = 1, first: int = 0):
    """Packed e2m1 bytes [n_mats, rows, cols/2] and E8M0 scales [n_mats, rows, cols/32].

    Matrix m of a stack occupies draws (first + m) * rows * cols/2 ... of stream
    ``seed`` (packed) and of stream ``seed + 1`` (scales), so one expert of a
    256-expert tensor can be regenerated alone.
    """
    pk = rows * cols // 2
    sc = rows * cols // 32
    packed = uniform_u8(seed, (first) * pk, n_mats * pk).reshape(n_mats, rows, cols // 2)
    scale = uniform_u8(seed + 1, (first) * sc, n_mats * sc, SCALE_LO, SCALE_HI).reshape(
        n_mats, rows, cols // 32)
    return packed, scale


# ------------------------------------------------------------------- FP8 ----

def _e4m3fn_grid() -> np.ndarray:
    """All 126 finite non-negative E4M3FN values (bytes 0x00..0x7E), ascending."""
    b = np.arange(0x7F, dtype=np.int64)
    e = b >> 3
    m = b & 7
    return np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))


_E4M3_POS = _e4m3fn_grid()


def e4m3fn_quantize(v: np.ndarray) -> np.ndarray:
    """Round float values (|v| <= 448) to E4M3FN bytes, nearest with ties to even code."""
    v = np.asarray(v, dtype=np.float64)
    a = np.abs(v)
    if np.any(a > 448.0):
        raise ValueError("value outside E4M3FN range")
    hi = np.searchsorted(_E4M3_POS, a, side="left").clip(0, 126)
    lo = (hi - 1).clip(0, 126)
    dlo = a - _E4M3_POS[lo]
    dhi = _E4M3_POS[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    sign = (np.signbit(v) & (code != 0)).astype(np.uint8) << 7
    return code | sign


def fp8_weight(seed: int, N: int, K: int, std: float = 0.02):
    """E4M3FN codes [N, K] and E8M0 tile scales [ceil(N/128), K/128] of N(0, std) weights."""
    w = std * normal_f64(seed, 0, N * K).reshape(N, K)
    nt, kt = (N + 127) // 128, K // 128
    pad = np.zeros((nt * 128, K))
    pad[:N] = w
    amax = np.abs(pad.reshape(nt, 128, kt, 128)).max(axis=(1, 3))
    amax = np.where(amax > 0, amax, 448.0)
    exp = np.ceil(np.log2(amax / 448.0)).astype(np.int64)
    scale_b = (exp + 127).astype(np.uint8)
    sfull = np.repeat(np.repeat(2.0 ** exp, 128, axis=0), 128, axis=1)[:N, :K]
    codes = e4m3fn_quantize(w / sfull)
    return codes, scale_b


def fp8_weight_f32s(seed: int, N: int, K: int, std: float = 0.02):
    """E4M3FN codes [N, K] and fp32 tile scales [ceil(N/128), K/128] of N(0, std)
    weights, one scale per 128x128 block: amax / 448 (the benchmark's FP8
    configuration), codes = RNE-to-E4M3(W / scale)."""
    w = std * normal_f64(seed, 0, N * K).reshape(N, K)
    nt, kt = (N + 127) // 128, K // 128
    pad = np.zeros((nt * 128, K))
    pad[:N] = w
    amax = np.abs(pad.reshape(nt, 128, kt, 128)).max(axis=(1, 3))
    scale = np.where(amax > 0, amax / 448.0, 1.0).astype(np.float32)
    sfull = np.repeat(np.repeat(scale.astype(np.float64), 128, axis=0), 128, axis=1)[:N, :K]
    # the scale rounded to fp32 can put the block's largest value a rounding
    # step above 448: saturate at the largest E4M3FN value
    codes = e4m3fn_quantize(np.clip(w / sfull, -448.0, 448.0))
    return codes, scale


# ---------------------------------------------------------------- routing ---

def gating_logits(seed: int, T: int, n_experts: int) -> np.ndarray:
    return normal_f64(seed, 0, T * n_experts).astype(np.float32).reshape(T, n_experts)


def zipf_routing(seed: int, steps: int, n_experts: int = 256, topk: int = 8, s: float = 1.1,
                 layer: int = 0):
    """Per-step top-k ids drawn by Gumbel-top-k on log p, p(rank r) ~ r^-s over a
    seeded expert permutation, plus sigmoid(N(0,1)) weights renormalised to 1."""
    rng_seed = seed * 1000003 + layer
    perm = np.argsort(splitmix64(rng_seed, 0, n_experts))
    logp = -s * np.log(np.arange(1, n_experts + 1, dtype=np.float64))
    logp_e = np.empty(n_experts)
    logp_e[perm] = logp
    z = splitmix64(rng_seed + 1, 0, steps * n_experts)
    u = ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)
    g = -np.log(-np.log(u)).reshape(steps, n_experts)
    ids = np.argsort(-(logp_e[None, :] + g), axis=1, kind="stable")[:, :topk].astype(np.int32)
    l = normal_f64(rng_seed + 2, 0, steps * topk).reshape(steps, topk)
    sg = 1.0 / (1.0 + np.exp(-l))
    w = (sg / sg.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids, w
