"""CPU pins of the number formats, bf16 rounding, packing and the input generator.

Each oracle decoder is checked against a source independent of oracle/mx.py:
torch's own float8 dtypes, math.ldexp, the OCP MX v1.0 tables, and published
SplitMix64 outputs. Mutation tests show the checks catch plausible mistakes.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import c_oracle as co
from oracle import mx
from runtime import synth

ALL_BYTES = np.arange(256, dtype=np.uint8)

# OCP Microscaling Formats v1.0, FP4 (E2M1) element values by encoding 0b0000..0b0111;
# encodings 0b1xxx are the negatives (0b1000 is -0).
OCP_FP4_POSITIVE = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def _f32_bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def test_e2m1_table_matches_ocp_spec():
    vals = mx.e2m1_value(np.arange(16))
    assert np.array_equal(vals[:8], np.array(OCP_FP4_POSITIVE, dtype=np.float32))
    assert np.array_equal(vals[8:], -np.array(OCP_FP4_POSITIVE, dtype=np.float32))
    assert np.signbit(vals[8]) and not np.signbit(vals[0])  # code 8 is -0.0


def test_e2m1_c_oracle_matches():
    L = co.lib()
    assert [L.mxo_e2m1(c) for c in range(16)] == [float(v) for v in mx.e2m1_value(np.arange(16))]


def test_e8m0_matches_torch_and_ldexp():
    ref = torch.from_numpy(ALL_BYTES.copy()).view(torch.float8_e8m0fnu).float().numpy()
    py = mx.e8m0_decode(ALL_BYTES, kernel_convention=False)
    assert np.array_equal(_f32_bits(py[:255]), _f32_bits(ref[:255]))
    assert np.isnan(py[255]) and np.isnan(ref[255])
    assert all(py[b] == np.float32(math.ldexp(1.0, b - 127)) for b in range(255))
    k = mx.e8m0_decode(ALL_BYTES, kernel_convention=True)
    assert k[255] == 0.0 and np.array_equal(k[:255], py[:255])
    assert k[0] == np.float32(2.0 ** -127) and k[0] != 0.0  # subnormal, not flushed
    L = co.lib()
    assert all(L.mxo_e8m0(b) == k[b] for b in range(256))


def test_e4m3fn_matches_torch_all_bytes():
    ref = torch.from_numpy(ALL_BYTES.copy()).view(torch.float8_e4m3fn).float().numpy()
    got = mx.e4m3fn_decode(ALL_BYTES)
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got))
    assert set(np.nonzero(nan)[0]) == {0x7F, 0xFF}
    assert np.array_equal(_f32_bits(got[~nan]), _f32_bits(ref[~nan]))
    L = co.lib()
    c = np.array([L.mxo_e4m3fn(int(b)) for b in ALL_BYTES], dtype=np.float32)
    assert np.array_equal(_f32_bits(c[~nan]), _f32_bits(ref[~nan]))


def test_e4m3fn_quantizer_matches_torch_cast():
    rng = np.random.default_rng(7)
    v = np.concatenate([rng.standard_normal(20000) * 50, rng.standard_normal(2000) * 1e-2,
                        np.array([0.0, -0.0, 448.0, -448.0, 2.0 ** -9, 3 * 2.0 ** -10])])
    v = np.clip(v, -448, 448).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = synth.e4m3fn_quantize(v)
    nz = mx.e4m3fn_decode(ref) != 0  # +-0 differ only in sign of zero
    assert np.array_equal(got[nz], ref[nz])


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    parts = [
        rng.standard_normal(200000).astype(np.float32) * 100,
        (rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
        # exact ties: low 16 bits == 0x8000 with even and odd bf16 lsb
        (np.arange(0x3F800000, 0x3F800000 + 2 * 65536 * 8, 65536, dtype=np.uint32)
         | np.uint32(0x8000)).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38], dtype=np.float32),
    ]
    a = np.concatenate(parts)
    ref = torch.from_numpy(a).to(torch.bfloat16).view(torch.uint16).numpy()
    got = mx.bf16_round(a)
    nan = np.isnan(a)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7FC0) == 0x7FC0)
    L = co.lib()
    sub = a[~nan][:5000]
    assert np.array_equal(np.array([L.mxo_bf16_rne(float(f)) for f in sub], dtype=np.uint16),
                          ref[~nan][:5000])
    assert np.array_equal(synth.f32_to_bf16_bits(a[~nan]), ref[~nan])


def test_nibble_order_known_answers():
    # byte = (code[2i+1] << 4) | code[2i]: 0x21 -> codes (1, 2) = (+0.5, +1.0)
    assert mx.mxfp4_unpack(np.array([0x21], np.uint8), (2,)).tolist() == [0.5, 1.0]
    v = mx.mxfp4_unpack(np.array([0x8F, 0x70], np.uint8), (4,))
    assert v.tolist() == [-6.0, -0.0, 0.0, 6.0]
    assert np.signbit(v[1]) and not np.signbit(v[2])


def test_pack_unpack_round_trip_exhaustive():
    vals = mx.mxfp4_unpack(ALL_BYTES, (512,))
    assert np.array_equal(mx.mxfp4_pack(vals), ALL_BYTES)
    with pytest.raises(ValueError):
        mx.mxfp4_pack(np.array([0.25, 1.0]))


def test_mxfp4_dequant_matches_torch_composition():
    """dequant == e2m1 value (OCP table) x torch float8_e8m0fnu scale, cast by torch to bf16."""
    p, s = synth.mxfp4_weight(11, 32, 128)
    p, s = p[0], s[0]
    s = s.copy()
    s[0, :4] = [0, 1, 200, 254]  # extremes of the finite scale range
    codes = np.empty((32, 128), np.int64)
    codes[:, 0::2] = p & 15
    codes[:, 1::2] = p >> 4
    table = np.array(OCP_FP4_POSITIVE + [-v for v in OCP_FP4_POSITIVE], np.float32)
    scale_t = torch.from_numpy(s).view(torch.float8_e8m0fnu).float()
    ref = (torch.from_numpy(table[codes]) * scale_t.repeat_interleave(32, dim=1)).to(torch.bfloat16)
    got = mx.mxfp4_dequant_bf16(p, s)
    assert np.array_equal(got, ref.view(torch.uint16).numpy())
    assert np.array_equal(co.mxfp4_dequant(p, s), got)


def test_fp8_dequant_matches_torch_composition():
    w, s = synth.fp8_weight(12, 200, 256)
    wt = torch.from_numpy(w).view(torch.float8_e4m3fn).float()
    st = torch.from_numpy(s).view(torch.float8_e8m0fnu).float()
    full = st.repeat_interleave(128, 0).repeat_interleave(128, 1)[:200, :256]
    ref = (wt * full).to(torch.bfloat16).view(torch.uint16).numpy()
    got = mx.fp8_dequant_bf16(w, s)
    assert np.array_equal(got, ref)
    assert np.array_equal(co.fp8_dequant(w, s), got)


def test_fp8_dequant_f32_scales_matches_torch_composition():
    """fp32 tile scales (the benchmark's FP8 configuration): every E4M3FN byte
    (NaN codes included) against non-power-of-two scales, through torch's
    float8_e4m3fn view times a float32 tile scale, cast to bfloat16 (the
    reference's dequantisation, runtime/dsv4_engine_mxfp4.py:539-548)."""
    w = np.tile(np.arange(256, dtype=np.uint8), (300, 2))           # [300, 512]
    rng = np.random.default_rng(7)
    sc = (rng.uniform(0.5, 2.0, (3, 4)) * 2.0 ** rng.integers(-12, 4, (3, 4))).astype(np.float32)
    wt = torch.from_numpy(w).view(torch.float8_e4m3fn).float()
    full = torch.from_numpy(sc).repeat_interleave(128, 0).repeat_interleave(128, 1)[:300, :512]
    ref = (wt * full).to(torch.bfloat16).view(torch.uint16).numpy()
    got = mx.fp8_dequant_bf16_f32s(w, sc)
    nan = np.isnan(mx.bf16_to_f32(ref))
    assert np.array_equal(np.isnan(mx.bf16_to_f32(got)), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    # the generator's scales are amax/448 per 128x128 block and its codes in range
    codes, scales = synth.fp8_weight_f32s(13, 200, 256)
    assert scales.dtype == np.float32 and scales.shape == (2, 2)
    deq = mx.bf16_to_f32(mx.fp8_dequant_bf16_f32s(codes, scales))
    w0 = 0.02 * synth.normal_f64(13, 0, 200 * 256).reshape(200, 256)
    assert np.abs(deq - w0).max() <= np.abs(w0).max() / 448 * 32 * 1.01   # half an e4m3 step at the top


def test_splitmix64_published_outputs():
    # First outputs of SplitMix64 seeded with 0 (Vigna's splitmix64.c).
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert [int(v) for v in synth.splitmix64(0, 0, 4)] == want
    assert [int(v) for v in synth.splitmix64(0, 2, 2)] == want[2:]


def test_uniform_bytes_ranges():
    b = synth.uniform_u8(5, 0, 200000)
    counts = np.bincount(b, minlength=256)
    assert counts.min() > 600 and counts.max() < 1000
    s = synth.uniform_u8(6, 0, 70000, synth.SCALE_LO, synth.SCALE_HI)
    assert s.min() == 119 and s.max() == 125
    n = synth.normal_f64(7, 0, 200000)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1) < 0.01


# ---------------------------------------------------- mutation checks --------
# A plausible mistake planted in the oracle must fail one of the pins above.

def test_mutation_swapped_nibbles_is_caught(monkeypatch):
    real = mx.mxfp4_unpack

    def swapped(packed, shape, dtype=np.float32):
        b = np.asarray(packed, np.uint8)
        return real(((b << 4) | (b >> 4)).astype(np.uint8), shape, dtype)

    monkeypatch.setattr(mx, "mxfp4_unpack", swapped)
    assert mx.mxfp4_unpack(np.array([0x21], np.uint8), (2,)).tolist() != [0.5, 1.0]


def test_mutation_scale_bias_off_by_one_is_caught():
    wrong = np.ldexp(np.float64(1.0), ALL_BYTES.astype(np.int32) - 126)[:254].astype(np.float32)
    ref = torch.from_numpy(ALL_BYTES.copy()).view(torch.float8_e8m0fnu).float().numpy()
    assert not np.array_equal(_f32_bits(wrong), _f32_bits(ref[:254]))
