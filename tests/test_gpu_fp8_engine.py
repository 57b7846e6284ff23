"""GPU parity of the FP8 GEMVs at the reference engine's MLA shapes
(kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:395-418, 404, 501): the
tile kernels at K = 1024 (wq_b, 32768 x 1024) and K = 8192 (wo_b, 4096 x
8192), several tokens with the weights read once, and the multi-matrix launch
(wq_a and wkv on one activation) against the oracle and, bit for bit, against
one launch per matrix. Bar: max rel err <= 1e-2, cosine >= 0.9999."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mx
from runtime import fp8_e4m3_gemv_binding as fp8b
from runtime import synth
from tests.gpu_util import announce, assert_close, dev_bf16, dev_u8, host_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K,T", [(32768, 1024, 1), (1040, 1024, 3), (130, 1024, 16),
                                   (4096, 8192, 1), (4096, 8192, 2), (4096, 8192, 5), (300, 8192, 16),
                                   (4096, 4096, 16), (1000, 2048, 11)])
def test_fp8_tile_engine_shapes(device, N, K, T):
    """K = 1024 and 8192 on the tile path (16 and 2 rows per workgroup), and
    token counts above the per-group register budget (4 at K = 8192, 16
    otherwise), which loop over token groups with the weights in registers."""
    announce(f"fp8_e4m3_gemv tile N={N} K={K} T={T}")
    w, s = synth.fp8_weight(15000 + N + K, N, K)
    x = synth.normal_bf16(15100 + T + K, (T, K))
    xd = dev_bf16(x, device)
    y = fp8b.fp8_e4m3_gemv(dev_u8(w, device), dev_u8(s, device), xd if T > 1 else xd[0])
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 N={N} K={K} T={T}")


@pytest.mark.parametrize("shapes,K,T", [([1536, 576], 4096, 1), ([1024, 512], 4096, 1), ([1536, 576], 4096, 4),
                                        ([130, 700, 64], 2048, 2), ([4096, 1024], 8192, 3),
                                        ([2048, 300], 1024, 1), ([1024, 576], 4096, 8), ([2048, 1024], 4096, 6)])
def test_fp8_gemv_multi(device, shapes, K, T):
    """Several matrices on one activation in one launch: each output has the
    bits of fp8_e4m3_gemv on that matrix alone and matches the oracle. At
    K = 4096 and T = 6 or 8 the launch runs the matrix-core tile kernel while
    each matrix alone (below 3072 rows) takes the two-block split kernel: the
    same per-block partials added in the same order, so the same bits."""
    announce(f"fp8_e4m3_gemv_multi N={shapes} K={K} T={T}")
    mats, dmats = [], []
    for i, N in enumerate(shapes):
        w, s = synth.fp8_weight(15200 + 10 * i + N, N, K)
        mats.append((w, s))
        dmats.append((dev_u8(w, device), dev_u8(s, device)))
    x = synth.normal_bf16(15300 + T, (T, K))
    xd = dev_bf16(x, device)
    xin = xd if T > 1 else xd[0]
    ys = fp8b.fp8_e4m3_gemv_multi(dmats, xin)
    for (w, s), (tw, ts), y, N in zip(mats, dmats, ys, shapes):
        got = host_bits(y).reshape(T, N)
        single = host_bits(fp8b.fp8_e4m3_gemv(tw, ts, xin)).reshape(T, N)
        assert np.array_equal(got, single), f"N={N}: multi launch differs from the single launch"
        assert_close(got, mx.fp8_gemv(x, w, s), f"multi N={N} K={K} T={T}")


@pytest.mark.parametrize("N,K,T", [(2048, 8192, 1), (512, 1024, 3)])
def test_fp8_swiglu_gemv_engine_k(device, N, K, T):
    announce(f"fp8_e4m3_swiglu_gemv N={N} K={K} T={T}")
    w1, s1 = synth.fp8_weight(15400 + N, N, K)
    w3, s3 = synth.fp8_weight(15500 + N, N, K)
    x = mx.bf16_round(24 * mx.bf16_to_f32(synth.normal_bf16(15600 + T, (T, K))))
    xd = dev_bf16(x, device)
    act = fp8b.fp8_e4m3_swiglu_gemv(dev_u8(w1, device), dev_u8(s1, device), dev_u8(w3, device),
                                    dev_u8(s3, device), xd if T > 1 else xd[0], 10.0, False)
    assert_close(host_bits(act).reshape(T, N), mx.fp8_swiglu(x, w1, s1, w3, s3, 10.0, False),
                 f"fp8 swiglu N={N} K={K} T={T}")


# Shapes on the matrix-core path (K = 1024: T >= 3 at N >= 2048, T >= 5 at
# any N; K = 2048: T >= 3 at N >= 4096, T >= 5 at any N; K = 4096: T >= 3 at
# N >= 4096, T >= 5 above 512 rows; K = 8192: T >= 2): every K of the tile
# set (2, 4, 8 and 16 waves per workgroup), a last 16-row block that is
# partly past N, K = 4096 below 3072 rows at T = 5 .. 8 (two 512-k blocks per
# MFMA, a last 8-row workgroup partly past N) and K = 8192 with at most 2048
# rows (four blocks per MFMA).
@pytest.mark.parametrize("N,K,T", [(2048, 1024, 8), (2050, 2048, 5), (4096, 2048, 4), (1540, 4096, 9),
                                   (4100, 4096, 3), (4096, 8192, 16), (64, 8192, 2), (600, 4096, 8),
                                   (2004, 4096, 5)])
def test_fp8_matrix_core_path(device, N, K, T):
    announce(f"fp8_e4m3_gemv matrix-core path N={N} K={K} T={T}")
    w, s = synth.fp8_weight(16000 + N + K, N, K)
    x = synth.normal_bf16(16100 + T + K, (T, K))
    y = fp8b.fp8_e4m3_gemv(dev_u8(w, device), dev_u8(s, device), dev_bf16(x, device))
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 N={N} K={K} T={T}")


@pytest.mark.parametrize("N,K,T", [(1, 1024, 5), (7, 2048, 9), (15, 1024, 16), (17, 2048, 8)])
def test_fp8_matrix_core_tiny_n(device, N, K, T):
    """Fewer than 16 rows (and just over 16) on the matrix cores, which take
    K = 1024 and 2048 from T = 5 at any N: the 16-row block reads its rows
    clamped to the last one and stores only the real ones. The single GEMV
    and the fused SwiGLU against the oracle, and a two-matrix launch (N rows
    and 3 rows) bit for bit against the single GEMVs."""
    announce(f"fp8_e4m3_gemv matrix-core tiny N={N} K={K} T={T}")
    w1, s1 = synth.fp8_weight(17900 + N + K, N, K)
    w3, s3 = synth.fp8_weight(17950 + N + K, N, K)
    w2, s2 = synth.fp8_weight(17990 + K, 3, K)
    x = mx.bf16_round(8 * mx.bf16_to_f32(synth.normal_bf16(18000 + T, (T, K))))
    xd = dev_bf16(x, device)
    d1, e1 = dev_u8(w1, device), dev_u8(s1, device)
    d2, e2 = dev_u8(w2, device), dev_u8(s2, device)
    y = host_bits(fp8b.fp8_e4m3_gemv(d1, e1, xd)).reshape(T, N)
    assert_close(y, mx.fp8_gemv(x, w1, s1), f"fp8 tiny N={N} K={K} T={T}")
    act = fp8b.fp8_e4m3_swiglu_gemv(d1, e1, dev_u8(w3, device), dev_u8(s3, device), xd, 10.0, True)
    assert_close(host_bits(act).reshape(T, N), mx.fp8_swiglu(x, w1, s1, w3, s3, 10.0, True), f"swiglu tiny N={N}")
    ya, yb = fp8b.fp8_e4m3_gemv_multi([(d1, e1), (d2, e2)], xd)
    assert np.array_equal(host_bits(ya).reshape(T, N), y)
    assert np.array_equal(host_bits(yb).reshape(T, 3), host_bits(fp8b.fp8_e4m3_gemv(d2, e2, xd)).reshape(T, 3))


@pytest.mark.parametrize("N,K,T", [(8192, 4096, 8), (16384, 4096, 9), (16400, 1024, 16), (8192, 2048, 13),
                                   (8200, 2048, 8), (16400, 4096, 12)])
def test_fp8_matrix_core_row_blocks(device, N, K, T):
    """Large N at T >= 8 runs 2 or 4 16-row blocks per wave on one set of
    activation registers (R = 2: 8192 x 4096, 16400 x 1024, 8192 x 2048,
    8200 x 2048; R = 4: 16384 x 4096, 16400 x 4096; a ragged N leaves the
    last workgroup's blocks partly past the matrix): against the oracle, and
    the first four tokens equal a T = 4 call (one block per wave) bit for bit,
    since the blocking does not change a row's sums."""
    announce(f"fp8_e4m3_gemv matrix-core row blocks N={N} K={K} T={T}")
    w, s = synth.fp8_weight(16800 + N + K, N, K)
    x = synth.normal_bf16(16900 + T + K, (T, K))
    tw, ts, xd = dev_u8(w, device), dev_u8(s, device), dev_bf16(x, device)
    got = host_bits(fp8b.fp8_e4m3_gemv(tw, ts, xd)).reshape(T, N)
    assert_close(got, mx.fp8_gemv(x, w, s), f"fp8 row blocks N={N} K={K} T={T}")
    four = host_bits(fp8b.fp8_e4m3_gemv(tw, ts, xd[:4].contiguous())).reshape(4, N)
    assert np.array_equal(four, got[:4])


@pytest.mark.parametrize("N", [8192, 8200])
def test_fp8_matrix_core_row_blocks_grouped(device, N):
    """Two groups at T = 8 with two 16-row blocks per wave in each group; with
    8200 rows the second group starts 8 rows into a scale tile and both end
    inside a workgroup. Against the oracle; a group that starts on a scale
    tile has the bits of a single GEMV on its slice."""
    G, K, T = 2, 2048, 8
    announce(f"fp8_e4m3_gemv_grouped matrix-core row blocks G={G} N={N} K={K} T={T}")
    w, s = synth.fp8_weight(17000 + N, G * N, K)
    x = synth.normal_bf16(17001, (T, G, K))
    tw, ts, xd = dev_u8(w, device), dev_u8(s, device), dev_bf16(x, device)
    got = host_bits(fp8b.fp8_e4m3_gemv_grouped(tw, ts, xd, G)).reshape(T, G, N)
    assert_close(got.reshape(T, -1), mx.fp8_gemv_grouped(x, w, s, G).reshape(T, -1), "grouped row blocks")
    for g in range(G):
        if (g * N) % 128:
            continue
        r0 = g * N // 128
        yg = fp8b.fp8_e4m3_gemv(tw[g * N:(g + 1) * N], ts[r0:r0 + (N + 127) // 128], xd[:, g].contiguous())
        assert np.array_equal(host_bits(yg).reshape(T, N), got[:, g])


def test_fp8_matrix_core_groups_straddle_scale_tiles(device):
    """Groups of 2056 rows: the second group starts 8 rows into a 16-row
    block, so its blocks straddle 128-row scale tiles; each group's bits equal
    a single GEMV on its slice (both on the matrix cores)."""
    G, N, K, T = 2, 2056, 2048, 5
    announce(f"fp8_e4m3_gemv_grouped matrix-core G={G} N={N} K={K} T={T}")
    w, s = synth.fp8_weight(16200, G * N, K)
    x = synth.normal_bf16(16201, (T, G, K))
    tw, ts = dev_u8(w, device), dev_u8(s, device)
    xd = dev_bf16(x, device)
    got = host_bits(fp8b.fp8_e4m3_gemv_grouped(tw, ts, xd, G)).reshape(T, G, N)
    assert_close(got.reshape(T, -1), mx.fp8_gemv_grouped(x, w, s, G).reshape(T, -1), "grouped straddle")
    # group 0 starts on a scale tile: its slice is a plain GEMV
    y0 = fp8b.fp8_e4m3_gemv(tw[:N], ts[:(N + 127) // 128], xd[:, 0].contiguous())
    assert np.array_equal(host_bits(y0).reshape(T, N), got[:, 0])


@pytest.mark.parametrize("N,K,T", [(2048, 1024, 4), (2048, 4096, 9), (2048, 8192, 3), (1536, 2048, 12),
                                   (8192, 2048, 8), (8200, 2048, 9)])
def test_fp8_swiglu_matrix_core(device, N, K, T):
    """The fused SwiGLU on the matrix cores (K = 8192 runs two passes per
    wave; 8192 rows at T = 8 two 16-row blocks per wave): against the oracle,
    and gate/up equal to the single GEMVs' bits."""
    announce(f"fp8_e4m3_swiglu_gemv matrix-core N={N} K={K} T={T}")
    w1, s1 = synth.fp8_weight(16300 + N + K, N, K)
    w3, s3 = synth.fp8_weight(16400 + N + K, N, K)
    x = mx.bf16_round(24 * mx.bf16_to_f32(synth.normal_bf16(16500 + T, (T, K))))
    t1, u1, t3, u3 = dev_u8(w1, device), dev_u8(s1, device), dev_u8(w3, device), dev_u8(s3, device)
    xd = dev_bf16(x, device)
    act = host_bits(fp8b.fp8_e4m3_swiglu_gemv(t1, u1, t3, u3, xd, 10.0, True)).reshape(T, N)
    gate = host_bits(fp8b.fp8_e4m3_gemv(t1, u1, xd)).reshape(T, N)
    up = host_bits(fp8b.fp8_e4m3_gemv(t3, u3, xd)).reshape(T, N)
    ref_bits = mx.swiglu_clamped(gate, up, 10.0, True)
    diff = np.abs(act.astype(np.int32) - ref_bits.astype(np.int32))
    diff[mx.bf16_to_f32(act) == mx.bf16_to_f32(ref_bits)] = 0
    assert diff.max() <= 1, f"max bf16 ulp difference {diff.max()}"
    assert_close(act, mx.fp8_swiglu(x, w1, s1, w3, s3, 10.0, True), f"swiglu matrix-core T={T}")


def test_fp8_multi_matrix_core(device):
    """Two matrices on the matrix cores in one launch: each output has the bits
    of the single launch on that matrix."""
    shapes, K, T = [4096, 2048], 4096, 9
    announce(f"fp8_e4m3_gemv_multi matrix-core N={shapes} K={K} T={T}")
    mats, dmats = [], []
    for i, N in enumerate(shapes):
        w, s = synth.fp8_weight(16600 + i, N, K)
        mats.append((w, s))
        dmats.append((dev_u8(w, device), dev_u8(s, device)))
    x = synth.normal_bf16(16700, (T, K))
    xd = dev_bf16(x, device)
    ys = fp8b.fp8_e4m3_gemv_multi(dmats, xd)
    for (w, s), (tw, ts), y, N in zip(mats, dmats, ys, shapes):
        got = host_bits(y).reshape(T, N)
        assert np.array_equal(got, host_bits(fp8b.fp8_e4m3_gemv(tw, ts, xd)).reshape(T, N))
        assert_close(got, mx.fp8_gemv(x, w, s), f"multi matrix-core N={N}")


@pytest.mark.parametrize("N,K,T", [(2048, 8192, 2), (2048, 8192, 3), (4096, 4096, 4), (2048, 1024, 4),
                                   (8192, 2048, 8)])
def test_fp8_swiglu_matrix_core_keeps_gemv_bits(device, N, K, T):
    """Gate and up of the fused SwiGLU on the matrix cores are exactly the
    bits of fp8_e4m3_gemv on each matrix (K = 8192 included, where a wave
    takes two 512-k blocks). Inputs make the SiLU exact in fp32: non-negative
    weights and activations give gate sums >= 17, where exp(-g) < 2^-24 and
    1 + exp(-g) rounds to 1, so act = bf16(bf16(gate) * bf16(up)) with an
    exact fp32 product, and any change in either sum's bits shows (0 ulp)."""
    announce(f"fp8_e4m3_swiglu_gemv bit equality N={N} K={K} T={T}")
    w1, s1 = synth.fp8_weight(16900 + N + K, N, K)
    w3, s3 = synth.fp8_weight(17000 + N + K, N, K)
    w1 = (w1 & 0x7F).astype(np.uint8)         # |W1| (no 0xFF codes, so no NaN appears)
    x = (synth.normal_bf16(17100 + T, (T, K)) & 0x7FFF).astype(np.uint16)
    x = mx.bf16_round(4 * mx.bf16_to_f32(x))
    t1, u1, t3, u3 = dev_u8(w1, device), dev_u8(s1, device), dev_u8(w3, device), dev_u8(s3, device)
    xd = dev_bf16(x, device)
    act = host_bits(fp8b.fp8_e4m3_swiglu_gemv(t1, u1, t3, u3, xd, 0.0, False)).reshape(T, N)
    gate = host_bits(fp8b.fp8_e4m3_gemv(t1, u1, xd)).reshape(T, N)
    up = host_bits(fp8b.fp8_e4m3_gemv(t3, u3, xd)).reshape(T, N)
    g = mx.bf16_to_f32(gate)
    assert g.min() >= 17.0, f"gate sums must be >= 17 for an exact SiLU, min {g.min()}"
    ref = mx.bf16_round((g * mx.bf16_to_f32(up)).astype(np.float32))
    assert np.array_equal(act, ref), f"{int(np.sum(act != ref))} outputs differ from bf16(gate * up)"


@pytest.mark.parametrize("N,K", [(1536, 4096), (576, 4096), (4096, 4096), (4096, 2048)])
@pytest.mark.parametrize("T", [1, 8])
def test_fp8_gemv_f32_scales_config_shapes(device, N, K, T):
    """fp8_e4m3_gemv_f32s at the benchmark's FP8 shapes with its literal scale
    format (one fp32 scale per 128x128 block, amax / 448): against the oracle's
    dequantise (fp32 product, bf16) then fp32 matmul."""
    announce(f"fp8_e4m3_gemv_f32s N={N} K={K} T={T}")
    w, s = synth.fp8_weight_f32s(17200 + N + K, N, K)
    x = synth.normal_bf16(17300 + T, (T, K))
    xd = dev_bf16(x, device)
    y = fp8b.fp8_e4m3_gemv_f32s(dev_u8(w, device), torch.from_numpy(s).to(device), xd[0] if T == 1 else xd)
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv_f32s(x, w, s), f"fp8 f32s N={N} K={K} T={T}")


@pytest.mark.parametrize("N,K,T,odd", [(1536, 4096, 1, False), (576, 4096, 8, False), (4096, 2048, 1, False),
                                       (200, 8192, 1, False), (130, 3200, 2, False), (50, 12288, 3, True),
                                       (45, 4096, 5, True)]
                         + [(200, K, T, False) for K in (1024, 2048, 4096) for T in (1, 2, 3, 5, 9)]
                         + [(90, K, T, odd) for K in (384, 1536, 2560) for T in (1, 2) for odd in (False, True)]
                         + [(70, 12288, 1, False)])
def test_fp8_gemv_f32_scales_equal_e8m0_bits(device, N, K, T, odd):
    """With fp32 scales equal to the E8M0 ones (2^(b-127)) the fp32-scale entry
    gives exactly the E8M0 entry's bits on the vector kernels: the tile kernel
    at K = 1024, 2048 and 4096 for the token groups of 1, 2 and 4 (T = 1, 2,
    3), at K = 4096 for those of 8 and 16 (T = 5, 9; at K = 1024 and 2048 these
    shapes take the matrix cores, and the far-apart-rows tests hold the vector
    kernels' 8- and 16-token groups there) and K = 8192 at T = 1, the general
    kernel with one to three 1 KiB chunks per lane and with segmented rows
    (K = 12288), aligned and unaligned. The scale format is the only
    difference."""
    announce(f"fp8_e4m3_gemv_f32s vs fp8_e4m3_gemv bits N={N} K={K} T={T} odd={odd}")
    w, sb = synth.fp8_weight(17400 + N + K + T, N, K)
    sf = np.ldexp(np.float32(1.0), sb.astype(np.int32) - 127).astype(np.float32)
    x = synth.normal_bf16(17500 + T, (T, K))
    xd = dev_bf16(x, device)
    xin = xd[0] if T == 1 else xd
    if odd:
        buf = torch.zeros(N, K + 1, dtype=torch.uint8, device=device)
        buf[:, :K] = dev_u8(w, device)
        tw = buf[:, :K]
    else:
        tw = dev_u8(w, device)
    a = host_bits(fp8b.fp8_e4m3_gemv_f32s(tw, torch.from_numpy(sf).to(device), xin))
    b = host_bits(fp8b.fp8_e4m3_gemv(tw, dev_u8(sb, device), xin))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("N,K,T", [(2048, 1024, 4), (16384, 1024, 8), (65536, 1024, 8), (4096, 2048, 3),
                                   (8192, 2048, 8), (32768, 2048, 8), (4096, 4096, 8), (8192, 4096, 8),
                                   (16384, 4096, 8), (4100, 8192, 2), (576, 6144, 8), (1000, 16384, 3),
                                   (100, 12800, 6), (300, 16384, 16), (4100, 6144, 8), (1000, 8192, 4), (2048, 8192, 6), (4100, 8192, 6)])
def test_fp8_gemv_f32_scales_matrix_cores_equal_e8m0_bits(device, N, K, T):
    """The fp32-scale entry takes the matrix cores by the E8M0 entry's rules:
    every row-block count R (1, 2, 4 at K = 1024, 2048, 4096; K = 8192) and
    every long-row kernel (two and four 512-k blocks per MFMA; one block per
    MFMA with 8 and 16 real rows per workgroup, 25 blocks leaving one wave a
    single block). With
    fp32 scales 2^(b-127) equal to the E8M0 bytes b the outputs are the same
    bits. Weights are filled on the device (finite E4M3 codes of both signs,
    scale bytes 119..125)."""
    from runtime import fill
    announce(f"fp8_e4m3_gemv_f32s vs fp8_e4m3_gemv bits on the matrix cores N={N} K={K} T={T}")
    w = torch.empty(N, K, dtype=torch.uint8, device=device)
    fill.fill_uniform_u8(w, 17600 + N + K + T, 0, 0, 255)
    w.bitwise_and_(0xF7)                      # even exponent fields: no 0x7F / 0xFF (NaN)
    sb = torch.empty((N + 127) // 128, K // 128, dtype=torch.uint8, device=device)
    fill.fill_uniform_u8(sb, 17700 + N + K + T, 0, 119, 125)
    sf = torch.ldexp(torch.ones(sb.shape, dtype=torch.float32, device=device), sb.to(torch.int32) - 127)
    xd = dev_bf16(synth.normal_bf16(17800 + T, (T, K)), device)
    a = host_bits(fp8b.fp8_e4m3_gemv_f32s(w, sf, xd))
    b = host_bits(fp8b.fp8_e4m3_gemv(w, sb, xd))
    assert np.isfinite(mx.bf16_to_f32(b)).all()
    assert np.array_equal(a, b), f"{int(np.sum(a != b))} outputs differ"
