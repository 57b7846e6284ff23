"""GPU parity of the four kernels (through the C ABI) against the CPU oracle.

Bar: dequantised weights bit-exact; outputs max rel err <= 1e-2 and cosine
>= 0.9999 against the oracle's dequant -> fp32 matmul -> bf16 path; integer
outputs (routing ids, residual sums) bit-exact. Sizes are those of the
benchmark configurations where the oracle finishes in seconds, smaller ones
for the exhaustive and edge cases.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mx
from runtime import fill, synth
from runtime import fp8_e4m3_gemv_binding as fp8b
from runtime import mxfp4_gemv_binding as mxb
from runtime import mxfp4_grouped_gemv_binding as gb
from runtime import rmsnorm_fuse_binding as rb
from tests.gpu_util import announce, assert_close, dev_bf16, dev_f32, dev_u8, host_bits

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ filler --

def test_device_fill_matches_numpy_generator(device):
    announce("dsv4_fill_uniform_u8 n=1000003 offset=77")
    t = torch.empty(1000003, dtype=torch.uint8, device=device)
    fill.fill_uniform_u8(t, 1234, 77)
    assert np.array_equal(t.cpu().numpy(), synth.uniform_u8(1234, 77, 1000003))
    s = torch.empty(4099, dtype=torch.uint8, device=device)
    fill.fill_uniform_u8(s, 99, 5, synth.SCALE_LO, synth.SCALE_HI)
    assert np.array_equal(s.cpu().numpy(), synth.uniform_u8(99, 5, 4099, 119, 125))


def test_read_floor_streams_without_writing(device):
    """The read-floor harness kernel (bench.py's `read_floor`): three launches
    rotating over two ranges of a ragged size (the last workgroup shorter)
    leave the source untouched and write nothing to the sink for fill data
    (it stores only when a thread's folded words hit one constant)."""
    announce("dsv4_read_floor 2 x 1000000 bytes, 3 launches, 1024 workgroups")
    n = 1_000_000
    src = torch.empty(2 * n, dtype=torch.uint8, device=device)
    fill.fill_uniform_u8(src, 4242)
    before = src.cpu().numpy().copy()
    sink = torch.zeros(1024 * 512, dtype=torch.int32, device=device)
    fill.read_floor(src, n, 1024, sink, rotate=2, launches=3)
    fill.read_floor(src, n, 300, sink, rotate=2, launches=2, threads=256)
    torch.cuda.synchronize()
    assert np.array_equal(src.cpu().numpy(), before)
    assert int(torch.count_nonzero(sink)) == 0
    with pytest.raises(RuntimeError):
        fill.read_floor(src, n - 8, 1024, sink)        # not a multiple of 16 bytes


# ----------------------------------------------------------------- dequant --

def test_mxfp4_dequant_exhaustive_bit_exact(device):
    """Every packed byte under every scale byte (0 -> 2^-127, 255 -> 0, 254 -> inf for code 6)."""
    announce("mxfp4_dequant_bf16 exhaustive 256x512")
    packed = np.tile(np.arange(256, dtype=np.uint8), (256, 1))
    scale = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)
    got = host_bits(mxb.mxfp4_dequant(dev_u8(packed, device), dev_u8(scale, device)))
    ref = mx.mxfp4_dequant_bf16(packed, scale, kernel_convention=True)
    assert np.array_equal(got, ref)


def test_mxfp4_dequant_config_weight_bit_exact(device):
    announce("mxfp4_dequant_bf16 cfg0 2048x4096 seed 1000")
    p, s = synth.mxfp4_weight(1000, 2048, 4096)
    got = host_bits(mxb.mxfp4_dequant(dev_u8(p[0], device), dev_u8(s[0], device)))
    assert np.array_equal(got, mx.mxfp4_dequant_bf16(p[0], s[0]))


def test_fp8_dequant_exhaustive_bit_exact(device):
    """All 256 E4M3FN bytes in every row, a distinct scale byte in each of 256 tiles."""
    announce("fp8_e4m3_dequant_bf16 exhaustive 2048x2048")
    w = np.tile(np.arange(256, dtype=np.uint8), (2048, 8))
    s = np.arange(256, dtype=np.uint8).reshape(16, 16)
    got = host_bits(fp8b.fp8_e4m3_dequant(dev_u8(w, device), dev_u8(s, device)))
    ref = mx.fp8_dequant_bf16(w, s, kernel_convention=True)
    gn = np.isnan(mx.bf16_to_f32(got))
    rn = np.isnan(mx.bf16_to_f32(ref))
    assert np.array_equal(gn, rn)
    assert np.array_equal(got[~gn], ref[~rn])


# ------------------------------------------------------------- MXFP4 GEMV --

@pytest.mark.parametrize("N,K", [(2048, 4096), (2047, 4096), (64, 32), (96, 96), (40, 2048),
                                 (33, 8192), (128, 6144), (1, 4096), (13, 2048)])
def test_mxfp4_gemv(device, N, K):
    announce(f"mxfp4_gemv_m1 N={N} K={K}")
    p, s = synth.mxfp4_weight(1000 + K, N, K)
    x = synth.normal_bf16(2000 + K, (K,))
    y = mxb.mxfp4_gemv(dev_u8(p[0], device), dev_u8(s[0], device), dev_bf16(x, device))
    assert_close(host_bits(y), mx.mxfp4_gemv(x, p[0], s[0]), f"mxfp4 N={N} K={K}")


def test_mxfp4_gemv_row_strides_and_unaligned(device):
    N, K = 300, 1024
    p, s = synth.mxfp4_weight(3001, N, K)
    x = synth.normal_bf16(3002, (K,))
    ref = mx.mxfp4_gemv(x, p[0], s[0])
    # rows inside wider buffers (caller strides), 16-byte aligned
    wide_p = np.zeros((N, K // 2 + 48), np.uint8)
    wide_p[:, :K // 2] = p[0]
    wide_s = np.zeros((N, K // 32 + 5), np.uint8)
    wide_s[:, :K // 32] = s[0]
    tp, ts = dev_u8(wide_p, device), dev_u8(wide_s, device)
    announce("mxfp4_gemv_m1 strided rows")
    y = mxb.mxfp4_gemv(tp[:, :K // 2], ts[:, :K // 32], dev_bf16(x, device))
    assert_close(host_bits(y), ref, "mxfp4 strided")
    # unaligned weight rows (offset 1 byte, odd stride) and unaligned activation
    odd_p = np.zeros((N, K // 2 + 1 + 7), np.uint8)
    odd_p[:, 1:1 + K // 2] = p[0]
    to = dev_u8(odd_p, device)
    xb = dev_bf16(np.concatenate([[0], x]).astype(np.uint16), device)
    announce("mxfp4_gemv_m1 unaligned rows and activation")
    y2 = mxb.mxfp4_gemv(to[:, 1:1 + K // 2], ts[:, :K // 32], xb[1:])
    assert_close(host_bits(y2), ref, "mxfp4 unaligned")


def test_mxfp4_gemv_one_hot_selects_column(device):
    announce("mxfp4_gemv_m1 one-hot 256x512")
    p, s = synth.mxfp4_weight(3003, 256, 512)
    deq = mx.bf16_to_f32(mx.mxfp4_dequant_bf16(p[0], s[0]))
    tp, ts = dev_u8(p[0], device), dev_u8(s[0], device)
    for k in (0, 33, 511):
        x = np.zeros(512, np.uint16)
        x[k] = 0x3F80
        got = mx.bf16_to_f32(host_bits(mxb.mxfp4_gemv(tp, ts, dev_bf16(x, device))))
        assert np.array_equal(got, deq[:, k])


# --------------------------------------------------------------- FP8 GEMV --

FP8_SHAPES = [(1536, 4096), (576, 4096), (4096, 4096), (4096, 2048)]


@pytest.mark.parametrize("N,K", FP8_SHAPES)
@pytest.mark.parametrize("T", [1, 8])
def test_fp8_gemv_config_shapes(device, N, K, T):
    announce(f"fp8_e4m3_gemv N={N} K={K} T={T}")
    w, s = synth.fp8_weight(1002 + N + K, N, K)
    x = synth.normal_bf16(2002 + T, (T, K))
    tw, ts = dev_u8(w, device), dev_u8(s, device)
    xt = dev_bf16(x, device)
    y = fp8b.fp8_e4m3_gemv(tw, ts, xt[0] if T == 1 else xt)
    ref = mx.fp8_gemv(x, w, s)
    assert_close(host_bits(y).reshape(T, N), ref, f"fp8 N={N} K={K} T={T}")


@pytest.mark.parametrize("N,K,T", [(130, 4096, 2), (77, 2048, 5), (300, 4096, 16), (1, 2048, 1),
                                   (9, 4096, 3)])
def test_fp8_gemv_tile_path_tokens_and_ragged_n(device, N, K, T):
    """The K in {2048, 4096} tile kernel: token counts padded to 2/4/8/16, rows
    not a multiple of the workgroup tile."""
    announce(f"fp8_e4m3_gemv tile N={N} K={K} T={T}")
    w, s = synth.fp8_weight(4100 + N + T, N, K)
    x = synth.normal_bf16(4200 + T, (T, K))
    xd = dev_bf16(x, device)
    y = fp8b.fp8_e4m3_gemv(dev_u8(w, device), dev_u8(s, device), xd if T > 1 else xd[0])
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 tile N={N} K={K} T={T}")


@pytest.mark.parametrize("N,K,T,odd_stride", [(77, 384, 1, False), (77, 384, 3, False), (130, 3200, 2, False),
                                              (64, 12288, 1, False), (50, 12288, 3, False),
                                              (33, 16384, 2, False), (140, 4096, 1, True),
                                              (45, 4096, 5, True), (20, 12288, 2, True)])
def test_fp8_gemv_general_path(device, N, K, T, odd_stride):
    """K off the tile set (a multiple of 128 up to the 16384 cap; rows longer
    than 4096 are walked in segments, once per group of 8 tokens) and weight
    rows at an odd byte stride (unaligned 16-byte loads): the general kernel,
    against the oracle. Aligned rows longer than 4096 at T >= 2 take the
    matrix cores (test_fp8_gemv_long_rows_matrix_cores)."""
    announce(f"fp8_e4m3_gemv general N={N} K={K} T={T} odd_stride={odd_stride}")
    w, s = synth.fp8_weight(4500 + N + K + T, N, K)
    x = synth.normal_bf16(4600 + T, (T, K))
    if odd_stride:
        buf = torch.zeros(N, K + 1, dtype=torch.uint8, device=device)
        buf[:, :K] = dev_u8(w, device)
        tw = buf[:, :K]
    else:
        tw = dev_u8(w, device)
    xd = dev_bf16(x, device)
    y = fp8b.fp8_e4m3_gemv(tw, dev_u8(s, device), xd if T > 1 else xd[0])
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 general N={N} K={K} T={T}")


@pytest.mark.parametrize("N,K,T", [(576, 6144, 8), (1536, 12288, 8), (64, 9216, 5), (4100, 5120, 4),
                                   (575, 6144, 4), (1000, 16384, 3), (300, 10240, 2),
                                   (200, 16384, 16), (130, 4608, 3), (300, 7680, 2), (100, 12800, 6),
                                   (4100, 6144, 8), (1000, 8192, 4), (2048, 8192, 2), (1000, 8192, 8)])
def test_fp8_gemv_long_rows_matrix_cores(device, N, K, T):
    """Aligned rows longer than the tile set (K a multiple of 512 above 4096,
    other than 8192) with several tokens, every branch of the long-row rule:
    two 512-k blocks per MFMA (T <= 8 at up to 2048 rows, K a multiple of
    1024), four per MFMA (T <= 4 at up to 1024 rows, K a multiple of 2048;
    575 rows: a ragged last workgroup), and one block per MFMA with 8 real
    rows per workgroup up to 2048 rows (T = 16, and block counts 9, 15 and 25
    that neither split divides, the last leaving one wave a single block) or
    16 above (4100 rows at T = 4 and 8). K = 8192, a tile shape, joins them
    at up to 2048 rows (1000 rows at T = 4 and 8, 2048 rows at T = 2). Each
    weight byte is read once for all tokens; against the oracle."""
    announce(f"fp8_e4m3_gemv long rows on the matrix cores N={N} K={K} T={T}")
    w, s = synth.fp8_weight(4700 + N + K + T, N, K)
    x = synth.normal_bf16(4800 + T, (T, K))
    y = fp8b.fp8_e4m3_gemv(dev_u8(w, device), dev_u8(s, device), dev_bf16(x, device))
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 long N={N} K={K} T={T}")


@pytest.mark.parametrize("T", [8, 16])
def test_fp8_gemv_long_rows_general_token_groups(device, T):
    """Rows longer than 4096 at an odd byte stride (the general kernel's
    segmented body): each segment is loaded once per group of 8 tokens; T = 16
    takes two groups. Against the oracle, and equal to the aligned rows'
    matrix-core result within the tolerance."""
    N, K = 96, 12288
    announce(f"fp8_e4m3_gemv general long rows N={N} K={K} T={T} odd stride")
    w, s = synth.fp8_weight(4900 + T, N, K)
    x = synth.normal_bf16(4950 + T, (T, K))
    buf = torch.zeros(N, K + 1, dtype=torch.uint8, device=device)
    buf[:, :K] = dev_u8(w, device)
    y = fp8b.fp8_e4m3_gemv(buf[:, :K], dev_u8(s, device), dev_bf16(x, device))
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 general long T={T}")


def test_fp8_gemv_long_rows_and_ragged_n(device):
    N, K, T = 200, 8192, 3
    announce(f"fp8_e4m3_gemv N={N} K={K} T={T} (K = 8192 on the tile path)")
    w, s = synth.fp8_weight(4001, N, K)
    x = synth.normal_bf16(4002, (T, K))
    y = fp8b.fp8_e4m3_gemv(dev_u8(w, device), dev_u8(s, device), dev_bf16(x, device))
    assert_close(host_bits(y), mx.fp8_gemv(x, w, s), "fp8 K=8192")


@pytest.mark.parametrize("G,N,K,T", [(8, 1024, 4096, 1), (8, 1024, 4096, 3), (8, 1024, 4096, 16), (3, 576, 2048, 2),
                                     (4, 64, 4096, 1), (2, 200, 1024, 2), (3, 100, 6144, 4), (2, 130, 12288, 8),
                                     (2, 2100, 5120, 8), (2, 60, 7680, 16), (2, 700, 4096, 6)])
def test_fp8_gemv_grouped(device, G, N, K, T):
    """G GEMVs in one launch (the wo_a shape G=8, N=1024, K=4096 first): against
    the oracle, and, for 128-row groups at T = 1 (where a group and a single
    GEMV on its slice both take the vector tile kernel), bit for bit against
    one fp8_e4m3_gemv call per group. At T = 3 the wo_a shape takes the
    matrix cores (its path rule counts all 8,192 rows). N=576 and N=64 put
    group boundaries inside a scale tile. Rows longer than 4096 take the
    long-row kernels per group: four and two 512-k blocks per MFMA (G=3,
    N=100, T=4; G=2, N=130, T=8), one block with 16 real rows once the groups
    hold more than 2048 rows (G=2, N=2100, T=8) and with 8 (15 blocks, T=16).
    K = 4096 below 3072 rows at T = 5 .. 8 takes two blocks per MFMA as well
    (G=2, N=700, T=6)."""
    announce(f"fp8_e4m3_gemv_grouped G={G} N={N} K={K} T={T}")
    w, s = synth.fp8_weight(4300 + G + N, G * N, K)
    x = synth.normal_bf16(4400 + T, (T, G, K))
    tw, ts = dev_u8(w, device), dev_u8(s, device)
    xd = dev_bf16(x, device)
    y = fp8b.fp8_e4m3_gemv_grouped(tw, ts, xd if T > 1 else xd[0], G)
    got = host_bits(y).reshape(T, G, N)
    assert_close(got.reshape(T, -1), mx.fp8_gemv_grouped(x, w, s, G).reshape(T, -1), f"fp8 grouped G={G}")
    if N % 128 == 0 and K in (2048, 4096) and T == 1:
        for g in range(G):
            yg = fp8b.fp8_e4m3_gemv(tw[g * N:(g + 1) * N], ts[g * N // 128:(g + 1) * N // 128],
                                    xd[:, g].contiguous() if T > 1 else xd[0, g].contiguous())
            assert np.array_equal(host_bits(yg).reshape(T, N), got[:, g]), f"group {g}"


@pytest.mark.parametrize("N,K,T,clamp_up", [(2048, 4096, 1, True), (2048, 4096, 1, False),
                                            (2048, 4096, 5, True), (2048, 4096, 16, False),
                                            (300, 2048, 3, True)])
def test_fp8_swiglu_gemv(device, N, K, T, clamp_up):
    """The shared expert's gate + up + SwiGLU in one launch (N=2048, K=4096):
    gate and up are the bits of the two single GEMVs, the clamp at 10 is
    exercised (activations scaled so some gate and up values pass it), and the
    result matches the oracle."""
    announce(f"fp8_e4m3_swiglu_gemv N={N} K={K} T={T} clamp_up={clamp_up}")
    w1, s1 = synth.fp8_weight(4500 + N, N, K)
    w3, s3 = synth.fp8_weight(4600 + N, N, K)
    x = mx.bf16_round(24 * mx.bf16_to_f32(synth.normal_bf16(4700 + T, (T, K))))
    t1, u1, t3, u3 = dev_u8(w1, device), dev_u8(s1, device), dev_u8(w3, device), dev_u8(s3, device)
    xd = dev_bf16(x, device)
    act = host_bits(fp8b.fp8_e4m3_swiglu_gemv(t1, u1, t3, u3, xd if T > 1 else xd[0], 10.0, clamp_up))
    act = act.reshape(T, N)
    gate = host_bits(fp8b.fp8_e4m3_gemv(t1, u1, xd if T > 1 else xd[0])).reshape(T, N)
    up = host_bits(fp8b.fp8_e4m3_gemv(t3, u3, xd if T > 1 else xd[0])).reshape(T, N)
    assert np.abs(mx.bf16_to_f32(gate)).max() > 10 and np.abs(mx.bf16_to_f32(up)).max() > 10
    # the epilogue on the single GEMVs' bits: equal up to expf's last bit
    ref_bits = mx.swiglu_clamped(gate, up, 10.0, clamp_up)
    diff = np.abs(act.astype(np.int32) - ref_bits.astype(np.int32))
    diff[mx.bf16_to_f32(act) == mx.bf16_to_f32(ref_bits)] = 0  # +0 and -0
    assert diff.max() <= 1, f"max bf16 ulp difference {diff.max()}"
    assert_close(act, mx.fp8_swiglu(x, w1, s1, w3, s3, 10.0, clamp_up), f"fp8 swiglu T={T}")


@pytest.mark.parametrize("N,K,T,resid", [(1536, 4096, 1, True), (576, 4096, 1, False), (300, 2048, 3, True),
                                         (4096, 4096, 4, True), (77, 2048, 2, False)])
def test_fp8_rmsnorm_gemv(device, N, K, T, resid):
    """RMSNorm (+ residual) folded into the FP8 GEMV: x_norm and new_residual
    are the bits of the RMSNorm library, y the bits of fp8_e4m3_gemv on x_norm,
    and all match the oracle."""
    announce(f"fp8_e4m3_rmsnorm_gemv N={N} K={K} T={T} residual={resid}")
    w, s = synth.fp8_weight(4800 + N, N, K)
    h = synth.normal_bf16(4801 + T, (T, K))
    r = synth.normal_bf16(4802 + T, (T, K), 0.0, 0.5)
    g = synth.normal_bf16(4803, (K,), 1.0, 0.1)
    tw, ts = dev_u8(w, device), dev_u8(s, device)
    hd, rd, gd = dev_bf16(h, device), dev_bf16(r, device), dev_bf16(g, device)
    y, xn, nr = fp8b.fp8_e4m3_rmsnorm_gemv(tw, ts, hd if T > 1 else hd[0], gd,
                                           (rd if T > 1 else rd[0]) if resid else None)
    if resid:
        ref_xn, ref_nr = rb.rmsnorm_fuse_residual_add(hd, rd, gd)
        assert np.array_equal(host_bits(nr).reshape(T, K), host_bits(ref_nr)), "new_residual bits"
        oracle_xn, oracle_nr = mx.rmsnorm_residual(h, r, g)
        assert np.array_equal(host_bits(nr).reshape(T, K), oracle_nr)
    else:
        ref_xn = rb.rmsnorm_fuse_fwd(hd, gd)
        oracle_xn = mx.rmsnorm(h, g)
    assert np.array_equal(host_bits(xn).reshape(T, K), host_bits(ref_xn)), "x_norm bits"
    ref_y = fp8b.fp8_e4m3_gemv(tw, ts, ref_xn if T > 1 else ref_xn.view(-1))
    assert np.array_equal(host_bits(y).reshape(T, N), host_bits(ref_y).reshape(T, N)), "y bits"
    assert_close(host_bits(xn).reshape(T, K), oracle_xn, "x_norm vs oracle")
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(oracle_xn, w, s), "y vs oracle")


# ------------------------------------------------------ grouped (drop-in) --

def _packed_experts(seed, n, K, H, O):
    W1p, W1s = synth.mxfp4_weight(seed, H, K, n)
    W3p, W3s = synth.mxfp4_weight(seed + 4, H, K, n)
    W2p, W2s = synth.mxfp4_weight(seed + 8, O, H, n)
    return W1p, W3p, W2p, W1s, W3s, W2s


def _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s):
    return ({"packed": dev_u8(W1p, device), "scale": dev_u8(W1s, device)},
            {"packed": dev_u8(W3p, device), "scale": dev_u8(W3s, device)},
            {"packed": dev_u8(W2p, device), "scale": dev_u8(W2s, device)})


@pytest.mark.parametrize("n_exp,K,H,O", [(8, 4096, 2048, 4096), (6, 4096, 2048, 4096),
                                         (1, 4096, 2048, 4096), (3, 1024, 96, 200)])
def test_grouped_gemv_topk(device, n_exp, K, H, O):
    announce(f"mxfp4_grouped_gemv_topk n_exp={n_exp} K={K} H={H} O={O}")
    mats = _packed_experts(5000 + n_exp, n_exp, K, H, O)
    x = synth.normal_bf16(5100 + n_exp, (K,))
    r = synth.normal_f64(5200 + n_exp, 0, n_exp)
    r = (1 / (1 + np.exp(-r)))
    r = (r / r.sum()).astype(np.float32)
    W1, W3, W2 = _dev_mats(device, *mats)
    out = gb.mxfp4_grouped_gemv(W1, W3, W2, None, dev_bf16(x, device), dev_f32(r, device))
    ref = mx.grouped_gemv_topk(x, *mats, r)
    got = host_bits(out)
    assert_close(got, ref, f"grouped n_exp={n_exp}")
    # deterministic: a second call is bit-identical
    out2 = gb.mxfp4_grouped_gemv(W1, W3, W2, None, dev_bf16(x, device), dev_f32(r, device))
    assert np.array_equal(host_bits(out2), got)


def test_grouped_gemv_invariants(device):
    n, K, H, O = 8, 4096, 2048, 4096
    mats = _packed_experts(6000, n, K, H, O)
    x = dev_bf16(synth.normal_bf16(6001, (K,)), device)
    r = np.linspace(0.05, 0.2, n).astype(np.float32)
    W1, W3, W2 = _dev_mats(device, *mats)
    announce("mxfp4_grouped_gemv_topk invariants: zero weights, permutation")
    zero = gb.mxfp4_grouped_gemv(W1, W3, W2, None, x, torch.zeros(n, device=device))
    assert np.all(mx.bf16_to_f32(host_bits(zero)) == 0)
    base = host_bits(gb.mxfp4_grouped_gemv(W1, W3, W2, None, x, dev_f32(r, device)))
    perm = torch.tensor([3, 7, 0, 5, 1, 6, 2, 4], device=device)
    Wp = [{k: w[k][perm].contiguous() for k in ("packed", "scale")} for w in (W1, W3, W2)]
    permuted = host_bits(gb.mxfp4_grouped_gemv(*Wp[:2], Wp[2], None, x,
                                               dev_f32(r, device)[perm].contiguous()))
    assert_close(permuted, base, "grouped permuted experts", cos_tol=0.99999)


# --------------------------------------------------- expert-indexed MoE -----

def test_route_sigmoid_topk(device):
    announce("mxfp4_moe_route_sigmoid_topk T=16 E=256 k=8")
    logits = synth.gating_logits(7001, 16, 256)
    ids, w = gb.route_sigmoid_topk(dev_f32(logits, device), 8)
    rids, rw = mx.route_sigmoid_topk(logits, 8)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-6)


def _gating_edge_logits():
    """Logit sets with equal values, signed zeros, -inf, NaN and expert counts
    that are not multiples of 64 (the wave holds 4, 8 or 16 logits per lane)."""
    rng = np.random.default_rng(7100)
    cases = []
    cases.append(("halves", np.round(rng.standard_normal((4, 256)) * 2) / 2, 8))
    z = np.zeros((2, 256), dtype=np.float32)
    z[:, ::3] = -0.0
    z[0, [7, 90, 200]] = [1.0, 2.0, 1.0]
    z[1, 250] = -1.0
    cases.append(("signed zeros", z, 8))
    ni = np.full((2, 256), -np.inf, dtype=np.float32)
    ni[0, [3, 77, 130]] = [0.5, -2.0, 0.5]
    cases.append(("minus inf", ni, 8))
    na = rng.standard_normal((2, 256)).astype(np.float32)
    na[:, 1::4] = np.nan
    cases.append(("nan entries", na, 8))
    cases.append(("E=200 k=16", rng.standard_normal((3, 200)), 16))
    cases.append(("E=300 k=5", rng.standard_normal((3, 300)), 5))
    cases.append(("E=1024 k=8", np.round(rng.standard_normal((2, 1024)) * 4) / 4, 8))
    cases.append(("E=8 k=8", rng.standard_normal((2, 8)), 8))
    return cases


@pytest.mark.parametrize("name,logits,k", _gating_edge_logits(), ids=lambda v: v if isinstance(v, str) else "")
def test_route_sigmoid_topk_edges(device, name, logits, k):
    """Ties go to the lower expert index, -0 equals +0, NaN ranks as -inf (the
    NaN case keeps enough finite logits that no NaN is picked, where the
    oracle's ordering of NaN below -inf would differ)."""
    logits = np.asarray(logits, dtype=np.float32)
    announce(f"mxfp4_moe_route_sigmoid_topk edge case {name} E={logits.shape[1]} k={k}")
    ids, w = gb.route_sigmoid_topk(dev_f32(logits, device), k)
    rids, rw = mx.route_sigmoid_topk(logits, k)
    assert np.array_equal(ids.cpu().numpy(), rids), name
    # a token whose logits are all -inf gets 0/0 weights in both
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-6, equal_nan=True), name


@pytest.mark.parametrize("name,logits,k", _gating_edge_logits(), ids=lambda v: v if isinstance(v, str) else "")
def test_moe_layer_one_token_gating_edges(device, name, logits, k):
    """The one-token layer ranks the logits inside stage A: every wave of every
    workgroup ranks them itself and stops after the pick its workgroup serves,
    and one wave ranks all k and publishes ids, weights and stage B's tables.
    On the edge sets each row, as a one-token call, must give the oracle's ids
    and weights, and the layer output must match the oracle on those ids."""
    logits = np.asarray(logits, dtype=np.float32)
    E = logits.shape[1]
    K, H, O = 2048, (32 if E > 256 else 64), 128        # K = 2048: the one-token kernel's shape
    announce(f"mxfp4_moe_layer one-token gating edge case {name} E={E} k={k} K={K} H={H} O={O}")
    mats = _packed_experts(9700 + E, E, K, H, O)
    W1p, W3p, W2p, W1s, W3s, W2s = mats
    W1, W3, W2 = _dev_mats(device, *mats)

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    for t in range(logits.shape[0]):
        x = synth.normal_bf16(9800 + t, (1, K))
        ids_out = torch.empty(1, k, dtype=torch.int32, device=device)
        w_out = torch.empty(1, k, dtype=torch.float32, device=device)
        out = gb.mxfp4_moe_layer(dev_bf16(x, device), dev_f32(logits[t:t + 1], device), W1, W3, W2, k,
                                 ids_out=ids_out, weights_out=w_out)
        rids, rw = mx.route_sigmoid_topk(logits[t:t + 1], k)
        assert np.array_equal(ids_out.cpu().numpy(), rids), f"{name} row {t}"
        # a row whose logits are all -inf gets 0/0 weights in both; its output is not compared
        assert np.allclose(w_out.cpu().numpy(), rw, rtol=1e-5, atol=1e-6, equal_nan=True), f"{name} row {t}"
        if np.all(np.isfinite(rw)):
            assert_close(host_bits(out), mx.moe_layer(x, fn, rids, rw, O, n_experts=E), f"{name} row {t}")


@pytest.mark.parametrize("T", [1, 4, 16])
def test_moe_indexed_small_dims(device, T):
    """All T of the config at reduced K/H/O so the oracle covers every expert quickly."""
    E, K, H, O, topk = 256, 512, 256, 384, 8
    announce(f"mxfp4_moe_grouped_gemv T={T} E={E} K={K} H={H} O={O}")
    W1p, W1s = synth.mxfp4_weight(8000, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8004, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8008, O, H, E)
    x = synth.normal_bf16(8100 + T, (T, K))
    ids, w = mx.route_sigmoid_topk(synth.gating_logits(8200 + T, T, E), topk)
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    out = gb.mxfp4_moe_grouped_gemv(dev_bf16(x, device), W1, W3, W2,
                                    torch.from_numpy(ids).to(device), dev_f32(w, device))

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    assert_close(host_bits(out), mx.moe_layer(x, fn, ids, w, O), f"moe T={T}")


def test_moe_duplicate_and_out_of_range_ids(device):
    """A token listing one expert twice gets both contributions; ids outside
    [0, n_experts) (negative or too large) contribute nothing."""
    E, K, H, O, T, topk = 16, 512, 128, 256, 3, 4
    announce(f"mxfp4_moe_grouped_gemv duplicate/invalid ids T={T} E={E}")
    W1p, W1s = synth.mxfp4_weight(8300, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8304, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8308, O, H, E)
    x = synth.normal_bf16(8310, (T, K))
    ids = np.array([[3, 3, 5, 15], [-1, 2, 16, 2], [7, 1000, 0, 7]], np.int32)
    w = np.array([[0.4, 0.3, 0.2, 0.1], [0.5, 0.25, 0.15, 0.1], [0.6, 0.2, 0.1, 0.1]], np.float32)
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    out = gb.mxfp4_moe_grouped_gemv(dev_bf16(x, device), W1, W3, W2,
                                    torch.from_numpy(ids).to(device), dev_f32(w, device))

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    ref = mx.moe_layer(x, fn, ids, w, O, n_experts=E)
    assert_close(host_bits(out), ref, "moe duplicate/invalid ids")
    # the duplicate listing equals one listing with the summed weight
    ids1 = np.array([[3, 5, 15, 15]], np.int32)
    w1 = np.array([[0.7, 0.2, 0.1, 0.0]], np.float32)
    out1 = gb.mxfp4_moe_grouped_gemv(dev_bf16(x[:1], device), W1, W3, W2,
                                     torch.from_numpy(ids1).to(device), dev_f32(w1, device))
    assert_close(host_bits(out1), host_bits(out)[:1], "duplicate merge", cos_tol=0.99999)


@pytest.mark.parametrize("K", [2048, 4096])
@pytest.mark.parametrize("ids_row", [[3, 5, 1, 7, 12, 0, 9, 14], [3, 3, 5, 15, 3, 8, 8, 1],
                                     [-1, 2, 16, 2, 1000, -7, 4, 2], [6, 6, 6, 6, 6, 6, 6, 6]],
                         ids=["distinct", "duplicates", "invalid-and-duplicates", "one-expert"])
def test_moe_one_token_ids_path(device, ids_row, K):
    """At T = 1 mxfp4_moe_grouped_gemv forms the routing inside stage A (two
    launches). Its slots (distinct in-range ids, ascending, summed weights of
    repeated listings) and results must equal the routing kernel's path
    (build_routing + swiglu + down) bit for bit, and the oracle. K = 2048 and
    4096 are the one-token kernel's two instantiations (one or two MX blocks
    per lane per row); 4096 is the configuration's."""
    E, H, O, topk = 16, 256, 256, 8
    announce(f"mxfp4_moe_grouped_gemv T=1 ids path K={K} {ids_row}")
    W1p, W1s = synth.mxfp4_weight(8400, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8404, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8408, O, H, E)
    x = synth.normal_bf16(8410, (1, K))
    ids = np.array([ids_row], np.int32)
    w = (np.arange(1, topk + 1, dtype=np.float32) / 36.0).reshape(1, topk)
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    ids_d, w_d, x_d = torch.from_numpy(ids).to(device), dev_f32(w, device), dev_bf16(x, device)
    out = host_bits(gb.mxfp4_moe_grouped_gemv(x_d, W1, W3, W2, ids_d, w_d))
    st = gb.MoEStages(W1, W3, W2, 1, topk, device)
    st.build_routing(ids_d, w_d)
    st.swiglu(x_d)
    ref_path = host_bits(st.down(torch.empty(1, O, dtype=torch.bfloat16, device=device)))
    assert np.array_equal(out, ref_path), "T=1 ids path differs from the routing-kernel path"

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    assert_close(out, mx.moe_layer(x, fn, ids, w, O, n_experts=E), "T=1 ids path vs oracle")


@pytest.mark.parametrize("K,routing", [(2048, "random"), (4096, "random"), (4096, "shared"),
                                       (2048, "ragged")])
def test_moe_multi_token_many_pairs_per_expert(device, K, routing):
    """Several tokens on the aligned path (K = 2048 or 4096, hidden = 2048) with
    16 experts, so each expert serves many tokens: the multi-token stage A
    stages the pairs after the first in passes, and the multi-token stage B
    loads their M slices on demand. "shared": every token routes to the same
    8 experts (16 pairs each); "ragged": 1 to 16 pairs per expert."""
    E, H, O, T, topk = 16, 2048, 256, 16, 8
    announce(f"mxfp4_moe_grouped_gemv T={T} E={E} K={K} routing={routing}")
    W1p, W1s = synth.mxfp4_weight(8500, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8504, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8508, O, H, E)
    x = synth.normal_bf16(8510 + K, (T, K))
    if routing == "random":
        ids, w = mx.route_sigmoid_topk(synth.gating_logits(8520 + K, T, E), topk)
    else:
        if routing == "shared":
            ids = np.tile(np.array([2, 5, 7, 11, 0, 15, 9, 4], np.int32), (T, 1))
        else:  # expert e < 8 taken by tokens t >= 2e, the rest fill each row
            ids = np.zeros((T, topk), np.int32)
            for t in range(T):
                hot = [e for e in range(8) if t >= 2 * e]
                cold = [8 + (t + i) % 8 for i in range(topk - len(hot))]
                ids[t] = hot + cold
        rng = np.random.default_rng(8530)
        w = rng.random((T, topk)).astype(np.float32)
        w /= w.sum(1, keepdims=True)
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    out = gb.mxfp4_moe_grouped_gemv(dev_bf16(x, device), W1, W3, W2,
                                    torch.from_numpy(ids).to(device), dev_f32(w, device))

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    assert_close(host_bits(out), mx.moe_layer(x, fn, ids, w, O), f"moe T={T} K={K} {routing}")


@pytest.mark.parametrize("T", [1, 4])
def test_moe_indexed_config_dims(device, T):
    """Config-3 shapes (256 experts, K=4096, H=2048, O=4096) with device-filled weights."""
    from runtime import moe

    E, K, H, O = 256, 4096, 2048, 4096
    announce(f"RoutedMoELayer T={T} E={E} (device-filled weights)")
    weights = moe.make_moe_weights(9000, E, K, H, O, device)
    layer = moe.RoutedMoELayer(weights, topk=8, max_tokens=16)
    x = synth.normal_bf16(9100 + T, (T, K))
    logits = synth.gating_logits(9200 + T, T, E)
    out = layer.forward(dev_bf16(x, device), logits=dev_f32(logits, device))
    ids = layer.ids[:T].cpu().numpy()
    w = layer.weights[:T].cpu().numpy()
    rids, rw = mx.route_sigmoid_topk(logits, 8)
    assert np.array_equal(ids, rids)

    def fn(e):
        # host copy of the device-filled expert (same bytes as the seeded generator)
        mats = []
        for m in (weights.W1, weights.W3, weights.W2):
            mats.append((m["packed"][e].cpu().numpy(), m["scale"][e].cpu().numpy()))
        return tuple(mats)

    if T == 1:  # the generator regenerates an expert on the host byte for byte
        e0 = int(ids[0, 0])
        h = moe.expert_host_weights(9000, e0, K, H, O)
        d = fn(e0)
        for (hp, hs), (dp, ds) in zip(h, d):
            assert np.array_equal(hp, dp) and np.array_equal(hs, ds)
    assert_close(host_bits(out), mx.moe_layer(x, fn, ids, w, O), f"moe cfg3 T={T}")
    del layer, weights
    torch.cuda.empty_cache()


def test_moe_indexed_equals_packed_dropin(device):
    """Full-size T=16 (configuration 3): three tokens' rows against the
    oracle directly, and each token's row equal to the drop-in call on its
    packed experts."""
    from runtime import moe

    E, K, H, O, T = 256, 4096, 2048, 4096, 16
    announce(f"mxfp4_moe_grouped_gemv vs oracle and mxfp4_grouped_gemv_topk T={T}")
    weights = moe.make_moe_weights(9500, E, K, H, O, device)
    layer = moe.RoutedMoELayer(weights, topk=8, max_tokens=16)
    xh = synth.normal_bf16(9600, (T, K))
    x = dev_bf16(xh, device)
    lh = synth.gating_logits(9601, T, E)
    logits = dev_f32(lh, device)
    out = host_bits(layer.forward(x, logits=logits))
    ids_h = layer.ids[:T].cpu().numpy()
    w_h = layer.weights[:T].cpu().numpy()
    rids, _ = mx.route_sigmoid_topk(lh, 8)
    assert np.array_equal(ids_h, rids)
    cache = {}

    def fn(e):
        if e not in cache:
            cache[e] = tuple((m["packed"][e].cpu().numpy(), m["scale"][e].cpu().numpy())
                             for m in (weights.W1, weights.W3, weights.W2))
        return cache[e]

    sel = [0, 7, 15]
    ref = mx.moe_layer(xh[sel], fn, ids_h[sel], w_h[sel], O)
    for i, t in enumerate(sel):
        assert_close(out[t], ref[i], f"T=16 token {t} vs the oracle")
    cache.clear()
    ids = layer.ids[:T].long()
    for t in range(T):
        sel = ids[t]
        W = [{k: m[k][sel].contiguous() for k in ("packed", "scale")}
             for m in (weights.W1, weights.W3, weights.W2)]
        ref = host_bits(gb.mxfp4_grouped_gemv(W[0], W[1], W[2], None, x[t].contiguous(),
                                              layer.weights[t].contiguous()))
        assert_close(out[t], ref, f"token {t}", cos_tol=0.99999)
    del layer, weights
    torch.cuda.empty_cache()


# ------------------------------------------------------- prefill (MFMA) ---

@pytest.mark.parametrize("T,topk,E", [(100, 4, 16), (7, 8, 8), (130, 2, 64), (1024, 8, 32), (1100, 8, 16)])
def test_moe_prefill_small_vs_oracle(device, T, topk, E):
    """MFMA prefill path against the oracle at small dims, including a
    duplicate id in a token and ids outside [0, n_experts). The routing keeps
    up to 8,192 entries in registers (1024 x 8 is the largest such chunk) and
    goes through memory above that (1100 x 8)."""
    K, H, O = 512, 512, 384
    announce(f"mxfp4_moe_prefill T={T} topk={topk} E={E} K={K} H={H} O={O}")
    W1p, W1s = synth.mxfp4_weight(8400 + E, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8404 + E, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8408 + E, O, H, E)
    x = synth.normal_bf16(8410 + T, (T, K))
    ids, w = mx.route_sigmoid_topk(synth.gating_logits(8420 + T, T, E), topk)
    ids = ids.copy()
    if topk >= 2:
        ids[0, 1] = ids[0, 0]          # duplicate listing
    ids[T - 1, 0] = -1                 # dropped
    ids[T // 2, topk - 1] = E + 3      # dropped
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    out = gb.mxfp4_moe_prefill(dev_bf16(x, device), W1, W3, W2,
                               torch.from_numpy(ids).to(device), dev_f32(w, device))

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    assert_close(host_bits(out), mx.moe_layer(x, fn, ids, w, O, n_experts=E), f"prefill T={T}")
    again = gb.mxfp4_moe_prefill(dev_bf16(x, device), W1, W3, W2,
                                 torch.from_numpy(ids).to(device), dev_f32(w, device))
    assert np.array_equal(host_bits(again), host_bits(out))   # deterministic


@pytest.mark.parametrize("K,H,O,T,topk,E", [(1024, 1024, 512, 40, 4, 16), (2048, 1024, 768, 40, 6, 24),
                                             (4096, 2048, 256, 48, 8, 32), (8192, 512, 256, 40, 4, 16),
                                             (1024, 8192, 256, 40, 4, 16), (1024, 4096, 256, 40, 4, 16)])
def test_moe_prefill_mixed_tiles(device, K, H, O, T, topk, E):
    """The prefill at K = 2048 and 4096 (the unrolled 16- and 32-super-step
    bodies) and 1024 (the rolled body), stage B at hidden = 2048 and 4096
    (unrolled), and at the reduction cap 8192 on either side (K_in = 8192:
    rolled stage A with the largest scale tile; hidden = 8192: rolled stage
    B), with one expert of more than 16 pairs
    (a tile of two or three token blocks) beside one-block tiles: against the oracle,
    deterministic, with a dropped id and a duplicate listing."""
    announce(f"mxfp4_moe_prefill mixed tiles T={T} topk={topk} E={E} K={K} H={H} O={O}")
    W1p, W1s = synth.mxfp4_weight(8500 + K + E, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8504 + K + E, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8508 + K + E, O, H, E)
    x = synth.normal_bf16(8510 + T, (T, K))
    ids, w = mx.route_sigmoid_topk(synth.gating_logits(8520 + T, T, E), topk)
    ids = ids.copy()
    ids[0, 1] = ids[0, 0]
    ids[T - 1, 0] = -1
    ids[:T // 2, 0] = 3                # one expert with more than 16 pairs
    counts = np.bincount(ids[ids >= 0].ravel(), minlength=E)
    assert (counts > 16).any() and ((counts >= 1) & (counts <= 16)).any()
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    xd, idd, wd = dev_bf16(x, device), torch.from_numpy(ids).to(device), dev_f32(w, device)
    out = host_bits(gb.mxfp4_moe_prefill(xd, W1, W3, W2, idd, wd))

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    assert_close(out, mx.moe_layer(x, fn, ids, w, O, n_experts=E), f"prefill mixed tiles K={K}")
    assert np.array_equal(host_bits(gb.mxfp4_moe_prefill(xd, W1, W3, W2, idd, wd)), out)


@pytest.mark.parametrize("T", [1, 4])
def test_moe_special_scale_bytes_decode(device, T):
    """The decode kernels (one-token and multi-token paths, K = 2048) with E8M0
    0xFF (decoded as 0) and 0 (2^-127) in some blocks of every matrix, against
    the oracle's kernel convention."""
    E, K, H, O, topk = 16, 2048, 256, 384, 8
    announce(f"mxfp4_moe_grouped_gemv special scale bytes T={T} E={E} K={K}")
    W1p, W1s = synth.mxfp4_weight(8720, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8724, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8728, O, H, E)
    rng = np.random.default_rng(8730)
    for s in (W1s, W3s, W2s):
        u = rng.random(s.shape)
        s[u < 0.03] = 0xFF
        s[(u >= 0.03) & (u < 0.06)] = 0
    x = synth.normal_bf16(8731 + T, (T, K))
    ids, w = mx.route_sigmoid_topk(synth.gating_logits(8732 + T, T, E), topk)
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    out = gb.mxfp4_moe_grouped_gemv(dev_bf16(x, device), W1, W3, W2,
                                    torch.from_numpy(ids).to(device), dev_f32(w, device))

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    assert_close(host_bits(out), mx.moe_layer(x, fn, ids, w, O, n_experts=E), f"special scales T={T}")


def test_moe_prefill_special_scale_bytes(device):
    """E8M0 0xFF (the kernels' zero) and 0 (2^-127, an fp32 subnormal) in some
    blocks of every matrix: the prefill path must still match the oracle (which
    keeps byte 0 as 2^-127; the blocks it affects contribute below the
    tolerance) and the decode path on the same inputs."""
    E, K, H, O, T, topk = 8, 512, 512, 384, 40, 4
    announce(f"mxfp4_moe_prefill special scale bytes T={T} topk={topk} E={E}")
    W1p, W1s = synth.mxfp4_weight(8700, H, K, E)
    W3p, W3s = synth.mxfp4_weight(8704, H, K, E)
    W2p, W2s = synth.mxfp4_weight(8708, O, H, E)
    rng = np.random.default_rng(8710)
    for s in (W1s, W3s, W2s):
        u = rng.random(s.shape)
        s[u < 0.03] = 0xFF
        s[(u >= 0.03) & (u < 0.06)] = 0
    x = synth.normal_bf16(8711, (T, K))
    ids, w = mx.route_sigmoid_topk(synth.gating_logits(8712, T, E), topk)
    W1, W3, W2 = _dev_mats(device, W1p, W3p, W2p, W1s, W3s, W2s)
    xd, idd, wd = dev_bf16(x, device), torch.from_numpy(ids).to(device), dev_f32(w, device)
    out = host_bits(gb.mxfp4_moe_prefill(xd, W1, W3, W2, idd, wd))

    def fn(e):
        return (W1p[e], W1s[e]), (W3p[e], W3s[e]), (W2p[e], W2s[e])

    assert_close(out, mx.moe_layer(x, fn, ids, w, O, n_experts=E), "prefill special scales vs oracle")
    dec = host_bits(gb.mxfp4_moe_grouped_gemv(xd[:16], W1, W3, W2, idd[:16], wd[:16]))
    assert_close(out[:16], dec, "prefill special scales vs decode path", cos_tol=0.99999)


def test_moe_prefill_config_chunk(device):
    """configs[4] prefill chunk: 512 tokens, top-8 of 256 experts with Zipf
    routing, full dims. Checked token by token against the oracle-checked
    decode path (64-token calls of mxfp4_moe_grouped_gemv) and, for two
    tokens, against the oracle itself."""
    from runtime import moe

    E, K, H, O, T, topk = 256, 4096, 2048, 4096, 512, 8
    announce(f"mxfp4_moe_prefill T={T} E={E} (configs[4] chunk)")
    weights = moe.make_moe_weights(9800, E, K, H, O, device)
    x = dev_bf16(synth.normal_bf16(9801, (T, K)), device)
    ids_h, w_h = synth.zipf_routing(9802, T, E, topk, 1.1)
    ids = torch.from_numpy(ids_h).to(device)
    w = torch.from_numpy(w_h).to(device)
    out = host_bits(gb.mxfp4_moe_prefill(x, weights.W1, weights.W3, weights.W2, ids, w))
    ref = np.concatenate([host_bits(gb.mxfp4_moe_grouped_gemv(x[i:i + 64], weights.W1, weights.W3,
                                                              weights.W2, ids[i:i + 64], w[i:i + 64]))
                          for i in range(0, T, 64)])
    assert_close(out, ref, "prefill vs decode path", cos_tol=0.99999)

    def fn(e):
        return tuple(expert_host(m, e) for m in (weights.W1, weights.W3, weights.W2))

    def expert_host(m, e):
        return m["packed"][e].cpu().numpy(), m["scale"][e].cpu().numpy()

    xh = synth.normal_bf16(9801, (T, K))
    for t in (0, T - 1):
        assert_close(out[t:t + 1], mx.moe_layer(xh[t:t + 1], fn, ids_h[t:t + 1], w_h[t:t + 1], O),
                     f"prefill token {t} vs oracle")
    del weights
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- RMSNorm ---

@pytest.mark.parametrize("T", [1, 8, 64])
def test_rmsnorm_residual_config(device, T):
    H = 4096
    announce(f"rmsnorm_fuse_residual_add T={T} H={H}")
    h = synth.normal_bf16(1001 + T, (T, H))
    r = synth.normal_bf16(1101 + T, (T, H), 0.0, 0.5)
    g = synth.normal_bf16(1201, (H,), 1.0, 0.1)
    y, nr = rb.rmsnorm_fuse_residual_add(dev_bf16(h, device), dev_bf16(r, device), dev_bf16(g, device))
    ry, rnr = mx.rmsnorm_residual(h, r, g)
    assert np.array_equal(host_bits(nr), rnr)  # single RNE rounding of an exact sum
    assert_close(host_bits(y), ry, f"rmsnorm residual T={T}")
    announce(f"rmsnorm_fuse_fwd T={T} H={H}")
    y2 = rb.rmsnorm_fuse_fwd(dev_bf16(h, device), dev_bf16(g, device))
    assert_close(host_bits(y2), mx.rmsnorm(h, g), f"rmsnorm fwd T={T}")


def test_rmsnorm_max_hidden(device):
    H, T = 8192, 2  # the largest hidden both entries accept
    announce(f"rmsnorm_fuse_residual_add T={T} H={H}")
    h = synth.normal_bf16(1401, (T, H))
    r = synth.normal_bf16(1402, (T, H), 0.0, 0.5)
    g = synth.normal_bf16(1403, (H,), 1.0, 0.1)
    y, nr = rb.rmsnorm_fuse_residual_add(dev_bf16(h, device), dev_bf16(r, device), dev_bf16(g, device))
    ry, rnr = mx.rmsnorm_residual(h, r, g)
    assert np.array_equal(host_bits(nr), rnr)
    assert_close(host_bits(y), ry, "rmsnorm H=8192")
    assert_close(host_bits(rb.rmsnorm_fuse_fwd(dev_bf16(h, device), dev_bf16(g, device))),
                 mx.rmsnorm(h, g), "rmsnorm fwd H=8192")


def test_rmsnorm_scalar_path_and_noop(device):
    H, T = 4001, 3  # H % 8 != 0 -> scalar kernel
    announce(f"rmsnorm_fuse_residual_add scalar path T={T} H={H}")
    h = synth.normal_bf16(1301, (T, H))
    r = synth.normal_bf16(1302, (T, H), 0.0, 0.5)
    g = synth.normal_bf16(1303, (H,), 1.0, 0.1)
    y, nr = rb.rmsnorm_fuse_residual_add(dev_bf16(h, device), dev_bf16(r, device), dev_bf16(g, device))
    ry, rnr = mx.rmsnorm_residual(h, r, g)
    assert np.array_equal(host_bits(nr), rnr)
    assert_close(host_bits(y), ry, "rmsnorm scalar")
    c = dev_bf16(np.full((2, 64), 0x3F40, np.uint16), device)  # constant rows 0.75
    gw = dev_bf16(np.full(64, 0x3F80, np.uint16), device)
    yc = mx.bf16_to_f32(host_bits(rb.rmsnorm_fuse_fwd(c, gw)))
    assert np.allclose(yc, 0.75 / np.sqrt(0.75 ** 2 + 1e-6), rtol=4e-3)


# ------------------------------------------------------------- HIP graphs ---

@pytest.mark.parametrize("T,K", [(2, 1024), (1, 2048)])
def test_moe_layer_graph_replays_match_eager(device, T, K):
    """A captured decode layer (gating + stages A/B, no memsets) replays
    bit-identically to the eager call, with eager work between replays. T = 1
    at K = 2048 takes the path with the gating inside stage A."""
    from runtime import moe

    E, H, O = 32, 512, 1024
    announce(f"mxfp4_moe_layer graph capture T={T} K={K} E={E}")
    weights = moe.make_moe_weights(9700, E, K, H, O, device)
    layer = moe.RoutedMoELayer(weights, topk=8, max_tokens=4)
    x = dev_bf16(synth.normal_bf16(9701, (T, K)), device)
    logits = dev_f32(synth.gating_logits(9702, T, E), device)
    eager = host_bits(layer.forward(x, logits=logits)).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer.forward(x, logits=logits)
    other = dev_f32(synth.gating_logits(9703, T, E), device)
    for rep in range(4):
        layer.out.zero_()
        g.replay()
        assert np.array_equal(host_bits(layer.out[:T]), eager), f"replay {rep}"
        layer.forward(x, logits=other)  # eager work between replays
        torch.cuda.synchronize()
