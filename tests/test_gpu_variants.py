"""GPU parity of the kernel variants that the entry points select by shape
and operand alignment and that the configuration-shaped tests do not reach:

- FP8: the general kernel for every segment count (K up to 1024, 2048, 3072,
  aligned and unaligned rows); the fused SwiGLU and the multi-matrix launch on
  the vector tile kernels for every K and token group; the matrix-core kernel
  with four row blocks per wave at K = 1024 and 2048 and the fused SwiGLU with
  two; the RMSNorm-folded GEMV for every token group, K and residual choice,
  with the GEMV on the vector units or on the matrix cores;
- MXFP4: the dense general kernel for two to four blocks per lane, aligned and
  unaligned; the routed layer's general stage-A and stage-B kernels, which take
  over when scale rows, the activation or W2 are not 16-byte aligned, for one
  and two blocks per lane; the router GEMV at K = 8192;
- RMSNorm: hidden 6144 (16 waves with a quarter of the threads past the row)
  and the scalar forward path.

Every case is checked against the oracle (max rel err <= 1e-2, cosine >=
0.9999); where two launches must agree, bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mx
from runtime import moe, synth
from runtime import fp8_e4m3_gemv_binding as fp8b
from runtime import mxfp4_gemv_binding as mxb
from runtime import mxfp4_grouped_gemv_binding as gb
from runtime import rmsnorm_fuse_binding as rb
from tests.gpu_util import announce, assert_close, dev_bf16, dev_f32, dev_u8, host_bits

pytestmark = pytest.mark.gpu


def _at_offset(t: torch.Tensor, nbytes: int) -> torch.Tensor:
    """A contiguous copy of t whose data starts nbytes past a 256-byte boundary."""
    n = t.numel() * t.element_size()
    buf = torch.zeros(n + 256, dtype=torch.uint8, device=t.device)
    v = buf[nbytes:nbytes + n]
    v.copy_(t.contiguous().reshape(-1).view(torch.uint8))
    out = v.view(t.dtype).view(t.shape)
    assert out.data_ptr() % 16 == nbytes % 16
    return out


def _fp8_uniform(seed: int, N: int, K: int):
    """E4M3 codes uniform over the non-NaN bytes and tile scales 2^-14 .. 2^-10:
    a quick stand-in for large weight matrices (any code is a valid weight)."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, (N, K), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] ^= 1
    s = rng.integers(113, 118, ((N + 127) // 128, K // 128), dtype=np.uint8)
    return w, s


def _x1(xd, T):
    return xd if T > 1 else xd[0]


# ---------------------------------------------------------------- FP8 -------

@pytest.mark.parametrize("N,K,T,odd_stride", [(77, 1024, 2, True), (90, 1536, 1, False), (90, 1536, 3, True),
                                              (70, 2560, 2, False), (70, 3072, 1, True)])
def test_fp8_general_kernel_segments(device, N, K, T, odd_stride):
    """The general kernel with one, two and three 1 KiB chunks per lane, on
    aligned and on odd-stride (unaligned) weight rows."""
    announce(f"fp8_e4m3_gemv general N={N} K={K} T={T} odd_stride={odd_stride}")
    w, s = synth.fp8_weight(20000 + N + K + T, N, K)
    x = synth.normal_bf16(20100 + T, (T, K))
    if odd_stride:
        buf = torch.zeros(N, K + 1, dtype=torch.uint8, device=device)
        buf[:, :K] = dev_u8(w, device)
        tw = buf[:, :K]
    else:
        tw = dev_u8(w, device)
    y = fp8b.fp8_e4m3_gemv(tw, dev_u8(s, device), _x1(dev_bf16(x, device), T))
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 general N={N} K={K} T={T}")


@pytest.mark.parametrize("K", [1024, 2048, 4096])
@pytest.mark.parametrize("T", [1, 2, 3, 8])
def test_fp8_swiglu_vector_tiles(device, K, T):
    """The fused SwiGLU on the vector tile kernel (300 rows: below the
    matrix-core rule) for every K up to 4096 and token group 1, 2, 4, 8."""
    N = 300
    announce(f"fp8_e4m3_swiglu_gemv vector N={N} K={K} T={T}")
    w1, s1 = synth.fp8_weight(20200 + K, N, K)
    w3, s3 = synth.fp8_weight(20300 + K, N, K)
    x = mx.bf16_round(24 * mx.bf16_to_f32(synth.normal_bf16(20400 + T, (T, K))))
    act = fp8b.fp8_e4m3_swiglu_gemv(dev_u8(w1, device), dev_u8(s1, device), dev_u8(w3, device), dev_u8(s3, device),
                                    _x1(dev_bf16(x, device), T), 10.0, True)
    assert_close(host_bits(act).reshape(T, N), mx.fp8_swiglu(x, w1, s1, w3, s3, 10.0, True),
                 f"fp8 swiglu vector K={K} T={T}")


def test_fp8_vector_tile_k1024_eight_tokens(device):
    N, K, T = 600, 1024, 6
    announce(f"fp8_e4m3_gemv vector tile N={N} K={K} T={T}")
    w, s = synth.fp8_weight(20500, N, K)
    x = synth.normal_bf16(20501, (T, K))
    y = fp8b.fp8_e4m3_gemv(dev_u8(w, device), dev_u8(s, device), dev_bf16(x, device))
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), "fp8 K=1024 T=6")


@pytest.mark.parametrize("K,T,shapes", [(1024, 1, [300, 200]), (1024, 2, [300, 200]), (1024, 3, [300, 200]),
                                        (1024, 8, [300, 200]), (1024, 12, [300, 200]),
                                        (2048, 1, [300, 200]), (2048, 2, [300, 200]), (2048, 3, [300, 200]),
                                        (2048, 8, [300, 200]), (2048, 12, [300, 200]),
                                        (4096, 2, [300, 200]), (4096, 8, [300, 200]), (4096, 12, [300, 200]),
                                        (8192, 1, [300, 200]),
                                        (1024, 4, [2048, 2048]), (2048, 5, [2048, 2048])])
def test_fp8_multi_launch_variants(device, K, T, shapes):
    """The multi-matrix launch for every K and token group on the vector
    kernels, and on the matrix cores at K = 1024 and 2048: each output has the
    bits of fp8_e4m3_gemv on its matrix alone and matches the oracle."""
    announce(f"fp8_e4m3_gemv_multi N={shapes} K={K} T={T}")
    mats, dmats = [], []
    for i, N in enumerate(shapes):
        w, s = synth.fp8_weight(20600 + 10 * i + K, N, K)
        mats.append((w, s))
        dmats.append((dev_u8(w, device), dev_u8(s, device)))
    x = synth.normal_bf16(20700 + T, (T, K))
    xin = _x1(dev_bf16(x, device), T)
    ys = fp8b.fp8_e4m3_gemv_multi(dmats, xin)
    for (w, s), (tw, ts), y, N in zip(mats, dmats, ys, shapes):
        got = host_bits(y).reshape(T, N)
        single = host_bits(fp8b.fp8_e4m3_gemv(tw, ts, xin)).reshape(T, N)
        assert np.array_equal(got, single), f"N={N}: multi launch differs from the single launch"
        assert_close(got, mx.fp8_gemv(x, w, s), f"multi N={N} K={K} T={T}")


@pytest.mark.parametrize("N,K", [(65536, 1024), (32768, 2048)])
def test_fp8_matrix_core_four_row_blocks_short_k(device, N, K):
    """Four 16-row blocks per wave at K = 1024 and 2048 (T = 8): the shapes at
    which the row-block rule first takes four."""
    T = 8
    announce(f"fp8_e4m3_gemv matrix cores N={N} K={K} T={T}")
    w, s = _fp8_uniform(20800 + K, N, K)
    x = synth.normal_bf16(20801, (T, K))
    y = fp8b.fp8_e4m3_gemv(dev_u8(w, device), dev_u8(s, device), dev_bf16(x, device))
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(x, w, s), f"fp8 R=4 N={N} K={K}")


@pytest.mark.parametrize("N,K", [(16384, 1024), (8192, 4096)])
def test_fp8_swiglu_matrix_core_two_row_blocks(device, N, K):
    """The fused SwiGLU with two 16-row blocks per wave (T = 8)."""
    T = 8
    announce(f"fp8_e4m3_swiglu_gemv matrix cores N={N} K={K} T={T}")
    w1, s1 = _fp8_uniform(20900 + K, N, K)
    w3, s3 = _fp8_uniform(20950 + K, N, K)
    x = synth.normal_bf16(20901, (T, K))
    act = fp8b.fp8_e4m3_swiglu_gemv(dev_u8(w1, device), dev_u8(s1, device), dev_u8(w3, device), dev_u8(s3, device),
                                    dev_bf16(x, device), 10.0, False)
    assert_close(host_bits(act).reshape(T, N), mx.fp8_swiglu(x, w1, s1, w3, s3, 10.0, False),
                 f"fp8 swiglu R=2 N={N} K={K}")


@pytest.mark.parametrize("K", [2048, 4096])
@pytest.mark.parametrize("T,N", [(1, 300), (2, 300), (3, 300), (4, 4096)])
@pytest.mark.parametrize("resid", [True, False])
def test_fp8_rmsnorm_gemv_variants(device, K, T, N, resid):
    """RMSNorm folded into the GEMV for token groups 1, 2 and 4, with and
    without the residual, the GEMV on the vector units (300 rows) or, at
    T = 4 and 4096 rows, on the matrix cores after the norm in one workgroup:
    x_norm and new_residual match the oracle (new_residual bit for bit), y
    has fp8_e4m3_gemv's bits on x_norm and matches the oracle."""
    announce(f"fp8_e4m3_rmsnorm_gemv N={N} K={K} T={T} residual={resid}")
    w, s = synth.fp8_weight(21000 + N + K, N, K)
    h = synth.normal_bf16(21001 + T, (T, K))
    r = synth.normal_bf16(21002 + T, (T, K), 0.0, 0.5)
    g = synth.normal_bf16(21003, (K,), 1.0, 0.1)
    tw, ts = dev_u8(w, device), dev_u8(s, device)
    hd, rd, gd = dev_bf16(h, device), dev_bf16(r, device), dev_bf16(g, device)
    y, xn, nr = fp8b.fp8_e4m3_rmsnorm_gemv(tw, ts, _x1(hd, T), gd, _x1(rd, T) if resid else None)
    if resid:
        oracle_xn, oracle_nr = mx.rmsnorm_residual(h, r, g)
        assert np.array_equal(host_bits(nr).reshape(T, K), oracle_nr), "new_residual bits"
    else:
        oracle_xn = mx.rmsnorm(h, g)
    assert_close(host_bits(xn).reshape(T, K), oracle_xn, "x_norm vs oracle")
    ref_y = fp8b.fp8_e4m3_gemv(tw, ts, xn.reshape(T, K) if T > 1 else xn.reshape(K))
    assert np.array_equal(host_bits(y).reshape(T, N), host_bits(ref_y).reshape(T, N)), "y bits"
    assert_close(host_bits(y).reshape(T, N), mx.fp8_gemv(oracle_xn, w, s), "y vs oracle")


# ------------------------------------------------------------ dense MXFP4 ---

@pytest.mark.parametrize("K,unaligned", [(3072, False), (3072, True), (6144, True), (7168, False), (8192, True)])
def test_mxfp4_gemv_general_kernel(device, K, unaligned):
    """The general dense kernel with two, three and four MX blocks per lane
    (K off the tile set, or unaligned rows and activation at any K)."""
    N = 50
    announce(f"mxfp4_gemv_m1 general N={N} K={K} unaligned={unaligned}")
    p, s = synth.mxfp4_weight(21100 + K, N, K)
    x = synth.normal_bf16(21101 + K, (K,))
    ref = mx.mxfp4_gemv(x, p[0], s[0])
    ts = dev_u8(s[0], device)
    if unaligned:
        odd_p = np.zeros((N, K // 2 + 1 + 7), np.uint8)
        odd_p[:, 1:1 + K // 2] = p[0]
        to = dev_u8(odd_p, device)
        xb = dev_bf16(np.concatenate([[0], x]).astype(np.uint16), device)
        y = mxb.mxfp4_gemv(to[:, 1:1 + K // 2], ts, xb[1:])
    else:
        y = mxb.mxfp4_gemv(dev_u8(p[0], device), ts, dev_bf16(x, device))
    assert_close(host_bits(y), ref, f"mxfp4 general K={K}")


# ------------------------------------------------------------- routed MoE ---

def _host_expert_fn(weights):
    cache = {}

    def fn(e):
        if e not in cache:
            cache[e] = tuple((m["packed"][e].cpu().numpy(), m["scale"][e].cpu().numpy())
                             for m in (weights.W1, weights.W3, weights.W2))
        return cache[e]

    return fn


@pytest.mark.parametrize("K,H", [(2048, 2048), (4096, 2048), (2048, 4096)])
@pytest.mark.parametrize("variant", ["scales_offset", "x_offset", "w2_offset"])
def test_moe_general_kernels(device, K, H, variant):
    """The routed layer when an operand is not 16-byte aligned, which moves it
    off the one-token and multi-token kernels onto the general ones: scale
    tensors 2 bytes past a boundary (the checked-alignment fast kernels), the
    activation 2 bytes past (stage A's unaligned loads), W2 1 byte past (stage
    B's unaligned loads); for one and two MX blocks per lane in stage A (K)
    and stage B (hidden), one and three tokens, and the drop-in."""
    E, O, topk = 8, 256, 2
    announce(f"mxfp4 routed general kernels {variant} K={K} H={H}")
    w = moe.make_moe_weights(21200 + K + H, E, K, H, O, device)
    fn = _host_expert_fn(w)
    mats = {m: dict(getattr(w, m)) for m in ("W1", "W3", "W2")}
    if variant == "scales_offset":
        for m in mats:
            mats[m]["scale"] = _at_offset(mats[m]["scale"], 2)
    if variant == "w2_offset":
        mats["W2"]["packed"] = _at_offset(mats["W2"]["packed"], 1)
    for T in (1, 3):
        x = synth.normal_bf16(21300 + T, (T, K))
        xd = dev_bf16(x, device)
        if variant == "x_offset":
            xd = _at_offset(xd, 2)
        ids, wt = mx.route_sigmoid_topk(synth.gating_logits(21400 + T, T, E), topk)
        out = host_bits(gb.mxfp4_moe_grouped_gemv(xd, mats["W1"], mats["W3"], mats["W2"],
                                                  torch.from_numpy(ids).to(device), dev_f32(wt, device)))
        assert_close(out, mx.moe_layer(x, fn, ids, wt, O, n_experts=E), f"{variant} T={T}")
        if T == 1:
            sub = {m: {"packed": mats[m]["packed"][:4], "scale": mats[m]["scale"][:4]} for m in mats}
            r = np.linspace(0.1, 0.4, 4).astype(np.float32)
            got = host_bits(gb.mxfp4_grouped_gemv(sub["W1"], sub["W3"], sub["W2"], None, xd[0], dev_f32(r, device)))
            ref = mx.moe_layer(x, fn, np.arange(4, dtype=np.int32)[None, :], r[None, :], O)
            assert_close(got, ref[0], f"{variant} drop-in")
    del w, mats
    torch.cuda.empty_cache()


def test_router_logits_longest_rows(device):
    """The router GEMV at K = 8192 (16 pieces of a row per lane)."""
    T, E, K = 2, 64, 8192
    announce(f"mxfp4_moe_router_logits T={T} E={E} K={K}")
    x = synth.normal_bf16(21500, (T, K))
    wg = synth.normal_bf16(21501, (E, K), 0.0, 0.02)
    got = gb.router_logits(dev_bf16(x, device), dev_bf16(wg, device)).cpu().numpy()
    ref = mx.router_logits(x, wg)
    bound = (np.abs(mx.bf16_to_f32(x)).astype(np.float64) @ np.abs(mx.bf16_to_f32(wg)).astype(np.float64).T) * 2e-6
    assert np.all(np.abs(got.astype(np.float64) - ref) <= bound + 1e-30)


# ---------------------------------------------------------------- RMSNorm ---

def test_rmsnorm_partial_block_and_scalar_forward(device):
    """hidden = 6144 (768 pieces in a 1,024-thread block: the last 256 threads
    hold no piece) through both entries, and the forward entry on its scalar
    path (hidden not a multiple of 8)."""
    for H, T in ((6144, 3), (4001, 2)):
        announce(f"rmsnorm H={H} T={T}")
        h = synth.normal_bf16(21600 + H, (T, H))
        r = synth.normal_bf16(21601 + H, (T, H), 0.0, 0.5)
        g = synth.normal_bf16(21602 + H, (H,), 1.0, 0.1)
        hd, rd, gd = dev_bf16(h, device), dev_bf16(r, device), dev_bf16(g, device)
        assert_close(host_bits(rb.rmsnorm_fuse_fwd(hd, gd)), mx.rmsnorm(h, g), f"rmsnorm fwd H={H}")
        y, nr = rb.rmsnorm_fuse_residual_add(hd, rd, gd)
        ry, rnr = mx.rmsnorm_residual(h, r, g)
        assert np.array_equal(host_bits(nr), rnr)
        assert_close(host_bits(y), ry, f"rmsnorm residual H={H}")


def _fp8_vector_tiles_far_apart_rows(device, K, Ts, seed):
    """Token rows just far enough apart that the T rows span more than 2^31
    bytes: the matrix-core kernels read the activation rows through one buffer
    of at most 2^31 bytes, so these calls stay on the vector tile kernels
    (single matrix, fused SwiGLU, multi-matrix, fp32 tile scales), called
    through the C ABI with the row stride. Each against the oracle; the
    multi-matrix and fp32-scale outputs bit for bit against the single GEMV."""
    import ctypes
    from runtime import _lib as rl

    lib = fp8b._load_lib()
    N = 300
    x = synth.normal_bf16(seed, (max(Ts), K))
    x = mx.bf16_round(8 * mx.bf16_to_f32(x))
    xd = dev_bf16(x, device)
    w1, s1 = synth.fp8_weight(seed + 1, N, K)
    w3, s3 = synth.fp8_weight(seed + 2, N, K)
    w2, s2 = synth.fp8_weight(seed + 3, 200, K)
    d1, e1, d3, e3 = dev_u8(w1, device), dev_u8(s1, device), dev_u8(w3, device), dev_u8(s3, device)
    d2, e2 = dev_u8(w2, device), dev_u8(s2, device)
    sf = torch.from_numpy(np.ldexp(np.float32(1.0), s1.astype(np.int32) - 127).astype(np.float32)).to(device)
    st = ctypes.c_void_p(rl.stream_ptr(device))
    for T in Ts:
        stride = (2**30 // (T - 1) // 8 + 1) * 8            # (T - 1) * stride * 2 bytes > 2^31
        assert ((T - 1) * stride + K) * 2 > 2**31 - 1
        announce(f"fp8 K={K} T={T} rows {stride} elements apart")
        xbuf = torch.zeros((T - 1) * stride + K, dtype=torch.bfloat16, device=device)
        for t in range(T):
            xbuf[t * stride:t * stride + K] = xd[t]
        y = torch.empty(T, N, dtype=torch.bfloat16, device=device)
        rc = lib.fp8_e4m3_gemv(rl.vp(xbuf), stride, rl.vp(d1), rl.vp(e1), K, N, T, K, K // 128, rl.vp(y), N, st)
        assert rc == 0
        single = host_bits(y)
        assert_close(single, mx.fp8_gemv(x[:T], w1, s1), f"fp8 far rows K={K} T={T}")
        act = torch.empty(T, N, dtype=torch.bfloat16, device=device)
        rc = lib.fp8_e4m3_swiglu_gemv(rl.vp(xbuf), stride, rl.vp(d1), rl.vp(e1), rl.vp(d3), rl.vp(e3), K, N, T,
                                      K, K // 128, 10.0, 1, rl.vp(act), N, st)
        assert rc == 0
        assert_close(host_bits(act), mx.fp8_swiglu(x[:T], w1, s1, w3, s3, 10.0, True),
                     f"swiglu far rows K={K} T={T}")
        ya = torch.empty(T, N, dtype=torch.bfloat16, device=device)
        yb = torch.empty(T, 200, dtype=torch.bfloat16, device=device)
        PA, IA, LA = ctypes.c_void_p * 2, ctypes.c_int * 2, ctypes.c_int64 * 2
        rc = lib.fp8_e4m3_gemv_multi(rl.vp(xbuf), stride, K, T, 2, PA(d1.data_ptr(), d2.data_ptr()),
                                     PA(e1.data_ptr(), e2.data_ptr()), IA(N, 200), LA(K, K), LA(K // 128, K // 128),
                                     PA(ya.data_ptr(), yb.data_ptr()), LA(N, 200), st)
        assert rc == 0
        assert np.array_equal(host_bits(ya), single), "multi launch differs from the single launch"
        assert_close(host_bits(yb), mx.fp8_gemv(x[:T], w2, s2), f"multi far rows K={K} T={T}")
        # the fp32-scale entry on the same vector tiles: scales 2^(b-127) give the E8M0 bits
        yf = torch.empty(T, N, dtype=torch.bfloat16, device=device)
        rc = lib.fp8_e4m3_gemv_f32s(rl.vp(xbuf), stride, rl.vp(d1), rl.vp(sf), K, N, T, K, K // 128, rl.vp(yf), N, st)
        assert rc == 0
        assert np.array_equal(host_bits(yf), single), "fp32-scale entry differs from the E8M0 entry"
        del xbuf
        torch.cuda.empty_cache()


def test_fp8_k8192_vector_tiles_far_apart_rows(device):
    """K = 8192 on the vector tile kernels (token groups of 2 and 4, two
    k-slices per thread): every other shape with T >= 2 at this K takes the
    matrix cores."""
    _fp8_vector_tiles_far_apart_rows(device, 8192, (2, 4), 21700)


@pytest.mark.parametrize("K", [1024, 2048])
def test_fp8_short_rows_vector_tiles_far_apart_rows(device, K):
    """K = 1024 and 2048 with 5 .. 16 tokens on the vector tile kernels (token
    groups of 8 and 16; the fused SwiGLU in groups of 8 and a last group of
    1): every other shape with T >= 5 at these K takes the matrix cores."""
    _fp8_vector_tiles_far_apart_rows(device, K, (5, 9, 16), 21710 + K)
