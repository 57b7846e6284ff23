// mxfp4_gemv.hip — dense MXFP4 GEMV (M = 1) and debug dequant for gfx950.
//
//   y[n] = bf16( sum_k e2m1(W[n,k]) * 2^(S[n,k/32]-127) * x[k] )
//
// Same data path as the routed kernel: lane l of a wave owns MX blocks
// l, l+64, ... of every row it visits, streams them with 16-byte loads
// (one wave-wide load = 1 KiB of a row), keeps its activation slice in
// registers, decodes with v_cvt_scalef32_pk_bf16_fp4, accumulates with
// v_dot2_f32_bf16 in fp32, applies the E8M0 scale once per block and reduces
// kRows rows per wave with one butterfly. Row strides are the caller's
// (reference kernel/mxfp4-dense/mxfp4_gemv.cu:131-166 honours them too).

#include <cstdio>

#include "dsv4_device.h"
#include "dsv4_kernels.h"

namespace {

using namespace dsv4;

constexpr int kBlkElems = 32;
constexpr int kMaxK = 8192;     // reference MXFP4_GEMV_MAX_K (mxfp4_gemv.cu:48-50)
constexpr int kWaves = 4;
constexpr int kRows = 4;        // rows per wave

struct GemvArgs {
    const uint16_t* x;
    const uint8_t* w;
    const uint8_t* s;
    int K;
    int N;
    int64_t wrow;               // packed row stride, bytes
    int64_t srow;               // scale row stride, bytes
    uint16_t* y;
};

template <bool ALIGNED>
__device__ __forceinline__ u32x4 load_w16(const uint8_t* p) {
    if constexpr (ALIGNED) return ld16(p);
    else return ld16_unaligned(p);
}

// grid = ceil(N / (kWaves*kRows)), block = 64*kWaves.
template <int NB, bool ALIGNED>
__global__ __launch_bounds__(64 * kWaves) void mxfp4_gemv_kernel(const GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * kWaves + wave) * kRows;
    if (n0 >= a.N) return;
    const int nblk = a.K / kBlkElems;

    bool bvalid[NB];
    uint32_t xs[NB][16];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int b = lane + 64 * j;
        bvalid[j] = b < nblk;
        if (bvalid[j]) {
            const uint16_t* src = a.x + b * kBlkElems;
            if constexpr (ALIGNED) {
                const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4 v = s4[q];
                    xs[j][4 * q + 0] = v[0];
                    xs[j][4 * q + 1] = v[1];
                    xs[j][4 * q + 2] = v[2];
                    xs[j][4 * q + 3] = v[3];
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    xs[j][q] = (uint32_t)src[2 * q] | ((uint32_t)src[2 * q + 1] << 16);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 16; ++q) xs[j][q] = 0u;
        }
    }

    u32x4 wv[kRows][NB];
    uint32_t sv[kRows][NB];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int n = n0 + r;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int b = lane + 64 * j;
            if (n < a.N && bvalid[j]) {
                wv[r][j] = load_w16<ALIGNED>(a.w + (int64_t)n * a.wrow + (int64_t)b * 16);
                sv[r][j] = a.s[(int64_t)n * a.srow + b];
            } else {
                wv[r][j] = u32x4{0u, 0u, 0u, 0u};
                sv[r][j] = 0u;
            }
        }
    }
    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < NB; ++j)
            s = fmaf(fp4_block_dot(wv[r][j], xs[j]), e8m0_to_f32(sv[r][j]), s);
        acc[r] = s;
    }
    wave_reduce_n<kRows>(acc, lane);
    const int r = reduced_index<kRows>(lane);
    if (reduced_owner<kRows>(lane) && n0 + r < a.N) a.y[n0 + r] = f32_to_bf16_bits(acc[0]);
}

// One thread per MX block: 16 packed bytes -> 32 bf16 outputs.
__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint8_t* w, const uint8_t* s,
                                                            int K, int N, int64_t wrow,
                                                            int64_t srow, uint16_t* out) {
    const int nblk = K / kBlkElems;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)N * nblk) return;
    const int n = (int)(idx / nblk);
    const int b = (int)(idx % nblk);
    const u32x4 v = ld16_unaligned(w + (int64_t)n * wrow + (int64_t)b * 16);
    const float sc = e8m0_to_f32(s[(int64_t)n * srow + b]);
    uint16_t* o = out + (int64_t)n * K + (int64_t)b * kBlkElems;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bf16x2 p0 = fp4x2_to_bf16x2<0>(v[i]);
        const bf16x2 p1 = fp4x2_to_bf16x2<1>(v[i]);
        const bf16x2 p2 = fp4x2_to_bf16x2<2>(v[i]);
        const bf16x2 p3 = fp4x2_to_bf16x2<3>(v[i]);
        const uint32_t q[4] = {as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[8 * i + 2 * k + 0] = f32_to_bf16_bits(bf16_bits_to_f32(q[k] & 0xFFFFu) * sc);
            o[8 * i + 2 * k + 1] = f32_to_bf16_bits(bf16_bits_to_f32(q[k] >> 16) * sc);
        }
    }
}

// Row kernel for K in {2048, 4096, 8192} with 16-byte aligned rows and
// activation: each wave owns kFastRows consecutive rows, lane l takes MX
// blocks l, l+64, ... (NB = K/2048 per row), so every wave load instruction
// reads 1 KiB of one row and the activation slice (NB blocks of 32 bf16) is
// loaded once per wave for both rows. Activation first, then the rows'
// weight blocks and scale bytes, all unconditional (rows clamped), so one
// issue pass puts everything in flight; each row is reduced by one butterfly
// and stored by one lane: no LDS and no barrier. The block scale is applied
// once per block: it is a power of two, so this equals the per-element
// scaling of kernel/mxfp4-dense/mxfp4_gemv.cu:116-117 up to the rounding of
// partial sums.
// Workgroup L (dispatched to XCD L % 8) takes row block (L % 8) * (G / 8) +
// L / 8 of the G = gridDim.x blocks (G a multiple of 8; blocks past the
// matrix exit), so the workgroups that write one 128-byte line of y run on
// one XCD. On MI355X (2048 x 4096, graph replay over 512 MB of weight
// copies) this layout took 2.88 us against 3.05 for two-block tiles of 256
// threads combined across waves in LDS (3.18-3.43 us with 4 or 8 rows per
// wave, 2.94 us for the tiles with the XCD mapping alone).
constexpr int kFastRows = 2;
constexpr int kFastWaves = 4;

template <int NB>
__global__ __launch_bounds__(64 * kFastWaves) void mxfp4_gemv_rows_kernel(const GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int G = gridDim.x;
    const int blk = (int)((blockIdx.x % 8) * (G / 8) + blockIdx.x / 8);
    const int n0 = (blk * kFastWaves + wave) * kFastRows;
    if (n0 >= a.N) return;
    uint32_t xs[NB][16];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const u32x4* s4 = reinterpret_cast<const u32x4*>(a.x + (lane + 64 * j) * kBlkElems);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = s4[q];
            xs[j][4 * q] = v[0]; xs[j][4 * q + 1] = v[1]; xs[j][4 * q + 2] = v[2]; xs[j][4 * q + 3] = v[3];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // activation loads first
    u32x4 w[kFastRows][NB];
    uint32_t sb[kFastRows][NB];
#pragma unroll
    for (int r = 0; r < kFastRows; ++r) {
        const int64_t n = min(n0 + r, a.N - 1);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            w[r][j] = ld16_stream(a.w + n * a.wrow + (int64_t)(lane + 64 * j) * 16);
            sb[r][j] = a.s[n * a.srow + lane + 64 * j];
        }
    }
    float acc[kFastRows];
    float chain = 0.f;
#pragma unroll
    for (int r = 0; r < kFastRows; ++r) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            reg_barrier_after(w[r][j], chain);
            s = fmaf(fp4_block_dot(w[r][j], xs[j]), e8m0_to_f32(sb[r][j]), s);
            chain = s;
        }
        acc[r] = s;
    }
    wave_reduce_n<kFastRows>(acc, lane);
    const int v = reduced_index<kFastRows>(lane);
    if (reduced_owner<kFastRows>(lane) && n0 + v < a.N) a.y[n0 + v] = f32_to_bf16_bits(acc[0]);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int mxfp4_gemv_m1(const dsv4_bf16_t* x, const uint8_t* W_packed, const uint8_t* W_scale,
                             int K, int N, int64_t packed_row_stride_bytes,
                             int64_t scale_row_stride_bytes, dsv4_bf16_t* y, hipStream_t stream) {
    if (K % kBlkElems != 0 || K < kBlkElems) {
        std::fprintf(stderr, "mxfp4_gemv_m1: K=%d not a positive multiple of %d\n", K, kBlkElems);
        return -1;
    }
    if (K > kMaxK) {
        std::fprintf(stderr, "mxfp4_gemv_m1: K=%d > %d\n", K, kMaxK);
        return -2;
    }
    if (N < 1) {
        std::fprintf(stderr, "mxfp4_gemv_m1: N=%d < 1\n", N);
        return -3;
    }
    GemvArgs a{reinterpret_cast<const uint16_t*>(x), W_packed, W_scale, K, N,
               packed_row_stride_bytes, scale_row_stride_bytes, reinterpret_cast<uint16_t*>(y)};
    const bool al = aligned16(x) && aligned16(W_packed) && (packed_row_stride_bytes % 16 == 0);
    if (al && (K == 2048 || K == 4096 || K == 8192)) {
        const int per_wg = kFastRows * kFastWaves;
        const unsigned blocks = (unsigned)((N + per_wg - 1) / per_wg);
        const dim3 g((blocks + 7u) / 8u * 8u);
        if (K == 2048) hipLaunchKernelGGL(mxfp4_gemv_rows_kernel<1>, g, dim3(64 * kFastWaves), 0, stream, a);
        else if (K == 4096) hipLaunchKernelGGL(mxfp4_gemv_rows_kernel<2>, g, dim3(64 * kFastWaves), 0, stream, a);
        else hipLaunchKernelGGL(mxfp4_gemv_rows_kernel<4>, g, dim3(64 * kFastWaves), 0, stream, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            std::fprintf(stderr, "mxfp4_gemv_m1 launch failed: %s\n", hipGetErrorString(e));
            return -3;
        }
        return 0;
    }
    const dim3 grid((unsigned)((N + kWaves * kRows - 1) / (kWaves * kRows)));
    const dim3 block(64 * kWaves);
    const int nb = (K / kBlkElems + 63) / 64;
#define DSV4_LAUNCH(NBV)                                                                        \
    if (al) hipLaunchKernelGGL((mxfp4_gemv_kernel<NBV, true>), grid, block, 0, stream, a);     \
    else hipLaunchKernelGGL((mxfp4_gemv_kernel<NBV, false>), grid, block, 0, stream, a);
    switch (nb) {
        case 1: DSV4_LAUNCH(1) break;
        case 2: DSV4_LAUNCH(2) break;
        case 3: DSV4_LAUNCH(3) break;
        default: DSV4_LAUNCH(4) break;
    }
#undef DSV4_LAUNCH
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4_gemv_m1 launch failed: %s\n", hipGetErrorString(e));
        return -3;
    }
    return 0;
}

extern "C" int mxfp4_dequant_bf16(const uint8_t* W_packed, const uint8_t* W_scale, int K, int N,
                                  int64_t packed_row_stride_bytes, int64_t scale_row_stride_bytes,
                                  dsv4_bf16_t* out, hipStream_t stream) {
    if (K % kBlkElems != 0 || K < kBlkElems) return -1;
    if (N < 1) return -3;
    if (!W_packed || !W_scale || !out) {
        std::fprintf(stderr, "mxfp4_dequant_bf16: a required pointer is null\n");
        return -10;
    }
    const int64_t total = (int64_t)N * (K / kBlkElems);
    const dim3 grid((unsigned)((total + 255) / 256));
    hipLaunchKernelGGL(mxfp4_dequant_kernel, grid, dim3(256), 0, stream, W_packed, W_scale, K, N,
                       packed_row_stride_bytes, scale_row_stride_bytes,
                       reinterpret_cast<uint16_t*>(out));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4_dequant_bf16 launch failed: %s\n", hipGetErrorString(e));
        return -3;
    }
    return 0;
}
