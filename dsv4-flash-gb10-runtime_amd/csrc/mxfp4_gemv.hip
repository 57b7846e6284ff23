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

// Tile kernel for K in {2048, 4096, 8192} with 16-byte aligned rows and
// activation. A workgroup of 256 threads owns R = C*256/KC rows (KC = K/32
// blocks per row); thread t takes blocks t, t+256, ... of the workgroup's
// [R, KC] block grid, so all of its blocks share one k-slice (block t % KC)
// and every wave instruction reads 1 KiB of a single row. The activation
// slice (32 bf16) is issued first, then the C weight blocks and scale bytes,
// all unconditional (rows clamped), so one issue pass puts everything in
// flight. Partials (C per wave, one butterfly) meet in LDS, fixed order.
// The block scale is applied once per block: it is a power of two, so this
// equals the per-element scaling of kernel/mxfp4-dense/mxfp4_gemv.cu:116-117
// up to the rounding of partial sums.
template <int C, int KC>
__global__ __launch_bounds__(256) void mxfp4_gemv_tile_kernel(const GemvArgs a) {
    constexpr int kRowsWG = C * 256 / KC;
    __shared__ float part[kWaves][C];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n0 = blockIdx.x * kRowsWG;
    const int b = t % KC;
    uint32_t xs[16];
    {
        const u32x4* s4 = reinterpret_cast<const u32x4*>(a.x + b * kBlkElems);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = s4[q];
            xs[4 * q] = v[0]; xs[4 * q + 1] = v[1]; xs[4 * q + 2] = v[2]; xs[4 * q + 3] = v[3];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // activation loads first
    u32x4 w[C];
    uint32_t sb[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
        const int n = min(n0 + (t + 256 * i) / KC, a.N - 1);
        w[i] = ld16_stream(a.w + (int64_t)n * a.wrow + b * 16);
        sb[i] = a.s[(int64_t)n * a.srow + b];
    }
    float acc[C];
    float chain = 0.f;
#pragma unroll
    for (int i = 0; i < C; ++i) {
        reg_barrier_after(w[i], chain);
        acc[i] = fp4_block_dot(w[i], xs) * e8m0_to_f32(sb[i]);
        chain = acc[i];
    }
    wave_reduce_n<C>(acc, lane);
    const int v = reduced_index<C>(lane);
    if (reduced_owner<C>(lane)) part[wave][v] = acc[0];
    __syncthreads();
    if (t < kRowsWG && n0 + t < a.N) {
        float sum = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; ++w2) {
#pragma unroll
            for (int i = 0; i < C; ++i)
                if ((64 * w2 + 256 * i) / KC == t) sum += part[w2][i];
        }
        a.y[n0 + t] = f32_to_bf16_bits(sum);
    }
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
        // Two blocks per thread: 8, 4 or 2 rows per workgroup at K = 2048, 4096, 8192.
        const int KC = K / kBlkElems;
        const int rows = 2 * 256 / KC;
        const dim3 g((unsigned)((N + rows - 1) / rows));
        if (KC == 64) hipLaunchKernelGGL((mxfp4_gemv_tile_kernel<2, 64>), g, dim3(256), 0, stream, a);
        else if (KC == 128) hipLaunchKernelGGL((mxfp4_gemv_tile_kernel<2, 128>), g, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((mxfp4_gemv_tile_kernel<2, 256>), g, dim3(256), 0, stream, a);
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
