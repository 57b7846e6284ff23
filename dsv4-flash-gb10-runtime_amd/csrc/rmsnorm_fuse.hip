// rmsnorm_fuse.hip — RMSNorm and fused residual-add + RMSNorm, gfx950.
//
//   rmsnorm_fuse_fwd:          y = bf16( (w * x) * rsqrt(sum(x^2) * (1/H) + eps) )
//   rmsnorm_fuse_residual_add: t = x + r (fp32), new_r = bf16(t),
//                              y = bf16( (w * bf16(t)) * rsqrt(sum(t^2) * (1/H) + eps) )
// The sum of squares runs over the unrounded fp32 t and the product order
// (w * v) * rms follows reference kernel/rmsnorm-fuse/rmsnorm_fuse.cu:138-155.
//
// One workgroup per row. On the vector path each thread holds one 16-byte
// piece (8 bf16) of the row, of the residual and of the weight, all loaded
// together before the reduction, so the row is read once; the workgroup has
// 4, 8 or 16 waves, enough for one piece per thread. The sum of squares is
// reduced with wave shuffles, then the wave totals are added in wave order
// through LDS.

#include <cstdint>

#include "dsv4_device.h"
#include "dsv4_kernels.h"

namespace {

using namespace dsv4;

constexpr int kThreads = 256;                          // scalar path
constexpr int kMaxHidden = 8192;                       // reference RMSF_MAX_HIDDEN
constexpr int kVec = 8;                                // bf16 per 16-byte access
constexpr int kMaxVecWaves = kMaxHidden / (kVec * 64); // 16

// Sum of v over the workgroup's W waves: a shuffle reduction in each wave,
// then the wave totals added in wave order.
template <int W>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) s += red[w];
    return s;
}

__device__ __forceinline__ void unpack8(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf16_bits_to_f32(v[i] & 0xFFFFu);
        f[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16);
    }
}

__device__ __forceinline__ u32x4 pack8(const uint16_t* h) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (uint32_t)h[2 * i] | ((uint32_t)h[2 * i + 1] << 16);
    return r;
}

// Vector path: rows 16-byte aligned and H % 8 == 0. Thread i holds piece i
// (elements 8i .. 8i+7) of a block of W = 4, 8 or 16 waves (H up to 2048,
// 4096, 8192); threads past the row load piece H/8 - 1 and contribute
// nothing. Every load (row, residual and weight) is issued up front, so the
// kernel waits on one memory round trip before the reduction. One piece per
// thread measured fastest on MI355X (HIP-graph replay, residual entry, T = 1):
// 2.66 us at H = 4096 against 3.25 with two pieces per thread of 256 threads,
// and 3.34 us at H = 8192 against 3.76 (512 threads) and 4.72 (256). A wave
// count chosen at run time (a loop over it in the block sum) was 2-6% slower.
template <bool RESID, int W>
__global__ __launch_bounds__(64 * W) void rmsnorm_vec_kernel(const uint16_t* x, const uint16_t* res,
                                                                        const uint16_t* w, uint16_t* y,
                                                                        uint16_t* new_res, int hidden,
                                                                        float eps) {
    __shared__ float red[W];
    const int64_t off = (int64_t)blockIdx.x * hidden;
    const int nvec = hidden / kVec;
    const int i = threadIdx.x;
    const int ic = min(i, nvec - 1);
    const u32x4 xv = *reinterpret_cast<const u32x4*>(x + off + (int64_t)ic * kVec);
    u32x4 rv{};
    if constexpr (RESID) rv = *reinterpret_cast<const u32x4*>(res + off + (int64_t)ic * kVec);
    const u32x4 gv = *reinterpret_cast<const u32x4*>(w + (int64_t)ic * kVec);
    float v[kVec];
    float ss = 0.f;
    if (i < nvec) {
        float a[kVec];
        unpack8(xv, a);
        if constexpr (RESID) {
            float b[kVec];
            unpack8(rv, b);
            uint16_t tb[kVec];
#pragma unroll
            for (int e = 0; e < kVec; ++e) {
                const float t = a[e] + b[e];
                ss = fmaf(t, t, ss);
                tb[e] = f32_to_bf16_bits(t);
                v[e] = bf16_bits_to_f32(tb[e]);
            }
            *reinterpret_cast<u32x4*>(new_res + off + (int64_t)i * kVec) = pack8(tb);
        } else {
#pragma unroll
            for (int e = 0; e < kVec; ++e) {
                ss = fmaf(a[e], a[e], ss);
                v[e] = a[e];
            }
        }
    }
    const float total = block_sum<W>(ss, red);
    const float rms = rsqrtf(total * (1.0f / (float)hidden) + eps);
    if (i < nvec) {
        float g[kVec];
        unpack8(gv, g);
        uint16_t o[kVec];
#pragma unroll
        for (int e = 0; e < kVec; ++e) o[e] = f32_to_bf16_bits((g[e] * v[e]) * rms);
        *reinterpret_cast<u32x4*>(y + off + (int64_t)i * kVec) = pack8(o);
    }
}

template <bool RESID>
void launch_vec(const uint16_t* x, const uint16_t* res, const uint16_t* w, uint16_t* y, uint16_t* new_res,
                int n_rows, int hidden, float eps, hipStream_t stream) {
    const int pieces = hidden / kVec;              // <= 1024 for hidden <= 8192
    const dim3 grid((unsigned)n_rows);
    if (pieces <= 256)
        hipLaunchKernelGGL((rmsnorm_vec_kernel<RESID, 4>), grid, dim3(256), 0, stream, x, res, w, y, new_res, hidden,
                           eps);
    else if (pieces <= 512)
        hipLaunchKernelGGL((rmsnorm_vec_kernel<RESID, 8>), grid, dim3(512), 0, stream, x, res, w, y, new_res, hidden,
                           eps);
    else
        hipLaunchKernelGGL((rmsnorm_vec_kernel<RESID, kMaxVecWaves>), grid, dim3(1024), 0, stream, x, res, w, y,
                           new_res, hidden, eps);
}

// Scalar path for any alignment / H: each thread walks h = tid, tid+256, ...
template <bool RESID>
__global__ __launch_bounds__(kThreads) void rmsnorm_scalar_kernel(const uint16_t* x,
                                                                  const uint16_t* res,
                                                                  const uint16_t* w, uint16_t* y,
                                                                  uint16_t* new_res, int hidden,
                                                                  float eps) {
    __shared__ float red[kThreads / 64];
    constexpr int kPer = kMaxHidden / kThreads;  // 32
    const int64_t off = (int64_t)blockIdx.x * hidden;
    float v[kPer];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
        const int h = threadIdx.x + c * kThreads;
        v[c] = 0.f;
        if (h < hidden) {
            const float a = bf16_bits_to_f32(x[off + h]);
            if constexpr (RESID) {
                const float t = a + bf16_bits_to_f32(res[off + h]);
                ss = fmaf(t, t, ss);
                const uint16_t tb = f32_to_bf16_bits(t);
                new_res[off + h] = tb;
                v[c] = bf16_bits_to_f32(tb);
            } else {
                ss = fmaf(a, a, ss);
                v[c] = a;
            }
        }
    }
    const float total = block_sum<kThreads / 64>(ss, red);
    const float rms = rsqrtf(total * (1.0f / (float)hidden) + eps);
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
        const int h = threadIdx.x + c * kThreads;
        if (h < hidden) y[off + h] = f32_to_bf16_bits((bf16_bits_to_f32(w[h]) * v[c]) * rms);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int rmsnorm_fuse_fwd(const void* x, const void* weight, void* y, int n_rows, int hidden,
                                float eps, hipStream_t stream) {
    if (n_rows <= 0 || hidden <= 0) return 0;
    if (hidden > kMaxHidden) return 1;
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint16_t*>(weight);
    auto* yp = static_cast<uint16_t*>(y);
    const bool vec = hidden % kVec == 0 && aligned16(x) && aligned16(weight) && aligned16(y);
    if (vec)
        launch_vec<false>(xp, nullptr, wp, yp, nullptr, n_rows, hidden, eps, stream);
    else
        hipLaunchKernelGGL(rmsnorm_scalar_kernel<false>, dim3((unsigned)n_rows), dim3(kThreads), 0,
                           stream, xp, nullptr, wp, yp, nullptr, hidden, eps);
    return (int)hipGetLastError();
}

extern "C" int rmsnorm_fuse_residual_add(const void* x, const void* residual, const void* weight,
                                         void* y_norm, void* new_residual, int n_rows, int hidden,
                                         float eps, hipStream_t stream) {
    if (n_rows <= 0 || hidden <= 0) return 0;
    if (hidden > kMaxHidden) return 1;
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* rp = static_cast<const uint16_t*>(residual);
    const auto* wp = static_cast<const uint16_t*>(weight);
    auto* yp = static_cast<uint16_t*>(y_norm);
    auto* np = static_cast<uint16_t*>(new_residual);
    const bool vec = hidden % kVec == 0 && aligned16(x) && aligned16(residual) &&
                     aligned16(weight) && aligned16(y_norm) && aligned16(new_residual);
    if (vec)
        launch_vec<true>(xp, rp, wp, yp, np, n_rows, hidden, eps, stream);
    else
        hipLaunchKernelGGL(rmsnorm_scalar_kernel<true>, dim3((unsigned)n_rows), dim3(kThreads), 0,
                           stream, xp, rp, wp, yp, np, hidden, eps);
    return (int)hipGetLastError();
}
