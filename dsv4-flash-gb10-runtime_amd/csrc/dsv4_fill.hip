// dsv4_fill.hip — seeded device filler for synthetic benchmark/test inputs.
//
// Counter-based SplitMix64 (Steele, Lea & Flood, "Fast splittable
// pseudorandom number generators", OOPSLA 2014): element i of stream `seed`
// is mix64(seed + (i + 1) * 0x9E3779B97F4A7C15). The same integer function
// is implemented in numpy (runtime/synth.py), so weights filled here on the
// GPU equal, byte for byte, the ones the CPU oracle generates for the same
// (seed, offset). Bytes uniform in [lo, hi] use the high 32 bits of the draw
// with a multiply-shift range reduction: lo + ((hi32 * (hi-lo+1)) >> 32).
//
// Not part of the reference's interface: a harness utility for the tests and
// the benchmark (filling 100+ GB of resident expert weights on the device,
// and a read-only streaming kernel that measures the HBM read floor).

#include <stdint.h>

#include <hip/hip_runtime.h>

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Each thread fills 16 consecutive bytes (one draw per byte).
__global__ __launch_bounds__(256) void fill_uniform_u8_kernel(uint8_t* dst, uint64_t n,
                                                              uint64_t seed, uint64_t offset,
                                                              uint32_t lo, uint32_t span) {
    const uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16ull;
    if (base >= n) return;
    uint8_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint64_t idx = offset + base + (uint64_t)i;
        const uint64_t z = mix64(seed + (idx + 1ull) * 0x9E3779B97F4A7C15ull);
        v[i] = (uint8_t)(lo + (uint32_t)(((z >> 32) * (uint64_t)span) >> 32));
    }
    if (base + 16 <= n && ((reinterpret_cast<uintptr_t>(dst + base) & 15u) == 0)) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)v[4 * i] | ((uint32_t)v[4 * i + 1] << 8) |
                   ((uint32_t)v[4 * i + 2] << 16) | ((uint32_t)v[4 * i + 3] << 24);
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<u32x4*>(dst + base) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
        for (int i = 0; i < 16 && base + i < n; ++i) dst[base + i] = v[i];
    }
}

// Read floor: workgroup b reads pieces [b*per, (b+1)*per) of the 16-byte
// pieces of src (the last workgroup fewer), kReadUnroll loads in flight per
// thread, with the streaming cache policy of the weight loads. The words are
// folded into one value per thread, which is stored only if it equals an
// arbitrary constant (so the loads cannot be removed; the sink is scratch).
constexpr int kReadUnroll = 8;
constexpr uint32_t kReadMagic = 0x9E3779B9u;

__global__ __launch_bounds__(512) void read_floor_kernel(const uint32_t* __restrict__ src, uint64_t n16,
                                                         uint64_t per, uint32_t* sink) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4* p = reinterpret_cast<const u32x4*>(src);
    const uint64_t b0 = (uint64_t)blockIdx.x * per;
    const uint64_t b1 = b0 + per < n16 ? b0 + per : n16;
    uint32_t acc = 0;
    for (uint64_t i = b0 + threadIdx.x; i < b1; i += (uint64_t)blockDim.x * kReadUnroll) {
        u32x4 v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) {
            const uint64_t j = i + (uint64_t)u * blockDim.x;
            v[u] = __builtin_nontemporal_load(p + (j < b1 ? j : b1 - 1));
        }
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == kReadMagic) sink[(uint64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

}  // namespace

// `launches` back-to-back launches on `stream`, launch i streaming the
// `bytes` at src + (i % rotate) * bytes once with `workgroups` workgroups of
// `threads` (256 or 512) threads (src holds rotate * bytes; 16-byte aligned,
// bytes a multiple of 16). The loop is here so that the host issues launches
// as fast as the runtime takes them. sink must hold workgroups * threads
// words and is written only in the case described at read_floor_kernel.
// Returns 0, -1 for a bad argument, or a hipError_t from a launch.
extern "C" int dsv4_read_floor(const void* src, uint64_t bytes, int rotate, int launches, int workgroups,
                               int threads, uint32_t* sink, hipStream_t stream) {
    if (!src || !sink || bytes == 0 || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) & 15u) != 0 ||
        rotate < 1 || launches < 1 || workgroups < 1 || workgroups > 65535 || (threads != 256 && threads != 512))
        return -1;
    const uint64_t n16 = bytes / 16;
    const uint64_t per = (n16 + (uint64_t)workgroups - 1) / (uint64_t)workgroups;
    const unsigned wgs = (unsigned)((n16 + per - 1) / per);
    for (int i = 0; i < launches; ++i) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(src) +
                                                              (uint64_t)(i % rotate) * bytes);
        hipLaunchKernelGGL(read_floor_kernel, dim3(wgs), dim3((unsigned)threads), 0, stream, p, n16, per, sink);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

// dst[i] = lo + uniform draw over [lo, hi] of SplitMix64 element (offset + i)
// of stream `seed`, for i < n. Returns 0, -1 for lo > hi or hi > 255, or a
// hipError_t from the launch.
extern "C" int dsv4_fill_uniform_u8(void* dst, uint64_t n, uint64_t seed, uint64_t offset, int lo,
                                    int hi, hipStream_t stream) {
    if (lo < 0 || hi > 255 || lo > hi) return -1;
    if (n == 0) return 0;
    const uint64_t threads = (n + 15) / 16;
    const uint64_t blocks = (threads + 255) / 256;
    hipLaunchKernelGGL(fill_uniform_u8_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<uint8_t*>(dst), n, seed, offset, (uint32_t)lo,
                       (uint32_t)(hi - lo + 1));
    return (int)hipGetLastError();
}
