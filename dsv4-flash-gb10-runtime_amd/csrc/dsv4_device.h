// dsv4_device.h — device helpers shared by the gfx950 decode kernels.
//
// Number formats (OCP Microscaling Formats v1.0):
//   e2m1  : 4-bit code s.ee.m, values {0, .5, 1, 1.5, 2, 3, 4, 6} with sign;
//           code 8 is -0.0. Two codes per byte, low nibble = even element
//           (reference runtime/mxfp4_unpack.py:105-112).
//   E8M0  : scale byte b -> 2^(b-127); b == 0xFF decodes to 0.0 on the kernel
//           path (reference kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:74-78),
//           b == 0 gives the fp32 subnormal 2^-127 exactly (no flush).
//   E4M3FN: 1.4.3, bias 7, no infinities, 0x7F/0xFF NaN, subnormals m*2^-9.
//
// Decode uses the gfx950 conversion instructions v_cvt_scalef32_pk_bf16_fp4 /
// _fp8 with a unit scale, which map each code to its exact bf16 value; the
// E8M0 block scale is applied once per block in fp32 (exact power of two).
// Dot products use v_dot2_f32_bf16 (two bf16 products added into an fp32
// accumulator), so one 16-byte MXFP4 block costs 16 conversions + 16 dots.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsv4 {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- scalars --

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
    return __uint_as_float(b << 16);
}

// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (sign kept).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// E8M0 byte -> fp32 scale, kernel convention (0xFF -> 0, 0 -> 2^-127).
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
    uint32_t bits = (b == 0u) ? 0x00400000u : (b << 23);
    bits = (b == 0xFFu) ? 0u : bits;
    return __uint_as_float(bits);
}

__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t u) {
    return __builtin_bit_cast(bf16x2, u);
}

__device__ __forceinline__ uint32_t as_u32(bf16x2 v) {
    return __builtin_bit_cast(uint32_t, v);
}

// Two e2m1 codes of byte SEL of w -> bf16 pair {low nibble, high nibble}.
template <int SEL>
__device__ __forceinline__ bf16x2 fp4x2_to_bf16x2(uint32_t w) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, SEL);
}

// Two E4M3FN bytes (low half-word when HI == false) -> bf16 pair.
template <bool HI>
__device__ __forceinline__ bf16x2 fp8x2_to_bf16x2(uint32_t w) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
}

__device__ __forceinline__ float dot2(bf16x2 a, bf16x2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
}

// ------------------------------------------------------------- block dots --

// Sum over one 32-element MXFP4 block (16 packed bytes in w) of code * x,
// with x given as 16 packed bf16 pairs (element order 2p, 2p+1 in pair p).
// The caller multiplies by the block's E8M0 scale.
__device__ __forceinline__ float fp4_block_dot(const u32x4 w, const uint32_t* xp) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = w[i];
        a0 = dot2(fp4x2_to_bf16x2<0>(d), as_bf16x2(xp[4 * i + 0]), a0);
        a1 = dot2(fp4x2_to_bf16x2<1>(d), as_bf16x2(xp[4 * i + 1]), a1);
        a0 = dot2(fp4x2_to_bf16x2<2>(d), as_bf16x2(xp[4 * i + 2]), a0);
        a1 = dot2(fp4x2_to_bf16x2<3>(d), as_bf16x2(xp[4 * i + 3]), a1);
    }
    return a0 + a1;
}

// Sum over 16 E4M3 bytes (w) of e4m3 * x, x as 8 packed bf16 pairs.
__device__ __forceinline__ float fp8_chunk_dot(const u32x4 w, const uint32_t* xp) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = w[i];
        a0 = dot2(fp8x2_to_bf16x2<false>(d), as_bf16x2(xp[2 * i + 0]), a0);
        a1 = dot2(fp8x2_to_bf16x2<true>(d), as_bf16x2(xp[2 * i + 1]), a1);
    }
    return a0 + a1;
}

// Marks a register value as modified (emits no instruction). Used inside
// loops whose weights stay in registers across iterations, so the compiler
// cannot hoist the per-iteration decode out of the loop and keep every decoded
// value live at once (which multiplies the register footprint).
__device__ __forceinline__ void reg_barrier(u32x4& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void reg_barrier(uint32_t& v) { asm volatile("" : "+v"(v)); }

// As reg_barrier, and additionally orders the decode of `v` after `dep` is
// computed: chaining blocks this way keeps one block's decoded values live at
// a time instead of letting the compiler decode every block up front.
__device__ __forceinline__ void reg_barrier_after(u32x4& v, float dep) {
    asm volatile("" : "+v"(v) : "v"(dep));
}

// ---------------------------------------------------------------- loads ----

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// Streaming (read-once) 16-byte load of weight data.
__device__ __forceinline__ u32x4 ld16_stream(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// 16-byte load without any alignment assumption (byte loads).
__device__ __forceinline__ u32x4 ld16_unaligned(const uint8_t* p) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = (uint32_t)p[4 * i] | ((uint32_t)p[4 * i + 1] << 8) |
               ((uint32_t)p[4 * i + 2] << 16) | ((uint32_t)p[4 * i + 3] << 24);
    return r;
}

// ----------------------------------------------------------- reductions ----

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Value held by the partner lane in a butterfly step over lane bit MASK.
// Partners differ in that bit (and, for 4 and 8, in lower bits too, via the
// mirror patterns); every pattern is an involution, which is all a butterfly
// needs. Bits 0-3 use DPP (quad_perm, row_half_mirror, row_mirror); bits 4
// and 5 use v_permlane16_swap / v_permlane32_swap, whose two results hold the
// own and the partner value, told apart by comparison with the own value.
template <int MASK>
__device__ __forceinline__ uint32_t wave_partner(uint32_t v) {
    if constexpr (MASK == 1) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false);
    else if constexpr (MASK == 2) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false);
    else if constexpr (MASK == 4) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false);
    else if constexpr (MASK == 8) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false);
    else if constexpr (MASK == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return r[0] == v ? r[1] : r[0];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return r[0] == v ? r[1] : r[0];
    }
}

__device__ __forceinline__ float partner_add(float keep, float send, int mask) {
    const uint32_t s = __float_as_uint(send);
    uint32_t o;
    switch (mask) {
        case 32: o = wave_partner<32>(s); break;
        case 16: o = wave_partner<16>(s); break;
        case 8: o = wave_partner<8>(s); break;
        case 4: o = wave_partner<4>(s); break;
        case 2: o = wave_partner<2>(s); break;
        default: o = wave_partner<1>(s); break;
    }
    return keep + __uint_as_float(o);
}

// Butterfly reduction of N values per lane over the 64 lanes of a wave
// (N a power of two, N <= 64), on the DPP / permlane paths. Each exchange step
// halves the number of live values, so N sums cost about N + 5 exchanges
// instead of 6N. On return every lane holds in v[0] the wave total of value
// index (lane >> (6 - log2 N)). Masks go 32, 16, ..., 1; the partner of a lane
// at mask m always has the opposite bit m, so "upper" is well defined.
template <int N>
struct WaveButterfly {
    static __device__ __forceinline__ void run(float* v, int lane, int mask) {
        constexpr int H = N / 2;
        const bool upper = (lane & mask) != 0;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float send = upper ? v[i] : v[i + H];
            const float keep = upper ? v[i + H] : v[i];
            v[i] = partner_add(keep, send, mask);
        }
        WaveButterfly<H>::run(v, lane, mask >> 1);
    }
};
template <>
struct WaveButterfly<1> {
    static __device__ __forceinline__ void run(float* v, int, int mask) {
#pragma unroll
        for (; mask > 0; mask >>= 1) v[0] = partner_add(v[0], v[0], mask);
    }
};

template <int N>
__device__ __forceinline__ void wave_reduce_n(float* v, int lane) {
    WaveButterfly<N>::run(v, lane, 32);
}

// Whole-wave reductions on the DPP / permlane paths (no LDS traffic):
// xor 1 and xor 2 via quad_perm, then row_half_mirror and row_mirror (which
// pair every lane with one in the other half of its 8- and 16-lane group),
// then v_permlane16_swap / v_permlane32_swap across rows and wave halves.
// Every lane ends with the result.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}

template <typename Op>
__device__ __forceinline__ uint32_t wave_allreduce_u32(uint32_t v, Op op) {
    v = op(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
    v = op(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
    v = op(v, dpp_u32<0x141>(v));  // row_half_mirror
    v = op(v, dpp_u32<0x140>(v));  // row_mirror
    {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = op(r[0], r[1]);
    }
    {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = op(r[0], r[1]);
    }
    return v;
}

// Maximum over the wave; NaN inputs are ignored (IEEE maxNum).
__device__ __forceinline__ float wave_max_f32(float v) {
    return __uint_as_float(wave_allreduce_u32(__float_as_uint(v), [](uint32_t a, uint32_t b) {
        return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    }));
}

__device__ __forceinline__ int wave_min_i32(int v) {
    return (int)wave_allreduce_u32((uint32_t)v, [](uint32_t a, uint32_t b) {
        return (uint32_t)min((int)a, (int)b);
    });
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return wave_allreduce_u32(v, [](uint32_t a, uint32_t b) { return max(a, b); });
}

// Maximum over the wave as a wave-uniform value: the four DPP steps reduce
// each 16-lane row, then the four row results meet through readlane and
// scalar max (shorter than the two permlane swaps plus a readfirstlane).
__device__ __forceinline__ uint32_t wave_max_u32_uniform(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    v = max(v, dpp_u32<0x140>(v));
    const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return max(max(r0, r1), max(r2, r3));
}

// Order-preserving key of a non-NaN float: a > b exactly when key(a) >
// key(b), except that -0 and +0 get different keys (callers map -0 to +0).
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    return __uint_as_float(wave_allreduce_u32(__float_as_uint(v), [](uint32_t a, uint32_t b) {
        return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
    }));
}

template <int N>
struct Log2 { static constexpr int value = 1 + Log2<N / 2>::value; };
template <>
struct Log2<1> { static constexpr int value = 0; };

// Index of the value whose total lane `lane` holds after wave_reduce_n<N>.
template <int N>
__device__ __forceinline__ int reduced_index(int lane) {
    return lane >> (6 - Log2<N>::value);
}
// True for exactly one lane per value index after wave_reduce_n<N>.
template <int N>
__device__ __forceinline__ bool reduced_owner(int lane) {
    return (lane & ((1 << (6 - Log2<N>::value)) - 1)) == 0;
}

__device__ __forceinline__ float silu_f32(float g) {
    return g / (1.0f + __expf(-g));
}

}  // namespace dsv4
