// fp8_e4m3_gemv.hip — FP8 E4M3FN GEMV with 128x128 E8M0 tile scales, gfx950.
//
//   y[t,n] = bf16( sum_k e4m3(W[n,k]) * 2^(S[n/128,k/128]-127) * x[t,k] )
//
// Three kernels share the decode (v_cvt_scalef32_pk_bf16_fp8: OCP e4m3fn
// on gfx950, exact in bf16) and the scale rule (the 128x128 tile scale is
// applied once per 16-byte chunk or 128-k tile sum):
//   - the general kernel (any K, unaligned operands): lane l owns the
//     16-byte chunks k = 1024*j + 16*l of every row it visits, kRows rows
//     per wave reduced together with one butterfly;
//   - the vector tile kernels (K in {1024, 2048, 4096, 8192}, aligned): one
//     wave instruction reads 1 KiB of one row, v_dot2_f32_bf16 per token;
//   - the matrix-core kernel for several tokens (v_mfma_f32_16x16x32_bf16),
//     taken by the shape rule use_mfma.
// N need not be a multiple of 128 (ceil(N/128) scale rows), unlike reference
// kernel/fp8-dense/fp8_e4m3_gemv.cu:148-154.

#include <algorithm>
#include <cstdio>
#include <initializer_list>

#include "dsv4_device.h"
#include "dsv4_kernels.h"

namespace {

using namespace dsv4;

constexpr int kTile = 128;
constexpr int kMaxK = 16384;    // reference FP8_GEMV_MAX_K (fp8_e4m3_gemv.cu:48-50)
constexpr int kMaxT = 16;
constexpr int kWaves = 4;
constexpr int kRows = 4;

struct Fp8Args {
    const uint16_t* x;
    int64_t xstride;            // elements between token rows of x
    const uint8_t* w;
    const uint8_t* s;
    int K;
    int N;
    int T;
    int64_t wrow;
    int64_t srow;
    uint16_t* y;
    int64_t ystride;            // elements between token rows of y
    // Groups (blockIdx.y): group g reads x + g*xgroup, weight rows
    // g*N .. g*N+N-1 (their scale rows (g*N+n)/128) and writes y + g*ygroup.
    int64_t xgroup;
    int64_t ygroup;
};

// A workgroup's view of its group: activation and output moved to the group,
// weight row index offset by g*N (the scale row follows the global row).
struct GroupView {
    const uint16_t* x;
    uint16_t* y;
    int64_t row0;
};

__device__ __forceinline__ GroupView group_view(const Fp8Args& a) {
    const int g = blockIdx.y;
    return GroupView{a.x + (int64_t)g * a.xgroup, a.y + (int64_t)g * a.ygroup, (int64_t)g * a.N};
}

template <bool ALIGNED>
__device__ __forceinline__ u32x4 load_w16(const uint8_t* p) {
    if constexpr (ALIGNED) return ld16(p);
    else return ld16_unaligned(p);
}

// Tile-scale formats: SF = 0, E8M0 bytes (the reference ABI,
// fp8_e4m3_gemv.cu:55-62); SF = 1, fp32 values (fp8_e4m3_gemv_f32s). A scale
// is loaded as its raw 32-bit pattern (the byte, or the float's bits) and
// turned into an fp32 multiplier where it is applied.
template <int SF>
__device__ __forceinline__ uint32_t scale_raw(const uint8_t* s, int64_t idx) {
    if constexpr (SF == 1) return reinterpret_cast<const uint32_t*>(s)[idx];
    else return s[idx];
}

template <int SF>
__device__ __forceinline__ float scale_value(uint32_t raw) {
    if constexpr (SF == 1) return __uint_as_float(raw);
    else return e8m0_to_f32(raw);
}

// grid = ceil(N / (kWaves*kRows)), block = 64*kWaves. A row is walked in
// segments of NC*1024 bytes (NC 16-byte chunks per lane, NC <= 4). With one
// segment (K <= 4096) the rows stay in registers across all T tokens;
// longer rows are streamed once per group of kGenTok tokens (every token of
// the group is accumulated from the segment in registers), so T <= 8 reads
// each weight byte once. Each token's sum runs over the segments and chunks
// in k order either way.
// LONG selects the segmented body (NC = 4, K > 4096) at compile time, so the
// one-segment kernels keep their smaller register budget.
constexpr int kGenTok = 8;

template <int NC, bool ALIGNED, bool LONG, int SF = 0>
__global__ __launch_bounds__(64 * kWaves) void fp8_gemv_kernel(const Fp8Args a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * kWaves + wave) * kRows;
    if (n0 >= a.N) return;
    const int nseg = (a.K + NC * 1024 - 1) / (NC * 1024);
    const GroupView gv = group_view(a);

    u32x4 wv[kRows][NC];
    float sc[kRows][NC];
    auto load_rows = [&](int seg) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int n = n0 + r;
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int k = (seg * NC + j) * 1024 + 16 * lane;
                if (n < a.N && k < a.K) {
                    const int64_t gn = gv.row0 + n;
                    wv[r][j] = load_w16<ALIGNED>(a.w + gn * a.wrow + k);
                    sc[r][j] = scale_value<SF>(scale_raw<SF>(a.s, (gn / kTile) * a.srow + k / kTile));
                } else {
                    wv[r][j] = u32x4{0u, 0u, 0u, 0u};
                    sc[r][j] = 0.f;
                }
            }
        }
    };
    auto accumulate = [&](const uint16_t* xt, int seg, float* acc) {
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            uint32_t xp[8];
            const int k = (seg * NC + j) * 1024 + 16 * lane;
            if (k < a.K) {
                if constexpr (ALIGNED) {
                    const u32x4* s4 = reinterpret_cast<const u32x4*>(xt + k);
                    const u32x4 v0 = s4[0], v1 = s4[1];
                    xp[0] = v0[0]; xp[1] = v0[1]; xp[2] = v0[2]; xp[3] = v0[3];
                    xp[4] = v1[0]; xp[5] = v1[1]; xp[6] = v1[2]; xp[7] = v1[3];
                } else {
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        xp[q] = (uint32_t)xt[k + 2 * q] | ((uint32_t)xt[k + 2 * q + 1] << 16);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) xp[q] = 0u;
            }
#pragma unroll
            for (int r = 0; r < kRows; ++r)
                acc[r] = fmaf(fp8_chunk_dot(wv[r][j], xp), sc[r][j], acc[r]);
        }
    };
    auto store = [&](int t, float* acc) {
        wave_reduce_n<kRows>(acc, lane);
        const int r = reduced_index<kRows>(lane);
        if (reduced_owner<kRows>(lane) && n0 + r < a.N)
            gv.y[(int64_t)t * a.ystride + n0 + r] = f32_to_bf16_bits(acc[0]);
    };
    if (!LONG || nseg == 1) {
        load_rows(0);
        for (int t = 0; t < a.T; ++t) {
            float acc[kRows];
#pragma unroll
            for (int r = 0; r < kRows; ++r) acc[r] = 0.f;
            accumulate(gv.x + (int64_t)t * a.xstride, 0, acc);
            store(t, acc);
        }
        return;
    }
    for (int t0 = 0; t0 < a.T; t0 += kGenTok) {
        float acc[kGenTok][kRows];
#pragma unroll
        for (int q = 0; q < kGenTok; ++q)
#pragma unroll
            for (int r = 0; r < kRows; ++r) acc[q][r] = 0.f;
        for (int seg = 0; seg < nseg; ++seg) {
            load_rows(seg);
#pragma unroll
            for (int q = 0; q < kGenTok; ++q)
                if (t0 + q < a.T) accumulate(gv.x + (int64_t)(t0 + q) * a.xstride, seg, acc[q]);
        }
#pragma unroll
        for (int q = 0; q < kGenTok; ++q)
            if (t0 + q < a.T) store(t0 + q, acc[q]);
    }
}

// The second matrix and the epilogue of the fused SwiGLU launch
// (fp8_e4m3_swiglu_gemv): y = bf16( silu(c(g)) * c_up(u) ), g and u the two
// GEMV outputs rounded to bf16, c a clamp to [-limit, limit] (none for
// limit <= 0), c_up the same clamp when clamp_up is set, else identity.
struct SwigluArgs {
    const uint8_t* w3;
    const uint8_t* s3;
    float limit;
    int clamp_up;
};

__device__ __forceinline__ float swiglu_clamp(float v, float limit) {
    return limit > 0.f ? fminf(fmaxf(v, -limit), limit) : v;
}

// Tile kernels for K in {1024, 2048, 4096, 8192} with 16-byte aligned rows
// and activations (the MLA projection shapes). A workgroup of 256 threads owns
// R = C*256/KC rows (KC = K/16 chunks per row); thread t takes the chunks
// t, t+256, ..., t+256*(C-1) of the workgroup's [R, KC] chunk grid, so every
// wave instruction reads 1 KiB of a single row, and its chunks use KS =
// max(1, KC/256) k-slices (one for K <= 4096, two for K = 8192). Each thread
// issues its activation slices for the first TT tokens first (16 bf16 per
// token and slice), then its C weight chunks (of each of the MAT matrices)
// and their tile-scale bytes, all unconditional (rows clamped, tokens past T
// clamped to T-1 and not stored), so everything is in flight after one issue
// pass. The weights stay in registers while the tokens are taken TT at a
// time: no weight byte is read twice, whatever T. Per-wave partials (C x TT
// values per matrix, one butterfly per matrix) meet in LDS and are added in a
// fixed order: deterministic, and with MAT = 2 each matrix's sums are the
// bits the single-matrix kernel produces.
template <int C, int TT, int KC, int MAT>
struct TileShape {
    static constexpr int kRowsWG = C * 256 / KC;
    static constexpr int KS = KC > 256 ? KC / 256 : 1;
    static constexpr int kVals = C * TT;
    static_assert(256 % KC == 0 || KC % 256 == 0, "chunks per row must divide or be a multiple of 256");
    static_assert(C % KS == 0, "every thread takes whole rows of slices");
};

// The body shared by the single-matrix, grouped and multi-matrix launches:
// workgroup `blk` of the matrix described by `a` and `gv`.
template <int C, int TT, int KC, int MAT, int SF = 0>
__device__ __forceinline__ void fp8_tile_body(const Fp8Args& a, const SwigluArgs& sw, const GroupView& gv,
                                              int blk, float (*part)[MAT][C][TT]) {
    static_assert(SF == 0 || MAT == 1, "fp32 tile scales on the single-matrix kernel only");
    using S = TileShape<C, TT, KC, MAT>;
    constexpr int kRowsWG = S::kRowsWG, KS = S::KS, kVals = S::kVals;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n0 = blk * kRowsWG;
    const int kb = 16 * (t % (KC < 256 ? KC : 256));   // k of slice 0; slice s adds 4096*s

    uint32_t xp[TT][KS][8];
    auto load_x = [&](int tok0) {
#pragma unroll
        for (int tok = 0; tok < TT; ++tok) {
            const uint16_t* xr = gv.x + (int64_t)min(tok0 + tok, a.T - 1) * a.xstride;
#pragma unroll
            for (int q = 0; q < KS; ++q) {
                const u32x4* s4 = reinterpret_cast<const u32x4*>(xr + kb + 4096 * q);
                const u32x4 v0 = s4[0], v1 = s4[1];
                xp[tok][q][0] = v0[0]; xp[tok][q][1] = v0[1]; xp[tok][q][2] = v0[2]; xp[tok][q][3] = v0[3];
                xp[tok][q][4] = v1[0]; xp[tok][q][5] = v1[1]; xp[tok][q][6] = v1[2]; xp[tok][q][7] = v1[3];
            }
        }
    };
    load_x(0);
    __builtin_amdgcn_sched_barrier(0);  // activation loads first
    u32x4 w[MAT][C];
    uint32_t sb[MAT][C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
        const int64_t gn = gv.row0 + min(n0 + (t + 256 * i) / KC, a.N - 1);
        const int k = kb + 4096 * (i % KS);
        w[0][i] = ld16_stream(a.w + gn * a.wrow + k);
        sb[0][i] = scale_raw<SF>(a.s, (gn / kTile) * a.srow + k / kTile);
        if constexpr (MAT == 2) {
            w[1][i] = ld16_stream(sw.w3 + gn * a.wrow + k);
            sb[1][i] = sw.s3[(gn / kTile) * a.srow + k / kTile];
        }
    }
    for (int tok0 = 0; tok0 < a.T; tok0 += TT) {
        if (tok0 > 0) {
            __syncthreads();    // the previous group's partials are consumed
            load_x(tok0);
        }
#pragma unroll
        for (int m = 0; m < MAT; ++m) {
            float acc[kVals];
#pragma unroll
            for (int i = 0; i < C; ++i) {
                const float sc = m == 0 ? scale_value<SF>(sb[m][i]) : e8m0_to_f32(sb[m][i]);
#pragma unroll
                for (int tok = 0; tok < TT; ++tok) acc[i * TT + tok] = fp8_chunk_dot(w[m][i], xp[tok][i % KS]) * sc;
            }
            wave_reduce_n<kVals>(acc, lane);
            const int v = reduced_index<kVals>(lane);
            if (reduced_owner<kVals>(lane)) part[wave][m][v / TT][v % TT] = acc[0];
        }
        __syncthreads();
        for (int o = t; o < kRowsWG * TT; o += 256) {
            const int r = o / TT;
            const int tok = o % TT;
            if (tok0 + tok >= a.T || n0 + r >= a.N) continue;
            float sum[MAT];
#pragma unroll
            for (int m = 0; m < MAT; ++m) {
                sum[m] = 0.f;
#pragma unroll
                for (int w2 = 0; w2 < kWaves; ++w2) {
#pragma unroll
                    for (int i = 0; i < C; ++i)
                        if ((64 * w2 + 256 * i) / KC == r) sum[m] += part[w2][m][i][tok];
                }
            }
            uint16_t out;
            if constexpr (MAT == 2) {
                const float g = swiglu_clamp(bf16_bits_to_f32(f32_to_bf16_bits(sum[0])), sw.limit);
                const float u0 = bf16_bits_to_f32(f32_to_bf16_bits(sum[1]));
                const float u = sw.clamp_up ? swiglu_clamp(u0, sw.limit) : u0;
                out = f32_to_bf16_bits(g / (1.0f + expf(-g)) * u);
            } else {
                out = f32_to_bf16_bits(sum[0]);
            }
            gv.y[(int64_t)(tok0 + tok) * a.ystride + n0 + r] = out;
        }
    }
}

// One matrix, or G row groups of one matrix (blockIdx.y, GroupView).
template <int C, int TT, int KC, int MAT, int SF = 0>
__global__ __launch_bounds__(256) void fp8_gemv_tile_kernel(const Fp8Args a, const SwigluArgs sw) {
    __shared__ float part[kWaves][MAT][C][TT];
    fp8_tile_body<C, TT, KC, MAT, SF>(a, sw, group_view(a), blockIdx.x, part);
}

// Several matrices that read the same activation (the pointer table of
// fp8_e4m3_gemv_multi): matrix m owns workgroups first[m] .. first[m+1]-1.
constexpr int kMaxMulti = 8;

struct MultiArgs {
    Fp8Args base;                       // x, xstride, K, T (w, s, N, strides, y per matrix below)
    int n_mats;
    int first[kMaxMulti + 1];
    const uint8_t* w[kMaxMulti];
    const uint8_t* s[kMaxMulti];
    int N[kMaxMulti];
    int64_t wrow[kMaxMulti];
    int64_t srow[kMaxMulti];
    uint16_t* y[kMaxMulti];
    int64_t ystride[kMaxMulti];
};

template <int C, int TT, int KC>
__global__ __launch_bounds__(256) void fp8_gemv_multi_kernel(const MultiArgs ma) {
    __shared__ float part[kWaves][1][C][TT];
    int m = 0;
#pragma unroll
    for (int j = 1; j < kMaxMulti; ++j) m += (j < ma.n_mats && (int)blockIdx.x >= ma.first[j]) ? 1 : 0;
    Fp8Args a = ma.base;
    a.w = ma.w[m];
    a.s = ma.s[m];
    a.N = ma.N[m];
    a.wrow = ma.wrow[m];
    a.srow = ma.srow[m];
    a.y = ma.y[m];
    a.ystride = ma.ystride[m];
    const GroupView gv{a.x, a.y, 0};
    fp8_tile_body<C, TT, KC, 1>(a, SwigluArgs{}, gv, (int)blockIdx.x - ma.first[m], part);
}

// Two to sixteen tokens on the matrix cores (v_mfma_f32_16x16x32_bf16). On
// the vector path every weight pair costs one v_dot2 per token, so at T = 8
// the dots, not the weight stream, set the time; here one instruction takes
// 16 rows x 32 k of weights against 32 k x 16 tokens.
//   Workgroup: R blocks of 16 rows (n0 .. n0+16R-1) x all of K; NW waves
//   split K, wave w owning k in [w*KW, (w+1)*KW), KW = 512*PASSES.
//   Lane l: row r = l%16 of each block and token column l%16, k-group
//   g = l/16. Per pass, load j (0..7) reads the 16 bytes k0 + 64j + 16g ..
//   +15 of row r of each block (one instruction covers 16 rows x 64 B) and
//   the activations of token l%16 at the same k (token columns T..15 read
//   zeros); each half (8 k) is one MFMA operand, exact bf16 from E4M3. The
//   R blocks share the activation registers. A 128-k scale tile is 2 loads;
//   its 4 MFMAs accumulate into a fresh fp32 tile sum, which is scaled and
//   added. The D operand gives lane l rows 4g..4g+3 for token l%16; each
//   row's tile scales come from the lane that loaded that row (ds_bpermute),
//   so 16-row blocks may straddle a 128-row scale tile (groups starting
//   mid-tile). The NW partial sums meet in LDS and are added in wave order.
constexpr int kMmaLoads = 8;        // 16-byte weight loads per lane per pass
constexpr int kMmaK = 64 * kMmaLoads;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 8 E4M3 bytes (two dwords) -> 8 bf16, element order kept.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t d0, uint32_t d1) {
    const bf16x2 p0 = fp8x2_to_bf16x2<false>(d0), p1 = fp8x2_to_bf16x2<true>(d0);
    const bf16x2 p2 = fp8x2_to_bf16x2<false>(d1), p3 = fp8x2_to_bf16x2<true>(d1);
    bf16x8 v;
    v[0] = p0[0]; v[1] = p0[1]; v[2] = p1[0]; v[3] = p1[1];
    v[4] = p2[0]; v[5] = p2[1]; v[6] = p3[0]; v[7] = p3[1];
    return v;
}

// Per-lane operand pointers of the matrix-core kernels. A-operand row rho
// (0..15) of a 16-row MFMA block is weight row n0 + RR*b + rho % RR at k
// offset 512 * (rho / RR) when S > 1 (S 512-k blocks per MFMA, RR = 16/S,
// fp8_gemv_mfma_split_kernel) and at offset 0 otherwise. RR < 16 with S = 1
// repeats the block's RR rows (their extra D rows are never stored). A row's
// sums do not depend on RR or S: they are the same MFMAs on the same operands.
// Weights are loaded as whole 128-byte lines, instruction q (0, 1) of a
// 128-k chunk giving lane l A-row 8q + l/8 and bytes 16(l%8)..+15 of the
// chunk (8 lines per instruction, where loads in the MFMA layout would touch
// 16 half lines), and reach the MFMA layout through the wave's LDS area.
template <int MAT, int R, int SF, int RR, int S>
struct MmaRows {
    const uint8_t* lw[MAT][R][2];   // this lane's line piece of A-rows lane/8 and 8 + lane/8, k = 0
    const uint8_t* s[MAT][R];       // the tile-scale row of this lane's A-row lane%16 (SF = 1: fp32 values)
    uint32_t xo[2];                 // byte offset in x of this lane's line piece of B-rows lane/8 and 8 + lane/8
                                    // (k = 0), or the buffer bound (zeros) for a token at or past T
    bool xq1;                       // B-rows 8..15 hold tokens (S > 1, or T > 8)
};

template <int MAT, int R, int SF, int RR, int S>
__device__ __forceinline__ MmaRows<MAT, R, SF, RR, S> mma_rows(const Fp8Args& a, const SwigluArgs& sw,
                                                               const GroupView& gv, int n0, int lane) {
    static_assert(RR == 16 || RR == 8 || RR == 4 || RR == 2, "real rows per block (a divisor of 16)");
    static_assert(S == 1 || S * RR == 16, "S blocks per MFMA take 16/S rows each");
    static_assert(SF == 0 || MAT == 1, "fp32 tile scales: one matrix");
    constexpr int sb = SF == 1 ? 4 : 1;                 // bytes per scale
    MmaRows<MAT, R, SF, RR, S> m;
    const int r = lane & 15;
    // B-row rho: token rho (S = 1), or token rho % RR at k offset 512 * (rho / RR).
    const uint32_t xbytes = (uint32_t)(((int64_t)(a.T - 1) * a.xstride + a.K) * 2);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int rho = 8 * q + (lane >> 3);
        const int tok = S > 1 ? rho % RR : rho;
        const int ko = S > 1 ? (rho / RR) * kMmaK : 0;
        m.xo[q] = tok < a.T ? (uint32_t)(((int64_t)tok * a.xstride + ko) * 2 + 16 * (lane & 7)) : xbytes;
    }
    m.xq1 = S > 1 || a.T > 8;
#pragma unroll
    for (int b = 0; b < R; ++b) {
        const int64_t gn = gv.row0 + min(n0 + RR * b + (r % RR), a.N - 1);
        const int64_t so = ((gn / kTile) * a.srow + (S > 1 ? (r / RR) * (kMmaK / kTile) : 0)) * sb;
        m.s[0][b] = a.s + so;
        if constexpr (MAT == 2) m.s[1][b] = sw.s3 + so;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int rho = 8 * q + (lane >> 3);
            const int64_t gl = gv.row0 + min(n0 + RR * b + (rho % RR), a.N - 1);
            const int64_t lo = gl * a.wrow + (S > 1 ? (rho / RR) * kMmaK : 0) + 16 * (lane & 7);
            m.lw[0][b][q] = a.w + lo;
            if constexpr (MAT == 2) m.lw[1][b][q] = sw.w3 + lo;
        }
    }
    return m;
}

// LDS operations of one wave run in order; the fences only keep the compiler
// from moving them across (the staged area is the wave's own, so no barrier).
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kStg = 9;                 // 16-byte slots per staged 128-byte weight row (144-byte stride)
constexpr int kXStg = 17;               // 16-byte slots per staged 256-byte activation row (272-byte stride)
// A wave's staging area in 16-byte slots: 16 activation rows, then 16 weight
// rows per matrix.
constexpr int stg_slots(int mat) { return 16 * kXStg + mat * 16 * kStg; }

// One 512-k block (k0 .. k0+511) of R 16-row blocks against the token
// columns. Every load of the block is issued before the first multiply
// (loads complete in issue order, so each multiply waits only for its own):
// per 128-k chunk c (one scale tile) the activation lines of B-rows
// 8q + lane/8 (bytes 128h + 16(lane%8) of the chunk's 256, h = 0, 1; the
// second half of the rows only where they hold tokens) and the weight lines
// of A-rows 8q + lane/8 (bytes 16(lane%8) of the chunk's 128). Then, chunk by
// chunk, the wave writes them to its staging area stg (activations: 16 rows
// at a 272-byte stride; weights of matrix m: 16 rows at a 144-byte stride
// each, reused for every row block) and reads back, as lane (r, g), B-row
// r's bytes 128h + 32g .. +31 and A-row r's bytes 16g and 64 + 16g: the
// operands the MFMA layout would have loaded, so the sums are unchanged (the
// B columns of tokens at or past T read zeros or stale slots, and their D
// columns are never stored). Each chunk's 4 MFMAs per (matrix, row block)
// accumulate into a fresh fp32 tile sum that is scaled and added to acc
// (fresh zeros on entry). With S = 1 and RR <= 8, A-rows 8..15 repeat rows
// 0..7: only the first weight line of a chunk is loaded and staged.
template <int MAT, int R, int SF, int RR, int S>
__device__ __forceinline__ void mma_kblock(const MmaRows<MAT, R, SF, RR, S>& rows, __amdgpu_buffer_rsrc_t xrs,
                                           int k0, int lane, u32x4* stg, f32x4 (&acc)[MAT][R]) {
    constexpr int kChunks = kMmaK / kTile;
    constexpr bool HALF = S == 1 && RR <= 8;
    const int g = lane >> 4;
    // This lane's A-row: the block's 4 tile scales (SF = 0: bytes packed in a
    // dword; SF = 1: the fp32 bit patterns).
    uint32_t s4[MAT][R];
    uint32_t sf[R][4];
#pragma unroll
    for (int m = 0; m < MAT; ++m)
#pragma unroll
        for (int b = 0; b < R; ++b) {
            if constexpr (SF == 0) {
                const uint8_t* sp = rows.s[m][b] + k0 / kTile;
                s4[m][b] = (uint32_t)sp[0] | ((uint32_t)sp[1] << 8) | ((uint32_t)sp[2] << 16) |
                           ((uint32_t)sp[3] << 24);
            } else {
                const uint32_t* sp = reinterpret_cast<const uint32_t*>(rows.s[m][b]) + k0 / kTile;
#pragma unroll
                for (int q = 0; q < 4; ++q) sf[b][q] = sp[q];
            }
        }
    u32x4 xl[kChunks][2][2];            // chunk, row half q, byte half h
    u32x4 wl[MAT][R][kChunks][2];       // chunk, row half q
    const bool xq1 = rows.xq1;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (q == 1 && !xq1) continue;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                xl[c][q][h] = __builtin_amdgcn_raw_buffer_load_b128(
                    xrs, (int)(rows.xo[q] + (uint32_t)(k0 + kTile * c) * 2u + 128u * h), 0, 0);
        }
#pragma unroll
        for (int b = 0; b < R; ++b)
#pragma unroll
            for (int m = 0; m < MAT; ++m)
#pragma unroll
                for (int q = 0; q < (HALF ? 1 : 2); ++q)
                    wl[m][b][c][q] = ld16_stream(rows.lw[m][b][q] + k0 + kTile * c);
    }
    __builtin_amdgcn_sched_barrier(0);
    // Rows 4g..4g+3 of each block's D operand: their tile scales come from
    // the lanes that hold those A-rows.
    uint32_t srow[MAT][R][4];
    if constexpr (SF == 0) {
#pragma unroll
        for (int m = 0; m < MAT; ++m)
#pragma unroll
            for (int b = 0; b < R; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    srow[m][b][i] = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * g + i), (int)s4[m][b]);
    }
    u32x4* stx = stg;
    const int xw = (lane >> 3) * kXStg + (lane & 7);                  // + 8 * kXStg for q = 1, + 8 for h = 1
    const int xr = (lane & 15) * kXStg + 2 * g;                       // + 8 for bytes 128..255
    const int wslot = (lane >> 3) * kStg + (lane & 7);                // + 8 * kStg for the second line
    const int rslot = (HALF ? (lane & 7) : (lane & 15)) * kStg + g;   // + 4 for bytes 64..127
#pragma unroll
    for (int tile = 0; tile < kChunks; ++tile) {
        wave_lds_order();   // the previous chunk's reads come first
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            stx[xw + 8 * h] = xl[tile][0][h];
            if (xq1) stx[xw + 8 * kXStg + 8 * h] = xl[tile][1][h];
        }
        wave_lds_order();
        u32x4 xv[2][2];     // [h][e]: B-row r's 16 bytes at 128h + 32g + 16e of the chunk
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 2; ++e) xv[h][e] = stx[xr + 8 * h + e];
#pragma unroll
        for (int b = 0; b < R; ++b)
#pragma unroll
            for (int m = 0; m < MAT; ++m) {
                u32x4* st = stg + 16 * kXStg + m * 16 * kStg;
                wave_lds_order();
                st[wslot] = wl[m][b][tile][0];
                if constexpr (!HALF) st[wslot + 8 * kStg] = wl[m][b][tile][1];
                wave_lds_order();
                const u32x4 wv[2] = {st[rslot], st[rslot + 4]};
                f32x4 ts = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const bf16x8 a0 = fp8x8_to_bf16x8(wv[h][0], wv[h][1]);
                    const bf16x8 a1 = fp8x8_to_bf16x8(wv[h][2], wv[h][3]);
                    ts = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, __builtin_bit_cast(bf16x8, xv[h][0]), ts, 0, 0, 0);
                    ts = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, __builtin_bit_cast(bf16x8, xv[h][1]), ts, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float sc;
                    if constexpr (SF == 0) sc = e8m0_to_f32((srow[m][b][i] >> (8 * tile)) & 0xFFu);
                    else sc = __uint_as_float((uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * g + i), (int)sf[b][tile]));
                    acc[m][b][i] = fmaf(ts[i], sc, acc[m][b][i]);
                }
            }
    }
}

// The activation rows through a buffer bounded at the T token rows: lanes
// whose B-row holds no token read zeros at the bound without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mma_x_buffer(const Fp8Args& a, const GroupView& gv) {
    const int xbytes = (int)(((int64_t)(a.T - 1) * a.xstride + a.K) * 2);   // < 2^31 (use_mfma)
    return __builtin_amdgcn_make_buffer_rsrc((void*)gv.x, (short)0, xbytes, 0x00020000);
}

// The workgroup's outputs: the partial sums of nblk 512-k blocks, part[kb],
// added in k order (kb = 0, 1, ...), then rounded to bf16 (with MAT = 2 the
// SwiGLU of the two rounded sums).
template <int MAT, int R, int RR, int NB>
__device__ __forceinline__ void mma_store(const Fp8Args& a, const SwigluArgs& sw, const GroupView& gv, int n0,
                                          int nblk, int nthreads, const float (*part)[MAT][16 * R][16]) {
    for (int o = threadIdx.x; o < 16 * RR * R; o += nthreads) {
        const int tok = o / (RR * R);
        const int rr = o % (RR * R);
        const int prow = 16 * (rr / RR) + rr % RR;   // the row's D row in its 16-row block
        if (tok >= a.T || n0 + rr >= a.N) continue;
        float sum[MAT];
#pragma unroll
        for (int m = 0; m < MAT; ++m) {
            sum[m] = 0.f;
            if constexpr (NB > 0) {
#pragma unroll
                for (int kb = 0; kb < NB; ++kb) sum[m] += part[kb][m][prow][tok];
            } else {
                for (int kb = 0; kb < nblk; ++kb) sum[m] += part[kb][m][prow][tok];
            }
        }
        uint16_t out;
        if constexpr (MAT == 2) {
            const float gt = swiglu_clamp(bf16_bits_to_f32(f32_to_bf16_bits(sum[0])), sw.limit);
            const float u0 = bf16_bits_to_f32(f32_to_bf16_bits(sum[1]));
            const float u = sw.clamp_up ? swiglu_clamp(u0, sw.limit) : u0;
            out = f32_to_bf16_bits(gt / (1.0f + expf(-gt)) * u);
        } else {
            out = f32_to_bf16_bits(sum[0]);
        }
        gv.y[(int64_t)tok * a.ystride + n0 + rr] = out;
    }
}

// stg: the workgroup's staging areas (stg_slots(MAT) per wave).
template <int NW, int PASSES, int MAT, int R, int SF = 0>
__device__ __forceinline__ void fp8_mfma_body(const Fp8Args& a, const SwigluArgs& sw, const GroupView& gv,
                                              int blk, float (*part)[MAT][16 * R][16], u32x4* stg) {
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int n0 = blk * 16 * R;
    const __amdgpu_buffer_rsrc_t xrs = mma_x_buffer(a, gv);
    const MmaRows<MAT, R, SF, 16, 1> rows = mma_rows<MAT, R, SF, 16, 1>(a, sw, gv, n0, lane);
    // One accumulator per pass: each 512-k block's sum starts from zero, so
    // a wave of several passes produces exactly the partials that one wave
    // per block would (the blocks are added in k order at the end).
    f32x4 acc[PASSES][MAT][R];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
#pragma unroll
        for (int m = 0; m < MAT; ++m)
#pragma unroll
            for (int b = 0; b < R; ++b) acc[p][m][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        mma_kblock<MAT, R, SF, 16, 1>(rows, xrs, (wave * PASSES + p) * kMmaK, lane, stg + wave * stg_slots(MAT),
                                      acc[p]);
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
#pragma unroll
        for (int m = 0; m < MAT; ++m)
#pragma unroll
            for (int b = 0; b < R; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) part[wave * PASSES + p][m][16 * b + 4 * g + i][r] = acc[p][m][b][i];
    __syncthreads();
    mma_store<MAT, R, 16, NW * PASSES>(a, sw, gv, n0, NW * PASSES, 64 * NW, part);
}

// One matrix, or G row groups of one matrix (blockIdx.y); grid.x = ceil(N/(16R)).
template <int NW, int PASSES, int MAT, int R, int SF = 0>
__global__ __launch_bounds__(64 * NW) void fp8_gemv_mfma_kernel(const Fp8Args a, const SwigluArgs sw) {
    __shared__ float part[NW * PASSES][MAT][16 * R][16];
    __shared__ u32x4 stg[NW * stg_slots(MAT)];
    fp8_mfma_body<NW, PASSES, MAT, R, SF>(a, sw, group_view(a), blockIdx.x, part, stg);
}

// Rows longer than the tile set (K > 4096, a multiple of 512, at most
// kLongBlocks blocks of 512 k): the workgroup's waves (blockDim.x / 64 of
// them) take the 512-k blocks kb = wave, wave + waves, ..., each into a fresh
// sum, so the partials, and their k-order total, do not depend on the wave
// count. RR real rows per workgroup (one 16-row MFMA block): fewer than 16
// spread a short matrix over more workgroups, each reading all of x.
constexpr int kLongBlocks = 32;

template <int RR, int SF>
__global__ __launch_bounds__(1024) void fp8_gemv_mfma_long_kernel(const Fp8Args a) {
    // long_lds_bytes: the partials of the K/512 blocks, then the waves' staging areas
    extern __shared__ __align__(16) uint8_t lds[];
    float (*part)[1][16][16] = reinterpret_cast<float (*)[1][16][16]>(lds);
    u32x4* stg = reinterpret_cast<u32x4*>(lds + (a.K / kMmaK) * 16 * 16 * 4);
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int waves = (int)(blockDim.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const GroupView gv = group_view(a);
    const int n0 = (int)blockIdx.x * RR;
    const __amdgpu_buffer_rsrc_t xrs = mma_x_buffer(a, gv);
    const MmaRows<1, 1, SF, RR, 1> rows = mma_rows<1, 1, SF, RR, 1>(a, SwigluArgs{}, gv, n0, lane);
    const int nblk = a.K / kMmaK;
    for (int kb = wave; kb < nblk; kb += waves) {
        f32x4 acc[1][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}};
        mma_kblock<1, 1, SF, RR, 1>(rows, xrs, kb * kMmaK, lane, stg + wave * stg_slots(1), acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) part[kb][0][4 * g + i][r] = acc[0][0][i];
    }
    __syncthreads();
    mma_store<1, 1, RR, 0>(a, SwigluArgs{}, gv, n0, nblk, (int)blockDim.x, part);
}

// Long rows with few tokens (T <= 16/S): one 16x16x32 MFMA multiplies S
// 512-k blocks at once. Lane r = 16h/S + q (q < 16/S) supplies A row r as
// weight row n0 + q at block S*kp + h and B column r as token q at the same
// block; the D quadrant of rows and columns 16h/S .. 16(h+1)/S - 1 is then
// block S*kp + h's product for the workgroup's 16/S rows and tokens, and the
// off-diagonal quadrants (rows of one block against tokens of another) are
// dropped. A lane holds D rows 4g..4g+3 of column r, so lanes with
// g / (4/S) == h hold the diagonal. Each block's partial is formed as in
// fp8_gemv_mfma_long_kernel (same MFMAs per 128-k tile, same tile scales,
// now taken from the lane that loaded the row at that block), and the
// partials are added in k order: the results are that kernel's bits, with
// no repeated rows or zero token columns (half or a quarter of the
// instructions per output).
template <int S, int SF>
__global__ __launch_bounds__(1024) void fp8_gemv_mfma_split_kernel(const Fp8Args a) {
    constexpr int RB = 16 / S;                       // rows and tokens per workgroup
    extern __shared__ __align__(16) uint8_t lds[];      // as fp8_gemv_mfma_long_kernel
    float (*part)[1][16][16] = reinterpret_cast<float (*)[1][16][16]>(lds);
    u32x4* stg = reinterpret_cast<u32x4*>(lds + (a.K / kMmaK) * 16 * 16 * 4);
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int waves = (int)(blockDim.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const int h = r / RB;
    const int q = r % RB;
    const GroupView gv = group_view(a);
    const int n0 = (int)blockIdx.x * RB;
    const __amdgpu_buffer_rsrc_t xrs = mma_x_buffer(a, gv);
    const MmaRows<1, 1, SF, RB, S> rows = mma_rows<1, 1, SF, RB, S>(a, SwigluArgs{}, gv, n0, lane);
    const int nq = a.K / (S * kMmaK);
    for (int kp = wave; kp < nq; kp += waves) {
        f32x4 acc[1][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}};
        mma_kblock<1, 1, SF, RB, S>(rows, xrs, kp * S * kMmaK, lane, stg + wave * stg_slots(1), acc);
        if (g / (4 / S) == h) {
#pragma unroll
            for (int i = 0; i < 4; ++i) part[S * kp + h][0][4 * g + i - RB * h][q] = acc[0][0][i];
        }
    }
    __syncthreads();
    mma_store<1, 1, RB, 0>(a, SwigluArgs{}, gv, n0, S * nq, (int)blockDim.x, part);
}

// The matrices of fp8_e4m3_gemv_multi: matrix m owns workgroups
// first[m] .. first[m+1]-1, 16 rows each.
template <int NW>
__global__ __launch_bounds__(64 * NW) void fp8_gemv_multi_mfma_kernel(const MultiArgs ma) {
    __shared__ float part[NW][1][16][16];
    __shared__ u32x4 stg[NW * stg_slots(1)];
    int m = 0;
#pragma unroll
    for (int j = 1; j < kMaxMulti; ++j) m += (j < ma.n_mats && (int)blockIdx.x >= ma.first[j]) ? 1 : 0;
    Fp8Args a = ma.base;
    a.w = ma.w[m];
    a.s = ma.s[m];
    a.N = ma.N[m];
    a.wrow = ma.wrow[m];
    a.srow = ma.srow[m];
    a.y = ma.y[m];
    a.ystride = ma.ystride[m];
    const GroupView gv{a.x, a.y, 0};
    fp8_mfma_body<NW, 1, 1, 1>(a, SwigluArgs{}, gv, (int)blockIdx.x - ma.first[m], part, stg);
}

// RMSNorm folded into the GEMV that consumes it (fp8_e4m3_rmsnorm_gemv):
//   v = x + residual (fp32; or x alone), new_residual = bf16(v),
//   x_norm = bf16( (g * bf16(v)) * rsqrt(sum(v^2) / K + eps) ),  y = W . x_norm
// with the bits of librmsnorm_fuse's kernels. The library gives thread q
// the 8-element piece q and reduces each wave's 64 sums of squares with the
// xor butterfly (lane distances 32, 16, ..., 1), then adds the wave totals
// in order. Here thread t's GEMV slice is pieces p = 2(t % KC) and p + 1, so
// the row is read once: lanes j of a wave hold the library's lanes 2j and
// 2j + 1 (mod 64) of waves 2w' and 2w' + 1 (lanes 0-31 and 32-63). The
// library's steps at distance 32 .. 2 pair those lanes' j ^ 16 .. j ^ 1 with
// the same piece slot, and its last step adds the two slots of one lane: the
// same additions on the same operands. Every element is then normalised by
// the same expression. The thread then normalises its own 16-element GEMV
// slice and proceeds as fp8_gemv_tile_kernel. Workgroup 0 writes x_norm and
// new_residual. The loads are issued activation, residual and weight-scale
// slices first, then the weights, so the norm is computed while the weights
// stream in.
struct NormArgs {
    const uint16_t* res;        // [T, K] or null
    const uint16_t* g;          // [K]
    float eps;
    uint16_t* xnorm;            // [T, K]
    uint16_t* new_res;          // [T, K] (with res)
};

__device__ __forceinline__ void unpack8_f32(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf16_bits_to_f32(v[i] & 0xFFFFu);
        f[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16);
    }
}

// GEMV = false: the norm alone (x_norm and new_residual, one workgroup); the
// multi-token entry then runs the matrix-core GEMV on x_norm.
template <int C, int TT, int KC, bool RESID, bool GEMV = true>
__global__ __launch_bounds__(256) void fp8_norm_gemv_tile_kernel(const Fp8Args a, const NormArgs nm) {
    constexpr int kRowsWG = C * 256 / KC;
    constexpr int kVals = C * TT;
    constexpr int kNV = KC / 128;               // 8-element chunks per thread in the norm's order
    __shared__ float part[kWaves][C][TT];
    __shared__ float red[TT][kWaves * kNV];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n0 = blockIdx.x * kRowsWG;
    const int k = 16 * (t % KC);
    const int K = a.K;

    // The GEMV slice of x, residual and g (the norm reads the same pieces).
    u32x4 sx[TT][2], sr[TT][2], sg[2];
#pragma unroll
    for (int tok = 0; tok < TT; ++tok) {
        const int64_t row = (int64_t)min(tok, a.T - 1) * K;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            sx[tok][h] = *reinterpret_cast<const u32x4*>(a.x + row + k + 8 * h);
            if constexpr (RESID) sr[tok][h] = *reinterpret_cast<const u32x4*>(nm.res + row + k + 8 * h);
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) sg[h] = *reinterpret_cast<const u32x4*>(nm.g + k + 8 * h);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 w[C];
    uint32_t sb[C];
    if constexpr (GEMV) {
#pragma unroll
        for (int i = 0; i < C; ++i) {
            const int64_t gn = min(n0 + (t + 256 * i) / KC, a.N - 1);
            w[i] = ld16_stream(a.w + gn * a.wrow + k);
            sb[i] = a.s[(gn / kTile) * a.srow + k / kTile];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // Sum of squares per token, in the order of rmsnorm_vec_kernel (above):
    // this wave's lanes 0-31 and 32-63 end with the totals of the library's
    // waves 2w' and 2w' + 1, w' = wave % (KC / 64) (with KC = 128 waves 2
    // and 3 repeat waves 0 and 1 and write nothing).
#pragma unroll
    for (int tok = 0; tok < TT; ++tok) {
        float ss[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float xa[8], ra[8];
            unpack8_f32(sx[tok][h], xa);
            if constexpr (RESID) unpack8_f32(sr[tok][h], ra);
            ss[h] = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = RESID ? xa[e] + ra[e] : xa[e];
                ss[h] = fmaf(v, v, ss[h]);
            }
#pragma unroll
            for (int m = 16; m > 0; m >>= 1) ss[h] += __shfl_xor(ss[h], m, 64);
        }
        const float wsum = ss[0] + ss[1];
        if ((lane & 31) == 0 && wave < KC / 64) red[tok][2 * wave + (lane >> 5)] = wsum;
    }
    __syncthreads();
    const bool writer = blockIdx.x == 0 && t < KC;
    uint32_t xp[TT][8];
    float gf[16];
    unpack8_f32(sg[0], gf);
    unpack8_f32(sg[1], gf + 8);
#pragma unroll
    for (int tok = 0; tok < TT; ++tok) {
        float total = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves * kNV; ++w2) total += red[tok][w2];
        const float rms = rsqrtf(total * (1.0f / (float)K) + nm.eps);
        float xa[16], ra[16];
        unpack8_f32(sx[tok][0], xa);
        unpack8_f32(sx[tok][1], xa + 8);
        if constexpr (RESID) {
            unpack8_f32(sr[tok][0], ra);
            unpack8_f32(sr[tok][1], ra + 8);
        }
        uint16_t nb[16], tb[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float v = xa[e];
            if constexpr (RESID) {
                tb[e] = f32_to_bf16_bits(xa[e] + ra[e]);
                v = bf16_bits_to_f32(tb[e]);
            }
            nb[e] = f32_to_bf16_bits((gf[e] * v) * rms);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) xp[tok][q] = (uint32_t)nb[2 * q] | ((uint32_t)nb[2 * q + 1] << 16);
        if (writer && tok < a.T) {
            const int64_t o = (int64_t)tok * K + k;
            u32x4 lo, hi;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                lo[q] = xp[tok][q];
                hi[q] = xp[tok][4 + q];
            }
            *reinterpret_cast<u32x4*>(nm.xnorm + o) = lo;
            *reinterpret_cast<u32x4*>(nm.xnorm + o + 8) = hi;
            if constexpr (RESID) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    lo[q] = (uint32_t)tb[2 * q] | ((uint32_t)tb[2 * q + 1] << 16);
                    hi[q] = (uint32_t)tb[8 + 2 * q] | ((uint32_t)tb[8 + 2 * q + 1] << 16);
                }
                *reinterpret_cast<u32x4*>(nm.new_res + o) = lo;
                *reinterpret_cast<u32x4*>(nm.new_res + o + 8) = hi;
            }
        }
    }

    if constexpr (!GEMV) return;
    float acc[kVals];
#pragma unroll
    for (int i = 0; i < C; ++i) {
        const float sc = e8m0_to_f32(sb[i]);
#pragma unroll
        for (int tok = 0; tok < TT; ++tok) acc[i * TT + tok] = fp8_chunk_dot(w[i], xp[tok]) * sc;
    }
    wave_reduce_n<kVals>(acc, lane);
    const int v = reduced_index<kVals>(lane);
    if (reduced_owner<kVals>(lane)) part[wave][v / TT][v % TT] = acc[0];
    __syncthreads();
    for (int o = t; o < kRowsWG * TT; o += 256) {
        const int r = o / TT;
        const int tok = o % TT;
        if (tok >= a.T || n0 + r >= a.N) continue;
        float sum = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; ++w2) {
#pragma unroll
            for (int i = 0; i < C; ++i)
                if ((64 * w2 + 256 * i) / KC == r) sum += part[w2][i][tok];
        }
        a.y[(int64_t)tok * a.ystride + n0 + r] = f32_to_bf16_bits(sum);
    }
}

// One thread per 16 bytes of a row.
__global__ __launch_bounds__(256) void fp8_dequant_kernel(const uint8_t* w, const uint8_t* s, int K,
                                                          int N, int64_t wrow, int64_t srow,
                                                          uint16_t* out) {
    const int nchunk = K / 16;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)N * nchunk) return;
    const int n = (int)(idx / nchunk);
    const int k = (int)(idx % nchunk) * 16;
    const u32x4 v = ld16_unaligned(w + (int64_t)n * wrow + k);
    const float sc = e8m0_to_f32(s[(int64_t)(n / kTile) * srow + k / kTile]);
    uint16_t* o = out + (int64_t)n * K + k;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = as_u32(fp8x2_to_bf16x2<false>(v[i]));
        const uint32_t hi = as_u32(fp8x2_to_bf16x2<true>(v[i]));
        o[4 * i + 0] = f32_to_bf16_bits(bf16_bits_to_f32(lo & 0xFFFFu) * sc);
        o[4 * i + 1] = f32_to_bf16_bits(bf16_bits_to_f32(lo >> 16) * sc);
        o[4 * i + 2] = f32_to_bf16_bits(bf16_bits_to_f32(hi & 0xFFFFu) * sc);
        o[4 * i + 3] = f32_to_bf16_bits(bf16_bits_to_f32(hi >> 16) * sc);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The extensions reject a null operand before any launch; the drop-in
// fp8_e4m3_gemv_m1 keeps the reference's checks (shapes only).
constexpr int kNullOperand = -10;

bool operands_set(const char* who, std::initializer_list<const void*> ps) {
    for (const void* p : ps) {
        if (p == nullptr) {
            std::fprintf(stderr, "%s: a required pointer is null\n", who);
            return false;
        }
    }
    return true;
}

int validate(int K, int N) {
    if (K % kTile != 0 || K < kTile) {
        std::fprintf(stderr, "fp8_e4m3_gemv: K=%d not a positive multiple of %d\n", K, kTile);
        return -1;
    }
    if (K > kMaxK) {
        std::fprintf(stderr, "fp8_e4m3_gemv: K=%d > %d\n", K, kMaxK);
        return -3;
    }
    if (N < 1) {
        std::fprintf(stderr, "fp8_e4m3_gemv: N=%d < 1\n", N);
        return -4;
    }
    return 0;
}

bool tile_k(int K) { return K == 1024 || K == 2048 || K == 4096 || K == 8192; }

bool tile_ok(const Fp8Args& a) {
    return aligned16(a.x) && aligned16(a.w) && (a.wrow % 16 == 0) && (a.T == 1 || a.xstride % 8 == 0) &&
           (a.xgroup % 8 == 0) && tile_k(a.K);
}

// Chunks per thread of the vector tile kernels: two up to K = 4096 (twice
// the workgroups of four, which measured 2-14% faster at the MLA shapes,
// most at small N and several tokens), four at K = 8192 (two k-slices per
// thread; two chunks there measured 8% slower). A row's chunks are reduced
// by the same lanes and waves either way, so the results do not depend on it.
constexpr int tile_c(int K) { return K > 4096 ? 4 : 2; }

// Rows per workgroup of the tile kernels.
int tile_rows(int K) { return tile_c(K) * 256 / (K / 16); }

// Tokens per group: all of them up to 16 (8 with two matrices), at most 4 per
// group with two k-slices per thread (K = 8192), which hold twice the
// activation registers.
int tile_tt(int T, int K, int MAT) {
    const int cap = K > 4096 ? 4 : (MAT == 2 ? 8 : 16);
    const int tt = T == 1 ? 1 : (T == 2 ? 2 : (T <= 4 ? 4 : (T <= 8 ? 8 : 16)));
    return tt < cap ? tt : cap;
}

// Launch the tile kernel for TT tokens per group at the row length K (K = 8192
// only with TT <= 4: tile_tt never asks for more there).
template <int TT, int MAT, int SF = 0>
void launch_tile_tt(const Fp8Args& a, const SwigluArgs& sw, dim3 grid, hipStream_t stream) {
    switch (a.K) {
        case 1024: hipLaunchKernelGGL((fp8_gemv_tile_kernel<tile_c(1024), TT, 64, MAT, SF>), grid, dim3(256), 0, stream, a, sw); break;
        case 2048: hipLaunchKernelGGL((fp8_gemv_tile_kernel<tile_c(2048), TT, 128, MAT, SF>), grid, dim3(256), 0, stream, a, sw); break;
        case 4096: hipLaunchKernelGGL((fp8_gemv_tile_kernel<tile_c(4096), TT, 256, MAT, SF>), grid, dim3(256), 0, stream, a, sw); break;
        default:
            if constexpr (TT <= 4)
                hipLaunchKernelGGL((fp8_gemv_tile_kernel<tile_c(8192), TT, 512, MAT, SF>), grid, dim3(256), 0, stream, a, sw);
            break;
    }
}

template <int TT>
void launch_multi_tt(const MultiArgs& ma, dim3 grid, hipStream_t stream) {
    switch (ma.base.K) {
        case 1024: hipLaunchKernelGGL((fp8_gemv_multi_kernel<tile_c(1024), TT, 64>), grid, dim3(256), 0, stream, ma); break;
        case 2048: hipLaunchKernelGGL((fp8_gemv_multi_kernel<tile_c(2048), TT, 128>), grid, dim3(256), 0, stream, ma); break;
        case 4096: hipLaunchKernelGGL((fp8_gemv_multi_kernel<tile_c(4096), TT, 256>), grid, dim3(256), 0, stream, ma); break;
        default:
            if constexpr (TT <= 4)
                hipLaunchKernelGGL((fp8_gemv_multi_kernel<tile_c(8192), TT, 512>), grid, dim3(256), 0, stream, ma);
            break;
    }
}

// G groups (grid.y). MAT = 2: the fused SwiGLU.
template <int MAT, int SF = 0>
hipError_t launch_tile(const Fp8Args& a, const SwigluArgs& sw, int G, hipStream_t stream) {
    const dim3 grid((unsigned)((a.N + tile_rows(a.K) - 1) / tile_rows(a.K)), (unsigned)G);
    switch (tile_tt(a.T, a.K, MAT)) {
        case 1: launch_tile_tt<1, MAT, SF>(a, sw, grid, stream); break;
        case 2: launch_tile_tt<2, MAT, SF>(a, sw, grid, stream); break;
        case 4: launch_tile_tt<4, MAT, SF>(a, sw, grid, stream); break;
        case 8: launch_tile_tt<8, MAT, SF>(a, sw, grid, stream); break;
        default:
            if constexpr (MAT == 1) launch_tile_tt<16, MAT, SF>(a, sw, grid, stream);
            break;
    }
    return hipGetLastError();
}

// The matrix-core path replaces the vector tile kernels once the per-token
// dots outweigh its fixed costs: at small N or few tokens the vector kernels
// (more workgroups, no transposition through LDS) are faster, and the longer
// the rows the more tokens it takes for the matrix cores to win. Measured on
// MI355X (graph replay over 512 MB of rotated weights; N = 256 .. 8192,
// K = 1024 .. 4096, T = 2 .. 16, matrix-core kernels loading whole lines):
//   K = 1024: T >= 3 at N >= 2048, T >= 5 at any N;
//   K = 2048: T >= 3 at N >= 4096, T >= 5 at any N;
//   K = 4096: T >= 3 at N >= 4096, T >= 5 above 512 rows (the split
//             kernel below 3072 rows up to T = 8: launch_sf; up to 512 rows
//             the vector kernels have at most one workgroup per CU, 3.43
//             against 3.83 us at 256 x 4096, T = 5, and 3.64 against 3.96 at
//             512 rows, T = 8);
//   K = 8192: T >= 2.
// At T <= 4 the boundary is where it was before the line loads (the matrix
// cores now win there from about 1536 rows at K = 4096, 3072 rows by 25%),
// because fp8_e4m3_rmsnorm_gemv (T <= 4, K = 2048 or 4096) follows this rule
// to keep fp8_e4m3_gemv's bits, and on the matrix cores it runs the norm as
// a launch of its own. The fused SwiGLU and the RMSNorm-folded GEMV apply the
// rule to one matrix's rows, so their GEMVs keep the bits of fp8_e4m3_gemv on
// the same rows. A grouped launch applies it to the rows of all its groups,
// which is what sets its workgroup count: 8 groups of 1024 x 4096 run on the
// matrix cores from T = 3 (9.5 against 11.8 us; 13.5 against 31.7 us at
// T = 16). The matrix-core kernels read the T activation rows through one
// buffer resource, whose byte extent must fit 31 bits.
bool use_mfma(int T, int K, int N, int64_t xstride) {
    if (T < 2 || ((int64_t)(T - 1) * xstride + K) * 2 > INT32_MAX) return false;
    if (K > 4096) return true;
    if (K <= 1024) return (T >= 3 && N >= 2048) || T >= 5;
    if (K <= 2048) return (T >= 3 && N >= 4096) || T >= 5;
    return (T >= 3 && N >= 4096) || (T >= 5 && N > 512);
}

// The matrix-core path (T >= 2 on the tile shapes): NW waves of 512 k each,
// except K = 8192 with two matrices (8 waves of two passes, which keeps the
// second matrix's registers within the 1,024-thread workgroup's budget).
template <int MAT, int R, int SF>
void launch_mfma_r(const Fp8Args& a, const SwigluArgs& sw, int G, hipStream_t stream) {
    const dim3 grid((unsigned)((a.N + 16 * R - 1) / (16 * R)), (unsigned)G);
    switch (a.K) {
        case 1024: hipLaunchKernelGGL((fp8_gemv_mfma_kernel<2, 1, MAT, R, SF>), grid, dim3(128), 0, stream, a, sw); break;
        case 2048: hipLaunchKernelGGL((fp8_gemv_mfma_kernel<4, 1, MAT, R, SF>), grid, dim3(256), 0, stream, a, sw); break;
        case 4096: hipLaunchKernelGGL((fp8_gemv_mfma_kernel<8, 1, MAT, R, SF>), grid, dim3(512), 0, stream, a, sw); break;
        default:  // K = 8192, R = 1 only
            if constexpr (R == 1) {
                if constexpr (MAT == 1)
                    hipLaunchKernelGGL((fp8_gemv_mfma_kernel<16, 1, 1, 1, SF>), grid, dim3(1024), 0, stream, a, sw);
                else
                    hipLaunchKernelGGL((fp8_gemv_mfma_kernel<8, 2, 2, 1>), grid, dim3(512), 0, stream, a, sw);
            }
            break;
    }
}

// Row blocks per wave (R): a wave multiplies R 16-row blocks against one set
// of activation registers, so R divides the activation loads per weight byte
// (at T = 16 they are twice the weight loads with R = 1). It also divides the
// workgroups, and those must still cover the GPU: for K <= 4096, R = 2 or 4
// is taken from T = 8 on when it leaves at least 256 workgroups (one per CU)
// and 512 * R waves. Measured on MI355X for N = 4096 .. 32768, K = 1024 ..
// 4096, T = 4, 8, 16: every 4096-row shape and 8192 x 1024 stay at R = 1;
// 8192 x {2048, 4096}, 16384 x {1024, 2048} and 32768 x 1024 take R = 2
// (9-17% faster at T = 16, e.g. 32768 x 1024: 13.9 -> 11.6 us); 16384 x
// 4096 takes R = 4 (18% at T = 16). Each row's sums are formed in the same
// order for every R, so R never changes the bits.
int mfma_rows(int T, int K, int N, int mat) {
    if (T < 8 || K > 4096) return 1;
    int best = 1;
    for (int R = 2; R <= (mat == 2 ? 2 : 4); R *= 2) {
        const int wgs = (N + 16 * R - 1) / (16 * R);
        if (wgs >= 256 && wgs * (K / 512) >= 512 * R) best = R;
    }
    return best;
}

template <int MAT, int SF = 0>
hipError_t launch_mfma(const Fp8Args& a, const SwigluArgs& sw, int G, hipStream_t stream) {
    const int R = mfma_rows(a.T, a.K, a.N, MAT);
    if constexpr (MAT == 1) {
        if (R == 4) launch_mfma_r<1, 4, SF>(a, sw, G, stream);
        else if (R == 2) launch_mfma_r<1, 2, SF>(a, sw, G, stream);
        else launch_mfma_r<1, 1, SF>(a, sw, G, stream);
    } else {
        if (R == 2) launch_mfma_r<2, 2, 0>(a, sw, G, stream);
        else launch_mfma_r<2, 1, 0>(a, sw, G, stream);
    }
    return hipGetLastError();
}

// Rows longer than 4096 (K a multiple of 512) with several tokens: the
// long-row matrix-core kernels, so each weight byte is read once for all T
// tokens. Operands as the tile kernels need them (16-byte aligned rows and
// activations). Returns the number of 512-k blocks, or 0 where the path does
// not apply. K = 8192, a tile shape, takes it only where it splits blocks
// across the MFMA (launch_sf).
int long_mfma_blocks(const Fp8Args& a) {
    const bool al = aligned16(a.x) && aligned16(a.w) && (a.wrow % 16 == 0) && (a.T == 1 || a.xstride % 8 == 0) &&
                    (a.xgroup % 8 == 0);
    if (!al || a.T < 2 || a.K <= 4096 || a.K % kMmaK != 0 ||
        ((int64_t)(a.T - 1) * a.xstride + a.K) * 2 > INT32_MAX)
        return 0;
    const int b = a.K / kMmaK;
    return b <= kLongBlocks ? b : 0;
}

// The matrix-core kernel for rows longer than 4096: S = 4 (4 rows and up to
// 4 tokens per workgroup) for T <= 4 and at most 1024 rows, S = 2 (8 rows, up
// to 8 tokens) for T <= 8 and at most 2048 rows, else one block per MFMA with
// 8 real rows per workgroup up to 2048 rows and 16 above (K must hold a whole
// number of S-block groups). K = 8192, a tile shape, takes these kernels up to
// 2048 rows and the one-block tile kernel above; K = 4096 takes S = 2 where
// the matrix cores win below 3072 rows at T = 5 .. 8 (launch_sf).
// Measured on MI355X (HIP-graph replay, weights rotated over 512 MB; µs, at
// T = 2 / 4 / 8 / 16):
//   1024 x 12288: S = 4 5.19 / 5.65, S = 2 6.41 / 6.55 / 7.78, 8 rows 7.55 /
//   7.79 / 8.62 / 11.3, 16 rows 8.60 / 9.07 / 10.1 / 14.2;
//   2048 x 12288: S = 2 7.00 / 7.19 / 8.46, S = 4 7.38 / 8.36, 8 rows 8.30 /
//   8.41 / 9.25 / 12.0, 16 rows 9.15 / 9.66 / 11.0 / 14.8;
//   3072 x 6144: 16 rows 5.71 / 5.92 / 6.60 / 8.28, S = 2 6.93 / 7.22 /
//   8.17, 8 rows 8.60 / 8.59 / 9.30 / 12.2;
//   1536 x 8192: S = 2 5.40 / 5.51 / 6.03, S = 4 5.54 / 6.16, the tile
//   kernel 5.95 / 6.24 / 7.00 / 9.06, 8 rows 5.67 / 5.81 / 6.25 / 8.28;
//   3072 x 8192: the tile kernel 6.77 / 7.04 / 7.75 / 9.80, 16 rows 6.87 /
//   7.16 / 7.97 / 9.97, S = 2 7.91 / 8.12 / 9.55;
//   2048 x 4096 (T = 5 / 8): S = 2 4.40 / 4.58, the tile kernel 4.60 / 4.86,
//   vector 6.46 / 6.75; 3072 x 4096: tile 4.95 / 5.12, S = 2 5.58 / 5.96.
int long_split(int64_t rows, int T, int K) {
    if (T <= 4 && rows <= 1024 && K % (4 * kMmaK) == 0) return 4;
    if (T <= 8 && rows <= 2048 && K % (2 * kMmaK) == 0) return 2;
    return 1;
}

// Real rows per workgroup of the one-block long-row kernel.
int long_rr(int64_t rows) { return rows > 2048 ? 16 : 8; }

// Dynamic LDS of the long-row kernels: fp32 partials of every 512-k block
// (1 KiB each) and each wave's staging area. Sized by the launch, so short
// rows and few waves leave room for a second workgroup per CU.
size_t long_lds_bytes(int blocks, int waves) { return (size_t)blocks * 16 * 16 * 4 + (size_t)waves * stg_slots(1) * 16; }

// S blocks per MFMA (1: one block, 8 or 16 real rows by long_rr); waves per
// workgroup: one per group of S blocks up to 16 groups, else one per two.
template <int SF>
hipError_t launch_mfma_long(const Fp8Args& a, int blocks, int G, int S, hipStream_t stream) {
    const int64_t rows = (int64_t)a.N * G;
    const int groups = blocks / S;
    const int waves = groups <= 16 ? groups : (groups + 1) / 2;
    const dim3 block((unsigned)(64 * waves));
    const size_t lds = long_lds_bytes(blocks, waves);
    if (S == 4)
        hipLaunchKernelGGL((fp8_gemv_mfma_split_kernel<4, SF>), dim3((unsigned)((a.N + 3) / 4), (unsigned)G), block, lds, stream, a);
    else if (S == 2)
        hipLaunchKernelGGL((fp8_gemv_mfma_split_kernel<2, SF>), dim3((unsigned)((a.N + 7) / 8), (unsigned)G), block, lds, stream, a);
    else if (long_rr(rows) == 8)
        hipLaunchKernelGGL((fp8_gemv_mfma_long_kernel<8, SF>), dim3((unsigned)((a.N + 7) / 8), (unsigned)G), block, lds, stream, a);
    else
        hipLaunchKernelGGL((fp8_gemv_mfma_long_kernel<16, SF>), dim3((unsigned)((a.N + 15) / 16), (unsigned)G), block, lds, stream, a);
    return hipGetLastError();
}

hipError_t launch_multi_mfma(const MultiArgs& ma, int blocks, hipStream_t stream) {
    const dim3 grid((unsigned)blocks);
    switch (ma.base.K) {
        case 1024: hipLaunchKernelGGL((fp8_gemv_multi_mfma_kernel<2>), grid, dim3(128), 0, stream, ma); break;
        case 2048: hipLaunchKernelGGL((fp8_gemv_multi_mfma_kernel<4>), grid, dim3(256), 0, stream, ma); break;
        case 4096: hipLaunchKernelGGL((fp8_gemv_multi_mfma_kernel<8>), grid, dim3(512), 0, stream, ma); break;
        default: hipLaunchKernelGGL((fp8_gemv_multi_mfma_kernel<16>), grid, dim3(1024), 0, stream, ma); break;
    }
    return hipGetLastError();
}

hipError_t launch_multi(const MultiArgs& ma, int blocks, hipStream_t stream) {
    const dim3 grid((unsigned)blocks);
    switch (tile_tt(ma.base.T, ma.base.K, 1)) {
        case 1: launch_multi_tt<1>(ma, grid, stream); break;
        case 2: launch_multi_tt<2>(ma, grid, stream); break;
        case 4: launch_multi_tt<4>(ma, grid, stream); break;
        case 8: launch_multi_tt<8>(ma, grid, stream); break;
        default: launch_multi_tt<16>(ma, grid, stream); break;
    }
    return hipGetLastError();
}

// Both tile-scale formats take the same kernels by the same rules (so equal
// scales give equal bits). Where use_mfma (or K > 4096) sends a call to the
// matrix cores, the kernel is the tile kernel or one of the long-row kernels
// (long_split); all of them form the same per-block partials and add them in
// k order, so the choice does not change the bits.
template <int SF>
int launch_sf(const Fp8Args& a, int G, hipStream_t stream) {
    hipError_t e;
    const int64_t rows64 = (int64_t)a.N * G;
    const int rows = (int)std::min<int64_t>(rows64, INT32_MAX);
    const int long_blocks = long_mfma_blocks(a);
    const bool mf = tile_ok(a) && use_mfma(a.T, a.K, rows, a.xstride);
    int S = 0;      // > 0: a long-row kernel with S blocks per MFMA
    if (long_blocks > 0 && (a.K != 8192 || rows64 <= 2048)) S = long_split(rows64, a.T, a.K);
    else if (mf && a.K == 4096 && a.T <= 8 && rows64 < 3072) S = 2;
    if (S > 0) {
        e = launch_mfma_long<SF>(a, a.K / kMmaK, G, S, stream);
    } else if (tile_ok(a)) {
        e = mf ? launch_mfma<1, SF>(a, SwigluArgs{}, G, stream) : launch_tile<1, SF>(a, SwigluArgs{}, G, stream);
    } else {
        const dim3 grid((unsigned)((a.N + kWaves * kRows - 1) / (kWaves * kRows)), (unsigned)G);
        const dim3 block(64 * kWaves);
        const int nc = (a.K + 1023) / 1024;
        const bool al = aligned16(a.x) && aligned16(a.w) && (a.wrow % 16 == 0) &&
                        (a.T == 1 || a.xstride % 8 == 0) && (a.xgroup % 8 == 0);
#define DSV4_LAUNCH(NCV, LV)                                                                        \
    if (al) hipLaunchKernelGGL((fp8_gemv_kernel<NCV, true, LV, SF>), grid, block, 0, stream, a);   \
    else hipLaunchKernelGGL((fp8_gemv_kernel<NCV, false, LV, SF>), grid, block, 0, stream, a);
        switch (nc) {
            case 1: DSV4_LAUNCH(1, false) break;
            case 2: DSV4_LAUNCH(2, false) break;
            case 3: DSV4_LAUNCH(3, false) break;
            case 4: DSV4_LAUNCH(4, false) break;
            default: DSV4_LAUNCH(4, true) break;
        }
#undef DSV4_LAUNCH
        e = hipGetLastError();
    }
    if (e != hipSuccess) {
        std::fprintf(stderr, "fp8_e4m3_gemv launch failed: %s\n", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

int launch(const Fp8Args& a, int G, hipStream_t stream) { return launch_sf<0>(a, G, stream); }

}  // namespace

extern "C" int fp8_e4m3_gemv_m1(const dsv4_bf16_t* x, const uint8_t* W_fp8, const uint8_t* W_scale,
                                int K, int N, int64_t weight_row_stride_bytes,
                                int64_t scale_row_stride_bytes, dsv4_bf16_t* y, hipStream_t stream) {
    const int v = validate(K, N);
    if (v != 0) return v;
    Fp8Args a{reinterpret_cast<const uint16_t*>(x), K, W_fp8, W_scale, K, N, 1,
              weight_row_stride_bytes, scale_row_stride_bytes, reinterpret_cast<uint16_t*>(y), N, 0, 0};
    return launch(a, 1, stream);
}

extern "C" int fp8_e4m3_gemv(const dsv4_bf16_t* x, int64_t x_row_stride, const uint8_t* W_fp8,
                             const uint8_t* W_scale, int K, int N, int T,
                             int64_t weight_row_stride_bytes, int64_t scale_row_stride_bytes,
                             dsv4_bf16_t* y, int64_t y_row_stride, hipStream_t stream) {
    const int v = validate(K, N);
    if (v != 0) return v;
    if (T < 1 || T > kMaxT) {
        std::fprintf(stderr, "fp8_e4m3_gemv: T=%d outside [1, %d]\n", T, kMaxT);
        return -5;
    }
    if (!operands_set("fp8_e4m3_gemv", {x, W_fp8, W_scale, y})) return kNullOperand;
    Fp8Args a{reinterpret_cast<const uint16_t*>(x), x_row_stride, W_fp8, W_scale, K, N, T,
              weight_row_stride_bytes, scale_row_stride_bytes, reinterpret_cast<uint16_t*>(y),
              y_row_stride, 0, 0};
    return launch(a, 1, stream);
}

extern "C" int fp8_e4m3_gemv_f32s(const dsv4_bf16_t* x, int64_t x_row_stride, const uint8_t* W_fp8,
                                  const float* W_scale, int K, int N, int T, int64_t weight_row_stride_bytes,
                                  int64_t scale_row_stride, dsv4_bf16_t* y, int64_t y_row_stride,
                                  hipStream_t stream) {
    const int v = validate(K, N);
    if (v != 0) return v;
    if (T < 1 || T > kMaxT) {
        std::fprintf(stderr, "fp8_e4m3_gemv_f32s: T=%d outside [1, %d]\n", T, kMaxT);
        return -5;
    }
    if (!operands_set("fp8_e4m3_gemv_f32s", {x, W_fp8, W_scale, y})) return kNullOperand;
    if ((reinterpret_cast<uintptr_t>(W_scale) & 3u) != 0 || scale_row_stride < K / kTile) {
        std::fprintf(stderr, "fp8_e4m3_gemv_f32s: scales must be 4-byte aligned fp32 with a row stride >= K/128\n");
        return -6;
    }
    Fp8Args a{reinterpret_cast<const uint16_t*>(x), x_row_stride, W_fp8, reinterpret_cast<const uint8_t*>(W_scale),
              K, N, T, weight_row_stride_bytes, scale_row_stride, reinterpret_cast<uint16_t*>(y), y_row_stride, 0, 0};
    return launch_sf<1>(a, 1, stream);
}

extern "C" int fp8_e4m3_gemv_grouped(const dsv4_bf16_t* x, int64_t x_row_stride, int64_t x_group_stride,
                                     const uint8_t* W_fp8, const uint8_t* W_scale, int G, int K, int N,
                                     int T, int64_t weight_row_stride_bytes, int64_t scale_row_stride_bytes,
                                     dsv4_bf16_t* y, int64_t y_row_stride, int64_t y_group_stride,
                                     hipStream_t stream) {
    const int v = validate(K, N);
    if (v != 0) return v;
    if (T < 1 || T > kMaxT) {
        std::fprintf(stderr, "fp8_e4m3_gemv_grouped: T=%d outside [1, %d]\n", T, kMaxT);
        return -5;
    }
    if (G < 1 || G > 65535) {
        std::fprintf(stderr, "fp8_e4m3_gemv_grouped: G=%d outside [1, 65535]\n", G);
        return -6;
    }
    if (!operands_set("fp8_e4m3_gemv_grouped", {x, W_fp8, W_scale, y})) return kNullOperand;
    Fp8Args a{reinterpret_cast<const uint16_t*>(x), x_row_stride, W_fp8, W_scale, K, N, T,
              weight_row_stride_bytes, scale_row_stride_bytes, reinterpret_cast<uint16_t*>(y),
              y_row_stride, x_group_stride, y_group_stride};
    return launch(a, G, stream);
}

extern "C" int fp8_e4m3_gemv_multi(const dsv4_bf16_t* x, int64_t x_row_stride, int K, int T, int n_mats,
                                   const uint8_t* const* W_fp8, const uint8_t* const* W_scale, const int* N,
                                   const int64_t* weight_row_stride_bytes, const int64_t* scale_row_stride_bytes,
                                   dsv4_bf16_t* const* y, const int64_t* y_row_stride, hipStream_t stream) {
    if (n_mats < 1 || n_mats > kMaxMulti || !W_fp8 || !W_scale || !N || !weight_row_stride_bytes ||
        !scale_row_stride_bytes || !y || !y_row_stride) {
        std::fprintf(stderr, "fp8_e4m3_gemv_multi: n_mats=%d outside [1, %d] or a null table\n", n_mats, kMaxMulti);
        return -6;
    }
    for (int m = 0; m < n_mats; ++m) {
        const int v = validate(K, N[m]);
        if (v != 0) return v;
    }
    if (T < 1 || T > kMaxT) {
        std::fprintf(stderr, "fp8_e4m3_gemv_multi: T=%d outside [1, %d]\n", T, kMaxT);
        return -5;
    }
    if (!operands_set("fp8_e4m3_gemv_multi", {x})) return kNullOperand;
    for (int m = 0; m < n_mats; ++m)
        if (!operands_set("fp8_e4m3_gemv_multi", {W_fp8[m], W_scale[m], y[m]})) return kNullOperand;
    MultiArgs ma{};
    ma.base = Fp8Args{reinterpret_cast<const uint16_t*>(x), x_row_stride, nullptr, nullptr, K, 0, T, 0, 0,
                      nullptr, 0, 0, 0};
    ma.n_mats = n_mats;
    bool tile = true;
    bool mfma = true;
    for (int m = 0; m < n_mats; ++m) mfma = mfma && use_mfma(T, K, N[m], x_row_stride);
    int blocks = 0;
    for (int m = 0; m < n_mats; ++m) {
        Fp8Args a = ma.base;
        a.w = W_fp8[m];
        a.s = W_scale[m];
        a.N = N[m];
        a.wrow = weight_row_stride_bytes[m];
        a.srow = scale_row_stride_bytes[m];
        a.y = reinterpret_cast<uint16_t*>(y[m]);
        a.ystride = y_row_stride[m];
        tile = tile && tile_ok(a);
        ma.first[m] = blocks;
        ma.w[m] = a.w;
        ma.s[m] = a.s;
        ma.N[m] = a.N;
        ma.wrow[m] = a.wrow;
        ma.srow[m] = a.srow;
        ma.y[m] = a.y;
        ma.ystride[m] = a.ystride;
        const int rows = mfma ? 16 : tile_rows(K);
        blocks += (N[m] + rows - 1) / rows;
    }
    ma.first[n_mats] = blocks;
    if (!tile) {
        // Shapes off the tile path: one launch per matrix.
        for (int m = 0; m < n_mats; ++m) {
            Fp8Args a = ma.base;
            a.w = ma.w[m];
            a.s = ma.s[m];
            a.N = ma.N[m];
            a.wrow = ma.wrow[m];
            a.srow = ma.srow[m];
            a.y = ma.y[m];
            a.ystride = ma.ystride[m];
            const int r = launch(a, 1, stream);
            if (r != 0) return r;
        }
        return 0;
    }
    const hipError_t e = mfma ? launch_multi_mfma(ma, blocks, stream) : launch_multi(ma, blocks, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "fp8_e4m3_gemv_multi launch failed: %s\n", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

extern "C" int fp8_e4m3_swiglu_gemv(const dsv4_bf16_t* x, int64_t x_row_stride, const uint8_t* W1_fp8,
                                    const uint8_t* W1_scale, const uint8_t* W3_fp8, const uint8_t* W3_scale,
                                    int K, int N, int T, int64_t weight_row_stride_bytes,
                                    int64_t scale_row_stride_bytes, float limit, int clamp_up,
                                    dsv4_bf16_t* act, int64_t act_row_stride, hipStream_t stream) {
    const int v = validate(K, N);
    if (v != 0) return v;
    if (T < 1 || T > kMaxT) {
        std::fprintf(stderr, "fp8_e4m3_swiglu_gemv: T=%d outside [1, %d]\n", T, kMaxT);
        return -5;
    }
    Fp8Args a{reinterpret_cast<const uint16_t*>(x), x_row_stride, W1_fp8, W1_scale, K, N, T,
              weight_row_stride_bytes, scale_row_stride_bytes, reinterpret_cast<uint16_t*>(act),
              act_row_stride, 0, 0};
    if (!tile_ok(a) || !aligned16(W3_fp8)) {
        std::fprintf(stderr, "fp8_e4m3_swiglu_gemv: needs K in {1024, 2048, 4096, 8192} and 16-byte aligned x, "
                             "W1, W3 and rows\n");
        return -6;
    }
    if (!operands_set("fp8_e4m3_swiglu_gemv", {x, W1_fp8, W1_scale, W3_fp8, W3_scale, act})) return kNullOperand;
    const SwigluArgs sw{W3_fp8, W3_scale, limit, clamp_up};
    if (use_mfma(T, K, N, x_row_stride)) {
        const hipError_t e = launch_mfma<2>(a, sw, 1, stream);
        if (e != hipSuccess) {
            std::fprintf(stderr, "fp8_e4m3_swiglu_gemv launch failed: %s\n", hipGetErrorString(e));
            return -4;
        }
        return 0;
    }
    // Vector path: at most 8 tokens per launch (registers of the two
    // matrices' partials).
    for (int t0 = 0; t0 < T; t0 += 8) {
        Fp8Args c = a;
        c.x = a.x + (int64_t)t0 * x_row_stride;
        c.y = a.y + (int64_t)t0 * act_row_stride;
        c.T = T - t0 < 8 ? T - t0 : 8;
        const hipError_t e = launch_tile<2>(c, sw, 1, stream);
        if (e != hipSuccess) {
            std::fprintf(stderr, "fp8_e4m3_swiglu_gemv launch failed: %s\n", hipGetErrorString(e));
            return -4;
        }
    }
    return 0;
}

extern "C" int fp8_e4m3_dequant_bf16(const uint8_t* W_fp8, const uint8_t* W_scale, int K, int N,
                                     int64_t weight_row_stride_bytes,
                                     int64_t scale_row_stride_bytes, dsv4_bf16_t* out,
                                     hipStream_t stream) {
    if (K % kTile != 0 || K < kTile) return -1;
    if (N < 1) return -4;
    if (!operands_set("fp8_e4m3_dequant_bf16", {W_fp8, W_scale, out})) return kNullOperand;
    const int64_t total = (int64_t)N * (K / 16);
    hipLaunchKernelGGL(fp8_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, W_fp8, W_scale, K, N, weight_row_stride_bytes,
                       scale_row_stride_bytes, reinterpret_cast<uint16_t*>(out));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "fp8_e4m3_dequant_bf16 launch failed: %s\n", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

extern "C" int fp8_e4m3_rmsnorm_gemv(const dsv4_bf16_t* x, const dsv4_bf16_t* residual,
                                     const dsv4_bf16_t* norm_weight, float eps, const uint8_t* W_fp8,
                                     const uint8_t* W_scale, int K, int N, int T,
                                     int64_t weight_row_stride_bytes, int64_t scale_row_stride_bytes,
                                     dsv4_bf16_t* y, dsv4_bf16_t* x_norm, dsv4_bf16_t* new_residual,
                                     hipStream_t stream) {
    const int v = validate(K, N);
    if (v != 0) return v;
    if (T < 1 || T > 4) {
        std::fprintf(stderr, "fp8_e4m3_rmsnorm_gemv: T=%d outside [1, 4]\n", T);
        return -5;
    }
    Fp8Args a{reinterpret_cast<const uint16_t*>(x), K, W_fp8, W_scale, K, N, T,
              weight_row_stride_bytes, scale_row_stride_bytes, reinterpret_cast<uint16_t*>(y), N, 0, 0};
    const bool ok = tile_ok(a) && (K == 2048 || K == 4096) && norm_weight && x_norm && aligned16(norm_weight) &&
                    aligned16(x_norm) &&
                    (!residual || (aligned16(residual) && new_residual && aligned16(new_residual)));
    if (!ok) {
        std::fprintf(stderr, "fp8_e4m3_rmsnorm_gemv: needs K in {2048, 4096}, 16-byte aligned operands, "
                             "x_norm, and new_residual with a residual\n");
        return -6;
    }
    if (!operands_set("fp8_e4m3_rmsnorm_gemv", {x, W_fp8, W_scale, y})) return kNullOperand;
    const NormArgs nm{reinterpret_cast<const uint16_t*>(residual), reinterpret_cast<const uint16_t*>(norm_weight),
                      eps, reinterpret_cast<uint16_t*>(x_norm), reinterpret_cast<uint16_t*>(new_residual)};
    const int KC = K / 16;
    hipError_t e;
    if (!use_mfma(T, K, N, K)) {
        // One launch: the norm, then the GEMV slice of each workgroup.
        const dim3 grid((unsigned)((N + 4 * 256 / KC - 1) / (4 * 256 / KC)));
#define DSV4_NG(TTV, RES)                                                                                          \
    if (KC == 256) hipLaunchKernelGGL((fp8_norm_gemv_tile_kernel<4, TTV, 256, RES>), grid, dim3(256), 0, stream, a, nm); \
    else hipLaunchKernelGGL((fp8_norm_gemv_tile_kernel<4, TTV, 128, RES>), grid, dim3(256), 0, stream, a, nm);
        if (residual) {
            if (T == 1) { DSV4_NG(1, true) }
            else if (T == 2) { DSV4_NG(2, true) }
            else { DSV4_NG(4, true) }
        } else {
            if (T == 1) { DSV4_NG(1, false) }
            else if (T == 2) { DSV4_NG(2, false) }
            else { DSV4_NG(4, false) }
        }
#undef DSV4_NG
        e = hipGetLastError();
    } else {
        // Where fp8_e4m3_gemv takes the matrix cores (use_mfma; with T <= 4
        // and K in {2048, 4096} that is T >= 3 with N >= 4096): the norm in
        // one workgroup, then that GEMV on x_norm (so y keeps its bits).
#define DSV4_NO(KCV, RES) \
    hipLaunchKernelGGL((fp8_norm_gemv_tile_kernel<4, 4, KCV, RES, false>), dim3(1), dim3(256), 0, stream, a, nm)
        if (residual) { if (KC == 256) DSV4_NO(256, true); else DSV4_NO(128, true); }
        else { if (KC == 256) DSV4_NO(256, false); else DSV4_NO(128, false); }
#undef DSV4_NO
        e = hipGetLastError();
        if (e == hipSuccess) {
            Fp8Args g = a;
            g.x = reinterpret_cast<const uint16_t*>(x_norm);
            e = launch_mfma<1>(g, SwigluArgs{}, 1, stream);
        }
    }
    if (e != hipSuccess) {
        std::fprintf(stderr, "fp8_e4m3_rmsnorm_gemv launch failed: %s\n", hipGetErrorString(e));
        return -4;
    }
    return 0;
}
