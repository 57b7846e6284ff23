// mxfp4_grouped_gemv.hip — routed MXFP4 SwiGLU MoE GEMV for gfx950 (MI355X).
//
// Computes, for each token t and its routed experts e with weights w_{t,e},
//   M[e,t]  = bf16( silu(W1_e . x_t) * (W3_e . x_t) )          (stage A)
//   out[t]  = bf16( sum_e w_{t,e} * (W2_e . M[e,t]) )            (stage B)
// with MXFP4 weights (e2m1 codes + one E8M0 scale per 32 elements), fp32
// accumulation and the routed intermediate rounded to bf16, as the reference
// kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:143-278 does.
//
// Design (gfx950, wave64):
//   * A wave streams whole weight rows with 16-byte loads: lane l of a row
//     pass takes MX block l (16 packed bytes = 32 codes), so one wave-wide
//     load covers 1 KiB of a row, fully coalesced. Rows of K=4096 take two
//     passes (NB=2 blocks per lane), rows of K=2048 one.
//   * Because a lane always owns the same K-blocks, its slice of the
//     activation (64 bf16 for K=4096) lives in registers for the whole wave;
//     no LDS staging and no per-row activation traffic.
//   * Decode: v_cvt_scalef32_pk_bf16_fp4 turns two codes into an exact bf16
//     pair, v_dot2_f32_bf16 multiplies-adds it against the activation pair
//     into fp32; the block's E8M0 scale is applied once per block.
//   * Several rows are reduced together with a butterfly (wave_reduce_n), so
//     the cross-lane cost per row is ~1-2 shuffles.
//   * Stage A writes M (bf16) to the workspace; stage B makes one workgroup
//     own a tile of output rows and split the routed experts over its waves;
//     per-wave partial sums meet in LDS and are added in a fixed order, so
//     the result is deterministic: no atomics, no memset, no cast kernel
//     (the reference uses fp32 atomicAdd + memset + a cast launch).
//   * Two entry styles share the kernels: the drop-in mxfp4_grouped_gemv_topk
//     (one token, experts packed contiguously [n_exp, ...]) and the
//     expert-indexed mxfp4_moe_grouped_gemv (T tokens, experts read in place
//     from the per-layer [n_experts, ...] tensors through device-built routing
//     tables, each unique expert streamed once for all of its tokens).

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "dsv4_device.h"
#include "dsv4_kernels.h"

namespace {

using namespace dsv4;

constexpr int kBlkElems = 32;           // elements per MX block
constexpr int kMaxRed = 4096;           // K_in / hidden cap of the drop-in ABI
constexpr int kMaxExpSlots = 256;       // n_exp cap of the drop-in entry
constexpr int kMaxTokens = 64;          // T cap of the expert-indexed entry
constexpr int kMaxTopk = 16;
constexpr int kMaxExperts = 1024;

constexpr int kWavesA = 4;              // waves per stage-A workgroup
constexpr int kHpw = 4;                 // hidden rows (of W1 and W3) per wave pass
constexpr int kRowsB = 8;               // output rows per stage-B workgroup
constexpr int kWavesB = 4;              // waves per stage-B workgroup

// ------------------------------------------------------------ routing set --

// Which experts a launch visits and which (token, weight) pairs each serves.
//   dense   (INDEXED=false): slot u is expert u of a packed [n_slots, ...]
//            tensor, with the single pair p = u (token 0, weight rweights[u]);
//   indexed (INDEXED=true):  slot u < *n_unique is expert uexp[u] of the
//            per-layer tensor, serving pairs off[u] .. off[u+1]-1.
struct ExpertSet {
    const int32_t* n_unique;
    const int32_t* uexp;
    const int32_t* off;
    const int32_t* pair_tok;
    const float* pair_w;
    const float* rweights;
    int n_slots;
};

template <bool INDEXED>
__device__ __forceinline__ bool slot_info(const ExpertSet& s, int u, int& expert, int& pbeg,
                                          int& pend) {
    if constexpr (INDEXED) {
        if (u >= *s.n_unique) return false;
        expert = s.uexp[u];
        pbeg = s.off[u];
        pend = s.off[u + 1];
    } else {
        if (u >= s.n_slots) return false;
        expert = u;
        pbeg = u;
        pend = u + 1;
    }
    return true;
}

template <bool INDEXED>
__device__ __forceinline__ void pair_info(const ExpertSet& s, int p, int& tok, float& w) {
    if constexpr (INDEXED) {
        tok = s.pair_tok[p];
        w = s.pair_w[p];
    } else {
        tok = 0;
        w = s.rweights[p];
    }
}

template <bool ALIGNED>
__device__ __forceinline__ u32x4 load_w16(const uint8_t* p) {
    if constexpr (ALIGNED) return ld16(p);
    else return ld16_unaligned(p);
}

// Activation slice of MX block b (32 bf16 = 16 packed pairs) into xp[0..15].
template <bool ALIGNED>
__device__ __forceinline__ void load_act_block(const uint16_t* src, uint32_t* xp) {
    if constexpr (ALIGNED) {
        const u32x4* s = reinterpret_cast<const u32x4*>(src);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = s[q];
            xp[4 * q + 0] = v[0];
            xp[4 * q + 1] = v[1];
            xp[4 * q + 2] = v[2];
            xp[4 * q + 3] = v[3];
        }
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q)
            xp[q] = (uint32_t)src[2 * q] | ((uint32_t)src[2 * q + 1] << 16);
    }
}

// ---------------------------------------------------------------- stage A --

struct StageAArgs {
    const uint16_t* x;          // [T, K] bf16
    const uint8_t* w1;          // expert-major packed weights
    const uint8_t* w3;
    const uint8_t* s1;          // expert-major E8M0 scales
    const uint8_t* s3;
    int64_t w_exp_stride;       // bytes per expert: hidden * K/2
    int64_t s_exp_stride;       // bytes per expert: hidden * K/32
    int K;
    int hidden;
    int h_per_wave;             // multiple of kHpw
    uint16_t* M;                // [pairs, hidden] bf16
    ExpertSet es;
};

// grid = (ceil(hidden / (kWavesA*h_per_wave)), expert slots), block = 64*kWavesA.
template <int NB, bool INDEXED, bool ALIGNED>
__global__ __launch_bounds__(64 * kWavesA) void moe_swiglu_kernel(const StageAArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int expert, pbeg, pend;
    if (!slot_info<INDEXED>(a.es, blockIdx.y, expert, pbeg, pend)) return;
    const int h_begin = (blockIdx.x * kWavesA + wave) * a.h_per_wave;
    if (h_begin >= a.hidden) return;
    const int h_end = min(h_begin + a.h_per_wave, a.hidden);

    const int K = a.K;
    const int nblk = K / kBlkElems;
    const int64_t wrow = K / 2;
    const uint8_t* W1 = a.w1 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* W3 = a.w3 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* S1 = a.s1 + (int64_t)expert * a.s_exp_stride;
    const uint8_t* S3 = a.s3 + (int64_t)expert * a.s_exp_stride;

    bool bvalid[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) bvalid[j] = (lane + 64 * j) < nblk;

    uint32_t xs[NB][16];
    auto load_x = [&](int tok) {
        const uint16_t* xt = a.x + (int64_t)tok * K;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (bvalid[j]) {
                load_act_block<ALIGNED>(xt + (lane + 64 * j) * kBlkElems, xs[j]);
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) xs[j][q] = 0u;
            }
        }
    };
    if constexpr (!INDEXED) load_x(0);

    for (int h0 = h_begin; h0 < h_end; h0 += kHpw) {
        u32x4 w1v[kHpw][NB], w3v[kHpw][NB];
        uint32_t s1v[kHpw][NB], s3v[kHpw][NB];
#pragma unroll
        for (int r = 0; r < kHpw; ++r) {
            const int h = h0 + r;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int b = lane + 64 * j;
                if (h < h_end && bvalid[j]) {
                    const int64_t wo = (int64_t)h * wrow + (int64_t)b * 16;
                    const int64_t so = (int64_t)h * nblk + b;
                    w1v[r][j] = load_w16<ALIGNED>(W1 + wo);
                    w3v[r][j] = load_w16<ALIGNED>(W3 + wo);
                    s1v[r][j] = S1[so];
                    s3v[r][j] = S3[so];
                } else {
                    w1v[r][j] = u32x4{0u, 0u, 0u, 0u};
                    w3v[r][j] = u32x4{0u, 0u, 0u, 0u};
                    s1v[r][j] = 0u;
                    s3v[r][j] = 0u;
                }
            }
        }
        for (int p = pbeg; p < pend; ++p) {
            if constexpr (INDEXED) {
                int tok;
                float wt;
                pair_info<INDEXED>(a.es, p, tok, wt);
                load_x(tok);
            }
            float g[kHpw], u[kHpw];
#pragma unroll
            for (int r = 0; r < kHpw; ++r) {
                float gg = 0.f, uu = 0.f;
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    gg = fmaf(fp4_block_dot(w1v[r][j], xs[j]), e8m0_to_f32(s1v[r][j]), gg);
                    uu = fmaf(fp4_block_dot(w3v[r][j], xs[j]), e8m0_to_f32(s3v[r][j]), uu);
                }
                g[r] = gg;
                u[r] = uu;
            }
            wave_reduce_n<kHpw>(g, lane);
            wave_reduce_n<kHpw>(u, lane);
            const int r = reduced_index<kHpw>(lane);
            if (reduced_owner<kHpw>(lane) && h0 + r < h_end) {
                a.M[(int64_t)p * a.hidden + h0 + r] = f32_to_bf16_bits(silu_f32(g[0]) * u[0]);
            }
        }
    }
}

// ---------------------------------------------------------------- stage B --

struct StageBArgs {
    const uint16_t* M;          // [pairs, hidden] bf16, 16-byte aligned rows
    const uint8_t* w2;          // expert-major packed [.., out_dim, hidden/2]
    const uint8_t* s2;          // expert-major scales [.., out_dim, hidden/32]
    int64_t w_exp_stride;
    int64_t s_exp_stride;
    int hidden;
    int out_dim;
    int T;
    uint16_t* out;              // [T, out_dim] bf16
    ExpertSet es;
};

// grid = ceil(out_dim / kRowsB), block = 64*kWavesB. Waves take expert slots
// wave, wave+kWavesB, ...; partial sums per (wave, token, row) meet in LDS.
template <int NBB, int TMAX, bool INDEXED, bool ALIGNED>
__global__ __launch_bounds__(64 * kWavesB) void moe_down_kernel(const StageBArgs a) {
    __shared__ float acc[kWavesB][TMAX][kRowsB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int o0 = blockIdx.x * kRowsB;
    float* accf = &acc[0][0][0];
    for (int i = threadIdx.x; i < kWavesB * TMAX * kRowsB; i += 64 * kWavesB) accf[i] = 0.f;
    __syncthreads();

    int U;
    if constexpr (INDEXED) U = *a.es.n_unique;
    else U = a.es.n_slots;
    const int nblk = a.hidden / kBlkElems;
    const int64_t wrow = a.hidden / 2;
    bool bvalid[NBB];
#pragma unroll
    for (int j = 0; j < NBB; ++j) bvalid[j] = (lane + 64 * j) < nblk;

    for (int u = wave; u < U; u += kWavesB) {
        int expert, pbeg, pend;
        slot_info<INDEXED>(a.es, u, expert, pbeg, pend);
        const uint8_t* W2 = a.w2 + (int64_t)expert * a.w_exp_stride;
        const uint8_t* S2 = a.s2 + (int64_t)expert * a.s_exp_stride;
        u32x4 wv[kRowsB][NBB];
        uint32_t sv[kRowsB][NBB];
#pragma unroll
        for (int r = 0; r < kRowsB; ++r) {
            const int o = o0 + r;
#pragma unroll
            for (int j = 0; j < NBB; ++j) {
                const int b = lane + 64 * j;
                if (o < a.out_dim && bvalid[j]) {
                    wv[r][j] = load_w16<ALIGNED>(W2 + (int64_t)o * wrow + (int64_t)b * 16);
                    sv[r][j] = S2[(int64_t)o * nblk + b];
                } else {
                    wv[r][j] = u32x4{0u, 0u, 0u, 0u};
                    sv[r][j] = 0u;
                }
            }
        }
        for (int p = pbeg; p < pend; ++p) {
            int tok;
            float wt;
            pair_info<INDEXED>(a.es, p, tok, wt);
            uint32_t ms[NBB][16];
#pragma unroll
            for (int j = 0; j < NBB; ++j) {
                if (bvalid[j]) {
                    load_act_block<true>(a.M + (int64_t)p * a.hidden + (lane + 64 * j) * kBlkElems,
                                         ms[j]);
                } else {
#pragma unroll
                    for (int q = 0; q < 16; ++q) ms[j][q] = 0u;
                }
            }
            float part[kRowsB];
#pragma unroll
            for (int r = 0; r < kRowsB; ++r) {
                float s = 0.f;
#pragma unroll
                for (int j = 0; j < NBB; ++j)
                    s = fmaf(fp4_block_dot(wv[r][j], ms[j]), e8m0_to_f32(sv[r][j]), s);
                part[r] = s;
            }
            wave_reduce_n<kRowsB>(part, lane);
            const int r = reduced_index<kRowsB>(lane);
            if (reduced_owner<kRowsB>(lane)) acc[wave][tok][r] += wt * part[0];
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.T * kRowsB; i += 64 * kWavesB) {
        const int t = i / kRowsB;
        const int r = i % kRowsB;
        const int o = o0 + r;
        if (o < a.out_dim) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < kWavesB; ++w) s += acc[w][t][r];
            a.out[(int64_t)t * a.out_dim + o] = f32_to_bf16_bits(s);
        }
    }
}

// ------------------------------------------------------------ routing ------

// Device routing tables of the expert-indexed path (in the workspace):
struct RouteTables {
    int32_t* header;            // [0] = unique experts U, [1] = pairs P
    int32_t* uexp;              // [max_unique] expert id per slot, ascending
    int32_t* off;               // [max_unique + 1] pair offsets per slot
    int32_t* pair_tok;          // [T*topk] token of each pair, grouped by slot
    float* pair_w;              // [T*topk] routing weight of each pair
};

// One workgroup of 1024 threads: histogram of expert ids, one scan giving each
// routed expert its slot and pair offset, then each routed expert lists its
// (token, weight) pairs in token order. Deterministic for any input order.
__global__ __launch_bounds__(1024) void moe_build_pairs_kernel(const int32_t* ids,
                                                               const float* w, int T,
                                                               int topk, int n_experts,
                                                               RouteTables rt) {
    __shared__ int cnt[kMaxExperts];
    __shared__ int scan[kMaxExperts];
    __shared__ int sid[kMaxTokens * kMaxTopk];
    const int tid = threadIdx.x;
    const int n = T * topk;
    if (tid < n_experts) cnt[tid] = 0;
    for (int i = tid; i < n; i += blockDim.x) sid[i] = ids[i];
    __syncthreads();
    for (int i = tid; i < n; i += blockDim.x) {
        const int e = sid[i];
        if (e >= 0 && e < n_experts) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // Inclusive scan of (routed flag << 16 | count): both fields stay < 2^16.
    const int c = tid < n_experts ? cnt[tid] : 0;
    const int v = ((c > 0) << 16) | c;
    scan[tid] = v;
    __syncthreads();
    for (int d = 1; d < kMaxExperts; d <<= 1) {
        const int add = tid >= d ? scan[tid - d] : 0;
        __syncthreads();
        scan[tid] += add;
        __syncthreads();
    }
    const int incl = scan[tid];
    const int excl = incl - v;
    if (c > 0) {
        const int slot = excl >> 16;
        const int poff = excl & 0xFFFF;
        rt.uexp[slot] = tid;
        rt.off[slot] = poff;
        int k = 0;
        for (int i = 0; i < n; ++i) {
            if (sid[i] == tid) {
                rt.pair_tok[poff + k] = i / topk;
                rt.pair_w[poff + k] = w[i];
                ++k;
            }
        }
    }
    if (tid == kMaxExperts - 1) {
        const int U = incl >> 16;
        const int P = incl & 0xFFFF;
        rt.header[0] = U;
        rt.header[1] = P;
        rt.off[U] = P;
    }
}

// One wave per token: top-k of the logits (descending, ties to the lower
// index) with weights sigmoid(l) renormalised to sum 1. Lane k keeps the k-th
// pick; a picked entry becomes NaN, which never compares greater or equal.
__global__ __launch_bounds__(64) void moe_route_sigmoid_topk_kernel(const float* logits,
                                                                     int n_experts, int topk,
                                                                     int32_t* ids, float* wout) {
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    const float* lt = logits + (int64_t)t * n_experts;
    constexpr int kPer = kMaxExperts / 64;
    float v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = lane + 64 * i;
        const float l = e < n_experts ? lt[e] : __uint_as_float(0x7FC00000u);
        v[i] = (e < n_experts && l != l) ? -INFINITY : l;  // NaN logit ranks last
    }
    int my_e = 0;
    float my_l = -INFINITY;
    for (int k = 0; k < topk; ++k) {
        float best = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int e = lane + 64 * i;
            if (v[i] > best || (v[i] == best && e < bi)) {
                best = v[i];
                bi = e;
            }
        }
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) {
            const float ob = __shfl_xor(best, m, 64);
            const int oi = __shfl_xor(bi, m, 64);
            if (ob > best || (ob == best && oi < bi)) {
                best = ob;
                bi = oi;
            }
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (lane + 64 * i == bi) v[i] = __uint_as_float(0x7FC00000u);
        if (lane == k) {
            my_e = bi;
            my_l = best;
        }
    }
    const float s = lane < topk ? 1.0f / (1.0f + __expf(-my_l)) : 0.f;
    const float tot = wave_sum(s);
    if (lane < topk) {
        ids[(int64_t)t * topk + lane] = my_e;
        wout[(int64_t)t * topk + lane] = s / tot;
    }
}

// ------------------------------------------------------------ host side ----

int env_int(const char* name, int def) {
    const char* s = std::getenv(name);
    if (!s || !*s) return def;
    const int v = std::atoi(s);
    return v > 0 ? v : def;
}

// hidden rows per stage-A wave (multiple of kHpw); tunable for sweeps.
int stage_a_rows_per_wave() {
    static const int v = [] {
        int r = env_int("DSV4_GROUPED_H_PER_WAVE", 8);
        r = (r + kHpw - 1) / kHpw * kHpw;
        return r;
    }();
    return v;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

uintptr_t align_up(uintptr_t v, uintptr_t a) { return (v + a - 1) / a * a; }

template <bool INDEXED, bool ALIGNED>
hipError_t launch_stage_a(const StageAArgs& a, int slots, hipStream_t stream) {
    const int hpw = a.h_per_wave;
    dim3 grid((unsigned)((a.hidden + kWavesA * hpw - 1) / (kWavesA * hpw)), (unsigned)slots);
    dim3 block(64 * kWavesA);
    const int nb = (a.K / kBlkElems + 63) / 64;
    switch (nb) {
        case 1: hipLaunchKernelGGL((moe_swiglu_kernel<1, INDEXED, ALIGNED>), grid, block, 0, stream, a); break;
        case 2: hipLaunchKernelGGL((moe_swiglu_kernel<2, INDEXED, ALIGNED>), grid, block, 0, stream, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int TMAX, bool INDEXED, bool ALIGNED>
hipError_t launch_stage_b(const StageBArgs& a, hipStream_t stream) {
    dim3 grid((unsigned)((a.out_dim + kRowsB - 1) / kRowsB));
    dim3 block(64 * kWavesB);
    const int nb = (a.hidden / kBlkElems + 63) / 64;
    switch (nb) {
        case 1: hipLaunchKernelGGL((moe_down_kernel<1, TMAX, INDEXED, ALIGNED>), grid, block, 0, stream, a); break;
        case 2: hipLaunchKernelGGL((moe_down_kernel<2, TMAX, INDEXED, ALIGNED>), grid, block, 0, stream, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

struct MoeWorkspaceLayout {
    size_t header, uexp, off, pair_tok, pair_w, M, total;
};

MoeWorkspaceLayout moe_layout(int T, int topk, int n_experts, int hidden) {
    const size_t P = (size_t)T * topk;
    const size_t maxu = (size_t)(n_experts < (int)P ? n_experts : (int)P);
    MoeWorkspaceLayout L;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    L.header = take(16);
    L.uexp = take(4 * maxu);
    L.off = take(4 * (maxu + 1));
    L.pair_tok = take(4 * P);
    L.pair_w = take(4 * P);
    L.M = take(2 * P * (size_t)hidden);
    L.total = o + 256;  // slack to 256-align a caller pointer
    return L;
}

}  // namespace

// ----------------------------------------------------------------- C ABI --

extern "C" size_t mxfp4_grouped_workspace_bytes(int n_exp, int hidden, int out_dim) {
    return (size_t)n_exp * hidden * sizeof(uint16_t) + (size_t)out_dim * sizeof(float);
}

extern "C" int mxfp4_grouped_gemv_topk(const dsv4_bf16_t* x, const uint8_t* W1_packed,
                                       const uint8_t* W3_packed, const uint8_t* W2_packed,
                                       const uint8_t* W1_scale, const uint8_t* W3_scale,
                                       const uint8_t* W2_scale, const float* rweights, int K_in,
                                       int hidden, int out_dim, int n_exp, dsv4_bf16_t* out,
                                       void* workspace, hipStream_t stream) {
    if (K_in % kBlkElems != 0 || K_in < kBlkElems) {
        std::fprintf(stderr, "mxfp4 grouped: K_in=%d not a positive multiple of %d\n", K_in,
                     kBlkElems);
        return -1;
    }
    if (hidden % kBlkElems != 0 || hidden < kBlkElems) {
        std::fprintf(stderr, "mxfp4 grouped: hidden=%d not a positive multiple of %d\n", hidden,
                     kBlkElems);
        return -2;
    }
    if (K_in > kMaxRed || hidden > kMaxRed) {
        std::fprintf(stderr, "mxfp4 grouped: K_in/hidden > %d\n", kMaxRed);
        return -3;
    }
    if (n_exp < 1 || n_exp > kMaxExpSlots) {
        std::fprintf(stderr, "mxfp4 grouped: n_exp=%d outside [1, %d]\n", n_exp, kMaxExpSlots);
        return -4;
    }
    if (out_dim < 1) {
        std::fprintf(stderr, "mxfp4 grouped: out_dim=%d < 1\n", out_dim);
        return -6;
    }
    // M [n_exp, hidden] bf16 at the first 16-byte boundary of the workspace; the
    // out_dim*4 tail the reference reserves for its fp32 accumulator is unused
    // here and covers the alignment shift.
    const uintptr_t ws = reinterpret_cast<uintptr_t>(workspace);
    const uintptr_t m_at = align_up(ws, 16);
    if (m_at - ws > (uintptr_t)out_dim * sizeof(float)) {
        std::fprintf(stderr, "mxfp4 grouped: workspace not 4-byte aligned\n");
        return -5;
    }
    uint16_t* M = reinterpret_cast<uint16_t*>(m_at);

    ExpertSet es{};
    es.rweights = rweights;
    es.n_slots = n_exp;

    StageAArgs A{};
    A.x = reinterpret_cast<const uint16_t*>(x);
    A.w1 = W1_packed;
    A.w3 = W3_packed;
    A.s1 = W1_scale;
    A.s3 = W3_scale;
    A.w_exp_stride = (int64_t)hidden * (K_in / 2);
    A.s_exp_stride = (int64_t)hidden * (K_in / kBlkElems);
    A.K = K_in;
    A.hidden = hidden;
    A.h_per_wave = stage_a_rows_per_wave();
    A.M = M;
    A.es = es;

    StageBArgs B{};
    B.M = M;
    B.w2 = W2_packed;
    B.s2 = W2_scale;
    B.w_exp_stride = (int64_t)out_dim * (hidden / 2);
    B.s_exp_stride = (int64_t)out_dim * (hidden / kBlkElems);
    B.hidden = hidden;
    B.out_dim = out_dim;
    B.T = 1;
    B.out = reinterpret_cast<uint16_t*>(out);
    B.es = es;

    const bool al_a = aligned16(x) && aligned16(W1_packed) && aligned16(W3_packed);
    const bool al_b = aligned16(W2_packed);
    hipError_t e = al_a ? launch_stage_a<false, true>(A, n_exp, stream)
                        : launch_stage_a<false, false>(A, n_exp, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 grouped: stage A launch failed: %s\n", hipGetErrorString(e));
        return -5;
    }
    e = al_b ? launch_stage_b<1, false, true>(B, stream) : launch_stage_b<1, false, false>(B, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 grouped: stage B launch failed: %s\n", hipGetErrorString(e));
        return -6;
    }
    return 0;
}

extern "C" int mxfp4_moe_route_sigmoid_topk(const float* logits, int T, int n_experts, int topk,
                                            int32_t* ids, float* weights, hipStream_t stream) {
    if (T < 1 || n_experts < 1 || n_experts > kMaxExperts || topk < 1 || topk > kMaxTopk ||
        topk > n_experts) {
        std::fprintf(stderr, "mxfp4 route: bad T=%d n_experts=%d topk=%d\n", T, n_experts, topk);
        return -1;
    }
    hipLaunchKernelGGL(moe_route_sigmoid_topk_kernel, dim3((unsigned)T), dim3(64), 0, stream,
                       logits, n_experts, topk, ids, weights);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 route: launch failed: %s\n", hipGetErrorString(e));
        return -5;
    }
    return 0;
}

extern "C" size_t mxfp4_moe_workspace_bytes(int T, int topk, int n_experts, int hidden) {
    if (T < 1 || topk < 1 || n_experts < 1 || hidden < 1) return 0;
    return moe_layout(T, topk, n_experts, hidden).total;
}

namespace {

struct MoeCall {
    RouteTables rt;
    uint16_t* M;
    ExpertSet es;
};

int moe_validate(int T, int topk, int n_experts, int K_in, int hidden, int out_dim) {
    if (K_in % kBlkElems != 0 || K_in < kBlkElems) return -1;
    if (hidden % kBlkElems != 0 || hidden < kBlkElems) return -2;
    if (K_in > kMaxRed || hidden > kMaxRed) return -3;
    if (T < 1 || T > kMaxTokens || topk < 1 || topk > kMaxTopk || n_experts < 1 ||
        n_experts > kMaxExperts || out_dim < 1) {
        std::fprintf(stderr, "mxfp4 moe: bad T=%d topk=%d n_experts=%d out_dim=%d\n", T, topk,
                     n_experts, out_dim);
        return -4;
    }
    return 0;
}

MoeCall moe_call(int T, int topk, int n_experts, int hidden, void* workspace) {
    const MoeWorkspaceLayout L = moe_layout(T, topk, n_experts, hidden);
    uint8_t* base = reinterpret_cast<uint8_t*>(align_up(reinterpret_cast<uintptr_t>(workspace), 256));
    MoeCall c;
    c.rt.header = reinterpret_cast<int32_t*>(base + L.header);
    c.rt.uexp = reinterpret_cast<int32_t*>(base + L.uexp);
    c.rt.off = reinterpret_cast<int32_t*>(base + L.off);
    c.rt.pair_tok = reinterpret_cast<int32_t*>(base + L.pair_tok);
    c.rt.pair_w = reinterpret_cast<float*>(base + L.pair_w);
    c.M = reinterpret_cast<uint16_t*>(base + L.M);
    c.es = ExpertSet{};
    c.es.n_unique = c.rt.header;
    c.es.uexp = c.rt.uexp;
    c.es.off = c.rt.off;
    c.es.pair_tok = c.rt.pair_tok;
    c.es.pair_w = c.rt.pair_w;
    const int P = T * topk;
    c.es.n_slots = n_experts < P ? n_experts : P;
    return c;
}

}  // namespace

extern "C" int mxfp4_moe_build_routing(const int32_t* ids, const float* weights, int T, int topk,
                                       int n_experts, int hidden, void* workspace,
                                       hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, kBlkElems, hidden, 1);
    if (v != 0) return v;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    hipLaunchKernelGGL(moe_build_pairs_kernel, dim3(1), dim3(kMaxExperts), 0, stream, ids, weights,
                       T, topk, n_experts, c.rt);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 moe: routing launch failed: %s\n", hipGetErrorString(e));
        return -5;
    }
    return 0;
}

extern "C" int mxfp4_moe_swiglu(const dsv4_bf16_t* x, const uint8_t* W1_packed,
                                const uint8_t* W3_packed, const uint8_t* W1_scale,
                                const uint8_t* W3_scale, int T, int topk, int n_experts, int K_in,
                                int hidden, void* workspace, hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, K_in, hidden, 1);
    if (v != 0) return v;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    StageAArgs A{};
    A.x = reinterpret_cast<const uint16_t*>(x);
    A.w1 = W1_packed;
    A.w3 = W3_packed;
    A.s1 = W1_scale;
    A.s3 = W3_scale;
    A.w_exp_stride = (int64_t)hidden * (K_in / 2);
    A.s_exp_stride = (int64_t)hidden * (K_in / kBlkElems);
    A.K = K_in;
    A.hidden = hidden;
    A.h_per_wave = stage_a_rows_per_wave();
    A.M = c.M;
    A.es = c.es;
    const bool al = aligned16(x) && aligned16(W1_packed) && aligned16(W3_packed);
    const hipError_t e = al ? launch_stage_a<true, true>(A, c.es.n_slots, stream)
                            : launch_stage_a<true, false>(A, c.es.n_slots, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 moe: stage A launch failed: %s\n", hipGetErrorString(e));
        return -6;
    }
    return 0;
}

extern "C" int mxfp4_moe_down(const uint8_t* W2_packed, const uint8_t* W2_scale, int T, int topk,
                              int n_experts, int hidden, int out_dim, dsv4_bf16_t* out,
                              void* workspace, hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, kBlkElems, hidden, out_dim);
    if (v != 0) return v;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    StageBArgs B{};
    B.M = c.M;
    B.w2 = W2_packed;
    B.s2 = W2_scale;
    B.w_exp_stride = (int64_t)out_dim * (hidden / 2);
    B.s_exp_stride = (int64_t)out_dim * (hidden / kBlkElems);
    B.hidden = hidden;
    B.out_dim = out_dim;
    B.T = T;
    B.out = reinterpret_cast<uint16_t*>(out);
    B.es = c.es;
    const hipError_t e = aligned16(W2_packed) ? launch_stage_b<kMaxTokens, true, true>(B, stream)
                                              : launch_stage_b<kMaxTokens, true, false>(B, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 moe: stage B launch failed: %s\n", hipGetErrorString(e));
        return -7;
    }
    return 0;
}

extern "C" int mxfp4_moe_grouped_gemv(const dsv4_bf16_t* x, const uint8_t* W1_packed,
                                      const uint8_t* W3_packed, const uint8_t* W2_packed,
                                      const uint8_t* W1_scale, const uint8_t* W3_scale,
                                      const uint8_t* W2_scale, const int32_t* ids,
                                      const float* weights, int T, int topk, int n_experts,
                                      int K_in, int hidden, int out_dim, dsv4_bf16_t* out,
                                      void* workspace, hipStream_t stream) {
    int v = moe_validate(T, topk, n_experts, K_in, hidden, out_dim);
    if (v != 0) return v;
    v = mxfp4_moe_build_routing(ids, weights, T, topk, n_experts, hidden, workspace, stream);
    if (v != 0) return v;
    v = mxfp4_moe_swiglu(x, W1_packed, W3_packed, W1_scale, W3_scale, T, topk, n_experts, K_in,
                         hidden, workspace, stream);
    if (v != 0) return v;
    return mxfp4_moe_down(W2_packed, W2_scale, T, topk, n_experts, hidden, out_dim, out, workspace,
                          stream);
}
