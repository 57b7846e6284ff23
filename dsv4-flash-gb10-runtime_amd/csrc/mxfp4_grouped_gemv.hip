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
#include <cstring>
#include <initializer_list>
#include <mutex>

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
constexpr int kMaxRouterK = 8192;       // router gate row length cap (16 KiB of bf16 per row)

constexpr int kWavesA = 4;              // waves per stage-A workgroup

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
    int n_pairs;                // rows of M / entries of pair_tok, pair_w (indexed)
    int n_experts;              // experts of the per-layer tensors (indexed)
};

// Slot u of a one-token launch (T == 1), with every table read unconditional
// and independent, so the weight loads that depend on the expert id are
// issued after a single round trip. With one token every routed expert serves
// exactly one pair and pairs are grouped by slot, so slot u's pair is pair u.
// Tables past the routed slots hold valid ids (the routing kernel fills them)
// and ids are clamped into range anyway; `valid` says whether u is routed.
template <bool INDEXED>
__device__ __forceinline__ void slot_info_t1(const ExpertSet& s, int u, int& expert, int& pbeg,
                                             float& w, bool& valid) {
    if constexpr (INDEXED) {
        const int U = *s.n_unique;
        expert = min(max(s.uexp[u], 0), s.n_experts - 1);
        pbeg = min(u, s.n_pairs - 1);
        w = s.pair_w[pbeg];
        valid = u < U;
    } else {
        expert = u;
        pbeg = u;
        w = s.rweights[u];
        valid = u < s.n_slots;
    }
}

// slot_info_t1 for slot `u` (wave-uniform) read by all lanes at once: lane l
// loads slot min(l, n_slots-1)'s entries (one round trip, no load depending
// on another) and the wave's slot is broadcast from lane u.
template <bool INDEXED>
__device__ __forceinline__ void slot_info_t1_wave(const ExpertSet& s, int u, int lane, int& expert,
                                                  int& pbeg, float& w, bool& valid) {
    const int t = min(lane, s.n_slots - 1);
    int e_l;
    float w_l;
    int U;
    if constexpr (INDEXED) {
        U = *s.n_unique;
        e_l = s.uexp[t];
        w_l = s.pair_w[min(t, s.n_pairs - 1)];
    } else {
        U = s.n_slots;
        e_l = t;
        w_l = s.rweights[t];
    }
    expert = __builtin_amdgcn_readlane(e_l, u);
    w = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(w_l), u));
    expert = INDEXED ? min(max(expert, 0), s.n_experts - 1) : expert;
    pbeg = min(u, s.n_pairs - 1);
    valid = u < U && u < s.n_slots;
}

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

// NB consecutive E8M0 bytes of a lane's blocks, packed little-endian; bytes of
// blocks at or past nblk read as 0 (their weights are zero-filled too).
template <int NB>
__device__ __forceinline__ uint32_t load_scales(const uint8_t* p, bool vec_ok, int avail) {
    if constexpr (NB == 1) {
        return avail > 0 ? (uint32_t)p[0] : 0u;
    } else {
        if (vec_ok) {
            if constexpr (NB == 2) return *reinterpret_cast<const uint16_t*>(p);
            else return *reinterpret_cast<const uint32_t*>(p);
        }
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < NB; ++j)
            if (j < avail) v |= (uint32_t)p[j] << (8 * j);
        return v;
    }
}

__device__ __forceinline__ float scale_of(uint32_t packed, int j) {
    return e8m0_to_f32((packed >> (8 * j)) & 0xFFu);
}

// Selection rounds over keys held 4 per lane (key 0 = absent or taken; slot
// i of lane l is expert l + 64*i). Each lane first sorts its keys, largest
// first, with an odd-even transposition network that swaps only strictly
// out-of-order neighbours, so equal keys keep their slot order. A round then
// reduces one head per lane, and one ballot names the lanes whose head is the
// maximum: a single such lane holds the pick (its head is the lowest slot
// among its equal keys); with several (equal logits), a wave min over
// 64*slot + lane of their heads finds the lowest expert index, on a
// wave-uniform branch. The winner shifts its list up by one. The state can
// be kept between calls of sorted_heads_rounds, so a wave can stop after the
// pick it needs and make the rest later.
struct SortedHeads {
    uint32_t k[4];   // this lane's remaining keys, largest first (0: none)
    uint32_t s[4];   // their slots
    int me;          // lane r < rounds done: index of pick r
    uint32_t mk;     // lane r < rounds done: key of pick r
};

__device__ __forceinline__ void sorted_heads_init(const uint32_t (&kv)[4], SortedHeads& h) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h.k[i] = kv[i];
        h.s[i] = i;
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
        for (int i = p & 1; i + 1 < 4; i += 2) {
            const bool sw = h.k[i + 1] > h.k[i];
            const uint32_t ka = sw ? h.k[i + 1] : h.k[i], kb = sw ? h.k[i] : h.k[i + 1];
            const uint32_t sa = sw ? h.s[i + 1] : h.s[i], sb = sw ? h.s[i] : h.s[i + 1];
            h.k[i] = ka;
            h.k[i + 1] = kb;
            h.s[i] = sa;
            h.s[i + 1] = sb;
        }
    }
    h.me = 0;
    h.mk = 0;
}

// Rounds r0 .. r1-1 (picks are made in order, so r0 is the number already
// made). KFIX > 0 bounds r1 at compile time (r1 <= KFIX), which unrolls the
// rounds; each unrolled round outside [r0, r1) is skipped by a wave-uniform
// branch.
template <int KFIX>
__device__ __forceinline__ void sorted_heads_rounds(SortedHeads& h, int r0, int r1, int lane) {
    auto round = [&](int r) {
        const uint32_t m = wave_max_u32_uniform(h.k[0]);
        const uint64_t b = __ballot(h.k[0] == m);
        int idx;
        if (__builtin_popcountll(b) == 1) {
            const int l = __builtin_ctzll(b);
            idx = 64 * __builtin_amdgcn_readlane(h.s[0], l) + l;
        } else {
            idx = __builtin_amdgcn_readfirstlane(
                wave_min_i32(h.k[0] == m ? (int)(64 * h.s[0]) + lane : 0x7FFFFFFF));
        }
        const bool hit = lane == (idx & 63);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            h.k[i] = hit ? h.k[i + 1] : h.k[i];
            h.s[i] = hit ? h.s[i + 1] : h.s[i];
        }
        h.k[3] = hit ? 0u : h.k[3];
        h.me = lane == r ? idx : h.me;
        h.mk = lane == r ? m : h.mk;
    };
    if constexpr (KFIX > 0) {
#pragma unroll
        for (int r = 0; r < KFIX; ++r)
            if (r >= r0 && r < r1) round(r);
    } else {
        for (int r = r0; r < r1; ++r) round(r);
    }
}

__device__ __forceinline__ void sorted_heads_rounds_any(SortedHeads& h, int topk, int r0, int r1, int lane) {
    if (topk == 8) sorted_heads_rounds<8>(h, r0, r1, lane);
    else sorted_heads_rounds<0>(h, r0, r1, lane);
}

// Expert index of pick y (0-based; the (y+1)-th largest key, equal keys in
// ascending expert index) by bisection on the key bits: 32 steps, each
// counting the keys at or above a candidate with one ballot per slot. Its
// latency does not grow with y, unlike y + 1 selection rounds; the keys are
// the unsorted ones (slot i of lane l is expert l + 64*i).
__device__ __forceinline__ int pick_by_bisection(const uint32_t (&kv)[4], int y) {
    uint32_t v = 0;
#pragma unroll
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t c = v | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) cnt += __builtin_popcountll(__ballot(kv[i] >= c));
        v = cnt > y ? c : v;
    }
    // v is pick y's key; n of the keys equal to v precede it in index order.
    int n = y;
#pragma unroll
    for (int i = 0; i < 4; ++i) n -= __builtin_popcountll(__ballot(kv[i] > v));
    int idx = 0;
    bool found = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint64_t b = __ballot(kv[i] == v);
        const int c = __builtin_popcountll(b);
        if (!found && n < c) {
            for (int j = 0; j < n; ++j) b &= b - 1;
            idx = 64 * i + __builtin_ctzll(b);
            found = true;
        } else if (!found) {
            n -= c;
        }
    }
    return idx;
}

// How the picks are scored and weighted:
//   kScoreSigmoid (the benchmark configuration): rank the logits; weight
//     w_k = sigmoid(l_k) / sum_k' sigmoid(l_k');
//   kScoreSqrtSoftplus (the reference engine's router,
//     kernel/cpp-engine-mxfp4/routed.cu:156-208): rank the scores
//     s = sqrt(softplus(l)), softplus(l) = max(l, 0) + log1p(exp(-|l|));
//     weight w_k = (s_k / (sum_k' s_k' + 1e-20f)) * scale, evaluated in double
//     with the sum taken in pick order, then rounded to float, as the
//     reference's host code does.
// Ranking is by value, descending, ties to the lower expert index. A NaN
// logit or score ranks below every number (the reference never picks one;
// with fewer than k numbers it aborts, here the NaN entries fill the picks).
enum ScoreMode : int { kScoreSigmoid = 0, kScoreSqrtSoftplus = 1 };

struct Scoring {
    int mode;
    float scale;            // kScoreSqrtSoftplus: the routed scaling factor
};

__device__ __forceinline__ float sqrt_softplus(float l) {
    return sqrtf(fmaxf(l, 0.f) + log1pf(expf(-fabsf(l))));
}

// Order-preserving keys of one token's scores, PER per lane (expert lane +
// 64*i): -0 is taken as +0 and NaN as -inf, so equal values give equal keys;
// entries past n_experts are key 0, below every value.
template <int PER>
__device__ __forceinline__ void keys_of_logits(const float (&lv)[PER], int n_experts, int lane,
                                               const Scoring& sc, uint32_t (&kv)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const float v = sc.mode == kScoreSqrtSoftplus ? sqrt_softplus(lv[i]) : lv[i];
        const float l = (v != v) ? -INFINITY : (v == 0.f ? 0.f : v);
        kv[i] = lane + 64 * i < n_experts ? order_key(l) : 0u;
    }
}

// The loads are unconditional (index clamped into the row) and all in flight
// together: the empty asm keeps the compiler from moving a load into the
// e < n_experts branch, where each would wait for the one before.
template <int PER>
__device__ __forceinline__ void logit_keys(const float* lt, int n_experts, int lane, const Scoring& sc,
                                           uint32_t (&kv)[PER]) {
    float lv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) lv[i] = lt[min(lane + 64 * i, n_experts - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < PER; ++i) asm volatile("" : "+v"(lv[i]));
    keys_of_logits<PER>(lv, n_experts, lane, sc, kv);
}

// Weights of the k picks (lane r < topk holds pick r's key; the result is
// for lane r's pick, 0 on lanes >= topk).
__device__ __forceinline__ float pick_weights(uint32_t mk, int topk, int lane, const Scoring& sc) {
    const float v = lane < topk ? key_value(mk) : 0.f;
    if (sc.mode == kScoreSqrtSoftplus) {
        double sum = 0.0;
        for (int k = 0; k < topk; ++k)
            sum += (double)__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), k));
        const double denom = sum + (double)1e-20f;
        return lane < topk ? (float)(((double)v / denom) * (double)sc.scale) : 0.f;
    }
    const float s = lane < topk ? 1.0f / (1.0f + __expf(-v)) : 0.f;
    return s / wave_sum_f32(s);
}

// Top-k of one token's logits on one wave: descending, ties to the lower
// expert index, weights as `sc` says (Scoring). Lane k < topk
// returns the k-th pick. Each lane holds PER logits (expert lane + 64*i) as
// order-preserving integer keys (larger logit <-> larger key; -0 is taken as
// +0 and NaN as -inf, so equal logits give equal keys); entries past
// n_experts and picked entries are key 0, below every logit. With up to 256
// experts (PER 4) the rounds run on sorted per-lane lists (SortedHeads).
// Otherwise each round is one integer max reduction over
// every key; the winner's index comes from one ballot per element slot
// (lowest slot first, then lowest lane: the lowest expert index among equal
// keys) and is removed by a select.
// `rounds` (1..topk, wave-uniform) stops after the first `rounds` picks: lanes
// at or past it return expert 0. The weights need every pick, so they are
// computed only when rounds == topk (my_w is 0 otherwise).
template <int PER>
__device__ __forceinline__ void wave_topk(const float* lt, int n_experts, int topk, int rounds,
                                          const Scoring& sc, int lane, int& my_e, float& my_w) {
    uint32_t kv[PER];
    logit_keys<PER>(lt, n_experts, lane, sc, kv);
    int me = 0;
    uint32_t mk = 0;
    if constexpr (PER == 4) {
        SortedHeads h;
        sorted_heads_init(kv, h);
        sorted_heads_rounds_any(h, topk, 0, rounds, lane);
        me = h.me;
        mk = h.mk;
    } else for (int k = 0; k < rounds; ++k) {
        uint32_t best = kv[0];
#pragma unroll
        for (int i = 1; i < PER; ++i) best = max(best, kv[i]);
        const uint32_t m = __builtin_amdgcn_readfirstlane(wave_max_u32(best));
        // The last (lowest) slot whose ballot is not empty holds the pick.
        int idx = 0;
#pragma unroll
        for (int i = PER - 1; i >= 0; --i) {
            const uint64_t b = __ballot(kv[i] == m);
            if (b != 0) idx = 64 * i + __builtin_ctzll(b);
        }
        const bool hit = lane == (idx & 63);
        const int slot = idx >> 6;
#pragma unroll
        for (int i = 0; i < PER; ++i) kv[i] = (hit && slot == i) ? 0u : kv[i];
        me = lane == k ? idx : me;
        mk = lane == k ? m : mk;
    }
    my_e = me;
    my_w = rounds == topk ? pick_weights(mk, topk, lane, sc) : 0.f;
}

__device__ __forceinline__ void wave_topk_any(const float* lt, int n_experts, int topk, int rounds,
                                              const Scoring& sc, int lane, int& e, float& w) {
    if (n_experts <= 256) wave_topk<4>(lt, n_experts, topk, rounds, sc, lane, e, w);
    else if (n_experts <= 512) wave_topk<8>(lt, n_experts, topk, rounds, sc, lane, e, w);
    else wave_topk<16>(lt, n_experts, topk, rounds, sc, lane, e, w);
}

// ---------------------------------------------------------------- stage A --

// Device routing tables of the expert-indexed path (in the workspace):
struct RouteTables {
    int32_t* header;            // [0] = unique experts U, [1] = pairs P
    int32_t* uexp;              // [max_unique] expert id per slot, ascending
    int32_t* off;               // [max_unique + 1] pair offsets per slot
    int32_t* pair_tok;          // [T*topk] token of each pair, grouped by slot
    float* pair_w;              // [T*topk] routing weight of each pair
    int n_slots;                // entries of uexp; those past U are set to expert 0
};

// One-token gating folded into stage A (mxfp4_moe_layer at T = 1): every
// workgroup computes the top-k of the logits itself and workgroup (0, 0)
// publishes ids, weights and the routing tables stage B reads.
// One-token routing inside stage A: from logits (the config gating), or
// from the caller's ids and weights (what the routing kernel would build).
struct GateArgs {
    const float* logits;        // [n_experts] fp32, or null when ids are given
    const int32_t* ids_in;      // [topk] given expert ids (logits == null)
    const float* w_in;          // [topk] given weights
    int n_experts;
    int topk;
    int32_t* ids_out;           // [topk] or null (logits only)
    float* w_out;               // [topk] or null
    RouteTables rt;
    Scoring sc;                 // logits only: scoring and weights of the picks
};

// The one-token routing that stage B and the caller read: pick r (lane r <
// topk) is slot r with pair r, token 0 and its weight.
__device__ __forceinline__ void publish_routing(const GateArgs& g, int e, float w, int lane) {
    if (lane < g.topk) {
        if (g.ids_out != nullptr) g.ids_out[lane] = e;
        if (g.w_out != nullptr) g.w_out[lane] = w;
        g.rt.uexp[lane] = e;
        g.rt.off[lane] = lane;
        g.rt.pair_tok[lane] = 0;
        g.rt.pair_w[lane] = w;
        if (lane == 0) {
            g.rt.header[0] = g.topk;
            g.rt.header[1] = g.topk;
            g.rt.off[g.topk] = g.topk;
        }
    }
}

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
    int scale_vec;              // scale rows allow NB-byte vector loads
    uint16_t* M;                // [pairs, hidden] bf16
    ExpertSet es;
    GateArgs gate;
};

// HC hidden rows of W1 and of W3 in registers: NB 16-byte blocks per lane per
// row plus the rows' packed scale bytes. The generic kernel gives lane l
// blocks NB*l .. NB*l+NB-1 (contiguous activation slice and scale bytes); the
// one-token and multi-token kernels give it blocks l, l+64, ... (each load
// instruction of a wave then reads one contiguous KiB of a row).
template <int NB, int HC>
struct GateUpChunk {
    u32x4 w1[HC][NB];
    u32x4 w3[HC][NB];
    uint32_t s1[HC];
    uint32_t s3[HC];
};

// grid = (ceil(hidden / (kWavesA*HC)), expert slots), block = 64*kWavesA.
// Each wave owns one chunk of HC hidden rows; occupancy, not a loop,
// overlaps the loads of different waves. On the FAST path every load is
// unconditional (rows past the end are clamped to the last row, loaded and
// never stored), so the compiler waits on exactly the loads a step needs.
template <int NB, int HC, bool INDEXED, bool FAST, bool MULTI>
__global__ __launch_bounds__(64 * kWavesA, 4) void moe_swiglu_kernel(const StageAArgs a) {
    constexpr bool ALIGNED = FAST;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int expert, pbeg, pend;
    if (!slot_info<INDEXED>(a.es, blockIdx.y, expert, pbeg, pend)) return;
    const int h_begin = (blockIdx.x * kWavesA + wave) * HC;
    if (h_begin >= a.hidden) return;
    const int h_end = min(h_begin + HC, a.hidden);

    const int K = a.K;
    const int nblk = K / kBlkElems;
    const int64_t wrow = K / 2;
    const int b0 = NB * lane;
    const int avail = nblk - b0;  // blocks of this lane inside the row (may be <= 0)
    const uint8_t* W1 = a.w1 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* W3 = a.w3 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* S1 = a.s1 + (int64_t)expert * a.s_exp_stride;
    const uint8_t* S3 = a.s3 + (int64_t)expert * a.s_exp_stride;

    // Rows h0 .. h0+HC-1; on the FAST path rows past h_end are clamped to the
    // last row (loaded, never stored).
    auto load_chunk = [&](int h0, GateUpChunk<NB, HC>& c) {
#pragma unroll
        for (int r = 0; r < HC; ++r) {
            if constexpr (FAST) {
                const int h = min(h0 + r, h_end - 1);
                const int64_t so = (int64_t)h * nblk + b0;
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int64_t wo = (int64_t)h * wrow + (int64_t)(b0 + j) * 16;
                    c.w1[r][j] = ld16_stream(W1 + wo);
                    c.w3[r][j] = ld16_stream(W3 + wo);
                }
                c.s1[r] = load_scales<NB>(S1 + so, true, NB);
                c.s3[r] = load_scales<NB>(S3 + so, true, NB);
            } else {
                const int h = h0 + r;
                const bool hv = h < h_end;
                const int64_t so = (int64_t)h * nblk + b0;
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    if (hv && j < avail) {
                        const int64_t wo = (int64_t)h * wrow + (int64_t)(b0 + j) * 16;
                        c.w1[r][j] = load_w16<ALIGNED>(W1 + wo);
                        c.w3[r][j] = load_w16<ALIGNED>(W3 + wo);
                    } else {
                        c.w1[r][j] = u32x4{0u, 0u, 0u, 0u};
                        c.w3[r][j] = u32x4{0u, 0u, 0u, 0u};
                    }
                }
                c.s1[r] = hv ? load_scales<NB>(S1 + so, a.scale_vec, avail) : 0u;
                c.s3[r] = hv ? load_scales<NB>(S3 + so, a.scale_vec, avail) : 0u;
            }
        }
    };

    uint32_t xs[NB][16];
    auto load_x = [&](int tok) {
        const uint16_t* xt = a.x + (int64_t)tok * K;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (FAST || j < avail) {
                load_act_block<ALIGNED>(xt + (b0 + j) * kBlkElems, xs[j]);
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) xs[j][q] = 0u;
            }
        }
    };

    // Dot products of one chunk against xs, reduced over the wave, SwiGLU'd
    // and stored as bf16 M[p, h0 + r] by one lane per row.
    auto emit = [&](GateUpChunk<NB, HC>& c, int h0, int p) {
        float g[HC], u[HC];
        float chain = 0.f;
#pragma unroll
        for (int r = 0; r < HC; ++r) {
            float gg = 0.f, uu = 0.f;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                reg_barrier_after(c.w1[r][j], chain);
                gg = fmaf(fp4_block_dot(c.w1[r][j], xs[j]), scale_of(c.s1[r], j), gg);
                reg_barrier_after(c.w3[r][j], gg);
                uu = fmaf(fp4_block_dot(c.w3[r][j], xs[j]), scale_of(c.s3[r], j), uu);
                chain = uu;
            }
            g[r] = gg;
            u[r] = uu;
        }
        wave_reduce_n<HC>(g, lane);
        wave_reduce_n<HC>(u, lane);
        const int r = reduced_index<HC>(lane);
        if (reduced_owner<HC>(lane) && h0 + r < h_end)
            a.M[(int64_t)p * a.hidden + h0 + r] = f32_to_bf16_bits(silu_f32(g[0]) * u[0]);
    };

    int tok;
    float wt;
    pair_info<INDEXED>(a.es, pbeg, tok, wt);
    load_x(tok);
    GateUpChunk<NB, HC> ca;
    load_chunk(h_begin, ca);
    emit(ca, h_begin, pbeg);
    if constexpr (MULTI) {
        // Further tokens of this expert: the chunk stays in registers and is
        // reduced against each token's activation.
#pragma unroll 1
        for (int p = pbeg + 1; p < pend; ++p) {
            pair_info<INDEXED>(a.es, p, tok, wt);
            load_x(tok);
#pragma unroll
            for (int r = 0; r < HC; ++r) {
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    reg_barrier(ca.w1[r][j]);
                    reg_barrier(ca.w3[r][j]);
                }
            }
            emit(ca, h_begin, p);
        }
    }
}

// One token (T = 1, or the drop-in entry) on the FAST path: a workgroup of
// kT1Waves waves covers R = kT1Waves*HC consecutive hidden rows of one expert
// slot. Lane l owns MX blocks l, l+64, ... of each row, so every 16-byte
// weight load instruction of a wave reads one contiguous KiB of a row. Each
// thread first issues its share of the token's activation and of the
// workgroup's scale tile (R rows x K/32 bytes of W1 and of W3, 16 bytes per
// thread), then its wave's weight loads (unconditional, rows clamped), and
// only then writes activation and scales to LDS: the wait covers the oldest
// loads only, so the weight stream starts at once. Rows past `hidden` and
// unrouted slots are loaded but not stored.
// GATE: 0 = routing tables given (the routing kernel ran); 1 = rank the
// logits; 2 = the caller's ids and weights.
template <int NB, int HC, bool INDEXED, int kT1Waves, int D, int GATE>
__global__ __launch_bounds__(64 * kT1Waves, 4) void moe_swiglu_t1_kernel(const StageAArgs a) {
    constexpr int kThreads = 64 * kT1Waves;
    constexpr int kRows = kT1Waves * HC;
    constexpr int kXPer = (kMaxRed / 8 + kThreads - 1) / kThreads;  // 16-byte x pieces per thread
    constexpr int kSTile = 2 * kRows * (kMaxRed / kBlkElems);          // scale tile bytes (max K)
    constexpr int kSPer = (kSTile / 16 + kThreads - 1) / kThreads;     // 16-byte scale pieces per thread
    __shared__ u32x4 xl[kMaxRed * 2 / 16];
    __shared__ u32x4 sl[kSTile / 16];
    __shared__ int s_pick[GATE == 2 ? kMaxTopk : 1];
    __shared__ int s_nu[1];
    const uint8_t* slb = reinterpret_cast<const uint8_t*>(sl);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hw = blockIdx.x * kRows;        // first row of the workgroup (hidden % kRows == 0)
    const int h0 = hw + wave * HC;
    const int K = a.K;
    const int nblk = K / kBlkElems;
    const int64_t wrow = K / 2;

    const u32x4* xg = reinterpret_cast<const u32x4*>(a.x);  // token 0
    const int nx = K / 8;
    const int ns = kRows * nblk / 16;                        // 16-byte scale pieces per matrix
    // Gated: the first 256 logits (ids given: the ids and weights) are
    // loaded before the activation, so that the routing waits for them alone
    // (loads complete in issue order).
    float lg[GATE == 1 ? 4 : 1];
    int id_l = 0;
    float idw_l = 0.f;
    if constexpr (GATE == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) lg[i] = a.gate.logits[min(lane + 64 * i, a.gate.n_experts - 1)];
    } else if constexpr (GATE == 2) {
        const int k = min(lane, a.gate.topk - 1);
        id_l = a.gate.ids_in[k];
        idw_l = a.gate.w_in[k];
    }
    u32x4 xv[kXPer];
#pragma unroll
    for (int i = 0; i < kXPer; ++i) xv[i] = xg[min((int)threadIdx.x + kThreads * i, nx - 1)];
    __builtin_amdgcn_sched_barrier(0);  // the activation loads go first

    int expert, pbeg;
    bool valid;
    SortedHeads heads;   // GATE == 1, up to 256 experts: the ranking state
    if constexpr (GATE == 2) {
        // Wave 0 forms the slots the routing kernel would (the same
        // computation in every workgroup): the distinct in-range ids in
        // ascending order, each with the summed weight of its listings (in
        // listing order). Workgroup (0, 0) publishes them for stage B.
        if (wave == 0) {
            const GateArgs& g = a.gate;
            const int e = id_l;
            const float wl = idw_l;
            const bool listed = lane < g.topk;
            bool first = true;
            float wsum = 0.f;
            for (int j = 0; j < g.topk; ++j) {
                const int ej = __builtin_amdgcn_readlane(e, j);
                const float wj = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(wl), j));
                first = first && !(j < lane && ej == e);
                wsum += (ej == e) ? wj : 0.f;
            }
            const bool take = listed && first && e >= 0 && e < g.n_experts;
            const uint64_t tk = __ballot(take);
            const int U = __builtin_popcountll(tk);
            int rank = 0;
            for (int j = 0; j < g.topk; ++j) {
                const int ej = __builtin_amdgcn_readlane(e, j);
                rank += ((tk >> j) & 1) && ej < e;
            }
            if (take) s_pick[rank] = e;
            if (lane >= U && lane < a.es.n_slots) s_pick[lane] = 0;   // valid id for addresses
            if (lane == 0) s_nu[0] = U;
            if (blockIdx.x == 0 && blockIdx.y == 0) {
                if (take) {
                    g.rt.uexp[rank] = e;
                    g.rt.off[rank] = rank;
                    g.rt.pair_tok[rank] = 0;
                    g.rt.pair_w[rank] = wsum;
                }
                if (lane >= U && lane < g.rt.n_slots) g.rt.uexp[lane] = 0;
                if (lane == 0) {
                    g.rt.header[0] = U;
                    g.rt.header[1] = U;
                    g.rt.off[U] = U;
                }
            }
        }
        __syncthreads();
        expert = s_pick[blockIdx.y];
        pbeg = blockIdx.y;
        valid = (int)blockIdx.y < s_nu[0];
    } else if constexpr (GATE == 1) {
        // Every wave ranks the logits itself, so no wave waits on another
        // before its weight loads, and it stops at pick blockIdx.y, the one
        // its workgroup serves: with up to 256 experts, slots 0-3 by selection
        // rounds on sorted per-lane lists and later slots by bisection, whose
        // latency does not grow with the slot. Wave 0 of workgroup (0, 0)
        // publishes the routing for stage B and the caller: with up to 256
        // experts it makes its own pick first and finishes the ranking once
        // its weight loads are in flight (below); with more it ranks all k
        // first.
        const GateArgs& g = a.gate;
        const bool publish = blockIdx.x == 0 && blockIdx.y == 0 && wave == 0;
        int e;
        if (g.n_experts <= 256) {
            uint32_t kv[4];
            keys_of_logits<4>(lg, g.n_experts, lane, g.sc, kv);
            if (blockIdx.y < 4 || publish) {
                sorted_heads_init(kv, heads);
                sorted_heads_rounds_any(heads, g.topk, 0, (int)blockIdx.y + 1, lane);
                e = heads.me;
            } else {
                // wave-wide ballots: called by every lane, wave-uniform result
                e = pick_by_bisection(kv, (int)blockIdx.y);
            }
        } else {
            float w;
            wave_topk_any(g.logits, g.n_experts, g.topk, publish ? g.topk : (int)blockIdx.y + 1, g.sc, lane, e, w);
            if (publish) publish_routing(g, e, w, lane);
        }
        expert = __builtin_amdgcn_readlane(e, (int)blockIdx.y);
        pbeg = blockIdx.y;
        valid = true;
    } else {
        float wt;
        slot_info_t1<INDEXED>(a.es, blockIdx.y, expert, pbeg, wt, valid);
        (void)wt;
    }
    const uint8_t* W1 = a.w1 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* W3 = a.w3 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* S1 = a.s1 + (int64_t)expert * a.s_exp_stride + (int64_t)hw * nblk;
    const uint8_t* S3 = a.s3 + (int64_t)expert * a.s_exp_stride + (int64_t)hw * nblk;
    u32x4 sv[kSPer];
#pragma unroll
    for (int i = 0; i < kSPer; ++i) {
        const int t = min((int)threadIdx.x + kThreads * i, 2 * ns - 1);
        const uint8_t* src = t < ns ? S1 + 16 * t : S3 + 16 * (t - ns);
        sv[i] = *reinterpret_cast<const u32x4*>(src);
    }
    __builtin_amdgcn_sched_barrier(0);  // then the scale tile, then the weights

    GateUpChunk<NB, HC> c;
    auto load_row = [&](int r) {
        const int h = h0 + r;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int64_t wo = (int64_t)h * wrow + (int64_t)(lane + 64 * j) * 16;
            c.w1[r][j] = ld16_stream(W1 + wo);
            c.w3[r][j] = ld16_stream(W3 + wo);
        }
    };
    // The first D rows are in flight before any compute; row r+D is issued
    // right after row r is reduced.
#pragma unroll
    for (int r = 0; r < D; ++r) load_row(r);
    if constexpr (GATE == 1) {
        // The publishing wave ranks the remaining picks while its rows are in
        // flight (keys and lists are in registers: no new load, so nothing
        // here waits for a row).
        const GateArgs& g = a.gate;
        if (g.n_experts <= 256 && blockIdx.x == 0 && blockIdx.y == 0 && wave == 0) {
            __builtin_amdgcn_sched_barrier(0);
            sorted_heads_rounds_any(heads, g.topk, 1, g.topk, lane);
            publish_routing(g, heads.me, pick_weights(heads.mk, g.topk, lane, g.sc), lane);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
        const int idx = threadIdx.x + kThreads * i;
        if (idx < nx) xl[idx] = xv[i];
    }
#pragma unroll
    for (int i = 0; i < kSPer; ++i) {
        const int idx = threadIdx.x + kThreads * i;
        if (idx < 2 * ns) sl[idx] = sv[i];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < HC; ++r) {
        const int row = wave * HC + r;
        uint32_t p1 = 0, p3 = 0;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            p1 |= (uint32_t)slb[row * nblk + lane + 64 * j] << (8 * j);
            p3 |= (uint32_t)slb[kRows * nblk + row * nblk + lane + 64 * j] << (8 * j);
        }
        c.s1[r] = p1;
        c.s3[r] = p3;
    }
    uint32_t xs[NB][16];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = xl[(lane + 64 * j) * 4 + q];
            xs[j][4 * q + 0] = v[0];
            xs[j][4 * q + 1] = v[1];
            xs[j][4 * q + 2] = v[2];
            xs[j][4 * q + 3] = v[3];
        }
    }

    float g[HC], u[HC];
    float chain = 0.f;
#pragma unroll
    for (int r = 0; r < HC; ++r) {
        float gg = 0.f, uu = 0.f;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            reg_barrier_after(c.w1[r][j], chain);
            gg = fmaf(fp4_block_dot(c.w1[r][j], xs[j]), scale_of(c.s1[r], j), gg);
            reg_barrier_after(c.w3[r][j], gg);
            uu = fmaf(fp4_block_dot(c.w3[r][j], xs[j]), scale_of(c.s3[r], j), uu);
            chain = uu;
        }
        g[r] = gg;
        u[r] = uu;
        if (r + D < HC) {
            __builtin_amdgcn_sched_barrier(0);
            load_row(r + D);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wave_reduce_n<HC>(g, lane);
    wave_reduce_n<HC>(u, lane);
    const int r = reduced_index<HC>(lane);
    if (valid && reduced_owner<HC>(lane) && h0 + r < a.hidden)
        a.M[(int64_t)pbeg * a.hidden + h0 + r] = f32_to_bf16_bits(silu_f32(g[0]) * u[0]);
}

// Several tokens (T > 1, expert-indexed routing tables) on the FAST path: the
// one-token kernel's layout with the expert's pairs looped over. A workgroup
// of kTNWaves waves covers R = kTNWaves*HC rows of one unique expert; each
// wave loads its HC rows of W1 and W3 once (lane l owns MX blocks l, l+64, so
// each load instruction reads one KiB of a row) and reduces them against the
// activation of every token that the expert serves. The loads depend on the
// routing tables (slot -> pairs -> tokens) and are issued in that order:
// tables, then the first pair's activation and the workgroup's scale tile,
// then the weight rows, so that waiting for the activation never waits for a
// weight row. Further pairs (an expert routed by several tokens) are staged
// TT at a time once the first pair's dots are done, while the weight rows
// stay in registers.
template <int NB, int HC, int kTNWaves, int TT>
__global__ __launch_bounds__(64 * kTNWaves, 4) void moe_swiglu_tn_kernel(const StageAArgs a) {
    constexpr int kThreads = 64 * kTNWaves;
    constexpr int kRows = kTNWaves * HC;
    constexpr int kXSlot = kMaxRed / 8;                                  // 16-byte pieces per staged activation
    constexpr int kX1 = (kXSlot + kThreads - 1) / kThreads;              // pieces per thread, one activation
    constexpr int kXPer = (TT * kXSlot + kThreads - 1) / kThreads;       // pieces per thread, TT activations
    constexpr int kSTile = 2 * kRows * (kMaxRed / kBlkElems);
    constexpr int kSPer = (kSTile / 16 + kThreads - 1) / kThreads;
    __shared__ u32x4 xl[TT * kXSlot];
    __shared__ u32x4 sl[kSTile / 16];
    const uint8_t* slb = reinterpret_cast<const uint8_t*>(sl);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hw = blockIdx.x * kRows;
    const int h0 = hw + wave * HC;
    const int K = a.K;
    const int nblk = K / kBlkElems;
    const int64_t wrow = K / 2;
    const int nx = K / 8;                      // 16-byte pieces of one token's activation
    const int ns = kRows * nblk / 16;

    const ExpertSet& es = a.es;
    const int y = blockIdx.y;
    const int U = *es.n_unique;
    const int e_raw = es.uexp[y];
    const int pbeg = es.off[y];
    const int pend = es.off[y + 1];
    if (y >= U) return;
    const int expert = min(max(e_raw, 0), es.n_experts - 1);

    const u32x4* xg = reinterpret_cast<const u32x4*>(a.x);
    // The first pair's activation into LDS slot 0.
    u32x4 x1[kX1];
    {
        const int tok = es.pair_tok[pbeg];
#pragma unroll
        for (int i = 0; i < kX1; ++i)
            x1[i] = xg[(int64_t)tok * nx + min((int)threadIdx.x + kThreads * i, nx - 1)];
    }

    const uint8_t* W1 = a.w1 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* W3 = a.w3 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* S1 = a.s1 + (int64_t)expert * a.s_exp_stride + (int64_t)hw * nblk;
    const uint8_t* S3 = a.s3 + (int64_t)expert * a.s_exp_stride + (int64_t)hw * nblk;
    u32x4 sv[kSPer];
#pragma unroll
    for (int i = 0; i < kSPer; ++i) {
        const int t = min((int)threadIdx.x + kThreads * i, 2 * ns - 1);
        const uint8_t* src = t < ns ? S1 + 16 * t : S3 + 16 * (t - ns);
        sv[i] = *reinterpret_cast<const u32x4*>(src);
    }
    __builtin_amdgcn_sched_barrier(0);  // activations and scales before the weights

    // Weights in the order the dots consume them: block pass j of every row,
    // then pass j+1.
    GateUpChunk<NB, HC> c;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
        for (int r = 0; r < HC; ++r) {
            const int64_t wo = (int64_t)(h0 + r) * wrow + (int64_t)(lane + 64 * j) * 16;
            c.w1[r][j] = ld16_stream(W1 + wo);
            c.w3[r][j] = ld16_stream(W3 + wo);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kX1; ++i) {
        const int idx = threadIdx.x + kThreads * i;
        if (idx < nx) xl[idx] = x1[i];
    }
#pragma unroll
    for (int i = 0; i < kSPer; ++i) {
        const int idx = threadIdx.x + kThreads * i;
        if (idx < 2 * ns) sl[idx] = sv[i];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < HC; ++r) {
        const int row = wave * HC + r;
        uint32_t p1 = 0, p3 = 0;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            p1 |= (uint32_t)slb[row * nblk + lane + 64 * j] << (8 * j);
            p3 |= (uint32_t)slb[kRows * nblk + row * nblk + lane + 64 * j] << (8 * j);
        }
        c.s1[r] = p1;
        c.s3[r] = p3;
    }

    // Dots of the wave's rows against staged activation tt, stored as M of
    // pair p. Block pass j of all rows, then pass j+1: only pass j's slice of
    // the activation is in registers, and each row still adds its blocks in
    // ascending order.
    auto emit = [&](int tt, int p) {
        float g[HC], u[HC];
#pragma unroll
        for (int r = 0; r < HC; ++r) g[r] = u[r] = 0.f;
        float chain = 0.f;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            uint32_t xs[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4 v = xl[tt * kXSlot + (lane + 64 * j) * 4 + q];
                xs[4 * q + 0] = v[0];
                xs[4 * q + 1] = v[1];
                xs[4 * q + 2] = v[2];
                xs[4 * q + 3] = v[3];
            }
#pragma unroll
            for (int r = 0; r < HC; ++r) {
                reg_barrier_after(c.w1[r][j], chain);
                g[r] = fmaf(fp4_block_dot(c.w1[r][j], xs), scale_of(c.s1[r], j), g[r]);
                reg_barrier_after(c.w3[r][j], g[r]);
                u[r] = fmaf(fp4_block_dot(c.w3[r][j], xs), scale_of(c.s3[r], j), u[r]);
                chain = u[r];
            }
        }
        wave_reduce_n<HC>(g, lane);
        wave_reduce_n<HC>(u, lane);
        const int r = reduced_index<HC>(lane);
        if (reduced_owner<HC>(lane) && h0 + r < a.hidden)
            a.M[(int64_t)p * a.hidden + h0 + r] = f32_to_bf16_bits(silu_f32(g[0]) * u[0]);
    };
    // The first pair in straight-line code, so that each row's dots start as
    // soon as that row has arrived.
    emit(0, pbeg);
    // Further pairs, TT at a time, against the rows still in registers.
#pragma unroll 1
    for (int pb = pbeg + 1; pb < pend; pb += TT) {
        u32x4 xv[kXPer];
#pragma unroll
        for (int i = 0; i < kXPer; ++i) {
            // pairs past pend repeat the last one: staged, never used
            const int idx = min((int)threadIdx.x + kThreads * i, TT * nx - 1);
            const int tt = idx / nx;
            const int tok = es.pair_tok[min(pb + tt, pend - 1)];
            xv[i] = xg[(int64_t)tok * nx + (idx - tt * nx)];
        }
        __syncthreads();  // every wave is done with the previous pass's slots
#pragma unroll
        for (int i = 0; i < kXPer; ++i) {
            const int idx = threadIdx.x + kThreads * i;
            if (idx < TT * nx) xl[(idx / nx) * kXSlot + idx % nx] = xv[i];
        }
        __syncthreads();
#pragma unroll 1
        for (int tt = 0; tt < min(TT, pend - pb); ++tt) emit(tt, pb + tt);
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
    int scale_vec;
    uint16_t* out;              // [T, out_dim] bf16
    ExpertSet es;
};

// A lane's share of a wave's staged scale rows: 8, 16 (or 4) bytes.
template <int BYTES>
struct ScalePiece;
template <>
struct ScalePiece<4> { typedef uint32_t type; };
template <>
struct ScalePiece<8> { typedef uint64_t type; };
template <>
struct ScalePiece<16> { typedef u32x4 type; };

template <int NBB, int RB>
struct DownRows {
    u32x4 w[RB][NBB];
    uint32_t s[RB];
};

// grid = ceil(out_dim / kRowsB), block = 64*kWavesB. Wave w takes expert
// slots w, w+kWavesB, ... for the workgroup's kRowsB output rows; partial sums
// per (wave, token, row) meet in LDS and are added in wave order. This is the
// general kernel: the one-token and multi-token kernels below cover the
// aligned config shapes; it serves the rest (other hidden sizes, unaligned
// operands, one token with more than 8 routed slots).
template <int NBB, int RB, int WB, int TMAX, bool INDEXED, bool FAST, bool MULTI>
__global__ __launch_bounds__(64 * WB, WB >= 8 ? 2 : 4) void moe_down_kernel(const StageBArgs a) {
    constexpr bool ALIGNED = FAST;
    constexpr int kRowsB = RB;
    constexpr int kWavesB = WB;
    __shared__ float acc[kWavesB][TMAX][kRowsB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar table loads
    const int o0 = blockIdx.x * kRowsB;
    {
        float* accf = &acc[0][0][0];
        for (int i = threadIdx.x; i < kWavesB * TMAX * kRowsB; i += 64 * kWavesB) accf[i] = 0.f;
        __syncthreads();
    }

    int U;
    if constexpr (INDEXED) U = *a.es.n_unique;
    else U = a.es.n_slots;
    const int nblk = a.hidden / kBlkElems;
    const int64_t wrow = a.hidden / 2;
    const int b0 = NBB * lane;
    const int avail = nblk - b0;

    auto load_rows = [&](int u, DownRows<NBB, RB>& d) {
        int expert, pbeg, pend;
        slot_info<INDEXED>(a.es, u, expert, pbeg, pend);
        const uint8_t* W2 = a.w2 + (int64_t)expert * a.w_exp_stride;
        const uint8_t* S2 = a.s2 + (int64_t)expert * a.s_exp_stride;
#pragma unroll
        for (int r = 0; r < kRowsB; ++r) {
            if constexpr (FAST) {
                const int o = min(o0 + r, a.out_dim - 1);
#pragma unroll
                for (int j = 0; j < NBB; ++j)
                    d.w[r][j] = ld16_stream(W2 + (int64_t)o * wrow + (int64_t)(b0 + j) * 16);
                d.s[r] = load_scales<NBB>(S2 + (int64_t)o * nblk + b0, true, NBB);
            } else {
                const int o = o0 + r;
                const bool ov = o < a.out_dim;
#pragma unroll
                for (int j = 0; j < NBB; ++j) {
                    if (ov && j < avail)
                        d.w[r][j] = load_w16<ALIGNED>(W2 + (int64_t)o * wrow + (int64_t)(b0 + j) * 16);
                    else
                        d.w[r][j] = u32x4{0u, 0u, 0u, 0u};
                }
                d.s[r] = ov ? load_scales<NBB>(S2 + (int64_t)o * nblk + b0, a.scale_vec, avail) : 0u;
            }
        }
    };
    auto process = [&](DownRows<NBB, RB>& d, int u) {
        int expert, pbeg, pend;
        slot_info<INDEXED>(a.es, u, expert, pbeg, pend);
        if constexpr (!MULTI) pend = pbeg + 1;  // one pair per slot (T == 1)
#pragma unroll 1
        for (int p = pbeg; p < pend; ++p) {
            int tok;
            float wt;
            pair_info<INDEXED>(a.es, p, tok, wt);
            if (MULTI && pend - pbeg > 1) {
#pragma unroll
                for (int r = 0; r < kRowsB; ++r) {
#pragma unroll
                    for (int j = 0; j < NBB; ++j) reg_barrier(d.w[r][j]);
                }
            }
            uint32_t ms[NBB][16];
#pragma unroll
            for (int j = 0; j < NBB; ++j) {
                if (FAST || j < avail) {
                    load_act_block<true>(a.M + (int64_t)p * a.hidden + (b0 + j) * kBlkElems, ms[j]);
                } else {
#pragma unroll
                    for (int q = 0; q < 16; ++q) ms[j][q] = 0u;
                }
            }
            float part[kRowsB];
            float chain = 0.f;
#pragma unroll
            for (int r = 0; r < kRowsB; ++r) {
                float s = 0.f;
#pragma unroll
                for (int j = 0; j < NBB; ++j) {
                    reg_barrier_after(d.w[r][j], chain);
                    s = fmaf(fp4_block_dot(d.w[r][j], ms[j]), scale_of(d.s[r], j), s);
                    chain = s;
                }
                part[r] = s;
            }
            wave_reduce_n<kRowsB>(part, lane);
            const int r = reduced_index<kRowsB>(lane);
            if (reduced_owner<kRowsB>(lane) && o0 + r < a.out_dim) acc[wave][tok][r] += wt * part[0];
        }
    };

    DownRows<NBB, RB> da;
#pragma unroll 1
    for (int u = wave; u < U; u += kWavesB) {
        load_rows(u, da);
        process(da, u);
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

// One token (T = 1) with whole 16-row tiles, 16-byte aligned scales and at
// most WB expert slots: the one-token path of moe_down_kernel as a kernel of
// its own (no other path shares its registers or code). Wave w takes slot
// w: its table reads are unconditional (slot_info_t1_wave); its M slice, then
// its RB scale rows (one load of RB*NBB bytes per lane, spread through the
// wave's LDS slot), then its W2 rows are issued, so the dots start as soon as
// the first row arrives. No branch surrounds a load. Slots past the routed
// ones load a valid expert's rows and contribute 0. The RB row sums of the
// WB waves meet in LDS and are added in wave order, then rounded to bf16.
template <int NBB, int RB, int WB, bool INDEXED>
__global__ __launch_bounds__(64 * WB, WB >= 8 ? 2 : 4) void moe_down_t1_kernel(const StageBArgs a) {
    __shared__ float acc[WB][RB];
    __shared__ __align__(16) uint8_t sstage[WB][RB * 64 * NBB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int o0 = blockIdx.x * RB;
    const int nblk = a.hidden / kBlkElems;
    const int64_t wrow = a.hidden / 2;
    const int b0 = NBB * lane;
    int expert, pbeg;
    float wt;
    bool valid;
    slot_info_t1_wave<INDEXED>(a.es, wave, lane, expert, pbeg, wt, valid);
    uint32_t ms[NBB][16];
#pragma unroll
    for (int j = 0; j < NBB; ++j)
        load_act_block<true>(a.M + (int64_t)pbeg * a.hidden + (b0 + j) * kBlkElems, ms[j]);
    const uint8_t* W2 = a.w2 + (int64_t)expert * a.w_exp_stride;
    const uint8_t* S2 = a.s2 + (int64_t)expert * a.s_exp_stride;
    using SPiece = typename ScalePiece<RB * NBB>::type;
    const SPiece spiece = *reinterpret_cast<const SPiece*>(S2 + (int64_t)o0 * nblk + lane * (RB * NBB));
    __builtin_amdgcn_sched_barrier(0);  // keep the M and scale loads oldest
    u32x4 w[RB][NBB];
    auto load_row = [&](int r) {
#pragma unroll
        for (int j = 0; j < NBB; ++j)
            w[r][j] = ld16_stream(W2 + (int64_t)(o0 + r) * wrow + (int64_t)(b0 + j) * 16);
    };
#pragma unroll
    for (int r = 0; r < RB; ++r) load_row(r);  // every row in flight before the first dot
    reinterpret_cast<SPiece*>(&sstage[wave][0])[lane] = spiece;
    __builtin_amdgcn_wave_barrier();
    uint32_t sc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < NBB; ++j) v |= (uint32_t)sstage[wave][r * nblk + b0 + j] << (8 * j);
        sc[r] = v;
    }
    float part[RB];
    float chain = 0.f;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < NBB; ++j) {
            reg_barrier_after(w[r][j], chain);
            sum = fmaf(fp4_block_dot(w[r][j], ms[j]), scale_of(sc[r], j), sum);
            chain = sum;
        }
        part[r] = sum;
    }
    wave_reduce_n<RB>(part, lane);
    const int r = reduced_index<RB>(lane);
    if (reduced_owner<RB>(lane)) acc[wave][r] = valid ? wt * part[0] : 0.f;
    __syncthreads();
    if (threadIdx.x < RB) {
        float sum = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < WB; ++w2) sum += acc[w2][threadIdx.x];
        a.out[o0 + threadIdx.x] = f32_to_bf16_bits(sum);
    }
}

// Several tokens (T > 1, expert-indexed) on the FAST path with one MX block
// per lane per row (hidden = 2048): moe_down_kernel's split of the work (a
// workgroup owns RB output rows; wave w takes expert slots w, w+WB, ...) with
// twice the bytes in flight per wave. Lane i of a wave first reads the
// routing entries of the wave's slot i (expert, pair range, first pair's
// token and weight: two round trips for all slots, the rows waiting only for
// the first). Each step then issues
// the loads of two slots at once (2*RB rows) and reduces them in order.
// Further pairs of a slot (an expert routed by several tokens) load their M
// slice on demand. Partial sums per (wave, token, row) meet in LDS and are
// added in wave order, the order of moe_down_kernel, so the results are the
// same bits.
template <int RB, int WB, int TM>
__global__ __launch_bounds__(64 * WB, 4) void moe_down_tn_kernel(const StageBArgs a) {
    __shared__ float acc[WB][TM][RB];
    __shared__ __align__(16) uint8_t sstage[WB][RB * 64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int o0 = blockIdx.x * RB;
    const int nblk = a.hidden / kBlkElems;     // 64
    const int64_t wrow = a.hidden / 2;
    const ExpertSet& es = a.es;
    // Each wave zeroes its own partial sums, so no barrier precedes the
    // loads (a barrier would wait for every table load first).
    for (int i = lane; i < TM * RB; i += 64) (&acc[wave][0][0])[i] = 0.f;

    // The slot count and the wave's table entries are read in one round trip
    // (entries are clamped to valid indices; those past the routed slots are
    // never used); the first pair's token and weight take a second one, which
    // the first slot's loads do not wait for.
    const int su = min(wave + WB * lane, es.n_slots - 1);
    const int U = min(*es.n_unique, es.n_slots);
    const int e_l = min(max(es.uexp[su], 0), es.n_experts - 1);
    const int pb_l = min(max(es.off[su], 0), es.n_pairs - 1);
    const int pe_l = min(max(es.off[su + 1], pb_l + 1), es.n_pairs);
    const int ns = U > wave ? (U - wave + WB - 1) / WB : 0;  // this wave's slots (<= 64, host-checked)
    const int tok_l = min(max(es.pair_tok[pb_l], 0), a.T - 1);
    const float w_l = es.pair_w[pb_l];

    using SPiece = typename ScalePiece<RB>::type;
    struct Rows {
        u32x4 w[RB];
        SPiece sp;
    };
    uint32_t m[16];  // the M slice of the pair being reduced (one at a time)
    auto issue_rows = [&](int i, Rows& b) {
        const int e = __builtin_amdgcn_readlane(e_l, i);
        const uint8_t* W2 = a.w2 + (int64_t)e * a.w_exp_stride;
        const uint8_t* S2 = a.s2 + (int64_t)e * a.s_exp_stride;
        b.sp = *reinterpret_cast<const SPiece*>(S2 + (int64_t)o0 * nblk + lane * RB);
#pragma unroll
        for (int r = 0; r < RB; ++r) b.w[r] = ld16_stream(W2 + (int64_t)(o0 + r) * wrow + lane * 16);
    };
    auto load_m = [&](int p) { load_act_block<true>(a.M + (int64_t)p * a.hidden + lane * kBlkElems, m); };
    // Row r's scale byte for this lane's block is read from the wave's LDS
    // slot where it is used. The barrier applies to the rows' own registers:
    // a copy would make the compiler wait for a row early.
    auto dots = [&](Rows& b, int tok, float wt) {
        float part[RB];
        float chain = 0.f;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            reg_barrier_after(b.w[r], chain);
            part[r] = fmaf(fp4_block_dot(b.w[r], m), scale_of(sstage[wave][r * nblk + lane], 0), 0.f);
            chain = part[r];
        }
        wave_reduce_n<RB>(part, lane);
        const int r = reduced_index<RB>(lane);
        if (reduced_owner<RB>(lane)) acc[wave][tok][r] += wt * part[0];
    };
    // Slot i with its first pair's M slice already loaded.
    auto process = [&](int i, Rows& b) {
        reinterpret_cast<SPiece*>(&sstage[wave][0])[lane] = b.sp;
        __builtin_amdgcn_wave_barrier();
        dots(b, __builtin_amdgcn_readlane(tok_l, i),
             __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(w_l), i)));
        const int p0 = __builtin_amdgcn_readlane(pb_l, i);
        const int p1 = __builtin_amdgcn_readlane(pe_l, i);
#pragma unroll 1
        for (int p = p0 + 1; p < p1; ++p) {
            const int tok = min(max(es.pair_tok[p], 0), a.T - 1);
            const float wt = es.pair_w[p];
            load_m(p);
            dots(b, tok, wt);
        }
    };

    // Two slots per step: the first slot's M slice, both slots' scale bytes
    // and rows, then the first slot is reduced (waiting for its own loads
    // only), then the second slot's M slice (an L2 hit, written by stage A)
    // is loaded into the same registers and the second slot is reduced.
    // Every path through the loop consumes both row buffers; an odd last
    // slot is reduced after the loop.
    int i = 0;
#pragma unroll 1
    for (; i + 1 < ns; i += 2) {
        Rows b0, b1;
        load_m(__builtin_amdgcn_readlane(pb_l, i));
        issue_rows(i, b0);
        issue_rows(i + 1, b1);
        __builtin_amdgcn_sched_barrier(0);
        process(i, b0);
        __builtin_amdgcn_sched_barrier(0);
        load_m(__builtin_amdgcn_readlane(pb_l, i + 1));
        process(i + 1, b1);
    }
    if (i < ns) {
        Rows b0;
        load_m(__builtin_amdgcn_readlane(pb_l, i));
        issue_rows(i, b0);
        process(i, b0);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.T * RB; i += 64 * WB) {
        const int t = i / RB;
        const int r = i % RB;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < WB; ++w) sum += acc[w][t][r];
        a.out[(int64_t)t * a.out_dim + o0 + r] = f32_to_bf16_bits(sum);
    }
}

// ------------------------------------------------------------ routing ------


constexpr int kRouteThreads = 1024;
constexpr int kExpPerThread = kMaxExperts / kRouteThreads;  // 1

// One workgroup of 1024 threads builds the routing tables of T tokens:
//  1. ids/weights: top-k + sigmoid of the logits (one wave per token, 16
//     tokens at a time), or the caller's ids/weights;
//  2. each (token, expert) pair is counted once per expert (an expert listed
//     twice for one token forms one pair whose weight is the sum), and one
//     scan over the experts gives each routed expert its slot (ascending
//     expert id) and pair offset;
//  3. each pair takes a position inside its expert's range with an LDS
//     atomic. Positions inside one expert are unordered, which cannot change
//     results: pairs of one expert belong to distinct tokens, and stage B
//     accumulates every token separately.
// All steps are data-parallel over the T*topk entries (no serial loops).
// Ids outside [0, n_experts) are dropped.
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(const float* logits,
                                                                  const int32_t* ids_in,
                                                                  const float* w_in, int T, int topk,
                                                                  int n_experts, int32_t* ids_out,
                                                                  float* w_out, RouteTables rt, Scoring sc) {
    __shared__ int cnt[kMaxExperts];
    __shared__ int scan[kRouteThreads / 64];
    __shared__ int sid[kMaxTokens * kMaxTopk];
    __shared__ float sw[kMaxTokens * kMaxTopk];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = T * topk;
#pragma unroll
    for (int q = 0; q < kExpPerThread; ++q) cnt[tid * kExpPerThread + q] = 0;
    if (logits != nullptr) {
        for (int t = wave; t < T; t += kRouteThreads / 64) {
            int e;
            float w;
            wave_topk_any(logits + (int64_t)t * n_experts, n_experts, topk, topk, sc, lane, e, w);
            if (lane < topk) {
                sid[t * topk + lane] = e;
                sw[t * topk + lane] = w;
            }
        }
    } else {
        for (int i = tid; i < n; i += kRouteThreads) {
            sid[i] = ids_in[i];
            sw[i] = w_in[i];
        }
    }
    __syncthreads();
    // Per entry: is it the first listing of its expert in its token, and the
    // summed weight of all listings (branch-free over the token's entries).
    constexpr int kEntries = kMaxTokens * kMaxTopk / kRouteThreads;  // 1
    bool take[kEntries];
    float wsum[kEntries];
#pragma unroll
    for (int q = 0; q < kEntries; ++q) {
        const int i = tid + q * kRouteThreads;
        take[q] = false;
        wsum[q] = 0.f;
        if (i < n) {
            const int e = sid[i];
            const int t0 = (i / topk) * topk;
            bool first = true;
            float w = 0.f;
            for (int k = 0; k < topk; ++k) {
                const int ek = sid[t0 + k];
                const float wk = sw[t0 + k];
                first = first && !(t0 + k < i && ek == e);
                w += (ek == e) ? wk : 0.f;
            }
            take[q] = first && e >= 0 && e < n_experts;
            wsum[q] = w;
            if (ids_out != nullptr) ids_out[i] = e;
            if (w_out != nullptr) w_out[i] = sw[i];
            if (take[q]) atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    // Thread tid owns experts kExpPerThread*tid .. +kExpPerThread-1. Scan of
    // (routed flag << 16 | count) (both fields stay < 2^16): serial over the
    // thread's experts, a shuffle scan inside each wave, then wave totals in
    // wave order.
    int c[kExpPerThread];
    int local = 0;
#pragma unroll
    for (int q = 0; q < kExpPerThread; ++q) {
        const int e = tid * kExpPerThread + q;
        c[q] = e < n_experts ? cnt[e] : 0;
        local += ((c[q] > 0) << 16) | c[q];
    }
    int incl = local;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int up = __shfl_up(incl, d, 64);
        if (lane >= d) incl += up;
    }
    if (lane == 63) scan[wave] = incl;
    __syncthreads();
    // The wave totals in wave order: lanes 0..15 of every wave hold them and
    // one shuffle scan gives this wave's offset and the grand total (no
    // serial pass over LDS).
    constexpr int kRouteWaves = kRouteThreads / 64;
    const int wt = lane < kRouteWaves ? scan[lane] : 0;
    int wincl = wt;
#pragma unroll
    for (int d = 1; d < kRouteWaves; d <<= 1) {
        const int up = __shfl_up(wincl, d, 64);
        if (lane >= d) wincl += up;
    }
    const int total = __shfl(wincl, kRouteWaves - 1, 64);
    incl += wave > 0 ? __shfl(wincl, wave - 1, 64) : 0;
    int run = incl - local;
#pragma unroll
    for (int q = 0; q < kExpPerThread; ++q) {
        const int e = tid * kExpPerThread + q;
        if (c[q] > 0) {
            rt.uexp[run >> 16] = e;
            rt.off[run >> 16] = run & 0xFFFF;
        }
        if (e < n_experts) cnt[e] = run & 0xFFFF;  // next free pair position of expert e
        run += ((c[q] > 0) << 16) | c[q];
    }
    if (tid == kRouteThreads - 1) {
        const int U = incl >> 16;
        const int P = incl & 0xFFFF;
        rt.header[0] = U;
        rt.header[1] = P;
        rt.off[U] = P;
    }
    {
        // Slots past the routed ones get a valid expert id, so the one-token
        // kernels may form weight addresses from any slot before checking it.
        for (int u = (total >> 16) + tid; u < rt.n_slots; u += kRouteThreads) rt.uexp[u] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kEntries; ++q) {
        const int i = tid + q * kRouteThreads;
        if (take[q]) {
            const int pos = atomicAdd(&cnt[sid[i]], 1);
            rt.pair_tok[pos] = i / topk;
            rt.pair_w[pos] = wsum[q];
        }
    }
}

// Gating only: one wave per token writes ids [T, topk] and weights [T, topk].
__global__ __launch_bounds__(64) void moe_route_topk_kernel(const float* logits, int n_experts, int topk,
                                                            Scoring sc, int32_t* ids, float* wout) {
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    int e;
    float w;
    wave_topk_any(logits + (int64_t)t * n_experts, n_experts, topk, topk, sc, lane, e, w);
    if (lane < topk) {
        ids[(int64_t)t * topk + lane] = e;
        wout[(int64_t)t * topk + lane] = w;
    }
}

// ------------------------------------------------------------ router -----

// Router gate GEMV (reference kernel/cpp-engine-mxfp4/routed.cu:124-153):
//   logits[t, n] = sum_k Wg[n, k] * x[t, k],  bf16 operands, fp32 accumulate.
// One workgroup per gate row (expert), its kRouterWaves waves splitting the
// row: wave s owns the 64*NJS consecutive 16-byte pieces from 64*NJS*s, lane
// l the pieces 64*(NJS*s + j) + l (each load instruction reads one
// contiguous KiB). The pieces stay in registers while the T tokens'
// activation pieces (L2 hits after the first workgroups) are dotted against
// them with v_dot2_f32_bf16; each wave reduces its sums, and the wave sums
// meet in LDS and are added in wave order. Pieces past the row (K not a
// multiple of 512) are loaded clamped and multiplied by zero activations.
// Four waves per row measured fastest on MI355X for 256 x 4096 (HIP-graph
// replay, weights rotated over 512 MB): 2.44 us at T = 1 and 3.55 at T = 4,
// against 3.13 and 6.40 with one wave per row, 2.45 / 3.63 with two and
// 2.47 / 3.53 with eight.
constexpr int kRouterWaves = 4;
constexpr int kRouterMaxT = 64;

template <int NJ>
__global__ __launch_bounds__(64 * kRouterWaves) void moe_router_gemv_kernel(const uint16_t* x, const uint16_t* wg,
                                                                            int T, int n_rows, int K,
                                                                            float* logits) {
    static_assert(NJ % kRouterWaves == 0, "whole pieces per wave");
    static_assert(kRouterMaxT >= kMaxTokens, "one LDS row per token");
    constexpr int NJS = NJ / kRouterWaves;
    __shared__ float part[kRouterMaxT][kRouterWaves];
    const int lane = threadIdx.x & 63;
    const int s = threadIdx.x >> 6;
    const int row = min((int)blockIdx.x, n_rows - 1);
    const int npc = K / 8;                     // 16-byte pieces per row
    const uint16_t* wr = wg + (int64_t)row * K;
    u32x4 w[NJS];
#pragma unroll
    for (int j = 0; j < NJS; ++j)
        w[j] = ld16_stream(reinterpret_cast<const uint8_t*>(wr + 8 * min(64 * (NJS * s + j) + lane, npc - 1)));
    for (int t = 0; t < T; ++t) {
        const uint16_t* xt = x + (int64_t)t * K;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NJS; ++j) {
            const int pc = 64 * (NJS * s + j) + lane;
            u32x4 xv = *reinterpret_cast<const u32x4*>(xt + 8 * min(pc, npc - 1));
            if (pc >= npc) xv = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = dot2(as_bf16x2(w[j][q]), as_bf16x2(xv[q]), acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) part[t][s] = acc;
    }
    __syncthreads();
    if ((int)threadIdx.x < T) {
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < kRouterWaves; ++q) sum += part[threadIdx.x][q];
        logits[(int64_t)threadIdx.x * n_rows + row] = sum;
    }
}

// Launch shapes (fixed; chosen by sweeps on MI355X):
//   stage A, one token: moe_swiglu_t1_kernel with 4 waves of 4 rows each per
//     workgroup (16 hidden rows of one expert slot);
//   stage A, several tokens: moe_swiglu_tn_kernel, 16 rows per workgroup,
//     two further activations staged per pass;
//   stage A otherwise: moe_swiglu_kernel, one chunk of 4 rows (2 on the
//     checked path) per wave;
//   stage B: 8 output rows per workgroup of 8 waves (one-token, multi-token
//     and general kernels alike).
constexpr int kT1Waves = 4;
constexpr int kChunkFast = 4;
constexpr int kChunkChecked = 2;
constexpr int kRowsDown = 8;
constexpr int kWavesDown = 8;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

uintptr_t align_up(uintptr_t v, uintptr_t a) { return (v + a - 1) / a * a; }

int blocks_per_lane(int K) { return (K / kBlkElems + 63) / 64; }

// NB-byte scale loads are legal when every row's lane offset stays NB-aligned.
int scale_vec_ok(int nb, int nblk, const void* s0, const void* s1) {
    const uintptr_t m = (uintptr_t)nb - 1;
    return nb > 1 && nblk % nb == 0 && (reinterpret_cast<uintptr_t>(s0) & m) == 0 &&
           (reinterpret_cast<uintptr_t>(s1) & m) == 0;
}

// FAST kernels: 16-byte aligned operands, every lane owning NB whole blocks of
// every row (K == 2048*NB) and NB-byte scale loads; other shapes take the
// checked path (HC = 2).
//
// Whether stage A of a one-token launch takes moe_swiglu_t1_kernel (16-byte
// aligned operands, K = 2048 or 4096, whole 16-row tiles, aligned scale rows).
bool stage_a_t1_ok(const StageAArgs& a, bool aligned) {
    const int nb = blocks_per_lane(a.K);
    const bool fast = aligned && a.K == 2048 * nb && (nb == 1 || scale_vec_ok(nb, a.K / kBlkElems, a.s1, a.s3));
    return fast && nb <= 2 && a.hidden % (kT1Waves * 4) == 0 && aligned16(a.s1) && aligned16(a.s3);
}

// gate: the one-token kernel also routes (1: ranks a.gate.logits; 2: takes
// a.gate.ids_in / w_in); requires stage_a_t1_ok and INDEXED.
template <bool INDEXED, bool ALIGNED, bool MULTI>
hipError_t launch_stage_a(StageAArgs a, int slots, hipStream_t stream, int gate = 0) {
    const int nb = blocks_per_lane(a.K);
    a.scale_vec = scale_vec_ok(nb, a.K / kBlkElems, a.s1, a.s3);
    const bool fast = ALIGNED && a.K == 2048 * nb && (nb == 1 || a.scale_vec);
    const bool t1 = !MULTI && stage_a_t1_ok(a, ALIGNED);
    if (gate && !(t1 && INDEXED)) return hipErrorInvalidValue;
    // Several tokens on the FAST path: the multi-token kernel (whole tiles of
    // 16 rows, 16-byte aligned scale rows).
    const bool tn = MULTI && INDEXED && fast && nb <= 2 && a.hidden % 16 == 0 && aligned16(a.s1) &&
                    aligned16(a.s3);
    if (tn) {
        const dim3 gn((unsigned)(a.hidden / 16), (unsigned)slots);
        if (nb == 1) hipLaunchKernelGGL((moe_swiglu_tn_kernel<1, 4, 4, 2>), gn, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((moe_swiglu_tn_kernel<2, 4, 4, 2>), gn, dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    if (t1) {
        const dim3 g1((unsigned)(a.hidden / (kT1Waves * 4)), (unsigned)slots);
        const dim3 b1(64 * kT1Waves);
#define DSV4_T1(NBV)                                                                                              \
    if (gate == 1) hipLaunchKernelGGL((moe_swiglu_t1_kernel<NBV, 4, INDEXED, kT1Waves, 4, INDEXED ? 1 : 0>), g1, b1, \
                                      0, stream, a);                                                             \
    else if (gate == 2) hipLaunchKernelGGL((moe_swiglu_t1_kernel<NBV, 4, INDEXED, kT1Waves, 4, INDEXED ? 2 : 0>),  \
                                           g1, b1, 0, stream, a);                                                 \
    else hipLaunchKernelGGL((moe_swiglu_t1_kernel<NBV, 4, INDEXED, kT1Waves, 4, 0>), g1, b1, 0, stream, a);
        if (nb == 1) { DSV4_T1(1) }
        else { DSV4_T1(2) }
#undef DSV4_T1
        return hipGetLastError();
    }
    const int hc = fast ? kChunkFast : kChunkChecked;
    const dim3 grid((unsigned)((a.hidden + kWavesA * hc - 1) / (kWavesA * hc)), (unsigned)slots);
    const dim3 block(64 * kWavesA);
#define DSV4_A(NBV, HCV, FASTV) \
    hipLaunchKernelGGL((moe_swiglu_kernel<NBV, HCV, INDEXED, FASTV, MULTI>), grid, block, 0, stream, a)
    if (nb == 1) {
        if (fast) DSV4_A(1, kChunkFast, true);
        else DSV4_A(1, kChunkChecked, false);
    } else if (nb == 2) {
        if (fast) DSV4_A(2, kChunkFast, true);
        else DSV4_A(2, kChunkChecked, false);
    } else {
        return hipErrorInvalidValue;
    }
#undef DSV4_A
    return hipGetLastError();
}

template <int TMAX, bool INDEXED, bool ALIGNED, bool MULTI>
hipError_t launch_stage_b(StageBArgs a, hipStream_t stream) {
    const int nb = blocks_per_lane(a.hidden);
    a.scale_vec = scale_vec_ok(nb, a.hidden / kBlkElems, a.s2, a.s2);
    const bool fast = ALIGNED && a.hidden == 2048 * nb && (nb == 1 || a.scale_vec);
    const dim3 grid((unsigned)((a.out_dim + kRowsDown - 1) / kRowsDown));
    const dim3 block(64 * kWavesDown);
    // One token, whole 16-row tiles, 16-byte aligned scales (staged with one
    // load per lane) and at most one expert slot per wave: the one-token kernel.
    if (TMAX == 1 && fast && (nb == 1 || nb == 2) && a.out_dim % 16 == 0 && aligned16(a.s2) &&
        a.es.n_slots <= kWavesDown) {
        if (nb == 1)
            hipLaunchKernelGGL((moe_down_t1_kernel<1, kRowsDown, kWavesDown, INDEXED>), grid, block, 0, stream, a);
        else
            hipLaunchKernelGGL((moe_down_t1_kernel<2, kRowsDown, kWavesDown, INDEXED>), grid, block, 0, stream, a);
        return hipGetLastError();
    }
    // Several tokens, one block per lane per row, whole 8-row tiles, at most
    // 64 slots per wave: the pipelined multi-token kernel.
    if (MULTI && INDEXED && fast && nb == 1 && a.out_dim % 8 == 0 && aligned16(a.s2) &&
        a.es.n_slots <= 64 * kWavesDown && a.T <= kMaxTokens) {
        if (a.T <= 16)
            hipLaunchKernelGGL((moe_down_tn_kernel<kRowsDown, kWavesDown, 16>), grid, block, 0, stream, a);
        else
            hipLaunchKernelGGL((moe_down_tn_kernel<kRowsDown, kWavesDown, kMaxTokens>), grid, block, 0, stream, a);
        return hipGetLastError();
    }
#define DSV4_B(NBV, FASTV) \
    hipLaunchKernelGGL((moe_down_kernel<NBV, kRowsDown, kWavesDown, TMAX, INDEXED, FASTV, MULTI>), grid, block, 0, stream, a)
    if (nb == 1) {
        if (fast) DSV4_B(1, true);
        else DSV4_B(1, false);
    } else if (nb == 2) {
        if (fast) DSV4_B(2, true);
        else DSV4_B(2, false);
    } else {
        return hipErrorInvalidValue;
    }
#undef DSV4_B
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

struct MoeCall {
    RouteTables rt;
    uint16_t* M;
    ExpertSet es;
};

// The extensions reject a null required pointer before any launch; the
// drop-in mxfp4_grouped_gemv_topk keeps the reference's checks (shapes only).
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
    c.es.n_pairs = P;
    c.es.n_experts = n_experts;
    c.rt.n_slots = c.es.n_slots;
    return c;
}

int launch_route(const float* logits, const int32_t* ids, const float* weights, int T, int topk,
                 int n_experts, int32_t* ids_out, float* w_out, const MoeCall& c,
                 hipStream_t stream, Scoring sc = Scoring{kScoreSigmoid, 1.0f}) {
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(kRouteThreads), 0, stream, logits, ids,
                       weights, T, topk, n_experts, ids_out, w_out, c.rt, sc);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 moe: routing launch failed: %s\n", hipGetErrorString(e));
        return -5;
    }
    return 0;
}

int launch_swiglu(const dsv4_bf16_t* x, const uint8_t* W1_packed, const uint8_t* W3_packed,
                  const uint8_t* W1_scale, const uint8_t* W3_scale, int K_in, int hidden, int T,
                  const MoeCall& c, hipStream_t stream, const GateArgs* gate = nullptr) {
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
    A.M = c.M;
    A.es = c.es;
    const bool al = aligned16(x) && aligned16(W1_packed) && aligned16(W3_packed);
    hipError_t e;
    if (gate != nullptr) {
        A.gate = *gate;
        e = launch_stage_a<true, true, false>(A, c.es.n_slots, stream, gate->logits != nullptr ? 1 : 2);
    } else if (T == 1)
        e = al ? launch_stage_a<true, true, false>(A, c.es.n_slots, stream)
               : launch_stage_a<true, false, false>(A, c.es.n_slots, stream);
    else
        e = al ? launch_stage_a<true, true, true>(A, c.es.n_slots, stream)
               : launch_stage_a<true, false, true>(A, c.es.n_slots, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 moe: stage A launch failed: %s\n", hipGetErrorString(e));
        return -6;
    }
    return 0;
}

int launch_down(const uint8_t* W2_packed, const uint8_t* W2_scale, int T, int hidden, int out_dim,
                dsv4_bf16_t* out, const MoeCall& c, hipStream_t stream) {
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
    const bool al = aligned16(W2_packed);
    hipError_t e;
    if (T == 1)
        e = al ? launch_stage_b<1, true, true, false>(B, stream)
               : launch_stage_b<1, true, false, false>(B, stream);
    else
        e = al ? launch_stage_b<kMaxTokens, true, true, true>(B, stream)
               : launch_stage_b<kMaxTokens, true, false, true>(B, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 moe: stage B launch failed: %s\n", hipGetErrorString(e));
        return -7;
    }
    return 0;
}


int router_validate(int T, int n_experts, int K) {
    if (T < 1 || T > kMaxTokens || n_experts < 1 || n_experts > kMaxExperts || K < 8 || K % 8 != 0 ||
        K > kMaxRouterK) {
        std::fprintf(stderr, "mxfp4 router: bad T=%d n_experts=%d K=%d\n", T, n_experts, K);
        return -1;
    }
    return 0;
}

int launch_router(const dsv4_bf16_t* x, const dsv4_bf16_t* W_gate, int T, int n_experts, int K,
                  float* logits, hipStream_t stream) {
    if (!x || !W_gate || !logits || !aligned16(x) || !aligned16(W_gate)) {
        std::fprintf(stderr, "mxfp4 router: x, W_gate and logits must be non-null, x and W_gate 16-byte aligned\n");
        return -3;
    }
    const dim3 grid((unsigned)n_experts), block(64 * kRouterWaves);
    const auto* xp = reinterpret_cast<const uint16_t*>(x);
    const auto* wp = reinterpret_cast<const uint16_t*>(W_gate);
    const int nj = (K / 8 + 63) / 64;
    if (nj <= 4) hipLaunchKernelGGL((moe_router_gemv_kernel<4>), grid, block, 0, stream, xp, wp, T, n_experts, K, logits);
    else if (nj <= 8) hipLaunchKernelGGL((moe_router_gemv_kernel<8>), grid, block, 0, stream, xp, wp, T, n_experts, K, logits);
    else hipLaunchKernelGGL((moe_router_gemv_kernel<16>), grid, block, 0, stream, xp, wp, T, n_experts, K, logits);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 router: launch failed: %s\n", hipGetErrorString(e));
        return -5;
    }
    return 0;
}

// The first half of the routed layer from logits: gating (scored as `sc`)
// and stage A. One token on the aligned path gates inside stage A (one
// launch); otherwise the routing kernel runs first.
int moe_gate_swiglu_impl(const dsv4_bf16_t* x, const float* logits, const uint8_t* W1_packed,
                         const uint8_t* W3_packed, const uint8_t* W1_scale, const uint8_t* W3_scale, int T,
                         int topk, int n_experts, int K_in, int hidden, int32_t* ids_out, float* weights_out,
                         const MoeCall& c, Scoring sc, hipStream_t stream) {
    if (T == 1) {
        StageAArgs probe{};
        probe.K = K_in;
        probe.hidden = hidden;
        probe.s1 = W1_scale;
        probe.s3 = W3_scale;
        const bool al = aligned16(x) && aligned16(W1_packed) && aligned16(W3_packed);
        if (stage_a_t1_ok(probe, al)) {
            GateArgs g{logits, nullptr, nullptr, n_experts, topk, ids_out, weights_out, c.rt, sc};
            return launch_swiglu(x, W1_packed, W3_packed, W1_scale, W3_scale, K_in, hidden, T, c, stream, &g);
        }
    }
    const int v = launch_route(logits, nullptr, nullptr, T, topk, n_experts, ids_out, weights_out, c, stream, sc);
    if (v != 0) return v;
    return launch_swiglu(x, W1_packed, W3_packed, W1_scale, W3_scale, K_in, hidden, T, c, stream);
}

// The routed layer from logits: gating + stage A, then stage B.
int moe_layer_impl(const dsv4_bf16_t* x, const float* logits, const uint8_t* W1_packed,
                   const uint8_t* W3_packed, const uint8_t* W2_packed, const uint8_t* W1_scale,
                   const uint8_t* W3_scale, const uint8_t* W2_scale, int T, int topk, int n_experts,
                   int K_in, int hidden, int out_dim, dsv4_bf16_t* out, int32_t* ids_out,
                   float* weights_out, const MoeCall& c, Scoring sc, hipStream_t stream) {
    const int v = moe_gate_swiglu_impl(x, logits, W1_packed, W3_packed, W1_scale, W3_scale, T, topk, n_experts,
                                       K_in, hidden, ids_out, weights_out, c, sc, stream);
    if (v != 0) return v;
    return launch_down(W2_packed, W2_scale, T, hidden, out_dim, out, c, stream);
}

// Bytes of the routed-dispatch workspace: the layer's workspace, then the
// router logits [T, n_experts] fp32 at a 256-byte boundary.
size_t dispatch_logits_offset(int T, int topk, int n_experts, int hidden) {
    return align_up(moe_layout(T, topk, n_experts, hidden).total, 256);
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
    es.n_pairs = n_exp;
    es.n_experts = n_exp;

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
    hipError_t e = al_a ? launch_stage_a<false, true, false>(A, n_exp, stream)
                        : launch_stage_a<false, false, false>(A, n_exp, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 grouped: stage A launch failed: %s\n", hipGetErrorString(e));
        return -5;
    }
    e = al_b ? launch_stage_b<1, false, true, false>(B, stream)
             : launch_stage_b<1, false, false, false>(B, stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 grouped: stage B launch failed: %s\n", hipGetErrorString(e));
        return -6;
    }
    return 0;
}

namespace {

int route_topk(const float* logits, int T, int n_experts, int topk, Scoring sc, int32_t* ids,
               float* weights, hipStream_t stream) {
    if (T < 1 || n_experts < 1 || n_experts > kMaxExperts || topk < 1 || topk > kMaxTopk ||
        topk > n_experts || (sc.mode != kScoreSigmoid && sc.mode != kScoreSqrtSoftplus)) {
        std::fprintf(stderr, "mxfp4 route: bad T=%d n_experts=%d topk=%d score_mode=%d\n", T, n_experts,
                     topk, sc.mode);
        return -1;
    }
    if (!operands_set("mxfp4 route", {logits, ids, weights})) return kNullOperand;
    hipLaunchKernelGGL(moe_route_topk_kernel, dim3((unsigned)T), dim3(64), 0, stream, logits, n_experts,
                       topk, sc, ids, weights);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::fprintf(stderr, "mxfp4 route: launch failed: %s\n", hipGetErrorString(e));
        return -5;
    }
    return 0;
}

}  // namespace

extern "C" int mxfp4_moe_route_sigmoid_topk(const float* logits, int T, int n_experts, int topk,
                                            int32_t* ids, float* weights, hipStream_t stream) {
    return route_topk(logits, T, n_experts, topk, Scoring{kScoreSigmoid, 1.0f}, ids, weights, stream);
}

extern "C" int mxfp4_moe_route_topk(const float* logits, int T, int n_experts, int topk, int score_mode,
                                    float routed_scale, int32_t* ids, float* weights, hipStream_t stream) {
    return route_topk(logits, T, n_experts, topk, Scoring{score_mode, routed_scale}, ids, weights, stream);
}

extern "C" int mxfp4_moe_router_logits(const dsv4_bf16_t* x, const dsv4_bf16_t* W_gate, int T, int n_experts,
                                       int K, float* logits, hipStream_t stream) {
    const int v = router_validate(T, n_experts, K);
    if (v != 0) return v;
    return launch_router(x, W_gate, T, n_experts, K, logits, stream);
}

extern "C" size_t mxfp4_moe_workspace_bytes(int T, int topk, int n_experts, int hidden) {
    if (T < 1 || topk < 1 || n_experts < 1 || hidden < 1) return 0;
    return moe_layout(T, topk, n_experts, hidden).total;
}

extern "C" int mxfp4_moe_build_routing(const int32_t* ids, const float* weights, int T, int topk,
                                       int n_experts, int hidden, void* workspace,
                                       hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, kBlkElems, hidden, 1);
    if (v != 0) return v;
    if (!operands_set("mxfp4_moe_build_routing", {ids, weights, workspace})) return kNullOperand;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    return launch_route(nullptr, ids, weights, T, topk, n_experts, nullptr, nullptr, c, stream);
}

extern "C" int mxfp4_moe_swiglu(const dsv4_bf16_t* x, const uint8_t* W1_packed,
                                const uint8_t* W3_packed, const uint8_t* W1_scale,
                                const uint8_t* W3_scale, int T, int topk, int n_experts, int K_in,
                                int hidden, void* workspace, hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, K_in, hidden, 1);
    if (v != 0) return v;
    if (!operands_set("mxfp4_moe_swiglu", {x, W1_packed, W3_packed, W1_scale, W3_scale, workspace}))
        return kNullOperand;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    return launch_swiglu(x, W1_packed, W3_packed, W1_scale, W3_scale, K_in, hidden, T, c, stream);
}

extern "C" int mxfp4_moe_gate_swiglu(const dsv4_bf16_t* x, const float* logits, const uint8_t* W1_packed,
                                     const uint8_t* W3_packed, const uint8_t* W1_scale, const uint8_t* W3_scale,
                                     int T, int topk, int n_experts, int K_in, int hidden, int32_t* ids_out,
                                     float* weights_out, void* workspace, hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, K_in, hidden, 1);
    if (v != 0) return v;
    if (topk > n_experts) return -4;
    if (!operands_set("mxfp4_moe_gate_swiglu", {x, logits, W1_packed, W3_packed, W1_scale, W3_scale, workspace}))
        return kNullOperand;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    return moe_gate_swiglu_impl(x, logits, W1_packed, W3_packed, W1_scale, W3_scale, T, topk, n_experts, K_in,
                                hidden, ids_out, weights_out, c, Scoring{kScoreSigmoid, 1.0f}, stream);
}

extern "C" int mxfp4_moe_down(const uint8_t* W2_packed, const uint8_t* W2_scale, int T, int topk,
                              int n_experts, int hidden, int out_dim, dsv4_bf16_t* out,
                              void* workspace, hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, kBlkElems, hidden, out_dim);
    if (v != 0) return v;
    if (!operands_set("mxfp4_moe_down", {W2_packed, W2_scale, out, workspace})) return kNullOperand;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    return launch_down(W2_packed, W2_scale, T, hidden, out_dim, out, c, stream);
}

// Device scratch of mxfp4_moe_grouped_gemv_noalloc: the routing tables and
// the SwiGLU intermediate that the workspace holds otherwise (4 MiB: T*topk
// rows of hidden bf16 plus the tables). Each GPU the library runs on holds its
// own copy until the process ends. Host code uses the per-device address from
// hipGetSymbolAddress, never the array's name.
constexpr size_t kScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

// mxfp4_moe_grouped_gemv after validation, on the given workspace.
int moe_grouped_impl(const dsv4_bf16_t* x, const uint8_t* W1_packed, const uint8_t* W3_packed,
                     const uint8_t* W2_packed, const uint8_t* W1_scale, const uint8_t* W3_scale,
                     const uint8_t* W2_scale, const int32_t* ids, const float* weights, int T, int topk,
                     int n_experts, int K_in, int hidden, int out_dim, dsv4_bf16_t* out, void* workspace,
                     hipStream_t stream) {
    int v;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    if (T == 1) {
        // One token: stage A forms the slots from the ids itself (two
        // launches in all; the same slots, weights and results as the
        // routing kernel's).
        StageAArgs probe{};
        probe.K = K_in;
        probe.hidden = hidden;
        probe.s1 = W1_scale;
        probe.s3 = W3_scale;
        const bool al = aligned16(x) && aligned16(W1_packed) && aligned16(W3_packed);
        if (stage_a_t1_ok(probe, al)) {
            GateArgs g{nullptr, ids, weights, n_experts, topk, nullptr, nullptr, c.rt, Scoring{kScoreSigmoid, 1.0f}};
            v = launch_swiglu(x, W1_packed, W3_packed, W1_scale, W3_scale, K_in, hidden, T, c, stream, &g);
            if (v != 0) return v;
            return launch_down(W2_packed, W2_scale, T, hidden, out_dim, out, c, stream);
        }
    }
    v = launch_route(nullptr, ids, weights, T, topk, n_experts, nullptr, nullptr, c, stream);
    if (v != 0) return v;
    v = launch_swiglu(x, W1_packed, W3_packed, W1_scale, W3_scale, K_in, hidden, T, c, stream);
    if (v != 0) return v;
    return launch_down(W2_packed, W2_scale, T, hidden, out_dim, out, c, stream);
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up on its first use.
int scratch_for_current_device(void** ptr) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        std::fprintf(stderr, "mxfp4 moe noalloc: no current device\n");
        return -9;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            std::fprintf(stderr, "mxfp4 moe noalloc: hipGetSymbolAddress failed: %s\n", hipGetErrorString(e));
            return -9;
        }
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" int mxfp4_moe_grouped_gemv(const dsv4_bf16_t* x, const uint8_t* W1_packed,
                                      const uint8_t* W3_packed, const uint8_t* W2_packed,
                                      const uint8_t* W1_scale, const uint8_t* W3_scale,
                                      const uint8_t* W2_scale, const int32_t* ids,
                                      const float* weights, int T, int topk, int n_experts,
                                      int K_in, int hidden, int out_dim, dsv4_bf16_t* out,
                                      void* workspace, hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, K_in, hidden, out_dim);
    if (v != 0) return v;
    if (!operands_set("mxfp4_moe_grouped_gemv", {x, W1_packed, W3_packed, W2_packed, W1_scale, W3_scale, W2_scale,
                                                 ids, weights, out, workspace}))
        return kNullOperand;
    return moe_grouped_impl(x, W1_packed, W3_packed, W2_packed, W1_scale, W3_scale, W2_scale, ids, weights, T,
                            topk, n_experts, K_in, hidden, out_dim, out, workspace, stream);
}

extern "C" int mxfp4_moe_grouped_gemv_noalloc(const dsv4_bf16_t* x, const uint8_t* W1_packed,
                                              const uint8_t* W3_packed, const uint8_t* W2_packed,
                                              const uint8_t* W1_scale, const uint8_t* W3_scale,
                                              const uint8_t* W2_scale, const int32_t* ids,
                                              const float* weights, int T, int topk, int n_experts,
                                              int K_in, int hidden, int out_dim, dsv4_bf16_t* out,
                                              hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, K_in, hidden, out_dim);
    if (v != 0) return v;
    const size_t need = moe_layout(T, topk, n_experts, hidden).total;
    if (need > kScratchBytes) {
        std::fprintf(stderr,
                     "mxfp4_moe_grouped_gemv_noalloc: T=%d topk=%d hidden=%d needs %zu bytes of scratch, "
                     "more than the %zu the library holds; use mxfp4_moe_grouped_gemv with a workspace\n",
                     T, topk, hidden, need, kScratchBytes);
        return -8;
    }
    if (!operands_set("mxfp4_moe_grouped_gemv_noalloc", {x, W1_packed, W3_packed, W2_packed, W1_scale, W3_scale,
                                                         W2_scale, ids, weights, out}))
        return kNullOperand;
    void* ws = nullptr;
    const int r = scratch_for_current_device(&ws);
    if (r != 0) return r;
    return moe_grouped_impl(x, W1_packed, W3_packed, W2_packed, W1_scale, W3_scale, W2_scale, ids, weights, T,
                            topk, n_experts, K_in, hidden, out_dim, out, ws, stream);
}

extern "C" int mxfp4_moe_layer(const dsv4_bf16_t* x, const float* logits,
                               const uint8_t* W1_packed, const uint8_t* W3_packed,
                               const uint8_t* W2_packed, const uint8_t* W1_scale,
                               const uint8_t* W3_scale, const uint8_t* W2_scale, int T, int topk,
                               int n_experts, int K_in, int hidden, int out_dim, dsv4_bf16_t* out,
                               int32_t* ids_out, float* weights_out, void* workspace,
                               hipStream_t stream) {
    const int v = moe_validate(T, topk, n_experts, K_in, hidden, out_dim);
    if (v != 0) return v;
    if (topk > n_experts) return -4;
    if (!operands_set("mxfp4_moe_layer", {x, logits, W1_packed, W3_packed, W2_packed, W1_scale, W3_scale, W2_scale,
                                          out, workspace}))
        return kNullOperand;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    return moe_layer_impl(x, logits, W1_packed, W3_packed, W2_packed, W1_scale, W3_scale, W2_scale, T, topk,
                          n_experts, K_in, hidden, out_dim, out, ids_out, weights_out, c,
                          Scoring{kScoreSigmoid, 1.0f}, stream);
}

extern "C" size_t mxfp4_moe_dispatch_workspace_bytes(int T, int topk, int n_experts, int hidden) {
    if (T < 1 || topk < 1 || n_experts < 1 || hidden < 1) return 0;
    return dispatch_logits_offset(T, topk, n_experts, hidden) + (size_t)T * n_experts * sizeof(float) + 256;
}

extern "C" int mxfp4_moe_routed_dispatch(const dsv4_bf16_t* x, const dsv4_bf16_t* W_gate,
                                         const uint8_t* W1_packed, const uint8_t* W3_packed,
                                         const uint8_t* W2_packed, const uint8_t* W1_scale,
                                         const uint8_t* W3_scale, const uint8_t* W2_scale, int T, int topk,
                                         int n_experts, int K_in, int hidden, int out_dim, float routed_scale,
                                         dsv4_bf16_t* out, int32_t* ids_out, float* weights_out,
                                         void* workspace, hipStream_t stream) {
    int v = moe_validate(T, topk, n_experts, K_in, hidden, out_dim);
    if (v != 0) return v;
    if (topk > n_experts) return -4;
    if (router_validate(T, n_experts, K_in) != 0) return -4;
    if (!operands_set("mxfp4_moe_routed_dispatch", {x, W_gate, W1_packed, W3_packed, W2_packed, W1_scale,
                                                    W3_scale, W2_scale, out, workspace}))
        return kNullOperand;
    const MoeCall c = moe_call(T, topk, n_experts, hidden, workspace);
    uint8_t* base = reinterpret_cast<uint8_t*>(align_up(reinterpret_cast<uintptr_t>(workspace), 256));
    float* logits = reinterpret_cast<float*>(base + dispatch_logits_offset(T, topk, n_experts, hidden));
    v = launch_router(x, W_gate, T, n_experts, K_in, logits, stream);
    if (v != 0) return v == -3 ? -3 : -5;
    return moe_layer_impl(x, logits, W1_packed, W3_packed, W2_packed, W1_scale, W3_scale, W2_scale, T, topk,
                          n_experts, K_in, hidden, out_dim, out, ids_out, weights_out, c,
                          Scoring{kScoreSqrtSoftplus, routed_scale}, stream);
}
