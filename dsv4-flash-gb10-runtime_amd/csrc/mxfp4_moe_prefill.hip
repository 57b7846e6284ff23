// mxfp4_moe_prefill.hip — routed MXFP4 SwiGLU MoE for a prefill chunk (many
// tokens) on the gfx950 matrix cores.
//
// Same result as the decode path (reference runtime/dsv4_engine_mxfp4.py:
// 372-423 applied to every token):
//   out[t] = bf16( sum_k w[t,k] * W2_e . bf16( silu(W1_e x_t) * (W3_e x_t) ) ),  e = ids[t,k]
// For hundreds of tokens the expert products are real GEMMs, so they run on
// v_mfma_f32_16x16x32_bf16. The MXFP4 weights are dequantised exactly to bf16
// in registers (v_cvt_scalef32_pk_bf16_fp4 with the block's E8M0 scale: every
// code * 2^e is a bf16 value) and the activations stay bf16, so the products
// are exact and the sums are fp32, as on the VALU decode path.
//
// Launches (one stream, caller's workspace, no allocation, no atomics on
// results):
//   1. routing: pairs (token, k) grouped by expert, 64-token tiles per expert
//      (listed longest first);
//   2. stage A: per (tile, 64 hidden rows) M[pair, h] = bf16(silu(g) * u);
//   3. stage B: per (tile, 64 output rows) Y[pair, o] = w * (W2_e . M[pair]) in fp32;
//   4. combine: out[t, o] = bf16( sum_k Y[pos(t, k), o] ), k in order.
// Each pair's row is computed independently of the other tokens of its tile,
// so results do not depend on the order of pairs inside an expert.
//
// MFMA tiling: a workgroup (4 waves) owns 64 weight rows x up to 64 tokens of
// one expert; wave w computes rows 16w..16w+15 against 4 token blocks of 16.
// K advances in super-steps of 128 (4 MX blocks): lane l takes row l%16 and
// MX block 4s + l/16 of the super-step, so its 16-byte load is one whole
// block with one scale byte; k-step j (of 4) of the super-step uses elements
// 8j..8j+7 of every lane's block, and the activation operand is read from an
// LDS tile with the same k order. The next super-step's weights and
// activation tile are loaded while the current one is multiplied.

#include <cstdio>

#include "dsv4_device.h"
#include "dsv4_kernels.h"

namespace {

using namespace dsv4;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlk = 32;             // MX block
constexpr int kTileTok = 64;         // tokens per tile
constexpr int kTileRows = 64;        // weight rows per workgroup
constexpr int kStep = 128;           // K per super-step
constexpr int kLdsRow = kStep + 8;   // padded bf16 row of the activation tile (272 B)
constexpr int kMaxTokens = 16384;
constexpr int kMaxTopk = 16;
constexpr int kMaxExperts = 1024;
constexpr int kMaxRed = 8192;
constexpr int kRouteThreads = 1024;
constexpr int kRouteRegs = 8;        // routing entries per thread held in registers

struct PrefillTables {
    int32_t* header;     // [0] tiles, [1] routed pairs
    int32_t* pair_tok;   // [P] token of each pair, grouped by expert
    float* pair_w;       // [P] routing weight of each pair
    int32_t* pos;        // [P] pair index of entry (t, k), -1 if its id is out of range
    int32_t* tile_e;     // [max_tiles] expert of each tile
    int32_t* tile_p0;    // [max_tiles] first pair of each tile
    int32_t* tile_n;     // [max_tiles] pairs in each tile (1..64)
};

// ------------------------------------------------------------- routing ----

// Inclusive scan of one value per thread over a 1024-thread workgroup.
__device__ __forceinline__ int block_scan(int v, int* wtot) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int up = __shfl_up(v, d, 64);
        if (lane >= d) v += up;
    }
    if (lane == 63) wtot[wave] = v;
    __syncthreads();
    // The 16 wave totals in wave order: one shuffle scan over lanes 0..15.
    constexpr int kWavesR = kRouteThreads / 64;
    const int wt = lane < kWavesR ? wtot[lane] : 0;
    int wincl = wt;
#pragma unroll
    for (int d = 1; d < kWavesR; d <<= 1) {
        const int up = __shfl_up(wincl, d, 64);
        if (lane >= d) wincl += up;
    }
    const int add = wave > 0 ? __shfl(wincl, wave - 1, 64) : 0;
    __syncthreads();
    return v + add;
}

// One workgroup: count the pairs of each expert (LDS atomics give each pair a
// slot inside its expert), scan the counts, then write the pair lists, the
// (t, k) -> pair map and the tile list: every full 64-pair tile first, then
// the partial tiles by decreasing size, so that the longest tiles are
// dispatched first and the grid does not end on a few long ones (2% of the
// layer against tiles in expert order). Pair order inside an expert and the
// order of tiles of one size may vary between runs; results depend on
// neither.
__global__ __launch_bounds__(kRouteThreads) void prefill_route_kernel(const int32_t* ids,
                                                                      const float* w, int P,
                                                                      int topk, int n_experts,
                                                                      PrefillTables pt) {
    __shared__ int cnt[kMaxExperts];
    __shared__ int off[kMaxExperts];
    __shared__ int wtot[kRouteThreads / 64];
    __shared__ int hcur[kTileTok];          // next position of a partial tile of each size
    __shared__ int nfull;
    const int tid = threadIdx.x;
    // Up to kRouteRegs * kRouteThreads entries, each thread keeps its
    // entries' ids, weights and slots in registers, with every load issued
    // at once; larger chunks go through pos[] in memory (a round trip per
    // entry and pass).
    const bool regs = P <= kRouteRegs * kRouteThreads;
    int e_r[kRouteRegs], s_r[kRouteRegs];
    float w_r[kRouteRegs];
    if (regs) {
#pragma unroll
        for (int q = 0; q < kRouteRegs; ++q) {
            const int i = min(tid + q * kRouteThreads, P - 1);
            e_r[q] = ids[i];
            w_r[q] = w[i];
        }
    }
    for (int e = tid; e < kMaxExperts; e += kRouteThreads) cnt[e] = 0;
    if (tid < kTileTok) hcur[tid] = 0;
    __syncthreads();
    if (regs) {
#pragma unroll
        for (int q = 0; q < kRouteRegs; ++q) {
            const int i = tid + q * kRouteThreads;
            const int e = e_r[q];
            s_r[q] = (i < P && e >= 0 && e < n_experts) ? atomicAdd(&cnt[e], 1) : -1;  // slot inside e
        }
    } else {
        for (int i = tid; i < P; i += kRouteThreads) {
            const int e = ids[i];
            pt.pos[i] = (e >= 0 && e < n_experts) ? atomicAdd(&cnt[e], 1) : -1;
        }
    }
    __syncthreads();
    const int c = tid < n_experts ? cnt[tid] : 0;
    const int nf = c / kTileTok;                 // full tiles
    const int rem = c % kTileTok;                // size of the partial tile (0: none)
    const int ci = block_scan(c, wtot);
    const int fi = block_scan(nf, wtot);
    if (rem > 0) atomicAdd(&hcur[rem], 1);
    if (tid < n_experts) off[tid] = ci - c;
    if (tid == kRouteThreads - 1) {
        nfull = fi;
        pt.header[1] = ci;
    }
    __syncthreads();
    // Tile list: full tiles first, then partial tiles by decreasing size, so
    // the longest tiles are dispatched first (the order does not change any
    // result). Wave 0 turns the size histogram into start positions.
    if (tid < 64) {
        const int s = 63 - tid;                  // lane l: size 63 - l (lane 63: size 0, none)
        const int h = s > 0 ? hcur[s] : 0;
        int incl = h;
        for (int d = 1; d < 64; d <<= 1) {
            const int up = __shfl_up(incl, d, 64);
            if (tid >= d) incl += up;
        }
        if (s > 0) hcur[s] = nfull + incl - h;
        if (tid == 63) pt.header[0] = nfull + incl;
    }
    __syncthreads();
    if (regs) {
#pragma unroll
        for (int q = 0; q < kRouteRegs; ++q) {
            const int i = tid + q * kRouteThreads;
            if (i < P) {
                int p = -1;
                if (s_r[q] >= 0) {
                    p = off[e_r[q]] + s_r[q];
                    pt.pair_tok[p] = i / topk;
                    pt.pair_w[p] = w_r[q];
                }
                pt.pos[i] = p;
            }
        }
    } else {
        for (int i = tid; i < P; i += kRouteThreads) {
            const int e = ids[i];
            const int slot = pt.pos[i];
            if (slot >= 0) {
                const int p = off[e] + slot;
                pt.pair_tok[p] = i / topk;
                pt.pair_w[p] = w[i];
                pt.pos[i] = p;
            }
        }
    }
    if (tid < n_experts) {
        for (int j = 0; j < nf; ++j) {
            const int t = fi - nf + j;
            pt.tile_e[t] = tid;
            pt.tile_p0[t] = off[tid] + kTileTok * j;
            pt.tile_n[t] = kTileTok;
        }
        if (rem > 0) {
            const int t = atomicAdd(&hcur[rem], 1);
            pt.tile_e[t] = tid;
            pt.tile_p0[t] = off[tid] + kTileTok * nf;
            pt.tile_n[t] = rem;
        }
    }
}

// --------------------------------------------------------------- GEMMs ----

struct GemmArgs {
    const uint16_t* act;        // activation rows: x [T, K] (stage A) or M [P, H] (stage B)
    int64_t act_stride;         // elements between rows
    int act_by_token;           // 1: act row = pair_tok[p] (stage A); 0: act row = p (stage B)
    const uint8_t* wa;          // first weight matrix (W1 or W2), expert-major
    const uint8_t* sa;
    const uint8_t* wb;          // second weight matrix (W3) or null
    const uint8_t* sb;
    int64_t w_exp_stride;       // bytes per expert (packed)
    int64_t s_exp_stride;
    int K;                      // reduction length
    int rows;                   // weight rows per expert (H or O)
    const int32_t* header;
    const int32_t* tile_e;
    const int32_t* tile_p0;
    const int32_t* tile_n;
    const int32_t* pair_tok;
    const float* pair_w;
    uint16_t* M;                // stage A output [P, H] bf16
    float* Y;                   // stage B output [P, O] fp32
};

// 16 bytes of e2m1 codes (one MX block) -> 32 bf16 in 4 operands of 8
// (elements 8j..8j+7 in op[j]), times the block scale 2^(s-127) applied by
// the conversion itself: exact for every byte, since every code times a
// power of two in [2^-127, 2^127] is a bf16 value. The conversion takes the
// scale from the exponent field of its fp32 operand (an E8M0 value), so the
// byte goes straight into that field: byte 0 gives 2^-127, as the decode path
// and reference runtime/e8m0_decode.py:8 do. Byte 0xFF decodes to a scale of 0
// (the kernels' convention): its codes keep only their sign bits (code 8 is
// -0), which the conversion turns into signed zeros.
__device__ __forceinline__ void dequant_block(u32x4 w, uint32_t s, bf16x8* op) {
    const bool zero = s == 0xFFu;
    const float scale = __uint_as_float(zero ? 0u : (s << 23));
    const uint32_t keep = zero ? 0x88888888u : 0xFFFFFFFFu;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t d = w[q] & keep;
        const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0);
        const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1);
        const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2);
        const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3);
        bf16x8 v;
        v[0] = p0[0]; v[1] = p0[1]; v[2] = p1[0]; v[3] = p1[1];
        v[4] = p2[0]; v[5] = p2[1]; v[6] = p3[0]; v[7] = p3[1];
        op[q] = v;
    }
}

// The GEMM of one tile with NTB (1..4) blocks of 16 tokens.
// Weights: each wave owns 16 rows of the workgroup's 64 and reads them in
// macro-steps of 256 k (128 bytes per row): two load instructions per
// matrix, each giving lane l row 8q + l/8 of the wave's 16 and bytes
// 16(l%8)..+15 of the macro-step, i.e. 8 whole 128-byte lines per
// instruction. The wave writes those 16 rows x 128 B to its own LDS staging
// area and reads back, as lane (r, g) (r = l%16, g = l/16), row r's blocks g
// and g + 4: the MX blocks 4s + g of super-steps s = 2m and 2m + 1, the
// operands of the MFMA layout. No other wave reads the area, so the
// hand-over needs no barrier (LDS operations of one wave run in order; the
// fences only keep the compiler from moving them). On MI355X, streaming the
// stage-A weights of 251 experts this way ran at 7.1 TB/s, against 5.9 TB/s
// when every load instruction takes the MFMA layout directly (16 rows x
// 64 bytes: 16 half-used lines per instruction).
// The weights of the next DW super-steps (DW/2 macro-steps) and the
// activation pieces of the next DX super-steps are kept in flight in
// registers: weights stream from HBM and need the deep ring; activations are
// re-read by every row block of the tile and mostly hit L2. Loads complete in
// issue order, so an activation piece issued DX steps ahead is waited for
// together with every weight load issued before it: one-block tiles, which
// have the registers, use DX = DW.
// Each super-step's activation tile is written to one of two LDS buffers
// before the barrier that precedes its multiply.
// SFIX > 0: the super-step count is a compile-time constant and the loop is
// unrolled completely; loads past the last super-step are then dropped at
// compile time and every wait for an in-flight load is exact (a wait at the
// top of a rolled loop covers all loads in flight). The rolled path (SFIX 0)
// needs S to be a multiple of DW and clamps loads to the last macro-step.
constexpr int kDepth = 4;   // super-steps per group of the rolled path (K granule = 512)
constexpr int kDX = 2;
constexpr int kDWDeep = 8;  // weight ring of the unrolled common-K bodies
constexpr int kStgRow = 9;  // 16-byte slots per staged row (8 used: 144-byte stride)

__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <bool TWO, int NTB, int SFIX, int DW, int DX>
__device__ __forceinline__ void prefill_gemm_tile(const GemmArgs& a, int e, int p0, int n, int rb,
                                                  uint16_t (*xs)[kTileTok * kLdsRow],
                                                  const int* s_row, uint8_t* sl, u32x4* stg) {
    static_assert(DW % 2 == 0 && DW % DX == 0 && (SFIX == 0 || SFIX % DW == 0), "ring depths");
    constexpr int DM = DW / 2;                        // weight ring in macro-steps
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int rl = wave * 16 + (lane & 15);           // row within the 64-row block
    const int g = lane >> 4;
    const int nblk = a.K / kBlk;
    // Buffer views of the workgroup's 64 weight rows. The weights are read
    // with the default cache policy: nontemporal loads measured 10% slower
    // here, because the tile's activation rows, which every row block of the
    // tile re-reads, then missed in L2 far more often.
    const int blk_bytes = kTileRows * (a.K / 2);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.wa + (int64_t)e * a.w_exp_stride + (int64_t)rb * blk_bytes), (short)0, blk_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rbv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(TWO ? a.wb + (int64_t)e * a.w_exp_stride + (int64_t)rb * blk_bytes : a.wa), (short)0, blk_bytes,
        0x00020000);
    const int S = SFIX > 0 ? SFIX : a.K / kStep;
    const int SM = S / 2;                             // macro-steps
    // this lane's line-layout piece: row 16*wave + 8q + lane/8, bytes 16*(lane%8) of each macro-step
    const int lq = (wave * 16 + (lane >> 3)) * (a.K / 2) + (lane & 7) * 16;
    const int lq8 = 8 * (a.K / 2);                    // + q * lq8 for the second instruction

    // Scale tile: the block's 64 scale rows of each matrix are one contiguous
    // run of 64*nblk bytes, read 16 bytes per thread per piece and staged in
    // LDS (sl: matrix A, then matrix B) before the first barrier of the loop,
    // each row padded by one dword (stride nblk + 4): the lanes of a scale
    // read take rows r = 0..15 at one column, and the odd dword stride puts
    // them in 16 different banks (at a stride of nblk bytes they all fell in
    // one bank at K = 4096, a 16-way conflict).
    const int spieces = kTileRows * nblk / 16;          // per matrix: 256 .. 1024
    const int srs = nblk + 4;                           // LDS row stride of the scale tile
    const u32x4* SAt = reinterpret_cast<const u32x4*>(a.sa + (int64_t)e * a.s_exp_stride + (int64_t)rb * kTileRows * nblk);
    const u32x4* SBt = TWO ? reinterpret_cast<const u32x4*>(a.sb + (int64_t)e * a.s_exp_stride + (int64_t)rb * kTileRows * nblk) : nullptr;
    // pieces per thread: exact for a compile-time K, else at the K cap
    constexpr int kSAll = (TWO ? 2 : 1) * kTileRows * (SFIX > 0 ? 4 * SFIX : kMaxRed / kBlk) / 16;
    constexpr int kSPer = (kSAll + 255) / 256;
    u32x4 sv[kSPer];
#pragma unroll
    for (int i = 0; i < kSPer; ++i) {
        const int q = t + 256 * i;                          // piece index over A then B
        const int qa = min(q, spieces - 1);
        if constexpr (TWO) {
            const int qb = min(max(q - spieces, 0), spieces - 1);
            sv[i] = q < spieces ? SAt[qa] : SBt[qb];
        } else {
            sv[i] = SAt[qa];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // Activation tile: 16*NTB token rows x 128 columns, 16 bytes per thread
    // per token block: piece t + 256*i is row (t + 256*i) / 16, columns
    // 8*((t + 256*i) % 16) .. +8.
    const uint16_t* xsrc[NTB];
    int xoff[NTB];
#pragma unroll
    for (int i = 0; i < NTB; ++i) {
        const int pi = t + 256 * i;
        xsrc[i] = a.act + (int64_t)s_row[pi >> 4] * a.act_stride + (pi & 15) * 8;
        xoff[i] = (pi >> 4) * kLdsRow + (pi & 15) * 8;
    }
    u32x4 xv[DX][NTB];
    auto load_x = [&](int d, int s) {
        if (SFIX > 0 && s >= S) return;              // compile-time in the unrolled body
        const int so = min(s, S - 1) * kStep;
#pragma unroll
        for (int i = 0; i < NTB; ++i) xv[d][i] = *reinterpret_cast<const u32x4*>(xsrc[i] + so);
    };
    u32x4 la[DM][2], lb[DM][2];
    auto load_w = [&](int d, int m) {
        if (SFIX > 0 && m >= SM) return;
        const int off = lq + min(m, SM - 1) * 128;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            la[d][q] = __builtin_amdgcn_raw_buffer_load_b128(ra, off + q * lq8, 0, 0);
            if constexpr (TWO) lb[d][q] = __builtin_amdgcn_raw_buffer_load_b128(rbv, off + q * lq8, 0, 0);
        }
    };
#pragma unroll
    for (int d = 0; d < DX; ++d) load_x(d, d);
#pragma unroll
    for (int d = 0; d < DM; ++d) load_w(d, d);
    __builtin_amdgcn_sched_barrier(0);
    const int ppr = nblk / 16;                          // 16-byte pieces per scale row
#pragma unroll
    for (int i = 0; i < kSPer; ++i) {
        const int q = t + 256 * i;
        if (q < (TWO ? 2 : 1) * spieces) {
            const int row = q / ppr;                    // over matrix A's 64 rows, then B's
            uint32_t* dst = reinterpret_cast<uint32_t*>(sl + row * srs + (q % ppr) * 16);
#pragma unroll
            for (int c = 0; c < 4; ++c) dst[c] = sv[i][c];
        }
    }
    __syncthreads();  // the scale tile is read before each step's barrier
    const uint8_t* sla = sl + rl * srs + g;                // + 4*s: this lane's block of super-step s
    const uint8_t* slb = sl + kTileRows * srs + rl * srs + g;
    // the wave's staging area: matrix A rows 0..15, then matrix B rows 0..15
    u32x4* sta = stg + wave * (TWO ? 2 : 1) * 16 * kStgRow;
    u32x4* stb = sta + 16 * kStgRow;
    const int wslot = (lane >> 3) * kStgRow + (lane & 7);  // + 8 * kStgRow for q = 1
    const int rslot = (lane & 15) * kStgRow + g;           // + 4 for the second super-step

    f32x4 acc_a[NTB], acc_b[NTB];
#pragma unroll
    for (int b = 0; b < NTB; ++b) {
        acc_a[b] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc_b[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int m0 = 0; m0 < (SFIX > 0 ? SFIX / 2 : SM); m0 += DM) {
#pragma unroll
        for (int dm = 0; dm < DM; ++dm) {
            // macro-step m0 + dm: through the staging area into the MFMA layout
            u32x4 wa_m[2], wb_m[2];
            wave_lds_order();   // the previous macro-step's reads come first
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                sta[wslot + q * 8 * kStgRow] = la[dm][q];
                if constexpr (TWO) stb[wslot + q * 8 * kStgRow] = lb[dm][q];
            }
            wave_lds_order();
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                wa_m[h] = sta[rslot + 4 * h];
                if constexpr (TWO) wb_m[h] = stb[rslot + 4 * h];
            }
            load_w(dm, m0 + dm + DM);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int d = 2 * dm + h;            // super-step within the DW group
                const int s = 2 * m0 + d;
                const int dx = d % DX;
                uint16_t* xb = xs[d & 1];            // s & 1 (m0 a multiple of DM, so 2*m0 is even)
#pragma unroll
                for (int i = 0; i < NTB; ++i) *reinterpret_cast<u32x4*>(xb + xoff[i]) = xv[dx][i];
                load_x(dx, s + DX);
                // The dequantisation needs only this wave's registers and the
                // scale tile, so it runs before the barrier and overlaps the
                // wait for the other waves' activation pieces.
                const uint32_t sa_c = sla[4 * s];
                const uint32_t sb_c = TWO ? slb[4 * s] : 0u;
                bf16x8 opa[4], opb[4];
                dequant_block(wa_m[h], sa_c, opa);
                if constexpr (TWO) dequant_block(wb_m[h], sb_c, opb);
                __syncthreads();
#pragma unroll
                for (int b = 0; b < NTB; ++b) {
                    const uint16_t* xrow = xb + (16 * b + (lane & 15)) * kLdsRow + 32 * g;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const bf16x8 xop = *reinterpret_cast<const bf16x8*>(xrow + 8 * j);
                        acc_a[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(opa[j], xop, acc_a[b], 0, 0, 0);
                        if constexpr (TWO)
                            acc_b[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(opb[j], xop, acc_b[b], 0, 0, 0);
                    }
                }
            }
        }
    }
    // Epilogue: lane holds rows 4g..4g+3 of the wave's 16 (consecutive output
    // columns of one pair row) for token column lane%16 of each block.
    const int c0 = rb * kTileRows + wave * 16 + 4 * g;
#pragma unroll
    for (int b = 0; b < NTB; ++b) {
        const int j = 16 * b + (lane & 15);
        if (j < n) {
            const int p = p0 + j;
            if constexpr (TWO) {
                const uint32_t lo = f32_to_bf16_bits(silu_f32(acc_a[b][0]) * acc_b[b][0]) |
                                    ((uint32_t)f32_to_bf16_bits(silu_f32(acc_a[b][1]) * acc_b[b][1]) << 16);
                const uint32_t hi = f32_to_bf16_bits(silu_f32(acc_a[b][2]) * acc_b[b][2]) |
                                    ((uint32_t)f32_to_bf16_bits(silu_f32(acc_a[b][3]) * acc_b[b][3]) << 16);
                *reinterpret_cast<uint2*>(a.M + (int64_t)p * a.rows + c0) = make_uint2(lo, hi);
            } else {
                const float wt = a.pair_w[p];
                *reinterpret_cast<float4*>(a.Y + (int64_t)p * a.rows + c0) =
                    make_float4(wt * acc_a[b][0], wt * acc_a[b][1], wt * acc_a[b][2], wt * acc_a[b][3]);
            }
        }
    }
}

// grid = tiles8 * (rows / 64) (tiles8 = tiles rounded up to a multiple of
// 8), block = 256. Workgroup L is taken as running on XCD L % 8 (the
// dispatcher's round robin; only locality depends on it): the XCD's k-th
// workgroup, k = L / 8, takes row block k % RB of tile 8 * (k / RB) + L % 8,
// so one tile's row blocks run back to back on one XCD and share its L2
// copy of the tile's activation rows. TWO: stage A (W1 and W3, SwiGLU
// epilogue into M); otherwise stage B (W2, weighted fp32 rows into Y). SFIX:
// the super-step count K / 128 when it is 4, 16 or 32 (unrolled bodies, the
// scale tile sized for that K), else 0 (rolled body, scale tile at the K
// cap). The tile's token-block count selects a specialised body.
template <bool TWO, int SFIX>
__global__ __launch_bounds__(256, 2) void prefill_gemm_kernel(const GemmArgs a, int RB) {
    constexpr int kNblkMax = SFIX > 0 ? 4 * SFIX : kMaxRed / kBlk;
    constexpr int kMats = TWO ? 2 : 1;
    __shared__ __align__(16) uint16_t xs[2][kTileTok * kLdsRow];   // 2 x 17 KB
    __shared__ __align__(16) uint8_t sl[kMats * kTileRows * (kNblkMax + 4)];
    __shared__ u32x4 stg[4 * kMats * 16 * kStgRow];                 // 4.5 KB per wave and matrix
    __shared__ int s_row[kTileTok];
    const int L = blockIdx.x;
    const int k = L >> 3;
    const int rb = k % RB;
    const int ti = 8 * (k / RB) + (L & 7);
    if (ti >= a.header[0]) return;                                  // whole workgroup
    const int t = threadIdx.x;
    const int e = a.tile_e[ti];
    const int p0 = a.tile_p0[ti];
    const int n = a.tile_n[ti];
    if (t < kTileTok) {
        const int p = p0 + min(t, n - 1);
        s_row[t] = a.act_by_token ? a.pair_tok[p] : p;
    }
    __syncthreads();
    // One-block tiles (most tiles of a prefill chunk) keep as many activation
    // pieces in flight as weight super-steps.
    constexpr int DW = (SFIX == 16 || SFIX == 32) ? kDWDeep : kDepth;
    switch ((n + 15) / 16) {
        case 1: prefill_gemm_tile<TWO, 1, SFIX, DW, DW>(a, e, p0, n, rb, xs, s_row, sl, stg); break;
        case 2: prefill_gemm_tile<TWO, 2, SFIX, DW, kDX>(a, e, p0, n, rb, xs, s_row, sl, stg); break;
        case 3: prefill_gemm_tile<TWO, 3, SFIX, DW, kDX>(a, e, p0, n, rb, xs, s_row, sl, stg); break;
        default: prefill_gemm_tile<TWO, 4, SFIX, DW, kDX>(a, e, p0, n, rb, xs, s_row, sl, stg); break;
    }
}

// out[t, o] = bf16( sum_k Y[pos(t, k), o] ), k in order; grid = (T, O / 1024).
__global__ __launch_bounds__(256) void prefill_combine_kernel(const float* Y, const int32_t* pos,
                                                              int topk, int O, uint16_t* out) {
    const int tok = blockIdx.x;
    const int o = (blockIdx.y * 256 + threadIdx.x) * 4;
    if (o >= O) return;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < topk; ++k) {
        const int p = pos[tok * topk + k];
        if (p >= 0) {
            const float4 v = *reinterpret_cast<const float4*>(Y + (int64_t)p * O + o);
            s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
        }
    }
    const uint32_t lo = f32_to_bf16_bits(s.x) | ((uint32_t)f32_to_bf16_bits(s.y) << 16);
    const uint32_t hi = f32_to_bf16_bits(s.z) | ((uint32_t)f32_to_bf16_bits(s.w) << 16);
    *reinterpret_cast<uint2*>(out + (int64_t)tok * O + o) = make_uint2(lo, hi);
}

// ---------------------------------------------------------------- host ----

uintptr_t align_up(uintptr_t v, uintptr_t a) { return (v + a - 1) / a * a; }

// The stage kernel for the reduction length a.K (super-steps of 128).
template <bool TWO>
void launch_gemm(const GemmArgs& a, dim3 grid, int RB, hipStream_t stream) {
    switch (a.K / kStep) {
        case 32: hipLaunchKernelGGL((prefill_gemm_kernel<TWO, 32>), grid, dim3(256), 0, stream, a, RB); break;
        case 16: hipLaunchKernelGGL((prefill_gemm_kernel<TWO, 16>), grid, dim3(256), 0, stream, a, RB); break;
        case 4: hipLaunchKernelGGL((prefill_gemm_kernel<TWO, 4>), grid, dim3(256), 0, stream, a, RB); break;
        default: hipLaunchKernelGGL((prefill_gemm_kernel<TWO, 0>), grid, dim3(256), 0, stream, a, RB); break;
    }
}
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct PrefillLayout {
    size_t header, pair_tok, pair_w, pos, tile_e, tile_p0, tile_n, M, Y, total;
    int max_tiles;
};

PrefillLayout prefill_layout(int T, int topk, int n_experts, int hidden, int out_dim) {
    const size_t P = (size_t)T * topk;
    PrefillLayout L;
    L.max_tiles = (int)((P + kTileTok - 1) / kTileTok) + (n_experts < (int)P ? n_experts : (int)P);
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    L.header = take(16);
    L.pair_tok = take(4 * P);
    L.pair_w = take(4 * P);
    L.pos = take(4 * P);
    L.tile_e = take(4 * (size_t)L.max_tiles);
    L.tile_p0 = take(4 * (size_t)L.max_tiles);
    L.tile_n = take(4 * (size_t)L.max_tiles);
    L.M = take(2 * P * (size_t)hidden);
    L.Y = take(4 * P * (size_t)out_dim);
    L.total = o + 256;
    return L;
}

int prefill_validate(int T, int topk, int n_experts, int K_in, int hidden, int out_dim) {
    constexpr int kRed = kStep * kDepth;   // whole groups of super-steps
    if (K_in % kRed != 0 || K_in < kRed || K_in > kMaxRed) {
        std::fprintf(stderr, "mxfp4_moe_prefill: K_in=%d must be a multiple of %d in [%d, %d]\n",
                     K_in, kRed, kRed, kMaxRed);
        return -1;
    }
    if (hidden % kRed != 0 || hidden < kRed || hidden > kMaxRed) {
        std::fprintf(stderr, "mxfp4_moe_prefill: hidden=%d must be a multiple of %d in [%d, %d]\n",
                     hidden, kRed, kRed, kMaxRed);
        return -2;
    }
    if (out_dim % kTileRows != 0 || out_dim < kTileRows) {
        std::fprintf(stderr, "mxfp4_moe_prefill: out_dim=%d not a positive multiple of %d\n",
                     out_dim, kTileRows);
        return -3;
    }
    if (T < 1 || T > kMaxTokens || topk < 1 || topk > kMaxTopk || n_experts < 1 ||
        n_experts > kMaxExperts) {
        std::fprintf(stderr, "mxfp4_moe_prefill: bad T=%d topk=%d n_experts=%d\n", T, topk,
                     n_experts);
        return -4;
    }
    return 0;
}

}  // namespace

namespace {

// One thread per MX block: the prefill GEMMs' own decode (dequant_block).
__global__ __launch_bounds__(256) void prefill_dequant_kernel(const uint8_t* w, const uint8_t* s, int nblk,
                                                              int64_t total, uint16_t* out) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= total) return;
    const u32x4 v = *reinterpret_cast<const u32x4*>(w + 16 * b);
    bf16x8 op[4];
    dequant_block(v, s[b], op);
    u32x4* o = reinterpret_cast<u32x4*>(out + 32 * b);
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = __builtin_bit_cast(u32x4, op[q]);
}

}  // namespace

extern "C" int mxfp4_moe_prefill_dequant_bf16(const uint8_t* W_packed, const uint8_t* W_scale, int K, int N,
                                              dsv4_bf16_t* out, hipStream_t stream) {
    if (K % kBlk != 0 || K < kBlk) return -1;
    if (N < 1 || !W_packed || !W_scale || !out || !aligned16(W_packed) || !aligned16(out)) return -3;
    const int64_t total = (int64_t)N * (K / kBlk);
    hipLaunchKernelGGL(prefill_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       W_packed, W_scale, K / kBlk, total, reinterpret_cast<uint16_t*>(out));
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

extern "C" size_t mxfp4_moe_prefill_workspace_bytes(int T, int topk, int n_experts, int hidden,
                                                    int out_dim) {
    if (prefill_validate(T, topk, n_experts, kStep * kDepth, hidden,
                         out_dim < kTileRows ? kTileRows : out_dim) != 0)
        return 0;
    return prefill_layout(T, topk, n_experts, hidden, out_dim).total;
}

extern "C" int mxfp4_moe_prefill(const dsv4_bf16_t* x, const uint8_t* W1_packed,
                                 const uint8_t* W3_packed, const uint8_t* W2_packed,
                                 const uint8_t* W1_scale, const uint8_t* W3_scale,
                                 const uint8_t* W2_scale, const int32_t* ids, const float* weights,
                                 int T, int topk, int n_experts, int K_in, int hidden, int out_dim,
                                 dsv4_bf16_t* out, void* workspace, hipStream_t stream) {
    int v = prefill_validate(T, topk, n_experts, K_in, hidden, out_dim);
    if (v != 0) return v;
    if (!x || !W1_packed || !W3_packed || !W2_packed || !W1_scale || !W3_scale || !W2_scale || !ids ||
        !weights || !out || !workspace) {
        std::fprintf(stderr, "mxfp4_moe_prefill: null operand\n");
        return -3;
    }
    if (!aligned16(x) || !aligned16(W1_packed) || !aligned16(W3_packed) || !aligned16(W2_packed) ||
        !aligned16(out)) {
        std::fprintf(stderr, "mxfp4_moe_prefill: x, weights and out must be 16-byte aligned\n");
        return -3;
    }
    const PrefillLayout L = prefill_layout(T, topk, n_experts, hidden, out_dim);
    uint8_t* base = reinterpret_cast<uint8_t*>(align_up(reinterpret_cast<uintptr_t>(workspace), 256));
    PrefillTables pt;
    pt.header = reinterpret_cast<int32_t*>(base + L.header);
    pt.pair_tok = reinterpret_cast<int32_t*>(base + L.pair_tok);
    pt.pair_w = reinterpret_cast<float*>(base + L.pair_w);
    pt.pos = reinterpret_cast<int32_t*>(base + L.pos);
    pt.tile_e = reinterpret_cast<int32_t*>(base + L.tile_e);
    pt.tile_p0 = reinterpret_cast<int32_t*>(base + L.tile_p0);
    pt.tile_n = reinterpret_cast<int32_t*>(base + L.tile_n);
    uint16_t* M = reinterpret_cast<uint16_t*>(base + L.M);
    float* Y = reinterpret_cast<float*>(base + L.Y);
    const int P = T * topk;

    hipLaunchKernelGGL(prefill_route_kernel, dim3(1), dim3(kRouteThreads), 0, stream, ids, weights,
                       P, topk, n_experts, pt);
    if (hipGetLastError() != hipSuccess) return -5;

    GemmArgs A{};
    A.act = reinterpret_cast<const uint16_t*>(x);
    A.act_stride = K_in;
    A.act_by_token = 1;
    A.wa = W1_packed;
    A.sa = W1_scale;
    A.wb = W3_packed;
    A.sb = W3_scale;
    A.w_exp_stride = (int64_t)hidden * (K_in / 2);
    A.s_exp_stride = (int64_t)hidden * (K_in / kBlk);
    A.K = K_in;
    A.rows = hidden;
    A.header = pt.header;
    A.tile_e = pt.tile_e;
    A.tile_p0 = pt.tile_p0;
    A.tile_n = pt.tile_n;
    A.pair_tok = pt.pair_tok;
    A.pair_w = pt.pair_w;
    A.M = M;
    const unsigned tiles8 = (unsigned)((L.max_tiles + 7) / 8 * 8);
    launch_gemm<true>(A, dim3(tiles8 * (unsigned)(hidden / kTileRows)), hidden / kTileRows, stream);
    if (hipGetLastError() != hipSuccess) return -6;

    GemmArgs B = A;
    B.act = M;
    B.act_stride = hidden;
    B.act_by_token = 0;
    B.wa = W2_packed;
    B.sa = W2_scale;
    B.wb = nullptr;
    B.sb = nullptr;
    B.w_exp_stride = (int64_t)out_dim * (hidden / 2);
    B.s_exp_stride = (int64_t)out_dim * (hidden / kBlk);
    B.K = hidden;
    B.rows = out_dim;
    B.M = nullptr;
    B.Y = Y;
    launch_gemm<false>(B, dim3(tiles8 * (unsigned)(out_dim / kTileRows)), out_dim / kTileRows, stream);
    if (hipGetLastError() != hipSuccess) return -7;

    hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)T, (unsigned)((out_dim / 4 + 255) / 256)),
                       dim3(256), 0, stream, Y, pt.pos, topk, out_dim, reinterpret_cast<uint16_t*>(out));
    if (hipGetLastError() != hipSuccess) return -8;
    return 0;
}
