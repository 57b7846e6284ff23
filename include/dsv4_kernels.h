/*
 * dsv4_kernels.h — C ABI of the MI355X (gfx950) quantized decode kernels.
 *
 * Four shared libraries export these symbols under the reference's file names,
 * so a caller that dlopen()s / ctypes-loads the reference .so files can load
 * these instead:
 *
 *   kernel/mxfp4-routed/libmxfp4_grouped_gemv.so  mxfp4_grouped_gemv_topk,
 *                                                 mxfp4_grouped_workspace_bytes,
 *                                                 mxfp4_moe_* (extensions)
 *   kernel/mxfp4-dense/libmxfp4_gemv.so           mxfp4_gemv_m1,
 *                                                 mxfp4_dequant_bf16 (extension)
 *   kernel/fp8-dense/libfp8_e4m3_gemv.so          fp8_e4m3_gemv_m1,
 *                                                 fp8_e4m3_gemv, fp8_e4m3_gemv_grouped,
 *                                                 fp8_e4m3_gemv_multi,
 *                                                 fp8_e4m3_gemv_f32s, fp8_e4m3_swiglu_gemv,
 *                                                 fp8_e4m3_rmsnorm_gemv,
 *                                                 fp8_e4m3_dequant_bf16 (extensions)
 *   kernel/rmsnorm-fuse/librmsnorm_fuse.so        rmsnorm_fuse_fwd,
 *                                                 rmsnorm_fuse_residual_add
 *
 * Conventions shared by every entry point:
 *   - every pointer is a device pointer; the caller owns every buffer
 *     (the kernels never allocate device memory);
 *   - bf16 tensors are passed as raw 16-bit storage (dsv4_bf16_t);
 *   - `stream` is a hipStream_t (an opaque pointer; ctypes passes c_void_p);
 *   - host-side validation runs before any launch and returns the reference's
 *     error codes; only launch errors are detected (no device sync).
 *
 * MXFP4 layout (OCP MX v1.0): e2m1 codes packed two per byte, low nibble =
 * even element, high nibble = odd element; one E8M0 scale byte per 32
 * contiguous K-elements, scale = 2^(byte-127), byte 0xFF decodes to 0.0.
 * FP8 layout: one E4M3FN byte per element, one E8M0 byte per 128x128 tile.
 */
#ifndef DSV4_KERNELS_H
#define DSV4_KERNELS_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t dsv4_bf16_t;

/* ------------------------------------------------------------------------ */
/* libmxfp4_grouped_gemv.so                                                  */
/* ------------------------------------------------------------------------ */

/* Routed SwiGLU MoE for one decode token over n_exp packed experts:
 *   out = bf16( sum_e rweights[e] * W2_e . bf16( silu(W1_e x) * (W3_e x) ) )
 * Layouts: W1/W3 packed [n_exp, hidden, K_in/2], scales [n_exp, hidden, K_in/32];
 * W2 packed [n_exp, out_dim, hidden/2], scale [n_exp, out_dim, hidden/32].
 * Returns 0; -1 K_in%32 or K_in < 32; -2 hidden%32 or hidden < 32; -3 K_in or
 * hidden > 4096; -4 n_exp outside [1, 256] (the reference accepts only its
 * compiled-in 6); -5/-6 launch failure of stage A/B, also out_dim < 1 (-6).
 * Replaces mxfp4_grouped_gemv_topk, reference
 * kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:294-310. */
int mxfp4_grouped_gemv_topk(const dsv4_bf16_t* x,
                            const uint8_t* W1_packed, const uint8_t* W3_packed,
                            const uint8_t* W2_packed,
                            const uint8_t* W1_scale, const uint8_t* W3_scale,
                            const uint8_t* W2_scale,
                            const float* rweights,
                            int K_in, int hidden, int out_dim, int n_exp,
                            dsv4_bf16_t* out, void* workspace, hipStream_t stream);

/* Workspace bytes for mxfp4_grouped_gemv_topk: n_exp*hidden*2 + out_dim*4
 * (the same formula as the reference, so caller-side preallocation matches).
 * Replaces kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:406-409. */
size_t mxfp4_grouped_workspace_bytes(int n_exp, int hidden, int out_dim);

/* EXTENSION (no reference counterpart; the reference routes on the host,
 * kernel/cpp-engine-mxfp4/routed.cu:169-208). Device-side gating for T tokens:
 * ids[t, :] = top-`topk` expert indices of logits[t, :] (descending, ties to
 * the lower index); weights[t, k] = sigmoid(l_k) / sum_k' sigmoid(l_k').
 * Returns 0; -1 bad T/n_experts/topk (T<1, n_experts<1 or >1024, topk<1 or
 * > min(n_experts, 16)); -10 logits, ids or weights null; -5 launch failure. */
int mxfp4_moe_route_sigmoid_topk(const float* logits, int T, int n_experts, int topk,
                                 int32_t* ids, float* weights, hipStream_t stream);

/* EXTENSION: device gating with a choice of scoring, for T tokens:
 *   score_mode 0: rank the logits; weights[t,k] = sigmoid(l_k) / sum_k' sigmoid(l_k')
 *                 (as mxfp4_moe_route_sigmoid_topk; routed_scale is ignored);
 *   score_mode 1: the reference router (kernel/cpp-engine-mxfp4/routed.cu:156-208,
 *                 runtime/dsv4_engine_mxfp4.py:363-370): scores
 *                 s = sqrt(softplus(l)), softplus(l) = max(l,0) + log1p(exp(-|l|));
 *                 rank the scores; weights[t,k] = (s_k / (sum_k' s_k' + 1e-20f))
 *                 * routed_scale, evaluated in double (sum in pick order) and
 *                 rounded to float as the reference's host code does (it keeps
 *                 fp32 weights, routed.cu:205; the Python engine rounds them to
 *                 bf16, dsv4_engine_mxfp4.py:369).
 * Ranking is descending, ties to the lower expert index; NaN ranks below every
 * number (the reference never picks NaN and aborts when fewer than topk
 * numbers exist; here NaN entries then fill the last picks). Replaces the
 * sqrt_softplus_kernel launch, the D2H copy, the stream sync and
 * topk6_norm_scale_host of routed.cu:156-208, 418-446. Returns 0; -1 bad
 * T/n_experts/topk/score_mode (as mxfp4_moe_route_sigmoid_topk); -10 logits,
 * ids or weights null; -5 launch failure. */
int mxfp4_moe_route_topk(const float* logits, int T, int n_experts, int topk, int score_mode,
                         float routed_scale, int32_t* ids, float* weights, hipStream_t stream);

/* EXTENSION: the router gate GEMV, logits[t, n] = sum_k W_gate[n, k] * x[t, k]
 * (bf16 operands, fp32 accumulate and output), x [T, K], W_gate [n_experts, K]
 * row-major, logits [T, n_experts]. Replaces router_gate_gemv_kernel,
 * reference kernel/cpp-engine-mxfp4/routed.cu:124-153 (launched at :401-410
 * and by dsv4_routed_compute_router_logits_isolated, :614-636). Returns 0; -1
 * T outside [1, 64], n_experts outside [1, 1024], K not a positive multiple of
 * 8 or K > 8192; -3 x or W_gate not 16-byte aligned; -5 launch failure. */
int mxfp4_moe_router_logits(const dsv4_bf16_t* x, const dsv4_bf16_t* W_gate, int T, int n_experts,
                            int K, float* logits, hipStream_t stream);

/* EXTENSION: workspace bytes for mxfp4_moe_grouped_gemv. */
size_t mxfp4_moe_workspace_bytes(int T, int topk, int n_experts, int hidden);

/* EXTENSION (reference runs T single-token calls after 36 D2D pack copies,
 * kernel/cpp-engine-mxfp4/routed.cu:266-283, runtime/dsv4_engine_mxfp4.py:412-423).
 * Expert-indexed multi-token routed SwiGLU MoE: experts are read in place from
 * per-layer tensors W1/W3 [n_experts, hidden, K_in/2], W2 [n_experts, out_dim,
 * hidden/2] (+ scales), each unique routed expert is streamed once for all of
 * its tokens; one launch per projection (stage A: W1+W3, stage B: W2).
 *   out[t] = bf16( sum_k weights[t,k] * W2_{ids[t,k]} . bf16(silu(W1 x_t) * (W3 x_t)) )
 * x [T, K_in] bf16, ids/weights [T, topk], out [T, out_dim] bf16.
 * Returns 0; -1 K_in%32; -2 hidden%32; -3 K_in/hidden > 4096; -4 bad
 * T/topk/n_experts (T<1 or >64, topk<1 or >16, n_experts<1 or >1024);
 * -5/-6/-7 launch failure of routing/stage A/stage B; -10 a required pointer
 * is null (checked after the shapes, before any launch; the entries below
 * that return "as mxfp4_moe_grouped_gemv" or "as mxfp4_moe_layer" do the
 * same, ids_out and weights_out being optional). An id outside
 * [0, n_experts) is skipped (contributes nothing). */
int mxfp4_moe_grouped_gemv(const dsv4_bf16_t* x,
                           const uint8_t* W1_packed, const uint8_t* W3_packed,
                           const uint8_t* W2_packed,
                           const uint8_t* W1_scale, const uint8_t* W3_scale,
                           const uint8_t* W2_scale,
                           const int32_t* ids, const float* weights,
                           int T, int topk, int n_experts,
                           int K_in, int hidden, int out_dim,
                           dsv4_bf16_t* out, void* workspace, hipStream_t stream);

/* EXTENSION, no counterpart in the reference: mxfp4_moe_grouped_gemv without a
 * workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The routing tables and the SwiGLU intermediate live in a 4 MiB
 * device array that the library holds on each GPU it runs on (of the current
 * device, hipGetDevice; `stream` must belong to it) until the process ends;
 * the call allocates nothing. Calls that overlap on one GPU (two streams, two
 * threads) share that array and race; calls in order on one stream are safe,
 * and nothing carries over from one call to the next. Same arguments, results
 * (the same bits) and return codes as mxfp4_moe_grouped_gemv, plus -8 when
 * mxfp4_moe_workspace_bytes(T, topk, n_experts, hidden) exceeds 4 MiB
 * (e.g. T*topk*hidden*2 above about 4.1 million bytes) and -9 when the device
 * array cannot be located. The first call on each device looks the array's
 * address up (hipGetSymbolAddress, a runtime query, no stream work): make that
 * first call outside graph capture; captured calls after it record only the
 * kernel launches. */
int mxfp4_moe_grouped_gemv_noalloc(const dsv4_bf16_t* x,
                                   const uint8_t* W1_packed, const uint8_t* W3_packed,
                                   const uint8_t* W2_packed,
                                   const uint8_t* W1_scale, const uint8_t* W3_scale,
                                   const uint8_t* W2_scale,
                                   const int32_t* ids, const float* weights,
                                   int T, int topk, int n_experts,
                                   int K_in, int hidden, int out_dim,
                                   dsv4_bf16_t* out, hipStream_t stream);

/* EXTENSION: the three launches of mxfp4_moe_grouped_gemv as separate entry
 * points (same arguments and workspace), for callers that schedule or overlap
 * the projections themselves and for per-launch timing:
 *   mxfp4_moe_build_routing: device routing tables from ids/weights (1 launch);
 *   mxfp4_moe_swiglu:        stage A, W1/W3 + SiLU -> bf16 intermediate in the
 *                            workspace (1 launch);
 *   mxfp4_moe_down:          stage B, W2 + weighted combine -> out (1 launch).
 * They must run in this order on one stream with one workspace sized by
 * mxfp4_moe_workspace_bytes(T, topk, n_experts, hidden). Return codes as
 * mxfp4_moe_grouped_gemv. */
int mxfp4_moe_build_routing(const int32_t* ids, const float* weights, int T, int topk,
                            int n_experts, int hidden, void* workspace, hipStream_t stream);
int mxfp4_moe_swiglu(const dsv4_bf16_t* x, const uint8_t* W1_packed, const uint8_t* W3_packed,
                     const uint8_t* W1_scale, const uint8_t* W3_scale, int T, int topk,
                     int n_experts, int K_in, int hidden, void* workspace, hipStream_t stream);
int mxfp4_moe_down(const uint8_t* W2_packed, const uint8_t* W2_scale, int T, int topk,
                   int n_experts, int hidden, int out_dim, dsv4_bf16_t* out, void* workspace,
                   hipStream_t stream);

/* EXTENSION: one routed-MoE layer at decode in one call (three launches on
 * `stream`): device gating of logits [T, n_experts] (top-`topk`, sigmoid
 * weights renormalised to 1, as mxfp4_moe_route_sigmoid_topk), then stages A
 * and B of mxfp4_moe_grouped_gemv. ids_out / weights_out ([T, topk]; either
 * or both may be NULL) receive the routing. Workspace as mxfp4_moe_grouped_gemv. Return codes
 * as mxfp4_moe_grouped_gemv (-4 also for topk > n_experts). */
int mxfp4_moe_layer(const dsv4_bf16_t* x, const float* logits,
                    const uint8_t* W1_packed, const uint8_t* W3_packed, const uint8_t* W2_packed,
                    const uint8_t* W1_scale, const uint8_t* W3_scale, const uint8_t* W2_scale,
                    int T, int topk, int n_experts, int K_in, int hidden, int out_dim,
                    dsv4_bf16_t* out, int32_t* ids_out, float* weights_out, void* workspace,
                    hipStream_t stream);

/* EXTENSION: the first part of mxfp4_moe_layer (gating of logits and stage A,
 * one launch for one token on the aligned path, two otherwise); followed by
 * mxfp4_moe_down with the same workspace it completes the layer with the same
 * bits. For callers that schedule the projections themselves and for
 * per-launch timing. Arguments and return codes as mxfp4_moe_layer. */
int mxfp4_moe_gate_swiglu(const dsv4_bf16_t* x, const float* logits, const uint8_t* W1_packed,
                          const uint8_t* W3_packed, const uint8_t* W1_scale, const uint8_t* W3_scale,
                          int T, int topk, int n_experts, int K_in, int hidden, int32_t* ids_out,
                          float* weights_out, void* workspace, hipStream_t stream);

/* EXTENSION: the reference's routed dispatch of one MoE layer on the device
 * (replaces dsv4_routed_dispatch, reference kernel/cpp-engine-mxfp4/routed.cu:373-503,
 * for T tokens): the router gate GEMV (mxfp4_moe_router_logits over x), the
 * reference's scoring (mxfp4_moe_route_topk score_mode 1 with routed_scale,
 * 1.5 in the reference) and stages A and B of mxfp4_moe_grouped_gemv, with the
 * experts read in place from the per-layer tensors. No host sync, no pack
 * copies; three launches for one token (the scoring runs inside stage A), four
 * otherwise. W_gate [n_experts, K_in] bf16; ids_out / weights_out as
 * mxfp4_moe_layer. Workspace of mxfp4_moe_dispatch_workspace_bytes bytes.
 * Returns as mxfp4_moe_layer, plus -3 for an unaligned x or W_gate and -4 for
 * T, n_experts or K_in outside the router's limits. */
size_t mxfp4_moe_dispatch_workspace_bytes(int T, int topk, int n_experts, int hidden);
int mxfp4_moe_routed_dispatch(const dsv4_bf16_t* x, const dsv4_bf16_t* W_gate,
                              const uint8_t* W1_packed, const uint8_t* W3_packed, const uint8_t* W2_packed,
                              const uint8_t* W1_scale, const uint8_t* W3_scale, const uint8_t* W2_scale,
                              int T, int topk, int n_experts, int K_in, int hidden, int out_dim,
                              float routed_scale, dsv4_bf16_t* out, int32_t* ids_out, float* weights_out,
                              void* workspace, hipStream_t stream);

/* EXTENSION (no reference counterpart; the reference has no prefill MoE path,
 * though the benchmark configuration asks for a 512-token prefill chunk): the
 * routed MoE layer for a chunk of many tokens on the
 * matrix cores. Same result as mxfp4_moe_grouped_gemv for every token:
 *   out[t] = bf16( sum_k weights[t,k] * W2_e . bf16(silu(W1_e x_t) * (W3_e x_t)) ), e = ids[t,k]
 * with the MXFP4 weights dequantised exactly to bf16 and multiplied on
 * v_mfma_f32_16x16x32_bf16 (fp32 accumulate). x [T, K_in] bf16 (16-byte
 * aligned), ids/weights [T, topk], out [T, out_dim] bf16. Ids outside
 * [0, n_experts) contribute nothing. Four launches, no allocation; workspace
 * of mxfp4_moe_prefill_workspace_bytes bytes (0 for invalid arguments).
 * Returns 0; -1 K_in not a multiple of 512 in [512, 8192]; -2 hidden likewise;
 * -3 out_dim not a positive multiple of 64, a null or unaligned operand; -4 T outside
 * [1, 16384], topk outside [1, 16] or n_experts outside [1, 1024]; -5..-8
 * launch failure of routing / stage A / stage B / combine. */
size_t mxfp4_moe_prefill_workspace_bytes(int T, int topk, int n_experts, int hidden, int out_dim);
int mxfp4_moe_prefill(const dsv4_bf16_t* x,
                      const uint8_t* W1_packed, const uint8_t* W3_packed, const uint8_t* W2_packed,
                      const uint8_t* W1_scale, const uint8_t* W3_scale, const uint8_t* W2_scale,
                      const int32_t* ids, const float* weights, int T, int topk, int n_experts,
                      int K_in, int hidden, int out_dim, dsv4_bf16_t* out, void* workspace,
                      hipStream_t stream);

/* EXTENSION (debug): out[n,k] = bf16( e2m1(W[n,k]) * 2^(S[n,k/32]-127) ) with
 * the decode of the prefill GEMMs (the conversion applies the block scale),
 * for the bit-exact check against runtime/mxfp4_loader.py:272-309 (byte 0 ->
 * 2^-127, 0xFF -> 0 as the decode path). W [N, K/2] and out [N, K] contiguous
 * and 16-byte aligned, S [N, K/32]. Returns 0; -1 K%32; -3 bad operand; -4
 * launch failure. */
int mxfp4_moe_prefill_dequant_bf16(const uint8_t* W_packed, const uint8_t* W_scale, int K, int N,
                                   dsv4_bf16_t* out, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* libmxfp4_gemv.so                                                          */
/* ------------------------------------------------------------------------ */

/* y[n] = bf16( sum_k dequant(W)[n,k] * x[k] ), W packed [N, K/2] with row
 * stride packed_row_stride_bytes, scales [N, K/32] with row stride
 * scale_row_stride_bytes. Returns 0; -1 K%32 or K < 32; -2 K > 8192; -3 launch
 * failure, also N < 1 (the reference's zero-size grid fails its launch).
 * Replaces mxfp4_gemv_m1, reference kernel/mxfp4-dense/mxfp4_gemv.cu:131-166. */
int mxfp4_gemv_m1(const dsv4_bf16_t* x, const uint8_t* W_packed, const uint8_t* W_scale,
                  int K, int N, int64_t packed_row_stride_bytes,
                  int64_t scale_row_stride_bytes, dsv4_bf16_t* y, hipStream_t stream);

/* EXTENSION (debug): out[n,k] = bf16( e2m1(W[n,k]) * 2^(S[n,k/32]-127) ), using
 * the same device decode routine as the GEMVs, so a bit-exact comparison with
 * the reference dequant (runtime/mxfp4_loader.py:272-309) checks the kernels'
 * decode. out is [N, K] contiguous. Returns 0; -1 K%32; -3 N < 1 or launch
 * failure; -10 W_packed, W_scale or out null. */
int mxfp4_dequant_bf16(const uint8_t* W_packed, const uint8_t* W_scale, int K, int N,
                       int64_t packed_row_stride_bytes, int64_t scale_row_stride_bytes,
                       dsv4_bf16_t* out, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* libfp8_e4m3_gemv.so                                                       */
/* ------------------------------------------------------------------------ */

/* y[n] = bf16( sum_k e4m3(W[n,k]) * 2^(S[n/128, k/128]-127) * x[k] ).
 * W [N, K] bytes (row stride weight_row_stride_bytes), S [ceil(N/128), K/128]
 * (row stride scale_row_stride_bytes). Returns 0; -1 K%128 or K < 128;
 * -3 K > 16384; -4 launch failure, also N < 1 (the reference's zero-size grid
 * fails its launch). N need not be a multiple of 128: the reference returns -2
 * there (kernel/fp8-dense/fp8_e4m3_gemv.cu:148-154); this build accepts it so
 * the 576-row projection runs, with ceil(N/128) scale rows.
 * Replaces fp8_e4m3_gemv_m1, reference kernel/fp8-dense/fp8_e4m3_gemv.cu:132-174. */
int fp8_e4m3_gemv_m1(const dsv4_bf16_t* x, const uint8_t* W_fp8, const uint8_t* W_scale,
                     int K, int N, int64_t weight_row_stride_bytes,
                     int64_t scale_row_stride_bytes, dsv4_bf16_t* y, hipStream_t stream);

/* EXTENSION (reference loops fp8_e4m3_gemv_m1 per token,
 * runtime/dsv4_engine_mxfp4.py:310-319): T-token FP8 GEMV that streams W once.
 * x [T, K] (row stride x_row_stride elements), y [T, N] (row stride
 * y_row_stride elements). With K in {1024, 2048, 4096, 8192} and 16-byte
 * aligned operands it runs on the matrix cores (bf16 MFMA on the exact E4M3
 * values) at K = 8192 from T = 2; at K = 1024 from T = 3 with N >= 2048 and
 * from T = 5 at any N; at K = 2048 from T = 3 with N >= 4096 and from T = 5
 * at any N; at K = 4096 from T = 3 with N >= 4096 and from T = 5 with
 * N > 512. Aligned rows longer than 4096 (K a multiple of 512, at most
 * 16384) take the matrix cores from T = 2. Both need the T activation rows to
 * span fewer than 2^31 bytes ((T - 1) * x_row_stride + K elements).
 * Otherwise it runs on the vector units; the two paths agree within fp32
 * rounding of the sums. Returns as fp8_e4m3_gemv_m1, plus -5 for T<1 or T>16
 * and -10 for a null x, W_fp8, W_scale or y (after the shape checks, before
 * any launch; the other FP8 extensions likewise for their operands). */
int fp8_e4m3_gemv(const dsv4_bf16_t* x, int64_t x_row_stride, const uint8_t* W_fp8,
                  const uint8_t* W_scale, int K, int N, int T,
                  int64_t weight_row_stride_bytes, int64_t scale_row_stride_bytes,
                  dsv4_bf16_t* y, int64_t y_row_stride, hipStream_t stream);

/* EXTENSION: fp8_e4m3_gemv with one fp32 scale per 128x128 tile, W_scale
 * float [ceil(N/128), K/128] with row stride scale_row_stride (in floats, at
 * least K/128), 4-byte aligned: the scale format of the benchmark's FP8
 * configuration, where the reference ABI (kernel/fp8-dense/fp8_e4m3_gemv.cu:
 * 132-142, runtime/fp8_e4m3_gemv_binding.py:88) carries E8M0 bytes and the
 * reference's dequantisation (runtime/dsv4_engine_mxfp4.py:531-553) multiplies
 * e4m3(W) by the tile's scale in fp32 before rounding to bf16. The scale
 * multiplies each 16-element partial dot or 128-k tile sum (fp32), so
 * results agree with that dequantise-then-multiply path within fp32/bf16
 * rounding. The kernels and the path rule are fp8_e4m3_gemv's (vector and
 * matrix-core paths), so power-of-two scales give its bits. Return codes as
 * fp8_e4m3_gemv, plus -6 for a misaligned scale pointer or a scale row stride
 * below K/128. */
int fp8_e4m3_gemv_f32s(const dsv4_bf16_t* x, int64_t x_row_stride, const uint8_t* W_fp8,
                       const float* W_scale, int K, int N, int T, int64_t weight_row_stride_bytes,
                       int64_t scale_row_stride, dsv4_bf16_t* y, int64_t y_row_stride,
                       hipStream_t stream);

/* EXTENSION (replaces the per-group loop of 8 fp8_e4m3_gemv_m1 calls for the
 * grouped output projection wo_a, reference
 * kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:484-499, and the einsum
 * of runtime/dsv4_engine_mxfp4.py:515-528): G GEMVs in one launch.
 *   y[t, g, n] = bf16( sum_k W[g*N + n, k] x[t, g, k] ),  g < G, n < N, t < T
 * with W [G*N, K] (scale rows (g*N+n)/128), x element (t, g, k) at
 * x + t*x_row_stride + g*x_group_stride + k, y element (t, g, n) at
 * y + t*y_row_stride + g*y_group_stride + n. The path rule of fp8_e4m3_gemv
 * applies to the rows of all groups (G*N), so a group has the bits of
 * fp8_e4m3_gemv on its slice whenever that call takes the same path (always at
 * T = 1; within fp32 rounding of the sums otherwise). Returns as
 * fp8_e4m3_gemv, plus -6 for G < 1 or G > 65535. */
int fp8_e4m3_gemv_grouped(const dsv4_bf16_t* x, int64_t x_row_stride, int64_t x_group_stride,
                          const uint8_t* W_fp8, const uint8_t* W_scale, int G, int K, int N, int T,
                          int64_t weight_row_stride_bytes, int64_t scale_row_stride_bytes,
                          dsv4_bf16_t* y, int64_t y_row_stride, int64_t y_group_stride,
                          hipStream_t stream);

/* EXTENSION (replaces consecutive fp8_e4m3_gemv_m1 calls on one activation,
 * e.g. wq_a and wkv on the normalised row, reference
 * kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:395-418): n_mats GEMVs
 * that share x, K and T in one launch,
 *   y_m[t, n] = bf16( sum_k W_m[n, k] x[t, k] ),  n < N[m], m < n_mats,
 * with the bits fp8_e4m3_gemv writes for each matrix alone (the launch takes
 * the matrix cores only when every matrix would alone; a matrix that would
 * take them alone while another would not agrees within rounding). The per-matrix
 * arguments are host arrays of n_mats entries (pointers are device pointers):
 * W_fp8[m] [N[m], K] (row stride weight_row_stride_bytes[m]), W_scale[m]
 * [ceil(N[m]/128), K/128] (scale_row_stride_bytes[m]), y[m] [T, N[m]] (row
 * stride y_row_stride[m] elements); x [T, K] with row stride x_row_stride.
 * K in {1024, 2048, 4096, 8192} with 16-byte aligned x, weights and rows runs
 * as one launch; other shapes run one launch per matrix. Returns as
 * fp8_e4m3_gemv, plus -6 for n_mats outside [1, 8] or a null table. */
int fp8_e4m3_gemv_multi(const dsv4_bf16_t* x, int64_t x_row_stride, int K, int T, int n_mats,
                        const uint8_t* const* W_fp8, const uint8_t* const* W_scale, const int* N,
                        const int64_t* weight_row_stride_bytes, const int64_t* scale_row_stride_bytes,
                        dsv4_bf16_t* const* y, const int64_t* y_row_stride, hipStream_t stream);

/* EXTENSION (replaces the gate GEMV, the up GEMV and the SwiGLU launch of the
 * shared expert, reference kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:
 * 508-548 and runtime/dsv4_engine_mxfp4.py:399-410): one launch for
 *   act[t, n] = bf16( silu(c(g)) * c_up(u) ),  silu(v) = v / (1 + expf(-v)),
 * g = bf16(W1 x_t)[n] and u = bf16(W3 x_t)[n] (each exactly the bits
 * fp8_e4m3_gemv writes), c a clamp to [-limit, limit] (no clamp for
 * limit <= 0), c_up the same clamp if clamp_up != 0 (runtime/dsv4_engine_mxfp4.py:
 * 405-407 clamps both) else none (dsv4_engine_mxfp4_wire.cu:517-518 clamps the
 * gate only). W1, W3 share K, N and row strides. Needs K in {1024, 2048, 4096,
 * 8192} and 16-byte aligned x, W1, W3 and rows (-6 otherwise); T in [1, 16] (-5).
 * Returns as fp8_e4m3_gemv otherwise. */
int fp8_e4m3_swiglu_gemv(const dsv4_bf16_t* x, int64_t x_row_stride, const uint8_t* W1_fp8,
                         const uint8_t* W1_scale, const uint8_t* W3_fp8, const uint8_t* W3_scale,
                         int K, int N, int T, int64_t weight_row_stride_bytes,
                         int64_t scale_row_stride_bytes, float limit, int clamp_up,
                         dsv4_bf16_t* act, int64_t act_row_stride, hipStream_t stream);

/* EXTENSION (folds the RMSNorm launch into the GEMV that consumes it; the
 * reference runs rmsnorm then FP8 GEMVs as separate launches,
 * kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:395-418 and
 * kernel/rmsnorm-fuse/rmsnorm_fuse.cu:110-157): one launch for
 *   v = x + residual (fp32; v = x when residual is NULL)
 *   new_residual = bf16(v)                                  (with a residual)
 *   x_norm = bf16( (norm_weight * bf16(v)) * rsqrt(sum(v^2)/K + eps) )
 *   y = bf16( W . x_norm )                                   (as fp8_e4m3_gemv)
 * for T token rows; x, residual, x_norm, new_residual are [T, K] contiguous,
 * y [T, N] contiguous. x_norm and new_residual have the bits of
 * rmsnorm_fuse_fwd / rmsnorm_fuse_residual_add, y those of fp8_e4m3_gemv on
 * x_norm. Needs K in {2048, 4096}, T in [1, 4] (-5), 16-byte aligned
 * operands and x_norm (and new_residual with a residual) (-6). Returns as
 * fp8_e4m3_gemv otherwise. */
int fp8_e4m3_rmsnorm_gemv(const dsv4_bf16_t* x, const dsv4_bf16_t* residual,
                          const dsv4_bf16_t* norm_weight, float eps, const uint8_t* W_fp8,
                          const uint8_t* W_scale, int K, int N, int T,
                          int64_t weight_row_stride_bytes, int64_t scale_row_stride_bytes,
                          dsv4_bf16_t* y, dsv4_bf16_t* x_norm, dsv4_bf16_t* new_residual,
                          hipStream_t stream);

/* EXTENSION (debug): out[n,k] = bf16( e4m3(W[n,k]) * 2^(S[n/128,k/128]-127) ),
 * the device decode of the FP8 GEMVs, for the bit-exact check against
 * runtime/dsv4_engine_mxfp4.py:531-553. Returns 0; -1 K%128; -4 N < 1 or
 * launch failure; -10 W_fp8, W_scale or out null. */
int fp8_e4m3_dequant_bf16(const uint8_t* W_fp8, const uint8_t* W_scale, int K, int N,
                          int64_t weight_row_stride_bytes, int64_t scale_row_stride_bytes,
                          dsv4_bf16_t* out, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* librmsnorm_fuse.so                                                        */
/* ------------------------------------------------------------------------ */

/* y[r,h] = bf16( w[h] * x[r,h] * rsqrt(mean_h(x[r,:]^2) + eps) ), bf16 in/out.
 * Returns 0 (also for n_rows <= 0 or hidden <= 0: no-op); 1 hidden > 8192;
 * otherwise a hipError_t from the launch.
 * Replaces rmsnorm_fuse_fwd, reference kernel/rmsnorm-fuse/rmsnorm_fuse.cu:161-182. */
int rmsnorm_fuse_fwd(const void* x, const void* weight, void* y, int n_rows, int hidden,
                     float eps, hipStream_t stream);

/* t = x + residual (fp32); new_residual = bf16(t);
 * y_norm = bf16( w * bf16(t) * rsqrt(sum(t^2)/hidden + eps) ). Return codes as
 * rmsnorm_fuse_fwd.
 * Replaces rmsnorm_fuse_residual_add, reference rmsnorm_fuse.cu:184-209. */
int rmsnorm_fuse_residual_add(const void* x, const void* residual, const void* weight,
                              void* y_norm, void* new_residual, int n_rows, int hidden,
                              float eps, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_KERNELS_H */
