/*
 * mx_oracle.c — scalar C restatement of the decode hot path, fp64 accumulate.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through oracle/c_oracle.py) and
 * by bench.py's cpu_baseline leg; never part of the product path.
 *
 * Written independently of oracle/mx.py (no shared code): number formats are
 * decoded from their bit fields with ldexp, the GEMVs are plain loops that
 * accumulate in double over bf16-rounded dequantised weights. It serves as
 * the brute-force comparator for the vectorised numpy oracle and the GPU.
 * Reference semantics restated:
 *   e2m1 codebook        runtime/mxfp4_unpack.py:36-39
 *   nibble order         runtime/mxfp4_unpack.py:105-112
 *   E8M0 (0xFF -> 0)     kernel/mxfp4-dense/mxfp4_gemv.cu:65-69
 *   MXFP4 dequant        runtime/mxfp4_loader.py:272-309
 *   FP8 dequant          runtime/dsv4_engine_mxfp4.py:531-553
 *   routed SwiGLU        kernel/mxfp4-routed/mxfp4_grouped_gemv.cu:143-289
 *   fused RMSNorm        kernel/rmsnorm-fuse/rmsnorm_fuse.cu:110-157
 *   router GEMV + scores kernel/cpp-engine-mxfp4/routed.cu:124-208
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

uint16_t mxo_bf16_rne(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

float mxo_bf16_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

double mxo_e2m1(int code) {
    int s = (code >> 3) & 1, e = (code >> 1) & 3, m = code & 1;
    double mag = (e == 0) ? 0.5 * m : ldexp(1.0 + 0.5 * m, e - 1);
    return s ? -mag : mag;
}

float mxo_e8m0(uint8_t b) {
    if (b == 0xFF) return 0.0f;
    return (float)ldexp(1.0, (int)b - 127);
}

float mxo_e4m3fn(uint8_t b) {
    int s = (b >> 7) & 1, e = (b >> 3) & 15, m = b & 7;
    double mag;
    if (e == 15 && m == 7) return NAN;
    mag = (e == 0) ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
    return (float)(s ? -mag : mag);
}

/* out[n*K + k] = bf16( e2m1 * 2^(s-127) ), K % 32 == 0 */
void mxo_mxfp4_dequant(const uint8_t* packed, const uint8_t* scale, int N, int K, uint16_t* out) {
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            uint8_t byte = packed[(size_t)n * (K / 2) + k / 2];
            int code = (k & 1) ? (byte >> 4) : (byte & 15);
            float v = (float)mxo_e2m1(code) * mxo_e8m0(scale[(size_t)n * (K / 32) + k / 32]);
            out[(size_t)n * K + k] = mxo_bf16_rne(v);
        }
}

/* out[n*K + k] = bf16( e4m3 * 2^(S[n/128, k/128]-127) ), K % 128 == 0 */
void mxo_fp8_dequant(const uint8_t* w, const uint8_t* s, int N, int K, uint16_t* out) {
    int kt = K / 128;
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            float v = mxo_e4m3fn(w[(size_t)n * K + k]) * mxo_e8m0(s[(size_t)(n / 128) * kt + k / 128]);
            out[(size_t)n * K + k] = mxo_bf16_rne(v);
        }
}

/* y[t*N + n] = bf16( sum_k W_bf16[n,k] * x[t*K + k] ) with W given as bf16 bits */
static void gemv_bf16w(const uint16_t* x, int T, const uint16_t* W, int N, int K, float* yf) {
    for (int t = 0; t < T; ++t)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            const uint16_t* row = W + (size_t)n * K;
            const uint16_t* xt = x + (size_t)t * K;
            for (int k = 0; k < K; ++k) acc += (double)mxo_bf16_f32(row[k]) * mxo_bf16_f32(xt[k]);
            yf[(size_t)t * N + n] = (float)acc;
        }
}

void mxo_mxfp4_gemv(const uint16_t* x, int T, const uint8_t* packed, const uint8_t* scale, int N,
                    int K, uint16_t* y) {
    uint16_t* W = (uint16_t*)malloc((size_t)N * K * 2);
    float* yf = (float*)malloc((size_t)T * N * 4);
    mxo_mxfp4_dequant(packed, scale, N, K, W);
    gemv_bf16w(x, T, W, N, K, yf);
    for (size_t i = 0; i < (size_t)T * N; ++i) y[i] = mxo_bf16_rne(yf[i]);
    free(W);
    free(yf);
}

void mxo_fp8_gemv(const uint16_t* x, int T, const uint8_t* w, const uint8_t* s, int N, int K,
                  uint16_t* y) {
    uint16_t* W = (uint16_t*)malloc((size_t)N * K * 2);
    float* yf = (float*)malloc((size_t)T * N * 4);
    mxo_fp8_dequant(w, s, N, K, W);
    gemv_bf16w(x, T, W, N, K, yf);
    for (size_t i = 0; i < (size_t)T * N; ++i) y[i] = mxo_bf16_rne(yf[i]);
    free(W);
    free(yf);
}

/* Routed SwiGLU for one token over n_exp packed experts (expert-major
 * contiguous tensors), intermediate rounded to bf16, experts summed in order. */
void mxo_grouped_gemv(const uint16_t* x, const uint8_t* W1p, const uint8_t* W3p,
                      const uint8_t* W2p, const uint8_t* W1s, const uint8_t* W3s,
                      const uint8_t* W2s, const float* r, int K, int H, int O, int n_exp,
                      uint16_t* out) {
    uint16_t* Wa = (uint16_t*)malloc((size_t)H * K * 2);
    uint16_t* Wb = (uint16_t*)malloc((size_t)H * K * 2);
    uint16_t* W2 = (uint16_t*)malloc((size_t)O * H * 2);
    float* g = (float*)malloc((size_t)H * 4);
    float* u = (float*)malloc((size_t)H * 4);
    uint16_t* M = (uint16_t*)malloc((size_t)H * 2);
    float* y = (float*)malloc((size_t)O * 4);
    double* acc = (double*)calloc((size_t)O, sizeof(double));
    for (int e = 0; e < n_exp; ++e) {
        mxo_mxfp4_dequant(W1p + (size_t)e * H * (K / 2), W1s + (size_t)e * H * (K / 32), H, K, Wa);
        mxo_mxfp4_dequant(W3p + (size_t)e * H * (K / 2), W3s + (size_t)e * H * (K / 32), H, K, Wb);
        mxo_mxfp4_dequant(W2p + (size_t)e * O * (H / 2), W2s + (size_t)e * O * (H / 32), O, H, W2);
        gemv_bf16w(x, 1, Wa, H, K, g);
        gemv_bf16w(x, 1, Wb, H, K, u);
        for (int h = 0; h < H; ++h) {
            double gv = g[h];
            double sil = gv / (1.0 + exp(-gv));
            M[h] = mxo_bf16_rne((float)(sil * (double)u[h]));
        }
        gemv_bf16w(M, 1, W2, O, H, y);
        for (int o = 0; o < O; ++o) acc[o] += (double)r[e] * (double)y[o];
    }
    for (int o = 0; o < O; ++o) out[o] = mxo_bf16_rne((float)acc[o]);
    free(Wa); free(Wb); free(W2); free(g); free(u); free(M); free(y); free(acc);
}

/* t = x + r; new_res = bf16(t); y = bf16((w * bf16(t)) / sqrt(sum t^2 / H + eps)) */
void mxo_rmsnorm_residual(const uint16_t* x, const uint16_t* r, const uint16_t* w, int rows, int H,
                          float eps, uint16_t* y, uint16_t* new_res) {
    for (int i = 0; i < rows; ++i) {
        double ss = 0.0;
        for (int h = 0; h < H; ++h) {
            float t = mxo_bf16_f32(x[(size_t)i * H + h]) + mxo_bf16_f32(r[(size_t)i * H + h]);
            ss += (double)t * t;
            new_res[(size_t)i * H + h] = mxo_bf16_rne(t);
        }
        double rms = 1.0 / sqrt(ss / H + eps);
        for (int h = 0; h < H; ++h) {
            double v = (double)mxo_bf16_f32(w[h]) * mxo_bf16_f32(new_res[(size_t)i * H + h]);
            y[(size_t)i * H + h] = mxo_bf16_rne((float)(v * rms));
        }
    }
}

void mxo_rmsnorm(const uint16_t* x, const uint16_t* w, int rows, int H, float eps, uint16_t* y) {
    for (int i = 0; i < rows; ++i) {
        double ss = 0.0;
        for (int h = 0; h < H; ++h) {
            double v = mxo_bf16_f32(x[(size_t)i * H + h]);
            ss += v * v;
        }
        double rms = 1.0 / sqrt(ss / H + eps);
        for (int h = 0; h < H; ++h) {
            double v = (double)mxo_bf16_f32(w[h]) * mxo_bf16_f32(x[(size_t)i * H + h]);
            y[(size_t)i * H + h] = mxo_bf16_rne((float)(v * rms));
        }
    }
}

/* Router gate logits in fp64: logits[t, n] = sum_k W[n, k] x[t, k] (bf16
 * operands), rounded once to float. */
void mxo_router_logits(const uint16_t* x, int T, const uint16_t* W, int N, int K, float* logits) {
    for (int t = 0; t < T; ++t)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k)
                acc += (double)mxo_bf16_f32(W[(size_t)n * K + k]) * (double)mxo_bf16_f32(x[(size_t)t * K + k]);
            logits[(size_t)t * N + n] = (float)acc;
        }
}

/* The reference router's selection for one row of n logits: scores
 * s = sqrtf(max(l, 0) + log1pf(expf(-|l|))); `topk` selection passes, each
 * taking the first strictly larger untaken score (so ties go to the lower
 * index and NaN is never taken while a number is left; with none left the
 * pass takes the lowest untaken index); weights (s / (sum + 1e-20f)) * scale
 * in double, sum in pick order. Returns the number of passes that found a
 * number. */
int mxo_route_sqrt_softplus(const float* logits, int n, int topk, float scale, int* ids, float* w) {
    float* s = (float*)malloc((size_t)n * sizeof(float));
    char* taken = (char*)calloc((size_t)n, 1);
    for (int i = 0; i < n; ++i) {
        float l = logits[i];
        float sp = fmaxf(l, 0.0f) + log1pf(expf(-fabsf(l)));
        s[i] = sqrtf(sp);
    }
    int found = 0;
    for (int k = 0; k < topk; ++k) {
        int best = -1;
        float bv = -INFINITY;
        for (int i = 0; i < n; ++i)
            if (!taken[i] && s[i] > bv) { bv = s[i]; best = i; }
        if (best >= 0) ++found;
        else
            for (int i = 0; i < n && best < 0; ++i)
                if (!taken[i]) best = i;
        ids[k] = best;
        taken[best] = 1;
    }
    double sum = 0.0;
    for (int k = 0; k < topk; ++k) sum += (double)s[ids[k]];
    double denom = sum + (double)1e-20f;
    for (int k = 0; k < topk; ++k) w[k] = (float)(((double)s[ids[k]] / denom) * (double)scale);
    free(s);
    free(taken);
    return found;
}
