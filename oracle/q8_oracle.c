/*
 * q8_oracle.c -- CPU restatement of web-xpu-ops' matvecQ8 / quantize / packQ8.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or
 * shipped).  Build: oracle/Makefile, compiled with -O2 -ffp-contract=off so
 * that no multiply-add is fused: the reference's arithmetic is separate f64
 * multiplies and adds.
 *
 * The reference is TypeScript; its numbers are IEEE-754 binary64 and its
 * typed-array stores define the narrowing:
 *   Float32Array[i] = v   -> round-to-nearest-even binary32   (C: (float)v)
 *   Int32Array[i]   = v   -> ToInt32(v); NaN -> 0, -0 -> 0     (to_int32 below)
 *   Uint32Array[i]  = v   -> ToUint32(v)
 */
#define _DEFAULT_SOURCE /* sysconf */
#include "q8_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <unistd.h>

/* Math.max / Math.min: NaN if either operand is NaN (ECMAScript 21.3.2.24/25). */
static double js_max(double a, double b) {
    if (isnan(a) || isnan(b)) return NAN;
    if (a == 0.0 && b == 0.0) return signbit(a) ? b : a; /* +0 beats -0 */
    return a > b ? a : b;
}

static double js_min(double a, double b) {
    if (isnan(a) || isnan(b)) return NAN;
    if (a == 0.0 && b == 0.0) return signbit(a) ? a : b; /* -0 beats +0 */
    return a < b ? a : b;
}

/* Math.round (ECMAScript 21.3.2.28): the integral Number closest to v, ties
 * toward +Infinity.  floor(v) + (v - floor(v) >= 0.5) has no second rounding:
 * v - floor(v) is exact wherever the comparison can go either way (the band
 * the reference's numpy twin documents at llm/tools/quant_common.py:11-22).
 * v + 0.5 would round 0.49999999999999994 up to 1. */
double q8o_js_round(double v) {
    if (isnan(v) || isinf(v)) return v;
    double f = floor(v);
    return (v - f >= 0.5) ? f + 1.0 : f;
}

/* ToInt32 for the values quantize can produce: an integral double in
 * [-127, 127] or NaN. */
static int32_t to_int32(double v) {
    if (isnan(v) || isinf(v)) return 0;
    return (int32_t)v;
}

/* ops/quantize/reference.ts:13-38.  Per row: absmax in f64 over |x| with NaN
 * propagating through Math.max (:27); scale = absmax === 0 ? 1 : absmax/127
 * stored to Float32Array (:29); inverse = absmax === 0 ? 0 : 127/absmax in f64
 * (:30); code = clamp(Math.round(x * inverse), -127, 127) stored to
 * Int32Array (:33-34). */
void q8o_quantize(const float* input, size_t N, size_t D, int32_t* output, float* scales) {
    for (size_t row = 0; row < N; ++row) {
        const float* x = input + row * D;
        double absmax = 0.0;
        for (size_t col = 0; col < D; ++col) absmax = js_max(absmax, fabs((double)x[col]));
        scales[row] = absmax == 0.0 ? 1.0f : (float)(absmax / 127.0);
        const double inverse = absmax == 0.0 ? 0.0 : 127.0 / absmax;
        for (size_t col = 0; col < D; ++col) {
            const double value = q8o_js_round((double)x[col] * inverse);
            output[row * D + col] = to_int32(js_max(-127.0, js_min(127.0, value)));
        }
    }
}

/* ops/matvec/reference.ts:267-283.  wordsPerRow = ceil(K/4); lane `l` of
 * word `w` carries (codes[row*K + 4w + l] & 0xff) << 8l; lanes past K stay 0
 * (the `break` at :274); the word is stored through `>>> 0`. */
void q8o_pack_q8(const int32_t* codes, size_t N, size_t K, uint32_t* packed) {
    const size_t W = (K + 3) / 4;
    for (size_t row = 0; row < N; ++row) {
        for (size_t word = 0; word < W; ++word) {
            uint32_t bits = 0;
            for (size_t lane = 0; lane < 4; ++lane) {
                const size_t col = word * 4 + lane;
                if (col >= K) break;
                bits |= ((uint32_t)codes[row * K + col] & 0xffu) << (8 * lane);
            }
            packed[row * W + word] = bits;
        }
    }
}

/* llm/weights-q8.ts:137-139: packQ8 applied to an Int8Array; `& 0xff` of an
 * Int8Array element reads the same two's-complement byte. */
void q8o_pack_int8_rows(const int8_t* codes, size_t N, size_t K, uint32_t* packed) {
    const size_t W = (K + 3) / 4;
    for (size_t row = 0; row < N; ++row) {
        for (size_t word = 0; word < W; ++word) {
            uint32_t bits = 0;
            for (size_t lane = 0; lane < 4; ++lane) {
                const size_t col = word * 4 + lane;
                if (col >= K) break;
                bits |= ((uint32_t)(uint8_t)codes[row * K + col]) << (8 * lane);
            }
            packed[row * W + word] = bits;
        }
    }
}

/* The output rows of the matvec and matmul oracles are independent, so they
 * are split over threads; every output element is still one f64 sum over k
 * in ascending order, the same operations as one loop per element, so the
 * results do not depend on the thread count.  Threads: OMP_NUM_THREADS when
 * set, else the online CPUs, at most 16; small problems run on the caller's
 * thread. */
typedef void (*rows_fn)(size_t r0, size_t r1, void* ctx);
struct rows_task {
    rows_fn fn;
    void* ctx;
    size_t r0, r1;
};

static void* rows_thread(void* p) {
    struct rows_task* t = (struct rows_task*)p;
    t->fn(t->r0, t->r1, t->ctx);
    return NULL;
}

static void parallel_rows(size_t rows, size_t work, rows_fn fn, void* ctx) {
    long threads = 1;
    const char* env = getenv("OMP_NUM_THREADS");
    if (env && atol(env) > 0) threads = atol(env);
    else threads = sysconf(_SC_NPROCESSORS_ONLN);
    if (threads > 16) threads = 16;
    if (threads < 1 || work < ((size_t)1 << 24)) threads = 1;
    if ((size_t)threads > rows) threads = (long)rows;
    if (threads <= 1) {
        fn(0, rows, ctx);
        return;
    }
    pthread_t tid[16];
    struct rows_task task[16];
    int created[16] = {0};
    for (long i = 0; i < threads; ++i)
        task[i] = (struct rows_task){fn, ctx, rows * (size_t)i / (size_t)threads, rows * (size_t)(i + 1) / (size_t)threads};
    for (long i = 1; i < threads; ++i) created[i] = pthread_create(&tid[i], NULL, rows_thread, &task[i]) == 0;
    fn(task[0].r0, task[0].r1, ctx);
    for (long i = 1; i < threads; ++i) {
        if (created[i]) pthread_join(tid[i], NULL);
        else fn(task[i].r0, task[i].r1, ctx);  /* no thread: these rows run here */
    }
}

/* ops/matvec/reference.ts:113-115 (unpackI8: byte >= 128 ? byte - 256 : byte). */
static int unpack_i8(uint32_t byte) { return byte >= 128 ? (int)byte - 256 : (int)byte; }

struct matvec_job {
    const uint32_t* weight;
    const float* scale;
    const float* vector;
    size_t K;
    float* output;  /* matvecQ8, or */
    double* bound;  /* sum_k |s q x| */
};

/* ops/matvec/reference.ts:117-131.  Sum left to right in f64 over col < K only
 * (pad lanes are never read), then one f64 multiply by the row's scale and
 * one rounding to f32. */
static void matvec_rows(size_t r0, size_t r1, void* ctx) {
    const struct matvec_job* j = (const struct matvec_job*)ctx;
    const size_t K = j->K, W = (K + 3) / 4;
    for (size_t row = r0; row < r1; ++row) {
        const size_t rowOffset = row * W;
        double sum = 0.0;
        for (size_t col = 0; col < K; ++col) {
            const uint32_t word = j->weight[rowOffset + (col >> 2)];
            const uint32_t byte = (word >> ((col & 3) * 8)) & 0xffu;
            const double t = (double)unpack_i8(byte) * (double)j->vector[col];
            sum += j->output ? t : fabs(t);
        }
        if (j->output) j->output[row] = (float)(sum * (double)j->scale[row]);
        else j->bound[row] = sum * fabs((double)j->scale[row]);
    }
}

void q8o_matvec_q8(const uint32_t* weight, const float* scale, const float* vector,
                   size_t N, size_t K, float* output) {
    struct matvec_job job = {weight, scale, vector, K, output, NULL};
    parallel_rows(N, N * K, matvec_rows, &job);
}

/* M independent matvecQ8 calls: vectors [M, K], output [M, N]. */
void q8o_matvec_q8_batched(const uint32_t* weight, const float* scale, const float* vectors,
                           size_t N, size_t K, size_t M, float* output) {
    for (size_t m = 0; m < M; ++m)
        q8o_matvec_q8(weight, scale, vectors + m * K, N, K, output + m * N);
}

/* Per-row magnitude sum_k |s_n * q_nk * x_k| in f64: the scale of the f32
 * rounding error any summation order can make, used as the tolerance base
 * |y - y_ref| <= 1e-5 * bound + 1e-7. */
void q8o_matvec_q8_absterm(const uint32_t* weight, const float* scale, const float* vector,
                           size_t N, size_t K, double* bound) {
    struct matvec_job job = {weight, scale, vector, K, NULL, bound};
    parallel_rows(N, N * K, matvec_rows, &job);
}

/* ops/matvec/reference.ts:235-243 (matvecQ8Residual): projected = matvecQ8 row
 * (a Float32Array value), then residual[row] + projected[row] in f64, stored
 * to a Float32Array. */
void q8o_matvec_q8_residual(const uint32_t* weight, const float* scale, const float* vector,
                            const float* residual, size_t N, size_t K, float* output) {
    q8o_matvec_q8(weight, scale, vector, N, K, output);
    for (size_t row = 0; row < N; ++row)
        output[row] = (float)((double)residual[row] + (double)output[row]);
}

/* ops/activation/reference.ts:91-92: silu(x) = x / (1 + Math.exp(-x)) in f64,
 * stored to a Float32Array. */
float q8o_silu(float x) {
    const double xd = (double)x;
    return (float)(xd / (1.0 + exp(-xd)));
}

/* ops/matvec/reference.ts:196-207 (matvecQ8Ffn): gate and up are matvecQ8 rows
 * (Float32Array values), gated = silu(gate) (Float32Array), then
 * gated[row] * up[row] in f64 stored to a Float32Array. */
void q8o_matvec_q8_ffn(const uint32_t* weight_gate, const float* scale_gate, const uint32_t* weight_up,
                       const float* scale_up, const float* vector, size_t N, size_t K, float* output) {
    float* up = (float*)malloc((N ? N : 1) * sizeof(float));
    q8o_matvec_q8(weight_gate, scale_gate, vector, N, K, output);
    q8o_matvec_q8(weight_up, scale_up, vector, N, K, up);
    for (size_t row = 0; row < N; ++row)
        output[row] = (float)((double)q8o_silu(output[row]) * (double)up[row]);
    free(up);
}

/* The f32 that a Float32Array store of unpackI8(byte) * s holds: the product
 * of an int8 and an f32 is exact in f64, so this is one rounding to f32. */
static float dequant_term(uint32_t word, size_t lane, float s) {
    const uint32_t byte = (word >> (lane * 8)) & 0xffu;
    return (float)((double)unpack_i8(byte) * (double)s);
}

/* b[row * K + k]: the dequantized terms of weight row `row`, in k order. */
static float* dequant_rows(const uint32_t* weight, const float* scale, size_t M, size_t K) {
    const size_t W = (K + 3) / 4;
    float* b = (float*)malloc((K * M != 0 ? K * M : 1) * sizeof(float));
    for (size_t row = 0; row < M; ++row)
        for (size_t k = 0; k < K; ++k) b[row * K + k] = dequant_term(weight[row * W + (k >> 2)], k & 3, scale[row]);
    return b;
}

struct matmul_job {
    const float* a;
    const float* b;
    size_t N, M, K;
    float* output;  /* the matmul, or */
    double* bound;  /* sum_k |a * b| */
};

/* Columns c0 .. c0 + NC - 1 of one output row: NC independent sums, each
 * over k in ascending order.  ABS sums |a * b| instead (the error bound). */
#define MATMUL_COLUMNS(NAME, NC, ABS)                                                     \
    static void NAME(const float* ar, const float* b, size_t c0, size_t nc, size_t K,     \
                     double* out) {                                                       \
        double sum[NC];                                                                   \
        for (size_t c = 0; c < (NC); ++c) sum[c] = 0.0;                                   \
        for (size_t k = 0; k < K; ++k) {                                                  \
            const double x = (double)ar[k];                                               \
            for (size_t c = 0; c < (NC); ++c) {                                           \
                const double t = x * (double)b[(c0 + (c < nc ? c : 0)) * K + k];          \
                sum[c] += (ABS) ? fabs(t) : t;                                            \
            }                                                                             \
        }                                                                                 \
        for (size_t c = 0; c < nc; ++c) out[c] = sum[c];                                  \
    }
MATMUL_COLUMNS(columns8, 8, 0)
MATMUL_COLUMNS(columns8_abs, 8, 1)

static void matmul_rows(size_t r0, size_t r1, void* ctx) {
    const struct matmul_job* j = (const struct matmul_job*)ctx;
    const size_t M = j->M, K = j->K;
    double s[8];
    for (size_t row = r0; row < r1; ++row) {
        for (size_t c0 = 0; c0 < M; c0 += 8) {
            const size_t nc = M - c0 < 8 ? M - c0 : 8;
            if (j->output) {
                columns8(j->a + row * K, j->b, c0, nc, K, s);
                for (size_t c = 0; c < nc; ++c) j->output[row * M + c0 + c] = (float)s[c];
            } else {
                columns8_abs(j->a + row * K, j->b, c0, nc, K, s);
                for (size_t c = 0; c < nc; ++c) j->bound[row * M + c0 + c] = s[c];
            }
        }
    }
}

/* ops/matmul/reference.ts:124-137 (matmulQ8): b[k * M + row] =
 * Float32Array(unpackI8(byte) * scale[row]) for the weight's M rows, then
 * matmul({a, b, M: N, N: M, K}) (:37-49): for each output element, an f64
 * sum over k left to right of a[row * K + k] * b[k * M + col], stored to a
 * Float32Array.  output is [N, M]. */
void q8o_matmul_q8(const float* a, const uint32_t* weight, const float* scale, size_t N, size_t M, size_t K,
                   float* output) {
    float* b = dequant_rows(weight, scale, M, K);
    struct matmul_job job = {a, b, N, M, K, output, NULL};
    parallel_rows(N, (size_t)N * M * K, matmul_rows, &job);
    free(b);
}

/* sum_k |a[n, k] * b[k, m]| in f64 with b the dequantized term above: the
 * magnitude the f32 kernel's rounding error is measured against. */
void q8o_matmul_q8_absterm(const float* a, const uint32_t* weight, const float* scale, size_t N, size_t M,
                           size_t K, double* bound) {
    float* b = dequant_rows(weight, scale, M, K);
    struct matmul_job job = {a, b, N, M, K, NULL, bound};
    parallel_rows(N, (size_t)N * M * K, matmul_rows, &job);
    free(b);
}

void q8o_dequantize_packed_q8(const uint32_t* weight, const float* scale, size_t N, size_t K, float* output) {
    const size_t W = (K + 3) / 4;
    for (size_t row = 0; row < N; ++row)
        for (size_t col = 0; col < K; ++col)
            output[row * K + col] = dequant_term(weight[row * W + (col >> 2)], col & 3, scale[row]);
}

/* ops/dequant_transpose/reference.ts:40-59 (dequantTranspose): output
 * [inFeatures, outFeatures], output[col * outFeatures + row] = unpackI8 * s.
 * (The reference's length checks at :42-47 are the C ABI's validation.) */
void q8o_dequant_transpose(const uint32_t* weight, const float* scale, size_t out_features, size_t in_features,
                           float* output) {
    const size_t W = (in_features + 3) / 4;
    for (size_t row = 0; row < out_features; ++row)
        for (size_t col = 0; col < in_features; ++col)
            output[col * out_features + row] = dequant_term(weight[row * W + (col >> 2)], col & 3, scale[row]);
}

/* llm/weights-q8.ts:207-222 (gatherDequantRows): rows of an int8 table in
 * request order; an index outside [0, rows) leaves its output row zero (the
 * output starts zeroed, :211). */
void q8o_gather_dequant_rows(const int8_t* codes, const float* scale, size_t rows, size_t D,
                             const int64_t* indices, size_t count, float* output) {
    for (size_t i = 0; i < count; ++i) {
        const int64_t r = indices[i];
        for (size_t c = 0; c < D; ++c) output[i * D + c] = 0.0f;
        if (r < 0 || (uint64_t)r >= (uint64_t)rows) continue;
        const float s = scale[r];
        for (size_t c = 0; c < D; ++c)
            output[i * D + c] = (float)((double)codes[(size_t)r * D + c] * (double)s);
    }
}
