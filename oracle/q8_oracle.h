/*
 * q8_oracle.h -- CPU restatement of web-xpu-ops' matvecQ8 path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP path is compared
 * against, never part of the product: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it.
 *
 * Every function restates one reference function with the reference's own
 * ECMAScript semantics (JS numbers are IEEE f64; Float32Array stores round
 * to nearest-even; Int32Array stores truncate, NaN -> 0):
 *
 *   q8o_quantize          ops/quantize/reference.ts:13-38
 *   q8o_pack_q8           ops/matvec/reference.ts:267-283
 *   q8o_pack_int8_rows    llm/weights-q8.ts:137-139 (packQ8 over Int8Array)
 *   q8o_matvec_q8         ops/matvec/reference.ts:113-131 (unpackI8 + matvecQ8)
 *   q8o_matvec_q8_residual ops/matvec/reference.ts:235-243 (matvecQ8Residual)
 *   q8o_matvec_q8_ffn     ops/matvec/reference.ts:196-207 (matvecQ8Ffn), with
 *   q8o_silu              ops/activation/reference.ts:91-92 (silu)
 *   q8o_matvec_q8_absterm sum_k |s_n * q_nk * x_k| in f64: the per-row bound
 *                         the f32 kernels are judged against
 *   q8o_matmul_q8         ops/matmul/reference.ts:124-137 (matmulQ8: per-term
 *                         dequant into matmul's b, then matmul :37-49)
 *   q8o_matmul_q8_absterm sum_k |a_nk * fround(q_mk * s_m)| in f64 per output
 *   q8o_dequantize_packed_q8 llm/weights-q8.ts:161-177 (dequantizePackedQ8)
 *   q8o_dequant_transpose ops/dequant_transpose/reference.ts:40-59 (dequantTranspose)
 *   q8o_gather_dequant_rows llm/weights-q8.ts:207-222 (gatherDequantRows)
 *
 * Batched matvecQ8 (M vectors) has no reference function; it is M
 * independent matvecQ8 calls by definition, so the checker loops M times.
 */
#ifndef Q8_ORACLE_H
#define Q8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Math.round: nearest integer, ties toward +Infinity, no double rounding. */
double q8o_js_round(double v);

void q8o_quantize(const float* input, size_t N, size_t D, int32_t* output, float* scales);
void q8o_pack_q8(const int32_t* codes, size_t N, size_t K, uint32_t* packed);
void q8o_pack_int8_rows(const int8_t* codes, size_t N, size_t K, uint32_t* packed);
void q8o_matvec_q8(const uint32_t* weight, const float* scale, const float* vector,
                   size_t N, size_t K, float* output);
void q8o_matvec_q8_batched(const uint32_t* weight, const float* scale, const float* vectors,
                           size_t N, size_t K, size_t M, float* output);
void q8o_matvec_q8_residual(const uint32_t* weight, const float* scale, const float* vector,
                            const float* residual, size_t N, size_t K, float* output);
float q8o_silu(float x);
void q8o_matvec_q8_ffn(const uint32_t* weight_gate, const float* scale_gate, const uint32_t* weight_up,
                       const float* scale_up, const float* vector, size_t N, size_t K, float* output);
void q8o_matvec_q8_absterm(const uint32_t* weight, const float* scale, const float* vector,
                           size_t N, size_t K, double* bound);

void q8o_matmul_q8(const float* a, const uint32_t* weight, const float* scale, size_t N, size_t M, size_t K,
                   float* output);
void q8o_matmul_q8_absterm(const float* a, const uint32_t* weight, const float* scale, size_t N, size_t M,
                           size_t K, double* bound);
void q8o_dequantize_packed_q8(const uint32_t* weight, const float* scale, size_t N, size_t K, float* output);
void q8o_dequant_transpose(const uint32_t* weight, const float* scale, size_t out_features, size_t in_features,
                           float* output);
void q8o_gather_dequant_rows(const int8_t* codes, const float* scale, size_t rows, size_t D,
                             const int64_t* indices, size_t count, float* output);

#ifdef __cplusplus
}
#endif

#endif
