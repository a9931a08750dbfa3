/*
 * lux_oracle.h -- CPU restatement of the reference WGSL arithmetic on the
 * quantized-matmul path.  TEST INFRASTRUCTURE ONLY: the parity tests, the smoke
 * check and the CPU-baseline leg of bench.py use it as the checker.  Nothing in
 * the shipped plugin links or calls it.
 *
 * Every function restates one reference function (file:line under the
 * luxcpp/webgpu tree) in plain C with the same accumulation order, compiled with
 * -ffp-contract=off so each `a*b + c` of the WGSL source stays a separate
 * multiply and add.
 *
 * Layout conventions follow the reference: weights [rows x K] row-major with the
 * flat index r*K + k; 4-bit values packed 8 per u32 (element i of a word in bits
 * 4i..4i+3); 8-bit values packed 4 per u32 little-endian, which is byte-for-byte
 * a plain int8 array.  Activations for the grouped/int matmuls are [K x N] and
 * outputs [rows x N], exactly as the WGSL bindings declare them.
 */
#ifndef LUX_ORACLE_H
#define LUX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs ---------------------------------------------------- */
uint32_t lo_f32_to_f16_wgsl(float v);      /* fp_quantized.wgsl:65-128  */
float lo_f16_to_f32(uint32_t bits);        /* fp_quantized.wgsl:131-165 */
uint16_t lo_f32_to_f16_rne(float v);       /* IEEE binary16, round-nearest-even */
uint16_t lo_f32_to_bf16_rne(float v);      /* bfloat16, round-nearest-even      */
float lo_bf16_to_f32(uint16_t bits);

uint32_t lo_pack_int4_ob(const int32_t vals[8]);   /* quantized_nax.wgsl:94-102  */
void lo_unpack_int4_ob(uint32_t w, int32_t out[8]);/* quantized_nax.wgsl:105-112 */
uint32_t lo_pack_int4_tc(const int32_t vals[8]);   /* quantized.wgsl:130-136     */
void lo_unpack_int4_tc(uint32_t w, int32_t out[8]);/* quantized.wgsl:148-156     */
uint32_t lo_pack_int8x4(const int32_t vals[4]);    /* quantized_nax.wgsl:136-141 */
void lo_unpack_int8x4(uint32_t w, int32_t out[4]); /* quantized_nax.wgsl:143-151 */

/* ---- bulk codecs ------------------------------------------------------ */
void lo_f16_to_f32_array(const uint16_t* in, float* out, size_t n);
void lo_f32_to_f16_rne_array(const float* in, uint16_t* out, size_t n);
void lo_f32_to_f16_wgsl_array(const float* in, uint16_t* out, size_t n);
void lo_bf16_to_f32_array(const uint16_t* in, float* out, size_t n);
void lo_f32_to_bf16_rne_array(const float* in, uint16_t* out, size_t n);

/* ---- fp32 GEMV / GEMM ------------------------------------------------- */
/* WGSL_MATMUL::matmul, src/webgpu_plugin.cpp:138-205: C[M x N] = A[M x K] B[K x N],
 * one fp32 sum per output, k = 0..K-1 in order. */
void lo_matmul_f32(const float* A, const float* B, float* C, int M, int K, int N);
/* gemv.wgsl:49-96 gemv_row_parallel: 256 strided partial sums, tree reduce,
 * y = alpha*sum + beta*y (y is read even when beta == 0, as the WGSL does). */
void lo_gemv_row_parallel(const float* A, const float* x, float* y, int M, int N, int lda,
                          float alpha, float beta);
/* gemv.wgsl:103-149 gemv_transpose: y[c] = alpha*sum_r A[r,c] x[r] + beta*y[c]. */
void lo_gemv_transpose(const float* A, const float* x, float* y, int M, int N, int lda,
                       float alpha, float beta);
/* gemv.wgsl:204-274 gemv_vec4. */
void lo_gemv_vec4(const float* A, const float* x, float* y, int M, int N, int lda, float alpha,
                  float beta);
/* fp_quantized.wgsl:418-469 dot_product_fp16_fp32 generalised to a shared x:
 * y[r] = sum over pairs of widened fp16 products, 256 strided partials + tree. */
void lo_gemv_f16_f32(const uint16_t* A, const uint16_t* x, float* y, int M, int N, int lda);

/* ---- grouped int4 / int8 weight-only --------------------------------- */
/* quantized_nax.wgsl:568-626 matmul_nax_grouped:
 *   out[r, c] = sum_k (f32(nib(r,k) - 8) * scale[(r*K + k) / gs]) * act[k*N + c]
 * k in order.  nibble_coding 0 = offset-binary (this file), 1 = two's complement
 * (quantized.wgsl:148-156); scale[] is GroupScale.scale widened to f32. */
void lo_matmul_nax_grouped(const uint32_t* W, const float* scale, const float* act, float* out,
                           int M, int N, int K, int gs, int nibble_coding);
/* quantized_nax.wgsl:264-282 dequantize_nax_int4_sym. */
void lo_dequantize_nax_int4_sym(const uint32_t* packed, const float* scale, float* out,
                                size_t size, int gs, int nibble_coding);
/* quantized_nax.wgsl:364-386 dequantize_nax_int8_group (NAX_INT8_SYM). */
void lo_dequantize_nax_int8_group(const uint32_t* packed, const float* scale, float* out,
                                  size_t size, int gs);
/* The reference composition for int8 weights x fp activations: dequantize_nax_int8_group
 * followed by WGSL_MATMUL with A = dequantized W [M x K] and B = act [K x N]. */
void lo_matmul_int8_dequant(const int8_t* W, const float* scale, const float* act, float* out,
                            int M, int N, int K, int gs);

/* ---- integer matmuls -------------------------------------------------- */
/* quantized.wgsl:590-647 matmul_int4_int8: out[r,c] = sum_k w4(r,k) * a8(k,c), i32. */
void lo_matmul_int4_int8(const uint32_t* W, const int8_t* act, int32_t* out, int M, int N, int K,
                         int nibble_coding);
/* quantized.wgsl:497-555 matmul_int8. */
void lo_matmul_int8(const int8_t* A, const int8_t* B, int32_t* out, int M, int N, int K);
/* quantized.wgsl:264-280 / 282-297: per-channel int8 (i32 per element) with
 * PerChannelScale {scale, zero_point, pad, pad} (:51-56) per channel_stride elements;
 * quant_type 0 symmetric, otherwise asymmetric. */
void lo_quantize_int8_per_channel(const float* in, const void* channels, int32_t* out, size_t n,
                                  uint32_t stride, uint32_t quant_type);
void lo_dequantize_int8_per_channel(const int32_t* in, const void* channels, float* out, size_t n,
                                    uint32_t stride, uint32_t quant_type);

/* quantized.wgsl:572-580 requantize_int32_to_int8. */
void lo_requantize_int32_to_int8(const int32_t* in, int32_t* out, size_t n, float in_scale,
                                 float out_scale, int32_t out_zp);
/* W4A8 per-group partial sums: P[c, r, g] = sum_{k in group g} w4(r,k) * a8(c,k), with the
 * activations token-major [N x K] (the grouped form of matmul_int4_int8). */
void lo_w4a8_group_partials(const uint32_t* W, const int8_t* A, int32_t* P, int M, int N, int K,
                            int gs, int nibble_coding);

/* ---- producers (quantizers) ------------------------------------------- */
/* quantized_nax.wgsl:157-232 compute_group_scales (256-lane min/max tree). */
void lo_compute_group_scales(const float* in, size_t size, int gs, int format, float* scale,
                             int32_t* zero_point, float* gmin, float* gmax);
/* quantized_nax.wgsl:238-262 quantize_nax_int4_sym. */
void lo_quantize_nax_int4_sym(const float* in, size_t size, int gs, const float* scale,
                              uint32_t* packed);
/* quantized_nax.wgsl:336-362 quantize_nax_int8_group (NAX_INT8_SYM). */
void lo_quantize_nax_int8_group(const float* in, size_t size, int gs, const float* scale,
                                uint32_t* packed);

/* ---- GEMM epilogues ---------------------------------------------------- */
/* steel_gemm_fused.wgsl:80-127 apply_epilogue over y [m x n] in place: kind 1 relu,
 * 2 gelu (tanh form), 3 silu, 4 tanh, 5 sigmoid, 6 + bias[n], 7 + residual[m, n]. */
void lo_apply_epilogue(float* y, int m, int n, int kind, const float* bias, const float* residual);
/* steel_gemm_silu_mul (steel_gemm_fused.wgsl:452-558) output stage: out[m, n] =
 * silu(gu[m, n]) * gu[m, N + n] for gu [m x 2N] (gate columns, then up columns). */
void lo_silu_mul(const float* gu, float* out, int m, int N);

/* ---- around the path ---------------------------------------------------- */
/* rms_norm.wgsl:50-110: per row r = 1 / sqrt(sum(x^2) / hidden + eps) with the sum in
 * the shader's order (256 strided partial sums, then the tree), y = x * r * gamma[i],
 * rms_out[row] = r (rms_out may be NULL). */
void lo_rms_norm(const float* x, const float* gamma, float* y, float* rms_out, int rows, int hidden,
                 float eps);

/* ---- fp64 ground truth ------------------------------------------------ */
/* y[c, r] = sum_k (q(r,k) * s(r, k/gs)) * x(c, k) in double, token-major x and y.
 * wbits 4 (nibble_coding as above) or 8 (W int8 row-major). */
void lo_qmatmul_f64(const void* W, const float* scale, const float* X, double* Y, int n_out,
                    int K, int M, int gs, int wbits, int nibble_coding);

int lo_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
