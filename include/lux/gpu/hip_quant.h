/*
 * lux/gpu/hip_quant.h -- quantized-matmul entry points of libluxgpu_backend_hip.so.
 *
 * ABI v3 has exactly one matmul slot, op_matmul_f32 (reference
 * src/webgpu_plugin.cpp:1721-1771, vtable :4046).  The GEMV and quantized kernels
 * of the reference are library shaders with no vtable slot and no host bridge
 * (gemv.wgsl, quantized_nax.wgsl, quantized.wgsl, fp_quantized.wgsl).  This
 * header gives them one: extra extern "C" symbols that a loader resolves with
 * dlsym next to lux_gpu_backend_init.  Each function below names the reference
 * interface it replaces.
 *
 * Conventions shared by every entry point:
 *   - handles are the plugin's own LuxBackendContext / LuxBackendBuffer;
 *   - weights W are [n_out x k] row-major, packed along k (int4: 8 per u32, value i
 *     of a word in bits 4i..4i+3; int8: one byte each), the flat index being
 *     r*k + kk exactly as in the WGSL (quantized_nax.wgsl:587-593);
 *   - activations X are [m x k] and outputs Y [m x n_out], token-major.  For m == 1
 *     this is the reference layout; for m > 1 the reference's act[k*N + c] and
 *     out[r*N + c] are X^T and Y^T;
 *   - every call is synchronous by default (returns after the device finished,
 *     like dispatchCompute at src/webgpu_plugin.cpp:1005-1051); see
 *     lux_hip_context_set_synchronous.
 */
#ifndef LUX_GPU_HIP_QUANT_H
#define LUX_GPU_HIP_QUANT_H

#include "lux/gpu/backend_plugin.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LUX_HIP_QUANT_API_VERSION 5u

/* Element types.  The first four keep LuxDtype's numbering (docs/api.md:188-197). */
typedef enum LuxHipDtype {
    LUX_HIP_F32 = 0,
    LUX_HIP_F16 = 1,
    LUX_HIP_BF16 = 2,
    LUX_HIP_I32 = 3,
    LUX_HIP_I8 = 32, /* not in LuxDtype: int8 activations (W4A8) */
    LUX_HIP_I4 = 33  /* not in LuxDtype: packed int4 weights     */
} LuxHipDtype;

/* 4-bit value coding.  Offset-binary stores q+8 (quantized_nax.wgsl:94-112);
 * two's complement stores q & 0xF (quantized.wgsl:124-156).  ob = tc ^ 0x8. */
typedef enum LuxHipNibbleCoding {
    LUX_HIP_NIBBLE_OFFSET_BINARY = 0,
    LUX_HIP_NIBBLE_TWOS_COMPLEMENT = 1
} LuxHipNibbleCoding;

/* Per-group scale storage, [n_out x (k / group_size)] row-major. */
typedef enum LuxHipScaleFormat {
    LUX_HIP_SCALE_NONE = 0,       /* no scales: raw integer sums (W4A8, i32 out)   */
    LUX_HIP_SCALE_F16 = 1,        /* IEEE binary16                                 */
    LUX_HIP_SCALE_F32 = 2,        /* binary32                                      */
    LUX_HIP_SCALE_GROUPSCALE = 3  /* 16-byte GroupScale {f32 scale, i32 zero_point,
                                     f32 group_min, f32 group_max}
                                     (quantized_nax.wgsl:49-54); only .scale used */
} LuxHipScaleFormat;

/* Descriptor of one weight-only (or W4A8 / W8A8) quantized matmul
 *   Y[m, n] = sx[m] * sum_k (q(n, k) * s(n, k / group_size)) * X[m, k]
 * sx is 1 unless X is int8 with per-token scales. */
typedef struct LuxHipQMatmulDesc {
    uint32_t struct_size;   /* sizeof(LuxHipQMatmulDesc)                          */
    int32_t n_out;          /* weight rows = output channels                      */
    int32_t k;              /* reduction length; k % 32 == 0                        */
    int32_t m;              /* tokens (rows of X); 1 = GEMV                        */
    int32_t weight_bits;    /* 4 or 8                                              */
    int32_t group_size;     /* k elements per scale along k; k for per-row scales */
    int32_t nibble_coding;  /* LuxHipNibbleCoding (4-bit weights only)            */
    int32_t scale_format;   /* LuxHipScaleFormat                                   */
    int32_t x_dtype;        /* F16, BF16, F32, or I8 (W4A8 / W8A8)                 */
    int32_t y_dtype;        /* F16, BF16, F32, or I32 (W4A8 / W8A8 integer sums)   */
    int32_t flags;          /* LUX_HIP_QFLAG_*                                     */
} LuxHipQMatmulDesc;

/* W4A8 / W8A8 with y_dtype I32 and group_size < k: write the per-group int32 partial
 * sums P[m][n][g] instead of the full-k sum (checking aid, bit-exact). */
#define LUX_HIP_QFLAG_GROUP_PARTIALS (1 << 0)
/* W4A8 / W8A8 from fp activations: x_dtype F32/F16/BF16 is quantized per token to int8 first
 * (compute_group_scales NAX_INT8_SYM + quantize_nax_int8_group with group_size = k,
 * quantized_nax.wgsl:157-232,336-362; s = max|row| / 127, q = clamp(round(x / s)))
 * into the context workspace, then multiplied on the int8 MFMA as with x_dtype I8 and
 * x_scales = s.  Needs weight scales, an fp y_dtype and x_scales NULL. */
#define LUX_HIP_QFLAG_QUANTIZE_X (1 << 1)

/* Quantized matmul / GEMV.  Replaces, by descriptor:
 *   matmul_nax_grouped  quantized_nax.wgsl:568-626  (weight_bits 4, offset-binary,
 *                       group scales, fp activations; m == 1 is the GEMV case)
 *   dequantize_nax_int8_group + matmul  quantized_nax.wgsl:364-386 +
 *                       src/webgpu_plugin.cpp:138-205  (weight_bits 8)
 *   matmul_int4_int8    quantized.wgsl:590-647  (weight_bits 4, two's complement,
 *                       x_dtype I8, y_dtype I32, SCALE_NONE)
 *   matmul_int8         quantized.wgsl:497-555  (weight_bits 8, x_dtype I8,
 *                       y_dtype I32, SCALE_NONE; k % 128 == 0)
 * x_scales is read only for x_dtype I8 with y_dtype != I32 (f32 [m]); pass NULL
 * otherwise.  Returns INVALID_ARGUMENT for NULL handles, buffers smaller than the
 * descriptor implies or inconsistent sizes, NOT_SUPPORTED for combinations without
 * a kernel (the core then falls back to the CPU), DEVICE_LOST when the wait
 * deadline (LUX_HIP_WAIT_TIMEOUT_S, default 5 s) expires. */
LuxBackendError lux_hip_qmatmul(LuxBackendContext* ctx, const LuxHipQMatmulDesc* desc,
                                LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                LuxBackendBuffer* x, LuxBackendBuffer* x_scales,
                                LuxBackendBuffer* y);

/* Output epilogues fused into the matmul store, applied in fp32 before the rounding to
 * y_dtype.  NONE .. ADD_RESIDUAL keep the numbering and formulas of apply_epilogue
 * (steel_gemm_fused.wgsl:80-127): relu max(0, v); gelu 0.5 v (1 + tanh(0.7978845608
 * (v + 0.044715 v^3))); silu v / (1 + exp(-v)); tanh; sigmoid 1 / (1 + exp(-v));
 * v + bias[n] (f32 [n]); v + residual[m, n] (f32 [m x n]).  SILU_MUL is
 * steel_gemm_silu_mul (:452-558): the weight rows are [gate; up], n_out = 2 N, and
 * y[m, n] = silu(gate(m, n)) * up(m, n) has N columns. */
typedef enum LuxHipEpilogue {
    LUX_HIP_EPILOGUE_NONE = 0,
    LUX_HIP_EPILOGUE_RELU = 1,
    LUX_HIP_EPILOGUE_GELU = 2,
    LUX_HIP_EPILOGUE_SILU = 3,
    LUX_HIP_EPILOGUE_TANH = 4,
    LUX_HIP_EPILOGUE_SIGMOID = 5,
    LUX_HIP_EPILOGUE_ADD_BIAS = 6,
    LUX_HIP_EPILOGUE_ADD_RESIDUAL = 7,
    LUX_HIP_EPILOGUE_SILU_MUL = 8
} LuxHipEpilogue;

/* lux_hip_qmatmul with an output epilogue; replaces steel_gemm_fused
 * (steel_gemm_fused.wgsl, bias binding 3, residual binding 4, `epilogue` uniform) and
 * steel_gemm_silu_mul for the weight-only paths (fp activations; NOT_SUPPORTED for
 * W4A8).  bias / residual are read only for ADD_BIAS / ADD_RESIDUAL (pass NULL
 * otherwise).  y is [m x N] with N = n_out, or n_out / 2 for SILU_MUL. */
LuxBackendError lux_hip_qmatmul_ex(LuxBackendContext* ctx, const LuxHipQMatmulDesc* desc,
                                   LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                   LuxBackendBuffer* x, LuxBackendBuffer* x_scales, int epilogue,
                                   LuxBackendBuffer* bias, LuxBackendBuffer* residual,
                                   LuxBackendBuffer* y);

/* No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops that forbid hipMalloc).  Same arguments, checks
 * and results as lux_hip_qmatmul_ex, but the staging buffers of the kernels (activations
 * restaged as fp16 and their row factors, the weight rows' scale folds, per-token int8
 * activations for QUANTIZE_X) live in a fixed per-device array of
 * LUX_HIP_NOALLOC_SCRATCH_BYTES inside the library instead of the context workspace.
 * No hipMalloc / hipFree or other allocating call is made (the first call on a device
 * looks up that device's array).  A shape that needs more scratch than the maximum
 * returns NOT_SUPPORTED: the large-m int4 GEMM needs m*k*2 + m*4 + n_out*4 bytes (config 4:
 * 16.8 MB), QUANTIZE_X m*k + m*4, the small-m int4 GEMM n_out*4 (+ m*4 for bf16/f32 x).
 * The array holds the last call's contents; every kernel writes what it reads there
 * first, so nothing needs clearing.  All calls on one GPU share its array: calls that
 * overlap in time on one GPU (any context, any stream) race and must be serialised by
 * the caller. */
#define LUX_HIP_NOALLOC_SCRATCH_BYTES (32u << 20)
LuxBackendError lux_hip_qmatmul_noalloc(LuxBackendContext* ctx, const LuxHipQMatmulDesc* desc,
                                        LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                        LuxBackendBuffer* x, LuxBackendBuffer* x_scales, int epilogue,
                                        LuxBackendBuffer* bias, LuxBackendBuffer* residual,
                                        LuxBackendBuffer* y);

/* ---- producers and codecs of the matmul inputs ------------------------------ */

/* Descriptor of one symmetric group quantization of X [rows x k] along k. */
typedef struct LuxHipQuantizeDesc {
    uint32_t struct_size;   /* sizeof(LuxHipQuantizeDesc)                              */
    int32_t rows;
    int32_t k;
    int32_t weight_bits;    /* 4 or 8                                                  */
    int32_t group_size;     /* power of two >= 8 dividing k; k gives one scale per row
                               (per-channel weights, per-token W4A8 activations)      */
    int32_t nibble_coding;  /* LuxHipNibbleCoding of the int4 output                   */
    int32_t scale_format;   /* F16, F32 or GROUPSCALE                                  */
    int32_t x_dtype;        /* F32, F16 or BF16                                        */
} LuxHipQuantizeDesc;

/* Symmetric group quantizer; replaces compute_group_scales with NAX_INT4_SYM /
 * NAX_INT8_SYM (quantized_nax.wgsl:157-232) followed by quantize_nax_int4_sym
 * (:238-262) or quantize_nax_int8_group (:336-362), whose flat groups are the rows'
 * groups here because group_size divides k:
 *   s = max(|max x|, |min x|) / (7 for int4, 127 for int8), s == 0 -> 1;
 *   q = clamp(round_half_even(x / s), -8, 7) or (-128, 127).
 * q is written in the layout lux_hip_qmatmul reads (int4: 8 per u32 in nibble_coding;
 * int8: one byte each, [rows x k]); scales [rows x k/group_size] in scale_format
 * (GROUPSCALE: {s, 0, min x, max x} as the reference writes it).  With SCALE_F16 the
 * scale is rounded to binary16 first and q is computed with the rounded value, so that
 * q * s uses the stored scale.  x and q must be 16-byte aligned. */
LuxBackendError lux_hip_quantize(LuxBackendContext* ctx, const LuxHipQuantizeDesc* desc,
                                 LuxBackendBuffer* x, LuxBackendBuffer* q, LuxBackendBuffer* scales);

/* Dequantizers (no host bridge in the reference): dequantize_nax_int4_sym
 * (quantized_nax.wgsl:264-282) and dequantize_nax_int8_group, symmetric branch
 * (:364-386): out[r, k] = f32(q(r, k)) * s(r, k / group_size), computed in fp32 (exact for
 * fp16 scales) and rounded to nearest-even when x_dtype is F16 or BF16.  The descriptor is
 * the quantizer's: x_dtype names the output type, group_size a multiple of 8 dividing k,
 * q and out 16-byte aligned. */
LuxBackendError lux_hip_dequantize(LuxBackendContext* ctx, const LuxHipQuantizeDesc* desc,
                                   LuxBackendBuffer* q, LuxBackendBuffer* scales,
                                   LuxBackendBuffer* out);

/* Re-code `words` packed int4 words between offset-binary (quantized_nax.wgsl:94-112)
 * and two's complement (quantized.wgsl:124-156): every nibble xor 8 (ob = tc ^ 0x8), a
 * copy when the codings agree.  in == out is allowed.  No reference counterpart: the
 * reference keeps the two codings in separate shader families. */
LuxBackendError lux_hip_convert_nibbles(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                        LuxBackendBuffer* out, size_t words, int from_coding,
                                        int to_coding);

/* Convert `count` group scales between LuxHipScaleFormat F16, F32 and GROUPSCALE (the
 * 16-byte GroupScale of quantized_nax.wgsl:49-54).  F16 outputs round to nearest even; a
 * GROUPSCALE written from F16/F32 carries zero_point 0 and group_min = group_max = 0. */
LuxBackendError lux_hip_convert_scales(LuxBackendContext* ctx, LuxBackendBuffer* in, int in_format,
                                       LuxBackendBuffer* out, int out_format, size_t count);

/* PerChannelScale (quantized.wgsl:51-56), one per channel_stride elements. */
typedef struct LuxHipPerChannelScale {
    float scale;
    int32_t zero_point;
    uint32_t _pad0;
    uint32_t _pad1;
} LuxHipPerChannelScale;

/* quantize_int8_per_channel (quantized.wgsl:264-280) over `size` f32 elements of `in`
 * into one i32 per element of `out`: the element's channel is index / channel_stride
 * (ChannelQuantParams.channel_stride, :44-49) and channel_scales holds
 * ceil(size / channel_stride) LuxHipPerChannelScale.  quant_type is QuantParams.quant_type
 * (:37-42): 0 = quantize_int8_symmetric (:83-86), q = clamp(i32(round(x / s)), -128, 127);
 * any other value = quantize_int8_asymmetric (:92-95), q = clamp(i32(round(x / s) +
 * f32(zero_point)), -128, 127).  round() is half-to-even, x / s the IEEE quotient, i32()
 * saturating (NaN -> 0).  Buffers 4-byte aligned. */
LuxBackendError lux_hip_quantize_int8_per_channel(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                                  LuxBackendBuffer* channel_scales, LuxBackendBuffer* out,
                                                  size_t size, uint32_t channel_stride, uint32_t quant_type);

/* dequantize_int8_per_channel (quantized.wgsl:282-297): i32 per element in, f32 out;
 * quant_type 0 = dequantize_int8_symmetric (:88-90), f32(q) * s; otherwise
 * dequantize_int8_asymmetric (:97-99), f32(q - zero_point) * s with the i32 subtraction
 * wrapping.  Channels and alignment as lux_hip_quantize_int8_per_channel. */
LuxBackendError lux_hip_dequantize_int8_per_channel(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                                    LuxBackendBuffer* channel_scales, LuxBackendBuffer* out,
                                                    size_t size, uint32_t channel_stride, uint32_t quant_type);

/* requantize_int32_to_int8 (quantized.wgsl:560-580, RequantParams {size, input_scale,
 * output_scale, output_zero_point}): out[i] = clamp(i32(round(f32(in[i]) * input_scale /
 * output_scale) + output_zero_point), -128, 127), i32 in and out as in the reference. */
LuxBackendError lux_hip_requantize_i32(LuxBackendContext* ctx, LuxBackendBuffer* in,
                                       LuxBackendBuffer* out, size_t size, float input_scale,
                                       float output_scale, int32_t output_zero_point);

/* ---- around the path: RMS normalisation ------------------------------------ */

/* RMSNormParams of rms_norm.wgsl:25-30, plus the element types of input and output
 * (the WGSL is f32 only; F16/BF16 let the normalised activations feed the quantized
 * GEMV directly).  gamma and rms_out are f32. */
typedef struct LuxHipRmsNormParams {
    uint32_t batch_size;   /* rows                                          */
    uint32_t hidden_size;  /* elements per row                              */
    float eps;
    int32_t x_dtype;       /* F32, F16 or BF16                              */
    int32_t y_dtype;       /* F32, F16 or BF16                              */
} LuxHipRmsNormParams;

/* rms_norm (rms_norm.wgsl:50-110): per row, r = 1 / sqrt(sum(x^2) / hidden + eps),
 * y = x * r * gamma[i], rms_out[row] = r (rms_out may be NULL).  The ABI-v3 slot
 * op_rms_norm_f32 exists, but the reference leaves it NULL without a signature
 * (src/webgpu_plugin.cpp:4072), so this is an extra symbol.  The elementwise slots
 * op_add/sub/mul/div_f32 of the vtable are filled (src/webgpu_plugin.cpp:1637-1719). */
LuxBackendError lux_hip_rms_norm(LuxBackendContext* ctx, const LuxHipRmsNormParams* params,
                                 LuxBackendBuffer* input, LuxBackendBuffer* gamma,
                                 LuxBackendBuffer* output, LuxBackendBuffer* rms_out);

/* rms_norm followed by the quantized matmul, as one call: the composition of
 * rms_norm (rms_norm.wgsl:50-110) and lux_hip_qmatmul_ex (matmul_nax_grouped,
 * quantized_nax.wgsl:568-626, for the int4 GEMV); the reference has the two shaders and
 * no fused form.  Rows r < desc->m of x [m x k] (norm->x_dtype) are normalised as
 * lux_hip_rms_norm does, xn = x * r * gamma rounded to desc->x_dtype, and
 * y = lux_hip_qmatmul_ex(desc, w, w_scales, xn, NULL, epilogue, bias, residual).
 * norm->batch_size must equal desc->m, norm->hidden_size desc->k, norm->y_dtype
 * desc->x_dtype (F32, F16 or BF16; x_scales are not taken, so W4A8 only with
 * QUANTIZE_X).  The result is bit-identical to lux_hip_rms_norm into a buffer of
 * desc->x_dtype followed by lux_hip_qmatmul_ex.  At m == 1 with int4 weights, SCALE_F16,
 * x_dtype F16, flags 0 and k <= 8192 on the GEMV's fast path (k % 32 == 0, group_size a
 * power-of-two multiple of 32 with an even number of groups per row), where the GEMV
 * streams whole rows per wave (more than 16 rows per CU, or k < 4096: the gate/up and
 * QKV projections of a decode step), the GEMV computes the normalisation in its
 * prologue (one launch; the rms_norm kernel and its output round trip disappear).
 * Other descriptors run rms_norm and then the matmul, with xn in the context
 * workspace.  Errors as lux_hip_rms_norm and lux_hip_qmatmul_ex. */
LuxBackendError lux_hip_rms_norm_qmatmul(LuxBackendContext* ctx, const LuxHipRmsNormParams* norm,
                                         LuxBackendBuffer* gamma, const LuxHipQMatmulDesc* desc,
                                         LuxBackendBuffer* w, LuxBackendBuffer* w_scales,
                                         LuxBackendBuffer* x, int epilogue, LuxBackendBuffer* bias,
                                         LuxBackendBuffer* residual, LuxBackendBuffer* y);

/* GemvParams of gemv.wgsl:21-30. */
typedef struct LuxHipGemvParams {
    uint32_t M;     /* rows of A                               */
    uint32_t N;     /* columns of A                            */
    float alpha;
    float beta;     /* y is read only when beta != 0           */
    uint32_t lda;   /* leading dimension of A (>= N)           */
    uint32_t trans; /* 0: y[M] = alpha*A x + beta*y; 1: y[N] = alpha*A^T x + beta*y */
    uint32_t _pad0;
    uint32_t _pad1;
} LuxHipGemvParams;

/* fp32 GEMV, replaces gemv_row_parallel / gemv_vec4 / gemv_tiled / gemv_simple
 * (trans 0, gemv.wgsl:49-96,155-274,360-381), steel_gemv (trans 0, lda = N,
 * steel/gemm/gemm.wgsl:186-220) and gemv_transpose (trans 1, gemv.wgsl:103-149);
 * bindings 0..3 of the WGSL become a, x, y, params. */
LuxBackendError lux_hip_gemv_f32(LuxBackendContext* ctx, LuxBackendBuffer* a,
                                 LuxBackendBuffer* x, LuxBackendBuffer* y,
                                 const LuxHipGemvParams* params);

/* BatchGemvParams of gemv.wgsl:280-293: batch_count independent row GEMVs. */
typedef struct LuxHipGemvBatchedParams {
    uint32_t M;           /* rows of each A                          */
    uint32_t N;           /* columns of each A                       */
    float alpha;
    float beta;           /* y is read only when beta != 0           */
    uint32_t lda;         /* leading dimension of each A (>= N)      */
    uint32_t batch_count;
    uint32_t stride_a;    /* elements between consecutive matrices   */
    uint32_t stride_x;    /* elements between consecutive x vectors  */
    uint32_t stride_y;    /* elements between consecutive y vectors (>= M when batch_count > 1) */
    uint32_t _pad0;
    uint32_t _pad1;
    uint32_t _pad2;
} LuxHipGemvBatchedParams;

/* Batched fp32 GEMV, replaces gemv_batched (gemv.wgsl:297-354): for each batch b,
 * y_b[M] = alpha * A_b x_b + beta * y_b with A_b = a + b*stride_a (row-major, lda),
 * x_b = x + b*stride_x, y_b = y + b*stride_y.  stride_a or stride_x may be 0 (one
 * matrix or one vector shared by all batches); y vectors may not overlap, so
 * stride_y < M with batch_count > 1 is refused (the WGSL would race on y). */
LuxBackendError lux_hip_gemv_f32_batched(LuxBackendContext* ctx, LuxBackendBuffer* a,
                                         LuxBackendBuffer* x, LuxBackendBuffer* y,
                                         const LuxHipGemvBatchedParams* params);

/* fp16 GEMV with fp32 accumulation: y[M] (f32) = A[M x N] (f16) . x[N] (f16).
 * Replaces dot_product_fp16_fp32 (fp_quantized.wgsl:418-469) used with one shared
 * vector.  lda in elements, even. */
LuxBackendError lux_hip_gemv_f16(LuxBackendContext* ctx, LuxBackendBuffer* a,
                                 LuxBackendBuffer* x, LuxBackendBuffer* y, uint32_t M,
                                 uint32_t N, uint32_t lda);

/* DotParams of fp_quantized.wgsl:404-409. */
typedef struct LuxHipDotParams {
    uint32_t size;          /* elements per vector                                    */
    uint32_t num_vectors;
    uint32_t vector_stride; /* elements between consecutive vectors' starts           */
    uint32_t _pad;
} LuxHipDotParams;

/* Batched fp16 dot product with fp32 accumulation, replaces dot_product_fp16_fp32
 * (fp_quantized.wgsl:418-469), bindings 0..3 = a, b, result, params: result[v] (f32) =
 * sum_j a[e + j] * b[e + j] over j < size, e = 2 * floor(v * vector_stride / 2) (the WGSL
 * reads f16 pairs from u32 word base / 2, so an odd base starts one element early). */
LuxBackendError lux_hip_dot_f16(LuxBackendContext* ctx, LuxBackendBuffer* a, LuxBackendBuffer* b,
                                LuxBackendBuffer* result, const LuxHipDotParams* params);

/* ---- host packers: CPU code, no device or context -------------------------------
 * The weight/scale codec on the host, for a loader that prepares quantized weights
 * before upload; bit-identical to the device codecs above. */

/* Pack n (a multiple of 8) int4 values in [-8, 7] into n / 8 words, element i of a word
 * in bits 4i .. 4i+3: offset-binary q + 8 (pack_nax_int4_sym_x8, quantized_nax.wgsl:
 * 94-102) or two's complement (the coding unpack_int4x8 reads, quantized.wgsl:148-156).
 * A value outside [-8, 7] is refused with its index. */
LuxBackendError lux_hip_pack_int4_host(const int8_t* q, size_t n, int coding, uint32_t* words);

/* The inverse: n values from n / 8 words (unpack_nax_int4_sym_x8, quantized_nax.wgsl:
 * 105-112, or unpack_int4x8, quantized.wgsl:148-156). */
LuxBackendError lux_hip_unpack_int4_host(const uint32_t* words, size_t n, int coding, int8_t* q);

/* lux_hip_convert_scales on host memory: F16 <-> F32 <-> GROUPSCALE (quantized_nax.wgsl:
 * 49-54), binary16 by round to nearest even, a GROUPSCALE from F16/F32 as {s, 0, 0, 0}. */
LuxBackendError lux_hip_convert_scales_host(const void* in, int in_format, void* out, int out_format,
                                            size_t count);

/* ---- buffer / stream plumbing (no reference counterpart: the WebGPU plugin
 * hides device addresses, src/webgpu_plugin.cpp:1564) ------------------------ */

/* Wrap caller-owned device memory as a buffer handle; buffer_free releases only
 * the handle. */
LuxBackendBuffer* lux_hip_buffer_wrap(LuxBackendContext* ctx, void* device_ptr, size_t bytes);
void* lux_hip_buffer_device_ptr(LuxBackendBuffer* buf);
size_t lux_hip_buffer_size(LuxBackendBuffer* buf);

/* Run subsequent ops on `stream` (a hipStream_t; NULL restores the context's own). */
LuxBackendError lux_hip_context_set_stream(LuxBackendContext* ctx, void* stream);
void* lux_hip_context_get_stream(LuxBackendContext* ctx);
/* synchronous != 0 (default): every op waits for completion before returning.
 * 0: ops only enqueue; call vtbl->sync to wait. */
LuxBackendError lux_hip_context_set_synchronous(LuxBackendContext* ctx, int synchronous);

/* Message of the last failure on the calling thread ("" if none). */
const char* lux_hip_last_error(void);
uint32_t lux_hip_quant_api_version(void);

#ifdef __cplusplus
}
#endif
#endif /* LUX_GPU_HIP_QUANT_H */
