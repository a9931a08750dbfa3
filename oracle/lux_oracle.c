/*
 * lux_oracle.c -- CPU restatement of the luxcpp/webgpu WGSL arithmetic on the
 * quantized-matmul path.  TEST INFRASTRUCTURE ONLY (parity checker and CPU
 * baseline); the shipped HIP plugin never links or calls this file.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off).  With contraction
 * off every `a * b + c` below is a rounded multiply followed by a rounded add,
 * which is how the WGSL source reads; whether Tint/naga fuse them on a given
 * adapter is implementation-defined and cannot be pinned here.
 */
#include "lux_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define WG 256 /* WORKGROUP_SIZE of gemv.wgsl:14, quantized_nax.wgsl:20 */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

int lo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ======================================================================= */
/* Scalar codecs                                                           */
/* ======================================================================= */

/* fp_quantized.wgsl:65-128.  Note the two departures from IEEE RNE that the
 * WGSL makes: inputs with a zero exponent field (f32 denormals) flush to a
 * signed zero (:83-86), and results in the f16 denormal range are rounded by
 * adding the first dropped bit, i.e. round-half-up on the magnitude (:96-106). */
uint32_t lo_f32_to_f16_wgsl(float val) {
    uint32_t bits = f2u(val);
    uint32_t sign = (bits >> 16) & 0x8000u;
    uint32_t exp = (bits >> 23) & 0xFFu;
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 255u) return mant != 0u ? (sign | 0x7E00u) : (sign | 0x7C00u);
    if (exp == 0u) return sign;
    int32_t new_exp = (int32_t)exp - 127 + 15;
    if (new_exp >= 31) return sign | 0x7C00u;
    if (new_exp <= 0) {
        if (new_exp < -10) return sign;
        uint32_t shift = (uint32_t)(1 - new_exp);
        uint32_t m = mant | 0x800000u;
        uint32_t denorm = (m >> (13u + shift)) + ((m >> (12u + shift)) & 1u);
        return sign | denorm;
    }
    uint32_t trunc = mant >> 13;
    uint32_t round_bit = (mant >> 12) & 1u;
    int sticky = (mant & 0xFFFu) != 0u;
    uint32_t rounded = trunc;
    if (round_bit != 0u && (sticky || (trunc & 1u) != 0u)) {
        rounded += 1u;
        if (rounded >= 0x400u) {
            rounded = 0u;
            if (new_exp < 30) return sign | ((uint32_t)(new_exp + 1) << 10);
            return sign | 0x7C00u;
        }
    }
    return sign | ((uint32_t)new_exp << 10) | rounded;
}

/* fp_quantized.wgsl:131-165 (exact widening; NaN payload kept, quiet bit set). */
float lo_f16_to_f32(uint32_t bits) {
    uint32_t sign = (bits & 0x8000u) << 16;
    uint32_t exp = (bits >> 10) & 0x1Fu;
    uint32_t mant = bits & 0x3FFu;
    if (exp == 0u) {
        if (mant == 0u) return u2f(sign);
        uint32_t m = mant;
        int32_t e = 0;
        while ((m & 0x400u) == 0u) { m <<= 1; e -= 1; }
        m &= 0x3FFu;
        uint32_t ne = (uint32_t)(127 - 15 + 1 + e);
        return u2f(sign | (ne << 23) | (m << 13));
    }
    if (exp == 31u) {
        if (mant == 0u) return u2f(sign | 0x7F800000u);
        return u2f(sign | 0x7FC00000u | (mant << 13));
    }
    return u2f(sign | ((exp + 127u - 15u) << 23) | (mant << 13));
}

/* IEEE binary16 round-to-nearest-even, written from the format definition
 * (used to round fp32 results to an fp16 output dtype). */
uint16_t lo_f32_to_f16_rne(float v) {
    uint32_t x = f2u(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* < 2^-25 rounds to 0    */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); unit 2^-24 -> shift 126-e */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* carry may bump exp */
    return (uint16_t)(sign | q);
}

uint16_t lo_f32_to_bf16_rne(float v) {
    uint32_t x = f2u(v);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7FFFu + lsb;
    return (uint16_t)(x >> 16);
}

float lo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* quantized_nax.wgsl:94-102: stored nibble = value + 8. */
uint32_t lo_pack_int4_ob(const int32_t vals[8]) {
    uint32_t r = 0u;
    for (uint32_t i = 0; i < 8u; ++i) r |= (((uint32_t)(vals[i] + 8)) & 0xFu) << (i * 4u);
    return r;
}

/* quantized_nax.wgsl:105-112 */
void lo_unpack_int4_ob(uint32_t w, int32_t out[8]) {
    for (uint32_t i = 0; i < 8u; ++i) out[i] = (int32_t)((w >> (i * 4u)) & 0xFu) - 8;
}

/* quantized.wgsl:130-136: two's-complement nibbles. */
uint32_t lo_pack_int4_tc(const int32_t vals[8]) {
    uint32_t r = 0u;
    for (uint32_t i = 0; i < 8u; ++i) r |= ((uint32_t)vals[i] & 0xFu) << (i * 4u);
    return r;
}

/* quantized.wgsl:148-156: sign-extend values >= 8. */
void lo_unpack_int4_tc(uint32_t w, int32_t out[8]) {
    for (uint32_t i = 0; i < 8u; ++i) {
        int32_t v = (int32_t)((w >> (i * 4u)) & 0xFu);
        if (v >= 8) v -= 16;
        out[i] = v;
    }
}

/* quantized_nax.wgsl:136-141 */
uint32_t lo_pack_int8x4(const int32_t v[4]) {
    return ((uint32_t)(v[3] & 0xFF) << 24) | ((uint32_t)(v[2] & 0xFF) << 16) |
           ((uint32_t)(v[1] & 0xFF) << 8) | (uint32_t)(v[0] & 0xFF);
}

/* quantized_nax.wgsl:143-151 */
void lo_unpack_int8x4(uint32_t w, int32_t out[4]) {
    for (uint32_t i = 0; i < 4u; ++i) {
        int32_t v = (int32_t)((w >> (i * 8u)) & 0xFFu);
        if (v >= 128) v -= 256;
        out[i] = v;
    }
}

static inline int32_t nib_at(const uint32_t* W, size_t flat, int coding) {
    int32_t v = (int32_t)((W[flat >> 3] >> ((flat & 7u) * 4u)) & 0xFu);
    if (coding == 0) return v - 8;       /* offset-binary, quantized_nax.wgsl:109 */
    return v >= 8 ? v - 16 : v;          /* two's complement, quantized.wgsl:152 */
}

void lo_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = lo_f16_to_f32(in[i]);
}
void lo_f32_to_f16_rne_array(const float* in, uint16_t* out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = lo_f32_to_f16_rne(in[i]);
}
void lo_f32_to_f16_wgsl_array(const float* in, uint16_t* out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = (uint16_t)lo_f32_to_f16_wgsl(in[i]);
}
void lo_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = lo_bf16_to_f32(in[i]);
}
void lo_f32_to_bf16_rne_array(const float* in, uint16_t* out, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = lo_f32_to_bf16_rne(in[i]);
}

/* ======================================================================= */
/* fp32 GEMV / GEMM                                                        */
/* ======================================================================= */

/* Tree reduction of 256 partials with strides 128..1 (gemv.wgsl:84-89). */
static float tree256(float* s) {
    for (int stride = WG / 2; stride > 0; stride >>= 1)
        for (int t = 0; t < stride; ++t) s[t] = s[t] + s[t + stride];
    return s[0];
}

/* WGSL_MATMUL (src/webgpu_plugin.cpp:138-205).  The 16-wide K tiles are
 * consumed in order and each tile's 16 products in order, so the whole sum is
 * k = 0..K-1 sequential.  Blocked over (rows, cols) for cache reuse only. */
void lo_matmul_f32(const float* A, const float* B, float* C, int M, int K, int N) {
    const int RB = 16, CB = 512;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int r0 = 0; r0 < M; r0 += RB)
        for (int c0 = 0; c0 < N; c0 += CB) {
            int r1 = r0 + RB < M ? r0 + RB : M;
            int c1 = c0 + CB < N ? c0 + CB : N;
            float acc[16][512];
            for (int r = r0; r < r1; ++r)
                for (int c = c0; c < c1; ++c) acc[r - r0][c - c0] = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float* brow = B + (size_t)k * N;
                for (int r = r0; r < r1; ++r) {
                    float a = A[(size_t)r * K + k];
                    float* ac = acc[r - r0];
                    for (int c = c0; c < c1; ++c) ac[c - c0] = ac[c - c0] + a * brow[c];
                }
            }
            for (int r = r0; r < r1; ++r)
                for (int c = c0; c < c1; ++c) C[(size_t)r * N + c] = acc[r - r0][c - c0];
        }
}

/* gemv.wgsl:49-96 */
void lo_gemv_row_parallel(const float* A, const float* x, float* y, int M, int N, int lda,
                          float alpha, float beta) {
#pragma omp parallel for schedule(static)
    for (int row = 0; row < M; ++row) {
        float sh[WG];
        for (int t = 0; t < WG; ++t) {
            float p = 0.0f;
            for (int col = t; col < N; col += WG) p = p + A[(size_t)row * lda + col] * x[col];
            sh[t] = p;
        }
        float s = tree256(sh);
        float old = y[row];
        y[row] = alpha * s + beta * old;
    }
}

/* gemv.wgsl:297-354 (gemv_batched): workgroup b*M + row computes row `row` of batch b with
 * the row_parallel reduction, over A + b*stride_a, x + b*stride_x, y + b*stride_y.
 * Strides and lda are in elements, as the u32 fields of BatchGemvParams. */
void lo_gemv_batched(const float* A, const float* x, float* y, int M, int N, int lda,
                     float alpha, float beta, int batch, long stride_a, long stride_x,
                     long stride_y) {
    for (int b = 0; b < batch; ++b)
        lo_gemv_row_parallel(A + (size_t)b * stride_a, x + (size_t)b * stride_x,
                             y + (size_t)b * stride_y, M, N, lda, alpha, beta);
}

/* gemv.wgsl:103-149 */
void lo_gemv_transpose(const float* A, const float* x, float* y, int M, int N, int lda,
                       float alpha, float beta) {
#pragma omp parallel for schedule(static)
    for (int col = 0; col < N; ++col) {
        float sh[WG];
        for (int t = 0; t < WG; ++t) {
            float p = 0.0f;
            for (int row = t; row < M; row += WG) p = p + A[(size_t)row * lda + col] * x[row];
            sh[t] = p;
        }
        float s = tree256(sh);
        float old = y[col];
        y[col] = alpha * s + beta * old;
    }
}

/* gemv.wgsl:204-274 */
void lo_gemv_vec4(const float* A, const float* x, float* y, int M, int N, int lda, float alpha,
                  float beta) {
    int nv = N / 4;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < M; ++row) {
        const float* a = A + (size_t)row * lda;
        float sh[WG];
        for (int t = 0; t < WG; ++t) {
            float p = 0.0f;
            for (int v = t; v < nv; v += WG) {
                int c = v * 4;
                p = p + (((a[c] * x[c] + a[c + 1] * x[c + 1]) + a[c + 2] * x[c + 2]) +
                         a[c + 3] * x[c + 3]);
            }
            if (t == 0)
                for (int i = nv * 4; i < N; ++i) p = p + a[i] * x[i];
            sh[t] = p;
        }
        float s = tree256(sh);
        float old = y[row];
        y[row] = alpha * s + beta * old;
    }
}

/* fp_quantized.wgsl:418-469 as written (dot_product_fp16_fp32): vector v reads the f16
 * pairs of words base/2 + i, base = v*stride, of both a and b (an odd base starts one
 * element early), i < ceil(size/2); the second element of the last pair counts only when
 * size is even.  Strided partials over 256 threads, then the tree. */
void lo_dot_product_fp16_fp32(const uint16_t* a, const uint16_t* b, float* out, int size,
                              int num_vectors, int stride) {
    const int npairs = (size + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int v = 0; v < num_vectors; ++v) {
        const size_t w0 = ((size_t)v * (size_t)stride) / 2;  /* first u32 word */
        float sh[WG];
        for (int t = 0; t < WG; ++t) {
            float s = 0.0f;
            for (int i = t; i < npairs; i += WG) {
                const size_t e = 2 * (w0 + i);
                s = s + lo_f16_to_f32(a[e]) * lo_f16_to_f32(b[e]);
                if (2 * i + 1 < size) s = s + lo_f16_to_f32(a[e + 1]) * lo_f16_to_f32(b[e + 1]);
            }
            sh[t] = s;
        }
        out[v] = tree256(sh);
    }
}

/* fp_quantized.wgsl:418-469 with the row base r*lda and a shared x. */
void lo_gemv_f16_f32(const uint16_t* A, const uint16_t* x, float* y, int M, int N, int lda) {
    int npairs = (N + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < M; ++row) {
        const uint16_t* a = A + (size_t)row * lda;
        float sh[WG];
        for (int t = 0; t < WG; ++t) {
            float s = 0.0f;
            for (int i = t; i < npairs; i += WG) {
                float a0 = lo_f16_to_f32(a[2 * i]);
                float b0 = lo_f16_to_f32(x[2 * i]);
                s = s + a0 * b0;
                if (2 * i + 1 < N) {
                    float a1 = lo_f16_to_f32(a[2 * i + 1]);
                    float b1 = lo_f16_to_f32(x[2 * i + 1]);
                    s = s + a1 * b1;
                }
            }
            sh[t] = s;
        }
        y[row] = tree256(sh);
    }
}

/* ======================================================================= */
/* Grouped int4 / int8                                                     */
/* ======================================================================= */

/* quantized_nax.wgsl:568-626.  tile_a holds f32(q) * scale (:608), so each
 * product is (q*s)*act with the dequant multiply rounded first.  Blocked over
 * output rows and columns; per output the k order is 0..K-1. */
void lo_matmul_nax_grouped(const uint32_t* W, const float* scale, const float* act, float* out,
                           int M, int N, int K, int gs, int coding) {
    const int RB = 8, CB = 512;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int r0 = 0; r0 < M; r0 += RB)
        for (int c0 = 0; c0 < N; c0 += CB) {
            int r1 = r0 + RB < M ? r0 + RB : M;
            int c1 = c0 + CB < N ? c0 + CB : N;
            float acc[8][512];
            for (int r = r0; r < r1; ++r)
                for (int c = c0; c < c1; ++c) acc[r - r0][c - c0] = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float* brow = act + (size_t)k * N;
                for (int r = r0; r < r1; ++r) {
                    size_t flat = (size_t)r * K + k;
                    float w = (float)nib_at(W, flat, coding) * scale[flat / (size_t)gs];
                    float* ac = acc[r - r0];
                    for (int c = c0; c < c1; ++c) ac[c - c0] = ac[c - c0] + w * brow[c];
                }
            }
            for (int r = r0; r < r1; ++r)
                for (int c = c0; c < c1; ++c) out[(size_t)r * N + c] = acc[r - r0][c - c0];
        }
}

/* quantized_nax.wgsl:264-282 */
void lo_dequantize_nax_int4_sym(const uint32_t* packed, const float* scale, float* out,
                                size_t size, int gs, int coding) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < size; ++i)
        out[i] = (float)nib_at(packed, i, coding) * scale[(i & ~(size_t)7) / (size_t)gs];
}

/* quantized_nax.wgsl:364-386 (symmetric branch, :379) */
void lo_dequantize_nax_int8_group(const uint32_t* packed, const float* scale, float* out,
                                  size_t size, int gs) {
    const int8_t* q = (const int8_t*)packed;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < size; ++i)
        out[i] = (float)q[i] * scale[(i & ~(size_t)3) / (size_t)gs];
}

/* dequantize_nax_int8_group then WGSL_MATMUL (sequential k). */
void lo_matmul_int8_dequant(const int8_t* W, const float* scale, const float* act, float* out,
                            int M, int N, int K, int gs) {
    const int RB = 8, CB = 512;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int r0 = 0; r0 < M; r0 += RB)
        for (int c0 = 0; c0 < N; c0 += CB) {
            int r1 = r0 + RB < M ? r0 + RB : M;
            int c1 = c0 + CB < N ? c0 + CB : N;
            float acc[8][512];
            for (int r = r0; r < r1; ++r)
                for (int c = c0; c < c1; ++c) acc[r - r0][c - c0] = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float* brow = act + (size_t)k * N;
                for (int r = r0; r < r1; ++r) {
                    size_t flat = (size_t)r * K + k;
                    float w = (float)W[flat] * scale[(flat & ~(size_t)3) / (size_t)gs];
                    float* ac = acc[r - r0];
                    for (int c = c0; c < c1; ++c) ac[c - c0] = ac[c - c0] + w * brow[c];
                }
            }
            for (int r = r0; r < r1; ++r)
                for (int c = c0; c < c1; ++c) out[(size_t)r * N + c] = acc[r - r0][c - c0];
        }
}

/* ======================================================================= */
/* Integer matmuls (exact; i32 wrap-around arithmetic as in WGSL)          */
/* ======================================================================= */

/* quantized.wgsl:590-647 */
void lo_matmul_int4_int8(const uint32_t* W, const int8_t* act, int32_t* out, int M, int N, int K,
                         int coding) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        uint32_t* acc = (uint32_t*)calloc((size_t)N, sizeof(uint32_t));
        for (int k = 0; k < K; ++k) {
            int32_t w = nib_at(W, (size_t)r * K + k, coding);
            const int8_t* brow = act + (size_t)k * N;
            for (int c = 0; c < N; ++c) acc[c] += (uint32_t)(w * (int32_t)brow[c]);
        }
        for (int c = 0; c < N; ++c) out[(size_t)r * N + c] = (int32_t)acc[c];
        free(acc);
    }
}

/* quantized.wgsl:497-555 */
void lo_matmul_int8(const int8_t* A, const int8_t* B, int32_t* out, int M, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        uint32_t* acc = (uint32_t*)calloc((size_t)N, sizeof(uint32_t));
        for (int k = 0; k < K; ++k) {
            int32_t a = A[(size_t)r * K + k];
            const int8_t* brow = B + (size_t)k * N;
            for (int c = 0; c < N; ++c) acc[c] += (uint32_t)(a * (int32_t)brow[c]);
        }
        for (int c = 0; c < N; ++c) out[(size_t)r * N + c] = (int32_t)acc[c];
        free(acc);
    }
}

/* WGSL `i32(f32)` saturates out-of-range values; NaN maps to 0 here. */
static inline int32_t f2i_sat(float v) {
    if (v != v) return 0;
    if (v >= 2147483520.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* quantized.wgsl:572-580; round() is round-half-even (rintf under the default mode). */
void lo_requantize_int32_to_int8(const int32_t* in, int32_t* out, size_t n, float in_scale,
                                 float out_scale, int32_t out_zp) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float v = (float)in[i] * in_scale;
        float r = rintf(v / out_scale) + (float)out_zp;
        out[i] = clampi(f2i_sat(r), -128, 127);
    }
}

/* PerChannelScale (quantized.wgsl:51-56): {scale f32, zero_point i32, pad, pad}. */
typedef struct {
    float scale;
    int32_t zero_point;
    uint32_t pad0, pad1;
} lo_channel_scale;

/* quantized.wgsl:264-280 quantize_int8_per_channel: channel = i / channel_stride;
 * quant_type 0 -> quantize_int8_symmetric (:83-86) clamp(i32(round(x / s)), -128, 127),
 * otherwise quantize_int8_asymmetric (:92-95) clamp(i32(round(x / s) + f32(zp)), ...). */
void lo_quantize_int8_per_channel(const float* in, const void* channels, int32_t* out, size_t n,
                                  uint32_t stride, uint32_t quant_type) {
    const lo_channel_scale* ch = (const lo_channel_scale*)channels;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        const lo_channel_scale c = ch[i / stride];
        float r = rintf(in[i] / c.scale);
        if (quant_type != 0) r += (float)c.zero_point;
        out[i] = clampi(f2i_sat(r), -128, 127);
    }
}

/* quantized.wgsl:282-297 dequantize_int8_per_channel: quant_type 0 ->
 * dequantize_int8_symmetric (:88-90) f32(q) * s, otherwise dequantize_int8_asymmetric
 * (:97-99) f32(q - zp) * s, the i32 subtraction wrapping as WGSL's does. */
void lo_dequantize_int8_per_channel(const int32_t* in, const void* channels, float* out, size_t n,
                                    uint32_t stride, uint32_t quant_type) {
    const lo_channel_scale* ch = (const lo_channel_scale*)channels;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        const lo_channel_scale c = ch[i / stride];
        const int32_t q = quant_type != 0 ? (int32_t)((uint32_t)in[i] - (uint32_t)c.zero_point) : in[i];
        out[i] = (float)q * c.scale;
    }
}

void lo_w4a8_group_partials(const uint32_t* W, const int8_t* A, int32_t* P, int M, int N, int K,
                            int gs, int coding) {
    int G = K / gs;
#pragma omp parallel for schedule(static) collapse(2)
    for (int c = 0; c < N; ++c)
        for (int r = 0; r < M; ++r)
            for (int g = 0; g < G; ++g) {
                int64_t s = 0;
                for (int k = g * gs; k < (g + 1) * gs; ++k)
                    s += (int64_t)nib_at(W, (size_t)r * K + k, coding) * A[(size_t)c * K + k];
                P[((size_t)c * M + r) * G + g] = (int32_t)s;
            }
}

/* ======================================================================= */
/* Producers                                                               */
/* ======================================================================= */

/* quantized_nax.wgsl:157-232 */
void lo_compute_group_scales(const float* in, size_t size, int gs, int format, float* scale,
                             int32_t* zero_point, float* gmin, float* gmax) {
    size_t ngroups = (size + (size_t)gs - 1) / (size_t)gs;
#pragma omp parallel for schedule(static)
    for (size_t g = 0; g < ngroups; ++g) {
        size_t start = g * (size_t)gs;
        size_t end = start + (size_t)gs < size ? start + (size_t)gs : size;
        float smax[WG], smin[WG];
        for (int t = 0; t < WG; ++t) {
            float lmax = -1e30f, lmin = 1e30f;
            for (size_t i = start + (size_t)t; i < end; i += WG) {
                lmax = fmaxf(lmax, in[i]);
                lmin = fminf(lmin, in[i]);
            }
            smax[t] = lmax;
            smin[t] = lmin;
        }
        for (int stride = WG / 2; stride > 0; stride >>= 1)
            for (int t = 0; t < stride; ++t) {
                smax[t] = fmaxf(smax[t], smax[t + stride]);
                smin[t] = fminf(smin[t], smin[t + stride]);
            }
        float mx = smax[0], mn = smin[0], s;
        int32_t zp;
        if (format == 0 || format == 2) { /* NAX_INT4_SYM / NAX_INT8_SYM */
            float amax = fmaxf(fabsf(mx), fabsf(mn));
            s = amax / (format == 0 ? 7.0f : 127.0f);
            zp = 0;
        } else { /* asymmetric */
            float range = mx - mn;
            float qmax = format == 1 ? 15.0f : 255.0f;
            s = range / qmax;
            zp = clampi(f2i_sat(rintf(-mn / s)), 0, format == 1 ? 15 : 255);
        }
        if (s == 0.0f) s = 1.0f;
        scale[g] = s;
        if (zero_point) zero_point[g] = zp;
        if (gmin) gmin[g] = mn;
        if (gmax) gmax[g] = mx;
    }
}

/* quantized_nax.wgsl:238-262 */
void lo_quantize_nax_int4_sym(const float* in, size_t size, int gs, const float* scale,
                              uint32_t* packed) {
    size_t nw = (size + 7) / 8;
#pragma omp parallel for schedule(static)
    for (size_t o = 0; o < nw; ++o) {
        size_t e = o * 8;
        float s = scale[e / (size_t)gs];
        int32_t q[8];
        for (int i = 0; i < 8; ++i)
            q[i] = e + i < size ? clampi(f2i_sat(rintf(in[e + i] / s)), -8, 7) : 0;
        packed[o] = lo_pack_int4_ob(q);
    }
}

/* quantized_nax.wgsl:336-362 (NAX_INT8_SYM branch) */
void lo_quantize_nax_int8_group(const float* in, size_t size, int gs, const float* scale,
                                uint32_t* packed) {
    size_t nw = (size + 3) / 4;
#pragma omp parallel for schedule(static)
    for (size_t o = 0; o < nw; ++o) {
        size_t e = o * 4;
        float s = scale[e / (size_t)gs];
        int32_t q[4];
        for (int i = 0; i < 4; ++i)
            q[i] = e + i < size ? clampi(f2i_sat(rintf(in[e + i] / s)), -128, 127) : 0;
        packed[o] = lo_pack_int8x4(q);
    }
}

/* ======================================================================= */
/* GEMM epilogues                                                          */
/* ======================================================================= */

/* steel_gemm_fused.wgsl:80-93 */
static float ep_relu(float x) { return fmaxf(0.0f, x); }
static float ep_gelu(float x) {
    const float c = 0.7978845608f, a = 0.044715f;
    return 0.5f * x * (1.0f + tanhf(c * (x + a * x * x * x)));
}
static float ep_silu(float x) { return x / (1.0f + expf(-x)); }

/* steel_gemm_fused.wgsl:96-127 */
void lo_apply_epilogue(float* y, int m, int n, int kind, const float* bias, const float* residual) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < m; ++r)
        for (int c = 0; c < n; ++c) {
            const size_t i = (size_t)r * n + c;
            float v = y[i];
            switch (kind) {
                case 1: v = ep_relu(v); break;
                case 2: v = ep_gelu(v); break;
                case 3: v = ep_silu(v); break;
                case 4: v = tanhf(v); break;
                case 5: v = 1.0f / (1.0f + expf(-v)); break;
                case 6: v = v + bias[c]; break;
                case 7: v = v + residual[i]; break;
                default: break;
            }
            y[i] = v;
        }
}

/* steel_gemm_fused.wgsl:541-555: silu(gate) * up */
void lo_silu_mul(const float* gu, float* out, int m, int N) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < m; ++r)
        for (int c = 0; c < N; ++c)
            out[(size_t)r * N + c] = ep_silu(gu[(size_t)r * 2 * N + c]) * gu[(size_t)r * 2 * N + N + c];
}

/* rms_norm.wgsl:50-110 */
void lo_rms_norm(const float* x, const float* gamma, float* y, float* rms_out, int rows, int hidden,
                 float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * hidden;
        float sh[WG];
        for (int t = 0; t < WG; ++t) {
            float s = 0.0f;
            for (int i = t; i < hidden; i += WG) s += xr[i] * xr[i];
            sh[t] = s;
        }
        for (int stride = WG / 2; stride > 0; stride >>= 1)
            for (int t = 0; t < stride; ++t) sh[t] += sh[t + stride];
        const float mean_sq = sh[0] / (float)hidden;
        const float rms = 1.0f / sqrtf(mean_sq + eps);
        if (rms_out) rms_out[r] = rms;
        for (int i = 0; i < hidden; ++i) y[(size_t)r * hidden + i] = xr[i] * rms * gamma[i];
    }
}

/* ======================================================================= */
/* fp64 ground truth                                                       */
/* ======================================================================= */

void lo_qmatmul_f64(const void* W, const float* scale, const float* X, double* Y, int n_out,
                    int K, int M, int gs, int wbits, int coding) {
    int G = K / gs;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n_out; ++r) {
        double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
        for (int k = 0; k < K; ++k) {
            size_t flat = (size_t)r * K + k;
            double q = wbits == 4 ? (double)nib_at((const uint32_t*)W, flat, coding)
                                  : (double)((const int8_t*)W)[flat];
            wrow[k] = q * (double)scale[(size_t)r * G + k / gs];
        }
        for (int c = 0; c < M; ++c) {
            double s = 0.0;
            const float* xr = X + (size_t)c * K;
            for (int k = 0; k < K; ++k) s += wrow[k] * (double)xr[k];
            Y[(size_t)c * n_out + r] = s;
        }
        free(wrow);
    }
}
