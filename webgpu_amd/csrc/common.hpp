// Shared device helpers and kernel-launch declarations of libluxgpu_backend_hip.so.
// Every kernel targets gfx950 (CDNA4): wave64, MFMA, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace luxhip {

typedef _Float16 f16;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(16))) int i32x16;

// 16-byte GroupScale of quantized_nax.wgsl:49-54; kernels read .scale only.
struct GroupScale {
    float scale;
    int32_t zero_point;
    float group_min;
    float group_max;
};

enum class ScaleKind : int { None = 0, F16 = 1, F32 = 2, GroupScale = 3 };

// GEMM epilogue kinds: the numbering of apply_epilogue (steel_gemm_fused.wgsl:96-127),
// plus SiluMul, the gated pair of steel_gemm_silu_mul (:452-558).
enum class Epi : int { None = 0, Relu = 1, Gelu = 2, Silu = 3, Tanh = 4, Sigmoid = 5, Bias = 6, Residual = 7, SiluMul = 8 };
struct EpiArgs {
    int kind;                // Epi
    const float* bias;       // [n] for Bias
    const float* residual;   // [m x n] (n = output columns) for Residual
};
enum class XKind : int { F32 = 0, F16 = 1, BF16 = 2, I8 = 32 };
enum class YKind : int { F32 = 0, F16 = 1, BF16 = 2, I32 = 3 };

// rms_norm of the GEMV's activation row computed in the GEMV's own prologue
// (rms_norm.wgsl:50-110 fused ahead of the int4 GEMV).
struct RnArgs {
    const void* x;       // the row before normalisation, XKind xk
    const float* gamma;  // [k]
    float eps;
    int xk;              // XKind::F32, F16 or BF16
};

#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)
__device__ __forceinline__ float load_scale(const void* s, size_t idx, ScaleKind kind) {
    switch (kind) {
        case ScaleKind::F16: return (float)reinterpret_cast<const f16*>(s)[idx];
        case ScaleKind::F32: return reinterpret_cast<const float*>(s)[idx];
        case ScaleKind::GroupScale: return reinterpret_cast<const GroupScale*>(s)[idx].scale;
        default: return 1.0f;
    }
}

template <ScaleKind K>
__device__ __forceinline__ float load_scale_t(const void* s, size_t idx) {
    if constexpr (K == ScaleKind::F16) return (float)reinterpret_cast<const f16*>(s)[idx];
    else if constexpr (K == ScaleKind::F32) return reinterpret_cast<const float*>(s)[idx];
    else if constexpr (K == ScaleKind::GroupScale)
        return reinterpret_cast<const GroupScale*>(s)[idx].scale;
    else return 1.0f;
}

// Raw scale bits, converted only where used (keeps the load off the critical path).
template <ScaleKind K>
__device__ __forceinline__ uint32_t load_scale_raw(const void* s, size_t idx) {
    if constexpr (K == ScaleKind::F16) return reinterpret_cast<const uint16_t*>(s)[idx];
    else if constexpr (K == ScaleKind::F32) return reinterpret_cast<const uint32_t*>(s)[idx];
    else if constexpr (K == ScaleKind::GroupScale) return reinterpret_cast<const uint32_t*>(s)[4 * idx];
    else return 0x3F800000u;
}

template <ScaleKind K>
__device__ __forceinline__ float scale_from_raw(uint32_t b) {
    if constexpr (K == ScaleKind::F16) return (float)__builtin_bit_cast(f16, (uint16_t)b);
    else return __builtin_bit_cast(float, b);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
    return __builtin_bit_cast(float, b << 16);
}

// Cache-policy operand of the buffer-load builtins for data read once (streamed weights):
// the nt bit, which __builtin_nontemporal_load sets on global loads.
constexpr int kNontemporal = 2;

// bfloat16 round-to-nearest-even (NaN kept quiet): the hardware conversion
// (v_cvt_pk_bf16_f32 on gfx950), the same one store_y4 uses.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

template <YKind Y>
__device__ __forceinline__ void store_y(void* y, size_t idx, float v) {
    if constexpr (Y == YKind::F32) reinterpret_cast<float*>(y)[idx] = v;
    else if constexpr (Y == YKind::F16) reinterpret_cast<f16*>(y)[idx] = (f16)v;  // RNE
    else if constexpr (Y == YKind::BF16) reinterpret_cast<uint16_t*>(y)[idx] = f32_to_bf16_bits(v);
    else reinterpret_cast<int32_t*>(y)[idx] = (int32_t)v;
}

// Four consecutive outputs y[idx .. idx+3]; `vec`: one 8- or 16-byte store (the caller
// guarantees alignment and that all four are in range).  bf16 uses the hardware
// round-to-nearest-even conversion (v_cvt_pk_bf16_f32).
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
template <YKind Y>
__device__ __forceinline__ void store_y4(void* y, size_t idx, f32x4 v) {
    if constexpr (Y == YKind::F32) *reinterpret_cast<f32x4*>(static_cast<float*>(y) + idx) = v;
    else if constexpr (Y == YKind::F16)
        *reinterpret_cast<f16x4*>(static_cast<f16*>(y) + idx) = __builtin_convertvector(v, f16x4);
    else if constexpr (Y == YKind::BF16)
        *reinterpret_cast<bf16x4*>(static_cast<uint16_t*>(y) + idx) = __builtin_convertvector(v, bf16x4);
    else {
#pragma unroll
        for (int r = 0; r < 4; ++r) store_y<Y>(y, idx + r, v[r]);
    }
}

// silu(x) = x / (1 + exp(-x)) (steel_gemm_fused.wgsl:90-93)
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// apply_epilogue (steel_gemm_fused.wgsl:80-127) for output (m, n) of a [M x ny] result;
// the kind is uniform across the launch, so the switch does not diverge.
__device__ __forceinline__ float apply_epi(float x, const EpiArgs& e, int m, int n, int ny) {
    switch (e.kind) {
        case 1: return fmaxf(0.0f, x);
        case 2: return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
        case 3: return silu_f(x);
        case 4: return tanhf(x);
        case 5: return 1.0f / (1.0f + expf(-x));
        case 6: return x + e.bias[n];
        case 7: return x + e.residual[(size_t)m * ny + n];
        default: return x;
    }
}

template <XKind X>
__device__ __forceinline__ float load_x(const void* x, size_t idx) {
    if constexpr (X == XKind::F32) return reinterpret_cast<const float*>(x)[idx];
    else if constexpr (X == XKind::F16) return (float)reinterpret_cast<const f16*>(x)[idx];
    else if constexpr (X == XKind::BF16)
        return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(x)[idx]);
    else return (float)reinterpret_cast<const int8_t*>(x)[idx];
}

// Max / min across the 64 lanes with the DPP pattern of wave_sum (below); rows outside a step's row
// mask compare a lane with itself, so the operation only needs to be idempotent.  Every
// lane gets the result (lane 63's, read back as a uniform value).  Replaces six dependent
// ds_bpermute round trips of a __shfl_xor butterfly.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ int dpp_self(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROWMASK, 0xF, false);
}
template <typename Op>
__device__ __forceinline__ int wave_idem(int v, Op op) {
    v = op(v, dpp_self<0xB1, 0xF>(v));
    v = op(v, dpp_self<0x4E, 0xF>(v));
    v = op(v, dpp_self<0x141, 0xF>(v));
    v = op(v, dpp_self<0x140, 0xF>(v));
    v = op(v, dpp_self<0x142, 0xA>(v));
    v = op(v, dpp_self<0x143, 0xC>(v));
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return (uint32_t)wave_idem((int)v, [](int a, int b) { return (int)max((uint32_t)a, (uint32_t)b); });
}
__device__ __forceinline__ float wave_max_f32(float v) {
    return __builtin_bit_cast(float, wave_idem(__builtin_bit_cast(int, v), [](int a, int b) {
        return __builtin_bit_cast(int, fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)));
    }));
}
__device__ __forceinline__ float wave_min_f32(float v) {
    return __builtin_bit_cast(float, wave_idem(__builtin_bit_cast(int, v), [](int a, int b) {
        return __builtin_bit_cast(int, fminf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)));
    }));
}

// ---- fp16 staging of wide activations ---------------------------------------
// Kernels that feed bf16 / fp32 activations to fp16 MFMAs scale each activation row by
// a power of two first: fac = 2^(E - 14) with 2^E <= max|x| < 2^(E+1), so x / fac has
// its maximum in [2^14, 2^15), inside fp16's normal range (max 65504); dividing by fac
// and multiplying the row's output by fac are exact.  Rows that are all zero or
// subnormal, or that hold Inf/NaN, keep fac = 1 (an Inf/NaN input then propagates).
// `mx` is the largest |x| bit pattern of the row (sign cleared) and `mant` the
// mantissa width of the source type (7 for bf16, 23 for fp32).
__device__ __forceinline__ float row_pow2_factor(uint32_t mx, int mant) {
    const int ex = (int)((mx >> mant) & 0xFFu);
    if (ex == 0 || ex == 0xFF) return 1.0f;
    return ldexpf(1.0f, max(ex - 141, -126));
}

// ---- fp16 staging of dequantised int4 weights ------------------------------------
// Kernels that stage q * s as fp16 for fp16 MFMAs (q in [-8, 7]) first divide the scales
// of each weight row by a power of two, fold = 2^(E - 11) with 2^E <= max_g |s(n, g)| <
// 2^(E+1): the row's largest |s / fold| lies in [2^11, 2^12), so |q * s / fold| <= 2^15
// stays inside fp16's normal range for any finite scale (fp32 scales of any exponent,
// fp16 scales up to 65504), and groups down to 2^-25 of the row maximum keep full fp16
// precision.  The product is rounded to fp16 once; the epilogue multiplies the row's
// fp32 sum by fold (exact).  Rows whose scales are all zero, or hold Inf/NaN, keep
// fold = 1 (Inf/NaN then propagate as in the reference's f32(q) * s).  `mx` is the
// largest |s| of the row as binary32 bits (sign cleared).
__device__ __forceinline__ float scale_fold_factor(uint32_t mx) {
    if (mx == 0 || mx >= 0x7F800000u) return 1.0f;
    const int ex = (int)(mx >> 23);  // 0 for a binary32 subnormal maximum
    return ldexpf(1.0f, max(ex - 127 - 11, -126));
}

// |s| as binary32 bits from a raw scale word of load_scale_raw.
template <ScaleKind K>
__device__ __forceinline__ uint32_t scale_abs_bits(uint32_t raw) {
    return __builtin_bit_cast(uint32_t, scale_from_raw<K>(raw)) & 0x7FFFFFFFu;
}

// fold[row] of the G scales of one weight row, computed by one wave.
template <ScaleKind K>
__device__ __forceinline__ float row_scale_fold(const void* s, size_t row, int G, int lane) {
    uint32_t mx = 0;
    int g = lane;
    for (; g + 192 < G; g += 256) {  // four independent loads per lane per trip
        const uint32_t a = load_scale_raw<K>(s, row * G + g), b = load_scale_raw<K>(s, row * G + g + 64);
        const uint32_t c = load_scale_raw<K>(s, row * G + g + 128), d = load_scale_raw<K>(s, row * G + g + 192);
        mx = max(mx, max(max(scale_abs_bits<K>(a), scale_abs_bits<K>(b)), max(scale_abs_bits<K>(c), scale_abs_bits<K>(d))));
    }
    for (; g < G; g += 64) mx = max(mx, scale_abs_bits<K>(load_scale_raw<K>(s, row * G + g)));
    mx = wave_max_u32(mx);
    // A NaN scale compares above every finite value and Inf as bits, so it also keeps fold = 1.
    return scale_fold_factor(mx);
}

// Product q * s in fp32 (exact to binary32 rounding), then one RNE rounding to fp16, for
// one u32 of 8 offset-binary nibbles (k .. k+7), in the staging order
// (k, k+4, k+1, k+5, k+2, k+6, k+3, k+7).
__device__ __forceinline__ u32x4 dequant8_f32s(uint32_t w, float s) {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = (float)((int)((w >> (4 * i)) & 0xFu) - 8) * s;
        const float b = (float)((int)((w >> (4 * i + 16)) & 0xFu) - 8) * s;
        o[i] = __builtin_bit_cast(uint32_t, f16x2{(f16)a, (f16)b});
    }
    return u32x4{o[0], o[1], o[2], o[3]};
}

// Block-wide max of a per-thread value; `red` is __shared__ scratch of >= 16 words.
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
    v = wave_max_u32(v);
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wv] = v;
    __syncthreads();
    uint32_t r = 0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r = max(r, red[i]);
    __syncthreads();
    return r;
}

// One DPP step: v + (v as seen through the lane pattern CTRL), rows outside ROWMASK add 0.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xF, false);
    return v + __builtin_bit_cast(float, t);
}

// Sum across the 64 lanes of a wave; every lane gets the total.  VALU-only DPP steps
// (quad_perm xor 1 and xor 2, half-row mirror, row mirror, row_bcast:15 into rows 1/3,
// row_bcast:31 into rows 2/3) leave the total in lane 63, which is read back as a
// uniform value: no LDS round trips on the critical path.
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0xB1, 0xF>(v);
    v = dpp_add<0x4E, 0xF>(v);
    v = dpp_add<0x141, 0xF>(v);
    v = dpp_add<0x140, 0xF>(v);
    v = dpp_add<0x142, 0xA>(v);
    v = dpp_add<0x143, 0xC>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

#endif

// ---------------------------------------------------------------------------
// Launchers (host side).  Plain pointers and sizes; shapes are validated by the
// caller in plugin.hip before any launch, so every grid below stays in bounds.
// ---------------------------------------------------------------------------
// Compute units of the current device, cached per device (host code).
inline int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

struct QArgs {
    const void* w;        // packed weights
    const void* s;        // weight scales (may be null for ScaleKind::None)
    const void* x;        // activations [m x k]
    const float* xs;      // per-token activation scales [m] (W4A8) or null
    void* y;              // output [m x n_out]
    int n_out, k, m;
    int group_size;
    int wbits;            // 4 or 8
    uint32_t xor_mask;    // 0x88888888 turns two's-complement nibbles into offset-binary
    const float* xfac;    // per-row power-of-two factors of staged activations (set by launchers)
    const float* wfold;   // per-weight-row scale folds of fp16-staged int4 weights (set by launchers)
    ScaleKind scale_kind;
    XKind x_kind;
    YKind y_kind;
    bool group_partials;  // W4A8: write P[m][n][g]
    EpiArgs epi;          // output epilogue; SiluMul: n_out = 2 * (output columns),
                          // weight rows [0, n_out/2) gate and [n_out/2, n_out) up
    RnArgs rn;            // rn.gamma != null: x is rms_norm(rn.x) rounded to fp16, computed by the
                          // GEMV itself (m = 1 int4 fast path only; a.x is unused)
};

hipError_t launch_gemv_f32(const float* A, const float* x, float* y, int M, int K, int lda,
                           float alpha, float beta, hipStream_t s);
hipError_t launch_gemv_f32_batched(const float* A, const float* x, float* y, int M, int K, int lda,
                                   float alpha, float beta, int batch, size_t sa, size_t sx,
                                   size_t sy, hipStream_t s);
hipError_t launch_gemv_f32_t(const float* A, const float* x, float* y, int M, int N, int lda,
                             float alpha, float beta, float* workspace, hipStream_t s);
size_t gemv_t_workspace(int M, int N);  // bytes of the transposed GEMV's partial sums
hipError_t launch_gemm_f32(const float* A, const float* B, float* C, int M, int K, int N,
                           hipStream_t s);
hipError_t launch_dot_f16(const void* a, const void* b, float* out, int size, int nv, size_t stride,
                          hipStream_t s);
hipError_t launch_gemv_f16(const void* A, const void* x, float* y, int M, int K, int lda,
                           hipStream_t s);
// int4 weight-only GEMV, m == 1.
bool qgemv_i4_fast(const QArgs& a);  // the m = 1 int4 GEMV fast path applies (SiluMul needs it)
hipError_t launch_qgemv_i4(const QArgs& a, hipStream_t s);
// The GEMV can normalise its own activation row (a.rn): m = 1, int4, fp16 scales, k <= 8192.
bool qgemv_i4_rn_supported(const QArgs& a);
// Per-weight-row scale folds (scale_fold_factor) of int4 weights staged as fp16:
// fold[n] for n < n_out, one wave per row.
hipError_t launch_scale_fold(const void* s, ScaleKind sk, int n_out, int groups, float* fold, hipStream_t st);
// Weight-only int4/int8 matmul for small m (bandwidth regime), fp16/bf16/f32 X.
bool qgemm_small_supported(const QArgs& a);
// workspace: qgemm_small_workspace(a) bytes (int4: per-row scale folds; bf16/f32 X:
// per-row activation factors; 0 for int8 weights with fp16 X), 16-byte aligned
size_t qgemm_small_workspace(const QArgs& a);
hipError_t launch_qgemm_small(const QArgs& a, void* workspace, hipStream_t s);
// int4 grouped GEMM for large m (MFMA regime).  Needs a device workspace of
// qgemm_i4_large_workspace(a) bytes (X restaged as fp16), 16-byte aligned.
bool qgemm_i4_large_supported(const QArgs& a);
size_t qgemm_i4_large_workspace(const QArgs& a);
hipError_t launch_qgemm_i4_large(const QArgs& a, void* workspace, hipStream_t s);
// W4A8 integer MFMA.
bool w4a8_supported(const QArgs& a);
hipError_t launch_w4a8(const QArgs& a, hipStream_t s);

// Elementwise f32 ops of the ABI tensor slots: op 0 add, 1 sub, 2 mul, 3 div.
hipError_t launch_binary_f32(int op, const float* a, const float* b, float* out, size_t n, hipStream_t s);
hipError_t launch_fill_f32(float* out, size_t n, float v, hipStream_t s);
// RMS normalisation of rows x hidden (rms_norm.wgsl); rms_out may be null.
hipError_t launch_rms_norm(const void* x, XKind xk, const float* gamma, void* y, YKind yk, float* rms_out, int rows,
                           int hidden, float eps, hipStream_t s);

// Symmetric group quantizer (scales + packed values) over X [rows x k].
struct QuantArgs {
    const void* x;        // [rows x k], x_kind
    void* q;              // packed int4 (u32 words) or int8
    void* s;              // scales [rows x k / group_size], scale_kind
    int rows, k, group_size;  // group_size: a power of two >= 8 dividing k
    int bits;             // 4 or 8
    bool offset_binary;   // int4 nibble coding of q
    ScaleKind scale_kind;
    XKind x_kind;
};
hipError_t launch_quantize(const QuantArgs& a, hipStream_t s);
// out [rows x k] (x_kind F32/F16/BF16) = q * s: the inverse of launch_quantize (x unused).
hipError_t launch_dequantize(const QuantArgs& a, void* out, hipStream_t s);
// out[i] = in[i] ^ mask over `words` u32 words (nibble re-coding; in == out allowed).
hipError_t launch_xor_words(const void* in, void* out, size_t words, uint32_t mask, hipStream_t s);
hipError_t launch_convert_scales(const void* in, ScaleKind ik, void* out, ScaleKind ok, size_t n, hipStream_t s);
// PerChannelScale of quantized.wgsl:51-56.
struct ChannelScale {
    float scale;
    int32_t zero_point;
    uint32_t pad0, pad1;
};
// quantize_int8_per_channel (f32 -> i32) or dequantize_int8_per_channel (i32 -> f32),
// quantized.wgsl:264-297; asym: quant_type != 0.  Buffers 4-byte aligned.
hipError_t launch_int8_per_channel(bool dequantize, const void* in, const ChannelScale* ch, void* out, size_t n,
                                  uint32_t stride, bool asym, hipStream_t s);
hipError_t launch_requantize(const int32_t* in, int32_t* out, size_t n, float s_in, float s_out, int32_t zp,
                             hipStream_t s);

}  // namespace luxhip
