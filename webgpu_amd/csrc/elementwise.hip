// ABI-v3 tensor slots around the matmul path, and RMS normalisation.
//
// Reference:
//   op_add_f32 / op_sub_f32 / op_mul_f32  src/webgpu_plugin.cpp:1637-1719 with the
//       WGSL_BINARY_OPS shader (:92-135): out[i] = a[i] op b[i], strides 1, n elements.
//   op_div_f32  stubbed NOT_SUPPORTED in the reference (:3548); here the same
//       elementwise form with IEEE division.
//   rms_norm    kernels/wgsl/gpu/rms_norm.wgsl:25-110 (no bridge in the reference):
//       y = x * (1 / sqrt(mean(x^2) + eps)) * gamma[i] per row, rms_out[row] = that
//       reciprocal.
// All HBM-bound.  The binary ops move 16 bytes per lane per operand; rms_norm gives
// each row to one 256-thread block, keeps the row in registers between the
// sum-of-squares and the scaling, and reduces with DPP steps plus one LDS exchange.
#include "common.hpp"

namespace luxhip {

template <int OP>
__device__ __forceinline__ float bop(float a, float b) {
    if constexpr (OP == 0) return a + b;
    else if constexpr (OP == 1) return a - b;
    else if constexpr (OP == 2) return a * b;
    else return a / b;
}

template <int OP>
__global__ __launch_bounds__(256) void k_binary_f32(const float* __restrict__ a, const float* __restrict__ b,
                                                    float* __restrict__ out, size_t n) {
    const size_t n4 = n / 4;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        const f32x4 x = reinterpret_cast<const f32x4*>(a)[i], y = reinterpret_cast<const f32x4*>(b)[i];
        reinterpret_cast<f32x4*>(out)[i] = f32x4{bop<OP>(x[0], y[0]), bop<OP>(x[1], y[1]),
                                                 bop<OP>(x[2], y[2]), bop<OP>(x[3], y[3])};
    }
    const size_t t = 4 * n4 + (size_t)blockIdx.x * 256 + threadIdx.x;  // the last n % 4
    if (blockIdx.x == 0 && t < n) out[t] = bop<OP>(a[t], b[t]);
}

// Scalar form for buffers that are not 16-byte aligned.
template <int OP>
__global__ __launch_bounds__(256) void k_binary_f32_s(const float* __restrict__ a, const float* __restrict__ b,
                                                      float* __restrict__ out, size_t n) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = bop<OP>(a[i], b[i]);
}

static int grid_for(size_t items) {
    const size_t b = (items + 255) / 256;
    return (int)(b < 8192 ? (b ? b : 1) : 8192);  // grid-stride beyond 2M items
}

template <int OP>
static hipError_t launch_op(const float* a, const float* b, float* out, size_t n, hipStream_t s) {
    if ((((uintptr_t)a | (uintptr_t)b | (uintptr_t)out) & 15u) == 0)
        hipLaunchKernelGGL((k_binary_f32<OP>), dim3(grid_for(n / 4 ? n / 4 : 1)), dim3(256), 0, s, a, b, out, n);
    else
        hipLaunchKernelGGL((k_binary_f32_s<OP>), dim3(grid_for(n)), dim3(256), 0, s, a, b, out, n);
    return hipGetLastError();
}

hipError_t launch_binary_f32(int op, const float* a, const float* b, float* out, size_t n, hipStream_t s) {
    switch (op) {
        case 0: return launch_op<0>(a, b, out, n, s);
        case 1: return launch_op<1>(a, b, out, n, s);
        case 2: return launch_op<2>(a, b, out, n, s);
        case 3: return launch_op<3>(a, b, out, n, s);
        default: return hipErrorInvalidValue;
    }
}

__global__ __launch_bounds__(256) void k_fill_f32(float* __restrict__ out, size_t n, float v) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = v;
}

// A fill kernel rather than hipMemsetAsync, so that callers may capture it in a graph.
hipError_t launch_fill_f32(float* out, size_t n, float v, hipStream_t s) {
    hipLaunchKernelGGL(k_fill_f32, dim3(grid_for(n)), dim3(256), 0, s, out, n, v);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------- rms_norm
constexpr int RN_VPT = 16;  // elements per thread kept in registers (hidden <= 4096)

template <XKind XK, YKind YK>
__global__ __launch_bounds__(256) void k_rms_norm(const void* __restrict__ X, const float* __restrict__ gamma,
                                                  void* __restrict__ Y, float* __restrict__ rms_out, int hidden,
                                                  float eps) {
    __shared__ float part[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const size_t base = (size_t)row * hidden;
    float v[RN_VPT];
    float ss = 0.0f;
    const bool in_regs = hidden <= 256 * RN_VPT;
    if (in_regs) {
#pragma unroll
        for (int j = 0; j < RN_VPT; ++j) {
            const int i = tid + 256 * j;
            v[j] = i < hidden ? load_x<XK>(X, base + i) : 0.0f;
            ss = fmaf(v[j], v[j], ss);
        }
    } else {
        for (int i = tid; i < hidden; i += 256) {
            const float x = load_x<XK>(X, base + i);
            ss = fmaf(x, x, ss);
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float mean_sq = ((part[0] + part[1]) + (part[2] + part[3])) / (float)hidden;
    const float rms = 1.0f / sqrtf(mean_sq + eps);
    if (tid == 0 && rms_out) rms_out[row] = rms;
    if (in_regs) {
#pragma unroll
        for (int j = 0; j < RN_VPT; ++j) {
            const int i = tid + 256 * j;
            if (i < hidden) store_y<YK>(Y, base + i, v[j] * rms * gamma[i]);
        }
    } else {
        for (int i = tid; i < hidden; i += 256) store_y<YK>(Y, base + i, load_x<XK>(X, base + i) * rms * gamma[i]);
    }
}

template <XKind XK>
static hipError_t launch_rn_y(const void* x, const float* g, void* y, float* r, int rows, int hidden, float eps,
                              YKind yk, hipStream_t s) {
    const dim3 grid(rows), block(256);
    switch (yk) {
        case YKind::F32: hipLaunchKernelGGL((k_rms_norm<XK, YKind::F32>), grid, block, 0, s, x, g, y, r, hidden, eps); break;
        case YKind::F16: hipLaunchKernelGGL((k_rms_norm<XK, YKind::F16>), grid, block, 0, s, x, g, y, r, hidden, eps); break;
        case YKind::BF16: hipLaunchKernelGGL((k_rms_norm<XK, YKind::BF16>), grid, block, 0, s, x, g, y, r, hidden, eps); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rms_norm(const void* x, XKind xk, const float* gamma, void* y, YKind yk, float* rms_out, int rows,
                           int hidden, float eps, hipStream_t s) {
    switch (xk) {
        case XKind::F32: return launch_rn_y<XKind::F32>(x, gamma, y, rms_out, rows, hidden, eps, yk, s);
        case XKind::F16: return launch_rn_y<XKind::F16>(x, gamma, y, rms_out, rows, hidden, eps, yk, s);
        case XKind::BF16: return launch_rn_y<XKind::BF16>(x, gamma, y, rms_out, rows, hidden, eps, yk, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace luxhip
