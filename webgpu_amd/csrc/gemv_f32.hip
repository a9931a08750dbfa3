// fp32 / fp16 GEMV and the fp32 GEMM behind op_matmul_f32.
//
// Reference semantics: gemv.wgsl:49-96 (gemv_row_parallel: y = alpha*A.x + beta*y),
// gemv.wgsl:103-149 (gemv_transpose), fp_quantized.wgsl:418-469 (fp16 products with
// fp32 accumulation) and WGSL_MATMUL (src/webgpu_plugin.cpp:138-205).  The sums are
// reassociated (wave-wide partials instead of 256 strided lanes), which changes
// rounding only.
#include "common.hpp"

namespace luxhip {

// One wave per row; each lane streams 16-byte chunks of the row (HBM-bound:
// 4 B of A per multiply-add).  Four independent chunks per iteration keep 4 KB
// per wave in flight.
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemv_f32(const float* __restrict__ A,
                                                  const float* __restrict__ x,
                                                  float* __restrict__ y, int M, int K, int lda,
                                                  float alpha, float beta) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const float* a = A + (size_t)row * lda;
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
    if constexpr (VEC) {
        const f32x4* a4 = reinterpret_cast<const f32x4*>(a);
        const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
        const int K4 = K >> 2;
        int i = lane;
        for (; i + 192 < K4; i += 256) {
            f32x4 v0 = __builtin_nontemporal_load(a4 + i);
            f32x4 v1 = __builtin_nontemporal_load(a4 + i + 64);
            f32x4 v2 = __builtin_nontemporal_load(a4 + i + 128);
            f32x4 v3 = __builtin_nontemporal_load(a4 + i + 192);
            f32x4 u0 = x4[i], u1 = x4[i + 64], u2 = x4[i + 128], u3 = x4[i + 192];
            acc0 = fmaf(v0.x, u0.x, acc0); acc0 = fmaf(v0.y, u0.y, acc0);
            acc0 = fmaf(v0.z, u0.z, acc0); acc0 = fmaf(v0.w, u0.w, acc0);
            acc1 = fmaf(v1.x, u1.x, acc1); acc1 = fmaf(v1.y, u1.y, acc1);
            acc1 = fmaf(v1.z, u1.z, acc1); acc1 = fmaf(v1.w, u1.w, acc1);
            acc2 = fmaf(v2.x, u2.x, acc2); acc2 = fmaf(v2.y, u2.y, acc2);
            acc2 = fmaf(v2.z, u2.z, acc2); acc2 = fmaf(v2.w, u2.w, acc2);
            acc3 = fmaf(v3.x, u3.x, acc3); acc3 = fmaf(v3.y, u3.y, acc3);
            acc3 = fmaf(v3.z, u3.z, acc3); acc3 = fmaf(v3.w, u3.w, acc3);
        }
        for (; i < K4; i += 64) {
            f32x4 v = __builtin_nontemporal_load(a4 + i);
            f32x4 u = x4[i];
            acc0 = fmaf(v.x, u.x, acc0); acc0 = fmaf(v.y, u.y, acc0);
            acc0 = fmaf(v.z, u.z, acc0); acc0 = fmaf(v.w, u.w, acc0);
        }
        for (int k = (K4 << 2) + lane; k < K; k += 64) acc1 = fmaf(a[k], x[k], acc1);
    } else {
        for (int k = lane; k < K; k += 64) acc0 = fmaf(a[k], x[k], acc0);
    }
    float s = wave_sum((acc0 + acc1) + (acc2 + acc3));
    if (lane == 0) {
        float r = alpha * s;
        if (beta != 0.f) r = fmaf(beta, y[row], r);  // y untouched when beta == 0
        y[row] = r;
    }
}

// y[n] = alpha * sum_r A[r, n] x[r] + beta*y[n]: lanes own columns (coalesced),
// the 4 waves of a block split the rows, partials meet in LDS.
__global__ __launch_bounds__(256) void k_gemv_f32_t(const float* __restrict__ A,
                                                    const float* __restrict__ x,
                                                    float* __restrict__ y, int M, int N,
                                                    int lda, float alpha, float beta) {
    __shared__ float part[4][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + lane;
    float acc = 0.f;
    if (col < N) {
        const int per = (M + 3) / 4;
        const int r0 = wv * per, r1 = min(M, r0 + per);
        for (int r = r0; r < r1; ++r) acc = fmaf(A[(size_t)r * lda + col], x[r], acc);
    }
    part[wv][lane] = acc;
    __syncthreads();
    if (wv == 0 && col < N) {
        float s = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
        float r = alpha * s;
        if (beta != 0.f) r = fmaf(beta, y[col], r);
        y[col] = r;
    }
}

// General fp32 GEMM C[M x N] = A[M x K] B[K x N] (row-major): 64x64 tile per
// 256-thread block, 4x4 outputs per thread, K staged 16 at a time through LDS.
__global__ __launch_bounds__(256) void k_gemm_f32(const float* __restrict__ A,
                                                  const float* __restrict__ B,
                                                  float* __restrict__ C, int M, int K, int N) {
    __shared__ float sa[16][64 + 4];  // [k][m]
    __shared__ float sb[16][64 + 4];  // [k][n]
    const int tid = threadIdx.x;
    const int tm = (tid >> 4) * 4, tn = (tid & 15) * 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += 16) {
        for (int i = tid; i < 64 * 16; i += 256) {
            int r = i >> 4, c = i & 15;  // A tile: row r, k c
            int gr = m0 + r, gk = k0 + c;
            sa[c][r] = (gr < M && gk < K) ? A[(size_t)gr * K + gk] : 0.f;
            int kr = i >> 6, nc = i & 63;  // B tile: k kr, col nc
            int bk = k0 + kr, bn = n0 + nc;
            sb[kr][nc] = (bk < K && bn < N) ? B[(size_t)bk * N + bn] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { av[i] = sa[kk][tm + i]; bv[i] = sb[kk][tn + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int r = m0 + tm + i, c = n0 + tn + j;
            if (r < M && c < N) C[(size_t)r * N + c] = acc[i][j];
        }
}

// fp16 GEMV, fp32 accumulation: one wave per row, 16-byte chunks (8 halves),
// v_dot2_f32_f16 on each pair (exact fp16 x fp16 products).
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemv_f16(const f16* __restrict__ A,
                                                  const f16* __restrict__ x,
                                                  float* __restrict__ y, int M, int K, int lda) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const f16* a = A + (size_t)row * lda;
    float acc0 = 0.f, acc1 = 0.f;
    if constexpr (VEC) {
        const f16x8* a8 = reinterpret_cast<const f16x8*>(a);
        const f16x8* x8 = reinterpret_cast<const f16x8*>(x);
        const int K8 = K >> 3;
        for (int i = lane; i < K8; i += 64) {
            f16x8 v = __builtin_nontemporal_load(a8 + i);
            f16x8 u = x8[i];
            acc0 = __builtin_amdgcn_fdot2(f16x2{v[0], v[1]}, f16x2{u[0], u[1]}, acc0, false);
            acc1 = __builtin_amdgcn_fdot2(f16x2{v[2], v[3]}, f16x2{u[2], u[3]}, acc1, false);
            acc0 = __builtin_amdgcn_fdot2(f16x2{v[4], v[5]}, f16x2{u[4], u[5]}, acc0, false);
            acc1 = __builtin_amdgcn_fdot2(f16x2{v[6], v[7]}, f16x2{u[6], u[7]}, acc1, false);
        }
        for (int k = (K8 << 3) + lane; k < K; k += 64) acc0 = fmaf((float)a[k], (float)x[k], acc0);
    } else {
        for (int k = lane; k < K; k += 64) acc0 = fmaf((float)a[k], (float)x[k], acc0);
    }
    float s = wave_sum(acc0 + acc1);
    if (lane == 0) y[row] = s;
}

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t launch_gemv_f32(const float* A, const float* x, float* y, int M, int K, int lda,
                           float alpha, float beta, hipStream_t s) {
    dim3 grid((M + 3) / 4), block(256);
    bool vec = (lda % 4 == 0) && aligned16(A) && aligned16(x);
    if (vec)
        hipLaunchKernelGGL(k_gemv_f32<true>, grid, block, 0, s, A, x, y, M, K, lda, alpha, beta);
    else
        hipLaunchKernelGGL(k_gemv_f32<false>, grid, block, 0, s, A, x, y, M, K, lda, alpha, beta);
    return hipGetLastError();
}

hipError_t launch_gemv_f32_t(const float* A, const float* x, float* y, int M, int N, int lda,
                             float alpha, float beta, hipStream_t s) {
    hipLaunchKernelGGL(k_gemv_f32_t, dim3((N + 63) / 64), dim3(256), 0, s, A, x, y, M, N, lda,
                       alpha, beta);
    return hipGetLastError();
}

hipError_t launch_gemm_f32(const float* A, const float* B, float* C, int M, int K, int N,
                           hipStream_t s) {
    hipLaunchKernelGGL(k_gemm_f32, dim3((N + 63) / 64, (M + 63) / 64), dim3(256), 0, s, A, B, C,
                       M, K, N);
    return hipGetLastError();
}

hipError_t launch_gemv_f16(const void* A, const void* x, float* y, int M, int K, int lda,
                           hipStream_t s) {
    dim3 grid((M + 3) / 4), block(256);
    bool vec = (lda % 8 == 0) && aligned16(A) && aligned16(x);
    const f16* a = reinterpret_cast<const f16*>(A);
    const f16* xv = reinterpret_cast<const f16*>(x);
    if (vec) hipLaunchKernelGGL(k_gemv_f16<true>, grid, block, 0, s, a, xv, y, M, K, lda);
    else hipLaunchKernelGGL(k_gemv_f16<false>, grid, block, 0, s, a, xv, y, M, K, lda);
    return hipGetLastError();
}

}  // namespace luxhip
