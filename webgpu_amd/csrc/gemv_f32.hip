// fp32 / fp16 GEMV and the fp32 GEMM behind op_matmul_f32.
//
// Reference semantics: gemv.wgsl:49-96 (gemv_row_parallel: y = alpha*A.x + beta*y),
// gemv.wgsl:103-149 (gemv_transpose), gemv.wgsl:297-354 (gemv_batched),
// fp_quantized.wgsl:418-469 (fp16 products with fp32 accumulation: the batched dot as
// written, and a GEMV with a shared x) and WGSL_MATMUL (src/webgpu_plugin.cpp:138-205).
// The sums are reassociated (wave-wide partials instead of 256 strided lanes), which
// changes rounding only.
#include <algorithm>

#include "common.hpp"

namespace luxhip {

// One wave per row; each lane streams 16-byte chunks of the row (HBM-bound:
// 4 B of A per multiply-add).  Four independent chunks per iteration keep 4 KB
// per wave in flight.  Returns the wave's dot product (wave-uniform).
template <bool VEC>
__device__ __forceinline__ float gemv_dot(const float* __restrict__ a, const float* __restrict__ x, int K) {
    const int lane = threadIdx.x & 63;
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
    return wave_sum((acc0 + acc1) + (acc2 + acc3));
}

__device__ __forceinline__ void gemv_store(float* yr, float s, float alpha, float beta) {
    float r = alpha * s;
    if (beta != 0.f) r = fmaf(beta, *yr, r);  // y untouched when beta == 0
    *yr = r;
}

// MODE 0: one GEMV, row = blockIdx.x*4 + wave.  MODE 1: batch b = blockIdx.y.  MODE 2
// strides rows and batches over the grid, for shapes beyond its limits (more than 2^22
// rows or 65535 batches).  MODE 3: one GEMV with each row split between two waves
// (K halves, 16-B aligned) whose sums meet in LDS: twice the waves for the same bytes,
// for matrices with few rows (4096 x 4096: 11.5 us against 12.0 us).  The batch
// arithmetic alone costs ~1.5 % on a 4096 x 4096 GEMV and the loops ~4 %, so each form
// is only used where needed.
template <bool VEC, int MODE>
__global__ __launch_bounds__(256) void k_gemv_f32(const float* __restrict__ A,
                                                  const float* __restrict__ x,
                                                  float* __restrict__ y, int M, int K, int lda,
                                                  float alpha, float beta, int batch, size_t sa,
                                                  size_t sx, size_t sy) {
    const unsigned wv = threadIdx.x >> 6;
    const bool lead = (threadIdx.x & 63) == 0;
    if constexpr (MODE == 0) {
        const int row = blockIdx.x * 4 + wv;
        if (row >= M) return;
        const float d = gemv_dot<VEC>(A + (size_t)row * lda, x, K);
        if (lead) gemv_store(y + row, d, alpha, beta);
    } else if constexpr (MODE == 1) {
        const unsigned row = blockIdx.x * 4 + wv, b = blockIdx.y;
        if (row >= (unsigned)M) return;
        const float d = gemv_dot<VEC>(A + b * sa + (size_t)row * lda, x + b * sx, K);
        if (lead) gemv_store(y + b * sy + row, d, alpha, beta);
    } else if constexpr (MODE == 2) {
        // Unsigned counters: M and batch are at most INT32_MAX and the steps at most
        // 2^22, so neither wraps before its loop ends.
        for (unsigned b = blockIdx.y; b < (unsigned)batch; b += gridDim.y)
            for (unsigned row = blockIdx.x * 4 + wv; row < (unsigned)M; row += gridDim.x * 4) {
                const float d = gemv_dot<VEC>(A + b * sa + (size_t)row * lda, x + b * sx, K);
                if (lead) gemv_store(y + b * sy + row, d, alpha, beta);
            }
    } else {
        __shared__ float part[4];
        const int row = blockIdx.x * 2 + (wv >> 1), half = wv & 1;
        const int k1 = ((K >> 2) + 1) / 2 * 4;  // first half: a multiple of 4 floats
        const int lo = half ? k1 : 0, len = half ? K - k1 : k1;
        float d = 0.f;
        if (row < M) d = gemv_dot<VEC>(A + (size_t)row * lda + lo, x + lo, len);
        if (lead) part[wv] = d;
        __syncthreads();
        if (lead && !half && row < M) gemv_store(y + row, part[wv] + part[wv + 1], alpha, beta);
    }
}

// Few rows of fp32 (the config-1 shape, 4096 x 4096): each row splits into KS parts of
// k and each wave owns RW rows of one part, CPL 16-byte chunks per lane and row, with the
// next D rows' loads in flight while it computes a row.  The parts' sums meet in LDS and
// are added in k order.  Needs K / 4 = 64 * KS * CPL chunks and the vector layout.
// Measured at 4096 x 4096 (lab, same process): 16 rows per wave in 1,024 waves 11.14 us,
// 8 rows in 2,048 waves 11.26 us, 32 rows 12.4 us; one or three rows ahead instead of two
// within 0.2 %.
template <int RW, int KS, int CPL, int D = 2>
__global__ __launch_bounds__(256) void k_gemv_f32_parts(const float* __restrict__ A, const float* __restrict__ x,
                                                        float* __restrict__ y, int M, int K, int lda, float alpha,
                                                        float beta) {
    constexpr int RS = 4 / KS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * RS + wave % RS) * RW, kp = wave / RS;
    const int nrows = min(RW, M - row0);
    const int c0 = kp * (64 * CPL) + lane;  // the lane's first chunk in the row
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
    f32x4 xr[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) xr[c] = x4[c0 + 64 * c];
    f32x4 q[RW][CPL];
    auto issue = [&](int r) {
        const f32x4* a4 = reinterpret_cast<const f32x4*>(A + (size_t)min(row0 + r, M - 1) * lda);
#pragma unroll
        for (int c = 0; c < CPL; ++c) q[r][c] = __builtin_nontemporal_load(a4 + c0 + 64 * c);
    };
#pragma unroll
    for (int r = 0; r < (D < RW ? D : RW); ++r) issue(r);
    float res = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        if (r + D < RW) issue(r + D);
        __builtin_amdgcn_sched_barrier(0);
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            float& acc = (c & 1) ? a1 : a0;
            acc = fmaf(q[r][c].x, xr[c].x, acc);
            acc = fmaf(q[r][c].y, xr[c].y, acc);
            acc = fmaf(q[r][c].z, xr[c].z, acc);
            acc = fmaf(q[r][c].w, xr[c].w, acc);
        }
        const float d = wave_sum(a0 + a1);
        res = lane == r ? d : res;
        __builtin_amdgcn_sched_barrier(0);
    }
    __shared__ float part_k[KS > 1 ? KS - 1 : 1][RS][64];
    if (kp > 0) part_k[kp - 1][wave % RS][lane] = res;
    __syncthreads();
    float tot = res;
#pragma unroll
    for (int i = 0; i < KS - 1; ++i) tot += part_k[i][wave % RS][lane];
    if (kp == 0 && lane < nrows) gemv_store(y + row0 + lane, tot, alpha, beta);
}

// Short rows (K <= 4L floats, L = 8, 16 or 32): a wave holds 64/L rows side by side,
// L lanes each, and four such row groups per wave, so every lane keeps four 16-B loads
// in flight as in the long-row kernel (a 128-float row would leave half of a one-row
// wave idle).  Needs the vector layout (lda % 4 == 0, 16-B aligned A and x).  Partials
// meet by xor shuffles inside each L-lane segment.  Batch b = blockIdx.y.
template <int L>
__global__ __launch_bounds__(256) void k_gemv_f32_short(const float* __restrict__ A,
                                                        const float* __restrict__ x,
                                                        float* __restrict__ y, int M, int K, int lda,
                                                        float alpha, float beta, size_t sa, size_t sx,
                                                        size_t sy) {
    constexpr int R = 64 / L, U = 4;  // rows side by side, row groups per wave
    const int lane = threadIdx.x & 63, seg = lane / L, sl = lane % L;
    const size_t b = blockIdx.y;
    A += b * sa;
    x += b * sx;
    y += b * sy;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (U * R) + seg;
    float acc[U] = {};
    const int K4 = K >> 2;
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
    for (int k4 = sl; k4 < K4; k4 += L) {
        const f32x4 u = x4[k4];
        f32x4 v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int row = row0 + j * R;
            v[j] = row < M ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(A + (size_t)row * lda) + k4)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
            acc[j] = fmaf(v[j].x, u.x, acc[j]); acc[j] = fmaf(v[j].y, u.y, acc[j]);
            acc[j] = fmaf(v[j].z, u.z, acc[j]); acc[j] = fmaf(v[j].w, u.w, acc[j]);
        }
    }
    for (int k = (K4 << 2) + sl; k < K; k += L) {
        const float u = x[k];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int row = row0 + j * R;
            if (row < M) acc[j] = fmaf(A[(size_t)row * lda + k], u, acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
        for (int o = L / 2; o > 0; o >>= 1) acc[j] += __shfl_xor(acc[j], o, 64);
        const int row = row0 + j * R;
        if (sl == 0 && row < M) {
            float r = alpha * acc[j];
            if (beta != 0.f) r = fmaf(beta, y[row], r);  // y untouched when beta == 0
            y[row] = r;
        }
    }
}

// y[n] = alpha * sum_r A[r, n] x[r] + beta * y[n] (gemv_transpose) in two passes.  Pass 1:
// a block takes a strip of 64 * CPL columns (CPL = 4 with 16-B loads) and a chunk of
// rows; its 4 waves take every 4th row of the chunk, 8 rows in flight per lane, and their
// sums meet in LDS: one partial per (chunk, column) in P[chunk][n].  Pass 2 adds the
// chunks' partials in chunk order and applies alpha and beta.  Every sum has a fixed
// order, so results are deterministic.  (One block per 64-column strip walking all rows,
// one load in flight per lane, ran at 2 % of HBM on 4096 x 4096.)
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemv_t_partial(const float* __restrict__ A, const float* __restrict__ x,
                                                        float* __restrict__ P, int M, int N, int lda, int R) {
    constexpr int CPL = VEC ? 4 : 1, U = 8;
    __shared__ float red[4][64 * CPL];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int col = (blockIdx.x * 64 + lane) * CPL;
    const int r0 = blockIdx.y * R, r1 = min(M, r0 + R);
    float acc[CPL] = {};
    if (col < N) {
        for (int r = r0 + wv; r < r1; r += 4 * U) {
            float v[U][CPL], xv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int rr = r + 4 * u;
                const bool in = rr < r1;
                xv[u] = in ? x[rr] : 0.f;
                // rows past the chunk reload row r and count as 0 (not 0 * A: A may hold inf)
                const float* a = A + (size_t)(in ? rr : r) * lda + col;
                if constexpr (VEC) {
                    const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a));
#pragma unroll
                    for (int c = 0; c < CPL; ++c) v[u][c] = in ? t[c] : 0.f;
                } else {
                    const float t = __builtin_nontemporal_load(a);
                    v[u][0] = in ? t : 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int c = 0; c < CPL; ++c) acc[c] = fmaf(v[u][c], xv[u], acc[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) red[wv][lane * CPL + c] = acc[c];
    __syncthreads();
    if (wv == 0 && col < N) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int e = lane * CPL + c;
            P[(size_t)blockIdx.y * N + col + c] = (red[0][e] + red[1][e]) + (red[2][e] + red[3][e]);
        }
    }
}

// Pass 2: a block takes 64 columns.  With N % 4 == 0 (VEC), 16 lanes cover the 64 columns
// with 16-B loads and the block's 16 such groups take chunks g, g + 16, ... (at most 16
// per thread for 256 chunks, issued 8 at a time), so one round trip covers 64 chunks;
// otherwise lane = column and wave w takes chunks w, w + 4, ....  The group sums meet in
// LDS and are added in group order.  (One thread per column walking all chunks took 19 us
// for 64 chunks x 4096 columns: one load round trip per chunk.)
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemv_t_reduce(const float* __restrict__ P, float* __restrict__ y, int N,
                                                       int C, float alpha, float beta) {
    constexpr int CPL = VEC ? 4 : 1, NG = VEC ? 16 : 4;  // columns per lane, chunk groups
    __shared__ float red[NG][64];
    const int tid = threadIdx.x;
    const int cl = VEC ? (tid & 15) * 4 : (tid & 63);  // first column of the thread in the block
    const int g = VEC ? tid >> 4 : tid >> 6;
    const int n = blockIdx.x * 64 + cl;
    float s[CPL] = {};
    if (n < N) {
        for (int c0 = g; c0 < C; c0 += 8 * NG) {
            float v[8][CPL];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = c0 + NG * u;
                if constexpr (VEC) {
                    const f32x4 t = c < C ? *reinterpret_cast<const f32x4*>(P + (size_t)c * N + n) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[u][e] = t[e];
                } else {
                    v[u][0] = c < C ? P[(size_t)c * N + n] : 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int e = 0; e < CPL; ++e) s[e] += v[u][e];
        }
    }
#pragma unroll
    for (int e = 0; e < CPL; ++e) red[g][cl + e] = s[e];
    __syncthreads();
    if (tid < 64 && blockIdx.x * 64 + tid < N) {
        float t = 0.f;
#pragma unroll
        for (int h = 0; h < NG; ++h) t += red[h][tid];
        const int col = blockIdx.x * 64 + tid;
        float r = alpha * t;
        if (beta != 0.f) r = fmaf(beta, y[col], r);  // y untouched when beta == 0
        y[col] = r;
    }
}

// Row chunks of the transposed GEMV: about 64 rows each, at most 256 chunks and at most
// 16 Mi partials (64 MiB of workspace).
static int gemv_t_chunks(int M, int N) {
    int64_t c = ((int64_t)M + 63) / 64;
    c = std::min<int64_t>(c, 256);
    c = std::min<int64_t>(c, std::max<int64_t>(1, (int64_t)(16 << 20) / std::max(N, 1)));
    return (int)std::max<int64_t>(c, 1);
}

size_t gemv_t_workspace(int M, int N) { return (size_t)gemv_t_chunks(M, N) * (size_t)N * sizeof(float); }

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

// General fp32 GEMM on the fp32 matrix cores (v_mfma_f32_32x32x2_f32), for row-major
// A [M x K] and B [K x N] whose rows start 16-byte aligned (K % 4 == 0, N % 4 == 0):
//   - block tile BM x BN (128 x 128, or 64 x 64 when the larger tile leaves CUs idle),
//     4 waves in 2 x 2, each a (BM / 2) x (BN / 2) grid of 32 x 32 MFMA tiles;
//   - K advances 32 per stage through double-buffered LDS; the stage's global loads
//     (16 bytes per lane, rows past M / N or k past K read as zeros) are issued before the
//     MFMAs of the previous stage and written to the other buffer after them;
//   - an MFMA k-step s (0..15) takes k = 16 kh + s, kh = lane / 32, so a lane's A values of a
//     stage are 16 consecutive k of one row (4 ds_read_b128); its B values are one column
//     of the stage (ds_read_b32, row pitch 132 floats: the two k-halves land in different
//     banks).
// Sums run in a different order from the reference's sequential k (fp32, rel error ~1e-6).
template <int BM, int BN>
__global__ __launch_bounds__(256) void k_gemm_f32_mfma(const float* __restrict__ A, const float* __restrict__ B,
                                                      float* __restrict__ C, int M, int K, int N) {
    constexpr int BK = 32, AP = BK + 4, BP = BN + 4;  // LDS pitches (floats)
    constexpr int TM = BM / 64, TN = BN / 64;          // 32x32 tiles per wave (each way)
    __shared__ __attribute__((aligned(16))) float sa[2][BM * AP];
    __shared__ __attribute__((aligned(16))) float sb[2][BK * BP];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int i32 = lane & 31, kh = lane >> 5;

    // staging: A tile BM x 32 = BM * 8 float4, B tile 32 x BN = 8 * BN float4; stage st + 1
    // is loaded into registers while stage st computes.  (Loading two stages ahead was
    // measured: 10 % slower at 1024^3, 3 % faster at 4096^3.)
    constexpr int AL = BM * 8 / 256, BL = BN * 8 / 256;
    f32x4 ra[AL], rb[BL];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int e = tid + 256 * i, r = e >> 3, c4 = (e & 7) * 4;
            const int gm = m0 + r, gk = k0 + c4;
            ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const f32x4*>(A + (size_t)gm * K + gk) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const int e = tid + 256 * i, r = e / (BN / 4), c4 = (e % (BN / 4)) * 4;
            const int gk = k0 + r, gn = n0 + c4;
            rb[i] = (gk < K && gn < N) ? *reinterpret_cast<const f32x4*>(B + (size_t)gk * N + gn) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int e = tid + 256 * i, r = e >> 3, c4 = (e & 7) * 4;
            *reinterpret_cast<f32x4*>(&sa[buf][r * AP + c4]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const int e = tid + 256 * i, r = e / (BN / 4), c4 = (e % (BN / 4)) * 4;
            *reinterpret_cast<f32x4*>(&sb[buf][r * BP + c4]) = rb[i];
        }
    };

    // One 32x32 tile per wave (64 x 64 blocks) keeps two accumulator chains (even and odd
    // k-steps), added at the end.
    constexpr int CH = TM * TN == 1 ? 2 : 1;
    f32x16 acc[TM][TN], acc2[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = acc2[a][b] = f32x16{};

    const int nst = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        if (st + 1 < nst) gload((st + 1) * BK);
        float av[TM][16];
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(&sa[buf][(wm * (BM / 2) + 32 * a + i32) * AP + 16 * kh + 4 * q]);
#pragma unroll
                for (int e = 0; e < 4; ++e) av[a][4 * q + e] = v[e];
            }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            float bv[TN];
#pragma unroll
            for (int b = 0; b < TN; ++b) bv[b] = sb[buf][(16 * kh + s) * BP + wn * (BN / 2) + 32 * b + i32];
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) {
                    if (CH == 2 && (s & 1))
                        acc2[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a][s], bv[b], acc2[a][b], 0, 0, 0);
                    else
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a][s], bv[b], acc[a][b], 0, 0, 0);
                }
        }
        if (st + 1 < nst) lstore(buf ^ 1);  // buf ^ 1 was last read before the previous barrier
        __syncthreads();
    }

    if constexpr (CH == 2) {
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) acc[a][b] += acc2[a][b];
    }
    // D[i][j] of a 32x32 tile: lane j + 32 * ((i / 4) & 1), register 4 * (i / 8) + i % 4.
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int n = n0 + wn * (BN / 2) + 32 * b + i32;
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * (BM / 2) + 32 * a + 8 * (r / 4) + 4 * kh + (r % 4);
                if (m < M) C[(size_t)m * N + n] = acc[a][b][r];
            }
        }
}

// fp16 dot product of one row with fp32 accumulation, by one wave: 16-byte chunks (8
// halves), v_dot2_f32_f16 on each pair (exact fp16 x fp16 products).  Wave-uniform result.
template <bool VEC>
__device__ __forceinline__ float f16_dot(const f16* __restrict__ a, const f16* __restrict__ x, int K) {
    const int lane = threadIdx.x & 63;
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
    return wave_sum(acc0 + acc1);
}

// fp16 GEMV: one wave per row of A against the shared x.
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemv_f16(const f16* __restrict__ A,
                                                  const f16* __restrict__ x,
                                                  float* __restrict__ y, int M, int K, int lda) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const float s = f16_dot<VEC>(A + (size_t)row * lda, x, K);
    if ((threadIdx.x & 63) == 0) y[row] = s;
}

// fp16 GEMV in the shape of k_gemv_f32_parts: rows split into KS parts of k, a wave owns
// RW rows of one part, CPL 16-byte chunks (8 halves) per lane and row, two rows ahead;
// exact fp16 products (v_dot2_f32_f16) summed in fp32, the parts' sums added in k order.
// Needs K / 8 = 64 * KS * CPL chunks and the vector layout.  The launcher uses whole rows
// (KS = 1) at 8 waves per CU: at 14336 x 4096, 7 rows per wave 18.34-18.38 us, quarters of
// 14 rows in 4,096 waves 18.37-18.42 us, halves of 14 rows 18.7-18.8 us (lab).
template <int RW, int KS, int CPL>
__global__ __launch_bounds__(256) void k_gemv_f16_parts(const f16* __restrict__ A, const f16* __restrict__ x,
                                                        float* __restrict__ y, int M, int lda) {
    constexpr int RS = 4 / KS, D = 2;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * RS + wave % RS) * RW, kp = wave / RS;
    const int nrows = min(RW, M - row0);
    const int c0 = kp * (64 * CPL) + lane;
    const f16x8* x8 = reinterpret_cast<const f16x8*>(x);
    f16x8 xr[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) xr[c] = x8[c0 + 64 * c];
    f16x8 q[RW][CPL];
    auto issue = [&](int r) {
        const f16x8* a8 = reinterpret_cast<const f16x8*>(A + (size_t)min(row0 + r, M - 1) * lda);
#pragma unroll
        for (int c = 0; c < CPL; ++c) q[r][c] = __builtin_nontemporal_load(a8 + c0 + 64 * c);
    };
#pragma unroll
    for (int r = 0; r < (D < RW ? D : RW); ++r) issue(r);
    float res = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        if (r + D < RW) issue(r + D);
        __builtin_amdgcn_sched_barrier(0);
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const f16x8 v = q[r][c], u = xr[c];
            a0 = __builtin_amdgcn_fdot2(f16x2{v[0], v[1]}, f16x2{u[0], u[1]}, a0, false);
            a1 = __builtin_amdgcn_fdot2(f16x2{v[2], v[3]}, f16x2{u[2], u[3]}, a1, false);
            a0 = __builtin_amdgcn_fdot2(f16x2{v[4], v[5]}, f16x2{u[4], u[5]}, a0, false);
            a1 = __builtin_amdgcn_fdot2(f16x2{v[6], v[7]}, f16x2{u[6], u[7]}, a1, false);
        }
        const float d = wave_sum(a0 + a1);
        res = lane == r ? d : res;
        __builtin_amdgcn_sched_barrier(0);
    }
    __shared__ float part_k[KS > 1 ? KS - 1 : 1][RS][64];
    if (kp > 0) part_k[kp - 1][wave % RS][lane] = res;
    if constexpr (KS > 1) __syncthreads();
    float tot = res;
#pragma unroll
    for (int i = 0; i < KS - 1; ++i) tot += part_k[i][wave % RS][lane];
    if (kp == 0 && lane < nrows) y[row0 + lane] = tot;
}

// dot_product_fp16_fp32 (fp_quantized.wgsl:418-469): vector v of a and of b starts at
// element 2 * (v * stride / 2) (the WGSL reads whole f16 pairs from word base / 2, so an
// odd base starts one element early) and has `size` elements.  One wave per vector.
template <bool VEC>
__global__ __launch_bounds__(256) void k_dot_f16(const f16* __restrict__ a, const f16* __restrict__ b,
                                                 float* __restrict__ out, int size, int nv, size_t stride) {
    const int v = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (v >= nv) return;
    const size_t e0 = 2 * ((size_t)v * stride / 2);
    const float s = f16_dot<VEC>(a + e0, b + e0, size);
    if ((threadIdx.x & 63) == 0) out[v] = s;
}

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t launch_gemv_f32_batched(const float* A, const float* x, float* y, int M, int K, int lda,
                                   float alpha, float beta, int batch, size_t sa, size_t sx,
                                   size_t sy, hipStream_t s) {
    const int64_t row_blocks = ((int64_t)M + 3) / 4;
    int mode = (row_blocks > (1 << 20) || batch > 65535) ? 2 : batch > 1 ? 1 : 0;
    if (mode == 0 && M <= 8192 && K >= 1024) mode = 3;
    dim3 grid((unsigned)std::min<int64_t>(row_blocks, 1 << 20), (unsigned)std::min(batch, 65535)),
        block(256);
    const bool vec = (lda % 4 == 0) && aligned16(A) && aligned16(x) && sa % 4 == 0 && sx % 4 == 0;
    if (mode == 3 && vec && M >= 1024 && (K == 1024 || K == 2048 || K == 4096)) {
        // k in quarters, RW rows per wave (4096 x 4096: 11.14 us against 11.58 us with
        // the rows split in halves, one half row per wave)
        const int rw = M >= 4096 ? 16 : M >= 2048 ? 8 : 4;
        const dim3 g((unsigned)((M + rw - 1) / rw)), b(256);  // four waves (quarters) per row set
        auto gp = [&](auto kern) { hipLaunchKernelGGL(kern, g, b, 0, s, A, x, y, M, K, lda, alpha, beta); };
        if (K == 4096) {
            if (rw == 16) gp(k_gemv_f32_parts<16, 4, 4>);
            else if (rw == 8) gp(k_gemv_f32_parts<8, 4, 4>);
            else gp(k_gemv_f32_parts<4, 4, 4>);
        } else if (K == 2048) {
            if (rw == 16) gp(k_gemv_f32_parts<16, 4, 2>);
            else if (rw == 8) gp(k_gemv_f32_parts<8, 4, 2>);
            else gp(k_gemv_f32_parts<4, 4, 2>);
        } else {
            if (rw == 16) gp(k_gemv_f32_parts<16, 4, 1>);
            else if (rw == 8) gp(k_gemv_f32_parts<8, 4, 1>);
            else gp(k_gemv_f32_parts<4, 4, 1>);
        }
        return hipGetLastError();
    }
    if (mode == 3) grid.x = (unsigned)((M + 1) / 2);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, s, A, x, y, M, K, lda, alpha, beta, batch, sa, sx, sy);
    };
    if (vec && mode != 2 && K <= 128) {
        // short rows: 16 (L = 32), 32 (L = 16) or 64 (L = 8) rows per 256-thread block
        const int L = K <= 32 ? 8 : K <= 64 ? 16 : 32, rows_per_block = 4 * 4 * (64 / L);
        const dim3 g2((unsigned)((M + rows_per_block - 1) / rows_per_block), (unsigned)batch);
        auto go2 = [&](auto kern) {
            hipLaunchKernelGGL(kern, g2, block, 0, s, A, x, y, M, K, lda, alpha, beta, sa, sx, sy);
        };
        if (L == 8) go2(k_gemv_f32_short<8>);
        else if (L == 16) go2(k_gemv_f32_short<16>);
        else go2(k_gemv_f32_short<32>);
    } else if (vec) {
        if (mode == 0) go(k_gemv_f32<true, 0>);
        else if (mode == 1) go(k_gemv_f32<true, 1>);
        else if (mode == 2) go(k_gemv_f32<true, 2>);
        else go(k_gemv_f32<true, 3>);
    } else {
        if (mode == 0) go(k_gemv_f32<false, 0>);
        else if (mode == 1) go(k_gemv_f32<false, 1>);
        else if (mode == 2) go(k_gemv_f32<false, 2>);
        else go(k_gemv_f32<false, 3>);
    }
    return hipGetLastError();
}

hipError_t launch_gemv_f32(const float* A, const float* x, float* y, int M, int K, int lda,
                           float alpha, float beta, hipStream_t s) {
    return launch_gemv_f32_batched(A, x, y, M, K, lda, alpha, beta, 1, 0, 0, 0, s);
}

hipError_t launch_gemv_f32_t(const float* A, const float* x, float* y, int M, int N, int lda,
                             float alpha, float beta, float* ws, hipStream_t s) {
    const int C = gemv_t_chunks(M, N), R = (int)(((int64_t)M + C - 1) / C);
    const bool vec = N % 4 == 0 && lda % 4 == 0 && aligned16(A);
    if (vec)
        hipLaunchKernelGGL(k_gemv_t_partial<true>, dim3((unsigned)((N + 255) / 256), (unsigned)C), dim3(256), 0, s,
                           A, x, ws, M, N, lda, R);
    else
        hipLaunchKernelGGL(k_gemv_t_partial<false>, dim3((unsigned)((N + 63) / 64), (unsigned)C), dim3(256), 0, s,
                           A, x, ws, M, N, lda, R);
    if (N % 4 == 0)  // the partials then start 16-byte aligned (ws is)
        hipLaunchKernelGGL(k_gemv_t_reduce<true>, dim3((unsigned)((N + 63) / 64)), dim3(256), 0, s, ws, y, N, C, alpha, beta);
    else
        hipLaunchKernelGGL(k_gemv_t_reduce<false>, dim3((unsigned)((N + 63) / 64)), dim3(256), 0, s, ws, y, N, C, alpha, beta);
    return hipGetLastError();
}

hipError_t launch_gemm_f32(const float* A, const float* B, float* C, int M, int K, int N,
                           hipStream_t s) {
    if (K % 4 == 0 && N % 4 == 0 && aligned16(A) && aligned16(B)) {
        // 128 x 128 tiles when they still give every CU a block, else 64 x 64
        const int64_t big = ((int64_t)(M + 127) / 128) * ((N + 127) / 128);
        if (big >= device_cus())
            hipLaunchKernelGGL((k_gemm_f32_mfma<128, 128>), dim3((N + 127) / 128, (M + 127) / 128), dim3(256), 0, s,
                               A, B, C, M, K, N);
        else
            hipLaunchKernelGGL((k_gemm_f32_mfma<64, 64>), dim3((N + 63) / 64, (M + 63) / 64), dim3(256), 0, s, A, B,
                               C, M, K, N);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_gemm_f32, dim3((N + 63) / 64, (M + 63) / 64), dim3(256), 0, s, A, B, C,
                       M, K, N);
    return hipGetLastError();
}

hipError_t launch_dot_f16(const void* a, const void* b, float* out, int size, int nv, size_t stride,
                          hipStream_t s) {
    const bool vec = stride % 8 == 0 && aligned16(a) && aligned16(b);
    const f16* pa = reinterpret_cast<const f16*>(a);
    const f16* pb = reinterpret_cast<const f16*>(b);
    const dim3 grid((unsigned)(((int64_t)nv + 3) / 4)), block(256);
    if (vec) hipLaunchKernelGGL(k_dot_f16<true>, grid, block, 0, s, pa, pb, out, size, nv, stride);
    else hipLaunchKernelGGL(k_dot_f16<false>, grid, block, 0, s, pa, pb, out, size, nv, stride);
    return hipGetLastError();
}

template <int CPL>
static void launch_gemv_f16_rows(const f16* a, const f16* xv, float* y, int M, int lda, hipStream_t s) {
    const int target_waves = device_cus() * 8;
    int rw = (M + target_waves - 1) / target_waves;
    rw = rw < 1 ? 1 : rw > 8 ? 8 : rw;
    auto go = [&](auto kern, int r) {
        hipLaunchKernelGGL(kern, dim3((unsigned)(((M + r - 1) / r + 3) / 4)), dim3(256), 0, s, a, xv, y, M, lda);
    };
    switch (rw) {
        case 1: go(k_gemv_f16_parts<1, 1, CPL>, 1); break;
        case 2: go(k_gemv_f16_parts<2, 1, CPL>, 2); break;
        case 3: go(k_gemv_f16_parts<3, 1, CPL>, 3); break;
        case 4: go(k_gemv_f16_parts<4, 1, CPL>, 4); break;
        case 5: go(k_gemv_f16_parts<5, 1, CPL>, 5); break;
        case 6: go(k_gemv_f16_parts<6, 1, CPL>, 6); break;
        case 7: go(k_gemv_f16_parts<7, 1, CPL>, 7); break;
        default: go(k_gemv_f16_parts<8, 1, CPL>, 8); break;
    }
}

hipError_t launch_gemv_f16(const void* A, const void* x, float* y, int M, int K, int lda,
                           hipStream_t s) {
    dim3 grid((M + 3) / 4), block(256);
    bool vec = (lda % 8 == 0) && aligned16(A) && aligned16(x);
    const f16* a = reinterpret_cast<const f16*>(A);
    const f16* xv = reinterpret_cast<const f16*>(x);
    // Whole rows of 512 to 4096 halves: RW rows per wave, 8 waves per CU (14336 x 4096:
    // 7 rows per wave, 18.34-18.38 us against 19.15 us for one row per wave, lab)
    if (vec && M >= 1024 && (K == 512 || K == 1024 || K == 2048 || K == 4096)) {
        if (K == 4096) launch_gemv_f16_rows<8>(a, xv, y, M, lda, s);
        else if (K == 2048) launch_gemv_f16_rows<4>(a, xv, y, M, lda, s);
        else if (K == 1024) launch_gemv_f16_rows<2>(a, xv, y, M, lda, s);
        else launch_gemv_f16_rows<1>(a, xv, y, M, lda, s);
        return hipGetLastError();
    }
    if (vec) hipLaunchKernelGGL(k_gemv_f16<true>, grid, block, 0, s, a, xv, y, M, K, lda);
    else hipLaunchKernelGGL(k_gemv_f16<false>, grid, block, 0, s, a, xv, y, M, K, lda);
    return hipGetLastError();
}

}  // namespace luxhip
