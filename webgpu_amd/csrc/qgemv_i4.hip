// int4 weight-only GEMV (m == 1): y[n] = sum_k (q(n,k) * s(n, k/gs)) * x[k].
//
// Reference: matmul_nax_grouped with N == 1 (quantized_nax.wgsl:568-626), whose
// per-element dequant is f32(nib - 8) * GroupScale.scale (:589-608).  Here the
// group scale is applied once per 32-element slice to an fp32 partial sum
// (s * sum q*x instead of sum (q*s)*x): the products q*x are exact, so only the
// fp32 summation order differs.
//
// HBM-bound design (config: W 14336 x 4096, g32, fp16 scales, fp16 x):
//   - a "slice" is 32 consecutive k of one row = 16 bytes of packed nibbles = one
//     global_load_dwordx4; with g32 it is exactly one scale group;
//   - lane l of a wave owns slices l, l+64, ... of every row, so its slice of x is
//     loop-invariant and lives in registers, pre-permuted into the (k, k+4) fp16
//     pairs the nibble decode produces;
//   - a masked nibble pair is read directly as two fp16 subnormals (n * 2^-24),
//     v_dot2_f32_f16 accumulates the exact products n*x in fp32, and the offset
//     of the offset-binary code is removed once per slice as -8 * sum(x);
//   - x is read once per block and shared through LDS;
//   - each wave owns a run of rows and keeps two rows of loads in flight ahead of
//     its math; the row sums use a VALU-only DPP wave reduction.
// lux_hip_rms_norm_qmatmul instantiates the same kernel with RN: every block normalises
// the activation row itself (rms_norm.wgsl:50-110, k_rms_norm's arithmetic and order)
// while its first weight rows are in flight, so a decode step needs no rms_norm launch.
#include <cstdlib>

#include "common.hpp"

namespace luxhip {

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// sum_{i<32} nib_i * x_i * 2^-24 for one 16-byte slice.  A masked nibble read as
// an fp16 bit pattern is the subnormal n * 2^-24 (no implicit bit, no offset to
// remove), so decode is one AND per pair; v_dot2_f32_f16 multiplies exactly
// (f16 denormals are preserved) and accumulates in fp32.  The odd nibbles are
// masked in place (16n * 2^-24) and rescaled by 1/16 at the end.  9 VALU ops
// per 8 weights.
__device__ __forceinline__ float dot_slice_sub(const uint32_t (&q)[4], const f16x2 (&xp)[4][4]) {
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t word = q[w];
        const uint32_t w8 = word >> 8;
        lo = __builtin_amdgcn_fdot2(as_h2(word & 0x000F000Fu), xp[w][0], lo, false);  // n0, n4
        hi = __builtin_amdgcn_fdot2(as_h2(word & 0x00F000F0u), xp[w][1], hi, false);  // 16 n1, 16 n5
        lo = __builtin_amdgcn_fdot2(as_h2(w8 & 0x000F000Fu), xp[w][2], lo, false);    // n2, n6
        hi = __builtin_amdgcn_fdot2(as_h2(w8 & 0x00F000F0u), xp[w][3], hi, false);    // 16 n3, 16 n7
    }
    return fmaf(hi, 0.0625f, lo);
}

// One wave owns RW consecutive rows (the last wave may own fewer) and keeps D rows of
// weight slices and scales in flight: it issues rows 0..D-1, then for each row r issues
// row r+D and consumes row r, so the math of row r overlaps the loads of later rows.
// x is read from HBM/L2 once per block (one 16-byte chunk per thread and SPL pass) and
// shared through LDS.  The host sizes the grid to 8 waves per CU with equal rows per wave.
// SM (SiluMul epilogue): the wave's rows are read as interleaved pairs, gate row g then
// up row n_out/2 + g (virtual row v -> v even: v/2, v odd: n_out/2 + v/2; RW is even, so a
// pair never straddles two waves), and lane 2p stores silu(gate) * up to y[g].
// RN: x is not read; the block computes x = fp16(rn.x * r * gamma), r = 1 / sqrt(sum(rn.x^2)
// / K + eps), with k_rms_norm's arithmetic in k_rms_norm's order (thread t sums elements
// t + 256 j, j ascending, then the DPP wave sum and the four wave sums in a fixed order),
// so the staged row is bit-identical to what k_rms_norm would have written.
// KS = 2 or 4 (few, long rows: the decode down-projection): the block's waves w, w + 4/KS,
// ... take the same RW rows, each one KS-th of k in order, so each wave has KS times the
// rows to pipeline; the parts' sums meet in LDS and are added in k order.
template <int SPL, int RW, int D, ScaleKind SK, YKind YK, bool XOR, bool SM, bool RN, int KS = 1>
__global__ __launch_bounds__(256) void k_qgemv_i4_f16(const u32x4* __restrict__ W,
                                                      const void* __restrict__ S,
                                                      const f16* __restrict__ x,
                                                      void* __restrict__ y, int n_out, int K,
                                                      int spg_shift, uint32_t xor_mask, EpiArgs epi, RnArgs rn) {
    static_assert(KS == 1 || ((KS == 2 || KS == 4) && !SM && !RN), "k parts: plain rows only");
    constexpr int RS = 4 / KS;  // row sets per block: wave w takes row set w % RS, k part w / RS
    __shared__ u32x4 xs[KS * SPL * 256];  // K <= KS * SPL * 2048 halves
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * RS + wave % RS) * RW;
    const bool active = row0 < n_out;
    const int nrows = min(RW, n_out - row0);
    const int s_row = K >> 5;        // slices per row
    const int g_row = s_row >> spg_shift;  // groups per row (slices per group: a power of two)
    const int s_part = s_row / KS;   // slices of the wave's part of k (s_row is a multiple of KS)
    const int s_base = (wave / RS) * s_part;

    // Load order matters: vmcnt retires loads in issue order, so the block's x chunks
    // (L2 hits) go first, then the first D rows of weight slices and raw scales.  All
    // addresses are clamped to valid ones; out-of-range slices get x = 0 after the
    // loads, and rows past the wave's share are never computed or stored.
    u32x4 xv[KS * SPL];
    constexpr int NJ = RN ? 8 * SPL : 1;  // RN: row elements per thread (K <= 2048 * SPL)
    float xe[NJ], ge[NJ];
    if constexpr (RN) {
        const int last = K - 1;
        if (rn.xk == (int)XKind::F32) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) xe[j] = load_x<XKind::F32>(rn.x, min((int)threadIdx.x + 256 * j, last));
        } else if (rn.xk == (int)XKind::F16) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) xe[j] = load_x<XKind::F16>(rn.x, min((int)threadIdx.x + 256 * j, last));
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j) xe[j] = load_x<XKind::BF16>(rn.x, min((int)threadIdx.x + 256 * j, last));
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) ge[j] = rn.gamma[min((int)threadIdx.x + 256 * j, last)];
    } else {
#pragma unroll
        for (int j = 0; j < KS * SPL; ++j) {
            const int c = threadIdx.x + 256 * j;
            xv[j] = c < K / 8 ? reinterpret_cast<const u32x4*>(x)[c] : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep x loads ahead of the weight stream
    int sl[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) sl[j] = s_base + min(lane + 64 * j, s_part - 1);

    u32x4 q[RW][SPL];
    uint32_t sraw[RW][SPL];
    // Rows past n_out (last wave only) read the last matrix row instead (an L2 hit);
    // they are computed but never stored.  Straight-line, in-order issue keeps the
    // waitcnt bookkeeping exact.
    auto issue = [&](int r) {
        const int v = min(row0 + r, n_out - 1);
        const size_t row = SM ? (size_t)((v & 1) ? (n_out >> 1) + (v >> 1) : (v >> 1)) : (size_t)v;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            q[r][j] = __builtin_nontemporal_load(W + row * s_row + sl[j]);
            if constexpr (SK == ScaleKind::F16)  // aligned u32 holding this scale (g_row is even)
                sraw[r][j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(S) +
                                                        ((row * g_row + (sl[j] >> spg_shift)) >> 1));
            else
                sraw[r][j] = load_scale_raw<SK>(S, row * g_row + (sl[j] >> spg_shift));
        }
    };
#pragma unroll
    for (int r = 0; r < (D < RW ? D : RW); ++r) issue(r);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (RN) {
        __shared__ float part[4];
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const float v = (int)threadIdx.x + 256 * j < K ? xe[j] : 0.0f;
            ss = fmaf(v, v, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) part[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float mean_sq = ((part[0] + part[1]) + (part[2] + part[3])) / (float)K;
        const float r = 1.0f / sqrtf(mean_sq + rn.eps);
        f16* xh = reinterpret_cast<f16*>(xs);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int i = threadIdx.x + 256 * j;
            if (i < K) xh[i] = (f16)(xe[j] * r * ge[j]);  // RNE, as k_rms_norm's fp16 store
        }
    } else {
#pragma unroll
        for (int j = 0; j < KS * SPL; ++j) {
            const int c = threadIdx.x + 256 * j;
            if (c < K / 8) xs[c] = xv[j];
        }
    }
    __syncthreads();  // every wave of the block reaches this before any returns
    // KS > 1: waves without rows still run (on clamped rows) to the parts' barrier
    if (KS == 1 && !active) return;

    // x pairs in decode order and, per slice, -8 * sum(x) (offset-binary q = n - 8).
    f16x2 xp[SPL][4][4];
    float xoff[SPL];
    const f16x2 ONES = {(f16)1.0f, (f16)1.0f};
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        const uint32_t keep = lane + 64 * j < s_part ? ~0u : 0u;  // bitwise: no branch
        float sx = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const u32x4 u = xs[4 * sl[j] + w] & keep;
            const f16x8 v = __builtin_bit_cast(f16x8, u);
            xp[j][w][0] = f16x2{v[0], v[4]};
            xp[j][w][1] = f16x2{v[1], v[5]};
            xp[j][w][2] = f16x2{v[2], v[6]};
            xp[j][w][3] = f16x2{v[3], v[7]};
#pragma unroll
            for (int p = 0; p < 4; ++p) sx = __builtin_amdgcn_fdot2(xp[j][w][p], ONES, sx, false);
        }
        xoff[j] = -8.0f * sx;
    }

    // Software pipeline: keep D rows in flight; issue row r + D, then compute row r.
    float res = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        if (r + D < RW) issue(r + D);
        __builtin_amdgcn_sched_barrier(0);
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            uint32_t sb = sraw[r][j];
            if constexpr (SK == ScaleKind::F16) sb = (sb >> (((sl[j] >> spg_shift) & 1) * 16)) & 0xFFFFu;
            uint32_t qq[4] = {q[r][j].x, q[r][j].y, q[r][j].z, q[r][j].w};
            if constexpr (XOR) {
#pragma unroll
                for (int w = 0; w < 4; ++w) qq[w] ^= xor_mask;
            }
            const float part = fmaf(dot_slice_sub(qq, xp[j]), 16777216.0f, xoff[j]);  // * 2^24
            acc = fmaf(part, scale_from_raw<SK>(sb), acc);
        }
        acc = wave_sum(acc);
        res = lane == r ? acc : res;
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (SM) {
        const float up = __shfl_down(res, 1, 64);  // the pair's up row sits in the next lane
        if (lane < nrows && !(lane & 1)) store_y<YK>(y, (row0 + lane) >> 1, silu_f(res) * up);
    } else if constexpr (KS > 1) {  // the parts' sums meet in LDS, added in k order
        __shared__ float part_k[KS - 1][RS][64];
        const int kp = wave / RS, rs = wave % RS;
        if (kp > 0) part_k[kp - 1][rs][lane] = res;
        __syncthreads();
        float tot = res;
#pragma unroll
        for (int i = 0; i < KS - 1; ++i) tot += part_k[i][rs][lane];
        if (kp == 0 && lane < nrows) store_y<YK>(y, row0 + lane, apply_epi(tot, epi, 0, row0 + lane, n_out));
    } else {
        if (lane < nrows) store_y<YK>(y, row0 + lane, apply_epi(res, epi, 0, row0 + lane, n_out));
    }
}

// Any activation dtype, any group size that is a multiple of 8: one wave per row,
// one u32 word (8 nibbles, always inside one group) per lane step.
template <XKind XK, YKind YK>
__global__ __launch_bounds__(256) void k_qgemv_i4_generic(const uint32_t* __restrict__ W,
                                                          const void* __restrict__ S,
                                                          ScaleKind sk, const void* __restrict__ x,
                                                          void* __restrict__ y, int n_out, int K,
                                                          int gs, uint32_t xor_mask, EpiArgs epi) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_out) return;
    const int words = K >> 3, g_row = K / gs;
    float acc = 0.f;
    for (int wi = lane; wi < words; wi += 64) {
        const uint32_t word = W[(size_t)row * words + wi] ^ xor_mask;
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            part = fmaf((float)((int)((word >> (4 * i)) & 0xFu) - 8), load_x<XK>(x, 8 * wi + i), part);
        acc = fmaf(part, load_scale(S, (size_t)row * g_row + (8 * wi) / gs, sk), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) store_y<YK>(y, row, apply_epi(acc, epi, 0, row, n_out));
}

template <int SPL, int RW, int D, ScaleKind SK, YKind YK, bool RN, int KS = 1>
static void launch_rwd(const QArgs& a, hipStream_t s) {
    const int waves = (a.n_out + RW - 1) / RW * KS;
    const dim3 grid((waves + 3) / 4), block(256);
    const u32x4* w = reinterpret_cast<const u32x4*>(a.w);
    const f16* x = reinterpret_cast<const f16*>(a.x);
    const int shift = __builtin_ctz(a.group_size / 32);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, s, w, a.s, x, a.y, a.n_out, a.k, shift, a.xor_mask, a.epi, a.rn);
    };
    if constexpr (KS > 1) {
        if (a.xor_mask) go(k_qgemv_i4_f16<SPL, RW, D, SK, YK, true, false, false, KS>);
        else go(k_qgemv_i4_f16<SPL, RW, D, SK, YK, false, false, false, KS>);
        return;
    }
    const bool sm = a.epi.kind == (int)Epi::SiluMul;
    if constexpr (RW % 2 == 0) {
        if (sm) {
            if (a.xor_mask) go(k_qgemv_i4_f16<SPL, RW, D, SK, YK, true, true, RN>);
            else go(k_qgemv_i4_f16<SPL, RW, D, SK, YK, false, true, RN>);
            return;
        }
    }
    if (a.xor_mask) go(k_qgemv_i4_f16<SPL, RW, D, SK, YK, true, false, RN>);
    else go(k_qgemv_i4_f16<SPL, RW, D, SK, YK, false, false, RN>);
}

// Two rows of prefetch (issue row r+2, then compute row r) measured best on MI355X for
// config 2 (7.0 us against 7.1 us with one row, 7.2 us with three and 7.4 us with four);
// issuing all rows up front bunches the arrivals and lengthens the tail (8.6 us).
template <int SPL, int RW, ScaleKind SK, YKind YK, bool RN, int KS = 1>
static void launch_rw(const QArgs& a, hipStream_t s) {
    launch_rwd<SPL, RW, 2, SK, YK, RN, KS>(a, s);
}

// Rows per wave: enough for 8 waves per CU with equal shares (14336 rows on 256
// CUs -> 7 rows per wave, 2048 waves).  The rows' registers are reused as the rows
// retire, so the count is bounded by instantiations, not registers: up to 8 in general,
// and for fp16 scales with whole rows of at most two slices per lane also 10 to 16 (even
// counts), so the decode gate/up GEMV (2 x 14336 rows in pairs) runs 14 rows in 2048
// waves: 11.75 us against 12.5 us with 8 rows in 3584 waves (lab, same process).
template <int SPL, ScaleKind SK, YKind YK, bool RN, int KS = 1>
static void launch_fast(const QArgs& a, hipStream_t s) {
    constexpr bool WIDE = SK == ScaleKind::F16 && KS == 1 && SPL <= 2;
    constexpr int RWMAX = WIDE ? 16 : (SPL <= 2 ? 8 : 16 / SPL);
    const int target_waves = device_cus() * 8;
    int rw = (KS * a.n_out + target_waves - 1) / target_waves;
    rw = rw < 1 ? 1 : (rw > RWMAX ? RWMAX : rw);
    if (a.epi.kind == (int)Epi::SiluMul || rw > 8) rw += rw & 1;  // whole gate/up pairs; even above 8
    switch (rw) {
        case 1: launch_rw<SPL, 1, SK, YK, RN, KS>(a, s); break;
        case 2: launch_rw<SPL, 2, SK, YK, RN, KS>(a, s); break;
        case 3: if constexpr (RWMAX >= 3) launch_rw<SPL, 3, SK, YK, RN, KS>(a, s); break;
        case 4: if constexpr (RWMAX >= 4) launch_rw<SPL, 4, SK, YK, RN, KS>(a, s); break;
        case 5: if constexpr (RWMAX >= 5) launch_rw<SPL, 5, SK, YK, RN, KS>(a, s); break;
        case 6: if constexpr (RWMAX >= 6) launch_rw<SPL, 6, SK, YK, RN, KS>(a, s); break;
        case 7: if constexpr (RWMAX >= 7) launch_rw<SPL, 7, SK, YK, RN, KS>(a, s); break;
        case 8: if constexpr (RWMAX >= 8) launch_rw<SPL, 8, SK, YK, RN, KS>(a, s); break;
        case 10: if constexpr (RWMAX >= 10) launch_rw<SPL, 10, SK, YK, RN, KS>(a, s); break;
        case 12: if constexpr (RWMAX >= 12) launch_rw<SPL, 12, SK, YK, RN, KS>(a, s); break;
        case 14: if constexpr (RWMAX >= 14) launch_rw<SPL, 14, SK, YK, RN, KS>(a, s); break;
        default: if constexpr (RWMAX >= 16) launch_rw<SPL, 16, SK, YK, RN, KS>(a, s); break;
    }
}

// Parts of k per row (KS = 2 or 4) when rows are few and long: at 8 waves per CU each wave
// would get at most two rows (nothing to overlap its math with), k is at least 4096 and
// splits into whole slices.  Halves while each fits two slices per lane (k <= 8192),
// quarters above that (two slices per lane up to k = 16384), so a wave keeps the config-2
// shape of two slices per lane and up to 8 rows.  Measured at 4096 rows: k = 14336 7.13 us
// in quarters against 7.60 us in halves, k = 12288 6.49 against 7.20 us, k = 8192 5.06
// against 4.97 us.  fp16 scales, no gated pairs, no fused rms_norm.  1: whole rows.
static int k_parts(const QArgs& a) {
    static const bool off = [] {  // LUX_HIP_GEMV_NO_KSPLIT=1: whole rows per wave (A/B timing)
        const char* e = getenv("LUX_HIP_GEMV_NO_KSPLIT");
        return e && e[0] == '1';
    }();
    const int target_waves = device_cus() * 8;
    if (off || a.scale_kind != ScaleKind::F16 || a.epi.kind == (int)Epi::SiluMul || a.rn.gamma ||
        a.n_out > 2 * target_waves || a.k < 4096 || a.k % 64 != 0 || a.k > 16384)
        return 1;
    return a.k > 8192 && a.k % 128 == 0 ? 4 : 2;
}

// RN (the GEMV normalises its own row): one to four slices per lane (k <= 8192), so that
// the row's elements and gamma stay in registers through the prologue (8 * SPL each).
template <ScaleKind SK, YKind YK, bool RN>
static bool dispatch_spl(const QArgs& a, hipStream_t s) {
    const int slices = a.k / 32;
    if constexpr (SK == ScaleKind::F16 && !RN) {
        const int kp = k_parts(a);
        if (kp == 4) {  // 8192 < k <= 16384: 65 to 128 slices per quarter
            launch_fast<2, SK, YK, RN, 4>(a, s);
            return true;
        }
        if (kp == 2) {
            const int sph = (slices / 2 + 63) / 64;  // slices per lane in each half
            if (sph <= 1) launch_fast<1, SK, YK, RN, 2>(a, s);
            else if (sph <= 2) launch_fast<2, SK, YK, RN, 2>(a, s);
            else launch_fast<4, SK, YK, RN, 2>(a, s);
            return true;
        }
    }
    const int spl = (slices + 63) / 64;
    if (spl <= 1) launch_fast<1, SK, YK, RN>(a, s);
    else if (spl <= 2) launch_fast<2, SK, YK, RN>(a, s);
    else if (spl <= 4) launch_fast<4, SK, YK, RN>(a, s);
    else if constexpr (!RN) {
        if (spl <= 8) launch_fast<8, SK, YK, RN>(a, s);
        else return false;
    } else {
        return false;
    }
    return true;
}

template <ScaleKind SK, bool RN>
static bool dispatch_y(const QArgs& a, hipStream_t s) {
    switch (a.y_kind) {
        case YKind::F32: return dispatch_spl<SK, YKind::F32, RN>(a, s);
        case YKind::F16: return dispatch_spl<SK, YKind::F16, RN>(a, s);
        case YKind::BF16: return dispatch_spl<SK, YKind::BF16, RN>(a, s);
        default: return false;
    }
}

template <XKind XK>
static bool launch_generic(const QArgs& a, hipStream_t s) {
    dim3 grid((a.n_out + 3) / 4), block(256);
    const uint32_t* w = reinterpret_cast<const uint32_t*>(a.w);
    switch (a.y_kind) {
        case YKind::F32:
            hipLaunchKernelGGL((k_qgemv_i4_generic<XK, YKind::F32>), grid, block, 0, s, w, a.s,
                               a.scale_kind, a.x, a.y, a.n_out, a.k, a.group_size, a.xor_mask, a.epi);
            return true;
        case YKind::F16:
            hipLaunchKernelGGL((k_qgemv_i4_generic<XK, YKind::F16>), grid, block, 0, s, w, a.s,
                               a.scale_kind, a.x, a.y, a.n_out, a.k, a.group_size, a.xor_mask, a.epi);
            return true;
        case YKind::BF16:
            hipLaunchKernelGGL((k_qgemv_i4_generic<XK, YKind::BF16>), grid, block, 0, s, w, a.s,
                               a.scale_kind, a.x, a.y, a.n_out, a.k, a.group_size, a.xor_mask, a.epi);
            return true;
        default: return false;
    }
}

bool qgemv_i4_fast(const QArgs& a) {
    // slices per group must be a power of two (the kernel shifts instead of dividing);
    // up to 8 slices per lane (k <= 16384)
    const int spg = a.group_size / 32;
    return a.x_kind == XKind::F16 && a.k % 32 == 0 && a.k <= 16384 && a.group_size % 32 == 0 && spg > 0 &&
           (spg & (spg - 1)) == 0 && (a.scale_kind != ScaleKind::F16 || (a.k / a.group_size) % 2 == 0) &&
           a.scale_kind != ScaleKind::None && ((uintptr_t)a.w & 15u) == 0 &&
           (a.rn.gamma != nullptr || ((uintptr_t)a.x & 15u) == 0) &&
           ((uintptr_t)a.s & 3u) == 0;  // fp16 scales are read as aligned u32 pairs
}

// The fused form stays bit-identical to rms_norm followed by the plain GEMV only where the
// plain GEMV gives whole rows to one wave; shapes whose k it splits run both kernels.
bool qgemv_i4_rn_supported(const QArgs& a) {
    QArgs plain = a;
    plain.rn.gamma = nullptr;
    QArgs b = a;
    if (!b.rn.gamma) b.rn.gamma = reinterpret_cast<const float*>(16);  // only the x-alignment test differs
    return a.m == 1 && a.wbits == 4 && a.scale_kind == ScaleKind::F16 && a.k <= 8192 && qgemv_i4_fast(b) &&
           k_parts(plain) == 1;
}

hipError_t launch_qgemv_i4(const QArgs& a, hipStream_t s) {
    if (a.rn.gamma) {  // the caller checked qgemv_i4_rn_supported
        if (!qgemv_i4_rn_supported(a) || !dispatch_y<ScaleKind::F16, true>(a, s)) return hipErrorInvalidValue;
        return hipGetLastError();
    }
    const bool fast = qgemv_i4_fast(a);
    if (a.epi.kind == (int)Epi::SiluMul && !fast) return hipErrorInvalidValue;  // the caller checks
    bool launched = false;
    if (fast) {
        switch (a.scale_kind) {
            case ScaleKind::F16: launched = dispatch_y<ScaleKind::F16, false>(a, s); break;
            case ScaleKind::F32: launched = dispatch_y<ScaleKind::F32, false>(a, s); break;
            case ScaleKind::GroupScale: launched = dispatch_y<ScaleKind::GroupScale, false>(a, s); break;
            default: break;
        }
    }
    if (!launched) {
        switch (a.x_kind) {
            case XKind::F32: launched = launch_generic<XKind::F32>(a, s); break;
            case XKind::F16: launched = launch_generic<XKind::F16>(a, s); break;
            case XKind::BF16: launched = launch_generic<XKind::BF16>(a, s); break;
            default: break;
        }
    }
    if (!launched) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace luxhip
