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
//   - nibbles become fp16 with the 0x6400 exponent trick (1024 + n, or 1024 + 16n
//     for the odd nibbles), one v_pk_add_f16 removes the offset exactly, and
//     v_dot2_f32_f16 accumulates exact products in fp32;
//   - each wave handles RPW rows with all RPW*SPL loads issued before any math.
#include "common.hpp"

namespace luxhip {

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// sum_{i<32} (nib_i - 8) * x_i for one 16-byte slice.
__device__ __forceinline__ float dot_slice_f16(const uint32_t (&q)[4], const f16x2 (&xp)[4][4]) {
    const uint32_t MAGIC = 0x64006400u;
    const f16x2 OFF1 = {(f16)1032.0f, (f16)1032.0f};  // 1024 + 8
    const f16x2 OFF16 = {(f16)1152.0f, (f16)1152.0f}; // 1024 + 16*8
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t word = q[w];
        const uint32_t w8 = word >> 8;
        f16x2 v0 = as_h2((word & 0x000F000Fu) | MAGIC) - OFF1;   // (n0, n4) - 8
        f16x2 v1 = as_h2((word & 0x00F000F0u) | MAGIC) - OFF16;  // 16*((n1, n5) - 8)
        f16x2 v2 = as_h2((w8 & 0x000F000Fu) | MAGIC) - OFF1;     // (n2, n6) - 8
        f16x2 v3 = as_h2((w8 & 0x00F000F0u) | MAGIC) - OFF16;    // 16*((n3, n7) - 8)
        lo = __builtin_amdgcn_fdot2(v0, xp[w][0], lo, false);
        hi = __builtin_amdgcn_fdot2(v1, xp[w][1], hi, false);
        lo = __builtin_amdgcn_fdot2(v2, xp[w][2], lo, false);
        hi = __builtin_amdgcn_fdot2(v3, xp[w][3], hi, false);
    }
    return fmaf(hi, 0.0625f, lo);
}

template <int SPL, int RPW, ScaleKind SK, YKind YK>
__global__ __launch_bounds__(256) void k_qgemv_i4_f16(const u32x4* __restrict__ W,
                                                      const void* __restrict__ S,
                                                      const f16* __restrict__ x,
                                                      void* __restrict__ y, int n_out, int K,
                                                      int spg, uint32_t xor_mask) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
    if (row0 >= n_out) return;
    const int s_row = K >> 5;        // slices per row
    const int g_row = s_row / spg;   // groups per row

    f16x2 xp[SPL][4][4];
    int gid[SPL];
    bool ok[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        const int s = lane + 64 * j;
        ok[j] = s < s_row;
        gid[j] = s / spg;
        const f16x8* x8 = reinterpret_cast<const f16x8*>(x) + 4 * s;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            f16x8 v = ok[j] ? x8[w] : f16x8{};
            xp[j][w][0] = f16x2{v[0], v[4]};
            xp[j][w][1] = f16x2{v[1], v[5]};
            xp[j][w][2] = f16x2{v[2], v[6]};
            xp[j][w][3] = f16x2{v[3], v[7]};
        }
    }

    uint32_t q[RPW][SPL][4];
    float sc[RPW][SPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const int row = row0 + r;
            if (row < n_out && ok[j]) {
                u32x4 v = __builtin_nontemporal_load(W + (size_t)row * s_row + lane + 64 * j);
                q[r][j][0] = v.x ^ xor_mask; q[r][j][1] = v.y ^ xor_mask;
                q[r][j][2] = v.z ^ xor_mask; q[r][j][3] = v.w ^ xor_mask;
                sc[r][j] = load_scale_t<SK>(S, (size_t)row * g_row + gid[j]);
            } else {
                q[r][j][0] = q[r][j][1] = q[r][j][2] = q[r][j][3] = 0x88888888u;  // q = 0
                sc[r][j] = 0.f;
            }
        }

    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        acc[r] = 0.f;
#pragma unroll
        for (int j = 0; j < SPL; ++j) acc[r] = fmaf(dot_slice_f16(q[r][j], xp[j]), sc[r][j], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = wave_sum(acc[r]);
    if (lane < RPW) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < RPW; ++r) v = lane == r ? acc[r] : v;
        if (row0 + lane < n_out) store_y<YK>(y, row0 + lane, v);
    }
}

// Any activation dtype, any group size that is a multiple of 8: one wave per row,
// one u32 word (8 nibbles, always inside one group) per lane step.
template <XKind XK, YKind YK>
__global__ __launch_bounds__(256) void k_qgemv_i4_generic(const uint32_t* __restrict__ W,
                                                          const void* __restrict__ S,
                                                          ScaleKind sk, const void* __restrict__ x,
                                                          void* __restrict__ y, int n_out, int K,
                                                          int gs, uint32_t xor_mask) {
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
    if (lane == 0) store_y<YK>(y, row, acc);
}

template <int SPL, ScaleKind SK, YKind YK>
static void launch_fast(const QArgs& a, hipStream_t s) {
    constexpr int RPW = 4;
    const int waves = (a.n_out + RPW - 1) / RPW;
    hipLaunchKernelGGL((k_qgemv_i4_f16<SPL, RPW, SK, YK>), dim3((waves + 3) / 4), dim3(256), 0, s,
                       reinterpret_cast<const u32x4*>(a.w), a.s,
                       reinterpret_cast<const f16*>(a.x), a.y, a.n_out, a.k, a.group_size / 32,
                       a.xor_mask);
}

template <ScaleKind SK, YKind YK>
static bool dispatch_spl(const QArgs& a, hipStream_t s) {
    const int slices = a.k / 32;
    const int spl = (slices + 63) / 64;
    if (spl <= 1) launch_fast<1, SK, YK>(a, s);
    else if (spl <= 2) launch_fast<2, SK, YK>(a, s);
    else if (spl <= 4) launch_fast<4, SK, YK>(a, s);
    else if (spl <= 8) launch_fast<8, SK, YK>(a, s);
    else return false;
    return true;
}

template <ScaleKind SK>
static bool dispatch_y(const QArgs& a, hipStream_t s) {
    switch (a.y_kind) {
        case YKind::F32: return dispatch_spl<SK, YKind::F32>(a, s);
        case YKind::F16: return dispatch_spl<SK, YKind::F16>(a, s);
        case YKind::BF16: return dispatch_spl<SK, YKind::BF16>(a, s);
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
                               a.scale_kind, a.x, a.y, a.n_out, a.k, a.group_size, a.xor_mask);
            return true;
        case YKind::F16:
            hipLaunchKernelGGL((k_qgemv_i4_generic<XK, YKind::F16>), grid, block, 0, s, w, a.s,
                               a.scale_kind, a.x, a.y, a.n_out, a.k, a.group_size, a.xor_mask);
            return true;
        case YKind::BF16:
            hipLaunchKernelGGL((k_qgemv_i4_generic<XK, YKind::BF16>), grid, block, 0, s, w, a.s,
                               a.scale_kind, a.x, a.y, a.n_out, a.k, a.group_size, a.xor_mask);
            return true;
        default: return false;
    }
}

hipError_t launch_qgemv_i4(const QArgs& a, hipStream_t s) {
    const bool fast = a.x_kind == XKind::F16 && a.k % 32 == 0 && a.group_size % 32 == 0 &&
                      ((uintptr_t)a.w & 15u) == 0 && ((uintptr_t)a.x & 15u) == 0;
    bool launched = false;
    if (fast) {
        switch (a.scale_kind) {
            case ScaleKind::F16: launched = dispatch_y<ScaleKind::F16>(a, s); break;
            case ScaleKind::F32: launched = dispatch_y<ScaleKind::F32>(a, s); break;
            case ScaleKind::GroupScale: launched = dispatch_y<ScaleKind::GroupScale>(a, s); break;
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
