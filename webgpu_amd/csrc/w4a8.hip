// W4A8: int4 weights x int8 activations on the int8 MFMA, exact int32 sums.
//
// Reference: matmul_int4_int8 (quantized.wgsl:590-647): out[r, c] = sum_k w4(r, k) *
// a8(k, c) in i32, two's-complement nibbles (unpack_int4x8, quantized.wgsl:148-156).
// Config 5 of BASELINE.json adds group scales: W 11008 x 4096 int4 g128 (fp16
// scales), A 256 x 4096 int8 with per-token scales; int32 partial sums per group,
// then y = a_scale[m] * sum_g s[n, g] * P_g[m, n].
//
// Output modes (lux_hip_qmatmul descriptor):
//   y I32, no GROUP_PARTIALS : full-K int32 sums (the reference kernel's output);
//   y I32, GROUP_PARTIALS    : P[m][n][g] int32 per group (bit-exact checking aid);
//   y F16/BF16/F32           : the scaled sum above, fp32 accumulation of s * P_g.
//
// Layout (gfx950, v_mfma_i32_16x16x64_i8): A = weight rows (16 per wave), B = A8^T
// (16 tokens per m-tile), K = 64 per instruction.  Per 128-k group a lane (row l % 16,
// quarter q = l / 16) loads 16 packed bytes = k 32 q .. 32 q + 31 and sign-extends the
// nibbles into bytes with a SWAR add/xor, in the order (k0 k2 k4 k6 | k1 k3 k5 k7) per 8;
// the two MFMA k-steps of the group take nibbles 0-15 and 16-31.  Activations are
// staged per block in LDS with the same byte order.  int32 accumulation is exact.
#include <algorithm>

#include "common.hpp"

namespace luxhip {

namespace {

constexpr int GK = 128;            // k per stage (one group of 128 when gs == 128)
constexpr int AROW = GK + 16;      // LDS bytes per staged activation row (padded)
constexpr int BT = 256;            // tokens per block (m tile of the block)

// 8 offset-binary nibbles (k0..k7) -> two words of signed bytes
// (k0, k2, k4, k6) and (k1, k3, k5, k7): byte = ((u + 0x78) ^ 0x80) with u = q + 8.
__device__ __forceinline__ void unpack_i4_to_i8(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u0 = w & 0x0F0F0F0Fu, u1 = (w >> 4) & 0x0F0F0F0Fu;
    lo = (u0 + 0x78787878u) ^ 0x80808080u;
    hi = (u1 + 0x78787878u) ^ 0x80808080u;
}

// 8 activation bytes (a0..a7 as two words) -> (a0 a2 a4 a6) (a1 a3 a5 a7).
__device__ __forceinline__ void perm_bytes(uint32_t x, uint32_t y, uint32_t& lo, uint32_t& hi) {
    // v_perm_b32 selects bytes of {src0, src1}: src1 bytes are 0-3, src0 bytes 4-7.
    lo = __builtin_amdgcn_perm(y, x, 0x06040200u);
    hi = __builtin_amdgcn_perm(y, x, 0x07050301u);
}

}  // namespace

// MODE 0: full-K int32; 1: per-group int32 partials; 2: scaled fp output.
template <int MODE, int MT, ScaleKind SK, YKind YK>
__global__ __launch_bounds__(256) void k_w4a8(const uint32_t* __restrict__ W,
                                              const void* __restrict__ S,
                                              const int8_t* __restrict__ A,
                                              const float* __restrict__ AS,
                                              void* __restrict__ Y, int M, int N, int K, int gs,
                                              uint32_t xor_mask) {
    __shared__ __attribute__((aligned(16))) uint8_t as[2][BT][AROW];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // block: 32 weight rows x BT tokens; wave: 16 rows (wv & 1) x 16*MT tokens (wv >> 1)
    const int n0 = blockIdx.x * 32 + (wv & 1) * 16;
    const int tb = blockIdx.y * BT;                    // first token of the block
    const int t0 = (wv >> 1) * 16 * MT;                // first token of the wave (in block)
    const int r16 = lane & 15, q = lane >> 4;
    const int G = K / gs;
    const int row = min(n0 + r16, N - 1);
    const uint8_t* wrow = reinterpret_cast<const uint8_t*>(W) + (size_t)row * (K / 2) + 16 * q;

    // ---- activation staging: BT tokens x GK bytes; thread t stages token t (8 x 16 B)
    auto stage_a = [&](int buf, int k0) {
        const int tok = tb + tid;
        uint8_t* dst = &as[buf][tid][0];
        if (tok < M) {
            const u32x4* src = reinterpret_cast<const u32x4*>(A + (size_t)tok * K + k0);
#pragma unroll
            for (int c = 0; c < GK / 16; ++c) {
                const u32x4 v = src[c];
                uint32_t a, b, cc, d;
                perm_bytes(v.x, v.y, a, b);
                perm_bytes(v.z, v.w, cc, d);
                *reinterpret_cast<u32x4*>(dst + 16 * c) = u32x4{a, b, cc, d};
            }
        } else {
#pragma unroll
            for (int c = 0; c < GK / 16; ++c) *reinterpret_cast<u32x4*>(dst + 16 * c) = u32x4{0u, 0u, 0u, 0u};
        }
    };

    i32x4 iacc[MT];
    f32x4 facc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        iacc[t] = i32x4{0, 0, 0, 0};
        facc[t] = f32x4{};
    }

    const int nst = K / GK;
    u32x4 wq = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow));
    stage_a(0, 0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        const int k0 = st * GK;
        u32x4 wn = wq;
        if (st + 1 < nst) {
            wn = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + (size_t)(st + 1) * (GK / 2)));
            stage_a(buf ^ 1, k0 + GK);
        }
        // weights of this stage: k 32 q .. 32 q + 31 -> two k-steps of 16 bytes each
        uint32_t b8[8];
        const uint32_t wwords[4] = {wq.x ^ xor_mask, wq.y ^ xor_mask, wq.z ^ xor_mask, wq.w ^ xor_mask};
#pragma unroll
        for (int i = 0; i < 4; ++i) unpack_i4_to_i8(wwords[i], b8[2 * i], b8[2 * i + 1]);
        // A group spans gs / 128 stages: the int32 partial is carried across them and
        // emitted (MODE 1) or scaled into fp32 (MODE 2) at the group's last stage.
        const bool gstart = k0 % gs == 0, gend = (k0 + GK) % gs == 0;
        float sr[4] = {1.f, 1.f, 1.f, 1.f};
        if constexpr (MODE == 2) {
            if (gend) {
                const int g = k0 / gs;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sr[r] = load_scale_t<SK>(S, (size_t)min(n0 + 4 * q + r, N - 1) * G + g);
            }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint8_t* arow = &as[buf][t0 + 16 * t + r16][32 * q];
            i32x4 p = (MODE == 0 || !gstart) ? iacc[t] : i32x4{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const i32x4 a = i32x4{(int)b8[4 * ks], (int)b8[4 * ks + 1], (int)b8[4 * ks + 2], (int)b8[4 * ks + 3]};
                const i32x4 b = *reinterpret_cast<const i32x4*>(arow + 16 * ks);
                p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, p, 0, 0, 0);
            }
            iacc[t] = p;
            if constexpr (MODE == 1) {
                // P[m][n][g]: D[i][j] = lane j + 16 (i / 4), register i % 4; i = row, j = token
                const int m = tb + t0 + 16 * t + r16;
                const int g = k0 / gs;
                if (gend && m < M) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = n0 + 4 * q + r;
                        if (n < N) reinterpret_cast<int32_t*>(Y)[((size_t)m * N + n) * G + g] = p[r];
                    }
                }
            } else if constexpr (MODE == 2) {
                if (gend) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) facc[t][r] = fmaf((float)p[r], sr[r], facc[t][r]);
                }
            }
        }
        wq = wn;
        __syncthreads();
    }

    if constexpr (MODE != 1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int m = tb + t0 + 16 * t + r16;
            if (m >= M) continue;
            const float asc = MODE == 2 ? AS[m] : 1.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = n0 + 4 * q + r;
                if (n >= N) continue;
                if constexpr (MODE == 0) reinterpret_cast<int32_t*>(Y)[(size_t)m * N + n] = iacc[t][r];
                else store_y<YK>(Y, (size_t)m * N + n, facc[t][r] * asc);
            }
        }
    }
}

bool w4a8_supported(const QArgs& a) {
    // groups must hold whole 128-k stages; activations/weights 16-byte aligned
    if (a.wbits != 4 || a.x_kind != XKind::I8) return false;
    if (a.k % GK != 0 || a.group_size % GK != 0) return false;
    if (((uintptr_t)a.w & 15u) != 0 || ((uintptr_t)a.x & 15u) != 0) return false;
    if (a.y_kind == YKind::I32) return true;  // raw sums or per-group partials: no scales used
    return a.scale_kind != ScaleKind::None && a.xs != nullptr;
}

template <int MODE, ScaleKind SK, YKind YK>
static void launch_t(const QArgs& a, hipStream_t s) {
    constexpr int MT = BT / 2 / 16;  // 8 m-tiles of 16 tokens per wave
    const dim3 grid((a.n_out + 31) / 32, (a.m + BT - 1) / BT), block(256);
    hipLaunchKernelGGL((k_w4a8<MODE, MT, SK, YK>), grid, block, 0, s,
                       reinterpret_cast<const uint32_t*>(a.w), a.s,
                       reinterpret_cast<const int8_t*>(a.x), a.xs, a.y, a.m, a.n_out, a.k,
                       a.group_size, a.xor_mask);
}

template <ScaleKind SK>
static bool launch_scaled(const QArgs& a, hipStream_t s) {
    switch (a.y_kind) {
        case YKind::F32: launch_t<2, SK, YKind::F32>(a, s); return true;
        case YKind::F16: launch_t<2, SK, YKind::F16>(a, s); return true;
        case YKind::BF16: launch_t<2, SK, YKind::BF16>(a, s); return true;
        default: return false;
    }
}

hipError_t launch_w4a8(const QArgs& a, hipStream_t s) {
    bool ok = true;
    if (a.y_kind == YKind::I32) {
        if (a.group_partials) launch_t<1, ScaleKind::None, YKind::I32>(a, s);
        else launch_t<0, ScaleKind::None, YKind::I32>(a, s);
    } else {
        switch (a.scale_kind) {
            case ScaleKind::F16: ok = launch_scaled<ScaleKind::F16>(a, s); break;
            case ScaleKind::F32: ok = launch_scaled<ScaleKind::F32>(a, s); break;
            case ScaleKind::GroupScale: ok = launch_scaled<ScaleKind::GroupScale>(a, s); break;
            default: ok = false;
        }
    }
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace luxhip
