// Weight-only quantized matmul for small m (decode batches, m <= 64 per pass):
//   Y[m, n] = sum_k (q(n, k) * s(n, k / gs)) * X[m, k]
// int8 weights (per-row or per-group scales) and int4 weights (group scales).
//
// Reference: int8 -- dequantize_nax_int8_group then WGSL_MATMUL
// (quantized_nax.wgsl:364-386, src/webgpu_plugin.cpp:138-205); int4 --
// matmul_nax_grouped (quantized_nax.wgsl:568-626).  Config 3 of BASELINE.json:
// W 28672 x 8192 int8, per-row fp16 scales, X m x 8192 fp16 (m = 8, 32), fp16 out.
// At 16 to 63 flop per weight byte this is HBM-bound (the MFMA ridge is ~300).
//
// Numerics: int8 values are exact in fp16 and so are the fp16 activations, so every
// MFMA product is exact; the row scale multiplies the fp32 sum at the end (per-group
// scales multiply fp32 partial sums), which reassociates the reference's
// sum of (q*s)*x without extra rounding of the weights.  int4 weights are staged as
// fp16(q*s/fold) with one RNE rounding (relative error <= 2^-11), fold being the
// weight row's power-of-two scale fold (scale_fold_factor), which the epilogue
// multiplies back: any finite fp16 / fp32 / GroupScale scale stays in range.
//
// Layout (gfx950, v_mfma_f32_16x16x32_f16): A = W rows (16 per wave), B = X^T (16 tokens
// per m-tile).  Lane l owns weight row l % 16 and k-quarter l / 16: each lane streams
// 16 contiguous bytes of its row per load straight from HBM into registers (no LDS),
// decodes them to fp16 and feeds two (int8) or four (int4) MFMA k-steps.  X is staged
// once per block in LDS, in the element order the decode produces, and shared by the
// block's waves.  A block is NW waves x 16 rows; the host picks NW so that every CU
// gets one block when it can (28672 rows on 256 CUs: 7 waves of 16 rows).
#include <algorithm>

#include "common.hpp"

namespace luxhip {

namespace {

constexpr int KC = 256;            // k per staged X chunk
constexpr int XROW = KC + 8;       // LDS halves per staged X row (pad: conflict-free reads)
constexpr int MAXW = 8;            // max waves per block (256 VGPRs per lane)

__device__ __forceinline__ uint32_t pack_h2s(f16 a, f16 b) {
    return __builtin_bit_cast(uint32_t, f16x2{a, b});
}

__device__ __forceinline__ uint32_t and_or_s(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

// 4 signed bytes -> fp16 (b0, b2, b1, b3), exact: (b ^ 0x80) = b + 128 in [0, 255],
// (1024 + u) - 1152 = b.
__device__ __forceinline__ uint2 i8x4_to_f16(uint32_t w, uint32_t magic) {
    const f16x2 OFF = {(f16)1152.0f, (f16)1152.0f};
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t lo = and_or_s(u, 0x00FF00FFu, magic);
    const uint32_t hi = and_or_s(u >> 8, 0x00FF00FFu, magic);
    return uint2{__builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo) - OFF),
                 __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi) - OFF)};
}

// 8 offset-binary nibbles times an fp16 scale -> fp16(q*s) (RNE) in the order
// (k, k+4, k+1, k+5, k+2, k+6, k+3, k+7).
__device__ __forceinline__ f16x8 i4x8_to_f16(uint32_t w, f16x2 s2, uint32_t magic) {
    const f16x2 OFF = {(f16)1032.0f, (f16)1032.0f};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = and_or_s(w >> (4 * i), 0x000F000Fu, magic);
        o[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, t) - OFF) * s2);
    }
    return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}

}  // namespace

// WB: weight bits (8 or 4).  MT: m-tiles of 16 tokens (m <= 16 MT).  PERROW: int8 with
// one scale per row (applied after the k loop); otherwise int8 scales are applied per
// 32-k step (group size a multiple of 64) and int4 scales inside the decode.
template <int WB, int MT, bool PERROW, ScaleKind SK, XKind XK, YKind YK>
__global__ __launch_bounds__(64 * MAXW) void k_qgemm_small(
    const uint8_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ X,
    void* __restrict__ Y, int M, int N, int K, int gs, uint32_t xor_mask, const float* __restrict__ xfac,
    const float* __restrict__ wfold, EpiArgs epi) {
    __shared__ __attribute__((aligned(16))) f16 xs[2][16 * MT][XROW];

    const int nw = blockDim.x >> 6;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n0 = (blockIdx.x * nw + wv) * 16;
    // Weight row of tile row i (0..15).  SiluMul: the tile holds 8 gate rows g0 .. g0+7
    // (rows 0-7) and the matching up rows nh + g0 .. (rows 8-15), so a gate value and its
    // up value sit in lanes l and l + 32 of the accumulator.
    const bool sm = epi.kind == (int)Epi::SiluMul;
    const int nh = N / 2, g0 = n0 / 2;
    auto wrow_of = [&](int i) {
        if (!sm) return min(n0 + i, N - 1);
        return i < 8 ? min(g0 + i, nh - 1) : nh + min(g0 + i - 8, nh - 1);
    };
    const int r16 = lane & 15, kq = lane >> 4;
    const int G = K / gs;
    const uint32_t magic = 0x64006400u;

    // Per-row power-of-two factors of bf16 / fp32 activations, once per block.
    __shared__ float sfac[16 * MT];
    if constexpr (XK != XKind::F16) {
        if (tid < 16 * MT) sfac[tid] = tid < M ? xfac[tid] : 1.0f;
        __syncthreads();
    }

    // ---- X staging: 16*MT rows x KC k per chunk = 512*MT chunks of 8 elements.  A chunk is
    // loaded as one 16-byte vector (two for fp32) two k-chunks ahead of its use, into one of
    // two register sets, and written to LDS (converted to fp16, reordered into the decode
    // order) after the MFMAs of the chunk before it.  The L2 round trip of the X load is
    // then covered by a whole chunk of work; loaded one chunk ahead, the LDS write waited
    // for it every chunk (2 % at config 3 m = 32; lab copies without the weight stream
    // took 23 and 32 us of the 49 and 60).
    // Three or four m-tiles, and int8 with group scales and two, keep one register set (X
    // one chunk ahead): a second set does not fit beside their accumulators and scales.
    constexpr int XS = 2 * MT;                 // chunks per thread (blocks have >= 4 waves)
    constexpr int XV = XK == XKind::F32 ? 2 : 1;
    constexpr bool X2 = MT <= 2 && !(WB == 8 && !PERROW && MT == 2);
    const int xchunks = 16 * MT * (KC / 8);
    u32x4 xrs[X2 ? 2 : 1][XS][XV];
    auto load_xc = [&](int set, int k0) __attribute__((always_inline)) {
        u32x4 (&xr)[XS][XV] = xrs[set];
#pragma unroll
        for (int i = 0; i < XS; ++i) {
            const int c = tid + i * (int)blockDim.x;
            const int row = c / (KC / 8), kc = (c % (KC / 8)) * 8;
            if (c < xchunks && row < M) {
                const size_t e = (size_t)row * K + k0 + kc;
#pragma unroll
                for (int v = 0; v < XV; ++v)
                    xr[i][v] = reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(X) +
                                                              e * (XK == XKind::F32 ? 4 : 2))[v];
            } else {
#pragma unroll
                for (int v = 0; v < XV; ++v) xr[i][v] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_xc = [&](int set, int buf) __attribute__((always_inline)) {
        const u32x4 (&xr)[XS][XV] = xrs[set];
#pragma unroll
        for (int i = 0; i < XS; ++i) {
            const int c = tid + i * (int)blockDim.x;
            if (c >= xchunks) continue;
            const int row = c / (KC / 8), kc = (c % (KC / 8)) * 8;
            f16 h[8];
            if constexpr (XK == XKind::F16) {
                const f16x8 f = __builtin_bit_cast(f16x8, xr[i][0]);
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = f[e];
            } else if constexpr (XK == XKind::BF16) {
                // bf16 / fp32 rows are divided by their power-of-two factor (exact)
                const float inv = 1.0f / sfac[row];
                const uint32_t w[4] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    h[2 * q] = (f16)(__builtin_bit_cast(float, w[q] << 16) * inv);
                    h[2 * q + 1] = (f16)(__builtin_bit_cast(float, w[q] & 0xFFFF0000u) * inv);
                }
            } else {
                const float inv = 1.0f / sfac[row];
                const uint32_t w[8] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w,
                                       xr[i][XV - 1].x, xr[i][XV - 1].y, xr[i][XV - 1].z, xr[i][XV - 1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = (f16)(__builtin_bit_cast(float, w[e]) * inv);
            }
            u32x4 v;
            if constexpr (WB == 8)  // (0, 2, 1, 3) inside every 4
                v = u32x4{pack_h2s(h[0], h[2]), pack_h2s(h[1], h[3]), pack_h2s(h[4], h[6]), pack_h2s(h[5], h[7])};
            else                    // (0, 4, 1, 5, 2, 6, 3, 7) inside every 8
                v = u32x4{pack_h2s(h[0], h[4]), pack_h2s(h[1], h[5]), pack_h2s(h[2], h[6]), pack_h2s(h[3], h[7])};
            *reinterpret_cast<u32x4*>(&xs[buf][row][kc]) = v;
        }
    };

    // ---- weight stream: lane (row r16, quarter kq) reads 16 B per load.  int8: a load
    // covers 64 k (the quarter's 16 bytes = k 16 kq .. 16 kq + 15); int4: 128 k
    // (32 nibbles = k 32 kq .. 32 kq + 31).  The scales a load needs are fetched with it.
    constexpr int KPL = WB == 8 ? 64 : 128;    // k per load (whole wave)
    constexpr int LPC = KC / KPL;              // loads per X chunk
    constexpr int SPLD = WB == 8 ? (PERROW ? 0 : 4) : 1;  // scales per load per lane
    const int row = wrow_of(r16);
    // int4: 1 / fold of this lane's weight row (a power of two, so the division is exact)
    float winv = 1.0f;
    if constexpr (WB == 4) winv = 1.0f / wfold[row];
    const size_t rowbytes = (size_t)K * WB / 8;
    const uint8_t* wrow = W + (size_t)row * rowbytes + 16 * kq;

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{};

    const int nchunks = K / KC;
    u32x4 wq[2][LPC];                          // two chunks of weights in flight
    uint32_t sq[2][LPC][SPLD > 0 ? SPLD : 1];  // their raw scales
    auto load_w = [&](int slot, int chunk) __attribute__((always_inline)) {
        chunk = min(chunk, nchunks - 1);
#pragma unroll
        for (int l = 0; l < LPC; ++l) {
            wq[slot][l] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(wrow + (size_t)(chunk * LPC + l) * (KPL * WB / 8)));
            const int kbase = chunk * KC + l * KPL;
            if constexpr (WB == 4) {
                sq[slot][l][0] = load_scale_raw<SK>(S, (size_t)row * G + (kbase + 32 * kq) / gs);
            } else if constexpr (!PERROW) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sq[slot][l][r] = load_scale_raw<SK>(S, (size_t)wrow_of(4 * kq + r) * G + kbase / gs);
            }
        }
    };

    // One chunk: KC k from X buffer `buf` and weight registers `slot` (static).  The
    // slot's weights are decoded first, so its registers take the loads of chunk `next`
    // before this chunk's MFMAs run: the prefetch distance is two chunks plus the MFMA
    // and X-read time of one.
    constexpr int SPL = WB == 8 ? 2 : 4;       // 32-k steps per load
    auto chunk = [&](int buf, int slot, int next) __attribute__((always_inline)) {
        f16x8 av[LPC][SPL];
        uint32_t sc[LPC][SPLD > 0 ? SPLD : 1];
#pragma unroll
        for (int l = 0; l < LPC; ++l) {
            const u32x4 q = wq[slot][l];
            if constexpr (WB == 8) {
                // two k-steps of 32: bytes 0-7 and 8-15 of the lane's 16
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const uint2 p0 = i8x4_to_f16(st ? q.z : q.x, magic);
                    const uint2 p1 = i8x4_to_f16(st ? q.w : q.y, magic);
                    av[l][st] = __builtin_bit_cast(f16x8, u32x4{p0.x, p0.y, p1.x, p1.y});
                }
#pragma unroll
                for (int r = 0; r < (SPLD > 0 ? SPLD : 1); ++r) sc[l][r] = sq[slot][l][r];
            } else {
                // four k-steps of 32: word w covers k 32 kq + 8 w .. + 7 of this load
                const float sf = scale_from_raw<SK>(sq[slot][l][0]) * winv;
                const uint32_t words[4] = {q.x, q.y, q.z, q.w};
                if constexpr (SK == ScaleKind::F16) {
                    // an fp16 scale times a power of two is exact in fp16: q * s rounds once
                    const f16 s16 = (f16)sf;
                    const f16x2 s2 = {s16, s16};
#pragma unroll
                    for (int st = 0; st < 4; ++st) av[l][st] = i4x8_to_f16(words[st] ^ xor_mask, s2, magic);
                } else {
#pragma unroll
                    for (int st = 0; st < 4; ++st)
                        av[l][st] = __builtin_bit_cast(f16x8, dequant8_f32s(words[st] ^ xor_mask, sf));
                }
            }
        }
        load_w(slot, next);
#pragma unroll
        for (int l = 0; l < LPC; ++l)
#pragma unroll
            for (int st = 0; st < SPL; ++st)
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const int kx = WB == 8 ? l * KPL + 16 * kq + 8 * st : l * KPL + 32 * kq + 8 * st;
                    const f16x8 bx = *reinterpret_cast<const f16x8*>(&xs[buf][16 * t + r16][kx]);
                    if constexpr (WB == 4 || PERROW) {
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[l][st], bx, acc[t], 0, 0, 0);
                    } else {
                        const f32x4 pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[l][st], bx, f32x4{}, 0, 0, 0);
                        // D rows 4*(lane/16) + r: scales of those rows for this group
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(pr[r], scale_from_raw<SK>(sc[l][r]), acc[t][r]);
                    }
                }
    };

    // Chunks in pairs so the register slots are static; weights and X both run two chunks
    // ahead of use (X register set c % 2, then LDS buffer c % 2).
    if constexpr (X2) {
        load_xc(0, 0);
        if (nchunks > 1) load_xc(X2 ? 1 : 0, KC);
        load_w(0, 0);
        load_w(1, 1);
        store_xc(0, 0);
        __syncthreads();
        for (int c = 0; c < nchunks; c += 2) {
            if (c + 2 < nchunks) load_xc(0, (c + 2) * KC);
            chunk(0, 0, c + 2);
            if (c + 1 < nchunks) store_xc(X2 ? 1 : 0, 1);
            __syncthreads();
            if (c + 1 < nchunks) {
                if (c + 3 < nchunks) load_xc(X2 ? 1 : 0, (c + 3) * KC);
                chunk(1, 1, c + 3);
                if (c + 2 < nchunks) store_xc(0, 0);
                __syncthreads();
            }
        }
    } else {  // X one chunk ahead, one register set
        load_xc(0, 0);
        load_w(0, 0);
        load_w(1, 1);
        store_xc(0, 0);
        __syncthreads();
        for (int c = 0; c < nchunks; c += 2) {
            if (c + 1 < nchunks) load_xc(0, (c + 1) * KC);
            chunk(0, 0, c + 2);
            if (c + 1 < nchunks) store_xc(0, 1);
            __syncthreads();
            if (c + 1 < nchunks) {
                if (c + 2 < nchunks) load_xc(0, (c + 2) * KC);
                chunk(1, 1, c + 3);
                if (c + 2 < nchunks) store_xc(0, 0);
                __syncthreads();
            }
        }
    }

    // ---- epilogue: D[i][j] of a 16x16 tile sits in lane j + 16 * (i / 4), register i % 4;
    // i = weight row (n), j = token (m).  The scalings, then the output epilogue.
    float wf[4] = {1.0f, 1.0f, 1.0f, 1.0f};  // int4: scale folds of rows 4 kq .. 4 kq + 3
    if constexpr (WB == 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r) wf[r] = wfold[wrow_of(4 * kq + r)];
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int m = 16 * t + r16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 4 * kq + r;
            float v = acc[t][r];
            if constexpr (WB == 8 && PERROW) v *= load_scale_t<SK>(S, (size_t)wrow_of(i));
            if constexpr (WB == 4) v *= wf[r];
            if constexpr (XK != XKind::F16) v *= sfac[m];
            if (sm) {
                const float up = __shfl_xor(v, 32, 64);  // tile row i + 8 of the same token
                const int n = g0 + i;
                if (kq < 2 && m < M && n < nh) store_y<YK>(Y, (size_t)m * nh + n, silu_f(v) * up);
            } else {
                const int n = n0 + i;
                if (m < M && n < N) store_y<YK>(Y, (size_t)m * N + n, apply_epi(v, epi, m, n, N));
            }
        }
    }
}

// ---------------------------------------------------------------- int8, per-row scales, fp16 X
// The config-3 shape (int8 weights, one scale per row, fp16 activations, m <= 32) as a
// streaming kernel: HBM delivers contiguous spans far better than the 16 rows x 64 bytes
// per instruction that loading the MFMA layout straight into registers takes (on a
// 235 MB stream with 7 waves per CU: 7.1 against 5.4 TB/s), so
//   - each wave streams its 16 weight rows into its own LDS ring with direct-to-LDS loads,
//     4 rows x 256 contiguous bytes per instruction (one 256-k chunk of 16 rows = 4 loads),
//     R_PD chunks ahead; 16-byte unit b of tile row r sits at unit b ^ r of the row, so the
//     fragment reads (16 rows of one unit) hit 16 distinct bank groups;
//   - X goes global -> LDS the same way in super-chunks of R_SKC k (all rows of the
//     m-tiles, double-buffered): the block meets at a barrier once per super-chunk;
//   - int8 -> fp16 is exact and in natural k order: v_cvt_f16_i16 with SDWA reads a
//     sign-extended byte and writes one half of the register, 4 VALU per 4 weights.
//   - Lane (row r16, quarter kq) feeds k = 64 l + 16 kq + 8 st + 0..7 of a chunk to k-step
//     (l, st); the X fragment of token t is the same 16 bytes of X row t.
// A wave waits only for its own loads (s_waitcnt); the barrier publishes X.
namespace {
constexpr int R_PD = 3;      // weight chunks (256 k) in flight per wave
constexpr int R_XJ = 8;      // X loads per wave per super-chunk (<= 32 jobs, >= 4 waves)
// k per X super-chunk: 1024 with one m-tile, 512 with two (the double-buffered X then fits
// beside 7 weight rings)
constexpr int r_skc(int mt) { return mt == 1 ? 1024 : 512; }
constexpr int r_xp(int mt) { return 2 * r_skc(mt) + 16; }  // bytes per staged X row (+16: conflict-free)

// Two signed bytes of w (BYTE_0/1 or BYTE_2/3) -> two fp16, exact.
__device__ __forceinline__ uint32_t i8pair_lo_f16(uint32_t w) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1"
        : "=&v"(r)
        : "v"(w));
    return r;
}
__device__ __forceinline__ uint32_t i8pair_hi_f16(uint32_t w) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(r)
        : "v"(w));
    return r;
}

// s_waitcnt vmcnt(n) with lgkmcnt(0) (expcnt at its maximum), and vmcnt(n) alone.
constexpr int r_vmcnt_lgkm0(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4); }
constexpr int r_vmcnt(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

template <int N>
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(r_vmcnt(N)); }

size_t i8row_lds(int mt, int nw) { return (size_t)2 * 16 * mt * r_xp(mt) + (size_t)nw * R_PD * 4096 + 1024; }
}  // namespace

template <int MT, ScaleKind SK, YKind YK>
__global__ __launch_bounds__(64 * MAXW) void k_qgemm_i8row(const uint8_t* __restrict__ W, const void* __restrict__ S,
                                                         const f16* __restrict__ X, void* __restrict__ Y, int M, int N,
                                                         int K, EpiArgs epi) {
    // LDS: X [2][16 MT][R_XP] | weight rings [nw][R_PD][16 rows x 256 B] | spare 1 KB
    extern __shared__ __attribute__((aligned(16))) uint8_t xl[];
    const int nw = blockDim.x >> 6;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n0 = (blockIdx.x * nw + wv) * 16;
    const int r16 = lane & 15, kq = lane >> 4;
    constexpr int R_SKC = r_skc(MT), R_XP = r_xp(MT), CPS = R_SKC / 256;
    constexpr int XB = 16 * MT * R_XP;  // bytes per X buffer
    uint8_t* ring = xl + 2 * XB + wv * (R_PD * 4096);
    uint8_t* spare = xl + 2 * XB + nw * (R_PD * 4096);
    const int nchunks = K / 256, nsc = K / R_SKC;

    // X super-chunk loads: job j = 1 KB segment j % SEGS of token row j / SEGS (at most 32
    // jobs); wave w takes j = w + nw i.  Every wave issues R_XJ of them (the ones past the
    // last job read zeros into the spare 1 KB), so the count between any two loads of a wave
    // is fixed.
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(X), (short)0, (int)((size_t)M * K * 2), 0x00020000);
    constexpr int SEGS = R_SKC / 512;  // 1 KB segments per X row and super-chunk
    auto load_x = [&](int sc) {
        uint8_t* buf = xl + (sc & 1) * XB;
        const int k0 = min(sc, nsc - 1) * R_SKC;  // past the end: re-read the last (never used)
#pragma unroll
        for (int i = 0; i < R_XJ; ++i) {
            const int j = wv + nw * i;  // job: row j / SEGS, segment j % SEGS
            const bool ok = j < M * SEGS;
            const int row = j / SEGS, sg = j % SEGS;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (__attribute__((address_space(3))) void*)(ok ? buf + row * R_XP + 1024 * sg : spare), 16,
                ok ? (row * K + k0 + 512 * sg) * 2 + 16 * lane : M * K * 2, 0, 0, 0);
        }
    };

    // Weight loads of chunk c: instruction j covers tile rows 4 j .. 4 j + 3, 256 bytes each;
    // lane l -> row r = 4 j + l / 16, unit p = l % 16 of its LDS row, global unit p ^ r.
    // Rows past N re-read row N - 1 (never stored).
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), (short)0, (int)((size_t)N * K), 0x00020000);
    int woff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + (lane >> 4), p = lane & 15;
        woff[j] = min(n0 + r, N - 1) * K + 16 * (p ^ r);
    }
    auto load_w = [&](int c) {
        const int cc = min(c, nchunks - 1);  // past the end: re-read the last chunk (never used)
        uint8_t* slot = ring + (c % R_PD) * 4096;
        const int so = __builtin_amdgcn_readfirstlane(cc * 256);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (__attribute__((address_space(3))) void*)(slot + 1024 * j), 16,
                                                     woff[j], so, 0, kNontemporal);
    };

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{};

    load_x(0);
#pragma unroll
    for (int i = 0; i < R_PD; ++i) load_w(i);

    // Issue order per super-chunk: chunk p = 0 refills W(c + R_PD) then X(sc + 1); chunks
    // 1 .. CPS-1 refill W(c + R_PD).  The prologue (X(0), W(0..2)) has the same shape, so
    // the counts below hold from the start:
    //   - at the barrier, X(sc) is complete once the weight loads issued after it may
    //     remain: CPS == 4: W(c+1 .. c+3) = 12 loads; CPS == 2: W(c+2) = 4 (the barrier then
    //     also completes W(c), W(c+1));
    //   - chunk c's weights: the loads issued after W(c) (4 per chunk, R_XJ for an X
    //     super-chunk): CPS == 4: 8 at p = 0 and 16 at p = 1..3; CPS == 2: covered by the
    //     barrier at p = 0, 24 at p = 1.
    constexpr int WB_BAR = CPS == 4 ? 12 : 4;
    const int wrd = r16 * 256;  // this lane's row in a ring slot
    for (int sc = 0; sc < nsc; ++sc) {
        // the barrier publishes every wave's share of X(sc) and retires the other X buffer
        // (read in super-chunk sc - 1) for X(sc + 1)
        __builtin_amdgcn_s_waitcnt(r_vmcnt_lgkm0(WB_BAR));
        asm volatile("s_barrier" ::: "memory");
        const uint8_t* xbuf = xl + (sc & 1) * XB;
#pragma unroll
        for (int p = 0; p < CPS; ++p) {
            const int c = CPS * sc + p;
            if (CPS == 4) {
                if (p == 0) wait_vm<8>();
                else wait_vm<16>();
            } else {
                if (p == 0) wait_vm<WB_BAR>();
                else wait_vm<24>();
            }
            const uint8_t* slot = ring + (c % R_PD) * 4096 + wrd;
            u32x4 q[4];
#pragma unroll
            for (int l = 0; l < 4; ++l) q[l] = *reinterpret_cast<const u32x4*>(slot + 16 * ((4 * l + kq) ^ r16));
            __builtin_amdgcn_s_waitcnt(r_vmcnt_lgkm0(63));  // the slot is read: refill it
            load_w(c + R_PD);
            if (p == 0) load_x(sc + 1);
            f16x8 av[4][2];
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                av[l][0] = __builtin_bit_cast(f16x8, u32x4{i8pair_lo_f16(q[l].x), i8pair_hi_f16(q[l].x),
                                                           i8pair_lo_f16(q[l].y), i8pair_hi_f16(q[l].y)});
                av[l][1] = __builtin_bit_cast(f16x8, u32x4{i8pair_lo_f16(q[l].z), i8pair_hi_f16(q[l].z),
                                                           i8pair_lo_f16(q[l].w), i8pair_hi_f16(q[l].w)});
            }
            const uint8_t* xb = xbuf + p * 512;
#pragma unroll
            for (int l = 0; l < 4; ++l)
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int t = 0; t < MT; ++t) {
                        const f16x8 bx =
                            *reinterpret_cast<const f16x8*>(xb + (16 * t + r16) * R_XP + 2 * (64 * l + 16 * kq + 8 * st));
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[l][st], bx, acc[t], 0, 0, 0);
                    }
        }
    }
    __builtin_amdgcn_s_waitcnt(r_vmcnt_lgkm0(0));  // no LDS load may land after the block ends

    // epilogue: D[i][j] of a 16x16 tile sits in lane j + 16 (i / 4), register i % 4;
    // i = weight row (n), j = token (m).
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int m = 16 * t + r16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = n0 + 4 * kq + r;
            if (m < M && n < N) {
                const float v = acc[t][r] * load_scale_t<SK>(S, (size_t)n);
                store_y<YK>(Y, (size_t)m * N + n, apply_epi(v, epi, m, n, N));
            }
        }
    }
}

// The fast path above: int8, one scale per row (or none), fp16 X, m <= 32, no gated pair,
// K a multiple of the super-chunk, byte offsets within 31 bits.
static bool i8row_ok(const QArgs& a) {
    const bool perrow = a.group_size == a.k || a.scale_kind == ScaleKind::None;
    return a.wbits == 8 && perrow && a.x_kind == XKind::F16 && a.m <= 32 && a.epi.kind != (int)Epi::SiluMul &&
           a.k % r_skc(a.m <= 16 ? 1 : 2) == 0 && (size_t)a.m * a.k * 2 < (1ull << 31) && (size_t)a.n_out * a.k < (1ull << 31) &&
           ((uintptr_t)a.x & 15u) == 0 && ((uintptr_t)a.w & 15u) == 0;
}

template <int MT, ScaleKind SK, YKind YK>
static void launch_i8row(const QArgs& a, hipStream_t s) {
    const int cus = device_cus();
    const int tiles = (a.n_out + 15) / 16;
    int nw = 4;
    if (tiles % cus == 0 && tiles / cus <= MAXW) nw = tiles / cus;
    else if (tiles <= cus * MAXW && tiles >= cus) nw = (tiles + cus - 1) / cus;
    nw = std::max(4, std::min(nw, MAXW));  // >= 4: the X loads of a super-chunk fit R_XJ per wave
    while (i8row_lds(MT, nw) > 160 * 1024) --nw;
    static bool attr = [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_qgemm_i8row<MT, SK, YK>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        return true;
    }();
    (void)attr;
    hipLaunchKernelGGL((k_qgemm_i8row<MT, SK, YK>), dim3((tiles + nw - 1) / nw), dim3(64 * nw), i8row_lds(MT, nw), s,
                       reinterpret_cast<const uint8_t*>(a.w), a.s, reinterpret_cast<const f16*>(a.x), a.y, a.m,
                       a.n_out, a.k, a.epi);
}

template <ScaleKind SK, YKind YK>
static void launch_i8row_m(const QArgs& a, hipStream_t s) {
    if (a.m <= 16) launch_i8row<1, SK, YK>(a, s);
    else launch_i8row<2, SK, YK>(a, s);
}

template <ScaleKind SK>
static bool launch_i8row_y(const QArgs& a, hipStream_t s) {
    switch (a.y_kind) {
        case YKind::F32: launch_i8row_m<SK, YKind::F32>(a, s); return true;
        case YKind::F16: launch_i8row_m<SK, YKind::F16>(a, s); return true;
        case YKind::BF16: launch_i8row_m<SK, YKind::BF16>(a, s); return true;
        default: return false;
    }
}

static bool launch_i8row_any(const QArgs& a, hipStream_t s) {
    switch (a.scale_kind) {
        case ScaleKind::F16: return launch_i8row_y<ScaleKind::F16>(a, s);
        case ScaleKind::F32: return launch_i8row_y<ScaleKind::F32>(a, s);
        case ScaleKind::GroupScale: return launch_i8row_y<ScaleKind::GroupScale>(a, s);
        case ScaleKind::None: return launch_i8row_y<ScaleKind::None>(a, s);
        default: return false;
    }
}

bool qgemm_small_supported(const QArgs& a) {
    if (a.x_kind == XKind::I8 || a.y_kind == YKind::I32) return false;
    // weights and activations are read with 16-byte vector loads
    if (a.k % KC != 0 || ((uintptr_t)a.w & 15u) != 0 || ((uintptr_t)a.x & 15u) != 0) return false;
    if (a.wbits == 8) {
        const bool perrow = a.group_size == a.k || a.scale_kind == ScaleKind::None;
        return perrow || a.group_size % 64 == 0;
    }
    return a.wbits == 4 && a.group_size % 32 == 0 && a.scale_kind != ScaleKind::None;
}

template <int WB, int MT, bool PERROW, ScaleKind SK, XKind XK, YKind YK>
static void launch_one(const QArgs& a, const void* x, void* y, const float* xfac, int m, EpiArgs epi,
                       hipStream_t s) {
    // Waves per block, 4 .. MAXW: the count that spreads the 16-row tiles evenly over the
    // CUs (one block per CU) when there is one, else 4.  The X staging assumes >= 4.
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
    }
    const bool sm = a.epi.kind == (int)Epi::SiluMul;
    const int tiles = sm ? (a.n_out / 2 + 7) / 8 : (a.n_out + 15) / 16;
    int nw = 4;
    if (tiles % cus == 0 && tiles / cus <= MAXW) nw = tiles / cus;
    else if (tiles <= cus * MAXW && tiles >= cus) nw = (tiles + cus - 1) / cus;
    nw = std::max(4, std::min(nw, MAXW));
    const dim3 grid((tiles + nw - 1) / nw), block(64 * nw);
    hipLaunchKernelGGL((k_qgemm_small<WB, MT, PERROW, SK, XK, YK>), grid, block, 0, s,
                       reinterpret_cast<const uint8_t*>(a.w), a.s, x, y, m, a.n_out, a.k,
                       a.group_size, a.xor_mask, xfac, a.wfold, epi);
}

template <int WB, bool PERROW, ScaleKind SK, XKind XK, YKind YK>
static void launch_m(const QArgs& a, hipStream_t s) {
    // m > 64: passes of 64 tokens (each re-reads the weights).  int8 with group scales
    // takes 32 per pass: its per-step scale registers do not fit beside four m-tiles.
    constexpr int PASS = (WB == 8 && !PERROW) ? 32 : 64;
    const size_t xel = a.x_kind == XKind::F32 ? 4 : 2;
    const size_t yel = a.y_kind == YKind::F32 ? 4 : 2;
    const int ny = a.epi.kind == (int)Epi::SiluMul ? a.n_out / 2 : a.n_out;  // output columns
    for (int m0 = 0; m0 < a.m; m0 += PASS) {
        const int m = std::min(PASS, a.m - m0);
        const void* x = reinterpret_cast<const uint8_t*>(a.x) + (size_t)m0 * a.k * xel;
        void* y = reinterpret_cast<uint8_t*>(a.y) + (size_t)m0 * ny * yel;
        const float* xf = a.xfac ? a.xfac + m0 : nullptr;
        EpiArgs e = a.epi;
        if (e.residual) e.residual += (size_t)m0 * ny;
        if (m <= 16) {
            launch_one<WB, 1, PERROW, SK, XK, YK>(a, x, y, xf, m, e, s);
        } else if (m <= 32) {
            launch_one<WB, 2, PERROW, SK, XK, YK>(a, x, y, xf, m, e, s);
        } else if constexpr (PASS == 64) {
            if (m <= 48) launch_one<WB, 3, PERROW, SK, XK, YK>(a, x, y, xf, m, e, s);
            else launch_one<WB, 4, PERROW, SK, XK, YK>(a, x, y, xf, m, e, s);
        }
    }
}

template <int WB, bool PERROW, ScaleKind SK, XKind XK>
static bool launch_y(const QArgs& a, hipStream_t s) {
    switch (a.y_kind) {
        case YKind::F32: launch_m<WB, PERROW, SK, XK, YKind::F32>(a, s); return true;
        case YKind::F16: launch_m<WB, PERROW, SK, XK, YKind::F16>(a, s); return true;
        case YKind::BF16: launch_m<WB, PERROW, SK, XK, YKind::BF16>(a, s); return true;
        default: return false;
    }
}

template <int WB, bool PERROW, ScaleKind SK>
static bool launch_x(const QArgs& a, hipStream_t s) {
    switch (a.x_kind) {
        case XKind::F16: return launch_y<WB, PERROW, SK, XKind::F16>(a, s);
        case XKind::BF16: return launch_y<WB, PERROW, SK, XKind::BF16>(a, s);
        case XKind::F32: return launch_y<WB, PERROW, SK, XKind::F32>(a, s);
        default: return false;
    }
}

template <int WB, bool PERROW>
static bool launch_s(const QArgs& a, hipStream_t s) {
    switch (a.scale_kind) {
        case ScaleKind::F16: return launch_x<WB, PERROW, ScaleKind::F16>(a, s);
        case ScaleKind::F32: return launch_x<WB, PERROW, ScaleKind::F32>(a, s);
        case ScaleKind::GroupScale: return launch_x<WB, PERROW, ScaleKind::GroupScale>(a, s);
        case ScaleKind::None:
            if constexpr (WB == 8 && PERROW) return launch_x<WB, PERROW, ScaleKind::None>(a, s);
            return false;
        default: return false;
    }
}

// Per-row power-of-two factors of bf16 / fp32 activations (row_pow2_factor).
template <XKind XK>
__global__ __launch_bounds__(256) void k_row_factors(const void* __restrict__ X, int K,
                                                     float* __restrict__ fac) {
    __shared__ uint32_t red[16];
    const int row = blockIdx.x;
    uint32_t mx = 0;
    if constexpr (XK == XKind::F32) {
        const uint32_t* xr = reinterpret_cast<const uint32_t*>(X) + (size_t)row * K;
        for (int k = threadIdx.x; k < K; k += 256) mx = max(mx, xr[k] & 0x7FFFFFFFu);
    } else {
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(X) + (size_t)row * K;
        for (int k = threadIdx.x; k < K; k += 256) mx = max(mx, (uint32_t)(xr[k] & 0x7FFFu));
    }
    mx = block_max_u32(mx, red);
    if (threadIdx.x == 0) fac[row] = row_pow2_factor(mx, XK == XKind::F32 ? 23 : 7);
}

// Workspace: [scale folds: n_out floats (int4), padded to 16 B] [activation factors: m floats].
static size_t fold_bytes(const QArgs& a) {
    return a.wbits == 4 ? (((size_t)a.n_out * sizeof(float) + 15) & ~(size_t)15) : 0;
}

size_t qgemm_small_workspace(const QArgs& a) {
    return fold_bytes(a) + (a.x_kind == XKind::F16 ? 0 : (size_t)a.m * sizeof(float));
}

hipError_t launch_qgemm_small(const QArgs& a0, void* workspace, hipStream_t s) {
    QArgs a = a0;
    a.xfac = nullptr;
    a.wfold = nullptr;
    if (a.wbits == 4) {
        float* fold = static_cast<float*>(workspace);
        if (hipError_t e = launch_scale_fold(a.s, a.scale_kind, a.n_out, a.k / a.group_size, fold, s);
            e != hipSuccess)
            return e;
        a.wfold = fold;
    }
    if (a.x_kind == XKind::BF16 || a.x_kind == XKind::F32) {
        float* fac = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + fold_bytes(a));
        if (a.x_kind == XKind::BF16)
            hipLaunchKernelGGL(k_row_factors<XKind::BF16>, dim3(a.m), dim3(256), 0, s, a.x, a.k, fac);
        else
            hipLaunchKernelGGL(k_row_factors<XKind::F32>, dim3(a.m), dim3(256), 0, s, a.x, a.k, fac);
        a.xfac = fac;
    }
    bool ok;
    if (i8row_ok(a)) {
        ok = launch_i8row_any(a, s);
    } else if (a.wbits == 8) {
        const bool perrow = a.group_size == a.k || a.scale_kind == ScaleKind::None;
        ok = perrow ? launch_s<8, true>(a, s) : launch_s<8, false>(a, s);
    } else {
        ok = launch_s<4, false>(a, s);
    }
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

// One wave per weight row: fold[n] = scale_fold_factor(max_g |s(n, g)|).
template <ScaleKind SK>
__global__ __launch_bounds__(256) void k_scale_fold(const void* __restrict__ S, int N, int G,
                                                    float* __restrict__ fold) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const float f = row_scale_fold<SK>(S, (size_t)row, G, threadIdx.x & 63);
    if ((threadIdx.x & 63) == 0) fold[row] = f;
}

hipError_t launch_scale_fold(const void* s, ScaleKind sk, int n_out, int groups, float* fold, hipStream_t st) {
    const dim3 grid((n_out + 3) / 4), block(256);
    switch (sk) {
        case ScaleKind::F16: hipLaunchKernelGGL(k_scale_fold<ScaleKind::F16>, grid, block, 0, st, s, n_out, groups, fold); break;
        case ScaleKind::F32: hipLaunchKernelGGL(k_scale_fold<ScaleKind::F32>, grid, block, 0, st, s, n_out, groups, fold); break;
        case ScaleKind::GroupScale:
            hipLaunchKernelGGL(k_scale_fold<ScaleKind::GroupScale>, grid, block, 0, st, s, n_out, groups, fold);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace luxhip
