// W4A8 / W8A8: int4 or int8 weights x int8 activations on the int8 MFMA, exact int32 sums.
//
// Reference: matmul_int4_int8 (quantized.wgsl:590-647): out[r, c] = sum_k w4(r, k) *
// a8(k, c) in i32, two's-complement nibbles (unpack_int4x8, quantized.wgsl:148-156);
// matmul_int8 (quantized.wgsl:497-555): the same with int8 weights (unpack_int8x4,
// :167-178).  int8 weights skip the nibble decode and keep the natural k order.
// Config 5 of BASELINE.json adds group scales: W 11008 x 4096 int4 g128 (fp16
// scales), A 256 x 4096 int8 with per-token scales; int32 partial sums per group,
// then y = a_scale[m] * sum_g s[n, g] * P_g[m, n].
//
// Output modes (lux_hip_qmatmul descriptor):
//   y I32, no GROUP_PARTIALS : full-K int32 sums (the reference kernel's output);
//   y I32, GROUP_PARTIALS    : P[m][n][g] int32 per group (bit-exact checking aid);
//   y F16/BF16/F32           : the scaled sum above, fp32 accumulation of s * P_g in
//                              group order g = 0 .. G-1.
//
// Tiling (gfx950, v_mfma_i32_16x16x64_i8, A = weight rows, B = tokens, K = 64):
//   a wave = 16 rows (one row tile) x 64 tokens (4 token tiles, 4 independent MFMA
//   chains); a block = NWB waves over 16 NWB rows and the same 64 tokens.  NWB = 4 lets
//   up to three blocks share a CU, so one block's barrier and memory waits overlap
//   another's MFMAs; NWB = 11 (176 rows, one block per CU; config 5: 252 blocks on 256
//   CUs) stages each token block's activations for 176 rows instead of 64.  Per 128-k
//   stage a lane (row l % 16, quarter q = l / 16) loads 16 packed bytes per row tile =
//   k 32 q .. 32 q + 31 and turns the nibbles into bytes in the order
//   (k0 k2 k4 k6 | k1 k3 k5 k7) per 8 k: sign-extended by a SWAR add/xor, or, for the
//   scaled g128 path with fp16 scales, left as 16 q in the top of each byte.  The two
//   MFMA k-steps take nibbles 0-15 and 16-31.  Activations of the stage (64 tokens x
//   128 B) are loaded as coalesced 16-B chunks PD stages ahead, byte-permuted into the
//   same order and written to LDS; all the block's waves read them.  The weights are
//   the only operand each wave owns, so nothing is decoded twice.
//   The scaled output costs two VALU per int32 sum and group (convert, fma), as many
//   issue cycles as the group's MFMAs; with NWB = 11 it runs a stage late, after the
//   next stage's MFMAs, so it never waits on a result just issued.
//
// Block order is XCD-aware: consecutive workgroups go to the 8 XCDs in turn, so the
// token blocks of one row block are given block ids that land on the same XCD and
// share its L2 copy of the block's weight rows.
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace luxhip {

namespace {

constexpr int GK = 128;    // k per stage (one group of 128 when gs == 128)
constexpr int AROW = GK + 16;  // LDS bytes per staged token row (padded)
constexpr int RT = 1;      // 16-row MFMA tiles per wave
constexpr int BT = 64;     // tokens per block
constexpr int NXCD = 8;
constexpr int PD = 3;      // stages fetched ahead
constexpr int GMAX = 128;  // groups per row held in LDS (scaled output)
constexpr int SCH = 8;     // 16-byte scale chunks per thread (block region <= 32 KB)

// 8 nibbles (k0..k7) of one word -> 16 x signed values as bytes, in the same order: the
// nibbles moved to the top of each byte (16 q for two's complement, 16 q + 128 for
// offset-binary, which the xor with 0x80 per byte turns into 16 q).  3 VALU per word
// instead of 7; the group partials come out 16 x larger (exact: |16 P_g| <= 2^21 at
// 128 k), and the staged scale is s / 16 (exact for fp16 scales), so every fma
// s * P_g + acc sees the same operands' product and rounds the same.
__device__ __forceinline__ void unpack_i4_to_i8x16(uint32_t w, uint32_t xm, uint32_t& lo, uint32_t& hi) {
    lo = ((w << 4) & 0xF0F0F0F0u) ^ xm;
    hi = (w & 0xF0F0F0F0u) ^ xm;
}

// 8 nibbles (k0..k7) of one word -> signed bytes (k0, k2, k4, k6) and (k1, k3, k5, k7).
// Offset-binary u = q + 8: byte = (u + 0x78) ^ 0x80.  Two's complement t: u = t ^ 8,
// folded in through `tc` (0x08080808 for two's complement, 0 for offset-binary).
__device__ __forceinline__ void unpack_i4_to_i8(uint32_t w, uint32_t tc, uint32_t& lo, uint32_t& hi) {
    const uint32_t u0 = w & 0x0F0F0F0Fu, u1 = (w >> 4) & 0x0F0F0F0Fu;
    lo = ((u0 ^ tc) + 0x78787878u) ^ 0x80808080u;
    hi = ((u1 ^ tc) + 0x78787878u) ^ 0x80808080u;
}

// 8 activation bytes (a0..a7 as two words) -> (a0 a2 a4 a6) (a1 a3 a5 a7).
__device__ __forceinline__ void perm_bytes(uint32_t x, uint32_t y, uint32_t& lo, uint32_t& hi) {
    // v_perm_b32 selects bytes of {src0, src1}: src1 bytes are 0-3, src0 bytes 4-7.
    lo = __builtin_amdgcn_perm(y, x, 0x06040200u);
    hi = __builtin_amdgcn_perm(y, x, 0x07050301u);
}

__device__ __forceinline__ u32x4 perm16(u32x4 v) {
    uint32_t a, b, c, d;
    perm_bytes(v.x, v.y, a, b);
    perm_bytes(v.z, v.w, c, d);
    return u32x4{a, b, c, d};
}

}  // namespace

// MODE 0: full-K int32; 1: per-group int32 partials; 2: scaled fp output.
// ONEG: group size == 128, every stage is one whole group (no carry across stages).
template <int WB, int MODE, bool ONEG, ScaleKind SK, YKind YK, int NWB = 4, bool DEF = false>
__global__ __launch_bounds__(64 * NWB, NWB == 4 ? (MODE == 1 ? 2 : 3) : 1) void k_w4a8(const uint8_t* __restrict__ W,
                                              const void* __restrict__ S,
                                              const int8_t* __restrict__ A,
                                              const float* __restrict__ AS,
                                              void* __restrict__ Y, int M, int N, int K, int gs,
                                              uint32_t tc, int nrb, int ntb, int vec_y) {
    constexpr int NTB = 64 * NWB;                      // threads
    constexpr int BR = 16 * RT * NWB;                  // weight rows of the block
    constexpr int CPT = (BT * 8 + NTB - 1) / NTB;      // activation chunks per thread and stage
    constexpr int SCHB = (256 * SCH + NTB - 1) / NTB;  // scale chunks per thread (<= 32 KB)
    __shared__ __attribute__((aligned(16))) uint8_t as[2][BT][AROW];
    extern __shared__ __attribute__((aligned(16))) float ssT[];  // MODE 2: [G][BR] scales

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wvu = __builtin_amdgcn_readfirstlane(wv);  // the same, as a wave-uniform value
    const int b = blockIdx.x, j = b / NXCD;
    const int rb = (j / ntb) * NXCD + b % NXCD, tbk = j % ntb;
    if (rb >= nrb) return;  // whole block: no barrier is skipped by part of it
    const int n0 = rb * BR + wv * 16 * RT;  // first weight row of the wave
    const int tb = tbk * BT;           // first token of the block
    const int r16 = lane & 15, q = lane >> 4;
    const int G = K / gs;
    const int nst = K / GK;
    // Scaled output, one group per stage, fp16 scales: decode to 16 q (unpack_i4_to_i8x16).
    constexpr bool X16 = WB == 4 && MODE == 2 && ONEG && SK == ScaleKind::F16;
    // DEFER: the group scaling of stage s runs in stage s + 1, after that stage's MFMAs, so
    // the conversions read results finished a stage earlier; PD partial sets rotate with
    // the unrolled stages (same fma order, same results).
    constexpr bool DEFER = MODE == 2 && ONEG && DEF;
    const uint32_t xm = tc ? 0u : 0x80808080u;

    // Raw buffer loads: each lane keeps a fixed byte offset (voffset) and the stage
    // moves a uniform offset (soffset, scalar arithmetic only).  Reads past the end of
    // a buffer return zeros, so rows >= N and tokens >= M need no clamping (their
    // results are never stored); prefetches past the last stage read harmless data.
    // int4: a row is K / 2 bytes and a lane's 32 k are 16 bytes; int8: K bytes and 32.
    constexpr int LW = WB == 4 ? 1 : 2;  // 16-byte loads per lane, row tile and stage
    const int rowb = K / 8 * WB;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), (short)0, (int)((size_t)N * rowb), 0x00020000);
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(A), (short)0, (int)((size_t)M * K), 0x00020000);
    const int wv0 = (n0 + r16) * rowb + 16 * LW * q;
    // activation chunks of a stage: 64 tokens x 8 chunks of 16 B; chunk c = tid + NTB i is
    // token c / 8, part c % 8 (8 lanes read one token's 128 contiguous bytes)
    int av[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + NTB * i;
        av[i] = (tb + (c >> 3)) * K + 16 * (c & 7);
    }

    auto ldw = [&](u32x4 (&w)[RT * LW], int st) {
        const int so = __builtin_amdgcn_readfirstlane(st * (GK / 8 * WB));
#pragma unroll
        for (int f = 0; f < RT; ++f)
#pragma unroll
            for (int h = 0; h < LW; ++h)
                w[f * LW + h] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wv0 + f * 16 * rowb + 16 * h, so, 0));
    };
    auto lda = [&](u32x4 (&a)[CPT], int st) {
        const int so = __builtin_amdgcn_readfirstlane(st * GK);
#pragma unroll
        for (int i = 0; i < CPT; ++i)
            if (NTB * (i + 1) <= BT * 8 || 64 * wvu + NTB * i < BT * 8)  // whole waves
                a[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, av[i], so, 0));
    };
    // int4 weights decode to (k0 k2 k4 k6 | k1 k3 k5 k7) per 8 k, so the activations are
    // permuted the same way; int8 weights keep the natural order on both sides.
    auto sta = [&](int buf, const u32x4 (&a)[CPT]) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + NTB * i;
            if (NTB * (i + 1) <= BT * 8 || 64 * wvu + NTB * i < BT * 8)
                *reinterpret_cast<u32x4*>(&as[buf][c >> 3][16 * (c & 7)]) = WB == 4 ? perm16(a[i]) : a[i];
        }
    };

    i32x4 iacc[RT][4];
    f32x4 facc[RT][4];
#pragma unroll
    for (int f = 0; f < RT; ++f)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            iacc[f][t] = i32x4{0, 0, 0, 0};
            facc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

    // The block's group scales (rows rb * BR .. + BR - 1 of [N][G]: one contiguous
    // region) are loaded first, then the first PD stages; then the scales are
    // converted to fp32 and transposed into ssT[g][row] (rows past N read zeros).
    u32x4 sv[SCHB];
    constexpr int SB = SK == ScaleKind::F16 ? 2 : SK == ScaleKind::GroupScale ? 16 : 4;
    constexpr int EPC = SK == ScaleKind::F16 ? 8 : SK == ScaleKind::GroupScale ? 1 : 4;  // per 16 B
    const int nch = BR * G * SB / 16;
    if constexpr (MODE == 2) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void*>(S), (short)0, (int)((size_t)N * G * SB), 0x00020000);
        const int base = rb * BR * G * SB;
#pragma unroll
        for (int c = 0; c < SCHB; ++c) {
            const int ch = tid + NTB * c;
            if (ch < nch) sv[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, base + 16 * ch, 0, 0));
        }
    }
    // Weights and activations of stage st + PD are fetched while stage st computes:
    // PD register sets, the loop unrolled by PD so each set is a fixed set of
    // registers.  Set i: W[i] holds the weights of the stage it serves; A[i] its
    // activations, written to LDS at the end of the previous stage.
    u32x4 Wr[PD][RT * LW], Ar[PD][CPT];
#pragma unroll
    for (int i = 0; i < PD; ++i) {
        ldw(Wr[i], i);
        lda(Ar[i], i);
    }
    if constexpr (MODE == 2) {
#pragma unroll
        for (int c = 0; c < SCHB; ++c) {
            const int ch = tid + NTB * c;
            if (ch < nch) {
                int row = ch * EPC / G, g = ch * EPC % G;  // walked forward: one division per chunk
#pragma unroll
                for (int e = 0; e < EPC; ++e) {
                    const uint32_t wd = sv[c][SK == ScaleKind::F16 ? e / 2 : e];
                    const uint32_t raw = SK == ScaleKind::F16 ? (wd >> (16 * (e & 1))) & 0xFFFFu : wd;
                    ssT[g * BR + row] = X16 ? scale_from_raw<SK>(raw) * 0.0625f : scale_from_raw<SK>(raw);
                    if (++g == G) {
                        g = 0;
                        ++row;
                    }
                }
            }
        }
    }
    sta(0, Ar[0]);
    __syncthreads();

    i32x4 pb[DEFER ? PD : 1][RT][4];
    auto scale_into = [&](const i32x4 (&pp)[RT][4], int g) {
        f32x4 sg[RT];
#pragma unroll
        for (int f = 0; f < RT; ++f) sg[f] = *reinterpret_cast<const f32x4*>(&ssT[g * BR + wv * 16 * RT + 16 * f + 4 * q]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int f = 0; f < RT; ++f)
#pragma unroll
                for (int r = 0; r < 4; ++r) facc[f][t][r] = fmaf((float)pp[f][t][r], sg[f][r], facc[f][t][r]);
    };
    auto stage = [&](int st, u32x4 (&wc)[RT * LW], u32x4 (&ac)[CPT], const u32x4 (&an)[CPT], auto IDX) {
        constexpr int si = decltype(IDX)::value;  // the stage's slot in the unrolled group of PD
        const int buf = st & 1;
        const int k0 = st * GK;
        const bool gstart = ONEG || k0 % gs == 0, gend = ONEG || (k0 + GK) % gs == 0;
        const int g = ONEG ? st : k0 / gs;
        uint32_t b8[RT][8];
#pragma unroll
        for (int f = 0; f < RT; ++f) {
            if constexpr (WB == 4) {
                const uint32_t ww[4] = {wc[f].x, wc[f].y, wc[f].z, wc[f].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (X16) unpack_i4_to_i8x16(ww[i], xm, b8[f][2 * i], b8[f][2 * i + 1]);
                    else unpack_i4_to_i8(ww[i], tc, b8[f][2 * i], b8[f][2 * i + 1]);
                }
            } else {
                const u32x4 w0 = wc[2 * f], w1 = wc[2 * f + 1];
                const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) b8[f][i] = ww[i];
            }
        }
        ldw(wc, st + PD);
        lda(ac, st + PD);
        // B fragments of the 4 token tiles, then 8 independent MFMA chains (k-step 0 of
        // every tile before k-step 1), then the per-group epilogue of each tile.
        i32x4 bk[4][2];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint8_t* arow = &as[buf][16 * t + r16][32 * q];
            bk[t][0] = *reinterpret_cast<const i32x4*>(arow);
            bk[t][1] = *reinterpret_cast<const i32x4*>(arow + 16);
        }
        f32x4 sc[RT];
        if constexpr (MODE == 2 && !DEFER) {
            // scales of this lane's D rows 16 f + 4 q + r for the group
#pragma unroll
            for (int f = 0; f < RT; ++f) sc[f] = *reinterpret_cast<const f32x4*>(&ssT[g * BR + wv * 16 * RT + 16 * f + 4 * q]);
        }
        i32x4 (&p)[RT][4] = pb[DEFER ? si : 0];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int f = 0; f < RT; ++f) p[f][t] = (MODE == 0 || !gstart) ? iacc[f][t] : i32x4{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int f = 0; f < RT; ++f) {
                    const i32x4 a = i32x4{(int)b8[f][4 * ks], (int)b8[f][4 * ks + 1], (int)b8[f][4 * ks + 2],
                                          (int)b8[f][4 * ks + 3]};
                    p[f][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bk[t][ks], p[f][t], 0, 0, 0);
                }
        if constexpr (DEFER) {
            if (st > 0) scale_into(pb[(si + PD - 1) % PD], g - 1);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int f = 0; f < RT; ++f) {
                if (MODE == 0 || !ONEG) iacc[f][t] = p[f][t];
                if constexpr (MODE == 1) {
                    // P[m][n][g]: D row (weight) 16 f + 4 q + r, column (token) r16
                    const int m = tb + 16 * t + r16;
                    if (gend && m < M) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int n = n0 + 16 * f + 4 * q + r;
                            if (n < N) reinterpret_cast<int32_t*>(Y)[((size_t)m * N + n) * G + g] = p[f][t][r];
                        }
                    }
                } else if constexpr (MODE == 2 && !DEFER) {
                    if (gend) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) facc[f][t][r] = fmaf((float)p[f][t][r], sc[f][r], facc[f][t][r]);
                    }
                }
            }
        sta(buf ^ 1, an);  // buf ^ 1 was last read before the previous barrier
        __syncthreads();
    };

    static_assert(PD == 3, "the unrolled stage group below is written out for PD = 3");
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    int st = 0;
    for (; st + PD <= nst; st += PD) {
        stage(st, Wr[0], Ar[0], Ar[1], I0{});
        stage(st + 1, Wr[1], Ar[1], Ar[2], I1{});
        stage(st + 2, Wr[2], Ar[2], Ar[0], I2{});
    }
    if (st < nst) stage(st, Wr[0], Ar[0], Ar[1], I0{});
    if (st + 1 < nst) stage(st + 1, Wr[1], Ar[1], Ar[2], I1{});
    if constexpr (DEFER) {  // the last stage's scaling
        const int last = (nst - 1) % PD;
        if (last == 0) scale_into(pb[0], nst - 1);
        else if (last == 1) scale_into(pb[1], nst - 1);
        else scale_into(pb[DEFER ? 2 : 0], nst - 1);
    }

    if constexpr (MODE != 1) {
        const bool vec_n = vec_y != 0;  // N % 4 == 0 and Y 16-byte aligned
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int m = tb + 16 * t + r16;
            if (m >= M) continue;
            const float asc = MODE == 2 ? AS[m] : 1.0f;
#pragma unroll
            for (int f = 0; f < RT; ++f) {
                const int n = n0 + 16 * f + 4 * q;
                if (n >= N) continue;
                const bool full = vec_n && n + 3 < N;
                if constexpr (MODE == 0) {
                    int32_t* y = reinterpret_cast<int32_t*>(Y) + (size_t)m * N + n;
                    if (full) {
                        *reinterpret_cast<i32x4*>(y) = iacc[f][t];
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (n + r < N) y[r] = iacc[f][t][r];
                    }
                } else {
                    const f32x4 v = facc[f][t] * asc;
                    if (full) {
                        store_y4<YK>(Y, (size_t)m * N + n, v);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (n + r < N) store_y<YK>(Y, (size_t)m * N + n + r, v[r]);
                    }
                }
            }
        }
    }
}

bool w4a8_supported(const QArgs& a) {
    // groups must hold whole 128-k stages; activations/weights 16-byte aligned
    if (((uintptr_t)a.w & 15u) != 0 || ((uintptr_t)a.x & 15u) != 0) return false;
    if ((a.wbits != 4 && a.wbits != 8) || a.x_kind != XKind::I8) return false;
    if (a.k % GK != 0 || a.group_size % GK != 0) return false;
    // byte offsets of the buffer loads are 31-bit
    const size_t lim = (size_t)1 << 31;
    constexpr int BRMAX = 16 * RT * 12;  // rows of the largest block
    if ((size_t)(a.n_out + BRMAX) * a.k / 8 * a.wbits >= lim || (size_t)(a.m + BT) * a.k >= lim) return false;
    if ((size_t)(a.n_out + BRMAX) * (a.k / a.group_size) * 16 >= lim) return false;
    if (a.y_kind == YKind::I32) return true;  // raw sums or per-group partials: no scales used
    // scaled output: the block's scales are staged in LDS (at most GMAX groups per row)
    const int G = a.k / a.group_size;
    const int sb = a.scale_kind == ScaleKind::F16 ? 2 : a.scale_kind == ScaleKind::GroupScale ? 16 : 4;
    return a.scale_kind != ScaleKind::None && a.xs != nullptr && G <= GMAX && BRMAX * G * sb <= 256 * 16 * SCH;
}

template <int WB, int MODE, bool ONEG, ScaleKind SK, YKind YK, int NWB = 4, bool DEF = false>
static void launch_g(const QArgs& a, hipStream_t s) {
    constexpr int BRB = 16 * RT * NWB;
    const int nrb = (a.n_out + BRB - 1) / BRB, ntb = (a.m + BT - 1) / BT;
    const int nrb8 = (nrb + NXCD - 1) / NXCD * NXCD;  // row blocks padded to whole XCD rounds
    const dim3 grid(nrb8 * ntb), block(64 * NWB);
    // two's complement nibbles become offset-binary with a xor of 8 per nibble
    const uint32_t tc = a.xor_mask ? 0x08080808u : 0u;
    const size_t smem = MODE == 2 ? (size_t)BRB * (a.k / a.group_size) * sizeof(float) : 0;
    if (smem > 48 * 1024) {
        static bool raised = false;  // once per instantiation
        if (!raised) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_w4a8<WB, MODE, ONEG, SK, YK, NWB, DEF>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, BRB * GMAX * (int)sizeof(float));
            raised = true;
        }
    }
    hipLaunchKernelGGL((k_w4a8<WB, MODE, ONEG, SK, YK, NWB, DEF>), grid, block, smem, s, reinterpret_cast<const uint8_t*>(a.w),
                       a.s, reinterpret_cast<const int8_t*>(a.x), a.xs, a.y, a.m, a.n_out, a.k,
                       a.group_size, tc, nrb, ntb,
                       (a.n_out % 4 == 0 && ((uintptr_t)a.y & 15u) == 0) ? 1 : 0);
}

// Block shape of the scaled g128 kernel with fp16 scales.  4 waves (64 rows) let up
// to three blocks share a CU; 11 waves (176 rows, one block per CU, the group scaling
// deferred by a stage) read the activations a third as often and the weights as often.
// The wide block is taken when it needs no more wave rounds per SIMD: blocks of 11 waves
// put up to 3 waves on a SIMD per block, blocks of 4 waves one.  Config 5 (11008 rows, 256
// tokens): 688 blocks (3 per CU) or 252 blocks (1 per CU): 24.5 against 26.0 us with int4
// weights, 27.9 against 32.8 us with int8 weights.
static bool w4a8_wide(const QArgs& a) {
    const int cus = device_cus(), ntb = (a.m + BT - 1) / BT;
    const long b4 = (long)(a.n_out + 63) / 64 * ntb, b11 = (long)(a.n_out + 175) / 176 * ntb;
    const long per_simd4 = (b4 + cus - 1) / cus, per_simd11 = 3 * ((b11 + cus - 1) / cus);
    return per_simd11 <= per_simd4;
}

template <int WB, int MODE, ScaleKind SK, YKind YK>
static void launch_t(const QArgs& a, hipStream_t s) {
    if (MODE != 0 && a.group_size == GK) {
        if constexpr (MODE == 2 && SK == ScaleKind::F16) {
            if (w4a8_wide(a)) return launch_g<WB, MODE, true, SK, YK, 11, true>(a, s);
        }
        return launch_g<WB, MODE, true, SK, YK>(a, s);
    }
    return launch_g<WB, MODE, false, SK, YK>(a, s);
}

template <int WB, ScaleKind SK>
static bool launch_scaled(const QArgs& a, hipStream_t s) {
    switch (a.y_kind) {
        case YKind::F32: launch_t<WB, 2, SK, YKind::F32>(a, s); return true;
        case YKind::F16: launch_t<WB, 2, SK, YKind::F16>(a, s); return true;
        case YKind::BF16: launch_t<WB, 2, SK, YKind::BF16>(a, s); return true;
        default: return false;
    }
}

template <int WB>
static bool launch_wb(const QArgs& a, hipStream_t s) {
    if (a.y_kind == YKind::I32) {
        if (a.group_partials) launch_t<WB, 1, ScaleKind::None, YKind::I32>(a, s);
        else launch_t<WB, 0, ScaleKind::None, YKind::I32>(a, s);
        return true;
    }
    switch (a.scale_kind) {
        case ScaleKind::F16: return launch_scaled<WB, ScaleKind::F16>(a, s);
        case ScaleKind::F32: return launch_scaled<WB, ScaleKind::F32>(a, s);
        case ScaleKind::GroupScale: return launch_scaled<WB, ScaleKind::GroupScale>(a, s);
        default: return false;
    }
}

hipError_t launch_w4a8(const QArgs& a, hipStream_t s) {
    const bool ok = a.wbits == 8 ? launch_wb<8>(a, s) : launch_wb<4>(a, s);
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace luxhip
