// int4 grouped weight-only GEMM for large m (prefill): Y[m, n] = sum_k X[m, k] * Wd[n, k]
// with Wd[n, k] = q(n, k) * s(n, k / gs).
//
// Reference: matmul_nax_grouped (quantized_nax.wgsl:568-626).  Config 4 of
// X 2048 x 4096 bf16, W 14336 x 4096 int4 g32 with fp16 scales,
// bf16 output -- a dense contraction (2,216 flop per HBM byte), so the roofline
// is the fp16/bf16 MFMA peak.
//
// Numerics: X (bf16) is staged as fp16 after dividing each row by a power of two
// that puts its largest |x| in [2^14, 2^15); bf16 carries 8 significant bits and fp16
// 11, so the staging is exact for every element within 2^-28 of the row maximum and
// cannot overflow.  The epilogue multiplies the row back (exact).  The dequantised weight
// q*s/fold is staged as fp16 rounded to nearest-even, fold being the weight row's
// power-of-two scale fold (scale_fold_factor, computed by the pre-pass), which the
// epilogue multiplies back: any finite fp16 / fp32 / GroupScale scale stays in fp16's
// normal range.  The exact product needs up to 14 significant bits (more for fp32
// scales), so each staged weight carries one rounding, a relative error <= 2^-11.
// Products are exact in the MFMA and accumulate in fp32.  Against the
// fp32 oracle rounded to bf16 this measures rel-L2 ~8e-4 on config 4, inside
// the stated 1e-3 (the bf16 output rounding alone is worth 1.7e-3 against the
// unrounded oracle).
//
// Tiling (gfx950): 512 threads = 8 waves in a 2 (m) x 4 (n) grid, two per SIMD so
// one wave's MFMAs cover the other's loads and dequant; block tile 256 (m) x 256
// (n); each wave owns 128 x 64 = 4 x 2 tiles of v_mfma_f32_32x32x16_f16 (128 fp32
// accumulators per lane, in AGPRs).  K advances 64 per stage through
// double-buffered LDS (2 x 72 KB): while the MFMAs of stage s run, the global loads
// of stage s+1 are in flight; W is dequantised and both tiles are written to the
// other buffer before one barrier per stage.  X is restaged to fp16 once per call
// by a pre-pass.  For k <= 8192 the default is k_qgemm_i4_xr (below): 512 x 128 block
// tiles with X read from a fragment-ordered staging straight into registers and only the
// weights in LDS; LUX_HIP_C4_STAGED=1 selects the kernel described here.
#include <algorithm>
#include <cstdlib>

#include "common.hpp"

namespace luxhip {

namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int LDS_ROW = BK + 8;  // halves per LDS row: 144 B stride keeps b128 reads conflict-free
constexpr int NT = 512;  // 8 waves: 2 (m) x 4 (n), two per SIMD

__device__ __forceinline__ uint32_t pack_h2(f16 a, f16 b) {
    return __builtin_bit_cast(uint32_t, f16x2{a, b});
}

// (a & m) | o in one VOP3; the mask comes from an SGPR, the magic from a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

// One u32 of 8 offset-binary nibbles (k .. k+7) times scale s -> 8 fp16 (RNE) in the
// staging order (k, k+4, k+1, k+5, k+2, k+6, k+3, k+7).  (1024 + n) - 1032 is exact in
// fp16; v_pk_mul_f16 rounds the exact product q*s to nearest-even.  15 VALU ops.
__device__ __forceinline__ u32x4 dequant8(uint32_t w, f16x2 s2, uint32_t magic) {
    const f16x2 OFF = {(f16)1032.0f, (f16)1032.0f};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = and_or(w >> (4 * i), 0x000F000Fu, magic);  // (n_i, n_{i+4})
        o[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, t) - OFF) * s2);
    }
    return u32x4{o[0], o[1], o[2], o[3]};
}

}  // namespace

// X -> fp16 in staging order.  Runs once per call ahead of the GEMM, so each
// activation is converted once instead of once per n tile (56 times on config 4).
// Pre-pass, one wave per activation row: X -> fp16 in the staging order (groups of 8
// along k reordered (k, k+4, k+1, k+5, ...), the order in which dequant8 emits
// weights, so both MFMA operands agree element by element).  bf16 rows are first
// divided by their power-of-two factor fac[m] (row_pow2_factor), which the GEMM
// epilogue multiplies back; fp16 rows are copied as they are (fac = 1).  The first
// XR * 64 chunks of 8 stay in registers between the max and the conversion.
constexpr int XR = 8;

__device__ __forceinline__ uint32_t bf16x2_absmax(uint32_t w) {
    return max(w & 0x7FFFu, (w >> 16) & 0x7FFFu);
}

__device__ __forceinline__ u32x4 bf16x8_to_staged_f16(u32x4 v, float inv) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    f16 h[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        h[2 * q] = (f16)(__builtin_bit_cast(float, w[q] << 16) * inv);
        h[2 * q + 1] = (f16)(__builtin_bit_cast(float, w[q] & 0xFFFF0000u) * inv);
    }
    return u32x4{pack_h2(h[0], h[4]), pack_h2(h[1], h[5]), pack_h2(h[2], h[6]), pack_h2(h[3], h[7])};
}

// Blocks past the first ceil(M / 4) compute the weight rows' scale folds instead (one
// wave per weight row, row_scale_fold), so one launch prepares both operands.
template <XKind XK, ScaleKind SK>
__global__ __launch_bounds__(256) void k_x_to_f16_rows(const void* __restrict__ X,
                                                       u32x4* __restrict__ out,
                                                       float* __restrict__ fac, int M, int K,
                                                       const void* __restrict__ S, float* __restrict__ wfold,
                                                       int N, int G) {
    const int lane = threadIdx.x & 63;
    const int xblocks = (M + 3) / 4;
    if ((int)blockIdx.x >= xblocks) {
        const int wrow = ((int)blockIdx.x - xblocks) * 4 + (threadIdx.x >> 6);
        if (wrow >= N) return;
        const float f = row_scale_fold<SK>(S, (size_t)wrow, G, lane);
        if (lane == 0) wfold[wrow] = f;
        return;
    }
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int n8 = K / 8;
    const u32x4* xr = reinterpret_cast<const u32x4*>(X) + (size_t)row * n8;
    u32x4* orow = out + (size_t)row * n8;
    if constexpr (XK == XKind::F16) {
        for (int c = lane; c < n8; c += 64) {
            const f16x8 fv = __builtin_bit_cast(f16x8, xr[c]);
            orow[c] = u32x4{pack_h2(fv[0], fv[4]), pack_h2(fv[1], fv[5]), pack_h2(fv[2], fv[6]),
                            pack_h2(fv[3], fv[7])};
        }
        if (lane == 0) fac[row] = 1.0f;
    } else {
        u32x4 v[XR];
        uint32_t mx = 0;
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            const int c = lane + 64 * i;
            v[i] = c < n8 ? xr[c] : u32x4{0u, 0u, 0u, 0u};
            mx = max(mx, max(max(bf16x2_absmax(v[i].x), bf16x2_absmax(v[i].y)),
                             max(bf16x2_absmax(v[i].z), bf16x2_absmax(v[i].w))));
        }
        for (int c = lane + 64 * XR; c < n8; c += 64) {
            const u32x4 u = xr[c];
            mx = max(mx, max(max(bf16x2_absmax(u.x), bf16x2_absmax(u.y)), max(bf16x2_absmax(u.z), bf16x2_absmax(u.w))));
        }
        mx = wave_max_u32(mx);
        const float f = row_pow2_factor(mx, 7);
        const float inv = 1.0f / f;  // exact: f is a power of two
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            const int c = lane + 64 * i;
            if (c < n8) orow[c] = bf16x8_to_staged_f16(v[i], inv);
        }
        for (int c = lane + 64 * XR; c < n8; c += 64) orow[c] = bf16x8_to_staged_f16(xr[c], inv);
        if (lane == 0) fac[row] = f;
    }
}

// Pre-pass of the X-from-registers GEMM: the same conversion as k_x_to_f16_rows, written
// in MFMA fragment order.  Chunk (mt, ks) of 1 KB holds at 16-byte slot l the 8 staged
// halves of row 32 mt + l % 32, k = 16 ks + 8 (l / 32) .. + 7, so a wave loads one
// fragment as one contiguous 1 KB.  A block of 8 waves converts 8 consecutive rows into
// LDS (rows past M as zeros), then writes each (ks, l / 32) group of its 8 rows as one
// contiguous 128 bytes.  Blocks past 4 ceil(M / 32) compute the weight rows' scale folds,
// 64 rows per block (the launch's LDS size applies to every block, so few of them).
template <XKind XK, ScaleKind SK>
__global__ __launch_bounds__(512) void k_x_to_f16_frag(const void* __restrict__ X, u32x4* __restrict__ out,
                                                       float* __restrict__ fac, int M, int K,
                                                       const void* __restrict__ S, float* __restrict__ wfold,
                                                       int N, int G) {
    extern __shared__ u32x4 xl[];  // [8][K / 8 + 1]: one 16-byte pad per row (conflict-free column reads)
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int xblocks = (M + 31) / 32 * 4;
    if ((int)blockIdx.x >= xblocks) {
        const int w0 = ((int)blockIdx.x - xblocks) * 64 + wv * 8;
        if (w0 >= N) return;
        const int nr = min(8, N - w0);
        if (G <= 128) {
            // all 8 rows' loads first (indices clamped: repeats do not change a max)
            uint32_t mx[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const size_t row = (size_t)(w0 + min(r, nr - 1)) * G;
                mx[r] = max(scale_abs_bits<SK>(load_scale_raw<SK>(S, row + min(lane, G - 1))),
                            scale_abs_bits<SK>(load_scale_raw<SK>(S, row + min(lane + 64, G - 1))));
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                mx[r] = wave_max_u32(mx[r]);
                if (lane == 0 && r < nr) wfold[w0 + r] = scale_fold_factor(mx[r]);
            }
        } else {
            for (int r = 0; r < nr; ++r) {
                const float f = row_scale_fold<SK>(S, (size_t)(w0 + r), G, lane);
                if (lane == 0) wfold[w0 + r] = f;
            }
        }
        return;
    }
    const int n8 = K / 8, ld = n8 + 1;
    const int row = blockIdx.x * 8 + wv;
    u32x4* lrow = xl + wv * ld;
    if (row >= M) {
        for (int c = lane; c < n8; c += 64) lrow[c] = u32x4{0u, 0u, 0u, 0u};
    } else {
        const u32x4* xr = reinterpret_cast<const u32x4*>(X) + (size_t)row * n8;
        if constexpr (XK == XKind::F16) {
            for (int c = lane; c < n8; c += 64) {
                const f16x8 fv = __builtin_bit_cast(f16x8, xr[c]);
                lrow[c] = u32x4{pack_h2(fv[0], fv[4]), pack_h2(fv[1], fv[5]), pack_h2(fv[2], fv[6]),
                                pack_h2(fv[3], fv[7])};
            }
            if (lane == 0) fac[row] = 1.0f;
        } else {
            u32x4 v[XR];
            uint32_t mx = 0;
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                const int c = lane + 64 * i;
                v[i] = c < n8 ? xr[c] : u32x4{0u, 0u, 0u, 0u};
                mx = max(mx, max(max(bf16x2_absmax(v[i].x), bf16x2_absmax(v[i].y)),
                                 max(bf16x2_absmax(v[i].z), bf16x2_absmax(v[i].w))));
            }
            for (int c = lane + 64 * XR; c < n8; c += 64) {
                const u32x4 u = xr[c];
                mx = max(mx, max(max(bf16x2_absmax(u.x), bf16x2_absmax(u.y)),
                                 max(bf16x2_absmax(u.z), bf16x2_absmax(u.w))));
            }
            mx = wave_max_u32(mx);
            const float f = row_pow2_factor(mx, 7);
            const float inv = 1.0f / f;  // exact: f is a power of two
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                const int c = lane + 64 * i;
                if (c < n8) lrow[c] = bf16x8_to_staged_f16(v[i], inv);
            }
            for (int c = lane + 64 * XR; c < n8; c += 64) lrow[c] = bf16x8_to_staged_f16(xr[c], inv);
            if (lane == 0) fac[row] = f;
        }
    }
    __syncthreads();
    // thread t: row r8 = t % 8 of the block, chunk c8 = t / 8 + 64 i (ks = c8 / 2, half c8 % 2)
    const int r8 = threadIdx.x & 7;
    const int mt = (blockIdx.x * 8) >> 5, rbase = (blockIdx.x * 8) & 31;
    const size_t base = (size_t)mt * (n8 / 2) * 64 + rbase + r8;
    for (int c8 = threadIdx.x >> 3; c8 < n8; c8 += 64)
        out[base + (size_t)(c8 >> 1) * 64 + 32 * (c8 & 1)] = xl[r8 * ld + c8];
}

// GEMM over the staged X (fp16, staging order) and int4 W.
template <ScaleKind SK, YKind YK>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_qgemm_i4_large(const f16* __restrict__ X, const float* __restrict__ xfac,
                      const uint32_t* __restrict__ W, const void* __restrict__ S,
                      const float* __restrict__ wfold, void* __restrict__ Y,
                      int M, int N, int K, int gs, uint32_t xor_mask, int vec_y, EpiArgs epi) {
    extern __shared__ __attribute__((aligned(16))) f16 lds[];
    f16* xs = lds;                          // [2][BM][LDS_ROW]
    f16* ws = lds + 2 * BM * LDS_ROW;       // [2][BN][LDS_ROW]

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv >> 2, wn = wv & 3;    // wave tile: 128 (m) x 64 (n)
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int G = K / gs;

    // Raw buffer loads: one SGPR resource per operand, 32-bit VGPR offsets fixed across
    // stages, the K position in the scalar offset.  Rows past M / N get an offset past
    // the resource size, which the hardware reads as zeros.
    const uint32_t xbytes = (uint32_t)((size_t)M * K * 2), wbytes = (uint32_t)((size_t)N * K / 2);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(X), (short)0, (int)xbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(W), (short)0, (int)wbytes, 0x00020000);
    // X: 256 rows x 64 k = 2048 chunks of 8; thread t takes chunks t + 512 i (i < 4):
    // row = (t >> 3) + 64 i, k-chunk = t & 7 (each row read as 128 contiguous bytes).
    // W: 2 threads per row of the n tile; thread t takes row t / 2, k half t % 2
    // (32 nibbles = 16 B, one scale group of 32).
    const int xrow = tid >> 3, xk = (tid & 7) * 8;
    uint32_t xoff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + xrow + 64 * i;
        xoff[i] = m < M ? (uint32_t)(((size_t)m * K + xk) * 2) : xbytes;
    }
    // Weight row of LDS row rho.  SiluMul: wave wn's 64 rows are 32 gate rows g0 + 32 wn ..
    // (its j = 0 block) and the matching up rows nh + g0 + 32 wn .. (j = 1), g0 = 128 *
    // blockIdx.x, so a gate accumulator and its up accumulator share a lane and register.
    const bool sm = epi.kind == (int)Epi::SiluMul;
    const int nh = N / 2, g0 = blockIdx.x * (BN / 2);
    auto grow = [&](int rho) {  // -1: past the end
        if (!sm) return n0 + rho < N ? n0 + rho : -1;
        const int w = rho >> 6, o = rho & 63, g = g0 + 32 * w + (o & 31);
        return g < nh ? (o < 32 ? g : nh + g) : -1;
    };
    const int wr_row = tid >> 1, wh = tid & 1;
    const int wgr = grow(wr_row);
    const uint32_t woff = wgr >= 0 ? (uint32_t)((size_t)wgr * (K / 2) + 16 * wh) : wbytes;
    const int srow = wgr >= 0 ? wgr : N - 1;
    const float winv = 1.0f / wfold[srow];  // exact: the fold is a power of two
    const uint32_t magic = 0x64006400u;

    // Staging registers, two sets: the data of stage t is loaded during stage t-2 and
    // written to LDS early in stage t-1, interleaved with that stage's MFMAs.
    struct Regs {
        u32x4 xr[4], wr;
        uint32_t sr;
    };
    auto load_stage = [&](Regs& R, int k0) {
        k0 = __builtin_amdgcn_readfirstlane(min(k0, K - BK));  // uniform; clamped in range
#pragma unroll
        for (int i = 0; i < 4; ++i)
            R.xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xoff[i], k0 * 2, 0));
        R.wr = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)woff, k0 / 2, 0));
        R.sr = load_scale_raw<SK>(S, (size_t)srow * G + (k0 + 32 * wh) / gs);
    };
    auto store_stage = [&](const Regs& R, int buf) {
        f16* xb = xs + buf * BM * LDS_ROW;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x4*>(xb + (xrow + 64 * i) * LDS_ROW + xk) = R.xr[i];
        f16* wb = ws + buf * BN * LDS_ROW + wr_row * LDS_ROW + 32 * wh;
        const uint32_t words[4] = {R.wr.x, R.wr.y, R.wr.z, R.wr.w};
        if constexpr (SK == ScaleKind::F16) {
            // an fp16 scale times a power of two is exact in fp16: q * s rounds once
            const f16 sc = (f16)(scale_from_raw<SK>(R.sr) * winv);
            const f16x2 s2 = {sc, sc};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<u32x4*>(wb + 8 * q) = dequant8(words[q] ^ xor_mask, s2, magic);
        } else {
            const float sc = scale_from_raw<SK>(R.sr) * winv;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<u32x4*>(wb + 8 * q) = dequant8_f32s(words[q] ^ xor_mask, sc);
        }
    };

    // acc[j][i]: weight rows (n) are the MFMA's A operand and activation rows (m) its B
    // operand, so each lane ends up holding four consecutive n of one output row m.
    f32x16 acc[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] = f32x16{};

    // MFMA operand addressing (v_mfma_f32_32x32x16_f16): A row (weights) = lane % 32,
    // B column (activations) = lane % 32, both taking k = 8 * (lane / 32) + 0..7 of the
    // 16-k step.
    const int arow = wm * 128 + (lane & 31), brow = wn * 64 + (lane & 31);
    const int kofs = (lane >> 5) * 8;

    // 4 k-steps of 8 MFMAs from LDS buffer `buf`; operands double-buffered across
    // the k-steps (reads for step kk+1 go out ahead of the MFMAs of step kk).
    // One stage: 4 k-steps of 8 MFMAs from LDS buffer `buf`.  Operands are
    // double-buffered across the k-steps.  After the first k-step the next stage's
    // registers are dequantised into the other buffer, so that VALU work issues
    // while this wave's (and the sibling wave's) MFMAs occupy the matrix pipe.
    auto compute = [&](int buf, const Regs& nxt) {
        const f16* xb = xs + buf * BM * LDS_ROW;
        const f16* wb = ws + buf * BN * LDS_ROW;
        f16x8 a[2][4], b[2][2];
        auto read_ops = [&](int kk, f16x8 (&av)[4], f16x8 (&bv)[2]) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                av[i] = *reinterpret_cast<const f16x8*>(xb + (arow + 32 * i) * LDS_ROW + 16 * kk + kofs);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bv[j] = *reinterpret_cast<const f16x8*>(wb + (brow + 32 * j) * LDS_ROW + 16 * kk + kofs);
        };
        read_ops(0, a[0], b[0]);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            if (kk + 1 < 4) read_ops(kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[kk & 1][j], a[kk & 1][i], acc[j][i], 0, 0, 0);
            if (kk == 0) store_stage(nxt, buf ^ 1);
        }
    };

    // Stages past the end load a clamped (valid) stage into a buffer nobody reads.
    const int nstages = K / BK;
    Regs R0, R1;
    load_stage(R0, 0);
    load_stage(R1, BK);
    store_stage(R0, 0);
    __syncthreads();
    // Two stages per iteration (static register sets); an odd stage count ends with
    // one more stage from buffer 0.
    const int npairs = nstages >> 1;
    for (int p = 0; p < npairs; ++p) {
        const int s = 2 * p;
        load_stage(R0, (s + 2) * BK);
        compute(0, R1);            // stores stage s+1 into buffer 1
        __syncthreads();
        load_stage(R1, (s + 3) * BK);
        compute(1, R0);            // stores stage s+2 into buffer 0
        __syncthreads();
    }
    if (nstages & 1) compute(0, R1);

    // The block's 256 row factors of X and the scale folds of its 256 weight rows (fp32,
    // by LDS row of the weight tile) go to the now idle LDS, once.
    __syncthreads();
    float* fac = reinterpret_cast<float*>(lds);
    float* wf = fac + BM;
    if (tid < BM) fac[tid] = m0 + tid < M ? xfac[m0 + tid] : 0.0f;
    else if (tid < BM + BN) {
        const int g = grow(tid - BM);
        wf[tid - BM] = g >= 0 ? wfold[g] : 1.0f;
    }
    __syncthreads();

    // Epilogue: D[r][c] of a 32x32 tile (r = weight row, c = activation row) sits in
    // lane c + 32 * ((r / 4) & 1), register 4 * (r / 8) + r % 4: registers 4g .. 4g+3
    // of a lane are the four consecutive n = 8 g + 4 (lane / 32) + 0..3 of row m.
    const bool vec = vec_y != 0;  // N % 4 == 0 and Y aligned
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ml = wm * 128 + 32 * i + (lane & 31);
        const int m = m0 + ml;
        if (m >= M) continue;
        const float fm = fac[ml];
        if (sm) {  // silu(gate) * up: gate block j = 0, up block j = 1, output [M x nh]
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = g0 + wn * 32 + 8 * g + 4 * (lane >> 5);
                f32x4 v;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rho = wn * 64 + 8 * g + 4 * (lane >> 5) + r;  // gate row; its up row is rho + 32
                    v[r] = silu_f(acc[0][i][4 * g + r] * fm * wf[rho]) * (acc[1][i][4 * g + r] * fm * wf[rho + 32]);
                }
                if (vec && n + 3 < nh) {
                    store_y4<YK>(Y, (size_t)m * nh + n, v);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < nh) store_y<YK>(Y, (size_t)m * nh + n + r, v[r]);
                }
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + wn * 64 + 32 * j + 8 * g + 4 * (lane >> 5);
                const int rho = wn * 64 + 32 * j + 8 * g + 4 * (lane >> 5);
                f32x4 v = f32x4{acc[j][i][4 * g] * wf[rho], acc[j][i][4 * g + 1] * wf[rho + 1],
                                acc[j][i][4 * g + 2] * wf[rho + 2], acc[j][i][4 * g + 3] * wf[rho + 3]} * fm;
                if (epi.kind != 0) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = apply_epi(v[r], epi, m, min(n + r, N - 1), N);
                }
                if (vec && n + 3 < N) {
                    store_y4<YK>(Y, (size_t)m * N + n, v);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < N) store_y<YK>(Y, (size_t)m * N + n + r, v[r]);
                }
            }
    }
}

// The same GEMM with the activation operand read straight from X staged in fragment
// order (k_x_to_f16_frag) into MFMA registers, one contiguous 1 KB per fragment, so only
// the dequantised weights pass through LDS.  8 waves in a WGM (m) x 8 / WGM (n) grid, each
// with TM x TN tiles of 32 x 32.  The launcher uses WGM = 8, TM = 2, TN = 4: a 512 x 128
// block tile (each weight tile dequantised once per 512 rows of X) whose waves are
// stacked in m, 64 x 128 each, so every wave loads X fragments no other wave of the
// block needs and all eight read the weight tile from LDS.  With the waves in a 4 x 2
// grid (TM = 4, TN = 2) the two n-waves load the same X fragments, which doubles the
// vector-memory requests for X.  The MFMA sequence per output element is the staged
// kernel's, so the results are identical.
template <ScaleKind SK, YKind YK, int TM, int TN, int WGM = 4>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_qgemm_i4_xr(const f16* __restrict__ X, const float* __restrict__ xfac,
                   const uint32_t* __restrict__ W, const void* __restrict__ S,
                   const float* __restrict__ wfold, void* __restrict__ Y,
                   int M, int N, int K, int gs, uint32_t xor_mask, int vec_y, EpiArgs epi) {
    constexpr int WGN = 8 / WGM;                    // waves in m and n
    constexpr int TBM = 32 * TM * WGM, TBN = 32 * TN * WGN;  // block tile
    constexpr int NKK = BK / 16;                    // k-steps per 64-k stage
    constexpr int TPR = NT / TBN, KPT = BK / TPR;   // threads per weight row, k per thread
    constexpr int WPT = KPT / 8;                    // packed words (8 weights) per thread
    constexpr int HALF = 16 * TN;                   // SiluMul: gate rows per wave
    extern __shared__ __attribute__((aligned(16))) f16 lds[];
    f16* ws = lds;  // [2][TBN][LDS_ROW]

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv / WGN, wn = wv % WGN;  // wave tile: 32 TM (m) x 32 TN (n)
    const int m0 = blockIdx.y * TBM, n0 = blockIdx.x * TBN;
    const int G = K / gs;

    const uint32_t xbytes = (uint32_t)((size_t)(M + 31) / 32 * 32 * K * 2), wbytes = (uint32_t)((size_t)N * K / 2);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(X), (short)0, (int)xbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(W), (short)0, (int)wbytes, 0x00020000);
    // X in fragment order (k_x_to_f16_frag): the fragment of m-tile mt and k-step ks is the
    // 1 KB at (mt * K / 16 + ks) * 1024, lane l at + 16 l.  m-tiles past the staged rows
    // (ceil(M / 32) of them) read zeros.
    const int kofs = (lane >> 5) * 8;
    const int mtiles = (M + 31) / 32;
    uint32_t xoff[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int mt = (m0 >> 5) + TM * wm + i;
        xoff[i] = mt < mtiles ? (uint32_t)((size_t)mt * (K / 16) * 1024 + 16 * lane) : xbytes;
    }
    // Weight row of LDS row rho.  SiluMul: wave wn's 32 TN rows are HALF gate rows
    // g0 + HALF wn .. (tiles j < TN / 2) and the matching up rows (tiles j + TN / 2),
    // g0 = blockIdx.x * TBN / 2.
    const bool sm = epi.kind == (int)Epi::SiluMul;
    const int nh = N / 2, g0 = blockIdx.x * (TBN / 2);
    auto grow = [&](int rho) {  // -1: past the end
        if (!sm) return n0 + rho < N ? n0 + rho : -1;
        const int w = rho / (2 * HALF), o = rho % (2 * HALF), g = g0 + HALF * w + o % HALF;
        return g < nh ? (o < HALF ? g : nh + g) : -1;
    };
    // W: TPR threads per row of the n tile; thread t takes row t / TPR and KPT k (WPT words
    // of nibbles, inside one g32 group) from k = KPT * (t % TPR).
    const int wr_row = tid / TPR, wh = tid % TPR;
    const int wgr = grow(wr_row);
    const uint32_t woff = wgr >= 0 ? (uint32_t)((size_t)wgr * (K / 2) + KPT / 2 * wh) : wbytes;
    const int srow = wgr >= 0 ? wgr : N - 1;
    const float winv = 1.0f / wfold[srow];  // exact: the fold is a power of two
    const uint32_t magic = 0x64006400u;

    struct Regs {
        uint32_t w[WPT];
        uint32_t sr;
    };
    static_assert(WPT == 1 || WPT == 2 || WPT == 4, "8, 16 or 32 k per thread");
    auto load_w = [&](Regs& R, int k0) {
        k0 = __builtin_amdgcn_readfirstlane(min(k0, K - BK));
        if constexpr (WPT == 4) {
            const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)woff, k0 / 2, 0));
            R.w[0] = v.x, R.w[1] = v.y, R.w[2] = v.z, R.w[3] = v.w;
        } else if constexpr (WPT == 1) {
            R.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)woff, k0 / 2, 0);
        } else {
            const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, (int)woff, k0 / 2, 0));
            R.w[0] = v.x, R.w[1] = v.y;
        }
        R.sr = load_scale_raw<SK>(S, (size_t)srow * G + (k0 + KPT * wh) / gs);
    };
    // Word q (8 weights) of the next stage, one per k-step (WPT = 4) or every other k-step
    // (WPT = 2), so the dequantisation is spread over the stage's MFMAs instead of arriving
    // in one burst (the two waves of a SIMD reach each k-step together).
    auto store_w = [&](const Regs& R, int buf, int q) {
        f16* wb = ws + buf * TBN * LDS_ROW + wr_row * LDS_ROW + KPT * wh + 8 * q;
        const uint32_t word = R.w[q] ^ xor_mask;
        if constexpr (SK == ScaleKind::F16) {
            const f16 sc = (f16)(scale_from_raw<SK>(R.sr) * winv);
            *reinterpret_cast<u32x4*>(wb) = dequant8(word, f16x2{sc, sc}, magic);
        } else {
            const float sc = scale_from_raw<SK>(R.sr) * winv;
            *reinterpret_cast<u32x4*>(wb) = dequant8_f32s(word, sc);
        }
    };
    // X fragments, one register set per k-step of a stage: right after the MFMAs of k-step
    // kk of stage s have read set kk, it is reloaded with k-step kk of stage s+1.  The load
    // counter retires in issue order and the weights of stage s+2 are issued at the start
    // of stage s, so X loaded only a few k-steps ahead would make each k-step wait for HBM;
    // a stage ahead, both loads get a stage of latency.
    const int nks = K / 16;
    f16x8 xf[NKK][TM];
    auto load_x = [&](int kk, int gk) {
        const int so = __builtin_amdgcn_readfirstlane(min(gk, nks - 1) * 1024);
#pragma unroll
        for (int i = 0; i < TM; ++i)
            xf[kk][i] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xoff[i], so, 0));
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = f32x16{};

    const int brow = wn * 32 * TN + (lane & 31);
    auto compute = [&](int buf, const Regs& nxt, int s) {
        const f16* wb = ws + buf * TBN * LDS_ROW;
        f16x8 b[2][TN];
        auto read_w = [&](int kk, f16x8 (&bv)[TN]) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bv[j] = *reinterpret_cast<const f16x8*>(wb + (brow + 32 * j) * LDS_ROW + 16 * kk + kofs);
        };
        read_w(0, b[0]);
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
            if (kk + 1 < NKK) read_w(kk + 1, b[(kk + 1) & 1]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[kk & 1][j], xf[kk][i], acc[j][i], 0, 0, 0);
            load_x(kk, NKK * (s + 1) + kk);
            if (WPT == 4) store_w(nxt, buf ^ 1, kk);
            else if (WPT == 2 && (kk & 1) == 0) store_w(nxt, buf ^ 1, kk >> 1);
            else if (WPT == 1 && kk == 0) store_w(nxt, buf ^ 1, 0);
            // Issue order of the k-step: the next k-step's weight fragments, then each MFMA
            // followed by two VALU ops of the dequantisation, then the X loads and the LDS
            // store.  The barrier closes the k-step, so no load sinks to the stage's end.
            __builtin_amdgcn_sched_group_barrier(0x100, TN, 0);  // DS reads
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
            }
            __builtin_amdgcn_sched_group_barrier(0x020, TM, 0);  // VMEM reads
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // DS write
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    const int nstages = K / BK;
    Regs R0, R1;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) load_x(kk, kk);
    load_w(R0, 0);
    load_w(R1, BK);
#pragma unroll
    for (int q = 0; q < WPT; ++q) store_w(R0, 0, q);
    __syncthreads();
    const int npairs = nstages >> 1;
    for (int p = 0; p < npairs; ++p) {
        const int s = 2 * p;
        load_w(R0, (s + 2) * BK);
        __builtin_amdgcn_sched_barrier(0);
        compute(0, R1, s);  // stores stage s+1 into buffer 1
        __syncthreads();
        load_w(R1, (s + 3) * BK);
        __builtin_amdgcn_sched_barrier(0);
        compute(1, R0, s + 1);  // stores stage s+2 into buffer 0
        __syncthreads();
    }
    if (nstages & 1) compute(0, R1, nstages - 1);

    __syncthreads();
    float* fac = reinterpret_cast<float*>(lds);
    float* wf = fac + TBM;
    for (int t = tid; t < TBM + TBN; t += NT) {
        if (t < TBM) {
            fac[t] = m0 + t < M ? xfac[m0 + t] : 0.0f;
        } else {
            const int g = grow(t - TBM);
            wf[t - TBM] = g >= 0 ? wfold[g] : 1.0f;
        }
    }
    __syncthreads();

    // D[r][c] of a 32x32 tile (r = weight row, c = activation row) sits in lane
    // c + 32 * ((r / 4) & 1), register 4 * (r / 8) + r % 4.
    const bool vec = vec_y != 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int ml = wm * 32 * TM + 32 * i + (lane & 31);
        const int m = m0 + ml;
        if (m >= M) continue;
        const float fm = fac[ml];
        if (sm) {  // silu(gate) * up: gate tiles j < TN / 2, up tiles j + TN / 2, output [M x nh]
#pragma unroll
            for (int j = 0; j < TN / 2; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = g0 + wn * HALF + 32 * j + 8 * g + 4 * (lane >> 5);
                    f32x4 v;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int rho = wn * 32 * TN + 32 * j + 8 * g + 4 * (lane >> 5) + r;  // its up row: rho + HALF
                        v[r] = silu_f(acc[j][i][4 * g + r] * fm * wf[rho]) *
                               (acc[j + TN / 2][i][4 * g + r] * fm * wf[rho + HALF]);
                    }
                    if (vec && n + 3 < nh) {
                        store_y4<YK>(Y, (size_t)m * nh + n, v);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (n + r < nh) store_y<YK>(Y, (size_t)m * nh + n + r, v[r]);
                    }
                }
            continue;
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int rho = wn * 32 * TN + 32 * j + 8 * g + 4 * (lane >> 5);
                const int n = n0 + rho;
                f32x4 v = f32x4{acc[j][i][4 * g] * wf[rho], acc[j][i][4 * g + 1] * wf[rho + 1],
                                acc[j][i][4 * g + 2] * wf[rho + 2], acc[j][i][4 * g + 3] * wf[rho + 3]} * fm;
                if (epi.kind != 0) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = apply_epi(v[r], epi, m, min(n + r, N - 1), N);
                }
                if (vec && n + 3 < N) {
                    store_y4<YK>(Y, (size_t)m * N + n, v);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < N) store_y<YK>(Y, (size_t)m * N + n + r, v[r]);
                }
            }
    }
}

bool qgemm_i4_large_supported(const QArgs& a) {
    // Buffer resources carry 32-bit byte offsets: X (as fp16) and W stay below 2 GiB.
    return a.wbits == 4 && a.m >= 2 && (a.x_kind == XKind::BF16 || a.x_kind == XKind::F16) &&
           a.k % BK == 0 && a.group_size % 32 == 0 && a.scale_kind != ScaleKind::None &&
           a.y_kind != YKind::I32 && (size_t)(a.m + 31) / 32 * 32 * a.k * 2 < (1ull << 31) &&
           (size_t)a.n_out * a.k / 2 < (1ull << 31) && ((uintptr_t)a.x & 15u) == 0 &&
           ((uintptr_t)a.w & 15u) == 0;
}

// X through registers (k_x_to_f16_frag + k_qgemm_i4_xr) when the pre-pass's 8 rows fit in
// LDS; LUX_HIP_C4_STAGED=1 keeps both operands staged in LDS (k_qgemm_i4_large).
static bool use_xr(const QArgs& a) {
    static const bool staged = [] {
        const char* e = getenv("LUX_HIP_C4_STAGED");
        return e && e[0] == '1';
    }();
    return !staged && a.k <= 8192;
}

template <ScaleKind SK, YKind YK>
static void launch_t(const QArgs& a, const f16* xst, const float* xfac, const float* wfold, hipStream_t s) {
    const bool sm = a.epi.kind == (int)Epi::SiluMul;
    const int ny = sm ? a.n_out / 2 : a.n_out;  // output columns
    const dim3 grid(sm ? (ny + BN / 2 - 1) / (BN / 2) : (a.n_out + BN - 1) / BN, (a.m + BM - 1) / BM), block(NT);
    const bool xr = use_xr(a);
    static bool attr = [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_qgemm_i4_large<SK, YK>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);


        return true;
    }();
    (void)attr;
    const int vy = (ny % 4 == 0 && ((uintptr_t)a.y & 15u) == 0) ? 1 : 0;
    if (xr) {  // 512 x 128 block tiles
        const dim3 xgrid(sm ? (ny + 63) / 64 : (a.n_out + 127) / 128, (a.m + 511) / 512);
        const size_t lds = (size_t)2 * 128 * LDS_ROW * sizeof(f16);
        hipLaunchKernelGGL((k_qgemm_i4_xr<SK, YK, 2, 4, 8>), xgrid, block, lds, s, xst, xfac,
                           reinterpret_cast<const uint32_t*>(a.w), a.s, wfold, a.y, a.m, a.n_out, a.k,
                           a.group_size, a.xor_mask, vy, a.epi);
        return;
    }
    const size_t lds = (size_t)2 * (BM + BN) * LDS_ROW * sizeof(f16);
    hipLaunchKernelGGL((k_qgemm_i4_large<SK, YK>), grid, block, lds, s, xst, xfac,
                       reinterpret_cast<const uint32_t*>(a.w), a.s, wfold, a.y, a.m, a.n_out, a.k,
                       a.group_size, a.xor_mask, vy, a.epi);
}

template <ScaleKind SK>
static bool launch_y(const QArgs& a, u32x4* xst, float* xfac, float* wfold, hipStream_t s) {
    // pre-pass: X rows to fp16 and the weight rows' scale folds, one launch
    const int G = a.k / a.group_size;
    if (use_xr(a)) {
        static bool attr = [] {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_x_to_f16_frag<XKind::BF16, SK>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_x_to_f16_frag<XKind::F16, SK>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            return true;
        }();
        (void)attr;
        const dim3 fgrid((a.m + 31) / 32 * 4 + (a.n_out + 63) / 64), fblock(512);
        const size_t lds = (size_t)8 * (a.k / 8 + 1) * sizeof(u32x4);
        if (a.x_kind == XKind::BF16)
            hipLaunchKernelGGL((k_x_to_f16_frag<XKind::BF16, SK>), fgrid, fblock, lds, s, a.x, xst, xfac, a.m, a.k,
                               a.s, wfold, a.n_out, G);
        else
            hipLaunchKernelGGL((k_x_to_f16_frag<XKind::F16, SK>), fgrid, fblock, lds, s, a.x, xst, xfac, a.m, a.k,
                               a.s, wfold, a.n_out, G);
    } else {
        const dim3 pgrid((a.m + 3) / 4 + (a.n_out + 3) / 4), pblock(256);
        if (a.x_kind == XKind::BF16)
            hipLaunchKernelGGL((k_x_to_f16_rows<XKind::BF16, SK>), pgrid, pblock, 0, s, a.x, xst, xfac, a.m, a.k,
                               a.s, wfold, a.n_out, G);
        else
            hipLaunchKernelGGL((k_x_to_f16_rows<XKind::F16, SK>), pgrid, pblock, 0, s, a.x, xst, xfac, a.m, a.k,
                               a.s, wfold, a.n_out, G);
    }
    const f16* xh = reinterpret_cast<const f16*>(xst);
    switch (a.y_kind) {
        case YKind::F32: launch_t<SK, YKind::F32>(a, xh, xfac, wfold, s); return true;
        case YKind::F16: launch_t<SK, YKind::F16>(a, xh, xfac, wfold, s); return true;
        case YKind::BF16: launch_t<SK, YKind::BF16>(a, xh, xfac, wfold, s); return true;
        default: return false;
    }
}

// staged X (fp16; rows padded to a multiple of 32 for the fragment order), the per-row
// factors of X (fp32), the weight rows' scale folds (fp32); k % 64 keeps every part aligned
static size_t staged_x_bytes(const QArgs& a) { return (size_t)(a.m + 31) / 32 * 32 * a.k * sizeof(f16); }

size_t qgemm_i4_large_workspace(const QArgs& a) {
    return staged_x_bytes(a) + (size_t)a.m * sizeof(float) + (size_t)a.n_out * sizeof(float);
}

hipError_t launch_qgemm_i4_large(const QArgs& a, void* workspace, hipStream_t s) {
    u32x4* xst = reinterpret_cast<u32x4*>(workspace);
    float* xfac = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + staged_x_bytes(a));
    float* wfold = xfac + a.m;
    bool ok = false;
    switch (a.scale_kind) {
        case ScaleKind::F16: ok = launch_y<ScaleKind::F16>(a, xst, xfac, wfold, s); break;
        case ScaleKind::F32: ok = launch_y<ScaleKind::F32>(a, xst, xfac, wfold, s); break;
        case ScaleKind::GroupScale: ok = launch_y<ScaleKind::GroupScale>(a, xst, xfac, wfold, s); break;
        default: break;
    }
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace luxhip
