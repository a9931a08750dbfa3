// Producers and codecs of the quantized-matmul inputs.
//
// Reference (quantized_nax.wgsl, quantized.wgsl):
//   compute_group_scales   quantized_nax.wgsl:157-232  symmetric branch: s = max(|max|, |min|)
//                          / (7 | 127), s == 0 -> 1; GroupScale {s, 0, min, max}
//   quantize_nax_int4_sym  quantized_nax.wgsl:238-262  q = clamp(round(x / s), -8, 7), packed
//                          offset-binary 8 per u32 (:94-102)
//   quantize_nax_int8_group quantized_nax.wgsl:336-362 (NAX_INT8_SYM) q = clamp(round(x / s),
//                          -128, 127), 4 per u32 (:136-141)
//   requantize_int32_to_int8 quantized.wgsl:572-580  clamp(round(x * s_in / s_out) + zp)
//   dequantize_nax_int4_sym quantized_nax.wgsl:264-282 and dequantize_nax_int8_group
//                          :364-386 (symmetric branch): x = f32(q) * s, exact in fp32 for
//                          fp16 scales, then rounded (RNE) to the requested output type
// The reference runs the scale pass and the quantize pass as two dispatches over a
// flat tensor, with groups along the flat index; here one kernel does both for a
// [rows x k] tensor whose groups run along k (the same grouping when group_size
// divides k).  round() is round-half-to-even and x / s is the correctly rounded
// IEEE quotient (hipcc's default for fp32 division).
//
// HBM-bound: every input element is read once and every output written once.  A lane
// owns 8 consecutive elements (one int4 word, two int8 words); the lanes of one group
// (group_size / 8 of them, at most a wave) reduce max/min with xor shuffles.  Groups
// of up to 16384 elements (per-row scales) take one 256-thread block each, with the
// group in registers; longer ones one wave each, reading the group twice (the second
// pass hits L2).
#include "common.hpp"

namespace luxhip {

namespace {

template <XKind XK>
__device__ __forceinline__ void load8(const void* x, size_t chunk, float (&v)[8]) {
    if constexpr (XK == XKind::F32) {
        const f32x4* p = reinterpret_cast<const f32x4*>(x) + 2 * chunk;
        const f32x4 a = p[0], b = p[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    } else if constexpr (XK == XKind::F16) {
        const f16x8 h = __builtin_bit_cast(f16x8, reinterpret_cast<const u32x4*>(x)[chunk]);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
    } else {
        const u32x4 u = reinterpret_cast<const u32x4*>(x)[chunk];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __builtin_bit_cast(float, w[i] << 16);
            v[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xFFFF0000u);
        }
    }
}

// i32(f32) of the WGSL source, saturating; NaN -> 0.
__device__ __forceinline__ int f2i_sat(float r) {
    if (r != r) return 0;
    if (r >= 2147483520.0f) return 2147483647;
    if (r <= -2147483648.0f) return (-2147483647 - 1);
    return (int)r;
}

// Scale of a group from its max and min (the reference's thread-0 block).
template <int BITS>
__device__ __forceinline__ float group_scale(float mx, float mn) {
    const float amax = fmaxf(fabsf(mx), fabsf(mn));
    float s = amax / (BITS == 4 ? 7.0f : 127.0f);
    if (s == 0.0f) s = 1.0f;
    return s;
}

// q = clamp(i32(round(v / s))) with the correctly rounded quotient, as the reference.
// One IEEE division per group instead of one per value: t = v * (1/s) differs from the
// rounded quotient fl(v/s) by under 2^-15 (two roundings of 2^-24 relative, |v/s| < 2^8
// since |v| <= amax ~ 7s or 127s), so round(t) == round(fl(v/s)) unless t lies within
// that distance of a half-integer.  Those values (|frac(t) - 0.5| <= 2^-13, a wide
// margin) and groups whose 1/s overflows (s below 2^-128) take the exact division.
// NaN and infinite inputs give the same result on both paths.
template <int BITS>
struct QStep {
    float s, r;
    bool fast;
    __device__ __forceinline__ explicit QStep(float s_) : s(s_), r(1.0f / s_), fast(fabsf(r) <= 3.4028234e38f) {}
    __device__ __forceinline__ int operator()(float v) const {
        float t = v * r;
        if (!fast || fabsf(t - floorf(t) - 0.5f) <= 0x1p-13f) t = v / s;
        const int q = f2i_sat(rintf(t));
        return BITS == 4 ? min(max(q, -8), 7) : min(max(q, -128), 127);
    }
};

template <ScaleKind SK>
__device__ __forceinline__ void store_scale(void* S, size_t g, float s, float mn, float mx) {
    if constexpr (SK == ScaleKind::F16) reinterpret_cast<f16*>(S)[g] = (f16)s;
    else if constexpr (SK == ScaleKind::F32) reinterpret_cast<float*>(S)[g] = s;
    else reinterpret_cast<GroupScale*>(S)[g] = GroupScale{s, 0, mn, mx};
}

// The scale used for quantization is the stored one: an fp16 scale is rounded first.
template <ScaleKind SK>
__device__ __forceinline__ float stored_scale(float s) {
    if constexpr (SK == ScaleKind::F16) return (float)(f16)s;
    else return s;
}

// 8 quantized values -> packed output of chunk `c`.
template <int BITS>
__device__ __forceinline__ void store_q(void* Q, size_t c, const int (&q)[8], uint32_t ob) {
    if constexpr (BITS == 4) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) w |= (uint32_t)(q[i] & 0xF) << (4 * i);
        reinterpret_cast<uint32_t*>(Q)[c] = w ^ ob;  // two's complement nibbles, xor 8 -> offset-binary
    } else {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w0 |= (uint32_t)(q[i] & 0xFF) << (8 * i);
            w1 |= (uint32_t)(q[4 + i] & 0xFF) << (8 * i);
        }
        reinterpret_cast<u32x2*>(Q)[c] = u32x2{w0, w1};
    }
}

}  // namespace

// Groups of at most 512 elements: LPG = group_size / 8 lanes per group, one chunk of 8
// elements per lane.  `chunks` = rows * k / 8.
// Two rounds of 256 chunks per block (U = 2): both rounds' loads issue before the first
// reduction, 4 KB per wave in flight (1.5 % faster than one round, 4 rounds are slower).
template <XKind XK, int BITS, ScaleKind SK, int LPG>
__global__ __launch_bounds__(256) void k_quantize_small(const void* __restrict__ X, void* __restrict__ Q,
                                                        void* __restrict__ S, size_t chunks, uint32_t ob) {
    constexpr int U = 2;
    const size_t c0 = (size_t)blockIdx.x * 256 * U + threadIdx.x;
    float v[U][8];
    float mx[U], mn[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        mx[u] = -1e30f;  // the reference's initial values
        mn[u] = 1e30f;
        if (c0 + 256 * u < chunks) load8<XK>(X, c0 + 256 * u, v[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (c0 + 256 * u < chunks) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                mx[u] = fmaxf(mx[u], v[u][i]);
                mn[u] = fminf(mn[u], v[u][i]);
            }
        }
#pragma unroll
        for (int o = 1; o < LPG; o <<= 1) {
            mx[u] = fmaxf(mx[u], __shfl_xor(mx[u], o, 64));
            mn[u] = fminf(mn[u], __shfl_xor(mn[u], o, 64));
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t c = c0 + 256 * u;
        if (c >= chunks) break;
        const float s = group_scale<BITS>(mx[u], mn[u]);
        const float sq = stored_scale<SK>(s);
        if (c % LPG == 0) store_scale<SK>(S, c / LPG, s, mn[u], mx[u]);
        const QStep<BITS> qs(sq);
        int q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = qs(v[u][i]);
        store_q<BITS>(Q, c, q, ob);
    }
}

// Groups longer than 512 elements: one wave per group, two passes over it.
template <XKind XK, int BITS, ScaleKind SK>
__global__ __launch_bounds__(256) void k_quantize_large(const void* __restrict__ X, void* __restrict__ Q,
                                                        void* __restrict__ S, size_t groups, int cpg,
                                                        uint32_t ob) {
    const size_t g = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (g >= groups) return;
    const size_t c0 = g * (size_t)cpg;
    float mx = -1e30f, mn = 1e30f;
    for (int j = lane; j < cpg; j += 64) {
        float v[8];
        load8<XK>(X, c0 + j, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            mx = fmaxf(mx, v[i]);
            mn = fminf(mn, v[i]);
        }
    }
    mx = wave_max_f32(mx);
    mn = wave_min_f32(mn);
    const float s = group_scale<BITS>(mx, mn);
    const float sq = stored_scale<SK>(s);
    if (lane == 0) store_scale<SK>(S, g, s, mn, mx);
    const QStep<BITS> qs(sq);
    for (int j = lane; j < cpg; j += 64) {
        float v[8];
        load8<XK>(X, c0 + j, v);
        int q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = qs(v[i]);
        store_q<BITS>(Q, c0 + j, q, ob);
    }
}

// Groups of 513 .. 2048 * CPT elements (per-row scales of activations and weights): one
// 256-thread block per group, CPT chunks of 8 per thread held in registers, one pass.
template <XKind XK, int BITS, ScaleKind SK, int CPT, int NT = 256>
__global__ __launch_bounds__(NT) void k_quantize_rows(const void* __restrict__ X, void* __restrict__ Q,
                                                      void* __restrict__ S, int cpg, uint32_t ob) {
    constexpr int NW = NT / 64;
    __shared__ float red[2][NW];
    const size_t g = blockIdx.x;
    const int tid = threadIdx.x;
    const size_t c0 = g * (size_t)cpg;
    float v[CPT][8];
    float mx = -1e30f, mn = 1e30f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int cc = tid + NT * j;
        if (cc < cpg) {
            load8<XK>(X, c0 + cc, v[j]);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                mx = fmaxf(mx, v[j][i]);
                mn = fminf(mn, v[j][i]);
            }
        }
    }
    mx = wave_max_f32(mx);
    mn = wave_min_f32(mn);
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = mx;
        red[1][tid >> 6] = mn;
    }
    __syncthreads();
    mx = red[0][0];
    mn = red[1][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        mx = fmaxf(mx, red[0][w]);
        mn = fminf(mn, red[1][w]);
    }
    const float s = group_scale<BITS>(mx, mn);
    const float sq = stored_scale<SK>(s);
    if (tid == 0) store_scale<SK>(S, g, s, mn, mx);
    const QStep<BITS> qs(sq);
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int cc = tid + NT * j;
        if (cc < cpg) {
            int q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = qs(v[j][i]);
            store_q<BITS>(Q, c0 + cc, q, ob);
        }
    }
}

// xor of every word: offset-binary <-> two's complement nibbles (ob = tc ^ 0x8).
__global__ __launch_bounds__(256) void k_xor_words(const u32x4* __restrict__ in, u32x4* __restrict__ out,
                                                   size_t n4, uint32_t mask) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n4) out[i] = in[i] ^ mask;
}

__global__ __launch_bounds__(256) void k_xor_tail(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                  size_t from, size_t n, uint32_t mask) {
    const size_t i = from + (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = in[i] ^ mask;
}

// Scale format conversion.  A GroupScale written from F16/F32 carries zero_point 0 and
// group_min = group_max = 0 (the group's range is not known).
template <ScaleKind IN, ScaleKind OUT>
__global__ __launch_bounds__(256) void k_convert_scales(const void* __restrict__ in, void* __restrict__ out, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s;
    GroupScale gsv{};
    if constexpr (IN == ScaleKind::F16) s = (float)reinterpret_cast<const f16*>(in)[i];
    else if constexpr (IN == ScaleKind::F32) s = reinterpret_cast<const float*>(in)[i];
    else {
        gsv = reinterpret_cast<const GroupScale*>(in)[i];
        s = gsv.scale;
    }
    if constexpr (OUT == ScaleKind::F16) reinterpret_cast<f16*>(out)[i] = (f16)s;
    else if constexpr (OUT == ScaleKind::F32) reinterpret_cast<float*>(out)[i] = s;
    else reinterpret_cast<GroupScale*>(out)[i] = IN == ScaleKind::GroupScale ? gsv : GroupScale{s, 0, 0.0f, 0.0f};
}

// requantize_int32_to_int8 (quantized.wgsl:572-580): i32 in, i32 out in [-128, 127].
__global__ __launch_bounds__(256) void k_requantize(const int32_t* __restrict__ in, int32_t* __restrict__ out,
                                                    size_t n, float s_in, float s_out, int32_t zp) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = (float)in[i] * s_in;
    const float r = rintf(v / s_out) + (float)zp;
    out[i] = min(max(f2i_sat(r), -128), 127);
}

// quantize_int8_per_channel / dequantize_int8_per_channel (quantized.wgsl:264-297): one
// i32 per element and a 16-byte PerChannelScale {scale, zero_point, pad, pad} (:51-56)
// per channel_stride elements; quant_type 0 is the symmetric branch, any other value the
// asymmetric one.  HBM-bound (8 bytes per element); a thread takes 4 consecutive
// elements (16-byte accesses when both buffers are 16-byte aligned) and divides once for
// the channel of the first.
//   quantize:   q = clamp(i32(round(x / s) [+ f32(zp)]), -128, 127)   (:83-86, :92-95)
//   dequantize: x = f32(q [- zp]) * s, the i32 subtraction wrapping      (:88-90, :97-99)
template <bool DEQ, bool VEC>
__global__ __launch_bounds__(256) void k_int8_per_channel(const void* __restrict__ in,
                                                          const ChannelScale* __restrict__ ch,
                                                          void* __restrict__ out, size_t n, uint32_t stride,
                                                          int asym) {
    const size_t i0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 >= n) return;
    size_t c = i0 / stride;
    uint32_t rem = (uint32_t)(i0 - c * stride);
    ChannelScale cs = ch[c];
    uint32_t v[4] = {0u, 0u, 0u, 0u};
    const bool full = VEC && i0 + 4 <= n;
    if (full) {
        const u32x4 w = reinterpret_cast<const u32x4*>(in)[i0 / 4];
        v[0] = w.x, v[1] = w.y, v[2] = w.z, v[3] = w.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (i0 + e < n) v[e] = reinterpret_cast<const uint32_t*>(in)[i0 + e];
    }
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (rem == stride) {  // next channel
            ++c;
            rem = 0;
            if (i0 + e < n) cs = ch[c];
        }
        ++rem;
        if constexpr (DEQ) {
            const int32_t q = asym ? (int32_t)(v[e] - (uint32_t)cs.zero_point) : (int32_t)v[e];
            o[e] = __builtin_bit_cast(uint32_t, (float)q * cs.scale);
        } else {
            float r = rintf(__builtin_bit_cast(float, v[e]) / cs.scale);
            if (asym) r += (float)cs.zero_point;
            o[e] = (uint32_t)min(max(f2i_sat(r), -128), 127);
        }
    }
    if (full) {
        reinterpret_cast<u32x4*>(out)[i0 / 4] = u32x4{o[0], o[1], o[2], o[3]};
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (i0 + e < n) reinterpret_cast<uint32_t*>(out)[i0 + e] = o[e];
    }
}

// ---------------------------------------------------------------------------- host

// Dequantizer, 8-weight chunks (one int4 word or two int8 words; group_size % 8 == 0, so
// a chunk never straddles a group).  A wave covers 64 chunks per step and lane l takes
// half (l & 1) of chunk base + 32j + (l >> 1), j = 0, 1: its four outputs are elements
// 8*base + 256j + 4l .. +3, so every store instruction of the wave writes one contiguous
// span (1 KB of f32).  The natural layout (a lane's 8 outputs as two 16-B stores 32 B
// apart) half-fills each span per instruction and ran 1.5x slower (62 us against 40 us
// for 14336 x 4096 int4 -> f32).  Lane pairs read the same int4 word; int8 words are
// read contiguously.  One pass of the grid where it fits, grid-stride beyond.
template <int BITS, ScaleKind SK, YKind YK, bool POW2>
__device__ __forceinline__ void dequant_pair(const void* __restrict__ Q, const void* __restrict__ S,
                                             void* __restrict__ X, size_t base, size_t chunks, int gpr8,
                                             int gshift, uint32_t ob, bool full) {
    const int lane = threadIdx.x & 63, h = lane & 1;
    uint32_t w[2] = {0u, 0u};
    float sc[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const size_t c = base + 32 * j + (lane >> 1);
        if (full || c < chunks) {
            if constexpr (BITS == 4) w[j] = reinterpret_cast<const uint32_t*>(Q)[c] ^ ob;  // -> offset-binary
            else w[j] = reinterpret_cast<const uint32_t*>(Q)[2 * c + h];
            sc[j] = scale_from_raw<SK>(load_scale_raw<SK>(S, POW2 ? c >> gshift : c / (size_t)gpr8));
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const size_t c = base + 32 * j + (lane >> 1);
        if (!full && c >= chunks) break;
        f32x4 o;
        if constexpr (BITS == 4) {
            const uint32_t v = w[j] >> (16 * h);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (float)((int)((v >> (4 * i)) & 0xFu) - 8) * sc[j];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (float)(int)(int8_t)(w[j] >> (8 * i)) * sc[j];
        }
        store_y4<YK>(X, 8 * base + 256 * j + 4 * lane, o);
    }
}

// POW2: group_size / 8 is a power of two and the group index is a shift.  Waves whose
// 64 chunks are all in range take an unguarded copy of the body, so both word loads
// issue back to back.
template <int BITS, ScaleKind SK, YKind YK, bool POW2>
__global__ __launch_bounds__(256) void k_dequantize(const void* __restrict__ Q, const void* __restrict__ S,
                                                    void* __restrict__ X, size_t chunks, int gpr8,
                                                    int gshift, uint32_t ob) {
    const size_t waves = (size_t)gridDim.x * 4;
    for (size_t base = ((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 64; base < chunks; base += waves * 64) {
        if (base + 64 <= chunks) dequant_pair<BITS, SK, YK, POW2>(Q, S, X, base, chunks, gpr8, gshift, ob, true);
        else dequant_pair<BITS, SK, YK, POW2>(Q, S, X, base, chunks, gpr8, gshift, ob, false);
    }
}

template <XKind XK, int BITS, ScaleKind SK>
static hipError_t launch_q3(const QuantArgs& a, hipStream_t s) {
    const size_t chunks = (size_t)a.rows * a.k / 8;
    const int lpg = a.group_size / 8;
    const uint32_t ob = a.offset_binary ? 0x88888888u : 0u;
    if (lpg <= 64 && (lpg & (lpg - 1)) == 0) {
        const dim3 grid((unsigned)((chunks + 511) / 512)), block(256);  // 512 chunks per block
        switch (lpg) {
            case 1: hipLaunchKernelGGL((k_quantize_small<XK, BITS, SK, 1>), grid, block, 0, s, a.x, a.q, a.s, chunks, ob); break;
            case 2: hipLaunchKernelGGL((k_quantize_small<XK, BITS, SK, 2>), grid, block, 0, s, a.x, a.q, a.s, chunks, ob); break;
            case 4: hipLaunchKernelGGL((k_quantize_small<XK, BITS, SK, 4>), grid, block, 0, s, a.x, a.q, a.s, chunks, ob); break;
            case 8: hipLaunchKernelGGL((k_quantize_small<XK, BITS, SK, 8>), grid, block, 0, s, a.x, a.q, a.s, chunks, ob); break;
            case 16: hipLaunchKernelGGL((k_quantize_small<XK, BITS, SK, 16>), grid, block, 0, s, a.x, a.q, a.s, chunks, ob); break;
            case 32: hipLaunchKernelGGL((k_quantize_small<XK, BITS, SK, 32>), grid, block, 0, s, a.x, a.q, a.s, chunks, ob); break;
            case 64: hipLaunchKernelGGL((k_quantize_small<XK, BITS, SK, 64>), grid, block, 0, s, a.x, a.q, a.s, chunks, ob); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        const size_t groups = (size_t)a.rows * (a.k / a.group_size);
        const int cpt = (lpg + 255) / 256;  // chunks per thread with a block per group
        const dim3 gb((unsigned)groups), block(256);
        if (lpg > 256 && lpg <= 512)  // one chunk per thread, 8 waves per group
            hipLaunchKernelGGL((k_quantize_rows<XK, BITS, SK, 1, 512>), gb, dim3(512), 0, s, a.x, a.q, a.s, lpg, ob);
        else if (cpt <= 1) hipLaunchKernelGGL((k_quantize_rows<XK, BITS, SK, 1>), gb, block, 0, s, a.x, a.q, a.s, lpg, ob);
        else if (cpt <= 2) hipLaunchKernelGGL((k_quantize_rows<XK, BITS, SK, 2>), gb, block, 0, s, a.x, a.q, a.s, lpg, ob);
        else if (cpt <= 4) hipLaunchKernelGGL((k_quantize_rows<XK, BITS, SK, 4>), gb, block, 0, s, a.x, a.q, a.s, lpg, ob);
        else if (cpt <= 8) hipLaunchKernelGGL((k_quantize_rows<XK, BITS, SK, 8>), gb, block, 0, s, a.x, a.q, a.s, lpg, ob);
        else
            hipLaunchKernelGGL((k_quantize_large<XK, BITS, SK>), dim3((unsigned)((groups + 3) / 4)), dim3(256), 0, s,
                               a.x, a.q, a.s, groups, lpg, ob);
    }
    return hipGetLastError();
}

template <XKind XK, int BITS>
static hipError_t launch_q2(const QuantArgs& a, hipStream_t s) {
    switch (a.scale_kind) {
        case ScaleKind::F16: return launch_q3<XK, BITS, ScaleKind::F16>(a, s);
        case ScaleKind::F32: return launch_q3<XK, BITS, ScaleKind::F32>(a, s);
        case ScaleKind::GroupScale: return launch_q3<XK, BITS, ScaleKind::GroupScale>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <XKind XK>
static hipError_t launch_q1(const QuantArgs& a, hipStream_t s) {
    return a.bits == 4 ? launch_q2<XK, 4>(a, s) : launch_q2<XK, 8>(a, s);
}

hipError_t launch_quantize(const QuantArgs& a, hipStream_t s) {
    switch (a.x_kind) {
        case XKind::F32: return launch_q1<XKind::F32>(a, s);
        case XKind::F16: return launch_q1<XKind::F16>(a, s);
        case XKind::BF16: return launch_q1<XKind::BF16>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_xor_words(const void* in, void* out, size_t words, uint32_t mask, hipStream_t s) {
    const size_t n4 = ((uintptr_t)in | (uintptr_t)out) % 16 == 0 ? words / 4 : 0;
    if (n4)
        hipLaunchKernelGGL(k_xor_words, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                           static_cast<const u32x4*>(in), static_cast<u32x4*>(out), n4, mask);
    const size_t from = 4 * n4;
    if (from < words)
        hipLaunchKernelGGL(k_xor_tail, dim3((unsigned)((words - from + 255) / 256)), dim3(256), 0, s,
                           static_cast<const uint32_t*>(in), static_cast<uint32_t*>(out), from, words, mask);
    return hipGetLastError();
}

template <ScaleKind IN>
static hipError_t launch_cs(const void* in, void* out, ScaleKind ok, size_t n, hipStream_t s) {
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (ok) {
        case ScaleKind::F16: hipLaunchKernelGGL((k_convert_scales<IN, ScaleKind::F16>), grid, block, 0, s, in, out, n); break;
        case ScaleKind::F32: hipLaunchKernelGGL((k_convert_scales<IN, ScaleKind::F32>), grid, block, 0, s, in, out, n); break;
        case ScaleKind::GroupScale:
            hipLaunchKernelGGL((k_convert_scales<IN, ScaleKind::GroupScale>), grid, block, 0, s, in, out, n);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_convert_scales(const void* in, ScaleKind ik, void* out, ScaleKind ok, size_t n, hipStream_t s) {
    switch (ik) {
        case ScaleKind::F16: return launch_cs<ScaleKind::F16>(in, out, ok, n, s);
        case ScaleKind::F32: return launch_cs<ScaleKind::F32>(in, out, ok, n, s);
        case ScaleKind::GroupScale: return launch_cs<ScaleKind::GroupScale>(in, out, ok, n, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_int8_per_channel(bool dequantize, const void* in, const ChannelScale* ch, void* out, size_t n,
                                  uint32_t stride, bool asym, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const bool vec = ((uintptr_t)in & 15u) == 0 && ((uintptr_t)out & 15u) == 0;
    const dim3 grid((unsigned)((n + 1023) / 1024)), block(256);
    const int a = asym ? 1 : 0;
    if (dequantize) {
        if (vec) hipLaunchKernelGGL((k_int8_per_channel<true, true>), grid, block, 0, s, in, ch, out, n, stride, a);
        else hipLaunchKernelGGL((k_int8_per_channel<true, false>), grid, block, 0, s, in, ch, out, n, stride, a);
    } else {
        if (vec) hipLaunchKernelGGL((k_int8_per_channel<false, true>), grid, block, 0, s, in, ch, out, n, stride, a);
        else hipLaunchKernelGGL((k_int8_per_channel<false, false>), grid, block, 0, s, in, ch, out, n, stride, a);
    }
    return hipGetLastError();
}

hipError_t launch_requantize(const int32_t* in, int32_t* out, size_t n, float s_in, float s_out, int32_t zp,
                             hipStream_t s) {
    hipLaunchKernelGGL(k_requantize, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, out, n, s_in, s_out, zp);
    return hipGetLastError();
}


template <int BITS, ScaleKind SK>
static hipError_t launch_dq2(const QuantArgs& a, void* out, hipStream_t s) {
    const size_t chunks = (size_t)a.rows * a.k / 8;
    const size_t b = (chunks + 255) / 256;  // 64 chunks per wave, 4 waves per block
    const dim3 grid((unsigned)(b < (1u << 22) ? (b ? b : 1) : (1u << 22))), block(256);
    const int gpr8 = a.group_size / 8;  // chunks per group
    const int gshift = (gpr8 & (gpr8 - 1)) == 0 ? __builtin_ctz((unsigned)gpr8) : -1;
    const uint32_t ob = a.offset_binary ? 0u : 0x88888888u;
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, 0, s, a.q, a.s, out, chunks, gpr8, gshift, ob); };
    const bool p2 = gshift >= 0;
    switch (a.x_kind) {
        case XKind::F32: p2 ? go(k_dequantize<BITS, SK, YKind::F32, true>) : go(k_dequantize<BITS, SK, YKind::F32, false>); break;
        case XKind::F16: p2 ? go(k_dequantize<BITS, SK, YKind::F16, true>) : go(k_dequantize<BITS, SK, YKind::F16, false>); break;
        case XKind::BF16: p2 ? go(k_dequantize<BITS, SK, YKind::BF16, true>) : go(k_dequantize<BITS, SK, YKind::BF16, false>); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int BITS>
static hipError_t launch_dq1(const QuantArgs& a, void* out, hipStream_t s) {
    switch (a.scale_kind) {
        case ScaleKind::F16: return launch_dq2<BITS, ScaleKind::F16>(a, out, s);
        case ScaleKind::F32: return launch_dq2<BITS, ScaleKind::F32>(a, out, s);
        case ScaleKind::GroupScale: return launch_dq2<BITS, ScaleKind::GroupScale>(a, out, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dequantize(const QuantArgs& a, void* out, hipStream_t s) {
    return a.bits == 4 ? launch_dq1<4>(a, out, s) : launch_dq1<8>(a, out, s);
}

}  // namespace luxhip
