// common.hpp -- device helpers shared by the gfx950 MoE kernels.
//
// Wave64 reductions, bf16/fp16 conversions, the deterministic exp used by
// the routers, and the per-format "chunk" decoders: every weight format is
// consumed 16 bytes per lane at a time (one global_load_dwordx4), so a
// 64-lane wave streams 1 KiB per load instruction.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/grimoire_moe.h"

namespace grim {

constexpr int kWave = 64;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bits_f(uint32_t b) { return __uint_as_float(b); }
__device__ __forceinline__ uint32_t f_bits(float f) { return __float_as_uint(f); }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return bits_f(uint32_t(b) << 16); }

// round to nearest even; NaN stays NaN (include/b70/formats.hpp:88-97)
// (selects, not branches: it runs per element in the staging loops)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t u = f_bits(f);
    const uint32_t special = (u >> 16) | ((u & 0x7FFFFFu) ? 0x40u : 0u);   // inf / NaN (quieted)
    const uint32_t rounded = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;     // nearest even
    return uint16_t(((u >> 23) & 0xFFu) == 0xFFu ? special : rounded);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return float(v);
}

// e8m0 -> fp32 (include/b70/formats.hpp:105-109)
// (selects, not branches: it sits in the inner loops)
__device__ __forceinline__ float e8m0_to_f32(uint8_t x) {
    uint32_t b = uint32_t(x) << 23;
    b = x == 0x00 ? 0x00400000u : b;
    b = x == 0xFF ? 0x7FC00000u : b;
    return bits_f(b);
}

// exp(x): Cody-Waite reduction to |r| <= ln2/2, degree-7 Taylor polynomial
// in Horner form, and a 2^k scale applied as two exact power-of-two
// factors.  Written with explicit fma so that the host test oracle, which
// restates the same steps, gets identical bits.
__device__ __forceinline__ float det_expf(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -103.972084045410156f) return 0.0f;
    const float kf = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.428606765330187045e-06f, r);
    float p = 1.98412698412698413e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int k = int(kf);
    const int k1 = k / 2, k2 = k - k1;
    const float s1 = bits_f(uint32_t(k1 + 127) << 23);
    const float s2 = bits_f(uint32_t(k2 + 127) << 23);
    return (p * s1) * s2;
}

__device__ __forceinline__ float det_sigmoid(float x) {
#pragma clang fp contract(off)
    return 1.0f / (1.0f + det_expf(-x));
}

__device__ __forceinline__ float silu(float v) {
#pragma clang fp contract(off)
    return v / (1.0f + det_expf(-v));
}

// silu with the hardware exp2 / reciprocal (each ~1 ulp): for epilogues
// whose outputs are compared to a tolerance, not bit for bit.
__device__ __forceinline__ float fast_silu(float v) {
    const float e = __builtin_amdgcn_exp2f(v * -1.44269504088896341f);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// Cross-lane moves inside a 16-lane row (DPP, no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return __builtin_amdgcn_update_dpp(0u, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16

// Sum over aligned groups of LPR lanes (LPR a power of two <= 64); every
// lane of a group ends with the same value (each step adds a symmetric
// pair, so the partners compute identical sums).
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (LPR >= 2) v += dpp_f<kDppXor1>(v);
    if constexpr (LPR >= 4) v += dpp_f<kDppXor2>(v);
    if constexpr (LPR >= 8) v += dpp_f<kDppHalfMirror>(v);
    if constexpr (LPR >= 16) v += dpp_f<kDppMirror>(v);
    if constexpr (LPR >= 32) v += __shfl_xor(v, 16, kWave);
    if constexpr (LPR >= 64) v += __shfl_xor(v, 32, kWave);
    return v;
}

// ---------------------------------------------------------------------
// Format traits.  A chunk is 16 payload bytes holding CH elements.
//   dot(raw, x)  : sum over the chunk of code_j * x_j, where code_j is the
//                  element's integer code (INT4: 0..15 offset binary,
//                  INT8: 0..255 offset binary) or the unscaled value
//                  (BF16, MXFP4 e2m1); scales are applied by the caller.
// ---------------------------------------------------------------------
template <int F> struct Chunk;

template <> struct Chunk<GRIM_FMT_INT4> {
    static constexpr int CH = 32;
    static constexpr bool kOffset = true;    // needs sum(x) per chunk
    __device__ __forceinline__ static float dot(const u32x4 raw, const float* __restrict__ x) {
        float a0 = 0.0f, a1 = 0.0f;
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t lo = w[d] & 0x0F0F0F0Fu;
            const uint32_t hi = (w[d] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a0 = __builtin_fmaf(float((lo >> (8 * j)) & 0xFFu), x[8 * d + 2 * j], a0);
                a1 = __builtin_fmaf(float((hi >> (8 * j)) & 0xFFu), x[8 * d + 2 * j + 1], a1);
            }
        }
        return a0 + a1;
    }
};
template <> struct Chunk<GRIM_FMT_INT4_F16> : Chunk<GRIM_FMT_INT4> {};

template <> struct Chunk<GRIM_FMT_INT8> {
    static constexpr int CH = 16;
    static constexpr bool kOffset = true;
    // int8 codes are read as offset binary (x ^ 0x80 = q + 128); the caller
    // subtracts 128 * sum(x)
    __device__ __forceinline__ static float dot(const u32x4 raw, const float* __restrict__ x) {
        float a0 = 0.0f, a1 = 0.0f;
        const uint32_t w[4] = {raw.x ^ 0x80808080u, raw.y ^ 0x80808080u, raw.z ^ 0x80808080u,
                               raw.w ^ 0x80808080u};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            a0 = __builtin_fmaf(float(w[d] & 0xFFu), x[4 * d + 0], a0);
            a1 = __builtin_fmaf(float((w[d] >> 8) & 0xFFu), x[4 * d + 1], a1);
            a0 = __builtin_fmaf(float((w[d] >> 16) & 0xFFu), x[4 * d + 2], a0);
            a1 = __builtin_fmaf(float(w[d] >> 24), x[4 * d + 3], a1);
        }
        return a0 + a1;
    }
};

template <> struct Chunk<GRIM_FMT_BF16> {
    static constexpr int CH = 8;
    static constexpr bool kOffset = false;
    __device__ __forceinline__ static float dot(const u32x4 raw, const float* __restrict__ x) {
        float a0 = 0.0f, a1 = 0.0f;
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            a0 = __builtin_fmaf(bits_f(w[d] << 16), x[2 * d], a0);
            a1 = __builtin_fmaf(bits_f(w[d] & 0xFFFF0000u), x[2 * d + 1], a1);
        }
        return a0 + a1;
    }
};

template <> struct Chunk<GRIM_FMT_MXFP4> {
    static constexpr int CH = 32;
    static constexpr bool kOffset = false;
    // e2m1 pairs decoded by the CDNA4 fp4 converter (scale 1; the e8m0
    // block scale is applied to the chunk's partial sum).  Byte b of a
    // dword holds elements 2b (low nibble) and 2b+1 (high nibble).
    __device__ __forceinline__ static float dot(const u32x4 raw, const float* __restrict__ x) {
        float a0 = 0.0f, a1 = 0.0f;
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const f32x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 0);
            const f32x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 1);
            const f32x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 2);
            const f32x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 3);
            a0 = __builtin_fmaf(p0.x, x[8 * d + 0], a0);
            a1 = __builtin_fmaf(p0.y, x[8 * d + 1], a1);
            a0 = __builtin_fmaf(p1.x, x[8 * d + 2], a0);
            a1 = __builtin_fmaf(p1.y, x[8 * d + 3], a1);
            a0 = __builtin_fmaf(p2.x, x[8 * d + 4], a0);
            a1 = __builtin_fmaf(p2.y, x[8 * d + 5], a1);
            a0 = __builtin_fmaf(p3.x, x[8 * d + 6], a0);
            a1 = __builtin_fmaf(p3.y, x[8 * d + 7], a1);
        }
        return a0 + a1;
    }
};

// INT4 group shift from the shape (include/b70/weights.hpp:80-84)
__host__ __device__ __forceinline__ int int4_gshift(int row_scales, int K) {
    const int64_t rs = row_scales, k = K;
    return rs * 32 == k ? 5 : rs * 64 == k ? 6 : rs * 256 == k ? 8 : 7;
}

// Device copy of a weight view, passed by value to kernels.
struct WView {
    const uint8_t* payload;
    const void* scales;
    const uint8_t* zeros;
    int64_t row_bytes;
    int row_scales;
    int gshift;
    int default_zero;   // INT4_F16 without zeros: 8
};

// Apply chunk c's scale to its partial: returns the row contribution.
//   xs: sum of the chunk's x (offset formats), ignored otherwise.
template <int F>
__device__ __forceinline__ float chunk_scaled(const WView& w, int64_t row, int c, u32x4 raw,
                                              const float* __restrict__ x, float xs);

template <>
__device__ __forceinline__ float chunk_scaled<GRIM_FMT_BF16>(const WView&, int64_t, int, u32x4 raw,
                                                             const float* __restrict__ x, float) {
    return Chunk<GRIM_FMT_BF16>::dot(raw, x);
}
template <>
__device__ __forceinline__ float chunk_scaled<GRIM_FMT_INT8>(const WView&, int64_t, int, u32x4 raw,
                                                             const float* __restrict__ x, float xs) {
    // per-row scale applied by the caller at the end
    return Chunk<GRIM_FMT_INT8>::dot(raw, x) - 128.0f * xs;
}
template <>
__device__ __forceinline__ float chunk_scaled<GRIM_FMT_MXFP4>(const WView& w, int64_t row, int c,
                                                              u32x4 raw, const float* __restrict__ x,
                                                              float) {
    const uint8_t e = static_cast<const uint8_t*>(w.scales)[row * w.row_scales + c];
    return Chunk<GRIM_FMT_MXFP4>::dot(raw, x) * e8m0_to_f32(e);
}
template <int F>
__device__ __forceinline__ float int4_chunk(const WView& w, int64_t row, int c, u32x4 raw,
                                            const float* __restrict__ x, float xs) {
    const int g = (c * 32) >> w.gshift;
    const int64_t si = row * w.row_scales + g;
    const uint16_t sraw = static_cast<const uint16_t*>(w.scales)[si];
    const float s = F == GRIM_FMT_INT4 ? bf16_to_f32(sraw) : f16_to_f32(sraw);
    int z = w.zeros ? int(w.zeros[si]) : w.default_zero;
    if (z == 0xFF) {   // signed s4: xor 8 turns it into offset binary with zero 8
        raw.x ^= 0x88888888u; raw.y ^= 0x88888888u; raw.z ^= 0x88888888u; raw.w ^= 0x88888888u;
        z = 8;
    }
    return s * (Chunk<GRIM_FMT_INT4>::dot(raw, x) - float(z) * xs);
}
template <>
__device__ __forceinline__ float chunk_scaled<GRIM_FMT_INT4>(const WView& w, int64_t row, int c,
                                                             u32x4 raw, const float* __restrict__ x,
                                                             float xs) {
    return int4_chunk<GRIM_FMT_INT4>(w, row, c, raw, x, xs);
}
template <>
__device__ __forceinline__ float chunk_scaled<GRIM_FMT_INT4_F16>(const WView& w, int64_t row, int c,
                                                                 u32x4 raw,
                                                                 const float* __restrict__ x,
                                                                 float xs) {
    return int4_chunk<GRIM_FMT_INT4_F16>(w, row, c, raw, x, xs);
}

inline WView make_view(const grim_quant_weight& w) {
    WView v;
    v.payload = w.payload;
    v.scales = w.scales;
    v.zeros = w.zeros;
    v.row_bytes = w.row_bytes;
    v.row_scales = w.row_scales;
    v.gshift = (w.fmt == GRIM_FMT_INT4 || w.fmt == GRIM_FMT_INT4_F16) ? int4_gshift(w.row_scales, w.K) : 0;
    v.default_zero = w.fmt == GRIM_FMT_INT4_F16 ? 8 : 0;
    return v;
}

template <int F>
__device__ __forceinline__ float row_scale(const WView& w, int64_t row) {
    if constexpr (F == GRIM_FMT_INT8) return static_cast<const float*>(w.scales)[row];
    return 1.0f;
}

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

}  // namespace grim
