// gemv_impl.hpp -- the decode / batched-decode MoE kernel (slot form).
//
// Work items take three roles, one kernel each: router rows (fp32 router
// GEMV), gate_up rows (token, slot, row block) and down rows (token, row
// block).  The decode forward runs the three kernels back to back on one
// stream.  With `route_topk` every gate_up item runs its token's top-k from
// the logits (one wave, a few hundred cycles) instead of reading routes
// written by an earlier launch; with `fmt_h` it writes h already in the LDS
// layout the down kernel stages (formatted once, copied by every down
// work-group).  The standalone launchers read routes and keep plain fp32 h.
//
// Arithmetic: weights stream as 16-byte chunks per lane with their scales,
// all loads of an item issued before the activations are touched.  INT4,
// MXFP4 and BF16 weights are turned into exact bf16 pairs (INT4 codes as
// 128 + q by bit placement, e2m1 by the CDNA4 fp4 converter) and consumed
// by v_dot2c_f32_bf16 against the activations staged in LDS as bf16 pairs
// hi + lo (x = hi + lo to 2^-17; the lo pass is skipped when every lo is
// zero, e.g. for bf16 activations).  INT8 uses fp32 FMAs.  Routing-order
// semantics follow src/moe_kernels.cpp:82-445.
#pragma once

#include "common.hpp"
#include "gemv.hpp"
#include "topk.hpp"

#include <algorithm>

namespace grim {

// Phase timestamps for kernel studies: compiled in only with GRIM_TIMING.
#ifdef GRIM_TIMING
#define GRIM_TS(a, role, i)                                                          \
    do {                                                                             \
        if ((a).ts && threadIdx.x == 0 && blockIdx.x < 2048)                          \
            (a).ts[((role) * 2048 + blockIdx.x) * 8 + (i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define GRIM_TS(a, role, i) do {} while (0)
#endif

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kMaxJ = 4;          // chunk iterations prefetched per batch
constexpr int kRuGU = 2;          // (gate, up) pairs per gate_up lane group
constexpr int kPairsDN = 2;       // (slot, row) pairs per down lane group

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------ coherent I/O

// ------------------------------------------------------- activation staging
//
// Pair formats keep a staged vector of n elements as bf16 pair words:
//   hi[n/2], lo[n/2] (uint32, each plane in 16-byte quads stored
//   quad-major, see quad_pos), then one fp32 sum per chunk.
// INT4 pairs (x[8d+j], x[8d+j+4]) inside each dword d of a chunk, to match
// the nibble decoder; MXFP4 / BF16 pairs (x[2p], x[2p+1]).  INT8 keeps fp32
// x[n] then the chunk sums.

template <int F> struct Act {
    static constexpr bool kPair = F != GRIM_FMT_INT8;
    static constexpr bool kInterleave = F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16;
    // 16-byte quads per chunk in a plane (hi, lo, or the fp32 values)
    static constexpr int kQuads = (kPair ? Chunk<F>::CH / 2 : Chunk<F>::CH) / 4;
};

// Quads are stored quad-major: quad d of chunk c at d * nch + c.  Lanes
// that read consecutive chunks then read consecutive 16-byte LDS slots,
// free of bank conflicts, where chunk-major storage would put them 64 bytes
// apart.
template <int F>
__device__ __forceinline__ int quad_pos(int k, int nch) {
    constexpr int Q = Act<F>::kQuads;
    return (k % Q) * nch + k / Q;
}

__device__ __forceinline__ uint32_t split_hi_lo(float v, uint32_t& lo) {
    const uint16_t h = f32_to_bf16(v);
    lo = f32_to_bf16(v - bf16_to_f32(h));
    return h;
}

// Formatted group of eight activations: bf16 pair words hi / lo (INT4:
// (x[j], x[j+4]) to match the nibble decoder; else adjacent) and the sum
// of the staged values (hi + lo) in element order.
template <int F>
__device__ __forceinline__ float format_group(const float (&v)[8], uint32_t (&hw)[4],
                                              uint32_t (&lw)[4], int& any_lo) {
    uint32_t h[8], l[8];
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        h[i] = split_hi_lo(v[i], l[i]);
        part += bits_f(h[i] << 16) + bits_f(l[i] << 16);
        any_lo |= int(l[i] != 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e0 = Act<F>::kInterleave ? j : 2 * j;
        const int e1 = Act<F>::kInterleave ? j + 4 : 2 * j + 1;
        hw[j] = h[e0] | (h[e1] << 16);
        lw[j] = l[e0] | (l[e1] << 16);
    }
    return part;
}

// Chunk sums from per-group sums: the TPC threads of a chunk are aligned
// lanes; the first of them writes.
template <int F>
__device__ __forceinline__ void chunk_sum_out(float part, int g, float* sums) {
    constexpr int TPC = Chunk<F>::CH / 8;   // threads per chunk (4, 2 or 1)
    if constexpr (TPC >= 2) part += dpp_f<kDppXor1>(part);
    if constexpr (TPC >= 4) part += dpp_f<kDppXor2>(part);
    if (g >= 0 && (g % TPC) == 0) sums[g / TPC] = part;
}

// Stage src[0..n) (fp32, n % CH == 0, n % 8 == 0) into LDS, eight elements
// per thread and up to NB groups of eight in flight per thread; returns
// whether any lo half is non-zero (block-uniform).  The chunk sums are sums
// of the staged values (hi + lo), so that the offset correction of the INT4
// decoder cancels exactly what the dots added.
template <int F, int NB = 2>
__device__ __forceinline__ bool stage_act(const float* __restrict__ src, int n, uint32_t* lds) {
    int any_lo = 0;
    float* sums = reinterpret_cast<float*>(lds + n);
    const int ng = n / 8;
    const int nch = n / Chunk<F>::CH;
    const float4* s4 = reinterpret_cast<const float4*>(src);
    for (int g0 = 0; g0 < ng; g0 += NB * blockDim.x) {
        float4 p[NB], q[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int g = g0 + b * blockDim.x + threadIdx.x;
            if (g < ng) { p[b] = s4[2 * g]; q[b] = s4[2 * g + 1]; }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (g0 + b * blockDim.x >= ng) break;   // block-uniform
            const int gi = g0 + b * blockDim.x + threadIdx.x;
            const int g = gi < ng ? gi : -1;
            float part = 0.0f;
            if (g >= 0) {
                const float v[8] = {p[b].x, p[b].y, p[b].z, p[b].w, q[b].x, q[b].y, q[b].z, q[b].w};
                if constexpr (Act<F>::kPair) {
                    uint32_t hw[4], lw[4];
                    part = format_group<F>(v, hw, lw, any_lo);
                    const int qp = quad_pos<F>(g, nch);
                    reinterpret_cast<u32x4*>(lds)[qp] = u32x4{hw[0], hw[1], hw[2], hw[3]};
                    reinterpret_cast<u32x4*>(lds + n / 2)[qp] = u32x4{lw[0], lw[1], lw[2], lw[3]};
                } else {
                    reinterpret_cast<float4*>(lds)[quad_pos<F>(2 * g, nch)] = p[b];
                    reinterpret_cast<float4*>(lds)[quad_pos<F>(2 * g + 1, nch)] = q[b];
#pragma unroll
                    for (int i = 0; i < 8; ++i) part += v[i];
                }
            }
            chunk_sum_out<F>(part, g, sums);
        }
    }
    if constexpr (Act<F>::kPair) any_lo = __syncthreads_or(any_lo);
    else __syncthreads();
    return any_lo != 0;
}

// ------------------------------------------------------ formatted h vectors
//
// The gate_up kernel can write h already in the staged LDS layout (words
// [0, n): the planes, quad-major), followed by one fp32 sum per group of
// eight (words [n, n + n/8)); a down work-group then stages it by copying,
// with the chunk sums formed from the group sums by the same DPP steps as
// stage_act uses, so both paths give the same bits.

// Write group g (eight values) of a formatted vector of n elements at dst.
template <int F>
__device__ __forceinline__ void put_group_fmt(uint32_t* dst, int n, int g, const float (&v)[8]) {
    const int nch = n / Chunk<F>::CH;
    float part = 0.0f;
    if constexpr (Act<F>::kPair) {
        uint32_t hw[4], lw[4];
        int any = 0;
        part = format_group<F>(v, hw, lw, any);
        const int qp = quad_pos<F>(g, nch);
        reinterpret_cast<u32x4*>(dst)[qp] = u32x4{hw[0], hw[1], hw[2], hw[3]};
        reinterpret_cast<u32x4*>(dst + n / 2)[qp] = u32x4{lw[0], lw[1], lw[2], lw[3]};
    } else {
        reinterpret_cast<float4*>(dst)[quad_pos<F>(2 * g, nch)] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(dst)[quad_pos<F>(2 * g + 1, nch)] = make_float4(v[4], v[5], v[6], v[7]);
#pragma unroll
        for (int i = 0; i < 8; ++i) part += v[i];
    }
    reinterpret_cast<float*>(dst)[n + g] = part;
}

// Stage a formatted vector of n elements (NB quads per thread in flight);
// returns whether any lo half is non-zero (block-uniform).
template <int F, int NB = 4>
__device__ __forceinline__ bool stage_fmt(const uint32_t* __restrict__ src, int n, uint32_t* lds) {
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
    const float* ps = reinterpret_cast<const float*>(src) + n;
    float* sums = reinterpret_cast<float*>(lds + n);
    const int nq = n / 4, ng = n / 8;
    const int lo_q = Act<F>::kPair ? n / 8 : nq;   // first quad of the lo plane
    int any_lo = 0;
    // groups are half as many as quads: iteration q0 covers groups from q0 / 2
    for (int q0 = 0; q0 < nq; q0 += NB * blockDim.x) {
        u32x4 v[NB];
        float pv[NB / 2];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int q = q0 + b * blockDim.x + threadIdx.x;
            if (q < nq) v[b] = s4[q];
        }
#pragma unroll
        for (int c = 0; c < NB / 2; ++c) {
            const int g = q0 / 2 + c * blockDim.x + threadIdx.x;
            pv[c] = g < ng ? ps[g] : 0.0f;
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int q = q0 + b * blockDim.x + threadIdx.x;
            if (q < nq) {
                reinterpret_cast<u32x4*>(lds)[q] = v[b];
                if (q >= lo_q) any_lo |= int((v[b].x | v[b].y | v[b].z | v[b].w) != 0);
            }
        }
#pragma unroll
        for (int c = 0; c < NB / 2; ++c) {
            const int g = q0 / 2 + c * blockDim.x + threadIdx.x;
            chunk_sum_out<F>(pv[c], g < ng ? g : -1, sums);
        }
    }
    if constexpr (Act<F>::kPair) any_lo = __syncthreads_or(any_lo);
    else __syncthreads();
    return any_lo != 0;
}


// Activation staging split in two halves, so that the global loads can be
// issued together with the routing loads and the LDS formatting can run
// while the weight loads are in flight.  kXG groups of eight per thread
// cover n <= 8192; out-of-range groups reload the thread's first group
// (clamped address, no branch around the load).
constexpr int kXG = 4;
struct XRegs {
    float4 p[kXG], q[kXG];
};

__device__ __forceinline__ void x_load(const float* __restrict__ src, int n, XRegs& r) {
    const int ng = n / 8;
    const int tid = threadIdx.x;
    const int g_safe = tid < ng ? tid : ng - 1;
    const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
    for (int b = 0; b < kXG; ++b) {
        const int g = tid + b * kGemvThreads;
        const int gi = g < ng ? g : g_safe;
        r.p[b] = s4[2 * gi];
        r.q[b] = s4[2 * gi + 1];
    }
}

// Format the loaded groups into LDS (layout of stage_act); returns whether
// any lo half is non-zero (block-uniform).  Ends with a barrier.
template <int F>
__device__ __forceinline__ bool x_store(const XRegs& r, int n, uint32_t* lds) {
    int any_lo = 0;
    float* sums = reinterpret_cast<float*>(lds + n);
    const int ng = n / 8;
    const int nch = n / Chunk<F>::CH;
#pragma unroll
    for (int b = 0; b < kXG; ++b) {
        if (b * kGemvThreads >= ng) break;   // block-uniform
        const int gi = b * kGemvThreads + int(threadIdx.x);
        const int g = gi < ng ? gi : -1;
        float part = 0.0f;
        if (g >= 0) {
            const float v[8] = {r.p[b].x, r.p[b].y, r.p[b].z, r.p[b].w,
                                r.q[b].x, r.q[b].y, r.q[b].z, r.q[b].w};
            if constexpr (Act<F>::kPair) {
                uint32_t hw[4], lw[4];
                part = format_group<F>(v, hw, lw, any_lo);
                const int qp = quad_pos<F>(g, nch);
                reinterpret_cast<u32x4*>(lds)[qp] = u32x4{hw[0], hw[1], hw[2], hw[3]};
                reinterpret_cast<u32x4*>(lds + n / 2)[qp] = u32x4{lw[0], lw[1], lw[2], lw[3]};
            } else {
                reinterpret_cast<float4*>(lds)[quad_pos<F>(2 * g, nch)] = r.p[b];
                reinterpret_cast<float4*>(lds)[quad_pos<F>(2 * g + 1, nch)] = r.q[b];
#pragma unroll
                for (int i = 0; i < 8; ++i) part += v[i];
            }
        }
        chunk_sum_out<F>(part, g, sums);
    }
    if constexpr (Act<F>::kPair) any_lo = __syncthreads_or(any_lo);
    else __syncthreads();
    return any_lo != 0;
}

// The formatted h of one token (n elements: nq = n / 4 quads of planes,
// then n / 8 group sums), same two halves: the first kHQ quads and kHQ / 2
// sums per thread are loaded up front; h_store writes them and copies any
// remainder with ordinary loads.
constexpr int kHQ = 8;
struct HRegs {
    u32x4 v[kHQ];
    float s[kHQ / 2];
};

__device__ __forceinline__ void h_load(const uint32_t* __restrict__ src, int n, HRegs& r) {
    const int nq = n / 4, ng = n / 8;
    const int tid = threadIdx.x;
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
    const float* ps = reinterpret_cast<const float*>(src) + n;
    const int q_safe = tid < nq ? tid : nq - 1;
    const int g_safe = tid < ng ? tid : ng - 1;
#pragma unroll
    for (int b = 0; b < kHQ; ++b) {
        const int q = tid + b * kGemvThreads;
        r.v[b] = s4[q < nq ? q : q_safe];
    }
#pragma unroll
    for (int c = 0; c < kHQ / 2; ++c) {
        const int g = tid + c * kGemvThreads;
        r.s[c] = ps[g < ng ? g : g_safe];
    }
}

template <int F>
__device__ __forceinline__ bool h_store(const HRegs& r, const uint32_t* __restrict__ src, int n,
                                        uint32_t* lds) {
    const int nq = n / 4, ng = n / 8;
    const int lo_q = Act<F>::kPair ? n / 8 : nq;   // first quad of the lo plane
    const int tid = threadIdx.x;
    float* sums = reinterpret_cast<float*>(lds + n);
    int any_lo = 0;
#pragma unroll
    for (int b = 0; b < kHQ; ++b) {
        const int q = tid + b * kGemvThreads;
        if (q < nq) {
            reinterpret_cast<u32x4*>(lds)[q] = r.v[b];
            if (q >= lo_q) any_lo |= int((r.v[b].x | r.v[b].y | r.v[b].z | r.v[b].w) != 0);
        }
    }
#pragma unroll
    for (int c = 0; c < kHQ / 2; ++c) {
        if (c * kGemvThreads >= ng) break;   // block-uniform
        const int g = tid + c * kGemvThreads;
        chunk_sum_out<F>(g < ng ? r.s[c] : 0.0f, g < ng ? g : -1, sums);
    }
    // remainder (long h vectors)
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
    for (int q = kHQ * kGemvThreads + tid; q < nq; q += kGemvThreads) {
        const u32x4 v = s4[q];
        reinterpret_cast<u32x4*>(lds)[q] = v;
        if (q >= lo_q) any_lo |= int((v.x | v.y | v.z | v.w) != 0);
    }
    const float* ps = reinterpret_cast<const float*>(src) + n;
    for (int g0 = (kHQ / 2) * kGemvThreads; g0 < ng; g0 += kGemvThreads) {
        const int g = g0 + tid;
        chunk_sum_out<F>(g < ng ? ps[g] : 0.0f, g < ng ? g : -1, sums);
    }
    if constexpr (Act<F>::kPair) any_lo = __syncthreads_or(any_lo);
    else __syncthreads();
    return any_lo != 0;
}

template <int F>
__host__ __device__ constexpr int act_words(int n) {
    // LDS words of a staged vector of n elements (pairs or fp32, + sums)
    return n + n / Chunk<F>::CH;
}

// ------------------------------------------------------------- chunk math

// One weight chunk in flight: the raw loads only.  Scales are decoded where
// the chunk is consumed, so that issuing a load never waits for another.
struct Pre {
    u32x4 raw;
    uint32_t sb;   // INT4: bf16/fp16 group-scale bits, MXFP4: e8m0 byte, INT8: fp32 bits
    uint32_t zb;   // INT4: zero point (0xFF = signed s4)
};

template <int F>
__device__ __forceinline__ void prefetch(const WView& w, int64_t row, int c, Pre& p) {
    p.raw = load16(w.payload + row * w.row_bytes + int64_t(c) * 16);
    if constexpr (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) {
        const int64_t si = row * w.row_scales + ((c * 32) >> w.gshift);
        p.sb = static_cast<const uint16_t*>(w.scales)[si];
        // no branch around the load (a branch makes the compiler wait for
        // the loads before it): without zeros, read a payload byte and
        // substitute the default
        const bool hz = w.zeros != nullptr;
        const uint32_t zl = (hz ? w.zeros : w.payload)[hz ? si : 0];
        p.zb = hz ? zl : uint32_t(w.default_zero);
    } else if constexpr (F == GRIM_FMT_MXFP4) {
        p.sb = static_cast<const uint8_t*>(w.scales)[row * w.row_scales + c];
    } else if constexpr (F == GRIM_FMT_INT8) {
        p.sb = f_bits(static_cast<const float*>(w.scales)[row]);
    }
}

template <int F>
__device__ __forceinline__ float pre_scale(const Pre& p) {
    if constexpr (F == GRIM_FMT_INT4) return bf16_to_f32(uint16_t(p.sb));
    else if constexpr (F == GRIM_FMT_INT4_F16) return f16_to_f32(uint16_t(p.sb));
    else if constexpr (F == GRIM_FMT_MXFP4) return e8m0_to_f32(uint8_t(p.sb));
    else if constexpr (F == GRIM_FMT_INT8) return bits_f(p.sb);
    else return 1.0f;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    bf16x2_t x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    return __builtin_amdgcn_fdot2_f32_bf16(x, y, c, false);
}

// The activations of one chunk, read from LDS once and shared by every
// weight row a lane multiplies with them.
template <int F, bool LO>
struct XChunk {
    static constexpr int W = Act<F>::kPair ? Chunk<F>::CH / 2 : Chunk<F>::CH;
    uint32_t hi[W];
    uint32_t lo[LO ? W : 1];
    float xs;
};

template <int F, bool LO>
__device__ __forceinline__ void load_x(const uint32_t* act, int n, int c, XChunk<F, LO>& x) {
    constexpr int W = XChunk<F, LO>::W;
    const int nch = n / Chunk<F>::CH;
    const u32x4* h = reinterpret_cast<const u32x4*>(act) + c;
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
        const u32x4 v = h[i * nch];
        x.hi[4 * i] = v.x; x.hi[4 * i + 1] = v.y; x.hi[4 * i + 2] = v.z; x.hi[4 * i + 3] = v.w;
    }
    if constexpr (LO) {
        const u32x4* l = reinterpret_cast<const u32x4*>(act + n / 2) + c;
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const u32x4 v = l[i * nch];
            x.lo[4 * i] = v.x; x.lo[4 * i + 1] = v.y; x.lo[4 * i + 2] = v.z; x.lo[4 * i + 3] = v.w;
        }
    }
    x.xs = reinterpret_cast<const float*>(act + n)[c];
}

// Contribution of one prefetched weight chunk against x.
template <int F, bool LO>
__device__ __forceinline__ float dot_chunk(const Pre& p, const XChunk<F, LO>& x) {
    const uint32_t w[4] = {p.raw.x, p.raw.y, p.raw.z, p.raw.w};
    float a0 = 0.0f, a1 = 0.0f;
    if constexpr (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) {
        int z = int(p.zb);
        uint32_t xm = 0;
        if (z == 0xFF) { xm = 0x88888888u; z = 8; }   // signed s4 -> offset binary
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t ww = w[d] ^ xm;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t pr = ((ww >> (4 * j)) & 0x000F000Fu) | 0x43004300u;   // 128 + q
                a0 = dot2(pr, x.hi[4 * d + j], a0);
                if constexpr (LO) a1 = dot2(pr, x.lo[4 * d + j], a1);
            }
        }
        return pre_scale<F>(p) * ((a0 + a1) - (128.0f + float(z)) * x.xs);
    } else if constexpr (F == GRIM_FMT_MXFP4) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const bf16x2_t v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 0);
            const bf16x2_t v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 1);
            const bf16x2_t v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 2);
            const bf16x2_t v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 3);
            uint32_t q[4];
            __builtin_memcpy(&q[0], &v0, 4);
            __builtin_memcpy(&q[1], &v1, 4);
            __builtin_memcpy(&q[2], &v2, 4);
            __builtin_memcpy(&q[3], &v3, 4);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                a0 = dot2(q[b], x.hi[4 * d + b], a0);
                if constexpr (LO) a1 = dot2(q[b], x.lo[4 * d + b], a1);
            }
        }
        return (a0 + a1) * pre_scale<F>(p);
    } else if constexpr (F == GRIM_FMT_BF16) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            a0 = dot2(w[d], x.hi[d], a0);
            if constexpr (LO) a1 = dot2(w[d], x.lo[d], a1);
        }
        return a0 + a1;
    } else {   // INT8 on fp32 activations (hi holds the fp32 bits)
        float xv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) xv[i] = bits_f(x.hi[i]);
        return pre_scale<F>(p) * (Chunk<GRIM_FMT_INT8>::dot(p.raw, xv) - 128.0f * x.xs);
    }
}

// ------------------------------------------------------------------ roles

// Router rows: item b computes expert b's logits (plus the softmax router
// bias) for every token (router_row).
__device__ __forceinline__ void router_item(const DecodeArgs& a, int b) {
    __shared__ float red[4 * kRouterTok];
    const int e = b;
    const float s = router_row(a.router + int64_t(e) * a.H, a.x, a.M, a.H, red);
    if (int(threadIdx.x) < a.M)
        a.logits[int64_t(threadIdx.x) * a.E + e] = a.rbias ? s + a.rbias[e] : s;
}

// gate_up rows of one (token, slot, row block): RU (gate, up) row pairs per
// lane group, one chunk of the next iteration in flight while this one is
// multiplied.
template <int F, int LPR, bool LO>
__device__ __forceinline__ void gate_up_rows(const WView& v, int64_t gbase, int i0, int I, int C,
                                             int sub, const uint32_t* act, int n,
                                             Pre (&cur)[2][kRuGU], float* ga, float* ua) {
    for (int c = sub; c < C; c += LPR) {
        Pre nxt[2][kRuGU];
        const int cn = c + LPR;
        if (cn < C) {
#pragma unroll
            for (int r = 0; r < kRuGU; ++r) {
                const int i = i0 + r < I ? i0 + r : I - 1;
                prefetch<F>(v, gbase + i, cn, nxt[0][r]);
                prefetch<F>(v, gbase + I + i, cn, nxt[1][r]);
            }
        }
        XChunk<F, LO> x;
        load_x<F, LO>(act, n, c, x);
#pragma unroll
        for (int r = 0; r < kRuGU; ++r) {
            ga[r] += dot_chunk<F, LO>(cur[0][r], x);
            ua[r] += dot_chunk<F, LO>(cur[1][r], x);
        }
        if (cn < C) {
#pragma unroll
            for (int r = 0; r < kRuGU; ++r) { cur[0][r] = nxt[0][r]; cur[1][r] = nxt[1][r]; }
        }
    }
}

template <int F, int LPR, bool SH, bool RT>
__device__ __forceinline__ void gate_up_item(const DecodeArgs& a, int j, uint32_t* lds) {
    constexpr int GPW = kWave / LPR;
    constexpr int RU = kRuGU;
    constexpr int RB = kGemvWaves * GPW * RU;
    const int H = a.H, I = a.I, K = a.K;
    const int KS = K + (SH ? 1 : 0);
    const int C = H / Chunk<F>::CH;
    const int t = j / (KS * a.gu_rb);
    const int slot = (j / a.gu_rb) % KS;
    const int rb = j % a.gu_rb;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sub = lane % LPR;
    const int i0 = rb * RB + (wave * GPW + lane / LPR) * RU;
    const float* xt = a.x + int64_t(t) * H;
    float* ht = a.h + (int64_t(t) * KS + slot) * I;
    GRIM_TS(a, 1, 0);

    // (1) everything that does not depend on the routing is requested at
    // once: the token's activations and (RT) its router logits
    XRegs xr;
    x_load(xt, H, xr);
    const bool shr = SH && slot >= K;   // block-uniform
    int64_t gbase = 0;
    bool active = true;
    if constexpr (RT) {
        // (2) the token's top-k from the router logits of the previous
        // launch; the first item of the token also stores the routes
        __shared__ int sel_e[16];
        __shared__ float sel_w[16];
        __shared__ float tk_scratch[512 + 64];
        if (!shr) {
            float lv[kMaxV];
            if (wave == 0) {
                topk_load(a.logits + int64_t(t) * a.E, a.E, lv);
                topk_wave_regs(lv, a.E, K, a.mode, a.normalize, a.scaling, a.bias16, a.bias32,
                               a.n_group, a.topk_group, sel_e, sel_w, tk_scratch, tk_scratch + 512);
            }
            __syncthreads();
            if (slot == 0 && rb == 0 && int(threadIdx.x) < K) {
                a.rex[int64_t(t) * K + threadIdx.x] = sel_e[threadIdx.x];
                a.rwt[int64_t(t) * K + threadIdx.x] = sel_w[threadIdx.x];
            }
            const int e = sel_e[slot];
            if (e < 0 || e >= a.E) active = false;
            gbase = int64_t(e) * 2 * I;
        }
    } else if (!shr) {
        const int e = a.rex[int64_t(t) * K + slot];
        if (e < 0 || e >= a.E) active = false;   // route not computed here: h = 0
        gbase = int64_t(e) * 2 * I;
    }
    GRIM_TS(a, 1, 1);
    // (3) this item's weights, all requested before anything waits on them
    const WView v = (SH && shr) ? a.sgu : a.gu;
    if (!active) gbase = 0;   // rows of expert 0 are read and discarded
    float ga[RU], ua[RU];
    Pre cur[2][RU];
#pragma unroll
    for (int r = 0; r < RU; ++r) {
        ga[r] = 0.0f;
        ua[r] = 0.0f;
        const int i = i0 + r < I ? i0 + r : I - 1;
        const int c = sub < C ? sub : 0;
        prefetch<F>(v, gbase + i, c, cur[0][r]);
        prefetch<F>(v, gbase + I + i, c, cur[1][r]);
    }
    // (4) the activations into LDS while the weights are in flight
    const bool lo_pass = x_store<F>(xr, H, lds);
    GRIM_TS(a, 1, 2);
    if (active) {
        if (lo_pass) gate_up_rows<F, LPR, true>(v, gbase, i0, I, C, sub, lds, H, cur, ga, ua);
        else gate_up_rows<F, LPR, false>(v, gbase, i0, I, C, sub, lds, H, cur, ga, ua);
    }
    GRIM_TS(a, 1, 3);
    __shared__ float hrow[kGemvWaves * kWave / 8 * RU];   // this item's RB rows (fmt_h)
#pragma unroll
    for (int r = 0; r < RU; ++r) {
        const float g = group_sum<LPR>(ga[r]);
        const float u = group_sum<LPR>(ua[r]);
        const int i = i0 + r;
        const float hv = active ? silu(g) * u : 0.0f;
        if (a.fmt_h) {
            if (sub == 0) hrow[(wave * GPW + lane / LPR) * RU + r] = i < I ? hv : 0.0f;
        } else if (sub == 0 && i < I) {
            ht[i] = hv;
        }
    }
    if (a.fmt_h) {
        // the RB rows as RB / 8 formatted groups of the token's h vector
        __syncthreads();
        const int n = KS * I;
        const int i8 = rb * RB + 8 * int(threadIdx.x);
        if (int(threadIdx.x) < RB / 8 && i8 < I) {
            float hv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) hv[k] = hrow[8 * threadIdx.x + k];
            put_group_fmt<F>(a.hf + int64_t(t) * fmt_words(n), n, (slot * I + i8) / 8, hv);
        }
    }
    // shared_expert_gate: sigmoid(x . gate_w) (src/moe_kernels.cpp:162-172),
    // by the first item of each token
    if (a.gate_w && slot == 0 && rb == 0 && wave == 0) {
        float acc = 0.0f;
        for (int c = lane; c < H; c += kWave) acc = __builtin_fmaf(bf16_to_f32(a.gate_w[c]), xt[c], acc);
        acc = group_sum<kWave>(acc);
        if (lane == 0) a.gate[t] = det_sigmoid(acc);
    }
    GRIM_TS(a, 1, 4);
}

// Weight chunks of one batch of down rows: up to kDnBatch chunks per lane
// for each of its kPairsDN (slot, row) pairs, all requested at once.
constexpr int kDnBatch = 3;

template <int F, int LPR>
__device__ __forceinline__ void down_issue(const DecodeArgs& a, const bool* pvalid,
                                           const bool* pshared, const int64_t* wrow, int C,
                                           int c0, Pre (&w)[kDnBatch][kPairsDN]) {
    // clamped addresses instead of branches around the loads (chunks past
    // the row end and invalid pairs are loaded and never used)
#pragma unroll
    for (int b = 0; b < kDnBatch; ++b) {
        const int c = c0 + b * LPR;
        const int cc = c < C ? c : C - 1;
#pragma unroll
        for (int q = 0; q < kPairsDN; ++q)
            prefetch<F>(pshared[q] ? a.sdn : a.dn, pvalid[q] ? wrow[q] : 0, cc, w[b][q]);
    }
}

template <int F, int LPR, bool LO>
__device__ __forceinline__ void down_rows(const DecodeArgs& a, const int* pslot, const bool* pvalid,
                                          const bool* pshared, const int64_t* wrow, int C, int sub,
                                          const uint32_t* act, int n,
                                          Pre (&w)[kDnBatch][kPairsDN], float* acc) {
    for (int c0 = sub; c0 < C; c0 += kDnBatch * LPR) {
        if (c0 != sub) down_issue<F, LPR>(a, pvalid, pshared, wrow, C, c0, w);
#pragma unroll
        for (int b = 0; b < kDnBatch; ++b) {
            const int c = c0 + b * LPR;
            if (c >= C) break;
#pragma unroll
            for (int q = 0; q < kPairsDN; ++q) {
                if (!pvalid[q]) continue;
                XChunk<F, LO> x;
                load_x<F, LO>(act, n, pslot[q] * C + c, x);
                acc[q] += dot_chunk<F, LO>(w[b][q], x);
            }
        }
    }
}

// down rows of one (token, row block); (slot, row) pairs per lane group,
// combined in slot order.
template <int F, int LPR, bool SH>
__device__ __forceinline__ void down_item(const DecodeArgs& a, int j, uint32_t* lds) {
    constexpr int G = kGemvThreads / LPR;
    constexpr int NP = kPairsDN;
    const int H = a.H, I = a.I, K = a.K, E = a.E;
    const int KS = K + (SH ? 1 : 0);
    const int C = I / Chunk<F>::CH;
    const int RB = a.dn_rb;
    const int nb = (H + RB - 1) / RB;
    const int t = j / nb;
    const int o_base = (j % nb) * RB;
    const int grp = threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    const int npairs = KS * RB;
    const int n = KS * I;
    float* part = reinterpret_cast<float*>(lds + act_words<F>(n));   // [KS][RB]
    __shared__ float slot_w[32];   // routed weight per slot, 0 = skipped
    __shared__ int slot_e[32];     // expert per slot, -1 = skipped
    GRIM_TS(a, 2, 0);

    // (1) routes (earlier launch) and the token's h requested together
    HRegs hr;
    const uint32_t* hsrc = a.hf + int64_t(t) * fmt_words(n);
    if (a.fmt_h) h_load(hsrc, n, hr);
    {
        const int s = int(threadIdx.x) < K ? int(threadIdx.x) : 0;
        const int e = a.rex[int64_t(t) * K + s];
        const float rw = a.rwt[int64_t(t) * K + s];
        if (int(threadIdx.x) < K) {
            const bool ok = e >= 0 && e < E && rw != 0.0f;
            slot_w[threadIdx.x] = ok ? rw : 0.0f;
            slot_e[threadIdx.x] = ok ? e : -1;
        }
    }
    __syncthreads();
    GRIM_TS(a, 2, 1);
    int pslot[NP], prow[NP];
    int64_t wrow[NP];
    bool pshared[NP], pvalid[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const int p = grp + q * G;
        pslot[q] = p % KS;
        prow[q] = p / KS;
        const int o = min(o_base + prow[q], H - 1);
        pvalid[q] = p < npairs && o_base + prow[q] < H;
        pshared[q] = SH && pslot[q] >= K;
        wrow[q] = o;
        if (pvalid[q] && !pshared[q]) {
            const int e = slot_e[pslot[q]];
            if (e < 0) pvalid[q] = false;
            else wrow[q] = int64_t(e) * H + o;
        }
    }
    float acc[NP];
    Pre w[kDnBatch][NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) acc[q] = 0.0f;
    // (2) the first batch of weights, then h into LDS while they fly
    down_issue<F, LPR>(a, pvalid, pshared, wrow, C, sub, w);
    float gate_sh = 1.0f;
    if (SH && a.gate_in && int(threadIdx.x) < RB) gate_sh = a.gate_in[t];
    const bool lo_pass = a.fmt_h ? h_store<F>(hr, hsrc, n, lds)
                                  : stage_act<F, 4>(a.h + int64_t(t) * n, n, lds);
    GRIM_TS(a, 2, 2);
    if (lo_pass) down_rows<F, LPR, true>(a, pslot, pvalid, pshared, wrow, C, sub, lds, n, w, acc);
    else down_rows<F, LPR, false>(a, pslot, pvalid, pshared, wrow, C, sub, lds, n, w, acc);
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const float v = group_sum<LPR>(acc[q]);
        const int p = grp + q * G;
        if (sub == 0 && p < npairs) part[pslot[q] * RB + prow[q]] = pvalid[q] ? v : 0.0f;
    }
    GRIM_TS(a, 2, 3);
    __syncthreads();
    for (int r = threadIdx.x; r < RB; r += blockDim.x) {
        const int o = o_base + r;
        if (o >= H) continue;
        float total = 0.0f;
        for (int s = 0; s < K; ++s) {
            const float rw = slot_w[s];
            if (rw == 0.0f) continue;
            total = __builtin_fmaf(rw, part[s * RB + r], total);
        }
        if (SH) total = __builtin_fmaf(gate_sh, part[K * RB + r], total);
        a.y[int64_t(t) * H + o] = total;
    }
    GRIM_TS(a, 2, 4);
}

}  // namespace grim
#include "gemv_wave.hpp"
namespace grim {

template <int F>
constexpr bool kWaveGateUp = F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16 || F == GRIM_FMT_MXFP4;

// Router rows: the first launch of the decode forward; with xf, the same
// work-groups also format the activations for the wave-centric gate_up.
template <int F>
__global__ __launch_bounds__(kGemvThreads) void moe_router_kernel(DecodeArgs a) {
    GRIM_TS(a, 0, 0);
    if constexpr (kWaveGateUp<F>) {
        if (a.xf && a.M == 1) {
            // one token: the router row's loads first, the formatting of x
            // while they fly, then the dot (router_row's arithmetic)
            __shared__ float red[4 * kRouterTok];
            const int e = blockIdx.x;
            const float* wr = a.router + int64_t(e) * a.H;
            float s;
            if (a.H <= 2048) {
                RouterRegs<2> rr;
                router_row1_load(wr, a.x, a.H, rr);
                xf_format<F>(a, blockIdx.x);
                s = router_row1_finish(rr, a.H, red);
            } else if (a.H <= 4096) {
                RouterRegs<4> rr;
                router_row1_load(wr, a.x, a.H, rr);
                xf_format<F>(a, blockIdx.x);
                s = router_row1_finish(rr, a.H, red);
            } else {
                RouterRegs<8> rr;
                router_row1_load(wr, a.x, a.H, rr);
                xf_format<F>(a, blockIdx.x);
                s = router_row1_finish(rr, a.H, red);
            }
            if (threadIdx.x == 0) a.logits[e] = a.rbias ? s + a.rbias[e] : s;
            GRIM_TS(a, 0, 1);
            return;
        }
        if (a.xf) xf_format<F>(a, blockIdx.x);
    }
    router_item(a, blockIdx.x);
    GRIM_TS(a, 0, 1);
}

// The expert kernels.  gate_up: RT = the items run the top-k from the
// logits, else they read routes; down reads routes (and h) of earlier
// launches.
template <int F, int LPG, bool SH, bool RT>
__global__ __launch_bounds__(kGemvThreads) void moe_gate_up_kernel(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    gate_up_item<F, LPG, SH, RT>(a, blockIdx.x, lds);
}
template <int F, int LPD, bool SH>
__global__ __launch_bounds__(kGemvThreads) void moe_down_kernel(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    down_item<F, LPD, SH>(a, blockIdx.x, lds);
}

// ------------------------------------------------------------ launching

template <int F, int LPG, int LPD, bool SH>
inline hipError_t launch_t(hipStream_t st, const DecodeArgs& a) {
    if (a.NR) hipLaunchKernelGGL(moe_router_kernel<F>, dim3(a.NR), dim3(kGemvThreads), 0, st, a);
    DecodeArgs gu = a, dn = a;   // LDS of each kernel from its own role
    gu.NR = 0;
    gu.ND = 0;
    dn.NR = 0;
    dn.NG = 0;
    bool wave_done = false;
    if constexpr (kWaveGateUp<F>) {
        if (a.NG && a.xf) {
            // wave-centric gate_up: NCI chunk iterations of RU rows (4 for one iteration, else 2)
            const int nci = (a.H / 32 + kWave - 1) / kWave;
            if (nci == 1 && a.gu_ru == 6)
                hipLaunchKernelGGL((moe_gate_up_wave_kernel<F, 6, 1, SH>), dim3(a.NG), dim3(kGemvThreads), 0, st, a);
            else if (nci == 1 && a.gu_ru == 8)
                hipLaunchKernelGGL((moe_gate_up_wave_kernel<F, 8, 1, SH>), dim3(a.NG), dim3(kGemvThreads), 0, st, a);
            else if (nci == 1)
                hipLaunchKernelGGL((moe_gate_up_wave_kernel<F, 4, 1, SH>), dim3(a.NG), dim3(kGemvThreads), 0, st, a);
            else if (nci == 2)
                hipLaunchKernelGGL((moe_gate_up_wave_kernel<F, 2, 2, SH>), dim3(a.NG), dim3(kGemvThreads), 0, st, a);
            else
                hipLaunchKernelGGL((moe_gate_up_wave_kernel<F, 2, 4, SH>), dim3(a.NG), dim3(kGemvThreads), 0, st, a);
            wave_done = true;
        }
    }
    if (wave_done) {
    } else if (a.NG && a.route_topk)
        hipLaunchKernelGGL((moe_gate_up_kernel<F, LPG, SH, true>), dim3(a.NG), dim3(kGemvThreads),
                           decode_lds_bytes(F, gu), st, a);
    else if (a.NG)
        hipLaunchKernelGGL((moe_gate_up_kernel<F, LPG, SH, false>), dim3(a.NG), dim3(kGemvThreads),
                           decode_lds_bytes(F, gu), st, a);
    bool dn_done = false;
    if constexpr (kWaveGateUp<F>) {
        if (a.ND && a.dn_wave) {
            const int KS = a.K + (SH ? 1 : 0);
            const int nci = (a.I / 32 + 31) / 32;
            const dim3 blk(KS * kWave);
            if (nci == 1)
                hipLaunchKernelGGL((moe_down_wave_kernel<F, 4, 1, SH>), dim3(a.ND), blk, 0, st, a);
            else if (nci == 2)
                hipLaunchKernelGGL((moe_down_wave_kernel<F, 2, 2, SH>), dim3(a.ND), blk, 0, st, a);
            else
                hipLaunchKernelGGL((moe_down_wave_kernel<F, 2, 4, SH>), dim3(a.ND), blk, 0, st, a);
            dn_done = true;
        }
    }
    if (a.ND && !dn_done)
        hipLaunchKernelGGL((moe_down_kernel<F, LPD, SH>), dim3(a.ND), dim3(kGemvThreads),
                           decode_lds_bytes(F, dn), st, a);
    return hipGetLastError();
}

template <int F, int LPG, bool SH>
inline hipError_t pick_lpd(hipStream_t st, const DecodeArgs& a) {
    switch (a.lpr_dn) {
    case 4: return launch_t<F, LPG, 4, SH>(st, a);
    case 8: return launch_t<F, LPG, 8, SH>(st, a);
    case 16: return launch_t<F, LPG, 16, SH>(st, a);
    case 32: return launch_t<F, LPG, 32, SH>(st, a);
    }
    return hipErrorInvalidValue;
}

template <int F, bool SH>
inline hipError_t pick_lpg(hipStream_t st, const DecodeArgs& a) {
    switch (a.lpr_gu) {
    case 8: return pick_lpd<F, 8, SH>(st, a);
    case 16: return pick_lpd<F, 16, SH>(st, a);
    case 32: return pick_lpd<F, 32, SH>(st, a);
    case 64: return pick_lpd<F, 64, SH>(st, a);
    }
    return hipErrorInvalidValue;
}

}  // namespace grim
#include "gemv_fused.hpp"
namespace grim {

template <int F>
inline hipError_t fused_launch(hipStream_t st, const DecodeArgs& a) {
    if constexpr (kWaveGateUp<F>) {
        const dim3 g(a.fz_G), blk(kFzThreads);
        if (a.fz_ru == 3 && a.fz_rh == 4) hipLaunchKernelGGL((moe_decode_fused_kernel<F, 3, 4>), g, blk, 0, st, a);
        else if (a.fz_ru == 2 && a.fz_rh == 4) hipLaunchKernelGGL((moe_decode_fused_kernel<F, 2, 4>), g, blk, 0, st, a);
        else if (a.fz_ru == 4 && a.fz_rh == 4) hipLaunchKernelGGL((moe_decode_fused_kernel<F, 4, 4>), g, blk, 0, st, a);
        else if (a.fz_ru == 2 && a.fz_rh == 2) hipLaunchKernelGGL((moe_decode_fused_kernel<F, 2, 2>), g, blk, 0, st, a);
        else if (a.fz_ru == 3 && a.fz_rh == 2) hipLaunchKernelGGL((moe_decode_fused_kernel<F, 3, 2>), g, blk, 0, st, a);
        else if (a.fz_ru == 4 && a.fz_rh == 2) hipLaunchKernelGGL((moe_decode_fused_kernel<F, 4, 2>), g, blk, 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

#define GRIM_DECODE_INSTANTIATE(F)                                               \
    hipError_t decode_launch_fmt_##F(hipStream_t st, const DecodeArgs& a) {   \
        if (a.fused) return fused_launch<F>(st, a);                             \
        return a.shared ? pick_lpg<F, true>(st, a) : pick_lpg<F, false>(st, a); \
    }

}  // namespace grim
