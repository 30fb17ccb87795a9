// gemv_impl.hpp -- the decode / batched-decode MoE kernel (slot form).
//
// Work items take three roles: router rows (fp32 router GEMV; the last
// router item also runs the top-k), gate_up rows (token, slot, row block) and
// down rows (token, row block).  The standalone launchers run one role per
// kernel; the decode forward (`fused`) runs two launches, the router kernel
// and then one kernel holding every gate_up and down item, which hands h
// over on the device:
//
//   - one work-group per item, gate_up items first.  gate_up items never
//     wait; a down item waits only for gate_up items, whose work-group ids
//     are all lower, and work-groups are dispatched in id order, so a
//     waiting down item never holds a slot that a not-yet-dispatched gate_up
//     item needs;
//   - hand-off data (logits, routes, h, gate) is written and read with
//     device-coherent (sc1) accesses, and a producer waits for its own
//     stores (vmcnt 0) before it counts itself done, so no cache writeback
//     fence is needed;
//   - the h counter is spread over 64 cache lines (one same-address atomic
//     costs ~11 ns on this GPU, a per-block writeback fence ~45 ns); waits
//     are bounded and record a sticky timeout flag instead of hanging.
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

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kMaxJ = 4;          // chunk iterations prefetched per batch
constexpr int kRuGU = 2;          // (gate, up) pairs per gate_up lane group
constexpr int kPairsDN = 2;       // (slot, row) pairs per down lane group

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------ coherent I/O

__device__ __forceinline__ float ld_coh(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_coh(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// counters (int32 offsets inside ctr[])
constexpr int kCtrRouterDone = 0;
constexpr int kCtrRoutesReady = 32;
constexpr int kCtrTimeout = 64;
constexpr int kCtrHDone = 128;                 // 64 lines of 32 ints
constexpr int kCtrDnDone = kCtrHDone + 64 * 32;
constexpr int kSpinLimit = 1 << 16;   // ~0.1 s of polling, then give up

// Timeout codes recorded in ctr[kCtrTimeout] (sticky, never reset here).
constexpr int kTimeoutRoutes = 1, kTimeoutH = 2;

__device__ __forceinline__ void wait_flag(int* p, int* timeout) {
    if (threadIdx.x == 0) {
        int it = 0;
        while (ld_coh(p) == 0) {
            __builtin_amdgcn_s_sleep(2);
            if (++it > kSpinLimit) { st_coh(timeout, kTimeoutRoutes); break; }
        }
    }
    __syncthreads();
}

// sum of the 64 spread counters at base (one wave)
__device__ __forceinline__ int spread_sum(const int* base) {
    const int lane = threadIdx.x & (kWave - 1);
    return int(group_sum<kWave>(float(ld_coh(base + 32 * lane))));
}

__device__ __forceinline__ void wait_spread(const int* base, int target, int* timeout) {
    if (threadIdx.x < kWave) {
        int it = 0;
        while (spread_sum(base) < target) {
            __builtin_amdgcn_s_sleep(2);
            if (++it > kSpinLimit) {
                if (threadIdx.x == 0) st_coh(timeout, kTimeoutH);
                break;
            }
        }
    }
    __syncthreads();
}

// ------------------------------------------------------- activation staging
//
// Pair formats keep a staged vector of n elements as bf16 pair words:
//   hi[n/2], lo[n/2] (uint32), then one fp32 sum per chunk.
// INT4 pairs (x[8d+j], x[8d+j+4]) inside each dword d of a chunk, to match
// the nibble decoder; MXFP4 / BF16 pairs (x[2p], x[2p+1]).  INT8 keeps fp32
// x[n] then the chunk sums.

template <int F> struct Act {
    static constexpr bool kPair = F != GRIM_FMT_INT8;
    static constexpr bool kInterleave = F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16;
};

__device__ __forceinline__ uint32_t split_hi_lo(float v, uint32_t& lo) {
    const uint16_t h = f32_to_bf16(v);
    lo = f32_to_bf16(v - bf16_to_f32(h));
    return h;
}

// Two device-coherent 16-byte loads (sc1: served from the coherence point,
// never from a stale cache line), for data other work-groups of the same
// launch wrote.
__device__ __forceinline__ void ld_coh32(const float* p, float4& a, float4& b) {
    u32x4 ra, rb;
    asm volatile("global_load_dwordx4 %0, %2, off sc1\n\t"
                 "global_load_dwordx4 %1, %2, off offset:16 sc1\n\t"
                 "s_waitcnt vmcnt(0)"
                 : "=&v"(ra), "=&v"(rb)
                 : "v"(p)
                 : "memory");
    a = make_float4(bits_f(ra.x), bits_f(ra.y), bits_f(ra.z), bits_f(ra.w));
    b = make_float4(bits_f(rb.x), bits_f(rb.y), bits_f(rb.z), bits_f(rb.w));
}

// Stage src[0..n) (n % CH == 0, n % 8 == 0) into LDS, eight elements per
// thread; returns whether any lo half is non-zero (block-uniform).  The
// chunk sums are sums of the staged values (hi + lo), so that the offset
// correction of the INT4 decoder cancels exactly what the dots added.
template <int F, bool COH>
__device__ __forceinline__ bool stage_act(const float* __restrict__ src, int n, uint32_t* lds) {
    constexpr int CH = Chunk<F>::CH;
    constexpr int TPC = CH / 8;            // threads per chunk (4, 2 or 1)
    int any_lo = 0;
    float* sums = reinterpret_cast<float*>(lds + n);
    for (int g0 = 0; g0 < n / 8; g0 += blockDim.x) {
        const int g = g0 + threadIdx.x;    // group of elements [8g, 8g + 8)
        float part = 0.0f;
        if (g < n / 8) {
            float4 p, q;
            if (COH) {
                ld_coh32(src + 8 * g, p, q);
            } else {
                p = reinterpret_cast<const float4*>(src)[2 * g];
                q = reinterpret_cast<const float4*>(src)[2 * g + 1];
            }
            const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
            if constexpr (Act<F>::kPair) {
                uint32_t h[8], l[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    h[i] = split_hi_lo(v[i], l[i]);
                    part += bits_f(h[i] << 16) + bits_f(l[i] << 16);
                    any_lo |= int(l[i] != 0);
                }
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // INT4: (x[j], x[j+4]) to match the nibble decoder; else adjacent
                    const int e0 = Act<F>::kInterleave ? j : 2 * j;
                    const int e1 = Act<F>::kInterleave ? j + 4 : 2 * j + 1;
                    hw[j] = h[e0] | (h[e1] << 16);
                    lw[j] = l[e0] | (l[e1] << 16);
                }
                reinterpret_cast<u32x4*>(lds)[g] = u32x4{hw[0], hw[1], hw[2], hw[3]};
                reinterpret_cast<u32x4*>(lds + n / 2)[g] = u32x4{lw[0], lw[1], lw[2], lw[3]};
            } else {
                reinterpret_cast<float4*>(lds)[2 * g] = p;
                reinterpret_cast<float4*>(lds)[2 * g + 1] = q;
#pragma unroll
                for (int i = 0; i < 8; ++i) part += v[i];
            }
        }
        // chunk sum over the TPC threads of a chunk (aligned lane groups)
        if constexpr (TPC >= 2) part += dpp_f<kDppXor1>(part);
        if constexpr (TPC >= 4) part += dpp_f<kDppXor2>(part);
        if (g < n / 8 && (g % TPC) == 0) sums[g / TPC] = part;
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

struct Pre {
    u32x4 raw;
    float s;      // INT4: group scale, MXFP4: e8m0 scale, INT8: row scale
    int z;        // INT4: zero point (0xFF = signed s4)
};

template <int F>
__device__ __forceinline__ void prefetch(const WView& w, int64_t row, int c, Pre& p) {
    p.raw = load16(w.payload + row * w.row_bytes + int64_t(c) * 16);
    if constexpr (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) {
        const int64_t si = row * w.row_scales + ((c * 32) >> w.gshift);
        const uint16_t sraw = static_cast<const uint16_t*>(w.scales)[si];
        p.s = F == GRIM_FMT_INT4 ? bf16_to_f32(sraw) : f16_to_f32(sraw);
        p.z = w.zeros ? int(w.zeros[si]) : w.default_zero;
    } else if constexpr (F == GRIM_FMT_MXFP4) {
        p.s = e8m0_to_f32(static_cast<const uint8_t*>(w.scales)[row * w.row_scales + c]);
    } else if constexpr (F == GRIM_FMT_INT8) {
        p.s = static_cast<const float*>(w.scales)[row];
    }
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
    const u32x4* h = reinterpret_cast<const u32x4*>(act + c * W);
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
        const u32x4 v = h[i];
        x.hi[4 * i] = v.x; x.hi[4 * i + 1] = v.y; x.hi[4 * i + 2] = v.z; x.hi[4 * i + 3] = v.w;
    }
    if constexpr (LO) {
        const u32x4* l = reinterpret_cast<const u32x4*>(act + n / 2 + c * W);
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const u32x4 v = l[i];
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
        int z = p.z;
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
        return p.s * ((a0 + a1) - (128.0f + float(z)) * x.xs);
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
        return (a0 + a1) * p.s;
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
        return p.s * (Chunk<GRIM_FMT_INT8>::dot(p.raw, xv) - 128.0f * x.xs);
    }
}

// ------------------------------------------------------------------ roles

// Router rows: wave w of item b computes expert e = 4b + w for every token;
// the last router item to finish runs the top-k and raises routes_ready.
__device__ __forceinline__ void router_item(const DecodeArgs& a, int b, uint32_t* lds) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int e = b * kGemvWaves + wave;
    if (e < a.E) {
        const float* wr = a.router + int64_t(e) * a.H;
        for (int t = 0; t < a.M; ++t) {
            const float* xt = a.x + int64_t(t) * a.H;
            float acc = 0.0f;
            for (int k = lane * 4; k < a.H; k += kWave * 4) {
                const float4 wv = *reinterpret_cast<const float4*>(wr + k);
                const float4 xv = *reinterpret_cast<const float4*>(xt + k);
                acc = __builtin_fmaf(wv.x, xv.x, acc);
                acc = __builtin_fmaf(wv.y, xv.y, acc);
                acc = __builtin_fmaf(wv.z, xv.z, acc);
                acc = __builtin_fmaf(wv.w, xv.w, acc);
            }
            acc = group_sum<kWave>(acc);
            if (lane == 0) st_coh(a.logits + int64_t(t) * a.E + e, a.rbias ? acc + a.rbias[e] : acc);
        }
    }
    wait_stores();
    __syncthreads();
    __shared__ int last;
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(a.ctr + kCtrRouterDone, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == a.NR - 1;
    __syncthreads();
    if (last) {
        float* scratch = reinterpret_cast<float*>(lds) + wave * (512 + 64);
        for (int t = wave; t < a.M; t += kGemvWaves)
            topk_wave<true>(a.logits + int64_t(t) * a.E, a.E, a.K, a.mode, a.normalize, a.scaling,
                            a.bias16, a.bias32, a.n_group, a.topk_group, a.rex + int64_t(t) * a.K,
                            a.rwt + int64_t(t) * a.K, scratch, scratch + 512);
        wait_stores();
        __syncthreads();
        if (threadIdx.x == 0) st_coh(a.ctr + kCtrRoutesReady, 1);
    }
    __syncthreads();
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

template <int F, int LPR, bool SH>
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

    bool lo_pass = true, staged = false;
    if (a.fused) {   // stage x while the router is still running
        lo_pass = stage_act<F, false>(xt, H, lds);
        staged = true;
        wait_flag(a.ctr + kCtrRoutesReady, a.ctr + kCtrTimeout);
    }
    const bool shr = SH && slot >= K;
    int64_t gbase = 0;
    bool active = true;
    if (!shr) {
        const int e = ld_coh(a.rex + int64_t(t) * K + slot);
        if (e < 0 || e >= a.E) active = false;   // route not computed here: h = 0
        gbase = int64_t(e) * 2 * I;
    }
    const WView v = (SH && shr) ? a.sgu : a.gu;
    float ga[RU], ua[RU];
    Pre cur[2][RU];
#pragma unroll
    for (int r = 0; r < RU; ++r) {
        ga[r] = 0.0f;
        ua[r] = 0.0f;
        if (active && sub < C) {
            const int i = i0 + r < I ? i0 + r : I - 1;
            prefetch<F>(v, gbase + i, sub, cur[0][r]);
            prefetch<F>(v, gbase + I + i, sub, cur[1][r]);
        }
    }
    if (!staged) lo_pass = stage_act<F, false>(xt, H, lds);   // overlaps the first loads
    if (active) {
        if (lo_pass) gate_up_rows<F, LPR, true>(v, gbase, i0, I, C, sub, lds, H, cur, ga, ua);
        else gate_up_rows<F, LPR, false>(v, gbase, i0, I, C, sub, lds, H, cur, ga, ua);
    }
#pragma unroll
    for (int r = 0; r < RU; ++r) {
        const float g = group_sum<LPR>(ga[r]);
        const float u = group_sum<LPR>(ua[r]);
        const int i = i0 + r;
        if (sub == 0 && i < I) st_coh(ht + i, active ? silu(g) * u : 0.0f);
    }
    // shared_expert_gate: sigmoid(x . gate_w) (src/moe_kernels.cpp:162-172),
    // by the first item of each token
    if (a.gate_w && slot == 0 && rb == 0 && wave == 0) {
        float acc = 0.0f;
        for (int c = lane; c < H; c += kWave) acc = __builtin_fmaf(bf16_to_f32(a.gate_w[c]), xt[c], acc);
        acc = group_sum<kWave>(acc);
        if (lane == 0) st_coh(a.gate + t, det_sigmoid(acc));
    }
    if (a.fused) {
        wait_stores();
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(a.ctr + kCtrHDone + 32 * (j & 63), 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
}

template <int F, int LPR, bool LO>
__device__ __forceinline__ void down_rows(const DecodeArgs& a, const int* pslot, const bool* pvalid,
                                          const bool* pshared, const int64_t* wrow, int C, int sub,
                                          const uint32_t* act, int n, Pre (&cur)[kPairsDN],
                                          float* acc) {
    for (int c = sub; c < C; c += LPR) {
        Pre nxt[kPairsDN];
        const int cn = c + LPR;
#pragma unroll
        for (int q = 0; q < kPairsDN; ++q)
            if (cn < C && pvalid[q]) prefetch<F>(pshared[q] ? a.sdn : a.dn, wrow[q], cn, nxt[q]);
#pragma unroll
        for (int q = 0; q < kPairsDN; ++q) {
            if (!pvalid[q]) continue;
            XChunk<F, LO> x;
            load_x<F, LO>(act, n, pslot[q] * C + c, x);
            acc[q] += dot_chunk<F, LO>(cur[q], x);
        }
        if (cn < C) {
#pragma unroll
            for (int q = 0; q < kPairsDN; ++q) cur[q] = nxt[q];
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

    if (a.fused) wait_flag(a.ctr + kCtrRoutesReady, a.ctr + kCtrTimeout);
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
            const int e = ld_coh(a.rex + int64_t(t) * K + pslot[q]);
            const float rw = ld_coh(a.rwt + int64_t(t) * K + pslot[q]);
            if (e < 0 || e >= E || rw == 0.0f) pvalid[q] = false;
            else wrow[q] = int64_t(e) * H + o;
        }
    }
    float acc[NP];
    Pre cur[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        acc[q] = 0.0f;
        if (sub < C && pvalid[q]) prefetch<F>(pshared[q] ? a.sdn : a.dn, wrow[q], sub, cur[q]);
    }
    // h[t] into LDS while the first weights are in flight
    if (a.fused) wait_spread(a.ctr + kCtrHDone, a.NG, a.ctr + kCtrTimeout);
    const bool lo_pass = stage_act<F, true>(a.h + int64_t(t) * n, n, lds);
    if (lo_pass) down_rows<F, LPR, true>(a, pslot, pvalid, pshared, wrow, C, sub, lds, n, cur, acc);
    else down_rows<F, LPR, false>(a, pslot, pvalid, pshared, wrow, C, sub, lds, n, cur, acc);
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const float v = group_sum<LPR>(acc[q]);
        const int p = grp + q * G;
        if (sub == 0 && p < npairs) part[pslot[q] * RB + prow[q]] = pvalid[q] ? v : 0.0f;
    }
    __syncthreads();
    for (int r = threadIdx.x; r < RB; r += blockDim.x) {
        const int o = o_base + r;
        if (o >= H) continue;
        float total = 0.0f;
        for (int s = 0; s < K; ++s) {
            const int e = ld_coh(a.rex + int64_t(t) * K + s);
            const float rw = ld_coh(a.rwt + int64_t(t) * K + s);
            if (e < 0 || e >= E || rw == 0.0f) continue;
            total = __builtin_fmaf(rw, part[s * RB + r], total);
        }
        if (SH) total = __builtin_fmaf(a.gate_in ? ld_coh(a.gate_in + t) : 1.0f, part[K * RB + r], total);
        a.y[int64_t(t) * H + o] = total;
    }
    if (a.fused) {
        // count this item done; whoever sees every down item done zeroes the
        // counters (idempotent), ready for the next launch
        __syncthreads();
        __shared__ int prev_dn;
        if (threadIdx.x == 0)   // the returned value makes the add complete first
            prev_dn = __hip_atomic_fetch_add(a.ctr + kCtrDnDone + 32 * (j & 63), 1,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (threadIdx.x < kWave && prev_dn >= 0) {
            const int done = spread_sum(a.ctr + kCtrDnDone);
            if (done == a.ND) {
                const int lane = threadIdx.x;
                st_coh(a.ctr + kCtrHDone + 32 * lane, 0);
                st_coh(a.ctr + kCtrDnDone + 32 * lane, 0);
                if (lane == 0) {
                    st_coh(a.ctr + kCtrRouterDone, 0);
                    st_coh(a.ctr + kCtrRoutesReady, 0);
                }
            }
        }
    }
    __syncthreads();
}

// Router rows + top-k: the first launch of the decode forward (its
// registers are kept out of the expert kernel below).
template <int F>
__global__ __launch_bounds__(kGemvThreads) void moe_router_kernel(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    router_item(a, blockIdx.x, lds);
}

// gate_up then down items, one work-group per item.
template <int F, int LPG, int LPD, bool SH>
__global__ __launch_bounds__(kGemvThreads) void moe_decode_fused(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    const int it = blockIdx.x;
    if (it < a.NG) gate_up_item<F, LPG, SH>(a, it, lds);
    else down_item<F, LPD, SH>(a, it - a.NG, lds);
}

// Single-role kernels of the standalone launchers (routes and h are inputs).
template <int F, int LPG, bool SH>
__global__ __launch_bounds__(kGemvThreads) void moe_gate_up_kernel(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    gate_up_item<F, LPG, SH>(a, blockIdx.x, lds);
}
template <int F, int LPD, bool SH>
__global__ __launch_bounds__(kGemvThreads) void moe_down_kernel(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    down_item<F, LPD, SH>(a, blockIdx.x, lds);
}

// ------------------------------------------------------------ launching

template <int F, int LPG, int LPD, bool SH>
inline hipError_t launch_fused(hipStream_t st, const DecodeArgs& a) {
    const int items = a.NG + a.ND;
    DecodeArgs ex = a;
    ex.NR = 0;
    const size_t lds = decode_lds_bytes(F, ex);
    if (a.NR) {
        const size_t rl = size_t(kGemvWaves) * (512 + 64) * sizeof(float);
        hipLaunchKernelGGL(moe_router_kernel<F>, dim3(a.NR), dim3(kGemvThreads), rl, st, a);
    }
    if (items <= 0) return hipGetLastError();
    hipLaunchKernelGGL((moe_decode_fused<F, LPG, LPD, SH>), dim3(items), dim3(kGemvThreads), lds, st,
                       a);
    return hipGetLastError();
}

template <int F, int LPG, int LPD, bool SH>
inline hipError_t launch_t(hipStream_t st, const DecodeArgs& a) {
    if (a.NR + a.NG + a.ND <= 0) return hipSuccess;
    if (a.fused) return launch_fused<F, LPG, LPD, SH>(st, a);
    if (a.NR) return hipErrorInvalidValue;   // the router role runs fused only
    const size_t lds = decode_lds_bytes(F, a);
    if (a.NG)
        hipLaunchKernelGGL((moe_gate_up_kernel<F, LPG, SH>), dim3(a.NG), dim3(kGemvThreads), lds, st,
                           a);
    if (a.ND)
        hipLaunchKernelGGL((moe_down_kernel<F, LPD, SH>), dim3(a.ND), dim3(kGemvThreads), lds, st, a);
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

#define GRIM_DECODE_INSTANTIATE(F)                                               \
    hipError_t decode_launch_fmt_##F(hipStream_t st, const DecodeArgs& a) {   \
        return a.shared ? pick_lpg<F, true>(st, a) : pick_lpg<F, false>(st, a); \
    }

}  // namespace grim
