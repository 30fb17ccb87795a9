// topk.hpp -- per-wave router top-k, shared by the top-k kernel and the
// fused decode kernel.
//
// One wavefront per token with every score in VGPRs (lane l owns experts
// [l*V, l*V+V), V = ceil(E/64) <= 8).  Each round packs (order-preserving
// score bits, ~expert) into one 64-bit key, so one wave max gives the
// largest score and, among equal scores, the lowest expert index -- the tie
// rule of src/ops.cpp:1125-1131.  The weights are then formed in pick order
// with the reference kernels' operations (src/ops.cpp:1133-1147,
// :2126-2135), using det_expf so that the oracle reproduces them bit for
// bit.
#pragma once

#include "common.hpp"

namespace grim {

constexpr int kMaxV = 8;          // E <= 512

__device__ __forceinline__ uint64_t score_key(float v, int e) {
    if (v != v) return (uint64_t(1) << 32) | uint32_t(~e);   // NaN ranks below everything
    uint32_t u = f_bits(v + 0.0f);                           // -0 -> +0
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (uint64_t(u) << 32) | uint32_t(~e);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    const uint32_t lo = dpp_u<CTRL>(uint32_t(v)), hi = dpp_u<CTRL>(uint32_t(v >> 32));
    return (uint64_t(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Wave-wide max of a 64-bit key, uniform result: DPP inside each 16-lane
// row, then the four row results read into scalars.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
    k = max64(k, dpp64<kDppXor1>(k));
    k = max64(k, dpp64<kDppXor2>(k));
    k = max64(k, dpp64<kDppHalfMirror>(k));
    k = max64(k, dpp64<kDppMirror>(k));
    const uint32_t lo = uint32_t(k), hi = uint32_t(k >> 32);
    uint64_t r = 0;
#pragma unroll
    for (int row = 0; row < 4; ++row) {
        const uint64_t v = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(hi), row * 16))) << 32) |
                           uint32_t(__builtin_amdgcn_readlane(int(lo), row * 16));
        r = max64(r, v);
    }
    return r;
}

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Top-k of one token by one wave.  mode 0: softmax (decode semantics);
// 1: softmax batched semantics (normalize == 0 -> raw logits); 2: sigmoid +
// bf16 bias; 3: group-limited sigmoid + fp32 bias.  Lane s ends holding
// pick s and writes oe[s], ow[s].  gsel (512 floats) and gscore (64) are
// this wave's LDS scratch for mode 3.  COHERENT: the logits were written by
// other work-groups of the same launch, so they are read (and the routes
// written) with device-coherent accesses.
template <bool COHERENT = false>
__device__ __forceinline__ void topk_wave(const float* __restrict__ row, int E, int K, int mode,
                                          int normalize, float scaling,
                                          const uint16_t* __restrict__ bias16,
                                          const float* __restrict__ bias32, int n_group,
                                          int topk_group, int32_t* __restrict__ oe,
                                          float* __restrict__ ow, float* gsel_w, float* gscore_w) {
    const int lane = threadIdx.x & (kWave - 1);
    const int V = (E + kWave - 1) / kWave;

    uint64_t key[kMaxV];
    float wsrc[kMaxV];
#pragma unroll
    for (int j = 0; j < kMaxV; ++j) {
        const int e = lane * V + j;
        key[j] = 0;
        wsrc[j] = 0.0f;
        if (j < V && e < E) {
            const float l = COHERENT ? __hip_atomic_load(row + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                     : row[e];
            float sel;
            if (mode <= 1) {
                sel = l;
                wsrc[j] = l;
            } else {
                const float sc = det_sigmoid(l);
                const float b = mode == 2 ? (bias16 ? bf16_to_f32(bias16[e]) : 0.0f)
                                          : (bias32 ? bias32[e] : 0.0f);
                sel = sc + b;
                wsrc[j] = sc;
            }
            key[j] = score_key(sel, e);
            if (mode == 3) gsel_w[e] = sel;
        }
    }

    if (mode == 3) {
        // group score: sum of the two largest biased scores of each group
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int gs = E / n_group;
        if (lane < n_group) {
            int b1 = -1, b2 = -1;
            for (int e = lane * gs; e < (lane + 1) * gs; ++e) {
                const float v = gsel_w[e];
                if (b1 < 0 || v > gsel_w[b1]) { b2 = b1; b1 = e; }
                else if (b2 < 0 || v > gsel_w[b2]) b2 = e;
            }
            gscore_w[lane] = gs > 1 ? gsel_w[b1] + gsel_w[b2] : gsel_w[b1];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint64_t keep = 0;
        for (int j = 0; j < topk_group; ++j) {
            int best = -1;
            for (int g = 0; g < n_group; ++g) {
                if (keep & (uint64_t(1) << g)) continue;
                if (best < 0 || gscore_w[g] > gscore_w[best]) best = g;
            }
            keep |= uint64_t(1) << best;
        }
#pragma unroll
        for (int j = 0; j < kMaxV; ++j) {
            const int e = lane * V + j;
            if (j < V && e < E && !((keep >> (e / gs)) & 1)) key[j] = 0;
        }
    }

    int my_pick = -1;
    float my_val = 0.0f;
    for (int s = 0; s < K; ++s) {
        uint64_t best = 0;
        float bval = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxV; ++j)
            if (key[j] > best) { best = key[j]; bval = wsrc[j]; }
        const uint64_t win = wave_max_u64(best);
        const int e = win ? int(~uint32_t(win)) : -1;
        const int owner = e >= 0 ? e / V : 0;
        const float val = lane_f(bval, owner);
#pragma unroll
        for (int j = 0; j < kMaxV; ++j)
            if (key[j] == win) key[j] = 0;
        if (lane == s) { my_pick = e; my_val = val; }
    }

    // weights, serially in pick order through scalar reads (the reference
    // kernels' operation order, src/ops.cpp:1133-1147 and :2126-2135)
    float w;
    if (mode <= 1) {
        if (mode == 1 && !normalize) {
            w = my_val;
        } else {
            float m = lane_f(my_val, 0);
            for (int s = 1; s < K; ++s) m = fmaxf(m, lane_f(my_val, s));
            const float ev = det_expf(my_val - m);
            float sum = 0.0f;
            for (int s = 0; s < K; ++s) sum += lane_f(ev, s);
            w = (normalize && sum > 0.0f) ? ev / sum : ev;
        }
    } else {
        w = my_val;
        if (normalize) {
            float sum = 0.0f;
            for (int s = 0; s < K; ++s) sum += lane_f(w, s);
            if (sum > 0.0f) w /= sum;
        }
        if (scaling != 1.0f) w *= scaling;
    }
    if (lane < K) {
        if (COHERENT) {
            __hip_atomic_store(oe + lane, my_pick, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ow + lane, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            oe[lane] = my_pick;
            ow[lane] = w;
        }
    }
}


}  // namespace grim
