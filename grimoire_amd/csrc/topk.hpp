// topk.hpp -- per-wave router top-k, shared by the top-k kernel and the
// fused decode kernel.
//
// One wavefront per token with every score in VGPRs (lane l owns experts
// [l*V, l*V+V), V = ceil(E/64) <= 8).  Each round takes the wave max of
// order-preserving 32-bit score keys, then the lowest expert index holding
// it (lowest lane by ballot, then its lowest slot) -- the tie rule of
// src/ops.cpp:1125-1131.  The weights are then formed in pick order
// with the reference kernels' operations (src/ops.cpp:1133-1147,
// :2126-2135), using det_expf so that the oracle reproduces them bit for
// bit.
#pragma once

#include "common.hpp"

namespace grim {

constexpr int kMaxV = 8;          // E <= 512
static_assert(kMaxV % 4 == 0, "the E == 64 kMaxV loads move four logits at a time");
constexpr int kRouterTok = 8;     // tokens per router_row call

// Router logits of one expert row for nt <= kRouterTok tokens by one
// 256-thread work-group: thread i multiplies elements [4i + 1024m, +4), lanes
// reduce by DPP, the four waves add in wave order through red (LDS, 32
// floats).  Thread t < nt returns token t's dot product.  Shared by the
// router kernel and the decode kernel's router role, so both give the same
// bits.
__device__ __forceinline__ float router_row(const float* __restrict__ wr,
                                            const float* __restrict__ x, int nt, int H,
                                            float* red) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    float acc[kRouterTok];
#pragma unroll
    for (int i = 0; i < kRouterTok; ++i) acc[i] = 0.0f;
#pragma unroll 2
    for (int k = threadIdx.x * 4; k < H; k += 1024) {
        const float4 wv = *reinterpret_cast<const float4*>(wr + k);
#pragma unroll
        for (int i = 0; i < kRouterTok; ++i) {
            if (i < nt) {
                const float4 xv = *reinterpret_cast<const float4*>(x + int64_t(i) * H + k);
                acc[i] = __builtin_fmaf(wv.x, xv.x, acc[i]);
                acc[i] = __builtin_fmaf(wv.y, xv.y, acc[i]);
                acc[i] = __builtin_fmaf(wv.z, xv.z, acc[i]);
                acc[i] = __builtin_fmaf(wv.w, xv.w, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kRouterTok; ++i) {
        if (i < nt) {
            const float v = group_sum<kWave>(acc[i]);
            if (lane == 0) red[wave * kRouterTok + i] = v;
        }
    }
    __syncthreads();
    float r = 0.0f;
    const int t = threadIdx.x;
    if (t < nt)
        r = (red[t] + red[kRouterTok + t]) + (red[2 * kRouterTok + t] + red[3 * kRouterTok + t]);
    __syncthreads();
    return r;
}

// router_row for one token in two halves: every load of the row and of x
// issued up front (NK float4 of each per thread, clamped addresses), then
// the same FMA order and the same reduction as router_row, so both give the
// same bits.  NK * 1024 >= H.
template <int NK>
struct RouterRegs {
    float4 w[NK], x[NK];
};

template <int NK>
__device__ __forceinline__ void router_row1_load(const float* __restrict__ wr,
                                                 const float* __restrict__ x, int H,
                                                 RouterRegs<NK>& r) {
#pragma unroll
    for (int m = 0; m < NK; ++m) {
        const int k = int(threadIdx.x) * 4 + 1024 * m;
        const int kk = k < H ? k : 0;
        r.w[m] = *reinterpret_cast<const float4*>(wr + kk);
        r.x[m] = *reinterpret_cast<const float4*>(x + kk);
    }
}

template <int NK>
__device__ __forceinline__ float router_row1_finish(const RouterRegs<NK>& r, int H, float* red) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < NK; ++m) {
        const int k = int(threadIdx.x) * 4 + 1024 * m;
        float a2 = __builtin_fmaf(r.w[m].x, r.x[m].x, acc);
        a2 = __builtin_fmaf(r.w[m].y, r.x[m].y, a2);
        a2 = __builtin_fmaf(r.w[m].z, r.x[m].z, a2);
        a2 = __builtin_fmaf(r.w[m].w, r.x[m].w, a2);
        acc = k < H ? a2 : acc;
    }
    const float v = group_sum<kWave>(acc);
    if (lane == 0) red[wave * kRouterTok] = v;
    __syncthreads();
    float res = 0.0f;
    if (threadIdx.x == 0)
        res = (red[0] + red[kRouterTok]) + (red[2 * kRouterTok] + red[3 * kRouterTok]);
    __syncthreads();
    return res;
}

// Order-preserving 32-bit key of a score; 0 marks an empty or taken slot,
// NaN (1) ranks below every number.
__device__ __forceinline__ uint32_t score_key(float v) {
    if (v != v) return 1u;
    const uint32_t u = f_bits(v + 0.0f);                     // -0 -> +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);       // -inf -> 0x007fffff
}

// Wave-wide max, uniform result: DPP inside each 16-lane row, then the four
// row results read into scalars.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
    k = max(k, dpp_u<kDppXor1>(k));
    k = max(k, dpp_u<kDppXor2>(k));
    k = max(k, dpp_u<kDppHalfMirror>(k));
    k = max(k, dpp_u<kDppMirror>(k));
    const uint32_t r0 = __builtin_amdgcn_readlane(int(k), 0);
    const uint32_t r1 = __builtin_amdgcn_readlane(int(k), 16);
    const uint32_t r2 = __builtin_amdgcn_readlane(int(k), 32);
    const uint32_t r3 = __builtin_amdgcn_readlane(int(k), 48);
    return max(max(r0, r1), max(r2, r3));
}

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// The logits of one token as topk_wave holds them: lane l owns experts
// [l*V, l*V+V), V = ceil(E/64).  Loaded with clamped addresses and no
// branch, so that the loads can be issued together with others.
__device__ __forceinline__ void topk_load(const float* __restrict__ row, int E, float (&lv)[kMaxV]) {
    const int lane = threadIdx.x & (kWave - 1);
    const int V = (E + kWave - 1) / kWave;
    if (E == kWave * kMaxV) {
        // every lane's logits contiguous: 16-byte loads
        typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = 0; j < kMaxV; j += 4) {
            const f4 v = *reinterpret_cast<const f4*>(row + lane * kMaxV + j);
            lv[j] = v.x; lv[j + 1] = v.y; lv[j + 2] = v.z; lv[j + 3] = v.w;
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < kMaxV; ++j) {
        const int e = lane * V + j;
        lv[j] = row[(j < V && e < E) ? e : 0];
    }
}

// bf16 logits, widened exactly to fp32 (launch_router_topk_bf16_batched)
__device__ __forceinline__ void topk_load(const uint16_t* __restrict__ row, int E,
                                          float (&lv)[kMaxV]) {
    const int lane = threadIdx.x & (kWave - 1);
    const int V = (E + kWave - 1) / kWave;
#pragma unroll
    for (int j = 0; j < kMaxV; ++j) {
        const int e = lane * V + j;
        lv[j] = bf16_to_f32(row[(j < V && e < E) ? e : 0]);
    }
}

// Top-k of one token by one wave from logits held as topk_load leaves
// them.  mode 0: softmax (decode semantics); 1: softmax batched semantics
// (normalize == 0 -> raw logits); 2: sigmoid + bf16 bias; 3: group-limited
// sigmoid + fp32 bias.  Lane s ends holding pick s and writes oe[s],
// ow[s].  gsel (512 floats) and gscore (64) are this wave's LDS scratch
// for mode 3.
__device__ __forceinline__ void topk_wave_regs(const float (&lv)[kMaxV], int E, int K, int mode,
                                               int normalize, float scaling,
                                               const uint16_t* __restrict__ bias16,
                                               const float* __restrict__ bias32, int n_group,
                                               int topk_group, int32_t* __restrict__ oe,
                                               float* __restrict__ ow, float* gsel_w,
                                               float* gscore_w) {
    const int lane = threadIdx.x & (kWave - 1);
    const int V = (E + kWave - 1) / kWave;

    const int gsz = mode == 3 ? E / n_group : 0;
    const int lpg = gsz / V;   // lanes per group when groups are whole lanes
    const bool lane_groups = mode == 3 && gsz % V == 0 && lpg >= 1 && lpg <= kWave && (lpg & (lpg - 1)) == 0;
    uint32_t key[kMaxV];
    float wsrc[kMaxV], selv[kMaxV];
    auto sel_of = [&](int j) { return selv[j]; };
#pragma unroll
    for (int j = 0; j < kMaxV; ++j) {
        const int e = lane * V + j;
        key[j] = 0;
        wsrc[j] = 0.0f;
        selv[j] = 0.0f;
        if (j < V && e < E) {
            const float l = lv[j];
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
            key[j] = score_key(sel);
            selv[j] = sel;
            if (mode == 3 && !lane_groups) gsel_w[e] = sel;
        }
    }

    if (lane_groups) {
        // groups of lpg whole lanes: each lane's two largest biased scores,
        // merged across its group by butterflies (the two largest of a
        // multiset), group score = largest + second largest (the largest
        // alone for one-expert groups); group g is kept when fewer than
        // topk_group groups beat it (higher score, or equal and lower
        // index) -- the same groups and the same sums as the serial pass
        // below, with no LDS and no serial loop over a group
        float m1 = -__builtin_inff(), m2 = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < kMaxV; ++j) {
            const int e = lane * V + j;
            if (j < V && e < E) {
                const float v = sel_of(j);
                if (v > m1) { m2 = m1; m1 = v; }
                else if (v > m2) m2 = v;
            }
        }
        for (int o = 1; o < lpg; o <<= 1) {
            const float b1 = __shfl_xor(m1, o, kWave), b2 = __shfl_xor(m2, o, kWave);
            const float lo1 = fminf(m1, b1), hi2 = fmaxf(m2, b2);
            m1 = fmaxf(m1, b1);
            m2 = fmaxf(lo1, hi2);
        }
        const float score = gsz > 1 ? m1 + m2 : m1;
        const int gi = lane / lpg;
        int rank = 0;
        for (int g = 0; g < n_group; ++g) {
            const float o = lane_f(score, g * lpg);
            rank += (o > score || (o == score && g < gi)) ? 1 : 0;
        }
        if (rank >= topk_group) {
#pragma unroll
            for (int j = 0; j < kMaxV; ++j) key[j] = 0;
        }
    } else if (mode == 3) {
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

    // K rounds of: wave max of the keys, then the lowest expert holding it
    // (experts are lane-major, so the lowest lane, then its lowest slot)
    int my_pick = -1;
    float my_val = 0.0f;
    for (int s = 0; s < K; ++s) {
        uint32_t best = 0;
#pragma unroll
        for (int j = 0; j < kMaxV; ++j) best = max(best, key[j]);
        const uint32_t win = wave_max_u32(best);
        if (win == 0) break;                      // fewer than K experts left
        int jl = kMaxV;
        float bval = 0.0f;
#pragma unroll
        for (int j = kMaxV - 1; j >= 0; --j)
            if (key[j] == win) { jl = j; bval = wsrc[j]; }
        const uint64_t bal = __ballot(jl < kMaxV);
        const int owner = int(__builtin_ctzll(bal));
        const int jw = __builtin_amdgcn_readlane(jl, owner);
        const float val = lane_f(bval, owner);
        if (lane == owner) {
#pragma unroll
            for (int j = 0; j < kMaxV; ++j)
                if (j == jw) key[j] = 0;
        }
        if (lane == s) { my_pick = owner * V + jw; my_val = val; }
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
        oe[lane] = my_pick;
        ow[lane] = w;
    }
}

// Top-k of one token by one wave, reading its logits from memory.
__device__ __forceinline__ void topk_wave(const float* __restrict__ row, int E, int K, int mode,
                                          int normalize, float scaling,
                                          const uint16_t* __restrict__ bias16,
                                          const float* __restrict__ bias32, int n_group,
                                          int topk_group, int32_t* __restrict__ oe,
                                          float* __restrict__ ow, float* gsel_w, float* gscore_w) {
    float lv[kMaxV];
    topk_load(row, E, lv);
    topk_wave_regs(lv, E, K, mode, normalize, scaling, bias16, bias32, n_group, topk_group, oe, ow,
                   gsel_w, gscore_w);
}

// ---------------------------------------------------------------------
// Block-wide top-k by parallel rank counting (modes 0-2), for latency.
//
// One wave running K rounds of max-and-ballot is a chain of several
// hundred dependent instructions (~3 us on MI355X); here the ranks are
// counted in parallel instead: rank(e) = #experts whose 64-bit key
// (score key << 32 | ~e: larger score first, lower index on ties, the rule
// of src/ops.cpp:1125-1131) is larger.  Work item (expert e, segment s of
// 64 keys) per thread; a wave's 64 lanes share s, so every LDS key read is
// a broadcast.  The weights are then formed by wave 0 with the operations
// of topk_wave_regs in the same order (serial sums unrolled over 16 slots
// without branches), so both give the same routes and the same bits.

struct RankLds {
    uint64_t key[512];
    float val[512];
    int rank[512];
    int sel_e[16];
    float sel_v[16];
};

template <int NT>
__device__ __forceinline__ void topk_rank_block(const float* __restrict__ row, int E, int K, int mode,
                                                const uint16_t* __restrict__ bias16, RankLds& L,
                                                unsigned long long* ts = nullptr) {
    const int tid = threadIdx.x;
    const int Ep = (E + 63) & ~63;
#ifdef GRIM_TIMING
#define GRIM_TK_TS(i) if (ts && tid == 0) ts[i] = __builtin_amdgcn_s_memrealtime()
#else
#define GRIM_TK_TS(i) (void)ts
#endif
    // keys and values; padding keys are 0 (never larger than a real key)
#pragma unroll
    for (int q = 0; q < 512 / NT; ++q) {
        const int e = tid + q * NT;
        if (e < Ep) {
            const bool ok = e < E;
            const float l = row[ok ? e : 0];
            float sel = l, v = l;
            if (mode == 2) {
                const float sc = det_sigmoid(l);
                const float b = bias16 ? bf16_to_f32(bias16[ok ? e : 0]) : 0.0f;
                sel = sc + b;
                v = sc;
            }
            L.key[e] = ok ? (uint64_t(score_key(sel)) << 32) | uint64_t(0xFFFFFFFFu - uint32_t(e)) : 0;
            L.val[e] = v;
            L.rank[e] = 0;
        }
    }
    if (tid < 16) { L.sel_e[tid] = -1; L.sel_v[tid] = 0.0f; }
    __syncthreads();
    GRIM_TK_TS(5);
    // partial ranks over 64-key segments, four independent counters
    const int nseg = Ep / 64;
    for (int it = tid; it < Ep * nseg; it += NT) {
        const int sgm = it / Ep, e = it - sgm * Ep;
        const uint64_t me = L.key[e];
        const uint64_t* ks = L.key + 64 * sgm;
        int c0 = 0, c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
        for (int f = 0; f < 64; f += 4) {
            c0 += int(ks[f] > me);
            c1 += int(ks[f + 1] > me);
            c2 += int(ks[f + 2] > me);
            c3 += int(ks[f + 3] > me);
        }
        const int c = (c0 + c1) + (c2 + c3);
        if (e < E && c) atomicAdd(&L.rank[e], c);
    }
    __syncthreads();
    GRIM_TK_TS(6);
#pragma unroll
    for (int q = 0; q < 512 / NT; ++q) {
        const int e = tid + q * NT;
        if (e < E) {
            const int r = L.rank[e];
            if (r < K && (L.key[e] >> 32) != 0) { L.sel_e[r] = e; L.sel_v[r] = L.val[e]; }
        }
    }
    __syncthreads();
#undef GRIM_TK_TS
}

// The routing weights of the picks in L (after topk_rank_block), by one
// wave: lane s < K writes sel_e[s], sel_w[s].
__device__ __forceinline__ void topk_rank_weights(const RankLds& L, int K, int mode, int normalize,
                                                  float scaling, int* sel_e, float* sel_w) {
    const int lane = threadIdx.x & (kWave - 1);
    const bool in = lane < K;
    const int my_pick = lane < 16 ? L.sel_e[lane] : -1;
    const float my_val = lane < 16 ? L.sel_v[lane] : 0.0f;
    float w;
    if (mode <= 1 && !(mode == 1 && !normalize)) {
        // m = max over the K slots (fmaxf is exact, so any order gives the
        // serial chain's value)
        float mx = in ? my_val : -__builtin_inff();
        mx = fmaxf(mx, dpp_f<kDppXor1>(mx));
        mx = fmaxf(mx, dpp_f<kDppXor2>(mx));
        mx = fmaxf(mx, dpp_f<kDppHalfMirror>(mx));
        mx = fmaxf(mx, dpp_f<kDppMirror>(mx));
        const float m = lane_f(mx, 0);
        const float ev = det_expf(my_val - m);
        float sum = 0.0f;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float v = lane_f(ev, s);
            sum += s < K ? v : 0.0f;
        }
        w = (normalize && sum > 0.0f) ? ev / sum : ev;
    } else if (mode <= 1) {
        w = my_val;
    } else {
        w = my_val;
        if (normalize) {
            float sum = 0.0f;
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const float v = lane_f(w, s);
                sum += s < K ? v : 0.0f;
            }
            if (sum > 0.0f) w /= sum;
        }
        if (scaling != 1.0f) w *= scaling;
    }
    if (in) { sel_e[lane] = my_pick; sel_w[lane] = w; }
}

}  // namespace grim
